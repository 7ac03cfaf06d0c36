"""The compile-time bf16 sigmoid table (csrc/sigmoid_table.h, the data the prefill epilogue looks up) against the
oracle's table (oracle.experts.sigtab_bits, which restates sigmoid_table, engine/mimo_stream/kernels.py:138-146,
with the specified sigmoid): all 65,536 entries bit for bit.  The header is compiled for the host with ROCm's
clang, the compiler whose constant evaluator fills the device table, and the program writes the table out."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import experts as ox

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "mimo-on-a-mac_amd", "csrc", "sigmoid_table.h")
CLANG = "/opt/rocm/llvm/bin/clang++"

PROGRAM = r"""
#include <stdio.h>
#include "sigmoid_table.h"
static constexpr mimo::sigtab_gen::Table kTab = mimo::sigtab_gen::make();
int main(int argc, char** argv) {
  FILE* f = fopen(argv[1], "wb");
  if (!f) return 1;
  if (fwrite(kTab.v, sizeof(uint16_t), 65536, f) != 65536) return 2;
  return fclose(f) ? 3 : 0;
}
"""


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang not installed")
def test_compile_time_table_equals_oracle(tmp_path):
    src = tmp_path / "dump_sigtab.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "dump_sigtab"
    subprocess.run([CLANG, "-std=c++17", "-O1", "-fconstexpr-steps=100000000", "-I", os.path.dirname(HEADER),
                    str(src), "-o", str(exe)], check=True)
    out = tmp_path / "table.bin"
    subprocess.run([str(exe), str(out)], check=True)
    got = np.fromfile(out, dtype=np.uint16)
    want = ox.sigtab_bits()
    assert got.shape == (65536,)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} entries differ, first at bits {bad[:8]}: {got[bad[:8]]} vs {want[bad[:8]]}"
    # a few closed-form entries: sigmoid(0) = 0.5, sigmoid(+inf) = 1, sigmoid(-inf) = 0, NaN stays NaN
    assert got[0x0000] == 0x3F00 and got[0x8000] == 0x3F00
    assert got[0x7F80] == 0x3F80 and got[0xFF80] == 0x0000
    assert got[0x7FC0] == 0x7FC0
