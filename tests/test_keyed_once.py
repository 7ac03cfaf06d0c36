"""The per-(device, caller stream) side-stream map of the prefill entry points (csrc/keyed_once.h), on the CPU:
two caller streams of one device, or one stream handle on two devices, get distinct side streams; a pair gets the
same one on every call; a failed creation is retried; eight threads asking for the same new pair at once create
it once; past the cap a new pair gets none while the existing pairs keep theirs.  The header is compiled with the host compiler into a small program (no HIP types in it)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mimo-on-a-mac_amd", "csrc")

PROGRAM = r"""
#include <atomic>
#include <stdio.h>
#include <thread>
#include <utility>
#include <vector>
#include "keyed_once.h"

struct Side { int id; };
typedef std::pair<int, void*> Key;          // (device, caller stream handle), as in prefill.hip

int main() {
  mimo::KeyedOnce<Key, Side> per;
  std::atomic<int> made{0};
  auto make = [&]() { return std::unique_ptr<Side>(new Side{made++}); };
  void* sa = reinterpret_cast<void*>(0x1000);
  void* sb = reinterpret_cast<void*>(0x2000);
  Side* a0 = per.get(Key(0, sa), make);
  Side* b0 = per.get(Key(0, sb), make);
  Side* n0 = per.get(Key(0, nullptr), make);
  Side* a1 = per.get(Key(1, sa), make);
  if (!a0 || !b0 || !n0 || !a1) return 10;
  if (a0 == b0 || a0 == n0 || b0 == n0 || a0 == a1) return 11;        // distinct pairs, distinct side streams
  if (per.get(Key(0, sa), make) != a0 || per.get(Key(1, sa), make) != a1) return 12;   // same pair, same one
  if (made.load() != 4 || per.size() != 4) return 13;
  // a failed creation leaves the pair empty and the next request tries again
  auto fail = []() { return std::unique_ptr<Side>(); };
  if (per.get(Key(0, reinterpret_cast<void*>(0x3000)), fail) != nullptr) return 14;
  if (per.size() != 4) return 15;
  Side* c0 = per.get(Key(0, reinterpret_cast<void*>(0x3000)), make);
  if (!c0 || made.load() != 5) return 16;
  // concurrent first requests of one new pair make it once
  std::vector<std::thread> ts;
  std::vector<Side*> got(8, nullptr);
  for (int t = 0; t < 8; ++t)
    ts.emplace_back([&, t]() { got[t] = per.get(Key(2, sa), make); });
  for (auto& t : ts) t.join();
  for (int t = 1; t < 8; ++t) if (got[t] != got[0] || !got[0]) return 17;
  if (made.load() != 6) return 18;
  // a cap: at most 7 objects; a new pair past it gets none (and is not remembered), existing pairs keep theirs
  if (per.get(Key(3, sa), make, 7) == nullptr || per.size() != 7) return 19;
  if (per.get(Key(4, sa), make, 7) != nullptr || per.size() != 7 || made.load() != 7) return 20;
  if (per.get(Key(0, sa), make, 7) != a0) return 21;
  printf("ok\n");
  return 0;
}
"""


def test_side_streams_are_per_caller_stream(tmp_path):
    src = tmp_path / "keyed_once_check.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "keyed_once_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-pthread", "-I", CSRC, str(src), "-o", str(exe)], check=True)
    p = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True)
    assert p.returncode == 0 and p.stdout.strip() == "ok", f"check failed with code {p.returncode}"
