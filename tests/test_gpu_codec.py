"""GPU codec parity: MXFP4 quantise/dequantise, seeded pool fill, activation hi/lo split, sigmoid table."""
import numpy as np
import pytest
import torch

from oracle import experts as ox, mxfp4 as oq
from helpers import bf16_bits, to_dev_bf16

pytestmark = pytest.mark.gpu


def test_quantize_mxfp4_bit_exact(rng):
    from mimo_stream import kernels
    w = oq.round_bf16((rng.standard_normal((512, 1024)) * 0.02).astype(np.float32))
    w[0, :32] = 0.0
    w[1, :64] = np.linspace(-1, 1, 64)
    q, s = kernels.quantize_mxfp4(to_dev_bf16(w))
    qo, so = oq.quantize_mxfp4(w)
    np.testing.assert_array_equal(q.cpu().numpy().view(np.uint32), qo)
    np.testing.assert_array_equal(s.cpu().numpy(), so)


def test_dequantize_bit_exact(rng):
    from mimo_stream import kernels
    qo = rng.integers(0, 2 ** 32, (64, 32), dtype=np.uint64).astype(np.uint32)
    so = rng.integers(0, 256, (64, 8)).astype(np.uint8)
    so[0, :] = [0, 1, 126, 127, 128, 254, 255, 200]
    out = kernels.dequantize_mxfp4(torch.from_numpy(qo.view(np.int32)).cuda(), torch.from_numpy(so).cuda())
    ref = oq.dequantize_mxfp4(qo, so)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])


def test_fill_random_equals_quantized_random():
    from mimo_stream import kernels, pools
    from mimo_stream import _lib
    rows, cols = 300, 512
    w = kernels.random_bf16((rows, cols), seed=1234, stddev=0.02)
    q1, s1 = kernels.quantize_mxfp4(w)
    q2 = torch.empty_like(q1)
    s2 = torch.empty_like(s1)
    _lib.call("mimo_fill_random_mxfp4", 1234, 0.02, rows, cols, _lib.ptr(q2), _lib.ptr(s2), _lib.stream_ptr())
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    wf = w.float().cpu().numpy()
    assert abs(wf.mean()) < 1e-3 and abs(wf.std() - 0.02) < 1e-3
    qo, so = oq.quantize_mxfp4(wf)
    np.testing.assert_array_equal(q1.cpu().numpy().view(np.uint32), qo)
    np.testing.assert_array_equal(s1.cpu().numpy(), so)
    b = pools.random_bank(2, seed=5, hidden=256, inter=512)
    assert b["gate_w"].abs().sum() > 0 and b["down_s"].shape == (2, 256, 16)


def test_fp8_hilo_bit_exact(rng):
    from mimo_stream import kernels
    x = oq.round_bf16(rng.standard_normal((16, 4096)).astype(np.float32))
    x[0, :32] = 0.0
    x[1, :32] = oq.round_bf16(np.float32(1e-30))
    hi, hs, lo, ls = kernels.quantize_fp8_hilo(to_dev_bf16(x))
    ohi, ohs, olo, ols = oq.quantize_fp8_hilo(x)
    for got, ref in ((hi, ohi), (hs, ohs), (lo, olo), (ls, ols)):
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_fp8_hilo_every_finite_bf16(rng):
    """Every finite bf16 value, shuffled into 32-element blocks (wide ranges inside a block: subnormal and
    saturating E4M3 codes, negative values that round to zero), plus blocks mixing 1e30 with tiny values."""
    from mimo_stream import kernels
    bits = np.arange(65536, dtype=np.uint32)
    finite = ((bits >> 7) & 0xFF) != 0xFF
    vals = ((bits[finite] << 16).astype(np.uint32)).view(np.float32)
    vals = vals[rng.permutation(vals.size)]
    n = vals.size // 4096 * 4096
    x = vals[:n].reshape(-1, 4096).copy()
    x[0, :32] = oq.round_bf16(np.float32(1e30) * rng.standard_normal(32).astype(np.float32) ** 9)
    x[0, 32:64] = oq.round_bf16(np.array([-1e-20] * 31 + [3.0], np.float32))
    hi, hs, lo, ls = kernels.quantize_fp8_hilo(to_dev_bf16(x))
    ohi, ohs, olo, ols = oq.quantize_fp8_hilo(x)
    for got, ref in ((hi, ohi), (hs, ohs), (lo, olo), (ls, ols)):
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_sigmoid_table_bit_exact():
    from mimo_stream import kernels
    tab = bf16_bits(kernels.sigmoid_table())
    np.testing.assert_array_equal(tab, ox.sigtab_bits())
