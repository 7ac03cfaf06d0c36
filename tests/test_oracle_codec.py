"""Pins for oracle.mxfp4 against independent formulations (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import mxfp4


def test_e2m1_table_matches_reference_half_bit_trick():
    # engine/mimo_stream/kernels.py:21-23: half bits ((c & 7) << 9) | ((c & 8) << 12) is value * 2^-14
    c = np.arange(16, dtype=np.uint16)
    half = (((c & 7) << 9) | ((c & 8) << 12)).astype(np.uint16).view(np.float16).astype(np.float64)
    np.testing.assert_array_equal(half * 16384.0, mxfp4.E2M1_VALUES.astype(np.float64))
    assert np.signbit(mxfp4.E2M1_VALUES[8]) and not np.signbit(mxfp4.E2M1_VALUES[0])


def test_e2m1_table_matches_ocp_closed_form():
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        v = 0.5 * m if e == 0 else 2.0 ** (e - 1) * (1 + 0.5 * m)
        assert mxfp4.E2M1_VALUES[c] == (-v if s else v)


def test_e8m0_all_256():
    # kernels.py:25-29: s=0 -> bits 0x00400000 (2^-127), s=255 -> NaN, else bits s << 23
    s = np.arange(256)
    got = mxfp4.e8m0_to_float(s)
    assert got[0] == np.array([0x00400000], np.uint32).view(np.float32)[0]
    assert np.isnan(got[255])
    exp = (s[1:255].astype(np.uint32) << 23).view(np.float32)
    np.testing.assert_array_equal(got[1:255], exp)


def test_nibble_order_low_first():
    codes = np.array([[1, 2, 3, 4, 5, 6, 7, 8]], np.uint8)
    assert mxfp4.pack_nibbles(codes)[0, 0] == 0x87654321
    rng = np.random.default_rng(1)
    c = rng.integers(0, 16, (3, 5, 64)).astype(np.uint8)
    np.testing.assert_array_equal(mxfp4.unpack_nibbles(mxfp4.pack_nibbles(c)), c)


def test_bf16_rounding_against_torch():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(100000) * 10.0 ** rng.uniform(-30, 30, 100000)).astype(np.float32)
    x[:4] = [0.0, -0.0, np.inf, -np.inf]
    ours = mxfp4.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


def _brute_e2m1(y):
    """Nearest grid value, ties to the even mantissa bit, saturating at 6 (independent brute force)."""
    grid = [(0.0, 0), (0.5, 1), (1.0, 0), (1.5, 1), (2.0, 0), (3.0, 1), (4.0, 0), (6.0, 1)]
    if y >= 6.0:
        return 6.0
    best = None
    for v, mbit in grid:
        d = abs(y - v)
        if best is None or d < best[0] or (d == best[0] and mbit == 0):
            best = (d, v, mbit)
    return best[1]


def test_quantize_mxfp4_brute_force():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 64)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :32] = np.linspace(-1, 1, 32)       # exact ties appear on the grid
    w = mxfp4.round_bf16(w)
    q, s = mxfp4.quantize_mxfp4(w)
    deq = mxfp4.dequantize_mxfp4(q, s)
    for r in range(w.shape[0]):
        for b in range(2):
            blk = w[r, 32 * b:32 * b + 32].astype(np.float64)
            amax = np.abs(blk).max()
            X = int(np.floor(np.log2(amax))) - 2 if amax > 0 else -127
            assert s[r, b] == X + 127
            for j in range(32):
                mag = _brute_e2m1(abs(blk[j]) / 2.0 ** X)
                assert deq[r, 32 * b + j] == np.float32(np.copysign(mag, blk[j]) * 2.0 ** X) or mag == 0.0


def test_quantize_idempotent_on_grid():
    rng = np.random.default_rng(4)
    q = rng.integers(0, 2 ** 32, (8, 16), dtype=np.uint64).astype(np.uint32)
    s = rng.integers(100, 150, (8, 4)).astype(np.uint8)
    deq = mxfp4.dequantize_mxfp4(q, s)
    q2, s2 = mxfp4.quantize_mxfp4(deq)
    np.testing.assert_array_equal(mxfp4.dequantize_mxfp4(q2, s2), deq)


def test_dequantize_f64_table_equals_nibble_definition():
    """The byte-table float64 dequantisation (used by the oracle's dot products) gives exactly the values of the
    nibble-by-nibble definition: every byte value in both nibble positions, every scale byte (0 and 255
    included, NaN where the scale is NaN).  Scales 253 and 254 put +-3 .. +-6 above the float32 range: there the
    float32 definition overflows to +-inf and the float64 form keeps the exact product."""
    rng = np.random.default_rng(5)
    q = rng.integers(0, 2 ** 32, (256, 64), dtype=np.uint64).astype(np.uint32)
    q[0] = np.arange(256, dtype=np.uint32).reshape(64, 4) @ np.array([1, 256, 65536, 1 << 24], np.uint32)
    s = np.tile(np.arange(256, dtype=np.uint8)[:, None], (1, 16))
    a = mxfp4.dequantize_mxfp4(q, s).astype(np.float64)
    b = mxfp4.dequantize_mxfp4_f64(q, s)
    assert b.dtype == np.float64 and b.shape == a.shape
    np.testing.assert_array_equal(np.isnan(a), np.isnan(b))
    ok = ~np.isnan(a) & ~np.isinf(a)
    np.testing.assert_array_equal(a[ok], b[ok])
    np.testing.assert_array_equal(np.signbit(a[ok]), np.signbit(b[ok]))   # -0 codes stay -0
    big = np.isinf(a)
    assert big.any() and np.all(s.repeat(32, 1)[big] >= 253)
    vals = mxfp4.E2M1_VALUES[mxfp4.unpack_nibbles(q)].astype(np.float64)
    np.testing.assert_array_equal(b[big], np.ldexp(vals[big], s.repeat(32, 1)[big].astype(np.int64) - 127))


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ours = mxfp4.e4m3_to_float(codes)
    finite = ~np.isnan(theirs)
    np.testing.assert_array_equal(np.isnan(ours), ~finite)
    np.testing.assert_array_equal(ours[finite], theirs[finite])


def test_e4m3_encode_matches_torch_rne():
    rng = np.random.default_rng(5)
    y = np.concatenate([rng.uniform(0, 448, 200000), 2.0 ** rng.uniform(-12, 8.8, 200000),
                        np.arange(0, 448, 1 / 64.0)]).astype(np.float32)
    y = y[y <= 448]
    ours = mxfp4._e4m3_encode_mag(y.astype(np.float64))
    theirs = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)


def test_fp8_hilo_reconstructs_bf16_exactly():
    rng = np.random.default_rng(6)
    x = mxfp4.round_bf16(rng.standard_normal((8, 4096)).astype(np.float32))
    hi, hs, lo, ls = mxfp4.quantize_fp8_hilo(x)
    rec = mxfp4.dequantize_fp8_hilo(hi, hs, lo, ls)
    amax = np.abs(x.reshape(8, 128, 32)).max(-1, keepdims=True)
    near = (np.abs(x.reshape(8, 128, 32)) >= amax * 2.0 ** -14).reshape(x.shape)
    np.testing.assert_array_equal(rec[near], x[near].astype(np.float64))
    err = np.abs(rec - x).reshape(8, 128, 32)
    assert np.all(err <= amax * 2.0 ** -17)
    # hi alone is a plain MXFP8 quantisation: within half an E4M3 ulp (2^-4 relative) of x per element, or
    # half the subnormal quantum (2^-9 * scale, scale <= amax * 2^-7) for elements far below the block max
    hv = mxfp4.dequantize_fp8_hilo(hi, hs, np.zeros_like(lo), ls)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, (amax * 2.0 ** -17).repeat(32, -1).reshape(x.shape))
    assert np.all(np.abs(hv - x) <= bound)
    # scale rule: block max maps into (224, 448]
    amax = np.abs(x.reshape(8, 128, 32)).max(-1)
    ratio = amax / np.ldexp(1.0, hs.astype(np.int64) - 127)
    assert np.all((ratio > 224) & (ratio <= 448))


def test_fp8_hilo_zero_block():
    x = np.zeros((1, 64), np.float32)
    x[0, 32:] = -0.0
    hi, hs, lo, ls = mxfp4.quantize_fp8_hilo(x)
    assert np.all(hi == 0) and np.all(lo == 0) and np.all(hs == 127) and np.all(ls == 127)
