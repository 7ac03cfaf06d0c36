"""MXFP4 / MXFP8 codecs and the expert byte layout (oracle; test infrastructure only).

Reference layout: engine/mimo_stream/kernels.py:5-12 and scripts/convert-mimo-v26-mlx.py:6-12, :93-131:
  * E2M1 nibbles, eight per uint32, LOW nibble first: element k of a row sits in word k // 8, bits 4*(k % 8).
  * One E8M0 scale byte per 32 consecutive elements of a row.
  * Per projection: weights [S, out, in/8] uint32 + scales [S, out, in/32] uint8, slot-major.
Decode (engine/mimo_stream/kernels.py:19-30): e2m1(c) in {+-0, .5, 1, 1.5, 2, 3, 4, 6};
e8m0(s) = 2^(s-127) with s=0 -> 2^-127 and s=255 -> NaN.

The quantisers here are written from the OCP specification (the reference's mx.quantize is third-party MLX and only makes test
data: both sides of every parity check consume the same packed bytes).  quantize_mxfp4 follows the OCP
Microscaling v1.0 rule (shared exponent floor(log2(amax)) - 2, round-to-nearest-even onto the E2M1 grid,
saturate at 6).  quantize_fp8_hilo is the activation split used by the block-scaled MFMA paths: a bf16 value
x is written as hi + lo, both E4M3 with their own E8M0 block scale, which represents every bf16 value of a
block exactly unless it sits more than ~14 binades below the block maximum.
"""
import numpy as np

# E2M1 code -> value (OCP MX v1.0 table 6; sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0)
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


def e8m0_to_float(s):
    """E8M0 byte -> float32 scale 2^(s-127); 255 -> NaN.  kernels.py:24-29."""
    s = np.asarray(s, dtype=np.int64)
    out = np.ldexp(np.float64(1.0), s - 127)
    out = np.where(s == 255, np.nan, out)
    return out.astype(np.float32)


# ---------------------------------------------------------------- bf16 helpers
def f32_to_bf16_bits(x):
    """float32 -> bf16 bit pattern with round-to-nearest-even (NaN kept quiet)."""
    b = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    out = np.where(nan, (b >> 16) | 0x40, rounded)
    return out.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x):
    """float32 -> nearest bf16 value, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------- MXFP4 weights
def pack_nibbles(codes):
    """codes uint8 [..., K] (0..15) -> uint32 [..., K/8], low nibble first (kernels.py:5)."""
    codes = np.asarray(codes, dtype=np.uint32)
    K = codes.shape[-1]
    assert K % 8 == 0
    c = codes.reshape(*codes.shape[:-1], K // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def unpack_nibbles(q):
    """uint32 [..., K/8] -> codes uint8 [..., K]."""
    q = np.asarray(q, dtype=np.uint32)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    c = (q[..., None] >> shifts) & 0xF
    return c.reshape(*q.shape[:-1], q.shape[-1] * 8).astype(np.uint8)


def _e2m1_round(y):
    """|y| >= 0 (float64, already divided by the block scale) -> E2M1 magnitude code 0..7, RNE, saturating."""
    y = np.asarray(y, dtype=np.float64)
    v = np.where(y < 2.0, np.rint(y * 2.0) / 2.0,
                 np.where(y < 4.0, np.rint(y), np.rint(y / 2.0) * 2.0))
    v = np.minimum(v, 6.0)
    # value -> magnitude code
    lut_vals = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    return np.searchsorted(lut_vals, v).astype(np.uint8)


def quantize_mxfp4(w):
    """float32 [..., K] -> (q uint32 [..., K/8], s uint8 [..., K/32]).  OCP MX rule, group 32.

    Shared exponent X = floor(log2(amax)) - 2 clamped to [-127, 127] (amax == 0 -> X = -127); elements are
    w / 2^X rounded to nearest-even on the E2M1 grid and saturated to +-6; a zero magnitude is coded +0.
    Stands in for mx.quantize(mode="mxfp4") (engine/tests/test_kernels.py:26)."""
    w = np.asarray(w, dtype=np.float32)
    K = w.shape[-1]
    assert K % 32 == 0
    blocks = w.reshape(*w.shape[:-1], K // 32, 32).astype(np.float64)
    amax = np.abs(blocks).max(axis=-1)
    _, e = np.frexp(amax)                    # amax = f * 2^e with f in [0.5, 1): floor(log2 amax) = e - 1
    X = np.where(amax > 0, e - 1 - 2, -127)
    X = np.clip(X, -127, 127)
    y = np.abs(blocks) / np.ldexp(1.0, X)[..., None]
    mag = _e2m1_round(y)
    sign = ((blocks < 0) & (mag > 0)).astype(np.uint8) << 3
    codes = (mag | sign).reshape(w.shape)
    return pack_nibbles(codes), (X + 127).astype(np.uint8)


def dequantize_mxfp4(q, s):
    """(uint32 [..., K/8], uint8 [..., K/32]) -> float32 [..., K]: e2m1(code) * e8m0(scale).
    Stands in for mx.dequantize(mode="mxfp4") (engine/tests/test_kernels.py:34)."""
    codes = unpack_nibbles(q)
    vals = E2M1_VALUES[codes]
    sc = e8m0_to_float(s)
    K = vals.shape[-1]
    out = vals.reshape(*vals.shape[:-1], K // 32, 32) * sc[..., None]
    return out.reshape(vals.shape).astype(np.float32)


# the two E2M1 values of every byte of packed nibbles: [byte, 0] = low nibble (the earlier element), [byte, 1] = high
_BYTE_PAIRS = np.stack([E2M1_VALUES[np.arange(256) & 15], E2M1_VALUES[np.arange(256) >> 4]], 1).astype(np.float64)


def dequantize_mxfp4_f64(q, s):
    """dequantize_mxfp4 in float64, for the oracle's dot products: the same values (an E2M1 value times a power
    of two is exact in both types) wherever they fit float32, i.e. for every scale byte but 253 and 254, whose
    largest products the float32 form overflows to +-inf; computed through a byte -> value-pair table instead of
    one nibble at a time.  Elements of a uint32 word are its nibbles from the low end, i.e. its little-endian
    bytes' low then high nibbles (kernels.py:5)."""
    q = np.asarray(q, dtype=np.uint32)
    K = q.shape[-1] * 8
    b = np.ascontiguousarray(q.astype("<u4", copy=False)).view(np.uint8)
    out = np.take(_BYTE_PAIRS, b, axis=0).reshape(*q.shape[:-1], K // 32, 32)
    sc = e8m0_to_float(s).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        out *= sc[..., None]
    return out.reshape(*q.shape[:-1], K)


# ---------------------------------------------------------------- E4M3 + hi/lo activation split
def e4m3_to_float(c):
    """OCP E4M3 (bias 7, no inf, S.1111.111 = NaN) code -> float32."""
    c = np.asarray(c, dtype=np.int64)
    sgn = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    v = np.where(e == 0, np.ldexp(m / 8.0, -6), np.ldexp(1.0 + m / 8.0, e - 7))
    v = np.where((c & 0x7F) == 0x7F, np.nan, v)
    return (sgn * v).astype(np.float32)


def _e4m3_encode_mag(y):
    """y >= 0 float64 with y <= 448 -> E4M3 magnitude code (0..0x7E), round-to-nearest-even."""
    y = np.asarray(y, dtype=np.float64)
    sub = y < 2.0 ** -6
    n_sub = np.rint(y * 512.0)                            # quantum 2^-9; n == 8 is the smallest normal
    _, e = np.frexp(np.where(sub, 1.0, y))
    e = e - 1                                             # y = 1.m * 2^e
    mant = np.rint(np.ldexp(y, -e) * 8.0) - 8.0           # 0..8
    carry = mant >= 8.0
    e = np.where(carry, e + 1, e)
    mant = np.where(carry, 0.0, mant)
    code_norm = ((e + 7) << 3) + mant.astype(np.int64)
    code = np.where(sub, n_sub.astype(np.int64), code_norm)
    return np.minimum(code, 0x7E).astype(np.uint8)


def _fp8_block_quant(v):
    """v float32 [..., nb, 32] -> (codes uint8 same shape, scale byte uint8 [..., nb]).

    X = e - 8 if the block max mantissa m (amax = m * 2^e, m in [1,2)) is <= 1.75 else e - 7, so that
    amax / 2^X <= 448 (the E4M3 maximum); X clamped to [-127, 127]; amax == 0 -> X = 0 (scale 1)."""
    v = np.asarray(v, dtype=np.float32)
    amax = np.abs(v).max(axis=-1).astype(np.float32)
    bits = amax.view(np.uint32).astype(np.int64)
    E = (bits >> 23) & 0xFF
    F = bits & 0x7FFFFF
    e = np.where(E == 0, -127, E - 127)
    X = np.where(F > 0x600000, e - 7, e - 8)
    X = np.where(amax == 0, 0, X)
    X = np.clip(X, -127, 127)
    y = np.abs(v.astype(np.float64)) / np.ldexp(1.0, X)[..., None]
    mag = _e4m3_encode_mag(y)
    sign = ((v < 0) & (mag > 0)).astype(np.uint8) << 7
    return (mag | sign).astype(np.uint8), (X + 127).astype(np.uint8)


def quantize_fp8_hilo(x):
    """bf16-valued float32 [..., K] -> (hi uint8 [..., K], hi_s uint8 [..., K/32], lo, lo_s).

    hi = E4M3 block quantisation of x; lo = E4M3 block quantisation of the exact residual x - hi."""
    x = np.asarray(x, dtype=np.float32)
    K = x.shape[-1]
    blocks = x.reshape(*x.shape[:-1], K // 32, 32)
    hi, hs = _fp8_block_quant(blocks)
    hv = e4m3_to_float(hi).astype(np.float64) * np.ldexp(1.0, hs.astype(np.int64) - 127)[..., None]
    r = (blocks.astype(np.float64) - hv).astype(np.float32)
    lo, ls = _fp8_block_quant(r)
    return hi.reshape(x.shape), hs, lo.reshape(x.shape), ls


def dequantize_fp8_hilo(hi, hs, lo, ls):
    K = hi.shape[-1]
    def deq(c, s):
        v = e4m3_to_float(c).astype(np.float64).reshape(*c.shape[:-1], K // 32, 32)
        return v * np.ldexp(1.0, s.astype(np.int64) - 127)[..., None]
    return (deq(hi, hs) + deq(lo, ls)).reshape(hi.shape)
