"""The decoder-layer pieces around the MoE block (oracle; test infrastructure only).

Restated reference behaviour (engine/mimo_stream/model.py:296-340):
  * r = post_attention_layernorm(x) (:299): nn.RMSNorm(hidden, eps=layernorm_epsilon) (:75), i.e. MLX's
    mx.fast.rms_norm: r = w * (x * rsqrt(mean(x^2) + eps)), bf16 in and out, fp32 inside.
  * h = x + y (:340): a bf16 addition.

This build specifies the norm's fp32 arithmetic exactly, so the oracle reproduces the HIP kernels bit for bit:
  ss  = sum of x^2 in float32 (a bf16 square is exact in float32) as 4 x 64 partials: partial (w, l) adds the
        squares of the 8-element chunks starting at w H/4 + 512 c + 8 l (c = 0, 1, ...; chunks at or past
        (w + 1) H/4 are empty) in (chunk, element) order; within each group of 64 partials a butterfly
        (p[l] += p[l ^ s] for s = 32, 16, 8, 4, 2, 1); the 4 group sums as (g0 + g1) + (g2 + g3)
  inv = 1 / sqrt(ss / H + eps)           (float32, each operation correctly rounded)
  r_j = bf16(w_j * bf16(x_j * inv))
MLX applies the same rounding points with its own fp32 summation order; a different order moves inv by a few
float32 ulps, which can flip a bf16 rounding of r.  Against MLX the norm is therefore within one bf16 ulp (not
bit-exact); that bound is pinned below against a float64 evaluation, not against MLX itself (absent here).

Pinned by (tests/test_oracle_layer.py): a float64 evaluation of the definition (every element within one bf16 ulp
plus the float32 error bound), closed forms (constant rows, eps-dominated tiny rows, zero rows), scale
invariance, the tree sum against math.fsum, and the residual against exact float64 addition.
"""
import numpy as np

from .mxfp4 import bf16_bits_to_f32, f32_to_bf16_bits


def _tree_sum_sq(xf):
    """The kernels' float32 sum of squares of one row (H = 256 n)."""
    H = xf.shape[-1]
    q4 = H // 4
    nch = -(-q4 // 512)
    sq = np.zeros((4, nch * 512), np.float32)
    sq[:, :q4] = (xf * xf).astype(np.float32).reshape(4, q4)   # exact: bf16 squares fit in float32
    ch = sq.reshape(4, nch, 64, 8)                               # [wave, chunk, lane, element]
    g = np.zeros((4, 64), np.float32)
    for c in range(nch):                                         # empty chunks add zeros: exact on sums >= 0
        for j in range(8):
            g = (g + ch[:, c, :, j]).astype(np.float32)
    idx = np.arange(64)
    for s in (32, 16, 8, 4, 2, 1):                               # butterfly within each wave
        g = (g + g[:, idx ^ s]).astype(np.float32)
    w = g[:, 0]
    return np.float32(np.float32(w[0] + w[1]) + np.float32(w[2] + w[3]))


def rmsnorm(x_bits, w_bits, eps):
    """x_bits uint16 [T, H] (bf16), w_bits uint16 [H] -> r bits uint16 [T, H] (the kernel's arithmetic)."""
    x_bits = np.asarray(x_bits, np.uint16)
    T, H = x_bits.shape
    if H % 256:
        raise ValueError("H must be a multiple of 256")
    xf = bf16_bits_to_f32(x_bits)
    wf = bf16_bits_to_f32(np.asarray(w_bits, np.uint16))
    out = np.empty((T, H), np.uint16)
    e = np.float32(eps)
    for t in range(T):
        ss = _tree_sum_sq(xf[t])
        inv = np.float32(np.float32(1.0) / np.sqrt(np.float32(np.float32(ss / np.float32(H)) + e)))
        nv = bf16_bits_to_f32(f32_to_bf16_bits((xf[t] * inv).astype(np.float32)))
        out[t] = f32_to_bf16_bits((wf * nv).astype(np.float32))
    return out


def rmsnorm_f64(x_bits, w_bits, eps):
    """The definition in float64 (no intermediate rounding): w * x / sqrt(mean(x^2) + eps)."""
    x = bf16_bits_to_f32(np.asarray(x_bits, np.uint16)).astype(np.float64)
    w = bf16_bits_to_f32(np.asarray(w_bits, np.uint16)).astype(np.float64)
    return w * x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + float(np.float32(eps)))


def residual_add(x_bits, y_bits):
    """h = bf16(x + y) with the addition in float32 (model.py:340)."""
    xf = bf16_bits_to_f32(np.asarray(x_bits, np.uint16))
    yf = bf16_bits_to_f32(np.asarray(y_bits, np.uint16))
    return f32_to_bf16_bits((xf + yf).astype(np.float32))
