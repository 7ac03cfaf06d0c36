"""Pins of the decoder-layer oracle (oracle/layer.py): the post-attention RMSNorm and the residual h = x + y
(engine/mimo_stream/model.py:299, :340; nn.RMSNorm :75).

MLX's rms_norm is not available here, so the norm is pinned against what the mathematics fixes: a float64
evaluation of the definition (within one bf16 ulp), closed forms, scale invariance and exact sums.  A dropped
eps, a sum in place of the mean, a missing weight or a transposed reduction each fail one of these."""
import math

import numpy as np
import pytest

from oracle import layer as ol
from oracle.mxfp4 import bf16_bits_to_f32, f32_to_bf16_bits


def bits(a):
    return f32_to_bf16_bits(np.asarray(a, np.float32))


def vals(b):
    return bf16_bits_to_f32(b).astype(np.float64)


@pytest.mark.parametrize("H", [256, 1024, 4096])
def test_rmsnorm_within_one_bf16_ulp_of_float64(H):
    rng = np.random.default_rng(H)
    x = bits(rng.standard_normal((6, H)) * np.array([1e-3, 0.1, 1.0, 3.0, 40.0, 1e3])[:, None])
    w = bits(1.0 + 0.3 * rng.standard_normal(H))
    for eps in (1e-6, 1e-5):
        r = vals(ol.rmsnorm(x, w, eps))
        r64 = ol.rmsnorm_f64(x, w, eps)
        # two bf16 roundings (x * inv, then w * that): at most 2^-8 relative plus a half ulp, and float32 noise
        bound = np.abs(r64) * 2.0 ** -7 + 1e-30
        assert np.all(np.abs(r - r64) <= bound)
        # the rounding points: bf16(w * bf16(x * inv)) with inv from float64 agrees bit for bit except where the
        # float32 inv (its own last bits) flips a rounding; rounding once (bf16(w * x * inv)) would not
        xv, wv = vals(x), vals(w)
        inv64 = 1.0 / np.sqrt((xv * xv).mean(axis=-1, keepdims=True) + float(np.float32(eps)))
        inner = vals(bits(xv * inv64))
        r_ref = vals(bits(wv * inner))
        assert np.mean(r == r_ref) > 0.99
        once = vals(bits(wv * xv * inv64))
        assert np.mean(once == r_ref) < 0.99


def test_rmsnorm_closed_forms():
    H = 4096
    one = bits(np.ones(H))
    # constant row c with eps = 0: inv = 1 / |c| (c^2 and H c^2 exact), so r = sign(c) * w exactly
    for c in (1.5, -0.75, 3.0, 2.0 ** -20):
        x = bits(np.full((1, H), c))
        r = vals(ol.rmsnorm(x, one, 0.0))
        np.testing.assert_array_equal(r, np.full((1, H), math.copysign(1.0, c)))
    # weight applies elementwise: w = 2^j per element scales exactly
    wj = bits(2.0 ** (np.arange(H) % 5 - 2))
    x = bits(np.full((1, H), 1.5))
    np.testing.assert_array_equal(vals(ol.rmsnorm(x, wj, 0.0)), vals(wj)[None])
    # zero row: r = 0 (no NaN), whatever eps
    z = bits(np.zeros((1, H)))
    np.testing.assert_array_equal(vals(ol.rmsnorm(z, one, 1e-5)), np.zeros((1, H)))
    # eps-dominated row: x = 2^-14 everywhere, eps = 2^-10 >> mean(x^2) = 2^-28 -> r ~ x / sqrt(eps) = 2^-9;
    # dropping eps would give 1.0
    x = bits(np.full((1, H), 2.0 ** -14))
    r = vals(ol.rmsnorm(x, one, 2.0 ** -10))
    np.testing.assert_allclose(r, 2.0 ** -14 / math.sqrt(2.0 ** -28 + 2.0 ** -10), rtol=2.0 ** -8)


def test_rmsnorm_scale_invariance_and_mean():
    rng = np.random.default_rng(7)
    H = 4096
    x = bits(rng.standard_normal((4, H)))
    w = bits(1.0 + 0.1 * rng.standard_normal(H))
    # scaling x by a power of two is exact through squares, sums, sqrt and division (eps = 0)
    x4 = bits(vals(x) * 4.0)
    np.testing.assert_array_equal(ol.rmsnorm(x, w, 0.0), ol.rmsnorm(x4, w, 0.0))
    # the mean, not the sum: rows of H ones give r = w (a sum would give w / sqrt(H))
    ones = bits(np.ones((1, H)))
    np.testing.assert_array_equal(vals(ol.rmsnorm(ones, w, 0.0)), vals(w)[None])


def test_tree_sum_matches_exact_sum():
    rng = np.random.default_rng(3)
    for H in (256, 4096, 8192):
        x = vals(bits(rng.standard_normal(H))).astype(np.float32)
        ss = float(ol._tree_sum_sq(x))
        exact = math.fsum(float(v) * float(v) for v in x)
        assert abs(ss - exact) <= exact * 2.0 ** -24 * (H // 256 + 8)


def test_residual_add():
    rng = np.random.default_rng(11)
    x = bits(rng.standard_normal(10000))
    y = bits(rng.standard_normal(10000) * 0.05)
    h = vals(ol.residual_add(x, y))
    exact = vals(x) + vals(y)
    # one bf16 rounding of the (float32-exact here) sum: within half an ulp
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
    assert np.all(np.abs(h - exact) <= ulp / 2 + 1e-30)
    np.testing.assert_array_equal(ol.residual_add(x, bits(np.zeros(10000))), x)   # x + 0 = x
    np.testing.assert_array_equal(vals(ol.residual_add(x, bits(-vals(x)))), np.zeros(10000))


def _owner_sum_sq(xf):
    """The same sum from each element's owner (wave, lane, chunk, element), in plain Python float32 steps."""
    H = xf.shape[-1]
    q4 = H // 4
    parts = [[[] for _ in range(64)] for _ in range(4)]
    for e in range(H):
        w, off = divmod(e, q4)
        c, rem = divmod(off, 512)
        lane, j = divmod(rem, 8)
        parts[w][lane].append((c, j, np.float32(xf[e]) * np.float32(xf[e])))
    g = np.zeros((4, 64), np.float32)
    for w in range(4):
        for lane in range(64):
            acc = np.float32(0.0)
            for _, _, v in sorted(parts[w][lane], key=lambda t: (t[0], t[1])):
                acc = np.float32(acc + v)
            g[w, lane] = acc
    for s in (32, 16, 8, 4, 2, 1):
        g = np.array([[np.float32(g[w, l] + g[w, l ^ s]) for l in range(64)] for w in range(4)], np.float32)
    return np.float32(np.float32(g[0, 0] + g[1, 0]) + np.float32(g[2, 0] + g[3, 0]))


@pytest.mark.parametrize("H", [256, 2560, 4096])
def test_tree_sum_order_by_element_owner(H):
    """The vectorised sum equals the sum taken from each element's owner; rows of mixed magnitudes make the
    order visible (a thread-strided order gives a different float32 result on some of them)."""
    rng = np.random.default_rng(H + 1)
    differs = 0
    for t in range(6):
        x = vals(bits(rng.standard_normal(H) * np.exp(rng.uniform(-6, 6, H)))).astype(np.float32)
        ss = ol._tree_sum_sq(x)
        assert ss == _owner_sum_sq(x)
        # the thread-strided order (thread t adding x[t + 256 j]) for contrast
        sq = (x * x).astype(np.float32)
        p = np.zeros(256, np.float32)
        for j in range(H // 256):
            p = (p + sq[256 * j: 256 * (j + 1)]).astype(np.float32)
        g = p.reshape(4, 64)
        idx = np.arange(64)
        for s in (32, 16, 8, 4, 2, 1):
            g = (g + g[:, idx ^ s]).astype(np.float32)
        strided = np.float32(np.float32(g[0, 0] + g[1, 0]) + np.float32(g[2, 0] + g[3, 0]))
        differs += int(strided != ss)
    if H > 256:
        assert differs > 0
