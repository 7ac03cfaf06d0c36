"""Pins for oracle.experts (CPU only)."""
import numpy as np
import pytest

from oracle import experts, mxfp4, routing


def make_pool(S, H, I, seed=0):
    """Expert pool quantised from N(0, 0.02) bf16 weights (engine/tests/test_kernels.py:21-29 shape)."""
    rng = np.random.default_rng(seed)
    p = {}
    for name, (o, i) in {"gate": (I, H), "up": (I, H), "down": (H, I)}.items():
        w = mxfp4.round_bf16((rng.standard_normal((S, o, i)) * 0.02).astype(np.float32))
        p[f"{name}_w"], p[f"{name}_s"] = mxfp4.quantize_mxfp4(w)
    return p


@pytest.fixture(scope="module")
def tiny():
    return experts.ExpertPool(make_pool(8, 256, 512, seed=0))


def test_dot_matches_groupwise_kernel_loop(tiny):
    # Kernel A's structure (kernels.py:50-77): per 32-group partial of x * e2m1(code), times the e8m0 scale
    rng = np.random.default_rng(1)
    x = mxfp4.round_bf16(rng.standard_normal((2, 256)).astype(np.float32)).astype(np.float64)
    q, s = tiny.p["gate_w"][3], tiny.p["gate_s"][3]
    codes = mxfp4.unpack_nibbles(q)
    half = (((codes & 7).astype(np.uint16) << 9) | ((codes & 8).astype(np.uint16) << 12)).view(np.float16)
    out = np.zeros((2, codes.shape[0]))
    for r in range(2):
        for n in range(codes.shape[0]):
            acc = 0.0
            for g in range(8):
                part = float(np.dot(x[r, 32 * g:32 * g + 32], half[n, 32 * g:32 * g + 32].astype(np.float64)))
                acc += part * 2.0 ** (int(s[n, g]) - 127)
            out[r, n] = acc * 16384.0
    np.testing.assert_allclose(tiny.dot("gate", 3, x), out.astype(np.float32), rtol=1e-6, atol=1e-7)


def test_dot_closed_form_all_ones():
    q = np.full((1, 4, 8), 0x22222222, np.uint32)      # every code 2 -> 1.0
    s = np.full((1, 4, 2), 127, np.uint8)              # scale 1
    pool = experts.ExpertPool({"gate_w": q, "gate_s": s})
    x = np.arange(64, dtype=np.float32).reshape(1, 64)
    np.testing.assert_array_equal(pool.dot("gate", 0, x), np.full((1, 4), x.sum(), np.float32))


def test_swiglu_special_values():
    g = np.array([0.0, 200.0, -200.0, 1.0], np.float32)
    u = np.array([3.0, 2.0, 5.0, 1.0], np.float32)
    h = experts.swiglu_bf16(g, u)
    assert h[0] == 0.0 and h[1] == 400.0 and h[2] == 0.0
    sig1 = mxfp4.round_bf16(np.float32(1.0 / (1.0 + np.exp(-1.0))))
    assert h[3] == mxfp4.round_bf16(np.float32(sig1))


def _routes(rng, M, S, k):
    inds = np.stack([rng.choice(S, k, replace=False) for _ in range(M)])
    if M > 1:
        inds[1, :k // 2] = inds[0, :k // 2]          # shared experts across rows (test_kernels.py:73)
    scores = rng.random((M, k)).astype(np.float32)
    scores /= scores.sum(1, keepdims=True)
    return inds, scores


def test_kernel_path_vs_reference_fp32_metric(tiny):
    # the reference test's bar (engine/tests/test_kernels.py:79): max|y - ref| / max|ref| < 2e-2
    rng = np.random.default_rng(2)
    for M in (1, 2, 4, 8):
        x = mxfp4.round_bf16(rng.standard_normal((M, 256)).astype(np.float32))
        inds, scores = _routes(rng, M, 8, 2)
        uids, urows, ucnt, uw, gidx = routing.group_routes(inds, scores, R=8)
        y, _, _ = experts.moe_experts(x, tiny, uids, urows, ucnt, uw, gidx, 2, R=8)
        ref = experts.reference_fp32(x, tiny, inds, scores)
        e = experts.rel_err(y, ref)
        assert 1e-4 < e < 2e-2, (M, e)     # nonzero: the bf16 rounding points are really there


def test_nibble_swap_negative_control(tiny):
    # bench/reports/kernels.md:16: swapping the nibble order gives ~130% error
    rng = np.random.default_rng(3)
    x = mxfp4.round_bf16(rng.standard_normal((2, 256)).astype(np.float32))
    inds, scores = _routes(rng, 2, 8, 2)
    ref = experts.reference_fp32(x, tiny, inds, scores)
    swapped = dict(tiny.p)
    for n in ("gate", "up", "down"):
        q = swapped[f"{n}_w"]
        swapped[f"{n}_w"] = ((q & 0x0F0F0F0F) << 4) | ((q >> 4) & 0x0F0F0F0F)
    bad = experts.reference_fp32(x, experts.ExpertPool(swapped), inds, scores)
    assert experts.rel_err(bad, ref) > 0.5


def test_m1_gather_path_vs_kernel_path(tiny):
    rng = np.random.default_rng(4)
    x = mxfp4.round_bf16(rng.standard_normal((1, 256)).astype(np.float32))
    inds, scores = _routes(rng, 1, 8, 2)
    uids, urows, ucnt, uw, gidx = routing.group_routes(inds, scores, R=8)
    yk, _, _ = experts.moe_experts(x, tiny, uids, urows, ucnt, uw, gidx, 2, R=8)
    yg = experts.gather_m1(x[0], tiny, inds[0], scores[0])
    assert experts.rel_err(yg, yk[0]) < 1e-2       # they differ only by the bf16 rounding of y_e


def test_prefill_rows_equal_m1_path(tiny):
    rng = np.random.default_rng(5)
    T = 6
    x = mxfp4.round_bf16(rng.standard_normal((T, 256)).astype(np.float32))
    inds = np.stack([rng.choice(8, 2, replace=False) for _ in range(T)])
    w = rng.random((T, 2)).astype(np.float32)
    y = experts.moe_prefill(x, tiny, inds, w)
    for t in range(T):
        np.testing.assert_array_equal(y[t], experts.gather_m1(x[t], tiny, inds[t], w[t]))


def test_mimo_shape_error_level():
    # bench/reports/kernels.md:12-14: 0.40-0.45% max relative error at MiMo shapes for the kernel path
    pool = experts.ExpertPool(make_pool(4, 4096, 2048, seed=7))
    rng = np.random.default_rng(6)
    x = mxfp4.round_bf16(rng.standard_normal((2, 4096)).astype(np.float32))
    inds, scores = _routes(rng, 2, 4, 4)
    uids, urows, ucnt, uw, gidx = routing.group_routes(inds, scores, R=8)
    y, _, _ = experts.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, 4, R=8)
    e = experts.rel_err(y, experts.reference_fp32(x, pool, inds, scores))
    assert 1e-3 < e < 1e-2, e
