"""Known-answer cases for the oracle's bf16 rounding points, with the expected bits derived by hand (in the comments)
from bfloat16 arithmetic as the reference's Metal kernels and MLX perform it: every bf16 result is the fp32 result
rounded to nearest-even at 8 significant bits.  Each case is built so that a dropped or an extra rounding gives
different bits:

  * Kernel A's epilogue h = bf16(bf16(gt * sig) * ut) (engine/mimo_stream/kernels.py:79-82): two roundings, not one.
  * the per-expert bf16 output of the gather_qmm paths (engine/mimo_stream/model.py:181-182 for one row,
    :228 / :270 for prefill): y = bf16(sum_j bf16(y_e_j) * w_j), against the distinct-expert kernels' fp32
    partials (kernels.py:120, :198-199), y = bf16(sum_j y_e_j * w_j).  (CPU only.)"""
import numpy as np

from oracle import experts as ox, mxfp4 as oq

BF16_ONE = 0x3F80


def bits(v):
    return int(oq.f32_to_bf16_bits(np.array([v], np.float32))[0])


def test_swiglu_rounds_twice():
    # g = u = 1.5 (exact bf16).  sigmoid(1.5) = 1 / (1 + e^-1.5) = 1 / 1.2231302 = 0.8175745: in [0.5, 1) the bf16
    # step is 2^-8, 0.8175745 * 256 = 209.299 -> 209 -> sig = 209 / 256 = 0.81640625.
    # gt * sig = 1.5 * 0.81640625 = 1.224609375, in [1, 2) the step is 2^-7: 1.224609375 * 128 = 156.75 -> 157
    #   -> 1.2265625;   * ut = 1.2265625 * 1.5 = 1.83984375, * 128 = 235.5, a tie -> even 236 -> h = 1.84375.
    # One rounding of the exact product: 1.5 * 0.81640625 * 1.5 = 1.8369140625, * 128 = 235.125 -> 235
    #   -> 1.8359375.
    assert bits(1.84375) == 0x3FEC and bits(1.8359375) == 0x3FEB
    sig_bits = ox.sigtab_bits()[bits(1.5)]
    assert sig_bits == bits(0.81640625)
    h = ox.swiglu_bf16(np.array([1.5], np.float32), np.array([1.5], np.float32))
    assert bits(h[0]) == 0x3FEC
    # gt and ut are rounded first: g = 1.5 + 2^-10 and u = 1.5 - 2^-10 are below half a step from 1.5
    h2 = ox.swiglu_bf16(np.array([1.5 + 2 ** -10], np.float32), np.array([1.5 - 2 ** -10], np.float32))
    assert bits(h2[0]) == 0x3FEC


def _pool():
    """Two experts of hidden 32, intermediate 32 whose first output is a chosen exact sum (codes and scales set by
    hand; E2M1 codes 2 = 1.0, 3 = 1.5, 6 = 4.0; scale byte s means 2^(s - 127)).  With x = e_0:
      gate row n, n in {0, 1}: 4.0 * 2^2 = 16 at column 0, so g = 16, sigmoid(16) = 1 - 1.1e-7 rounds to 1.0 in
      bf16 (within 2^-9 of 1), gt * sig = 16;
      up row 0: 1.0 * 2^-4 -> ut = 2^-4 -> h_0 = bf16(16 * 2^-4) = 1.0;  up row 1: 1.0 * 2^-13 -> h_1 = 2^-9;
      every other row is zero (g = 0: gt * sig = 0, h = 0).
      expert 0, down row 0: 1.0 at columns 0 and 1 -> y_0 = 1 + 2^-9 (between bf16 1.0 and 1 + 2^-7);
      expert 1, down row 0: 1.5 at column 1 -> y_1 = 1.5 * 2^-9 = 0.0029296875 (exact in bf16)."""
    E, H, I = 2, 32, 32
    codes = {"gate": np.zeros((E, I, H), np.uint8), "up": np.zeros((E, I, H), np.uint8),
             "down": np.zeros((E, H, I), np.uint8)}
    scales = {"gate": np.full((E, I, H // 32), 127, np.uint8), "up": np.full((E, I, H // 32), 127, np.uint8),
              "down": np.full((E, H, I // 32), 127, np.uint8)}
    for e in range(E):
        for n in (0, 1):
            codes["gate"][e, n, 0] = 6
            scales["gate"][e, n, 0] = 129
            codes["up"][e, n, 0] = 2
        scales["up"][e, 0, 0] = 123
        scales["up"][e, 1, 0] = 114
    codes["down"][0, 0, 0] = 2
    codes["down"][0, 0, 1] = 2
    codes["down"][1, 0, 1] = 3
    p = {}
    for k in ("gate", "up", "down"):
        p[f"{k}_w"] = oq.pack_nibbles(codes[k])
        p[f"{k}_s"] = scales[k]
    return ox.ExpertPool(p)


def test_pool_builds_the_intended_h_and_outputs():
    pool = _pool()
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 1.0
    for e in (0, 1):
        h = ox.swiglu_bf16(pool.dot("gate", e, x), pool.dot("up", e, x))[0]
        assert h[0] == 1.0 and h[1] == 2.0 ** -9 and np.all(h[2:] == 0.0)
    hv = np.zeros((1, 32), np.float32)
    hv[0, 0], hv[0, 1] = 1.0, 2.0 ** -9
    assert pool.dot("down", 0, hv)[0, 0] == np.float32(1 + 2 ** -9)
    assert pool.dot("down", 1, hv)[0, 0] == np.float32(1.5 * 2 ** -9)


def test_one_row_and_prefill_round_each_expert_output():
    # gather_qmm paths: bf16(y_0) = bf16(1 + 2^-9): 1.001953125 * 128 = 128.25 -> 128 -> 1.0; bf16(y_1) = y_1.
    #   y = bf16(1.0 * 1 + 0.0029296875 * 1) = bf16(1.0029296875): * 128 = 128.375 -> 128 -> 1.0 (bits 0x3F80).
    # Without the per-expert rounding: bf16(1.001953125 + 0.0029296875 = 1.0048828125): * 128 = 128.625 -> 129
    #   -> 1.0078125 (bits 0x3F81).
    pool = _pool()
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    w = np.array([1.0, 1.0], np.float32)
    y = ox.gather_m1(x, pool, np.array([0, 1]), w)
    assert bits(y[0]) == BF16_ONE
    yp = ox.moe_prefill(np.stack([x, x]), pool, np.array([[0, 1], [1, 0]]), np.stack([w, w]))
    assert bits(yp[0, 0]) == BF16_ONE and bits(yp[1, 0]) == BF16_ONE


def test_distinct_expert_kernels_keep_fp32_partials():
    # Kernel B's partials stay fp32 (kernels.py:120) and the combine rounds once (:198-199): the row's two routes
    # give bf16(1.001953125 + 0.0029296875) = 1.0078125 (bits 0x3F81), one step above the gather_qmm result.
    pool = _pool()
    x = np.zeros((2, 32), np.float32)
    x[:, 0] = 1.0
    inds = np.array([[0, 1], [0, 1]])
    w = np.ones((2, 2), np.float32)
    from oracle import routing as orr
    uids, urows, ucnt, uw, gidx = orr.group_routes(inds, w, R=8)
    y, h, part = ox.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, 2, R=8)
    assert bits(y[0, 0]) == 0x3F81 and bits(y[1, 0]) == 0x3F81
    # and with round_expert_bf16 (the M = 1 use of the same kernels) the gather_qmm bits again
    y1, _, _ = ox.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, 2, R=8, round_expert_bf16=True)
    assert bits(y1[0, 0]) == BF16_ONE
