"""E8M0 scale corners and non-finite activations through the hot paths (fused decode at 1, 2 and 4 rows, the
distinct-expert path with its intermediates, and the prefill block), against the oracle.

Reference semantics (engine/mimo_stream/kernels.py:24-29, :59-77, :113-119): scale byte 0 is 2^-127 and byte 255
is NaN, applied to each 32-group's partial dot product, so a NaN scale makes that output NaN for every row routed
to the expert (gate/up: the whole h column, and through the down projection every output of those rows; down:
that output).  The block-scaled MFMA takes the same E8M0 bytes (v_mfma_scale_f32_16x16x128_f8f6f4): byte 255
gives NaN products, byte 0 products of at most 6 * 448 * 2^-127 per element, which no bf16 result can see.

Non-finite activations: a NaN element makes every dot product of its row NaN, in the reference and here (the
hi/lo split codes it as the E4M3 NaN).  An infinite element gives the reference +-inf or NaN per output of the
gate/up products, depending on the sign and zeroness of the weight it meets, and from there NaN in h and in every
output of the row's down projection (h holds infinities and NaNs; the down weights hold zero codes).  Here the
split codes an infinity as the E4M3 NaN too (E4M3 has no infinity), so h is NaN where the reference has +-inf
or NaN; the block output y is NaN at exactly the reference's positions.  The router sees the same +-inf / NaN
logits as the reference (IEEE fp32 arithmetic, NaN-insensitive to order) and selects bit-exactly.  Rows without
a non-finite element are unaffected and meet the usual tolerance."""
import numpy as np
import pytest
import torch

from oracle import experts as ox, routing as orr
from helpers import assert_bf16_close, bf16_np, pool_np, rand_bf16, to_dev_bf16

pytestmark = pytest.mark.gpu

H, I, E, K = 4096, 2048, 16, 8
F = 5          # the expert whose scales are patched; a large selection bias routes every row to it


def _block(rng, seed, patch):
    from mimo_stream import MoEBlock, Router, pools
    bank = pools.random_bank(E, seed=seed, hidden=H, inter=I)
    patch(bank)
    r = Router(H, E, K)
    W = rand_bf16(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * 1e-3).astype(np.float32)
    bias[F] = 10.0
    r.weight.copy_(to_dev_bf16(W))
    r.e_score_correction_bias.copy_(torch.from_numpy(bias))
    return MoEBlock(r, bank), bank, W, bias


def _set(bank, name, idx, byte):
    bank[name][idx] = byte
    torch.cuda.synchronize()


PATCHES = {
    # (patch, what the reference gives for the rows routed to F)
    "down_nan": lambda b: _set(b, "down_s", (F, 100, 5), 255),      # y[:, 100] NaN
    "gate_nan": lambda b: _set(b, "gate_s", (F, 7, 3), 255),        # the rows' whole y NaN
    "up_nan": lambda b: _set(b, "up_s", (F, 2047, 63), 255),        # the rows' whole y NaN
    "zero_scales": lambda b: (_set(b, "gate_s", (F, 11), 0), _set(b, "up_s", (F, 300, 17), 0),
                              _set(b, "down_s", (F, 4000), 0), _set(b, "down_s", (F + 1, 5, 9), 0)),
}


def _compare(got, ref, what):
    """Non-finite at exactly the reference's positions and NaN there (y); the finite elements within the
    parity tolerance."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    gbad, rbad = ~np.isfinite(got), ~np.isfinite(ref)
    n_diff = int((gbad != rbad).sum())
    assert n_diff == 0, (f"{what}: non-finite pattern differs at {n_diff} elements (GPU {int(gbad.sum())}, "
                         f"oracle {int(rbad.sum())}); first at {np.argwhere(gbad != rbad)[:4].tolist()}")
    assert np.isnan(got[gbad]).all(), f"{what}: GPU non-finite outputs are not all NaN"
    ok = ~rbad
    if ok.any():
        assert_bf16_close(got[ok], ref[ok], what=what)
    return int(rbad.sum())


def _decode_oracle(x, pool, gi, gw):
    if x.shape[0] == 1:
        return ox.gather_m1(x[0], pool, gi[0], gw[0])[None]
    uids, urows, ucnt, uw, gidx = orr.group_routes(gi, gw, R=8)
    return ox.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, K, R=8)[0]


def _check_routes(blk, x, inds, w, bias):
    """The block's routes equal the oracle selection on the GPU's logits (whose non-finite pattern equals the
    oracle's own logits)."""
    logits, _, _ = blk.router.logits_and_routes(to_dev_bf16(x))
    lg = logits.cpu().numpy()
    W = blk.router.weight.float().cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        ref = orr.router_logits(x, W)
    np.testing.assert_array_equal(np.isnan(lg), np.isnan(ref))
    np.testing.assert_array_equal(np.isposinf(lg), np.isposinf(ref))
    np.testing.assert_array_equal(np.isneginf(lg), np.isneginf(ref))
    fin = np.isfinite(ref)
    if fin.any():
        assert np.abs(lg[fin] - ref[fin]).max() <= 1e-5 * np.abs(ref[fin]).max() + 1e-6
    oi, ow = orr.select_topk(lg, bias, K)
    np.testing.assert_array_equal(inds, oi)
    np.testing.assert_array_equal(w, ow)       # NaN weights (rows whose keys are all NaN) in the same places


@pytest.mark.parametrize("case", list(PATCHES))
def test_scale_corners_decode_and_prefill(rng, case):
    blk, bank, W, bias = _block(rng, seed=401 + len(case), patch=PATCHES[case])
    pool = pool_np(bank)
    xs = rand_bf16(rng, (64, H))
    n_nan = 0
    for M in (1, 2, 4):
        x = xs[:M]
        y, inds, w = blk(to_dev_bf16(x), return_routes=True)
        gi, gw = inds.cpu().numpy(), w.cpu().numpy()
        assert (gi == F).any(1).all(), "every row is routed to the patched expert"
        _check_routes(blk, x, gi, gw, bias)
        with np.errstate(invalid="ignore", over="ignore"):
            oy = _decode_oracle(x, pool, gi, gw)
        n_nan += _compare(bf16_np(y), oy, f"{case}: decode {M} rows")
    # prefill block (router + sorted grouped GEMMs + combine) on 64 tokens
    y, inds, w = blk(to_dev_bf16(xs), return_routes=True)
    gi, gw = inds.cpu().numpy(), w.cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        oy = ox.moe_prefill(xs, pool, gi, gw)
    n_nan += _compare(bf16_np(y), oy, f"{case}: prefill 64 tokens")
    if case == "zero_scales":
        assert n_nan == 0
    else:
        assert n_nan > 0


def test_nan_scales_in_distinct_expert_intermediates(rng):
    """The distinct-expert path's h and fp32 partials (kernels.py:33-123) with NaN gate and down scales: NaN at
    exactly the oracle's positions, every other element within tolerance."""
    from mimo_stream import kernels

    def patch(b):
        _set(b, "gate_s", (F, 7, 3), 255)
        _set(b, "down_s", (F + 1, 100, 5), 255)
    blk, bank, _, _ = _block(rng, seed=433, patch=patch)
    pool = pool_np(bank)
    x = rand_bf16(rng, (4, H))
    gi = np.array([[F, F + 1, 0, 1, 2, 3, 4, 8], [F + 1, 9, 10, 11, 12, 13, 14, 15],
                   [F, 0, 1, 2, 3, 4, 8, 9], [0, 1, 2, 3, 4, 8, 9, 10]], np.int32)
    gw = rng.random((4, K)).astype(np.float32)
    uids, urows, ucnt, uw, gidx = orr.group_routes(gi, gw, R=8)
    y, h, part = kernels.moe_experts(to_dev_bf16(x), bank, uids, urows, ucnt, uw, R=8, gather_idx=gidx,
                                     return_intermediates=True)
    with np.errstate(invalid="ignore", over="ignore"):
        oy, oh, opart = ox.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, K, R=8)
    U = len(uids)
    _compare(bf16_np(h)[:U], oh, "h")
    _compare(part.cpu().numpy()[:U], opart, "fp32 partials")
    _compare(bf16_np(y), oy, "y")
    assert np.isnan(bf16_np(y)[[0, 2]]).all() and np.isfinite(bf16_np(y)[3]).all()


NONFINITE_ROWS = {0: (17, np.inf), 1: (1000, np.nan), 2: (4095, -np.inf), 5: (2048, np.inf), 6: (31, np.nan)}


def _with_nonfinite(x):
    x = x.copy()
    for r, (c, v) in NONFINITE_ROWS.items():
        if r < x.shape[0]:
            x[r, c] = v
    return x


def test_nonfinite_activations(rng):
    blk, bank, W, bias = _block(rng, seed=455, patch=lambda b: None)
    pool = pool_np(bank)
    xs = _with_nonfinite(rand_bf16(rng, (40, H)))
    bad_rows = np.array(sorted(NONFINITE_ROWS))
    for M in (1, 2, 4, 8):
        x = xs[:M]
        y, inds, w = blk(to_dev_bf16(x), return_routes=True)
        gi, gw = inds.cpu().numpy(), w.cpu().numpy()
        _check_routes(blk, x, gi, gw, bias)
        with np.errstate(invalid="ignore", over="ignore"):
            oy = _decode_oracle(x, pool, gi, gw)
        yn = bf16_np(y)
        _compare(yn, oy, f"non-finite activations: decode {M} rows")
        rows = bad_rows[bad_rows < M]
        assert np.isnan(yn[rows]).all(), "rows with a non-finite element come out NaN"
        good = np.setdiff1d(np.arange(M), rows)
        assert np.isfinite(yn[good]).all(), "the other rows are not touched"
    y, inds, w = blk(to_dev_bf16(xs), return_routes=True)     # 40 tokens: router + prefill block
    gi, gw = inds.cpu().numpy(), w.cpu().numpy()
    _check_routes(blk, xs, gi, gw, bias)
    with np.errstate(invalid="ignore", over="ignore"):
        oy = ox.moe_prefill(xs, pool, gi, gw)
    yn = bf16_np(y)
    _compare(yn, oy, "non-finite activations: prefill 40 tokens")
    assert np.isnan(yn[bad_rows]).all()
    assert np.isfinite(np.delete(yn, bad_rows, axis=0)).all()
