"""Shape sweep: the MoE block at hidden / intermediate sizes, expert counts and top-k other than MiMo's, with
ragged token counts, against the oracle (decode: the distinct-expert path and the M = 1 gather path;
prefill: the grouped GEMMs and combine).  Decode takes hidden sizes 256-4096 (powers of two) and intermediate
sizes 512, 1024 or 2048; prefill any hidden size that is a multiple of 256 and intermediate size that is a
multiple of 128 (narrow tiles of rarely chosen experts only when the intermediate size is a multiple of 256, whose
K-steps of 256 codes the down GEMM then divides into; every tile wide otherwise).
The bar is the one of the other parity tests."""
import numpy as np
import pytest
import torch

from oracle import experts as ox, routing as orr
from helpers import assert_bf16_close, bf16_np, pool_np, rand_bf16, to_dev_bf16, zipf_routes

pytestmark = pytest.mark.gpu

DECODE_SHAPES = [   # (hidden, inter, experts, top_k)
    (256, 512, 4, 1),
    (512, 1024, 16, 3),
    (1024, 512, 32, 4),
    (2048, 1024, 64, 6),
    (4096, 2048, 128, 8),
]
PREFILL_SHAPES = DECODE_SHAPES[:4] + [
    (256, 384, 8, 2),       # intermediate not a multiple of 256: wide tiles only
    (768, 640, 16, 3),      # hidden not a multiple of 512: wide tiles only
]


def _block(rng, H, I, E, k, seed):
    from mimo_stream import MoEBlock, Router, pools
    bank = pools.random_bank(E, seed=seed, hidden=H, inter=I)
    r = Router(H, E, k)
    W = rand_bf16(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * 1e-3).astype(np.float32)
    r.weight.copy_(to_dev_bf16(W))
    r.e_score_correction_bias.copy_(torch.from_numpy(bias))
    return MoEBlock(r, bank), bank, W, bias


@pytest.mark.parametrize("H,I,E,k", DECODE_SHAPES)
def test_decode_block_shapes(rng, H, I, E, k):
    blk, bank, W, bias = _block(rng, H, I, E, k, seed=H + I + E)
    pool = pool_np(bank)
    for M in (1, 2, 3, 8):
        x = rand_bf16(rng, (M, H))
        y, inds, w = blk(to_dev_bf16(x), return_routes=True)
        gi, gw = inds.cpu().numpy(), w.cpu().numpy()
        # the router entry point gives the decode block's routes; both bit-exact given its logits
        logits, rinds, rw = blk.router.logits_and_routes(to_dev_bf16(x))
        lg = logits.cpu().numpy()
        ref = orr.router_logits(x, W)
        assert np.abs(lg - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-6
        oi, ow = orr.select_topk(lg, bias, k)
        np.testing.assert_array_equal(gi, oi)
        np.testing.assert_array_equal(gw, ow)
        assert torch.equal(inds, rinds) and torch.equal(w, rw)
        if M == 1:
            oy = ox.gather_m1(x[0], pool, gi[0], gw[0])[None]
        else:
            uids, urows, ucnt, uw, gidx = orr.group_routes(gi, gw, R=8)
            oy, _, _ = ox.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, k, R=8)
        assert_bf16_close(bf16_np(y), oy, what=f"decode H={H} I={I} E={E} k={k} M={M}")


@pytest.mark.parametrize("H,I,E,k", PREFILL_SHAPES)
def test_prefill_block_shapes(rng, H, I, E, k):
    blk, bank, _, _ = _block(rng, H, I, E, k, seed=3 * H + I + E)
    pool = pool_np(bank)
    for T in (9, 77, 300):
        x = rand_bf16(rng, (T, H))
        inds = zipf_routes(rng, T, E, k)
        w = rng.random((T, k)).astype(np.float32)
        w /= w.sum(1, keepdims=True)
        y = blk._moe_prefill(to_dev_bf16(x), torch.from_numpy(inds).cuda(), torch.from_numpy(w).cuda())
        oy = ox.moe_prefill(x, pool, inds, w)
        assert_bf16_close(bf16_np(y), oy, what=f"prefill H={H} I={I} E={E} k={k} T={T}")


def test_two_row_decode_shared_experts(rng):
    """Two rows with identity slots take the path where every block finds its expert from the union of the two
    rows' selections: identical rows (every expert on both rows), nearby rows (partial overlap) and unrelated
    rows, at the MiMo shape (256 experts: all four ballot words)."""
    H, I, E, k = 4096, 2048, 256, 8
    blk, bank, W, bias = _block(rng, H, I, E, k, seed=2024)
    pool = pool_np(bank)
    base = rand_bf16(rng, (1, H))
    cases = {"identical": np.concatenate([base, base]),
             "nearby": np.concatenate([base, base + rand_bf16(rng, (1, H), 0.3)]),
             "unrelated": rand_bf16(rng, (2, H))}
    for name, x in cases.items():
        x = to_dev_bf16(x).float().cpu().numpy()          # bf16-exact rows
        y, inds, w = blk(to_dev_bf16(x), return_routes=True)
        gi, gw = inds.cpu().numpy(), w.cpu().numpy()
        logits, _, _ = blk.router.logits_and_routes(to_dev_bf16(x))
        oi, ow = orr.select_topk(logits.cpu().numpy(), bias, k)
        np.testing.assert_array_equal(gi, oi)
        np.testing.assert_array_equal(gw, ow)
        uids, urows, ucnt, uw, gidx = orr.group_routes(gi, gw, R=8)
        if name == "identical":
            assert len(uids) == k and (ucnt[:k] == 2).all()
        oy, _, _ = ox.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, k, R=8)
        assert_bf16_close(bf16_np(y), oy, what=f"two-row decode, {name} rows")
