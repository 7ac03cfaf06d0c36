"""Golden vectors (tests/golden/moe_golden.npz, written by tests/golden/make_golden.py from the oracle).

CPU: the oracle and the seeded tiny pool still reproduce the committed vectors bit for bit.
GPU: the HIP path on the same inputs — routes, grouping, selection and dispatch bit-exact; expert outputs
within the bf16 bar of the other parity tests (max|dy| / max|y| < 1e-2, >= 99% within two bf16 ulps)."""
import os

import numpy as np
import pytest

from golden import make_golden as mg
from helpers import assert_bf16_close
from oracle import mxfp4 as oq

GOLDEN = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe_golden.npz"))
f32 = lambda bits: oq.bf16_bits_to_f32(bits)


def test_tiny_pool_is_pinned():
    assert mg.pool_sha256(mg.tiny_pool()) == str(GOLDEN["tiny_pool_sha256"])


def test_oracle_reproduces_golden_vectors():
    d = mg.build()
    assert sorted(d) == sorted(GOLDEN.files)
    for key in GOLDEN.files:
        np.testing.assert_array_equal(d[key], GOLDEN[key], err_msg=key)


def test_golden_vectors_are_consistent():
    """Properties the vectors must have whatever the oracle: weights sum to 1 per row, routes distinct per row,
    the dispatch is a permutation sorted by slot and stable."""
    w = GOLDEN["tiny_w"]
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    assert all(len(set(r)) == len(r) for r in GOLDEN["tiny_inds"])
    assert all(len(set(r)) == len(r) for r in GOLDEN["sel_inds"])
    perm, offsets = GOLDEN["disp_perm"], GOLDEN["disp_offsets"]
    flat = GOLDEN["disp_slots"].reshape(-1)
    assert sorted(perm.tolist()) == list(range(flat.size))
    for s in range(8):
        seg = perm[offsets[s]:offsets[s + 1]]
        assert np.all(flat[seg] == s) and np.all(np.diff(seg) > 0)
    np.testing.assert_array_equal(GOLDEN["disp_inv"][perm], np.arange(flat.size))


def _tiny_block():
    import torch
    from mimo_stream import MoEBlock, Router
    pool = mg.tiny_pool()
    bank = {k: torch.from_numpy(v.view(np.int32) if k.endswith("_w") else v).cuda() for k, v in pool.items()}
    r = Router(mg.TINY["H"], mg.TINY["E"], mg.TINY["k"])
    r.weight.copy_(torch.from_numpy(f32(GOLDEN["tiny_wg"])).to(torch.bfloat16))
    r.e_score_correction_bias.copy_(torch.from_numpy(GOLDEN["tiny_bias"]))
    return MoEBlock(r, bank), bank


def _x():
    import torch
    return torch.from_numpy(f32(GOLDEN["tiny_x"])).to(torch.bfloat16).cuda()


@pytest.mark.gpu
def test_gpu_tiny_router():
    blk, _ = _tiny_block()
    logits, inds, w = blk.router.logits_and_routes(_x())
    ref = GOLDEN["tiny_logits"]
    lg = logits.cpu().numpy()
    assert np.abs(lg - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-6       # fp32 accumulation order only
    np.testing.assert_array_equal(inds.cpu().numpy(), GOLDEN["tiny_inds"])  # key gaps >= 0.018: same routes
    np.testing.assert_allclose(w.cpu().numpy(), GOLDEN["tiny_w"], rtol=1e-6)


@pytest.mark.gpu
def test_gpu_selection_group_and_dispatch_golden():
    import torch
    from mimo_stream import group_routes, prefill_dispatch, select_from_logits
    inds, w = select_from_logits(torch.from_numpy(GOLDEN["sel_logits"]).cuda(),
                                 torch.from_numpy(GOLDEN["sel_bias"]).cuda(), 8)
    np.testing.assert_array_equal(inds.cpu().numpy(), GOLDEN["sel_inds"])
    np.testing.assert_array_equal(w.cpu().numpy(), GOLDEN["sel_w"])
    got = group_routes(GOLDEN["tiny_inds"], GOLDEN["tiny_w"], R=8, n_slots=mg.TINY["E"])
    for g, key in zip(got, ("tiny_uids", "tiny_urows", "tiny_ucnt", "tiny_uw", "tiny_gidx")):
        ref = GOLDEN[key]
        np.testing.assert_array_equal(g.cpu().numpy(), ref.astype(g.cpu().numpy().dtype), err_msg=key)
    perm, offsets, inv = prefill_dispatch(torch.from_numpy(GOLDEN["disp_slots"]).cuda(), 8)
    np.testing.assert_array_equal(perm.cpu().numpy(), GOLDEN["disp_perm"])
    np.testing.assert_array_equal(offsets.cpu().numpy(), GOLDEN["disp_offsets"])
    np.testing.assert_array_equal(inv.cpu().numpy(), GOLDEN["disp_inv"])


@pytest.mark.gpu
def test_gpu_tiny_block_outputs():
    import torch
    from mimo_stream import group_routes, moe_experts
    blk, bank = _tiny_block()
    x = _x()
    # the full block (router + experts) on the 4 rows: the distinct-expert path
    y, inds, _ = blk(x, return_routes=True)
    np.testing.assert_array_equal(inds.cpu().numpy(), GOLDEN["tiny_inds"])
    assert_bf16_close(y.float().cpu().numpy(), f32(GOLDEN["tiny_y_small"]), what="tiny block y")
    # the same routes through moe_experts with the golden grouping
    uids, urows, ucnt, uw, gidx = group_routes(GOLDEN["tiny_inds"], GOLDEN["tiny_w"], R=8, n_slots=mg.TINY["E"])
    y2 = moe_experts(x, bank, uids, urows, ucnt, uw, R=8, gather_idx=gidx)
    assert_bf16_close(y2.float().cpu().numpy(), f32(GOLDEN["tiny_y_small"]), what="tiny moe_experts y")
    # one row at a time: the M = 1 path (each expert output rounded to bf16)
    for t in range(mg.TINY["T"]):
        yt = blk(x[t:t + 1])
        assert_bf16_close(yt.float().cpu().numpy()[0], f32(GOLDEN["tiny_y_m1"])[t], what=f"tiny row {t}")
    # prefill with the golden routes
    yp = blk._moe_prefill(x, torch.from_numpy(GOLDEN["tiny_inds"]).cuda(), torch.from_numpy(GOLDEN["tiny_w"]).cuda())
    assert_bf16_close(yp.float().cpu().numpy(), f32(GOLDEN["tiny_y_prefill"]), what="tiny prefill y")
