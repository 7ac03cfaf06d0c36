"""GPU prefill parity: grouped MXFP4 GEMMs over slot-sorted routes and the fixed-order combine."""
import numpy as np
import pytest
import torch

from oracle import experts as ox, routing as orr
from helpers import assert_bf16_close, bf16_np, pool_np, rand_bf16, to_dev_bf16, zipf_routes

pytestmark = pytest.mark.gpu
# Prefill rounds every expert output to bf16 before weighting (model.py:228, :270): one fp32-order rounding
# flip of the largest output moves it by one bf16 ulp (2^-8 relative), plus the final bf16 rounding of y
# (2^-9): the bar is 1e-2 of max|y|.
TOL = 1e-2


def _block(rng, bank, H, E, k):
    from mimo_stream import Router, MoEBlock
    r = Router(H, E, k)
    r.weight.copy_(to_dev_bf16(rand_bf16(rng, (E, H), 0.02)))
    return MoEBlock(r, bank)


def test_prefill_tiny_all_tokens(rng):
    from mimo_stream import pools
    bank = pools.random_bank(8, seed=21, hidden=256, inter=512)
    pool = pool_np(bank)
    blk = _block(rng, bank, 256, 8, 2)
    T = 100
    x = rand_bf16(rng, (T, 256))
    inds = zipf_routes(rng, T, 8, 2)
    w = rng.random((T, 2)).astype(np.float32)
    y = blk._moe_prefill(to_dev_bf16(x), torch.from_numpy(inds).cuda(), torch.from_numpy(w).cuda())
    oy = ox.moe_prefill(x, pool, inds, w)
    assert_bf16_close(bf16_np(y), oy, what="prefill tiny")


@pytest.fixture(scope="module")
def full_pool():
    from mimo_stream import pools
    return pools.random_bank(256, seed=31)


@pytest.mark.parametrize("T", [512, 2048])
def test_prefill_mimo_shape_sampled_tokens(rng, full_pool, T):
    bank = full_pool
    blk = _block(rng, bank, 4096, 256, 8)
    x = rand_bf16(rng, (T, 4096))
    inds = zipf_routes(rng, T, 256, 8)
    w = rng.random((T, 8)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    y = blk._moe_prefill(to_dev_bf16(x), torch.from_numpy(inds).cuda(), torch.from_numpy(w).cuda())
    yn = bf16_np(y)
    sample = rng.choice(T, 3, replace=False)
    need = np.unique(inds[sample])
    sub = {k: v[torch.from_numpy(need).long().cuda()] for k, v in bank.items()}
    pool = pool_np(sub)
    remap = {int(e): i for i, e in enumerate(need)}
    for t in sample:
        slots = np.array([remap[int(e)] for e in inds[t]])
        oy = ox.gather_m1(x[t], pool, slots, w[t])
        assert_bf16_close(yn[t], oy, what=f"prefill token {t}")
    y2 = blk._moe_prefill(to_dev_bf16(x), torch.from_numpy(inds).cuda(), torch.from_numpy(w).cuda())
    assert torch.equal(y, y2), "run-to-run bit-identical"


def test_prefill_block_router_and_decode_consistency(rng, full_pool):
    """Router + prefill on a 16-token chunk vs the M = 1 decode path of each token (same math: bf16 expert
    outputs, fixed-order weighted sum), compared within tolerance: the chunk router and the small-batch router
    sum the 4096 logit products in different fp32 orders, and the expert GEMMs split K differently."""
    bank = full_pool
    blk = _block(rng, bank, 4096, 256, 8)
    T = 16
    x = to_dev_bf16(rand_bf16(rng, (T, 4096)))
    y, inds, w = blk(x, return_routes=True)
    for t in range(0, T, 5):
        yt, it, wt = blk(x[t:t + 1], return_routes=True)
        assert torch.equal(it[0], inds[t])
        torch.testing.assert_close(wt[0], w[t], rtol=1e-5, atol=1e-7)
        assert_bf16_close(bf16_np(y[t]), bf16_np(yt[0]), what=f"decode vs prefill token {t}")


@pytest.mark.parametrize("S0", [1, 100, 255])
def test_prefill_staged_split_bank_equals_one_bank(rng, full_pool, S0):
    """mimo_moe_prefill_staged over a bank of the first S0 slots and a staging bank of the rest (slot ids
    unchanged) gives mimo_moe_prefill's y on the whole bank bit for bit: the tiles of slots below S0 read the
    first bank, the others the second at slot - S0, including a tile whose slot is the first staged one."""
    from mimo_stream import _lib, pools
    T, k, H, I = 1024, 8, 4096, 2048
    x = to_dev_bf16(rand_bf16(rng, (T, H)))
    inds = torch.from_numpy(zipf_routes(rng, T, 256, k)).cuda()
    w = torch.from_numpy(rng.random((T, k)).astype(np.float32)).cuda()
    want = _block(rng, full_pool, H, 256, k)._moe_prefill(x, inds, w)
    first = {n: t[:S0] for n, t in full_pool.items()}
    rest = {n: t[S0:] for n, t in full_pool.items()}
    y = torch.empty_like(want)
    status = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    nb = _lib.load().mimo_moe_prefill_workspace_size(T, k, 256, H, I)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    _lib.call("mimo_moe_prefill_staged", _lib.ptr(x), T, _lib.ptr(inds), _lib.ptr(w), k, pools.bank_struct(first),
              pools.bank_struct(rest), _lib.ptr(y), _lib.ptr(status), _lib.ptr(ws), nb, _lib.stream_ptr())
    assert int(status.item()) == 0
    assert torch.equal(y, want)
    # a slot id past both banks is flagged
    bad = inds.clone()
    bad[3, 2] = 256
    _lib.call("mimo_moe_prefill_staged", _lib.ptr(x), T, _lib.ptr(bad), _lib.ptr(w), k, pools.bank_struct(first),
              pools.bank_struct(rest), _lib.ptr(y), _lib.ptr(status), _lib.ptr(ws), nb, _lib.stream_ptr())
    assert int(status.item()) != 0
