"""HIP graph capture of the MoE block: a prefill chunk (narrow tiles on the library's side stream, wide tiles
on the caller's stream, joined by events) and a one-row decode step, captured once and replayed several times
with eager work and synchronisations between replays; every replay must equal the eager result bit for bit."""
import numpy as np
import pytest
import torch

from helpers import rand_bf16, to_dev_bf16, zipf_routes

pytestmark = pytest.mark.gpu


def test_prefill_and_decode_graph_replays_match_eager(rng):
    from mimo_stream import pools, Router, MoEBlock
    H, I, E, k = 4096, 2048, 64, 8
    bank = pools.random_bank(E, seed=77, hidden=H, inter=I)
    r = Router(H, E, k)
    r.weight.copy_(to_dev_bf16(rand_bf16(rng, (E, H), 0.02)))
    blk = MoEBlock(r, bank)
    T = 300
    xp = to_dev_bf16(rand_bf16(rng, (T, H)))
    inds = torch.from_numpy(zipf_routes(rng, T, E, k)).cuda()
    counts = np.bincount(inds.cpu().numpy().reshape(-1), minlength=E)
    assert (counts > 64).any() and ((counts > 0) & (counts <= 32)).any()   # wide and narrow tiles both
    w = torch.from_numpy(rng.random((T, k)).astype(np.float32)).cuda()
    x1 = to_dev_bf16(rand_bf16(rng, (1, H)))
    want_p = blk._moe_prefill(xp, inds, w)          # eager, also sizes the cached workspaces
    want_b = blk(xp)
    want_d = blk(x1)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got_p = blk._moe_prefill(xp, inds, w)
        got_b = blk(xp)
        got_d = blk(x1)
    other = to_dev_bf16(rand_bf16(rng, (T, H)))
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got_p, want_p), rep
        assert torch.equal(got_b, want_b), rep
        assert torch.equal(got_d, want_d), rep
        blk(other)                                   # eager work on the same workspaces between replays
        blk._moe_prefill(other, inds, w)
        torch.cuda.synchronize()
