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


def test_prefill_from_two_host_threads_on_two_streams(rng):
    """Two host threads run prefills of different inputs on two streams of the same device at once: the narrow
    tiles of both share the library's side stream, and each call's fork and join must wait on its own stream's
    work only, so both results equal the single-threaded ones."""
    import threading
    from mimo_stream import pools, Router, MoEBlock
    H, I, E, k = 4096, 2048, 64, 8
    bank = pools.random_bank(E, seed=78, hidden=H, inter=I)
    r = Router(H, E, k)
    r.weight.copy_(to_dev_bf16(rand_bf16(rng, (E, H), 0.02)))
    blocks = [MoEBlock(r, bank), MoEBlock(r, bank)]       # separate status words; same weights
    T = 300
    xs = [to_dev_bf16(rand_bf16(rng, (T, H))) for _ in range(2)]
    routes = [torch.from_numpy(zipf_routes(rng, T, E, k)).cuda() for _ in range(2)]
    ws = [torch.from_numpy(rng.random((T, k)).astype(np.float32)).cuda() for _ in range(2)]
    want = [blocks[i]._moe_prefill(xs[i], routes[i], ws[i]) for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got = [[None] * 4, [None] * 4]
    errors = []

    def run(i):
        try:
            with torch.cuda.stream(streams[i]):
                for rep in range(4):
                    got[i][rep] = blocks[i]._moe_prefill(xs[i], routes[i], ws[i])
            streams[i].synchronize()
        except Exception as e:          # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        for rep in range(4):
            assert torch.equal(got[i][rep], want[i]), (i, rep)
