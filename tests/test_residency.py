"""Layers with fewer HBM slots than experts (engine/mimo_stream/model.py:184-219, :230-271): experts read from
the checkpoint into the slots the decayed-LFU cache frees, on a side stream ordered against the compute stream.
The outputs must equal a fully resident layer's bit for bit (the same expert bytes and the same kernels)."""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H, I, N = 4096, 2048, 16


@pytest.fixture(scope="module")
def layer(tmp_path_factory):
    from safetensors.torch import save_file
    from mimo_stream import pools, store
    d = tmp_path_factory.mktemp("ckpt")
    bank = pools.random_bank(N, seed=21, hidden=H, inter=I)
    store.write_expert_layer(store.expert_file(d, 5), 5, bank)
    g = torch.Generator().manual_seed(8)
    wn, bn = store.router_names(5)
    save_file({wn: (torch.randn(N, H, generator=g) * 0.02).to(torch.bfloat16), bn: torch.zeros(N)},
              os.path.join(d, "dense.safetensors"))
    return d


def test_decode_steps_load_missing_experts(layer):
    from mimo_stream import store
    from mimo_stream.residency import StreamedMoEBlock
    full = store.load_block(layer, 5)
    st = store.ExpertStore(layer, [5])
    blk = StreamedMoEBlock(st, 5, n_slots=10, order=list(range(N))[::-1], decay_every=4)
    g = torch.Generator().manual_seed(3)
    for step in range(24):
        x = (torch.randn(1, H, generator=g) * (1 + step % 3)).to(torch.bfloat16).cuda()
        y, inds, _ = blk(x, return_routes=True)
        y2, inds2, _ = full(x, return_routes=True)
        assert torch.equal(inds, inds2), step
        assert torch.equal(y, y2), step
        res = set(np.nonzero(blk.cache.slot_of >= 0)[0])
        assert set(inds.cpu().numpy().reshape(-1)) <= res
    assert blk.cache.misses > 0 and blk.experts_read == blk.cache.misses
    for k in full.bank:                                     # every resident slot holds its expert's bytes
        for s, e in enumerate(blk.cache.expert_in):
            assert torch.equal(blk.block.bank[k][s], full.bank[k][e]), (k, s, e)


def test_prefill_with_non_resident_experts(layer):
    from mimo_stream import store
    from mimo_stream.residency import StreamedMoEBlock
    full = store.load_block(layer, 5)
    st = store.ExpertStore(layer, [5])
    blk = StreamedMoEBlock(st, 5, n_slots=9)
    g = torch.Generator().manual_seed(4)
    for T in (40, 300):
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).cuda()
        before = blk.cache.slot_of.copy()
        read0 = blk.experts_read
        _, inds, _ = full(x, return_routes=True)
        missing = set(inds.cpu().numpy().reshape(-1)) - set(np.nonzero(before >= 0)[0])
        assert torch.equal(blk(x), full(x)), T
        assert np.array_equal(blk.cache.slot_of, before)      # prefill leaves the resident set as it was
        assert blk.experts_read - read0 == len(missing)        # only the missing experts are staged
    # the block's own two staging banks of E - S slots, taken in turn by the two prefills
    from mimo_stream import pools
    assert blk.staging.n == N - 9 and blk.staging.nbytes() == 2 * (N - 9) * pools.expert_bytes(H, I)


def test_streamed_layers_share_two_staging_banks(layer):
    """Several streamed layers with one StagingBanks (model.py:140-143): the device memory they hold is their
    resident slots plus two banks of E - S slots, not a staging bank per layer; prefetch_stage streams a layer's
    non-resident experts ahead of its prefill, and a prefetch whose bank another layer has refilled since is
    staged again."""
    from mimo_stream import _lib, pools, store
    from mimo_stream.residency import StagingBanks, StreamedMoEBlock
    full = store.load_block(layer, 5)
    st = store.ExpertStore(layer, [5])
    eb = pools.expert_bytes(H, I)
    S, T, n_layers = 10, 300, 3
    g = torch.Generator().manual_seed(12)
    xs = [torch.randn(T, H, generator=g).to(torch.bfloat16).cuda() for _ in range(n_layers)]
    want = [full(x) for x in xs]
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    staging = StagingBanks(N - S, H, I)
    orders = [list(range(j, N)) + list(range(j)) for j in (0, 3, 6)]   # different resident sets per layer
    blks = [StreamedMoEBlock(st, 5, n_slots=S, order=o, staging=staging) for o in orders]
    ys = [blk(x) for blk, x in zip(blks, xs)]
    torch.cuda.synchronize()
    grown = torch.cuda.memory_allocated() - base
    for y, y2 in zip(ys, want):
        assert torch.equal(y, y2)
    resident = sum(sum(t.numel() * t.element_size() for t in b.block.bank.values()) for b in blks)
    assert resident == n_layers * S * eb
    assert staging.nbytes() == 2 * (N - S) * eb
    # what the layers may hold: resident slots, the two shared banks, routers, outputs, the prefill workspace and
    # small tables.  A staging bank of its own per layer would add n_layers * (N - S) * eb more.
    ws = _lib.load().mimo_moe_prefill_workspace_size(T, 8, N, H, I)
    bound = resident + staging.nbytes() + n_layers * (N * H * 2 + N * 4 + T * H * 2) + ws + (8 << 20)
    assert resident + staging.nbytes() <= grown <= bound, (grown, bound)
    assert bound < resident + n_layers * (N - S) * eb
    # prefetch_stage: the prefill then reads nothing more
    assert blks[0].prefetch_stage() == N - S
    read = blks[0].experts_read
    assert torch.equal(blks[0](xs[0]), want[0]) and blks[0].experts_read == read
    # three prefetches take the two banks in turn, so blks[2]'s refills the bank of blks[0]'s: blks[2] and blks[1]
    # read nothing at their prefill, blks[0] stages its missing experts again
    for blk in blks:
        assert blk.prefetch_stage() == N - S
    read = [b.experts_read for b in blks]
    for j in (2, 1, 0):
        assert torch.equal(blks[j](xs[j]), want[j]), j
    assert blks[2].experts_read == read[2] and blks[1].experts_read == read[1] and blks[0].experts_read > read[0]
    assert torch.cuda.memory_allocated() - base <= bound


def test_step_needing_more_experts_than_slots(layer):
    from mimo_stream import store
    from mimo_stream.residency import StreamedMoEBlock
    st = store.ExpertStore(layer, [5])
    blk = StreamedMoEBlock(st, 5, n_slots=8)
    W = blk.block.router.weight.float()
    Wn = W / W.norm(dim=1, keepdim=True)
    x = torch.stack([6 * Wn[:8].sum(0), 6 * Wn[8:].sum(0)]).to(torch.bfloat16)   # rows steered to disjoint halves
    _, inds, _ = store.load_block(layer, 5)(x, return_routes=True)
    assert len(set(inds.cpu().numpy().reshape(-1))) > 8
    with pytest.raises(ValueError):
        blk(x)
