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
        assert torch.equal(blk(x), full(x)), T
        assert np.array_equal(blk.cache.slot_of, before)      # prefill leaves the resident set as it was


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
