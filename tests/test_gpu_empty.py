"""Empty batches through the Python API: zero rows give correctly shaped empty outputs (the oracle's group_routes
of no routes is empty too) and launch nothing; a call on real rows afterwards is unaffected."""
import numpy as np
import pytest
import torch

from helpers import rand_bf16, to_dev_bf16
from oracle import routing as orr

pytestmark = pytest.mark.gpu

H, I, E, K = 512, 512, 16, 4


@pytest.fixture(scope="module")
def block():
    from mimo_stream import MoEBlock, Router, pools
    rng = np.random.default_rng(9)
    bank = pools.random_bank(E, seed=9, hidden=H, inter=I)
    r = Router(H, E, K)
    r.weight.copy_(to_dev_bf16(rand_bf16(rng, (E, H), 0.02)))
    return MoEBlock(r, bank)


def test_empty_batch_block_router_and_kernels(block):
    from mimo_stream import kernels
    x0 = torch.empty((0, H), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    y, inds, w = block(x0, return_routes=True)
    assert y.shape == (0, H) and y.dtype == torch.bfloat16
    assert inds.shape == (0, K) and w.shape == (0, K)
    logits, i2, w2 = block.router.logits_and_routes(x0)
    assert logits.shape == (0, E) and i2.shape == (0, K) and w2.shape == (0, K)
    e_inds = torch.empty((0, K), dtype=torch.int32, device="cuda")
    e_w = torch.empty((0, K), dtype=torch.float32, device="cuda")
    assert block._moe_small(x0, e_inds, e_w).shape == (0, H)
    assert block._moe_prefill(x0, e_inds, e_w).shape == (0, H)
    uids, urows, ucnt, uw, gidx = kernels.group_routes(e_inds, e_w, R=8, n_slots=E)
    ref = orr.group_routes(np.zeros((0, K), np.int32), np.zeros((0, K), np.float32), R=8)
    for got, want in zip((uids, urows, ucnt, uw, gidx), ref):
        assert tuple(got.shape) == tuple(np.asarray(want).shape)
    ye, he, pe = kernels.moe_experts(x0, block.bank, uids, urows, ucnt, uw, R=8, gather_idx=gidx,
                                     return_intermediates=True)
    assert ye.shape == (0, H) and he.shape == (0, 8, I) and pe.shape == (0, 8, H)
    # the block still works on real rows after the empty calls
    x = to_dev_bf16(rand_bf16(np.random.default_rng(1), (3, H)))
    y1 = block(x)
    y2 = block(x)
    torch.cuda.synchronize()
    assert y1.shape == (3, H) and torch.equal(y1, y2) and torch.isfinite(y1.float()).all()


def test_empty_batch_layer(block):
    from mimo_stream import MoELayer
    layer = MoELayer(block, torch.ones(H), 1e-6)
    x0 = torch.empty((0, H), dtype=torch.bfloat16, device="cuda")
    h, inds, w, r = layer(x0, return_routes=True, return_norm=True)
    assert h.shape == (0, H) and inds.shape == (0, K) and w.shape == (0, K) and r.shape == (0, H)
    assert layer.norm(x0).shape == (0, H)
    x3 = torch.empty((2, 0, H), dtype=torch.bfloat16, device="cuda")   # leading dims kept
    assert layer(x3).shape == (2, 0, H)
