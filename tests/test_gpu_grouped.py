"""The vendored noaux-tc gate's options on the GPU (engine/mimo_stream/mimo_v2.py:165-216): group-limited selection,
norm_topk_prob and routed_scaling_factor, bit-exact against oracle.routing.select_topk_grouped given the same fp32
logits; a MoE block whose router carries those options routes through them.  Also MoEBlock.forward_residual."""
import numpy as np
import pytest
import torch

from helpers import bf16_bits, rand_bf16, to_dev_bf16
from oracle import layer as ol, routing as orr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,n_group,topk_group,k,norm,scale", [
    (256, 8, 4, 8, True, 1.0), (256, 8, 1, 8, True, 2.5), (64, 4, 2, 6, False, 1.0), (256, 1, 1, 8, False, 2.5),
    (64, 32, 5, 4, True, 1.0), (16, 4, 1, 2, True, 1.0), (256, 16, 3, 1, True, 1.0)])
def test_grouped_selection_bit_exact(rng, E, n_group, topk_group, k, norm, scale):
    from mimo_stream import _lib
    T = 37
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    lg[1, : E // 2] = lg[1, 0]                        # exact ties inside and across groups
    lg[2, 5] = np.nan
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
    if E == 16:
        bias[:] = -2.0                                # every kept key negative: masked keys (0.0) outrank them
    ld, bd = torch.from_numpy(lg).cuda(), torch.from_numpy(bias).cuda()
    inds = torch.empty(T, k, dtype=torch.int32, device="cuda")
    w = torch.empty(T, k, dtype=torch.float32, device="cuda")
    _lib.call("mimo_router_select_grouped", _lib.ptr(ld), _lib.ptr(bd), T, E, k, n_group, topk_group, int(norm),
              scale, _lib.ptr(inds), _lib.ptr(w), _lib.stream_ptr())
    oi, ow = orr.select_topk_grouped(lg, bias, k, n_group, topk_group, norm, scale)
    np.testing.assert_array_equal(inds.cpu().numpy(), oi)
    np.testing.assert_array_equal(w.cpu().numpy(), ow)


def test_grouped_selection_rejects_bad_groups():
    from mimo_stream import _lib
    ld = torch.zeros(2, 60, device="cuda")
    bd = torch.zeros(60, device="cuda")
    inds = torch.empty(2, 4, dtype=torch.int32, device="cuda")
    w = torch.empty(2, 4, device="cuda")
    for ng, tg in ((7, 2), (4, 5), (60, 1)):          # not dividing E, topk_group > n_group, groups of one
        with pytest.raises(ValueError):
            _lib.call("mimo_router_select_grouped", _lib.ptr(ld), _lib.ptr(bd), 2, 60, 4, ng, tg, 1, 1.0,
                      _lib.ptr(inds), _lib.ptr(w), _lib.stream_ptr())


def test_block_with_gate_options(rng):
    from mimo_stream import MoEBlock, MoELayer, Router, pools
    H, I, E, k = 1024, 512, 64, 6
    bank = pools.random_bank(E, seed=5, hidden=H, inter=I)
    r = Router(H, E, k, n_group=8, topk_group=3, norm_topk_prob=True, routed_scaling_factor=2.5)
    W = rand_bf16(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * 1e-2).astype(np.float32)
    r.weight.copy_(to_dev_bf16(W))
    r.e_score_correction_bias.copy_(torch.from_numpy(bias))
    blk = MoEBlock(r, bank)
    for T in (1, 3, 40):
        x = to_dev_bf16(rand_bf16(rng, (T, H)))
        y, inds, w = blk(x, return_routes=True)
        lg, _, _ = r.logits_and_routes(x)
        oi, ow = orr.select_topk_grouped(lg.cpu().numpy(), bias, k, 8, 3, True, 2.5)
        np.testing.assert_array_equal(inds.cpu().numpy(), oi)
        np.testing.assert_array_equal(w.cpu().numpy(), ow)
        y2 = blk._moe_small(x, inds, w) if T <= 8 else blk._moe_prefill(x, inds, w)
        assert torch.equal(y, y2)
        # the layer wrapper takes the unfused path for such a router and still adds the residual exactly
        nw = to_dev_bf16(rand_bf16(rng, (H,), 0.1) + 1.0)
        layer = MoELayer(blk, nw, 1e-5)
        h, li, lw, rr = layer(x, return_routes=True, return_norm=True)
        y3 = blk(rr)
        np.testing.assert_array_equal(bf16_bits(h), ol.residual_add(bf16_bits(x), bf16_bits(y3)))


def test_forward_residual(rng):
    from mimo_stream import MoEBlock, Router, pools
    H, I, E = 1024, 512, 32
    bank = pools.random_bank(E, seed=6, hidden=H, inter=I)
    r = Router(H, E, 4)
    r.weight.copy_(to_dev_bf16(rand_bf16(rng, (E, H), 0.02)))
    blk = MoEBlock(r, bank)
    for T in (2, 20):
        x = to_dev_bf16(rand_bf16(rng, (T, H)))
        rr = to_dev_bf16(rand_bf16(rng, (T, H)))
        h = blk.forward_residual(x, rr)
        np.testing.assert_array_equal(bf16_bits(h), ol.residual_add(bf16_bits(x), bf16_bits(blk(rr))))
