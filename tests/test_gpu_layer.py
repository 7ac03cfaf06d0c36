"""The MoE half of a decoder layer on the GPU (engine/mimo_stream/model.py:296-340): post-attention RMSNorm,
the block, h = x + y; the next-layer route prediction and prefetch (:305-329); decode vs prefill through a
stack of layers (engine/tests/test_parity.py:99-110 at the MoE level).

Bars: the norm and the residual bit-exact against the oracle; the fused layer entry points bit-identical to the
unfused composition (mimo_rmsnorm, the block, mimo_residual_add); routes bit-exact; a streamed layer
bit-identical to the resident one; decode vs prefill within the block tests' bf16 tolerance."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bf16_bits, rand_bf16, to_dev_bf16
from oracle import layer as ol, routing as orr
from oracle.mxfp4 import bf16_bits_to_f32, f32_to_bf16_bits

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _dev_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).cuda().view(torch.bfloat16)


def _layer(rng, H, I, E, k, seed):
    from mimo_stream import MoEBlock, MoELayer, Router, pools
    bank = pools.random_bank(E, seed=seed, hidden=H, inter=I)
    r = Router(H, E, k)
    W = rand_bf16(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * 1e-3).astype(np.float32)
    r.weight.copy_(to_dev_bf16(W))
    r.e_score_correction_bias.copy_(torch.from_numpy(bias))
    nw = to_dev_bf16(rand_bf16(rng, (H,), 0.2) + 1.0)
    return MoELayer(MoEBlock(r, bank), nw, EPS), bank, W, bias


def test_rmsnorm_and_residual_bit_exact(rng):
    from mimo_stream import _lib
    for H in (256, 1024, 2560, 4096, 6144, 8192):    # one to four 8-element chunks per thread, partial chunks
        x = rand_bf16(rng, (7, H)) * np.array([1e-3, 0.1, 1, 1, 3, 50, 1e3], np.float32)[:, None]
        x[1] = 0.0                       # zero row
        x[2] = 1.5                       # constant row
        xb = f32_to_bf16_bits(x)
        wb = f32_to_bf16_bits(rand_bf16(rng, (H,), 0.3) + 1.0)
        r = torch.empty(7, H, dtype=torch.bfloat16, device="cuda")
        xd, wd = _dev_bits(xb), _dev_bits(wb)        # held: a temporary's memory could be reused by the next one
        _lib.call("mimo_rmsnorm", _lib.ptr(xd), 7, H, _lib.ptr(wd), EPS, _lib.ptr(r), _lib.stream_ptr())
        np.testing.assert_array_equal(bf16_bits(r), ol.rmsnorm(xb, wb, EPS))
    for n in (8, 4096 * 3, 1000, 13):
        xb = f32_to_bf16_bits(rand_bf16(rng, (n,)))
        yb = f32_to_bf16_bits(rand_bf16(rng, (n,), 0.05))
        xd, yd = _dev_bits(xb), _dev_bits(yb)
        h = torch.empty(n, dtype=torch.bfloat16, device="cuda")
        _lib.call("mimo_residual_add", _lib.ptr(xd), _lib.ptr(yd), n, _lib.ptr(h), _lib.stream_ptr())
        np.testing.assert_array_equal(bf16_bits(h), ol.residual_add(xb, yb))
        _lib.call("mimo_residual_add", _lib.ptr(xd), _lib.ptr(yd), n, _lib.ptr(xd), _lib.stream_ptr())   # h = x
        np.testing.assert_array_equal(bf16_bits(xd), ol.residual_add(xb, yb))


def test_rmsnorm_rejects_bad_shapes():
    from mimo_stream import _lib
    x = torch.zeros(2, 300, dtype=torch.bfloat16, device="cuda")
    w = torch.ones(300, dtype=torch.bfloat16, device="cuda")
    r = torch.empty_like(x)
    with pytest.raises(ValueError):
        _lib.call("mimo_rmsnorm", _lib.ptr(x), 2, 300, _lib.ptr(w), EPS, _lib.ptr(r), _lib.stream_ptr())
    # the kernel reads 16-byte chunks: rows that are not 16-byte aligned are refused before any launch
    xf = torch.zeros(2 * 256 + 8, dtype=torch.bfloat16, device="cuda")
    w2 = torch.ones(256, dtype=torch.bfloat16, device="cuda")
    r2 = torch.empty(2, 256, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        _lib.call("mimo_rmsnorm", _lib.ptr(xf[1:]), 2, 256, _lib.ptr(w2), EPS, _lib.ptr(r2), _lib.stream_ptr())


@pytest.mark.parametrize("T,shape", [(1, "mimo"), (3, "mimo"), (8, "mimo"), (40, "mimo"), (1, "tiny"), (4, "tiny")])
def test_layer_fused_equals_composition(rng, T, shape):
    """The layer entry point (norm inside the router kernel or its own kernel, block, residual in the combine) ==
    mimo_rmsnorm -> block -> residual add, bit for bit; r and the routes bit-exact against the oracle."""
    from mimo_stream import _lib
    H, I, E, k = (4096, 2048, 256, 8) if shape == "mimo" else (256, 512, 8, 2)
    layer, bank, W, bias = _layer(rng, H, I, E, k, seed=70 + T)
    x = to_dev_bf16(rand_bf16(rng, (T, H)))
    h, inds, w, r = layer(x, return_routes=True, return_norm=True)
    r_ref = layer.norm(x)
    assert torch.equal(r, r_ref)
    np.testing.assert_array_equal(bf16_bits(r), ol.rmsnorm(bf16_bits(x), bf16_bits(layer.norm_weight), EPS))
    y, inds2, w2 = layer.block(r_ref, return_routes=True)
    assert torch.equal(inds, inds2) and torch.equal(w, w2)
    h2 = torch.empty_like(x)
    _lib.call("mimo_residual_add", _lib.ptr(x), _lib.ptr(y), x.numel(), _lib.ptr(h2), _lib.stream_ptr())
    assert torch.equal(h, h2)
    # routes bit-exact given the router's logits (selection, renormalisation), logits within fp32 noise
    lg, _, _ = layer.block.router.logits_and_routes(r)
    lg = lg.cpu().numpy()
    ref = orr.router_logits(bf16_bits_to_f32(bf16_bits(r)), W)
    assert np.abs(lg - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-6
    oi, ow = orr.select_topk(lg, bias, k)
    np.testing.assert_array_equal(inds.cpu().numpy(), oi)
    np.testing.assert_array_equal(w.cpu().numpy(), ow)
    # in place through the C ABI: h may alias x
    blk, b = layer.block, layer.block._bank_struct
    xi = x.clone()
    args = (_lib.ptr(xi), T, _lib.ptr(layer.norm_weight), EPS, _lib.ptr(blk.router.weight),
            _lib.ptr(blk.router.e_score_correction_bias), None, E, k, b, _lib.ptr(xi), None, None, None, None)
    if T <= 8:
        nb = _lib.load().mimo_moe_layer_decode_workspace_size(T, E, k, H, I)
        ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
        _lib.call("mimo_moe_layer_decode", *args, _lib.ptr(ws), nb, _lib.stream_ptr())
    else:
        nb = _lib.load().mimo_moe_layer_prefill_workspace_size(T, E, k, E, H, I)
        ws = torch.zeros(nb, dtype=torch.uint8, device="cuda")
        _lib.call("mimo_moe_layer_prefill", *args, _lib.ptr(ws), nb, _lib.stream_ptr())
    assert torch.equal(xi, h)


def test_streamed_layer_matches_resident(rng, tmp_path):
    """A layer over a StreamedMoEBlock (norm, block with slot misses read from the checkpoint, residual add)
    gives the resident layer's h bit for bit; prediction and prefetch load the next step's experts ahead."""
    from mimo_stream import MoELayer, StreamedMoEBlock, store
    H, I, E, k = 4096, 2048, 32, 8
    layer, bank, W, bias = _layer(rng, H, I, E, k, seed=91)
    store.write_expert_layer(store.expert_file(tmp_path, 0), 0, bank)
    st = store.ExpertStore(tmp_path, [0])
    sblk = StreamedMoEBlock(st, 0, n_slots=20, router=layer.block.router)
    slayer = MoELayer(sblk, layer.norm_weight, EPS)
    for T in (1, 2, 20):          # a 2-row step needs at most 16 distinct experts: within the 20 slots
        x = to_dev_bf16(rand_bf16(rng, (T, H)))
        assert torch.equal(slayer(x), layer(x)), T
    # prediction: this layer's router on its norm of x (model.py:305-314)
    x = to_dev_bf16(rand_bf16(rng, (1, H)))
    pred = slayer.predict(x)
    r = layer.norm(x)
    ri, rw = layer.block.router(r)
    np.testing.assert_array_equal(pred, np.unique(ri.cpu().numpy()))
    top3 = slayer.predict(x, top=3)
    order = np.argsort(-rw.cpu().numpy()[-1], kind="stable")[:3]
    np.testing.assert_array_equal(top3, np.unique(ri.cpu().numpy()[-1][order]))
    # prefetch: misses are read now, without counting as uses or as cache hits / misses
    c = sblk.cache
    cnt0, hits0, miss0 = c.cnt.copy(), c.hits, c.misses
    read0 = sblk.experts_read
    n = slayer.prefetch(pred)
    assert sblk.experts_read == read0 + n and (c.slot_of[pred] >= 0).all()
    np.testing.assert_array_equal(c.cnt, cnt0)
    assert (c.hits, c.misses) == (hits0, miss0)
    # the step itself then needs no reads and still matches the resident layer
    read1 = sblk.experts_read
    assert torch.equal(slayer(x), layer(x))
    assert sblk.experts_read == read1


def test_decode_vs_prefill_through_a_layer_stack(rng):
    """Three layers chained h = L3(L2(L1(x))) over 12 tokens: one prefill chunk vs each token decoded alone
    (the MoE part of engine/tests/test_parity.py:99-110; attention is out of scope, so tokens are independent)."""
    H, I, E, k = 4096, 2048, 256, 8
    layers = [_layer(rng, H, I, E, k, seed=120 + j)[0] for j in range(3)]
    x = to_dev_bf16(rand_bf16(rng, (12, H)))
    hp = x
    for L in layers:
        hp = L(hp)
    hd = []
    for t in range(12):
        h = x[t:t + 1]
        for L in layers:
            h = L(h)
        hd.append(h)
    hd = torch.cat(hd)
    assert_bf16_close(hd.float().cpu().numpy(), hp.float().cpu().numpy(), what="decode vs prefill, 3 layers")


@pytest.mark.parametrize("H,I,E,k", [(512, 1024, 16, 3), (1024, 512, 32, 4), (2048, 1024, 64, 6)])
def test_layer_decode_other_hidden_sizes(rng, H, I, E, k):
    """The router kernel's own norm at hidden sizes where a wave holds partial chunk sets (H / 4 < 512): the
    layer step equals mimo_rmsnorm -> block -> residual add bit for bit, and r equals the oracle's norm."""
    from mimo_stream import _lib
    layer, bank, W, bias = _layer(rng, H, I, E, k, seed=H + E)
    for T in (1, 2, 5):
        x = to_dev_bf16(rand_bf16(rng, (T, H)))
        h, inds, w, r = layer(x, return_routes=True, return_norm=True)
        np.testing.assert_array_equal(bf16_bits(r), ol.rmsnorm(bf16_bits(x), bf16_bits(layer.norm_weight), EPS))
        y, inds2, w2 = layer.block(layer.norm(x), return_routes=True)
        assert torch.equal(inds, inds2) and torch.equal(w, w2)
        h2 = torch.empty_like(x)
        _lib.call("mimo_residual_add", _lib.ptr(x), _lib.ptr(y), x.numel(), _lib.ptr(h2), _lib.stream_ptr())
        assert torch.equal(h, h2), (H, T)
