"""GPU routing parity: selection given logits (bit-exact), router logits (tolerance), group_routes and the
prefill dispatch (bit-exact)."""
import numpy as np
import pytest
import torch

from oracle import routing as orr, mxfp4 as oq
from helpers import shared_routes, to_dev_bf16, zipf_routes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,E,k", [(1, 256, 8), (8, 256, 8), (2048, 256, 8), (4, 8, 2), (3, 1024, 16)])
def test_select_from_logits_bit_exact(rng, T, E, k):
    from mimo_stream import select_from_logits
    logits = (rng.standard_normal((T, E)) * 3).astype(np.float32)
    logits[0, :4] = logits[0, 4]              # exact ties
    logits[-1, 5] = np.float32(120.0)         # saturating sigmoid
    bias = (rng.standard_normal(E) * 1e-2).astype(np.float32)
    bias[:3] = 0.0
    inds, w = select_from_logits(torch.from_numpy(logits).cuda(), torch.from_numpy(bias).cuda(), k)
    oi, ow = orr.select_topk(logits, bias, k)
    np.testing.assert_array_equal(inds.cpu().numpy(), oi)
    np.testing.assert_array_equal(w.cpu().numpy(), ow)


def test_router_logits_and_routes(rng):
    from mimo_stream import Router
    T, H, E, k = 8, 4096, 256, 8
    x = oq.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    W = oq.round_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(E) * 1e-3).astype(np.float32)
    r = Router(H, E, k)
    r.weight.copy_(to_dev_bf16(W))
    r.e_score_correction_bias.copy_(torch.from_numpy(bias))
    logits, inds, w = r.logits_and_routes(to_dev_bf16(x))
    lg = logits.cpu().numpy()
    ref = orr.router_logits(x, W)
    assert np.abs(lg - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-6   # fp32 accumulation order only
    oi, ow = orr.select_topk(lg, bias, k)                               # bit-exact given the same logits
    np.testing.assert_array_equal(inds.cpu().numpy(), oi)
    np.testing.assert_array_equal(w.cpu().numpy(), ow)
    # the same through the prefill-sized path (tiled logits kernel)
    X = oq.round_bf16(rng.standard_normal((300, H)).astype(np.float32))
    logits2, inds2, w2 = r.logits_and_routes(to_dev_bf16(X))
    ref2 = orr.router_logits(X, W)
    assert np.abs(logits2.cpu().numpy() - ref2).max() <= 1e-5 * np.abs(ref2).max() + 1e-6
    oi2, ow2 = orr.select_topk(logits2.cpu().numpy(), bias, k)
    np.testing.assert_array_equal(inds2.cpu().numpy(), oi2)
    np.testing.assert_array_equal(w2.cpu().numpy(), ow2)


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_group_routes_bit_exact(rng, M):
    from mimo_stream import group_routes
    inds = shared_routes(rng, M, 24, 8)
    scores = rng.random((M, 8)).astype(np.float32)
    got = group_routes(inds, scores, R=8, n_slots=24)
    ref = orr.group_routes(inds, scores, R=8)
    for g, r in zip(got, ref):
        np.testing.assert_array_equal(g.cpu().numpy(), r.astype(g.cpu().numpy().dtype))


def test_group_routes_slot_table_and_overflow(rng):
    from mimo_stream import group_routes
    slot_of = np.full(32, -1, np.int32)
    slot_of[rng.permutation(32)[:16]] = np.arange(16)
    experts = np.nonzero(slot_of >= 0)[0]
    inds = np.stack([rng.choice(experts, 4, replace=False) for _ in range(3)]).astype(np.int32)
    scores = rng.random((3, 4)).astype(np.float32)
    got = group_routes(inds, scores, R=8, slot_of=slot_of, n_slots=16)
    ref = orr.group_routes(slot_of[inds], scores, R=8)
    for g, r in zip(got, ref):
        np.testing.assert_array_equal(g.cpu().numpy(), r.astype(g.cpu().numpy().dtype))
    with pytest.raises(ValueError):
        group_routes(np.zeros((3, 2), np.int32), np.ones((3, 2), np.float32), R=2, n_slots=4)
    bad = inds.copy()
    bad[0, 0] = int(np.nonzero(slot_of < 0)[0][0])
    with pytest.raises(ValueError):
        group_routes(bad, scores, R=8, slot_of=slot_of, n_slots=16)


@pytest.mark.parametrize("T,S,k", [(512, 256, 8), (2048, 256, 8), (4096, 256, 8), (5, 8, 2), (1, 256, 8),
                                   (300, 1024, 8), (1000, 1000, 3), (3000, 512, 8)])
def test_prefill_dispatch_bit_exact(rng, T, S, k):
    """Stable counting sort against the oracle; the last three cases take the largest slot count (1024), a slot
    count that is not a power of two and ragged chunks (T * k not a multiple of the 1024-route chunk)."""
    from mimo_stream import prefill_dispatch
    slots = zipf_routes(rng, T, S, k)
    perm, offsets, inv = prefill_dispatch(torch.from_numpy(slots).cuda(), S)
    operm, ooff, oinv = orr.prefill_dispatch(slots, S)
    np.testing.assert_array_equal(perm.cpu().numpy(), operm)
    np.testing.assert_array_equal(offsets.cpu().numpy(), ooff)
    np.testing.assert_array_equal(inv.cpu().numpy(), oinv)
