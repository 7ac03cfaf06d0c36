"""mimo_moe_layer_decode_noalloc (the layer decode step with the library's own per-GPU scratch instead of a caller
workspace) gives the bits of mimo_moe_layer_decode with a workspace: h, r, the routes and the status, on calls in
a row whose batches shrink (the scratch keeps the previous call's contents), at the MiMo layer shape and the tiny
one, with a slot table that leaves an expert out (status reported)."""
import numpy as np
import pytest
import torch

from helpers import rand_bf16, to_dev_bf16

pytestmark = pytest.mark.gpu


def _layer(rng, H, I, E, k, seed):
    from mimo_stream import pools
    bank = pools.random_bank(E, seed=seed, hidden=H, inter=I)
    W = to_dev_bf16(rand_bf16(rng, (E, H), 0.02))
    bias = torch.from_numpy((rng.standard_normal(E) * 1e-3).astype(np.float32)).cuda()
    nw = to_dev_bf16(rand_bf16(rng, (H,), 0.2) + 1.0)
    return bank, W, bias, nw


def _run(noalloc, x, M, nw, W, bias, slot_of, E, k, b, H):
    from mimo_stream import _lib
    dev = x.device
    h = torch.full((M, H), 7.0, dtype=torch.bfloat16, device=dev)
    r = torch.full((M, H), 7.0, dtype=torch.bfloat16, device=dev)
    inds = torch.full((M, k), -5, dtype=torch.int32, device=dev)
    w = torch.full((M, k), -5.0, dtype=torch.float32, device=dev)
    st = torch.full((1,), 99, dtype=torch.int32, device=dev)
    head = (_lib.ptr(x), M, _lib.ptr(nw), 1e-6, _lib.ptr(W), _lib.ptr(bias), _lib.ptr(slot_of), E, k, b,
            _lib.ptr(h), _lib.ptr(r), _lib.ptr(inds), _lib.ptr(w), _lib.ptr(st))
    if noalloc:
        _lib.call("mimo_moe_layer_decode_noalloc", *head, _lib.stream_ptr(dev))
    else:
        nb = _lib.load().mimo_moe_layer_decode_workspace_size(M, E, k, b.hidden, b.inter)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        _lib.call("mimo_moe_layer_decode", *head, _lib.ptr(ws), nb, _lib.stream_ptr(dev))
    torch.cuda.synchronize()
    return h, r, inds, w, int(st.item())


@pytest.mark.parametrize("shape", ["mimo", "tiny"])
def test_noalloc_matches_workspace_entry_point(rng, shape):
    from mimo_stream import pools
    H, I, E, k = (4096, 2048, 256, 8) if shape == "mimo" else (256, 512, 8, 2)
    bank, W, bias, nw = _layer(rng, H, I, E, k, seed=55)
    b = pools.bank_struct(bank)
    xs = to_dev_bf16(rand_bf16(rng, (8, H)))
    for M in (8, 3, 1):                       # shrinking batches: the scratch holds the larger call's data
        got = _run(True, xs[:M], M, nw, W, bias, None, E, k, b, H)
        ref = _run(False, xs[:M], M, nw, W, bias, None, E, k, b, H)
        for a, c in zip(got[:4], ref[:4]):
            assert torch.equal(a, c), (shape, M)
        assert got[4] == ref[4] == 0
    # a slot table with one selected expert left out: the status says so, as with a workspace
    h0, r0, inds0, w0, _ = _run(False, xs[:2], 2, nw, W, bias, None, E, k, b, H)
    tab = torch.arange(E, dtype=torch.int32, device="cuda")
    tab[int(inds0[0, 0])] = -1
    got = _run(True, xs[:2], 2, nw, W, bias, tab, E, k, b, H)
    ref = _run(False, xs[:2], 2, nw, W, bias, tab, E, k, b, H)
    assert got[4] == ref[4] != 0
    for a, c in zip(got[:4], ref[:4]):
        assert torch.equal(a, c)
