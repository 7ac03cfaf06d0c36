"""Device status of the fused entry points: a route to an expert that has no resident slot is reported (and the
Python blocks raise ValueError), never computed silently with another expert's weights.  The reference raises on
the same conditions (engine/mimo_stream/kernels.py:167-168) or loads the expert first (cache.py:45-46).

Every case routes a chosen expert through a large e_score_correction_bias, so the router is certain to select
it, and gives it no slot (slot_of entry -1 or n_slots) or only resident experts."""
import os

import numpy as np
import pytest
import torch

from mimo_stream import _lib, pools

pytestmark = pytest.mark.gpu
H, I, E, K = 256, 512, 16, 4
FORCED = 5                  # the expert every row selects


@pytest.fixture(scope="module")
def parts():
    bank = pools.random_bank(E, seed=31, hidden=H, inter=I)
    g = torch.Generator().manual_seed(31)
    W = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).cuda()
    bias = torch.zeros(E)
    bias[FORCED] = 10.0
    x = torch.randn(64, H, generator=g).to(torch.bfloat16).cuda()
    norm_w = (1.0 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).cuda()
    return bank, W, bias.cuda(), x, norm_w


def _tables():
    ident = torch.arange(E, dtype=torch.int32)
    missing = ident.clone()
    missing[FORCED] = -1
    beyond = ident.clone()
    beyond[FORCED] = E
    return {"identity": (ident.cuda(), _lib.MIMO_OK), "missing": (missing.cuda(), _lib.ERR_SLOT),
            "beyond": (beyond.cuda(), _lib.ERR_SLOT)}


def _status(fn):
    st = torch.full((1,), 12345, dtype=torch.int32, device="cuda")
    fn(st)
    torch.cuda.synchronize()
    return int(st.item())


def _ws(name, *size_args):
    nb = getattr(_lib.load(), name)(*size_args)
    return torch.empty(nb, dtype=torch.uint8, device="cuda"), nb


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_decode_status(parts, M):
    """With 16 experts and top-4 every batch here has at most 16 distinct experts (Umax = min(M k, E) <= 16), so
    the gate/up kernel's blocks select and group the routes themselves at every M (the one-row and two-row fast
    paths when no slot table is given); test_decode_status_selection_launch covers the separate selection
    launch."""
    bank, W, bias, x, _ = parts
    b = pools.bank_struct(bank)
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    ws, nb = _ws("mimo_moe_decode_workspace_size", M, E, K, H, I)
    for name, (tab, want) in _tables().items():
        def run(st):
            _lib.call("mimo_moe_decode", _lib.ptr(x[:M]), M, _lib.ptr(W), _lib.ptr(bias), _lib.ptr(tab), E, K, b,
                      _lib.ptr(y), None, None, _lib.ptr(st), _lib.ptr(ws), nb, _lib.stream_ptr())
        assert _status(run) == want, (name, M)
    # without a slot table (identity, the fast 1- and 2-row paths) the status is written too
    def run_none(st):
        _lib.call("mimo_moe_decode", _lib.ptr(x[:M]), M, _lib.ptr(W), _lib.ptr(bias), None, E, K, b, _lib.ptr(y),
                  None, None, _lib.ptr(st), _lib.ptr(ws), nb, _lib.stream_ptr())
    assert _status(run_none) == _lib.MIMO_OK


@pytest.mark.parametrize("M", [3, 8])
def test_decode_status_selection_launch(M):
    """Batches with more than 16 possible distinct experts (64 experts, top-8: Umax = min(M k, E) = 24 or 64)
    select and group their routes in the separate selection launch, which writes the status word there: OK,
    a selected expert missing from the slot table, and one mapped past the bank."""
    E2, K2 = 64, 8
    bank = pools.random_bank(E2, seed=37, hidden=H, inter=I)
    b = pools.bank_struct(bank)
    g = torch.Generator().manual_seed(37)
    W = (torch.randn(E2, H, generator=g) * 0.02).to(torch.bfloat16).cuda()
    bias = torch.zeros(E2)
    bias[FORCED] = 10.0
    bias = bias.cuda()
    x = torch.randn(M, H, generator=g).to(torch.bfloat16).cuda()
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    ws, nb = _ws("mimo_moe_decode_workspace_size", M, E2, K2, H, I)
    ident = torch.arange(E2, dtype=torch.int32)
    missing, beyond = ident.clone(), ident.clone()
    missing[FORCED] = -1
    beyond[FORCED] = E2
    for name, tab, want in (("identity", ident, _lib.MIMO_OK), ("missing", missing, _lib.ERR_SLOT),
                            ("beyond", beyond, _lib.ERR_SLOT)):
        tab = tab.cuda()

        def run(st):
            _lib.call("mimo_moe_decode", _lib.ptr(x), M, _lib.ptr(W), _lib.ptr(bias), _lib.ptr(tab), E2, K2, b,
                      _lib.ptr(y), None, None, _lib.ptr(st), _lib.ptr(ws), nb, _lib.stream_ptr())
        assert _status(run) == want, (name, M)


@pytest.mark.parametrize("M", [1, 4])
def test_layer_decode_status(parts, M):
    bank, W, bias, x, norm_w = parts
    b = pools.bank_struct(bank)
    h = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    ws, nb = _ws("mimo_moe_layer_decode_workspace_size", M, E, K, H, I)
    for name, (tab, want) in _tables().items():
        def run(st):
            _lib.call("mimo_moe_layer_decode", _lib.ptr(x[:M]), M, _lib.ptr(norm_w), 1e-6, _lib.ptr(W), _lib.ptr(bias),
                      _lib.ptr(tab), E, K, b, _lib.ptr(h), None, None, None, _lib.ptr(st), _lib.ptr(ws), nb,
                      _lib.stream_ptr())
        assert _status(run) == want, (name, M)


@pytest.mark.parametrize("T", [9, 64])
def test_prefill_block_and_layer_status(parts, T):
    bank, W, bias, x, norm_w = parts
    b = pools.bank_struct(bank)
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ws, nb = _ws("mimo_moe_layer_prefill_workspace_size", T, E, K, E, H, I)
    for name, (tab, want) in _tables().items():
        def run_block(st):
            _lib.call("mimo_moe_prefill_block", _lib.ptr(x[:T]), T, _lib.ptr(W), _lib.ptr(bias), _lib.ptr(tab), E, K,
                      b, _lib.ptr(y), None, None, _lib.ptr(st), _lib.ptr(ws), nb, _lib.stream_ptr())

        def run_layer(st):
            _lib.call("mimo_moe_layer_prefill", _lib.ptr(x[:T]), T, _lib.ptr(norm_w), 1e-6, _lib.ptr(W),
                      _lib.ptr(bias), _lib.ptr(tab), E, K, b, _lib.ptr(y), None, None, None, _lib.ptr(st),
                      _lib.ptr(ws), nb, _lib.stream_ptr())
        assert _status(run_block) == want, (name, T)
        assert _status(run_layer) == want, (name, T)


def test_prefill_given_slots_status(parts):
    """mimo_moe_prefill takes slot ids directly: ids outside [0, n_slots) are flagged."""
    bank, _, _, x, _ = parts
    b = pools.bank_struct(bank)
    T = 40
    rng = np.random.default_rng(3)
    si = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    w = torch.full((T, K), 1.0 / K, device="cuda")
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ws, nb = _ws("mimo_moe_prefill_workspace_size", T, K, E, H, I)
    for bad, want in ((None, _lib.MIMO_OK), (-1, _lib.ERR_SLOT), (E, _lib.ERR_SLOT), (1 << 20, _lib.ERR_SLOT)):
        s2 = si.copy()
        if bad is not None:
            s2[17, 2] = bad
        sd = torch.from_numpy(s2).cuda()

        def run(st):
            _lib.call("mimo_moe_prefill", _lib.ptr(x[:T]), T, _lib.ptr(sd), _lib.ptr(w), K, b, _lib.ptr(y),
                      _lib.ptr(st), _lib.ptr(ws), nb, _lib.stream_ptr())
        assert _status(run) == want, bad


def _router(W, bias):
    from mimo_stream import Router
    r = Router(H, E, K)
    r.weight.copy_(W)
    r.e_score_correction_bias.copy_(bias)
    return r


def test_partial_block_raises(parts):
    """A block whose slot table leaves the selected expert out raises ValueError on the decode and prefill paths
    (and in the layer step); routes among the resident experts run normally and match the full block."""
    from mimo_stream import MoEBlock, MoELayer
    bank, W, bias, x, norm_w = parts
    resident = [e for e in range(E) if e != FORCED][:10]
    sub = {k: v[resident].contiguous() for k, v in bank.items()}
    slot_of = np.full(E, -1, np.int32)
    slot_of[resident] = np.arange(len(resident), dtype=np.int32)
    blk = MoEBlock(_router(W, bias), sub, slot_of=slot_of)
    assert blk.partial
    for T in (1, 3, 8, 40):
        with pytest.raises(ValueError, match="no resident slot"):
            blk(x[:T])
    layer = MoELayer(blk, norm_w, 1e-6)
    for T in (2, 40):
        with pytest.raises(ValueError, match="no resident slot"):
            layer(x[:T])
    # a router that can only pick resident experts: no error, the same bits as the complete block
    bias2 = torch.full((E,), -10.0, device="cuda")
    bias2[resident[:K + 2]] = 10.0
    ok = MoEBlock(_router(W, bias2), sub, slot_of=slot_of)
    full = MoEBlock(_router(W, bias2), bank)
    assert not full.partial
    for T in (1, 3, 40):
        y, inds, _ = ok(x[:T], return_routes=True)
        y2, inds2, _ = full(x[:T], return_routes=True)
        assert torch.equal(inds, inds2) and torch.equal(y, y2)
    # the explicit-route paths check too
    inds = torch.full((2, K), FORCED, dtype=torch.int32, device="cuda")
    inds[:, 1:] = torch.tensor(resident[:K - 1], dtype=torch.int32)
    w = torch.full((2, K), 0.25, device="cuda")
    with pytest.raises(ValueError):
        blk._moe_small(x[:2], inds, w)
    with pytest.raises(ValueError):
        blk._moe_prefill(x[:2], inds, w)


def test_load_block_subset_raises(parts, tmp_path):
    """store.load_block(order=subset) gives a partial block: a row that selects an expert outside the subset
    raises instead of running slot 0's expert."""
    from safetensors.torch import save_file
    from mimo_stream import store
    bank, W, bias, x, _ = parts
    store.write_expert_layer(store.expert_file(tmp_path, 2), 2, {k: v.cpu() for k, v in bank.items()})
    wn, bn = store.router_names(2)
    save_file({wn: W.cpu(), bn: bias.cpu()}, os.path.join(tmp_path, "dense.safetensors"))
    order = [9, 3, 12, 0, 7, 1]                      # FORCED is not among them
    blk = store.load_block(tmp_path, 2, order=order)
    assert blk.partial
    with pytest.raises(ValueError, match="no resident slot"):
        blk(x[:1])
    with pytest.raises(ValueError, match="no resident slot"):
        blk(x[:20])
    whole = store.load_block(tmp_path, 2)
    assert not whole.partial
    whole(x[:1])
    whole.check_status()
