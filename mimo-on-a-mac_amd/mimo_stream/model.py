"""The MoE block of MiMo-V2.6-Flash on MI355X: Router and the decode / prefill dispatch of one MoE layer.

Mirrors engine/mimo_stream/model.py:
  Router                 :52-65   fp32 gate linear, sigmoid, noaux bias for selection, top-8, renormalised weights
  MoEBlock._moe_small    :184-219 T <= VERIFY_MAX rows: M == 1 gather_qmm rounding, M >= 2 distinct-expert kernels
  MoEBlock._moe_prefill  :230-271 stable sort of (token, k) routes by slot, grouped GEMMs, fixed-order combine
  MoEBlock.__call__      :303-340 router -> small or prefill path (the caller adds y to the residual, :340)
with every expert resident in HBM, so SlotCache.resolve / SSD reads (:191-217) reduce to the slot table.
Unlike the reference, routes never go back to the host: routing, grouping and dispatch run on the device
between the router and the expert kernels (the reference syncs at :315).
"""
import numpy as np
import torch

from . import _lib
from .pools import E, TOPK, VERIFY_MAX, bank_struct


class Router:
    """Router (model.py:52-65): weight bf16 [E, H], e_score_correction_bias fp32 [E].

    The defaults are the engine's router (renormalised weights for every k).  The options of the vendored
    noaux-tc gate (MoEGate, mimo_v2.py:195-216) apply when set: group-limited selection (n_group > 1,
    topk_group), norm_topk_prob (renormalise only when set and k > 1) and routed_scaling_factor; the routes then
    come from mimo_router_select_grouped, and blocks run their experts on the given routes."""

    def __init__(self, hidden, n_experts=E, top_k=TOPK, device="cuda", n_group=None, topk_group=None,
                 norm_topk_prob=None, routed_scaling_factor=None):
        self.weight = torch.zeros((n_experts, hidden), dtype=torch.bfloat16, device=device)
        self.e_score_correction_bias = torch.zeros(n_experts, dtype=torch.float32, device=device)
        self.top_k = top_k
        self.gate_options = None
        if any(v is not None for v in (n_group, topk_group, norm_topk_prob, routed_scaling_factor)):
            ng = 1 if n_group is None else int(n_group)
            tg = ng if topk_group is None else int(topk_group)
            if ng < 1 or n_experts % ng or not 1 <= tg <= ng:
                raise ValueError("need n_group dividing the experts and 1 <= topk_group <= n_group")
            self.gate_options = (ng, tg, True if norm_topk_prob is None else bool(norm_topk_prob),
                                 1.0 if routed_scaling_factor is None else float(routed_scaling_factor))

    def logits_and_routes(self, r):
        """r bf16 [..., T, H] -> (logits fp32 [T, E], inds int32 [T, k], w fp32 [T, k])."""
        _lib.require_cuda(r)
        r2 = r.reshape(-1, r.shape[-1]).to(torch.bfloat16).contiguous()
        T, H = r2.shape
        En = self.weight.shape[0]
        dev = r2.device
        logits = torch.empty((T, En), dtype=torch.float32, device=dev)
        inds = torch.empty((T, self.top_k), dtype=torch.int32, device=dev)
        w = torch.empty((T, self.top_k), dtype=torch.float32, device=dev)
        if T == 0:                          # an empty batch routes nothing (no launch)
            return logits, inds, w
        _lib.call("mimo_router", _lib.ptr(r2), _lib.ptr(self.weight.contiguous()),
                  _lib.ptr(self.e_score_correction_bias.contiguous()), T, H, En, self.top_k, _lib.ptr(logits),
                  _lib.ptr(inds), _lib.ptr(w), _lib.stream_ptr(dev))
        if self.gate_options is not None:
            ng, tg, norm, scale = self.gate_options
            _lib.call("mimo_router_select_grouped", _lib.ptr(logits), _lib.ptr(self.e_score_correction_bias.contiguous()),
                      T, En, self.top_k, ng, tg, int(norm), scale, _lib.ptr(inds), _lib.ptr(w), _lib.stream_ptr(dev))
        return logits, inds, w

    def __call__(self, r):
        _, inds, w = self.logits_and_routes(r)
        lead = r.shape[:-1]
        return inds.reshape(*lead, self.top_k), w.reshape(*lead, self.top_k)


def select_from_logits(logits, bias, k, scaling=1.0):
    """Selection given fp32 logits [T, E] (model.py:60-64): inds int32 [T, k], w fp32 [T, k]."""
    _lib.require_cuda(logits)
    logits = logits.to(torch.float32).contiguous()
    T, En = logits.shape
    bias = bias.to(device=logits.device, dtype=torch.float32).contiguous()
    inds = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, k), dtype=torch.float32, device=logits.device)
    _lib.call("mimo_router_select", _lib.ptr(logits), _lib.ptr(bias), T, En, k, float(scaling), _lib.ptr(inds),
              _lib.ptr(w), _lib.stream_ptr(logits.device))
    return inds, w


def prefill_dispatch(slot_inds, n_slots):
    """Stable sort of the flat (token, k) routes by slot (model.py:235-242) and its inverse (:266-268):
    perm int32 [T*k], offsets int32 [n_slots + 1], inv int32 [T*k]."""
    _lib.require_cuda(slot_inds)
    si = slot_inds.to(torch.int32).contiguous()
    T, k = si.shape
    dev = si.device
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_slots + 1, dtype=torch.int32, device=dev)
    nbytes = _lib.load().mimo_prefill_dispatch_workspace_size(T, k, n_slots)
    ws = _lib.workspace(nbytes, dev, "dispatch")
    _lib.call("mimo_prefill_dispatch", _lib.ptr(si), T, k, n_slots, _lib.ptr(perm), _lib.ptr(offsets), _lib.ptr(inv),
              _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
    return perm, offsets, inv


class MoEBlock:
    """One MoE layer: router, resident slot bank and expert -> slot table (slot_of None = identity).

    A table with experts outside the bank (entries outside [0, n_slots), e.g. a bank loaded for a subset of the
    experts) makes the block partial: the kernels cannot read such an expert, so they flag it in the block's
    device status word, and a partial block reads that word after every call (one synchronisation) and raises
    ValueError when a route reached an expert with no slot, as the reference raises rather than compute with
    the wrong expert (kernels.py:167-168; cache.py:45-46 loads the expert instead, which StreamedMoEBlock does).
    A complete table needs no check: every expert has a slot and a row picks an expert at most once."""

    def __init__(self, router, bank, slot_of=None):
        self.router = router
        self.bank = bank
        self._bank_struct = bank_struct(bank)
        dev = router.weight.device
        self.slot_of = None if slot_of is None else torch.as_tensor(slot_of, dtype=torch.int32).to(dev).contiguous()
        if self.slot_of is None:
            self.partial = router.weight.shape[0] > self._bank_struct.n_slots
        else:
            if self.slot_of.shape != (router.weight.shape[0],):
                raise ValueError(f"slot_of has {tuple(self.slot_of.shape)} entries for {router.weight.shape[0]} experts")
            tab = self.slot_of.cpu()
            self.partial = bool(((tab < 0) | (tab >= self._bank_struct.n_slots)).any())
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)

    def check_status(self, what="MoEBlock"):
        """Raise ValueError if the last call found a route to an expert with no slot (synchronises)."""
        _lib.check_status(self.status, what)

    @property
    def n_slots(self):
        return self._bank_struct.n_slots

    def _slots(self, inds):
        inds = inds.to(torch.int64)
        return (self.slot_of[inds] if self.slot_of is not None else inds).to(torch.int32).contiguous()

    def _moe_small(self, r2, inds, w, check=None):
        """T <= VERIFY_MAX rows with given routes (model.py:184-219): M == 1 rounds each expert's output to bf16
        (_gather_m1), M >= 2 sums fp32 partials (distinct-expert kernels).  No host synchronisation unless the
        grouping's status is checked (check, default: when the block is partial)."""
        _lib.require_cuda(r2)
        T, k = inds.shape
        if T > VERIFY_MAX:
            raise ValueError(f"_moe_small takes at most {VERIFY_MAX} rows")
        dev = r2.device
        if T == 0:
            return torch.empty((0, self._bank_struct.hidden), dtype=torch.bfloat16, device=dev)
        S = self.n_slots
        slot_inds = self._slots(inds)
        w = w.to(torch.float32).contiguous()
        Umax = min(T * k, S)
        R = VERIFY_MAX
        uids = torch.empty(Umax, dtype=torch.int32, device=dev)
        urows = torch.empty((Umax, R), dtype=torch.int32, device=dev)
        ucnt = torch.empty(Umax, dtype=torch.int32, device=dev)
        uw = torch.empty((Umax, R), dtype=torch.float32, device=dev)
        gidx = torch.empty(T * k, dtype=torch.int32, device=dev)
        nu = torch.empty(1, dtype=torch.int32, device=dev)
        st = _lib.stream_ptr(dev)
        _lib.call("mimo_group_routes", _lib.ptr(slot_inds), _lib.ptr(w), None, T, k, R, S, _lib.ptr(uids),
                  _lib.ptr(urows), _lib.ptr(ucnt), _lib.ptr(uw), _lib.ptr(gidx), _lib.ptr(nu), _lib.ptr(self.status), st)
        x = r2.to(torch.bfloat16).contiguous()
        y = torch.empty((T, self._bank_struct.hidden), dtype=torch.bfloat16, device=dev)
        H, I = self._bank_struct.hidden, self._bank_struct.inter
        nbytes = _lib.load().mimo_moe_experts_workspace_size(T, Umax, R, H, I)
        ws = _lib.workspace(nbytes, dev, "experts")
        _lib.call("mimo_moe_experts", _lib.ptr(x), T, self._bank_struct, _lib.ptr(uids), _lib.ptr(urows), _lib.ptr(ucnt),
                  _lib.ptr(uw), _lib.ptr(nu), Umax, R, _lib.ptr(gidx), k, 1 if T == 1 else 0, _lib.ptr(y), None,
                  None, _lib.ptr(ws), ws.numel(), st)
        if self.partial if check is None else check:
            self.check_status("MoEBlock._moe_small")
        return y

    def _moe_prefill(self, r2, inds, w, check=None):
        """Prefill with given routes (model.py:230-271): [T, H] bf16.  The status is checked (one synchronisation)
        when check, default: when the block is partial."""
        _lib.require_cuda(r2)
        T, k = inds.shape
        dev = r2.device
        if T == 0:
            return torch.empty((0, self._bank_struct.hidden), dtype=torch.bfloat16, device=dev)
        x = r2.to(torch.bfloat16).contiguous()
        slot_inds = self._slots(inds)
        w = w.to(torch.float32).contiguous()
        b = self._bank_struct
        y = torch.empty((T, b.hidden), dtype=torch.bfloat16, device=dev)
        nbytes = _lib.load().mimo_moe_prefill_workspace_size(T, k, b.n_slots, b.hidden, b.inter)
        ws = _lib.workspace(nbytes, dev, "prefill")
        _lib.call("mimo_moe_prefill", _lib.ptr(x), T, _lib.ptr(slot_inds), _lib.ptr(w), k, b, _lib.ptr(y),
                  _lib.ptr(self.status), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
        if self.partial if check is None else check:
            self.check_status("MoEBlock._moe_prefill")
        return y

    def __call__(self, r, return_routes=False):
        """Router + experts for r bf16 [T, H] (model.py:303-336): T <= 8 runs the fused decode block, larger T
        the prefill block.  Returns y bf16 [T, H] (and inds, w when return_routes).  A partial block raises
        ValueError when a row selected an expert that has no slot."""
        _lib.require_cuda(r)
        r2 = r.reshape(-1, r.shape[-1]).to(torch.bfloat16).contiguous()
        T = r2.shape[0]
        dev = r2.device
        b = self._bank_struct
        rt = self.router
        if rt.gate_options is not None:     # the vendored gate's options: route, then the experts on the routes
            inds, w = rt(r2)
            y = self._moe_small(r2, inds, w) if T <= VERIFY_MAX else self._moe_prefill(r2, inds, w)
            return (y, inds, w) if return_routes else y
        En, k = rt.weight.shape[0], rt.top_k
        y = torch.empty((T, b.hidden), dtype=torch.bfloat16, device=dev)
        inds = torch.empty((T, k), dtype=torch.int32, device=dev)
        w = torch.empty((T, k), dtype=torch.float32, device=dev)
        if T == 0:                          # an empty batch: empty outputs, no launch
            return (y, inds, w) if return_routes else y
        st = _lib.stream_ptr(dev)
        args = (_lib.ptr(r2), T, _lib.ptr(rt.weight), _lib.ptr(rt.e_score_correction_bias), _lib.ptr(self.slot_of), En, k,
                b, _lib.ptr(y), _lib.ptr(inds), _lib.ptr(w), _lib.ptr(self.status))
        if T <= VERIFY_MAX:
            nbytes = _lib.load().mimo_moe_decode_workspace_size(T, En, k, b.hidden, b.inter)
            ws = _lib.workspace(nbytes, dev, "decode")
            _lib.call("mimo_moe_decode", *args, _lib.ptr(ws), ws.numel(), st)
        else:
            nbytes = _lib.load().mimo_moe_prefill_block_workspace_size(T, En, k, b.n_slots, b.hidden, b.inter)
            ws = _lib.workspace(nbytes, dev, "prefill_block")
            _lib.call("mimo_moe_prefill_block", *args, _lib.ptr(ws), ws.numel(), st)
        if self.partial:
            self.check_status("MoEBlock")
        return (y, inds, w) if return_routes else y

    def forward_residual(self, x, r):
        """h = x + MoE(r) (model.py:340), the addition in the library (mimo_residual_add: bf16(x + y)).  For the
        whole MoE half of a layer (norm, block, residual in one call) see mimo_stream.layer.MoELayer."""
        y = self(r)
        x2 = x.reshape(y.shape).to(torch.bfloat16).contiguous()
        h = torch.empty_like(x2)
        _lib.call("mimo_residual_add", _lib.ptr(x2), _lib.ptr(y), x2.numel(), _lib.ptr(h), _lib.stream_ptr(x2.device))
        return h.reshape(x.shape)
