"""MoE expert kernels, organised by distinct expert: the API of engine/mimo_stream/kernels.py on MI355X.

  sigmoid_table()                     kernels.py:138-146
  group_routes(inds, scores, R)       kernels.py:149-173   (runs on the device)
  moe_experts(x, pools, uslot, ...)   kernels.py:176-199   (gate/up + SwiGLU, down * weight, fixed-order combine)

Every call goes through libmimo_moe.so; tensors are torch device tensors (numpy inputs are copied to the
device).  Weights stay in the reference's MXFP4 pool layout and are addressed by slot.
"""
import numpy as np
import torch

from . import _lib
from .pools import bank_struct


def _dev(a, dtype, device):
    if isinstance(a, torch.Tensor):
        return a.to(device=device, dtype=dtype).contiguous()
    return torch.as_tensor(np.ascontiguousarray(a)).to(device=device, dtype=dtype).contiguous()


def sigmoid_table(device="cuda"):
    """bf16 sigmoid of every bf16 bit pattern, as a bf16 tensor [65536] (kernels.py:138-146)."""
    out = torch.empty(1 << 16, dtype=torch.int16, device=device)
    _lib.call("mimo_sigmoid_table", _lib.ptr(out), _lib.stream_ptr(out.device))
    return out.view(torch.bfloat16)


def group_routes(inds, scores, R=8, slot_of=None, n_slots=None, device="cuda"):
    """Distinct-expert grouping (kernels.py:149-173) on the device.

    inds [M, k] expert (or slot) ids, scores [M, k].  slot_of (optional int32 [E]) maps expert -> slot first.
    Returns uids [U] (ascending slots), urows [U, R] int32, ucnt [U] int32, uw [U, R] float32, gidx [M*k]
    int32 (= u*R + c).  Raises ValueError when more than R routes land on one expert (kernels.py:167-168)
    or an expert has no slot.  Synchronises once to learn U, as the host version returns U-sized arrays."""
    inds_d = _dev(inds, torch.int32, device)
    scores_d = _dev(scores, torch.float32, device)
    M, k = inds_d.shape
    so = None if slot_of is None else _dev(slot_of, torch.int32, device)
    if M * k == 0:                          # no routes: no distinct experts (np.unique of nothing), no launch
        dev = inds_d.device
        return (torch.empty(0, dtype=torch.int32, device=dev), torch.empty((0, R), dtype=torch.int32, device=dev),
                torch.empty(0, dtype=torch.int32, device=dev), torch.empty((0, R), dtype=torch.float32, device=dev),
                torch.empty(0, dtype=torch.int32, device=dev))
    if n_slots is None:
        n_slots = int(so.max().item()) + 1 if so is not None else int(inds_d.max().item()) + 1
    Umax = min(M * k, n_slots)
    dev = inds_d.device
    uids = torch.empty(Umax, dtype=torch.int32, device=dev)
    urows = torch.empty((Umax, R), dtype=torch.int32, device=dev)
    ucnt = torch.empty(Umax, dtype=torch.int32, device=dev)
    uw = torch.empty((Umax, R), dtype=torch.float32, device=dev)
    gidx = torch.empty(M * k, dtype=torch.int32, device=dev)
    nu = torch.empty(2, dtype=torch.int32, device=dev)
    _lib.call("mimo_group_routes", _lib.ptr(inds_d), _lib.ptr(scores_d), _lib.ptr(so), M, k, R, n_slots,
              _lib.ptr(uids), _lib.ptr(urows), _lib.ptr(ucnt), _lib.ptr(uw), _lib.ptr(gidx), _lib.ptr(nu[0:1]),
              _lib.ptr(nu[1:2]), _lib.stream_ptr(dev))
    U, status = (int(v) for v in nu.cpu())
    if status == _lib.ERR_ROWS_PER_EXPERT:
        raise ValueError("more rows than R routed to one expert")
    if status != 0:
        raise ValueError(f"group_routes: expert without a resident slot (code {status})")
    return uids[:U], urows[:U], ucnt[:U], uw[:U], gidx


def _gidx_from_rows(urows, ucnt, M):
    """Deterministic gather order when no gather_idx is given: each row's routes in ascending expert order."""
    ur = urows.cpu().numpy()
    uc = ucnt.cpu().numpy()
    per_row = [[] for _ in range(M)]
    R = ur.shape[1]
    for u in range(len(uc)):
        for c in range(int(uc[u])):
            per_row[int(ur[u, c])].append(u * R + c)
    k = len(per_row[0])
    if any(len(p) != k for p in per_row):
        raise ValueError("moe_experts without gather_idx needs the same number of routes on every row")
    return torch.tensor(np.array(per_row, np.int32).reshape(-1)), k


def moe_experts(x, pools, uslot, urows, ucnt, uw, R=8, gather_idx=None, round_expert_bf16=False,
                n_unique=None, return_intermediates=False):
    """Routed expert output for M <= 8 token rows (kernels.py:176-199).

    x bf16 [M, H]; pools: dict gate_w, gate_s, up_w, up_s, down_w, down_s; uslot [U] slot per distinct
    expert; urows/ucnt/uw from group_routes; gather_idx [M*k] (route -> u*R + c).  Returns bf16 [M, H] =
    the fixed-order sum over each row's experts of weight * expert(x_row).  Without gather_idx each row's
    routes are summed in ascending expert order (the reference falls back to an order-nondeterministic
    scatter-add there, kernels.py:196-197).  round_expert_bf16 rounds each expert's output to bf16 before
    weighting (the gather_qmm path, model.py:173-182).  n_unique (optional int32 device scalar) lets U be
    decided on the device; then uslot/urows/... may be padded."""
    _lib.require_cuda(x)
    dev = x.device
    x = x.to(torch.bfloat16).contiguous()
    M = x.shape[0]
    if M == 0:                              # no rows: an empty output, no launch
        bank = bank_struct(pools)
        y = torch.empty((0, bank.hidden), dtype=torch.bfloat16, device=dev)
        if return_intermediates:
            return (y, torch.empty((0, R, bank.inter), dtype=torch.bfloat16, device=dev),
                    torch.empty((0, R, bank.hidden), dtype=torch.float32, device=dev))
        return y
    uslot, urows, ucnt = (_dev(a, torch.int32, dev) for a in (uslot, urows, ucnt))
    uw = _dev(uw, torch.float32, dev)
    Umax = uslot.shape[0]
    if gather_idx is None:
        gidx, k = _gidx_from_rows(urows, ucnt, M)
        gidx = gidx.to(dev)
    else:
        gidx = _dev(gather_idx, torch.int32, dev)
        k = gidx.numel() // M
    bank = bank_struct(pools)
    H, I = bank.hidden, bank.inter
    y = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    h = part = None
    if return_intermediates:
        h = torch.empty((Umax, R, I), dtype=torch.bfloat16, device=dev)
        part = torch.empty((Umax, R, H), dtype=torch.float32, device=dev)
    nbytes = _lib.load().mimo_moe_experts_workspace_size(M, Umax, R, H, I)
    ws = _lib.workspace(nbytes, dev, "experts")
    _lib.call("mimo_moe_experts", _lib.ptr(x), M, bank, _lib.ptr(uslot), _lib.ptr(urows), _lib.ptr(ucnt),
              _lib.ptr(uw), _lib.ptr(n_unique), Umax, R, _lib.ptr(gidx), k, int(bool(round_expert_bf16)),
              _lib.ptr(y), _lib.ptr(h), _lib.ptr(part), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
    if return_intermediates:
        return y, h, part
    return y


def quantize_mxfp4(w):
    """bf16 [..., K] -> (q int32 [..., K/8], s uint8 [..., K/32]) on the device (OCP MX rule)."""
    _lib.require_cuda(w)
    w = w.to(torch.bfloat16).contiguous()
    K = w.shape[-1]
    rows = w.numel() // K
    q = torch.empty((*w.shape[:-1], K // 8), dtype=torch.int32, device=w.device)
    s = torch.empty((*w.shape[:-1], K // 32), dtype=torch.uint8, device=w.device)
    _lib.call("mimo_quantize_mxfp4", _lib.ptr(w), rows, K, _lib.ptr(q), _lib.ptr(s), _lib.stream_ptr(w.device))
    return q, s


def dequantize_mxfp4(q, s):
    """(int32 [..., K/8], uint8 [..., K/32]) -> float32 [..., K] on the device."""
    _lib.require_cuda(q, s)
    K = q.shape[-1] * 8
    rows = q.numel() // q.shape[-1]
    out = torch.empty((*q.shape[:-1], K), dtype=torch.float32, device=q.device)
    _lib.call("mimo_dequantize_mxfp4", _lib.ptr(q.contiguous()), _lib.ptr(s.contiguous()), rows, K, _lib.ptr(out),
              _lib.stream_ptr(q.device))
    return out


def random_bf16(shape, seed, stddev=1.0, device="cuda"):
    """Seeded N(0, stddev) bf16 tensor; element i depends only on (seed, i)."""
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    _lib.call("mimo_random_bf16", seed & (2 ** 64 - 1), stddev, out.numel(), _lib.ptr(out), _lib.stream_ptr(out.device))
    return out


def quantize_fp8_hilo(x):
    """bf16 [rows, K] -> (hi, hs, lo, ls) uint8 tensors: the activation split the MFMA paths use."""
    _lib.require_cuda(x)
    x = x.to(torch.bfloat16).contiguous()
    rows, K = x.shape
    hi = torch.empty((rows, K), dtype=torch.uint8, device=x.device)
    lo = torch.empty_like(hi)
    hs = torch.empty((rows, K // 32), dtype=torch.uint8, device=x.device)
    ls = torch.empty_like(hs)
    _lib.call("mimo_quantize_fp8_hilo", _lib.ptr(x), rows, K, _lib.ptr(hi), _lib.ptr(hs), _lib.ptr(lo), _lib.ptr(ls),
              _lib.stream_ptr(x.device))
    return hi, hs, lo, ls
