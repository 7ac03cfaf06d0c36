"""Expert slot pools (one MoE layer's resident experts) in HBM.

Layout and names follow engine/mimo_stream/model.py:26-45 (E, TOPK, SHAPES, EXPERT_BYTES, alloc_bank): per
projection an E2M1 pool [S, out, in/8] uint32 (low nibble first) and an E8M0 pool [S, out, in/32] uint8,
addressed by slot.  With every expert resident (288 GB of HBM holds all 48 MiMo MoE layers) the slot table is
the identity unless a popularity order is given (engine/mimo_stream/cache.py:24-29).
"""
import torch

from . import _lib

E, TOPK = 256, 8
VERIFY_MAX = 8
HIDDEN, INTER = 4096, 2048
SHAPES = {"gate": (INTER, HIDDEN), "up": (INTER, HIDDEN), "down": (HIDDEN, INTER)}   # (out, in)
EXPERT_BYTES = sum(o * i // 2 + o * i // 32 for o, i in SHAPES.values())             # 13,369,344


def shapes(hidden=HIDDEN, inter=INTER):
    return {"gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}


def expert_bytes(hidden=HIDDEN, inter=INTER):
    return sum(o * i // 2 + o * i // 32 for o, i in shapes(hidden, inter).values())


def alloc_bank(S, hidden=HIDDEN, inter=INTER, device="cuda"):
    """Slot bank {gate_w, gate_s, up_w, up_s, down_w, down_s} of S zeroed slots (model.py:32-45)."""
    bank = {}
    for k, (o, i) in shapes(hidden, inter).items():
        bank[f"{k}_w"] = torch.zeros((S, o, i // 8), dtype=torch.int32, device=device)
        bank[f"{k}_s"] = torch.zeros((S, o, i // 32), dtype=torch.uint8, device=device)
    return bank


def random_bank(S, seed, hidden=HIDDEN, inter=INTER, stddev=0.02, device="cuda"):
    """Bank whose weights are MXFP4 quantisations of seeded N(0, stddev) bf16 values (engine/tests/
    test_kernels.py:21-29), generated and quantised in place on the device (no bf16 intermediate)."""
    bank = alloc_bank(S, hidden, inter, device)
    st = _lib.stream_ptr(torch.device(device))
    for j, (k, (o, i)) in enumerate(shapes(hidden, inter).items()):
        _lib.call("mimo_fill_random_mxfp4", (seed * 3 + j) & (2 ** 64 - 1), stddev, S * o, i,
                  _lib.ptr(bank[f"{k}_w"]), _lib.ptr(bank[f"{k}_s"]), st)
    return bank


def bank_struct(bank):
    """ctypes struct mimo_bank for a bank dict (keeps no reference: the dict must outlive the call)."""
    S, inter, hw = bank["gate_w"].shape
    hidden = hw * 8
    for k, (o, i) in shapes(hidden, inter).items():
        w, s = bank[f"{k}_w"], bank[f"{k}_s"]
        if tuple(w.shape) != (S, o, i // 8) or tuple(s.shape) != (S, o, i // 32):
            raise ValueError(f"bank {k}: shapes {tuple(w.shape)}, {tuple(s.shape)} do not match [S, out, in/8] / [S, out, in/32]")
        if not (w.is_contiguous() and s.is_contiguous()):
            raise ValueError(f"bank {k}: pools must be contiguous")
        _lib.require_cuda(w, s)
    return _lib.MimoBank(bank["gate_w"].data_ptr(), bank["gate_s"].data_ptr(), bank["up_w"].data_ptr(),
                         bank["up_s"].data_ptr(), bank["down_w"].data_ptr(), bank["down_s"].data_ptr(),
                         S, hidden, inter)
