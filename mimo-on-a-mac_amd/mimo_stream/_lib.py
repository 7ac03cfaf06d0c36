"""ctypes binding of libmimo_moe.so (the C ABI declared in include/mimo_moe.h).

The library is the only compute path: if it is not built this module raises, there is no fallback.
"""
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmimo_moe.so")
ABI_VERSION = 2

MIMO_OK = 0
ERR_SHAPE, ERR_ALIGN, ERR_ROWS_PER_EXPERT, ERR_SLOT, ERR_WORKSPACE, ERR_HIP, ERR_ARG = -1, -2, -3, -4, -5, -6, -7
_VALUE_ERRORS = {ERR_SHAPE, ERR_ALIGN, ERR_ROWS_PER_EXPERT, ERR_SLOT, ERR_WORKSPACE, ERR_ARG}


class MimoBank(ctypes.Structure):
    """struct mimo_bank (include/mimo_moe.h)."""
    _fields_ = [("gate_w", ctypes.c_void_p), ("gate_s", ctypes.c_void_p),
                ("up_w", ctypes.c_void_p), ("up_s", ctypes.c_void_p),
                ("down_w", ctypes.c_void_p), ("down_s", ctypes.c_void_p),
                ("n_slots", ctypes.c_int32), ("hidden", ctypes.c_int32), ("inter", ctypes.c_int32)]


P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
U64 = ctypes.c_uint64
F32 = ctypes.c_float
SZ = ctypes.c_size_t
BANKP = ctypes.POINTER(MimoBank)

SIGNATURES = {
    "mimo_abi_version": (I32, []),
    "mimo_last_error": (ctypes.c_char_p, []),
    "mimo_quantize_mxfp4": (I32, [P, I64, I64, P, P, P]),
    "mimo_dequantize_mxfp4": (I32, [P, P, I64, I64, P, P]),
    "mimo_random_bf16": (I32, [U64, F32, I64, P, P]),
    "mimo_fill_random_mxfp4": (I32, [U64, F32, I64, I64, P, P, P]),
    "mimo_quantize_fp8_hilo": (I32, [P, I64, I64, P, P, P, P, P]),
    "mimo_sigmoid_table": (I32, [P, P]),
    "mimo_router_select": (I32, [P, P, I32, I32, I32, F32, P, P, P]),
    "mimo_router": (I32, [P, P, P, I32, I32, I32, I32, P, P, P, P]),
    "mimo_router_select_grouped": (I32, [P, P, I32, I32, I32, I32, I32, I32, F32, P, P, P]),
    "mimo_group_routes": (I32, [P, P, P, I32, I32, I32, I32, P, P, P, P, P, P, P, P]),
    "mimo_prefill_dispatch": (I32, [P, I32, I32, I32, P, P, P, P, SZ, P]),
    "mimo_prefill_dispatch_workspace_size": (SZ, [I32, I32, I32]),
    "mimo_moe_experts": (I32, [P, I32, BANKP, P, P, P, P, P, I32, I32, P, I32, I32, P, P, P, P, SZ, P]),
    "mimo_moe_experts_workspace_size": (SZ, [I32, I32, I32, I32, I32]),
    "mimo_moe_decode": (I32, [P, I32, P, P, P, I32, I32, BANKP, P, P, P, P, P, SZ, P]),
    "mimo_moe_decode_workspace_size": (SZ, [I32, I32, I32, I32, I32]),
    "mimo_moe_prefill": (I32, [P, I32, P, P, I32, BANKP, P, P, P, SZ, P]),
    "mimo_moe_prefill_workspace_size": (SZ, [I32, I32, I32, I32, I32]),
    "mimo_moe_prefill_staged": (I32, [P, I32, P, P, I32, BANKP, BANKP, P, P, P, SZ, P]),
    "mimo_moe_prefill_block": (I32, [P, I32, P, P, P, I32, I32, BANKP, P, P, P, P, P, SZ, P]),
    "mimo_moe_prefill_block_workspace_size": (SZ, [I32, I32, I32, I32, I32, I32]),
    "mimo_rmsnorm": (I32, [P, I32, I32, P, F32, P, P]),
    "mimo_residual_add": (I32, [P, P, I64, P, P]),
    "mimo_moe_layer_decode": (I32, [P, I32, P, F32, P, P, P, I32, I32, BANKP, P, P, P, P, P, P, SZ, P]),
    "mimo_moe_layer_decode_workspace_size": (SZ, [I32, I32, I32, I32, I32]),
    "mimo_moe_layer_prefill": (I32, [P, I32, P, F32, P, P, P, I32, I32, BANKP, P, P, P, P, P, P, SZ, P]),
    "mimo_moe_layer_prefill_workspace_size": (SZ, [I32, I32, I32, I32, I32, I32]),
    "mimo_moe_layer_decode_noalloc": (I32, [P, I32, P, F32, P, P, P, I32, I32, BANKP, P, P, P, P, P, P]),
    "mimo_profile_enable": (I32, [I32]),
    "mimo_profile_read": (I32, [I32, P, P, P]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load and bind libmimo_moe.so; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                                   "(or python mimo-on-a-mac_amd/build.py)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.mimo_abi_version() != ABI_VERSION:
                raise RuntimeError(f"libmimo_moe ABI {lib.mimo_abi_version()} != {ABI_VERSION}")
            _lib = lib
    return _lib


def check(rc, what=""):
    if rc == MIMO_OK:
        return
    msg = load().mimo_last_error().decode(errors="replace")
    if rc in _VALUE_ERRORS:
        raise ValueError(f"{what}: {msg} (code {rc})")
    raise RuntimeError(f"{what}: {msg} (code {rc})")


def call(name, *args):
    check(getattr(load(), name)(*args), name)


STATUS_MESSAGES = {ERR_SLOT: "a selected expert has no resident slot (slot_of entry outside the bank)",
                   ERR_ROWS_PER_EXPERT: "more than 8 rows routed to one slot"}


def check_status(status, what=""):
    """Raise ValueError if a device status word (int32 tensor, written by a fused entry point on the current
    stream) holds an error code.  Synchronises with the stream that wrote it."""
    code = int(status.reshape(-1)[0].item())
    if code != MIMO_OK:
        raise ValueError(f"{what}: {STATUS_MESSAGES.get(code, 'device error')} (code {code})")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_ptr(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("libmimo_moe works on device tensors; got a CPU tensor")


_ws = {}


def workspace(nbytes, device, tag):
    """Device workspace of at least nbytes, cached per (device, stream, entry point tag).

    The library needs no initialised workspace (every kernel writes what it later reads); each entry point gets
    its own buffer because their layouts differ."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (device.index, torch.cuda.current_stream(device).cuda_stream, tag)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _ws[key] = buf
    return buf


def profile_enable(on=True):
    """Start (or stop) per-kernel event timing inside the library; starting clears earlier records."""
    load().mimo_profile_enable(1 if on else 0)


def profile_read(max_kernels=32):
    """{kernel name: (total ms, launches)} of the launches recorded since profile_enable (synchronises)."""
    names = ctypes.create_string_buffer(64 * max_kernels)
    tot = (ctypes.c_float * max_kernels)()
    cnt = (ctypes.c_int * max_kernels)()
    n = load().mimo_profile_read(max_kernels, names, tot, cnt)
    check(n if n < 0 else 0, "profile_read")
    out = {}
    for j in range(min(n, max_kernels)):
        nm = names.raw[64 * j:64 * j + 64].split(b"\0")[0].decode()
        out[nm] = (float(tot[j]), int(cnt[j]))
    return out
