"""Expert and router weights in the converted checkpoint's on-disk format, loaded into HBM slot banks.

Format (the format contract of scripts/convert-mimo-v26-mlx.py:6-12, :67-131 and the reader
engine/mimo_stream/store.py:15-44):
  experts-LNN.safetensors  one file per MoE layer L; tensors model.layers.L.mlp.switch_mlp.{gate,up,down}_proj.
                           {weight, scales}, U32 [n_experts, out, in/8] (E2M1 nibbles, low first) and
                           U8 [n_experts, out, in/32] (E8M0), in that order.  The JSON header is padded with spaces
                           so the data section starts on a 16 KiB boundary, and every tensor's size is a multiple
                           of 16 KiB, so expert e of a tensor starts at data_start + offset + e * stride.
  dense.safetensors        the router of MoE layer L: model.layers.L.mlp.gate.weight (bf16 [n_experts, hidden])
                           and model.layers.L.mlp.gate.e_score_correction_bias (f32 [n_experts])
                           (engine/mimo_stream/model.py:120-124 loads them as the layer's Router).

ExpertStore reads headers and offsets (as the reference's ExpertStore does) and fills a slot bank
(pools.alloc_bank layout) with whole tensors, or with the experts of a slot order, through pinned host
staging and asynchronous copies.  Every expert of MiMo-V2.6-Flash fits in one MI355X's HBM (48 x 3.42 GB), so
there is no eviction or SSD streaming here.  Only safetensors data is read: no pickle, no code from the file.
"""
import json
import os
import struct
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import pools

ALIGN = 16384
PROJ = ("gate_proj", "up_proj", "down_proj")
KEYS = ("gate", "up", "down")
_DTYPES = {"U32": (np.uint32, 4), "U8": (np.uint8, 1), "BF16": (None, 2), "F32": (np.float32, 4)}


def expert_file(model_dir, L):
    return os.path.join(model_dir, f"experts-L{L:02d}.safetensors")


def tensor_name(L, proj, suffix):
    return f"model.layers.{L}.mlp.switch_mlp.{proj}.{suffix}"


def read_header(path):
    """(data_start, header dict) of a safetensors file."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file (short header)")
        n = struct.unpack("<Q", raw)[0]
        if n > 1 << 26:
            raise ValueError(f"{path}: header length {n} is implausible")
        hdr = json.loads(f.read(n))
    return 8 + n, hdr


class ExpertStore:
    """Offsets of every MoE layer's expert tensors (engine/mimo_stream/store.py:15-44).

    loc[(L, key, kind)] = (path, absolute offset, per-expert stride, shape), key in gate/up/down, kind w/s.
    The constructor checks names, dtypes, shapes (consistent hidden / intermediate sizes and expert count) and
    the 16 KiB alignment the format promises, and raises ValueError on any mismatch."""

    def __init__(self, model_dir, moe_layers, n_experts=None):
        self.model_dir = model_dir
        self.loc = {}
        self.n = n_experts
        self.hidden = self.inter = None
        for L in moe_layers:
            path = expert_file(model_dir, L)
            base, hdr = read_header(path)
            if base % ALIGN:
                raise ValueError(f"{path}: data section starts at {base}, not on a {ALIGN}-byte boundary")
            size = os.path.getsize(path)
            for proj, key in zip(PROJ, KEYS):
                for kind, suffix, dt, div in (("w", "weight", "U32", 8), ("s", "scales", "U8", 32)):
                    name = tensor_name(L, proj, suffix)
                    if name not in hdr:
                        raise ValueError(f"{path}: missing tensor {name}")
                    t = hdr[name]
                    if t["dtype"] != dt or len(t["shape"]) != 3:
                        raise ValueError(f"{path}: {name} is {t['dtype']} {t['shape']}, expected {dt} [n, out, in/{div}]")
                    n, o, c = t["shape"]
                    a, b = t["data_offsets"]
                    if b - a != n * o * c * _DTYPES[dt][1] or base + b > size:
                        raise ValueError(f"{path}: {name} byte range [{a}, {b}) does not match its shape or the file")
                    if a % ALIGN or (b - a) % ALIGN:
                        raise ValueError(f"{path}: {name} is not 16 KiB aligned (offsets {a}, {b})")
                    self.n = n if self.n is None else self.n
                    if n != self.n:
                        raise ValueError(f"{path}: {name} holds {n} experts, expected {self.n}")
                    inp = c * div
                    if key == "down":
                        hid, inter = o, inp
                    else:
                        hid, inter = inp, o
                    self.hidden = hid if self.hidden is None else self.hidden
                    self.inter = inter if self.inter is None else self.inter
                    if (hid, inter) != (self.hidden, self.inter):
                        raise ValueError(f"{path}: {name} shape {t['shape']} disagrees with hidden {self.hidden}, "
                                         f"intermediate {self.inter}")
                    self.loc[(L, key, kind)] = (path, base + a, (b - a) // n, (n, o, c))

    def jobs(self, L, expert, dst):
        """dst: {(key, kind): writable memoryview of one slot}.  Returns [(path, offset, memoryview)] reading
        expert `expert` of layer L into it (the reference's ExpertStore.jobs, store.py:37-46)."""
        out = []
        for key in KEYS:
            for kind in ("w", "s"):
                path, base, stride, _ = self.loc[(L, key, kind)]
                mv = dst[(key, kind)]
                if mv.nbytes != stride:
                    raise ValueError(f"layer {L} {key}_{kind}: slot holds {mv.nbytes} bytes, expert is {stride}")
                out.append((path, base + expert * stride, mv))
        return out

    def load_bank(self, L, order=None, device="cuda", threads=8, chunk=64 << 20):
        """Slot bank of layer L: slot s <- expert order[s] (default: every expert, slot = expert).

        Reads go through `threads` preads of up to `chunk` bytes into host staging (pinned when the target is a
        GPU), then one asynchronous copy per pool; returns the bank dict once the copies are done."""
        order = list(range(self.n)) if order is None else [int(e) for e in order]
        if any(e < 0 or e >= self.n for e in order):
            raise ValueError(f"expert ids must lie in [0, {self.n})")
        device = torch.device(device)
        bank = pools.alloc_bank(len(order), self.hidden, self.inter, device=device)
        whole = order == list(range(self.n))
        pin = device.type == "cuda"
        with ThreadPoolExecutor(threads) as ex:
            for key in KEYS:
                for kind in ("w", "s"):
                    path, base, stride, _ = self.loc[(L, key, kind)]
                    dst = bank[f"{key}_{kind}"]
                    nbytes = stride * len(order)
                    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=pin)
                    hv = memoryview(host.numpy())
                    reads = []
                    if whole:
                        reads = [(base + o, hv[o:o + min(chunk, nbytes - o)]) for o in range(0, nbytes, chunk)]
                    else:
                        for s, e in enumerate(order):
                            for o in range(0, stride, chunk):
                                n = min(chunk, stride - o)
                                reads.append((base + e * stride + o, hv[s * stride + o:s * stride + o + n]))
                    fd = os.open(path, os.O_RDONLY)
                    try:
                        list(ex.map(lambda r: _pread_into(fd, *r), reads))
                    finally:
                        os.close(fd)
                    dst.view(-1).view(torch.uint8).copy_(host, non_blocking=pin)
                    if pin:
                        torch.cuda.current_stream(device).synchronize()   # staging is reused per pool
        return bank


def _pread_into(fd, off, mv):
    got, n = 0, mv.nbytes
    while got < n:
        r = os.preadv(fd, [mv[got:]], off + got)
        if r <= 0:
            raise IOError(f"short read at {off + got}")
        got += r
    return n


def write_expert_layer(path, L, bank):
    """Write a slot bank as experts-LNN.safetensors in the converter's layout (16 KiB-aligned data section,
    tensors gate/up/down weight then scales; scripts/convert-mimo-v26-mlx.py:67-131).  Every tensor's size
    must be a multiple of 16 KiB, as the format requires."""
    tensors = []
    for proj, key in zip(PROJ, KEYS):
        for suffix, kind, dt in (("weight", "w", "U32"), ("scales", "s", "U8")):
            t = bank[f"{key}_{kind}"].detach().contiguous().cpu()
            raw = t.view(torch.uint8).numpy().tobytes() if t.dtype != torch.uint8 else t.numpy().tobytes()
            if len(raw) % ALIGN:
                raise ValueError(f"{key}_{kind}: {len(raw)} bytes is not a multiple of {ALIGN}")
            tensors.append((tensor_name(L, proj, suffix), dt, list(t.shape), raw))
    hdr, off = {}, 0
    for name, dt, shape, raw in tensors:
        hdr[name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    hdr["__metadata__"] = {"format": "mlx"}
    hj = json.dumps(hdr, separators=(",", ":")).encode()
    hj += b" " * ((-(8 + len(hj))) % ALIGN)
    tmp = path + ".partial"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for _, _, _, raw in tensors:
            f.write(raw)
    os.replace(tmp, path)


def router_names(L):
    return f"model.layers.{L}.mlp.gate.weight", f"model.layers.{L}.mlp.gate.e_score_correction_bias"


def load_router(model_dir, L, device="cuda", n_experts=pools.E, top_k=pools.TOPK):
    """Router of MoE layer L from dense.safetensors (engine/mimo_stream/model.py:120-124): bf16 weight
    [n_experts, hidden] and fp32 bias [n_experts], read with the safetensors loader (no pickle)."""
    from safetensors import safe_open
    from .model import Router
    wn, bn = router_names(L)
    with safe_open(os.path.join(model_dir, "dense.safetensors"), framework="pt") as f:
        names = set(f.keys())
        if wn not in names:
            raise ValueError(f"dense.safetensors: missing {wn}")
        W = f.get_tensor(wn)
        bias = f.get_tensor(bn) if bn in names else torch.zeros(W.shape[0], dtype=torch.float32)
    if W.dim() != 2 or W.shape[0] != n_experts or bias.shape != (n_experts,):
        raise ValueError(f"layer {L} router: weight {tuple(W.shape)}, bias {tuple(bias.shape)} for {n_experts} experts")
    r = Router(W.shape[1], n_experts, top_k, device=device)
    r.weight.copy_(W.to(torch.bfloat16))
    r.e_score_correction_bias.copy_(bias.to(torch.float32))
    return r


def load_block(model_dir, L, order=None, device="cuda", store=None):
    """MoEBlock of layer L: its router from dense.safetensors and its experts (all, or a slot order) from
    experts-LNN.safetensors; the slot table maps each loaded expert to its slot."""
    from .cache import SlotCache
    from .model import MoEBlock
    store = store or ExpertStore(model_dir, [L])
    router = load_router(model_dir, L, device=device, n_experts=store.n)
    bank = store.load_bank(L, order=order, device=device)
    if order is None:
        return MoEBlock(router, bank)
    sc = SlotCache(len(order), store.n)
    sc.preload(order)
    return MoEBlock(router, bank, slot_of=sc.slot_of)
