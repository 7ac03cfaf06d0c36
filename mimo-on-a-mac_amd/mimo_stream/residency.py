"""MoE layers that keep fewer HBM slots than experts: missing experts are read from the converted checkpoint.

The MiMo-V2.6-Flash stack fits one MI355X's HBM (48 x 3.42 GB), so the engine's normal path keeps every expert
resident (`store.load_block`).  This module is the path for a smaller HBM budget, following the reference
engine (engine/mimo_stream/model.py:184-219 decode, :230-271 prefill, cache.py decayed LFU, store.py offsets):

  decode / verify (T <= 8 rows): the routes come back to the host (one synchronisation, as model.py:315), the
    slot cache assigns slots to the step's missing experts, their bytes are read from experts-LNN.safetensors
    into pinned host buffers and copied into the freed slots on a side stream that first waits for the work
    already queued on the compute stream (earlier steps may still read the victims' slots); the compute stream
    waits for the copies, takes the updated expert -> slot table and runs the block.  The decayed counts halve
    every `decay_every` decode calls (model.py:348-353).
  prefill (T > 8): the resident slots do not change (the reference streams non-resident experts into staging
    banks); here every needed expert goes to one staging bank (resident ones gathered from their slots on the
    device, the rest read from the checkpoint) and the prefill runs on it, so the result is bit-identical to a
    fully resident layer.
"""
import os

import numpy as np
import torch

from . import pools
from .cache import SlotCache
from .model import MoEBlock
from .store import KEYS, load_router


class StreamedMoEBlock:
    def __init__(self, store, L, n_slots, order=None, router=None, device="cuda", decay_every=16):
        self.dev = torch.device(device)
        self.store, self.L = store, L
        E = store.n
        if not 1 <= n_slots <= E:
            raise ValueError(f"n_slots must lie in [1, {E}]")
        order = list(range(E)) if order is None else [int(e) for e in order]
        self.cache = SlotCache(n_slots, E)
        self.cache.preload(order)
        bank = store.load_bank(L, order=order[:n_slots], device=self.dev)
        router = router or load_router(store.model_dir, L, device=self.dev, n_experts=E)
        self.block = MoEBlock(router, bank, slot_of=self.cache.slot_of)
        self.copy_stream = torch.cuda.Stream(self.dev)
        self.decay_every = decay_every
        self.decode_calls = 0
        self.experts_read = 0
        self._stage = None

    # ---------------------------------------------------------------- expert bytes into slots
    def _read_host(self, e):
        """Pinned host copies of expert e's six pool pieces (store.py:37-46 offsets)."""
        bufs, dst = {}, {}
        for key in KEYS:
            for kind in ("w", "s"):
                stride = self.store.loc[(self.L, key, kind)][2]
                t = torch.empty(stride, dtype=torch.uint8, pin_memory=True)
                bufs[(key, kind)] = t
                dst[(key, kind)] = memoryview(t.numpy())
        fds = {}
        try:
            for path, off, mv in self.store.jobs(self.L, e, dst):
                fd = fds.get(path)
                if fd is None:
                    fd = fds[path] = os.open(path, os.O_RDONLY)
                got = 0
                while got < mv.nbytes:
                    n = os.preadv(fd, [mv[got:]], off + got)
                    if n <= 0:
                        raise IOError(f"short read of expert {e} at {off + got}")
                    got += n
        finally:
            for fd in fds.values():
                os.close(fd)
        return bufs

    def _fill(self, bank, items):
        """items [(expert, slot)]: checkpoint bytes into bank slots, after the work queued so far on the current
        stream and before the work queued after this call (no host wait)."""
        if not items:
            return
        cur = torch.cuda.current_stream(self.dev)
        ready = torch.cuda.Event()
        ready.record(cur)
        hosts = [(s, self._read_host(e)) for e, s in items]
        self.copy_stream.wait_event(ready)
        with torch.cuda.stream(self.copy_stream):
            for s, bufs in hosts:
                for (key, kind), t in bufs.items():
                    bank[f"{key}_{kind}"][s].view(-1).view(torch.uint8).copy_(t, non_blocking=True)
        done = torch.cuda.Event()
        done.record(self.copy_stream)
        cur.wait_event(done)
        self.experts_read += len(items)

    def _push_table(self):
        tab = torch.empty(self.cache.E, dtype=torch.int32, pin_memory=True)
        tab.numpy()[:] = self.cache.slot_of
        self.block.slot_of.copy_(tab, non_blocking=True)

    def prefetch(self, experts):
        """Predicted experts of a coming step (model.py:320-329): the ones not resident get slots in the same
        eviction order, without counting as uses (resolve(count=False, stats=False)); their bytes are read now and
        copied on the side stream after the work already queued, so the reads overlap the GPU work queued before
        this call.  At most n_slots experts (the first ids given).  Returns the number of experts read."""
        ids = np.unique(np.asarray(experts, dtype=np.int64).reshape(-1))[: self.cache.S]
        if ids.size == 0:
            return 0
        loads = self.cache.resolve(ids, count=False, stats=False)
        self._fill(self.block.bank, loads)
        if loads:
            self._push_table()
        return len(loads)

    # ---------------------------------------------------------------- forward
    def __call__(self, r, return_routes=False):
        r2 = r.reshape(-1, r.shape[-1]).to(torch.bfloat16).contiguous()
        T = r2.shape[0]
        inds, w = self.block.router(r2)
        inds_h = inds.cpu().numpy()               # the host needs the routes to decide what to load
        if T <= pools.VERIFY_MAX:
            loads = self.cache.resolve(np.unique(inds_h))
            self._fill(self.block.bank, loads)
            if loads:
                self._push_table()
            y = self.block._moe_small(r2, inds, w, check=False)   # resolve gave every selected expert a slot
            self.decode_calls += 1
            if self.decode_calls % self.decay_every == 0:
                self.cache.decay()
        else:
            y = self._prefill(r2, inds_h, inds, w)
        return (y, inds, w) if return_routes else y

    def _prefill(self, r2, inds_h, inds, w):
        needed = np.unique(inds_h)
        held = self.cache.slot_of[needed]
        if (held >= 0).all():
            return self.block._moe_prefill(r2, inds, w, check=False)
        b = self.block._bank_struct
        if self._stage is None:
            self._stage = pools.alloc_bank(self.cache.E, b.hidden, b.inter, device=self.dev)
        res, mis = needed[held >= 0], needed[held < 0]
        n = needed.size
        stage = {k: v[:n] for k, v in self._stage.items()}
        stage_of = np.full(self.cache.E, -1, np.int32)
        stage_of[res] = np.arange(res.size, dtype=np.int32)
        stage_of[mis] = res.size + np.arange(mis.size, dtype=np.int32)
        if res.size:
            src = torch.from_numpy(self.cache.slot_of[res].astype(np.int64)).to(self.dev)
            for k, v in self.block.bank.items():
                torch.index_select(v, 0, src, out=stage[k][: res.size])
        self._fill(stage, [(int(e), int(stage_of[e])) for e in mis])
        return MoEBlock(self.block.router, stage, slot_of=stage_of)._moe_prefill(r2, inds, w, check=False)
