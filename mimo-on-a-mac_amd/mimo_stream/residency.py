"""MoE layers that keep fewer HBM slots than experts: missing experts are read from the converted checkpoint.

The MiMo-V2.6-Flash stack fits one MI355X's HBM (48 x 3.42 GB), so the engine's normal path keeps every expert
resident (`store.load_block`).  This module is the path for a smaller HBM budget, following the reference
engine (engine/mimo_stream/model.py:184-219 decode, :230-271 prefill, :273-285 staging prefetch, cache.py
decayed LFU, store.py offsets):

  decode / verify (T <= 8 rows): the routes come back to the host (one synchronisation, as model.py:315), the
    slot cache assigns slots to the step's missing experts, their bytes are read from experts-LNN.safetensors
    into pinned host buffers and copied into the freed slots on a side stream that first waits for the work
    already queued on the compute stream (earlier steps may still read the victims' slots); the compute stream
    waits for the copies, takes the updated expert -> slot table and runs the block.  The decayed counts halve
    every `decay_every` decode calls (model.py:348-353).
  prefill (T > 8): the resident slots do not change.  The non-resident experts the chunk needs are copied into
    one of two staging banks of E - S slots that every streamed layer of a stack shares (StagingBanks,
    model.py:140-143), and one mimo_moe_prefill_staged call reads resident routes from the layer's bank and
    staged routes from the staging bank, so the result is bit-identical to a fully resident layer.  The copies
    into a staging bank wait only for the last prefill that read that bank, so a layer's staging overlaps the
    previous layer's prefill; prefetch_stage() streams all of a layer's non-resident experts ahead of its routes
    (model.py:273-285, started after the previous layer's prefill is queued, :336-339).
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import _lib, pools
from .cache import SlotCache
from .model import MoEBlock
from .store import KEYS, load_router


class StagingBanks:
    """Two staging banks of n slots each, shared by the streamed layers of a stack (model.py:140-143: E - S
    slots, double buffered).  A prefill computes from one bank while the next layer's experts are copied into
    the other; each bank is allocated on first use and keeps the event after the last prefill that read it."""

    def __init__(self, n, hidden=pools.HIDDEN, inter=pools.INTER, device="cuda"):
        if n < 1:
            raise ValueError("a staging bank needs at least one slot")
        self.n, self.hidden, self.inter = int(n), int(hidden), int(inter)
        self.dev = torch.device(device)
        self.banks = [None, None]
        self.last_read = [None, None]     # event recorded after the last prefill that read bank i
        self.fills = [0, 0]               # bumped whenever bank i's contents are replaced
        self.turn = 0

    def take(self):
        """The bank to fill next (alternating); allocates it on first use."""
        i = self.turn
        self.turn ^= 1
        if self.banks[i] is None:
            self.banks[i] = pools.alloc_bank(self.n, self.hidden, self.inter, device=self.dev)
        self.fills[i] += 1
        return i

    def nbytes(self):
        """Device bytes held by the allocated banks."""
        return sum(t.numel() * t.element_size() for b in self.banks if b is not None for t in b.values())


class StreamedMoEBlock:
    def __init__(self, store, L, n_slots, order=None, router=None, device="cuda", decay_every=16, staging=None):
        """staging: StagingBanks shared with the stack's other streamed layers (at least E - n_slots slots); by
        default the block makes its own, allocated at its first prefill that needs a non-resident expert."""
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
        b = self.block._bank_struct
        if staging is None and n_slots < E:
            staging = StagingBanks(E - n_slots, b.hidden, b.inter, device=self.dev)
        if staging is not None:
            if staging.n < E - n_slots or (staging.hidden, staging.inter) != (b.hidden, b.inter):
                raise ValueError(f"staging banks of {staging.n} slots ({staging.hidden} x {staging.inter}) for "
                                 f"{E - n_slots} non-resident experts ({b.hidden} x {b.inter})")
        self.staging = staging
        self._stage_pref = None           # (bank, fill id, expert -> staging slot) of a prefetch_stage
        self.status = torch.zeros(1, dtype=torch.int32, device=self.dev)

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

    def _fill(self, bank, items, after=False):
        """items [(expert, slot)]: checkpoint bytes into bank slots, before the work queued after this call on
        the current stream (no host wait).  The copies start after `after` (an event; None: at once), by default
        after the work queued so far on the current stream."""
        if not items:
            return
        cur = torch.cuda.current_stream(self.dev)
        if after is False:
            after = torch.cuda.Event()
            after.record(cur)
        if len(items) > 1:
            with ThreadPoolExecutor(max_workers=min(8, len(items))) as ex:
                hosts = list(zip([s for _, s in items], ex.map(self._read_host, [e for e, _ in items])))
        else:
            hosts = [(s, self._read_host(e)) for e, s in items]
        if after is not None:
            self.copy_stream.wait_event(after)
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
        if T == 0:                          # an empty batch: nothing to route or load
            return self.block(r2, return_routes=return_routes)
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

    def prefetch_stage(self):
        """Stream every expert without a resident slot into the next staging bank, ahead of this layer's prefill
        (model.py:273-285; the reference starts it once the previous layer's prefill is queued, :336-339, so
        the reads overlap that prefill).  The next prefill takes its staged experts from this bank when the bank
        has not been refilled meanwhile.  Returns the number of experts read."""
        if self.staging is None:
            return 0
        nonres = np.nonzero(self.cache.slot_of < 0)[0]
        if nonres.size == 0:
            return 0
        i = self.staging.take()
        stage_of = np.full(self.cache.E, -1, np.int32)
        stage_of[nonres] = np.arange(nonres.size, dtype=np.int32)
        self._fill(self.staging.banks[i], [(int(e), int(stage_of[e])) for e in nonres], after=self.staging.last_read[i])
        self._stage_pref = (i, self.staging.fills[i], stage_of)
        return int(nonres.size)

    def _prefill(self, r2, inds_h, inds, w):
        needed = np.unique(inds_h)
        held = self.cache.slot_of[needed]
        pref, self._stage_pref = self._stage_pref, None
        if (held >= 0).all():
            return self.block._moe_prefill(r2, inds, w, check=False)
        mis = needed[held < 0]
        sg = self.staging
        if pref is not None and sg.fills[pref[0]] == pref[1] and (pref[2][mis] >= 0).all():
            i, _, stage_of = pref             # a prefetch_stage already holds them
        else:
            i = sg.take()
            stage_of = np.full(self.cache.E, -1, np.int32)
            stage_of[mis] = np.arange(mis.size, dtype=np.int32)
            self._fill(sg.banks[i], [(int(e), int(stage_of[e])) for e in mis], after=sg.last_read[i])
        S = self.cache.S
        tab = self.cache.slot_of.astype(np.int32)
        tab[mis] = S + stage_of[mis]
        tab_h = torch.from_numpy(tab).pin_memory()
        slot_inds = tab_h.to(self.dev, non_blocking=True)[inds.to(torch.int64)].contiguous()
        y = self._prefill_staged(r2, slot_inds, w, sg.banks[i])
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(self.dev))
        sg.last_read[i] = done
        return y

    def _prefill_staged(self, r2, slot_inds, w, stage):
        """mimo_moe_prefill_staged: slot ids below S read the layer's bank, S + j slot j of the staging bank."""
        T, k = slot_inds.shape
        dev = r2.device
        x = r2.to(torch.bfloat16).contiguous()
        w = w.to(torch.float32).contiguous()
        b = self.block._bank_struct
        sb = pools.bank_struct(stage)
        y = torch.empty((T, b.hidden), dtype=torch.bfloat16, device=dev)
        nbytes = _lib.load().mimo_moe_prefill_workspace_size(T, k, b.n_slots + sb.n_slots, b.hidden, b.inter)
        ws = _lib.workspace(nbytes, dev, "prefill")
        _lib.call("mimo_moe_prefill_staged", _lib.ptr(x), T, _lib.ptr(slot_inds), _lib.ptr(w), k, b, sb,
                  _lib.ptr(y), _lib.ptr(self.status), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
        return y
