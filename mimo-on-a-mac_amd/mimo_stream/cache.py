"""Per-layer expert -> slot table (the slot-indexing contract of engine/mimo_stream/cache.py:13-29) with
decayed-LFU eviction (cache.py:31-65) for layers that keep fewer slots than experts.

Kernels address experts by slot.  SlotCache.preload fills slot s with the s-th expert of the given order
(engine/mimo_stream/model.py:158-167: popularity order, or expert s when no profile is given).  With every
expert resident (the MiMo-V2.6-Flash stack fits one MI355X's HBM) the table never changes.  With fewer slots,
resolve() makes a step's experts resident: each selection adds 1 to the expert's count (halved by decay(),
every 16 decode tokens in the engine, model.py:348-353) and stamps its last use; missing experts take the slots
of unneeded experts in the order empty slot, lowest count, least recently used.  Exact ties (same count and
same last use) go to the lower slot index here; the reference leaves them to np.argpartition's internal order.
A step needing more distinct experts than there are slots raises ValueError (the reference checks only the
missing ones against the slot count, cache.py:45-46, so such a step could evict experts it needs).
"""
import numpy as np
import torch


class SlotCache:
    def __init__(self, n_slots, n_experts=256):
        self.S = n_slots
        self.E = n_experts
        self.slot_of = np.full(n_experts, -1, np.int32)   # expert -> slot or -1
        self.expert_in = np.full(n_slots, -1, np.int32)   # slot -> expert or -1
        self.cnt = np.zeros(n_experts, np.float64)        # decayed selection count
        self.last = np.zeros(n_experts, np.int64)         # step of the last selection
        self.t = 0
        self.hits = 0
        self.misses = 0

    def preload(self, experts):
        experts = list(experts)[: self.S]
        for s, e in enumerate(experts):
            self.slot_of[e] = s
            self.expert_in[s] = e
        return list(zip(experts, range(len(experts))))

    def resolve(self, needed, count=True, stats=True):
        """needed: distinct experts of one step.  Returns [(expert, slot)] for the ones to load, after assigning
        them the slots of unneeded experts (empty first, then lowest decayed count, then least recent use)."""
        needed = np.unique(np.asarray(needed, dtype=np.int64))
        if needed.size and (needed[0] < 0 or needed[-1] >= self.E):
            raise ValueError(f"expert ids must lie in [0, {self.E})")
        if needed.size > self.S:   # the reference tests len(missing) > S, which lets such a step evict its own experts
            raise ValueError(f"step needs {needed.size} distinct experts but the layer holds {self.S} slots")
        self.t += 1
        if count:
            self.cnt[needed] += 1
        self.last[needed] = self.t
        missing = needed[self.slot_of[needed] < 0]
        if stats:
            self.hits += int(needed.size - missing.size)
            self.misses += int(missing.size)
        if missing.size == 0:
            return []
        protected = np.zeros(self.S, bool)
        held = self.slot_of[needed]
        protected[held[held >= 0]] = True
        cand = np.nonzero(~protected)[0]
        occ = self.expert_in[cand]
        empty = occ < 0
        e_safe = np.where(empty, 0, occ)
        # lexicographic (occupied, count, last use, slot): np.lexsort takes the primary key last
        order = np.lexsort((cand, np.where(empty, 0, self.last[e_safe]), np.where(empty, 0.0, self.cnt[e_safe]),
                            (~empty).astype(np.int8)))
        victims = cand[order[: missing.size]]
        loads = []
        for e, s in zip(missing, victims):
            old = self.expert_in[s]
            if old >= 0:
                self.slot_of[old] = -1
            self.expert_in[s] = e
            self.slot_of[e] = s
            loads.append((int(e), int(s)))
        return loads

    def decay(self):
        self.cnt *= 0.5

    def hit_rate(self):
        n = self.hits + self.misses
        return self.hits / n if n else 1.0

    def device_table(self, device="cuda"):
        """slot_of as an int32 device tensor (the form the kernels read)."""
        return torch.from_numpy(self.slot_of.copy()).to(device)
