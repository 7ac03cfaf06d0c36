"""Per-layer expert -> slot table (the slot-indexing contract of engine/mimo_stream/cache.py:13-29).

Kernels address experts by slot.  SlotCache.preload fills slot s with the s-th expert of the given order
(engine/mimo_stream/model.py:158-167: popularity order, or expert s when no profile is given).  Eviction and
SSD streaming (cache.py:31-65) are not needed when every expert is resident in HBM.
"""
import numpy as np
import torch


class SlotCache:
    def __init__(self, n_slots, n_experts=256):
        self.S = n_slots
        self.slot_of = np.full(n_experts, -1, np.int32)   # expert -> slot or -1
        self.expert_in = np.full(n_slots, -1, np.int32)   # slot -> expert or -1

    def preload(self, experts):
        experts = list(experts)[: self.S]
        for s, e in enumerate(experts):
            self.slot_of[e] = s
            self.expert_in[s] = e
        return list(zip(experts, range(len(experts))))

    def device_table(self, device="cuda"):
        """slot_of as an int32 device tensor (the form the kernels read)."""
        return torch.from_numpy(self.slot_of.copy()).to(device)
