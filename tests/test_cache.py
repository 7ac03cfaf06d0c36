"""Expert slot cache with decayed-LFU eviction (engine/mimo_stream/cache.py:13-65): policy cases, invariants on
random traces, and agreement with the oracle's restatement of the reference's scoring on every step whose
eviction choice the reference determines (no score tie at the eviction boundary)."""
import numpy as np
import pytest

from mimo_stream.cache import SlotCache
from oracle import routing as orr


def _check_consistent(c):
    occ = c.expert_in >= 0
    assert np.all(c.slot_of[c.expert_in[occ]] == np.nonzero(occ)[0])
    res = np.nonzero(c.slot_of >= 0)[0]
    assert np.all(c.expert_in[c.slot_of[res]] == res)


def test_empty_slots_first_then_lowest_count_then_lru():
    c = SlotCache(4, 16)
    assert c.resolve([3, 5]) == [(3, 0), (5, 1)]            # empty slots, lowest index first
    assert c.resolve([3, 7]) == [(7, 2)]
    assert c.resolve([9]) == [(9, 3)]
    # counts: 3 -> 2, 5 -> 1, 7 -> 1, 9 -> 1; last use: 5 at step 1, 7 at 2, 9 at 3
    assert c.resolve([3, 11]) == [(11, 1)]                 # evicts 5: count 1, least recently used
    assert c.slot_of[5] == -1 and (c.hits, c.misses) == (2, 5)
    assert c.resolve([7, 9, 3, 11]) == []                  # all resident
    # counts 3: 4, 7: 2, 9: 2, 11: 2, all last used at step 5: the tie among 7, 9 and 11 goes to the lowest slot,
    # slot 1 (expert 11)
    assert c.resolve([13]) == [(13, 1)]
    _check_consistent(c)


def test_needed_experts_are_never_evicted():
    c = SlotCache(3, 8)
    c.preload([0, 1, 2])
    for _ in range(5):
        c.resolve([0, 1])                                  # 0 and 1 become frequent
    loads = c.resolve([2, 5, 6])                           # 2 is needed although its count is the lowest
    assert sorted(s for _, s in loads) == [0, 1] and c.slot_of[2] == 2
    assert c.slot_of[0] == -1 and c.slot_of[1] == -1


def test_decay_lets_recent_experts_win():
    c = SlotCache(2, 8)
    for _ in range(4):
        c.resolve([0])
    c.resolve([1])
    c.resolve([1])
    c.resolve([2])                                         # 0 (count 4) survives, 1 (count 2) is evicted
    assert c.slot_of[0] >= 0 and c.slot_of[1] == -1
    c.resolve([1])                                         # 1 comes back in place of 2 (count 1)
    c.resolve([1])
    c.resolve([1])                                         # counts: 0 -> 4 (last used long ago), 1 -> 5
    for _ in range(3):
        c.decay()
    assert np.allclose(c.cnt[0], 4 / 8) and np.allclose(c.cnt[1], 5 / 8)
    c.resolve([3])                                         # 0 has the lower decayed count now
    assert c.slot_of[0] == -1 and c.slot_of[1] >= 0


def test_too_many_experts_and_bad_ids():
    c = SlotCache(2, 8)
    with pytest.raises(ValueError):
        c.resolve([0, 1, 2])
    c = SlotCache(4, 8)
    c.preload([0, 1, 2, 3])
    with pytest.raises(ValueError):                        # only 4 are missing, but 8 cannot share 4 slots
        c.resolve(list(range(8)))
    with pytest.raises(ValueError):
        c.resolve([8])


@pytest.mark.parametrize("S,E,k,seed", [(8, 32, 4, 0), (16, 64, 8, 1), (49, 256, 8, 2), (128, 256, 8, 3)])
def test_random_traces_match_reference_scoring(S, E, k, seed):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    c = SlotCache(S, E)
    st = {"slot_of": np.full(E, -1, np.int32), "expert_in": np.full(S, -1, np.int32), "cnt": np.zeros(E),
          "last": np.zeros(E, np.int64), "t": 0}
    compared = 0
    for step in range(400):
        rows = 1 + int(rng.integers(0, 2))
        needed = np.unique(np.concatenate([rng.choice(E, k, replace=False, p=p) for _ in range(rows)]))
        if needed.size > S:
            continue
        before = set(np.nonzero(c.slot_of >= 0)[0])
        loads = c.resolve(needed)
        loaded, evicted, tie = orr.lfu_resolve(st, needed)
        after = set(np.nonzero(c.slot_of >= 0)[0])
        assert set(needed) <= after and len(after) <= S
        assert sorted(e for e, _ in loads) == loaded
        assert {e for e, _ in loads}.isdisjoint(before)
        _check_consistent(c)
        if tie:                                            # the reference leaves this choice unspecified
            st["slot_of"][:] = c.slot_of
            st["expert_in"][:] = c.expert_in
            continue
        assert sorted(before - after) == evicted, step
        compared += 1
        if step % 16 == 15:
            c.decay()
            st["cnt"] *= 0.5
    assert compared > 200 and c.hits + c.misses > 0
