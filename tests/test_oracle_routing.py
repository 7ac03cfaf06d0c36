"""Pins for oracle.routing (CPU only)."""
import numpy as np
import pytest

from oracle import routing, mxfp4


def test_exp_spec_within_one_ulp_of_libm():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-200, 200, 200000), rng.uniform(-1, 1, 100000), [0.0, 1.0, -1.0]])
    ours = routing.exp_spec(x)
    ref = np.exp(x)
    ulp = np.spacing(ref)
    assert np.max(np.abs(ours - ref) / ulp) <= 1.0
    assert routing.exp_spec(np.array([0.0]))[0] == 1.0


def test_sigmoid_f32_matches_libm_rounding():
    # fp32 rounding of the fp64 sigmoid computed with libm exp: equal except where the fp64 value lies
    # within one fp64 ulp of an fp32 rounding boundary (none expected in this sample)
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(300000) * 4, rng.uniform(-110, 110, 100000)]).astype(np.float32)
    ours = routing.sigmoid_f32(x)
    ref = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    np.testing.assert_array_equal(ours, ref)
    sp = routing.sigmoid_f32(np.array([np.inf, -np.inf, np.nan, 0.0], np.float32))
    assert sp[0] == 1.0 and sp[1] == 0.0 and np.isnan(sp[2]) and sp[3] == 0.5
    assert sp[2:3].view(np.uint32)[0] == 0x7FC00000       # canonical quiet NaN


def test_select_topk_set_matches_argpartition():
    rng = np.random.default_rng(2)
    T, E, k = 64, 256, 8
    logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 1e-3).astype(np.float32)
    inds, w = routing.select_topk(logits, bias, k)
    s = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
    key = s + bias
    part = np.argpartition(-key, kth=k - 1, axis=-1)[:, :k]       # model.py:62 with numpy's argpartition
    for t in range(T):
        assert set(inds[t]) == set(part[t])
        assert np.all(np.diff(key[t, inds[t]]) <= 0)               # canonical order: descending key
        ws = s[t, inds[t]].astype(np.float64)
        np.testing.assert_allclose(w[t], ws / ws.sum(), rtol=3e-7)
        assert abs(float(w[t].astype(np.float64).sum()) - 1.0) < 1e-6


def test_select_topk_ties_go_to_lower_id():
    logits = np.zeros((1, 16), np.float32)
    bias = np.zeros(16, np.float32)
    bias[[3, 9, 12]] = 0.5
    inds, w = routing.select_topk(logits, bias, 5)
    assert list(inds[0]) == [3, 9, 12, 0, 1]
    np.testing.assert_array_equal(w[0], np.float32(0.5) / np.float32(np.float32(2.5) + np.float32(1e-20)))


def test_select_bias_changes_selection_not_weights():
    # bias only steers selection (model.py:61); the weights come from the unbiased scores (:63)
    logits = np.array([[0.0, 1.0, 2.0, 3.0]], np.float32)
    inds, w = routing.select_topk(logits, np.array([10.0, 0, 0, 0], np.float32), 2)
    assert list(inds[0]) == [0, 3]
    s = routing.sigmoid_f32(logits)[0]
    np.testing.assert_allclose(w[0], [s[0] / (s[0] + s[3]), s[3] / (s[0] + s[3])], rtol=1e-6)


def test_group_routes_hand_example():
    inds = np.array([[5, 2], [2, 7]])
    scores = np.array([[0.6, 0.4], [0.3, 0.7]], np.float32)
    uids, urows, ucnt, uw, gidx = routing.group_routes(inds, scores, R=4)
    assert list(uids) == [2, 5, 7]
    assert list(ucnt) == [2, 1, 1]
    assert urows[0, :2].tolist() == [0, 1] and urows[1, 0] == 0 and urows[2, 0] == 1
    np.testing.assert_array_equal(uw[0, :2], np.array([0.4, 0.3], np.float32))
    assert gidx.tolist() == [1 * 4 + 0, 0 * 4 + 0, 0 * 4 + 1, 2 * 4 + 0]


def test_group_routes_invariants_and_overflow():
    rng = np.random.default_rng(3)
    for M in (1, 2, 4, 8):
        inds = np.stack([rng.choice(24, 8, replace=False) for _ in range(M)])
        if M > 1:
            inds[1, :4] = inds[0, :4]
        scores = rng.random((M, 8)).astype(np.float32)
        uids, urows, ucnt, uw, gidx = routing.group_routes(inds, scores, R=8)
        np.testing.assert_array_equal(uids, np.unique(inds))
        assert len(set(gidx.tolist())) == M * 8                       # every route has its own slot
        for t in range(M * 8):
            u, c = divmod(int(gidx[t]), 8)
            assert uids[u] == inds.reshape(-1)[t] and urows[u, c] == t // 8 and uw[u, c] == scores.reshape(-1)[t]
            assert c < ucnt[u]
        # rows of one expert appear in route order
        for u in range(len(uids)):
            assert np.all(np.diff(urows[u, :ucnt[u]]) >= 0)
    with pytest.raises(ValueError):
        routing.group_routes(np.zeros((3, 2), np.int64), np.ones((3, 2), np.float32), R=4)


def test_prefill_dispatch_is_stable_sort():
    rng = np.random.default_rng(4)
    T, k, S = 300, 8, 32
    slots = np.stack([rng.choice(S, k, replace=False) for _ in range(T)])
    perm, offsets, inv = routing.prefill_dispatch(slots, S)
    flat = slots.reshape(-1)
    brute = sorted(range(T * k), key=lambda i: (flat[i], i))
    assert perm.tolist() == brute
    np.testing.assert_array_equal(inv[perm], np.arange(T * k))
    np.testing.assert_array_equal(np.diff(offsets), np.bincount(flat, minlength=S))
    for s in range(S):
        assert np.all(flat[perm[offsets[s]:offsets[s + 1]]] == s)


def test_slot_table():
    so = routing.slot_table(8, order=[3, 1, 4], n_slots=3)
    assert so.tolist() == [-1, 1, -1, 0, 2, -1, -1, -1]
    assert routing.slot_table(4).tolist() == [0, 1, 2, 3]
