"""Pins of the group-limited selection of the vendored noaux-tc gate (engine/mimo_stream/mimo_v2.py:165-193)
restated in oracle.routing.select_topk_grouped: the n_group == 1 case against select_topk, a brute force
written from the definition on small rows, and the cases that tell its choices apart (masked keys set to 0
rather than excluded, no renormalisation for k == 1 or without norm_topk_prob, the scaling factor)."""
import itertools

import numpy as np
import pytest

from oracle import routing as orr


def brute(logits_row, bias, k, n_group, topk_group, norm, scale):
    s = orr.sigmoid_f32(logits_row[None])[0]
    key = [np.float32(np.float32(a) + np.float32(b)) for a, b in zip(s, bias)]
    E = len(key)
    G = E // n_group
    gscore = []
    for g in range(n_group):
        vals = sorted((v for v in key[g * G:(g + 1) * G] if v == v), reverse=True)
        vals += [np.float32(-np.inf)] * 2
        sc = np.float32(vals[0] + vals[1])
        gscore.append((-np.inf if sc != sc else float(sc), g))
    kept = {g for _, g in sorted(gscore, key=lambda p: (-p[0], p[1]))[:topk_group]}
    masked = [key[e] if e // G in kept else np.float32(0.0) for e in range(E)]
    order = sorted(range(E), key=lambda e: (masked[e] != masked[e], -float(masked[e]) if masked[e] == masked[e] else 0, e))
    sel = order[:k]
    w = [s[e] for e in sel]
    if norm and k > 1:
        acc = np.float32(0.0)
        for v in w:
            acc = np.float32(acc + v)
        w = [np.float32(v / np.float32(acc + np.float32(1e-20))) for v in w]
    if scale != 1.0:
        w = [np.float32(v * np.float32(scale)) for v in w]
    return np.array(sel, np.int32), np.array(w, np.float32)


def test_single_group_is_the_engine_router():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((16, 256)).astype(np.float32)
    b = (rng.standard_normal(256) * 0.1).astype(np.float32)
    for k in (2, 8):
        i1, w1 = orr.select_topk(lg, b, k, routed_scaling_factor=2.5)
        i2, w2 = orr.select_topk_grouped(lg, b, k, 1, 1, True, 2.5)
        np.testing.assert_array_equal(i1, i2)
        np.testing.assert_array_equal(w1, w2)


@pytest.mark.parametrize("E,n_group,topk_group,k", [(16, 4, 2, 3), (24, 3, 1, 4), (32, 8, 3, 6), (64, 8, 4, 8)])
def test_brute_force(E, n_group, topk_group, k):
    rng = np.random.default_rng(E + k)
    for norm, scale in itertools.product((True, False), (1.0, 2.5)):
        lg = rng.standard_normal((6, E)).astype(np.float32)
        lg[1, : E // 2] = lg[1, 0]                     # exact ties inside and across groups
        lg[2, 3] = np.nan                              # a NaN key
        b = (rng.standard_normal(E) * 0.3).astype(np.float32)
        inds, w = orr.select_topk_grouped(lg, b, k, n_group, topk_group, norm, scale)
        for t in range(6):
            bi, bw = brute(lg[t], b, k, n_group, topk_group, norm, scale)
            np.testing.assert_array_equal(inds[t], bi)
            np.testing.assert_array_equal(w[t], bw)


def test_masked_keys_are_zero_not_excluded():
    # every kept key is negative (bias -2): the masked groups' keys (0.0) outrank them
    E, n_group = 16, 4
    lg = np.zeros((1, E), np.float32)
    lg[0, :4] = 3.0                                    # group 0 scores highest
    b = np.full(E, -2.0, np.float32)
    inds, _ = orr.select_topk_grouped(lg, b, 2, n_group, 1)
    assert all(e >= 4 for e in inds[0])                # masked experts (key 0.0) beat group 0's negative keys
    np.testing.assert_array_equal(inds[0], [4, 5])     # ties at 0.0 to the lower ids


def test_renormalisation_and_scaling_rules():
    rng = np.random.default_rng(3)
    lg = rng.standard_normal((4, 64)).astype(np.float32)
    b = np.zeros(64, np.float32)
    s = orr.sigmoid_f32(lg)
    i1, w1 = orr.select_topk_grouped(lg, b, 1, 1, 1, True, 1.0)      # k == 1: no renormalisation (:190)
    np.testing.assert_array_equal(w1[:, 0], s[np.arange(4), i1[:, 0]])
    i2, w2 = orr.select_topk_grouped(lg, b, 4, 1, 1, False, 3.0)     # norm off: raw scores times the factor
    np.testing.assert_array_equal(w2, (s[np.arange(4)[:, None], i2] * np.float32(3.0)).astype(np.float32))
    i3, w3 = orr.select_topk_grouped(lg, b, 4, 1, 1, True, 1.0)
    np.testing.assert_allclose(w3.sum(1), 1.0, rtol=1e-6)
