"""Router, distinct-expert grouping and prefill dispatch (oracle; test infrastructure only).

Reference functions restated here:
  * Router.__call__            engine/mimo_stream/model.py:58-65
  * group_expert_select        engine/mimo_stream/mimo_v2.py:165-193 (select_topk: n_group == 1 with
                               renormalisation; select_topk_grouped: every option of the vendored gate)
  * SlotCache.slot_of          engine/mimo_stream/cache.py:16-17, :24-29 (expert -> slot)
  * group_routes               engine/mimo_stream/kernels.py:149-173
  * _moe_prefill dispatch      engine/mimo_stream/model.py:235-242, :266-268 (stable sort by slot, inverse)

Two choices the reference leaves to MLX internals are fixed here, identically on CPU and GPU:
  * sigmoid: sigmoid_f32(l) = fp32(1 / (1 + exp_spec(-l))) evaluated in IEEE double with the fixed operation
    sequence of exp_spec (Cody-Waite reduction by ln 2, degree-13 Taylor polynomial in Horner form, exact
    ldexp).  Every step is a correctly rounded IEEE operation, so any platform that does not contract the
    multiply-adds reproduces it bit for bit.
  * top-k order: descending selection key, ties to the lower expert id, NaN keys last.  MLX's argpartition
    returns the same index *set* (up to exact ties) in an unspecified order; this order fixes the fp32
    renormalisation sum (sequential in selection order) and the route order the combine sums in.
"""
import math
import numpy as np

# Cody-Waite split of ln 2 (fdlibm constants): LN2_HI has 32 significant bits, so n * LN2_HI is exact for
# |n| < 2^20.
LN2_HI = float.fromhex("0x1.62e42feep-1")
LN2_LO = float.fromhex("0x1.a39ef35793c76p-33")
INV_LN2 = float.fromhex("0x1.71547652b82fep+0")
# 1/k! for k = 0..13, each correctly rounded to double
EXP_TAYLOR = [1.0 / math.factorial(k) for k in range(14)]
SIGMOID_CLAMP = 200.0     # |x| beyond this cannot change the fp32 result of the sigmoid


def exp_spec(x):
    """exp(x) for float64 arrays, |x| <= 200, with the fixed IEEE operation sequence described above."""
    x = np.asarray(x, dtype=np.float64)
    n = np.rint(x * INV_LN2)
    r = (x - n * LN2_HI) - n * LN2_LO
    p = np.full_like(r, EXP_TAYLOR[13])
    for k in range(12, -1, -1):
        p = p * r + EXP_TAYLOR[k]
    return np.ldexp(p, n.astype(np.int64))


def sigmoid_f32(logits):
    """Elementwise fp32 sigmoid, exactly specified (see module docstring); a NaN input gives the canonical
    quiet NaN 0x7FC00000.  model.py:60."""
    x = np.asarray(logits, dtype=np.float32).astype(np.float64)
    nan = np.isnan(x)
    x = np.where(nan, 0.0, x)
    x = np.where(x < -SIGMOID_CLAMP, -SIGMOID_CLAMP, np.where(x > SIGMOID_CLAMP, SIGMOID_CLAMP, x))
    e = exp_spec(-x)
    out = (1.0 / (1.0 + e)).astype(np.float32)
    return np.where(nan, np.array([0x7FC00000], np.uint32).view(np.float32)[0], out).astype(np.float32)


def router_logits(x_bf16_as_f32, W_bf16_as_f32):
    """logits = r.f32 @ W.f32^T (model.py:59), accumulated in float64 then rounded to fp32.

    The reference accumulates in fp32 in MLX's order; any fp32 order differs from this by rounding only, so
    logits are compared with a tolerance and the selection is checked bit-exactly *given* the same logits."""
    x = np.asarray(x_bf16_as_f32, dtype=np.float64)
    W = np.asarray(W_bf16_as_f32, dtype=np.float64)
    return (x @ W.T).astype(np.float32)


def select_topk(logits, bias, k, routed_scaling_factor=1.0):
    """Selection given fp32 logits [T, E]: model.py:60-64 (and mimo_v2.py:175-192 with n_group == 1).

    Returns inds int32 [T, k] in canonical order and w float32 [T, k]:
      s = sigmoid_f32(logits); key = s + bias (fp32); order by (-key, expert id) with NaN keys last;
      w = s[inds] / (sum_in_selection_order(s[inds]) + 1e-20f), then * routed_scaling_factor (fp32)."""
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    s = sigmoid_f32(logits)
    key = (s + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    inds = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    ids = np.arange(E)
    for t in range(T):
        kt = key[t]
        nan = np.isnan(kt)
        # lexsort: last key is primary -> (nan last, -key descending, id ascending)
        order = np.lexsort((ids, -np.where(nan, 0, kt), nan))
        sel = order[:k]
        inds[t] = sel
        acc = np.float32(0.0)
        for j in range(k):
            acc = np.float32(acc + s[t, sel[j]])
        denom = np.float32(acc + np.float32(1e-20))
        w[t] = (s[t, sel] / denom).astype(np.float32)
        if routed_scaling_factor != 1.0:
            w[t] = (w[t] * np.float32(routed_scaling_factor)).astype(np.float32)
    return inds, w


def group_mask_keys(key, n_group, topk_group):
    """mimo_v2.py:178-186 on one row of fp32 keys [E]: the experts split into n_group consecutive groups; a
    group's score is the fp32 sum of its two largest keys (mx.topk(scores, 2)); every group outside the
    topk_group highest scores has its keys set to 0.0.  Fixed here where MLX leaves it open: ties between group
    scores go to the lower group index; NaN keys never count among a group's two largest (a group with fewer
    than two non-NaN keys scores -inf), and a NaN score ranks lowest."""
    key = np.asarray(key, np.float32)
    E = key.shape[0]
    G = E // n_group
    scores = np.empty(n_group, np.float32)
    for g in range(n_group):
        v = key[g * G:(g + 1) * G]
        v = np.sort(v[~np.isnan(v)])[::-1]
        top = list(v[:2]) + [np.float32(-np.inf)] * (2 - min(2, len(v)))
        sc = np.float32(np.float32(top[0]) + np.float32(top[1]))
        scores[g] = -np.inf if np.isnan(sc) else sc
    order = np.lexsort((np.arange(n_group), -scores))        # score descending, lower index first
    out = key.copy()
    for g in order[topk_group:]:
        out[g * G:(g + 1) * G] = np.float32(0.0)
    return out


def select_topk_grouped(logits, bias, k, n_group=1, topk_group=1, norm_topk_prob=True, routed_scaling_factor=1.0):
    """group_expert_select (mimo_v2.py:165-193) given fp32 logits [T, E]: s = sigmoid_f32(logits); key = s + bias;
    with n_group > 1 the group mask of group_mask_keys; canonical order of the keys (descending, ties to the
    lower id, NaN last); w = s at the chosen experts, divided by (their sum in selection order + 1e-20f) only when
    norm_topk_prob and k > 1 (:190-191), times routed_scaling_factor (:192)."""
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    s = sigmoid_f32(logits)
    key = (s + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    inds = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    ids = np.arange(E)
    for t in range(T):
        kt = group_mask_keys(key[t], n_group, topk_group) if n_group > 1 else key[t]
        nan = np.isnan(kt)
        order = np.lexsort((ids, -np.where(nan, 0, kt), nan))
        sel = order[:k]
        inds[t] = sel
        wt = s[t, sel].astype(np.float32)
        if norm_topk_prob and k > 1:
            acc = np.float32(0.0)
            for j in range(k):
                acc = np.float32(acc + wt[j])
            wt = (wt / np.float32(acc + np.float32(1e-20))).astype(np.float32)
        if routed_scaling_factor != 1.0:
            wt = (wt * np.float32(routed_scaling_factor)).astype(np.float32)
        w[t] = wt
    return inds, w


def router(x_bf16_as_f32, W_bf16_as_f32, bias, k):
    """Router.__call__ (model.py:58-65): (logits, inds, w)."""
    logits = router_logits(x_bf16_as_f32, W_bf16_as_f32)
    inds, w = select_topk(logits, bias, k)
    return logits, inds, w


def slot_table(n_experts, order=None, n_slots=None):
    """SlotCache.preload (cache.py:24-29) on an empty table: slot s <- order[s]; returns slot_of int32 [E]
    (-1 = not resident).  order=None means expert s in slot s (model.py:163, profile=None)."""
    order = np.arange(n_experts) if order is None else np.asarray(order)
    n_slots = len(order) if n_slots is None else n_slots
    slot_of = np.full(n_experts, -1, np.int32)
    for s, e in enumerate(list(order)[:n_slots]):
        slot_of[e] = s
    return slot_of


def group_routes(inds, scores, R=8):
    """Distinct-expert grouping, kernels.py:149-173, restated line for line.

    inds [M, k] slot ids, scores [M, k] -> uids [U] ascending, urows int32 [U, R] (0-padded),
    ucnt int32 [U], uw float32 [U, R] (0-padded), gidx uint32 [M*k] = u*R + c.
    Raises ValueError when more than R routes land on one expert (kernels.py:167-168)."""
    inds = np.asarray(inds)
    M, k = inds.shape
    flat = inds.reshape(-1)
    uids, inv = np.unique(flat, return_inverse=True)
    U = len(uids)
    urows = np.zeros((U, R), np.int32)
    uw = np.zeros((U, R), np.float32)
    ucnt = np.zeros(U, np.int32)
    rows = np.repeat(np.arange(M), k)
    sc = np.asarray(scores, dtype=np.float32).reshape(-1)
    gidx = np.zeros(flat.size, np.uint32)
    for t in range(flat.size):
        u = inv[t]
        c = ucnt[u]
        if c >= R:
            raise ValueError("more rows than R routed to one expert")
        urows[u, c] = rows[t]
        uw[u, c] = sc[t]
        gidx[t] = u * R + c
        ucnt[u] = c + 1
    return uids, urows, ucnt, uw, gidx


def prefill_dispatch(slot_inds, n_slots):
    """Stable sort of the flat (token, k) routes by slot: model.py:235-242 and the inverse of :266-268.

    slot_inds int [T, k] -> perm int32 [T*k] (sorted position -> flat route index t*k + j),
    offsets int32 [n_slots + 1] (rows of slot s are perm[offsets[s]:offsets[s+1]]),
    inv int32 [T*k] (flat route -> sorted position)."""
    flat = np.asarray(slot_inds).reshape(-1)
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=n_slots)
    offsets = np.zeros(n_slots + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size, dtype=np.int32)
    return perm, offsets, inv


def lfu_resolve(state, needed, count=True):
    """Decayed-LFU slot assignment of cache.py:31-62 for one step.

    state: dict with slot_of [E], expert_in [S], cnt [E] float64, last [E] int64, t (mutated in place).
    Victim score of an occupied slot: cnt * 1e12 + last; empty slots score -1; slots of needed experts are
    protected; the len(missing) lowest scores are evicted.  Returns (sorted loaded experts, evicted experts,
    boundary_tie): boundary_tie is True when the last victim's score equals the next candidate's, where the
    reference's np.argpartition choice is unspecified (callers compare only tie-free steps)."""
    needed = np.unique(np.asarray(needed))
    state["t"] += 1
    if count:
        state["cnt"][needed] += 1
    state["last"][needed] = state["t"]
    slot_of, exp = state["slot_of"], state["expert_in"]
    missing = needed[slot_of[needed] < 0]
    if len(missing) == 0:
        return [], [], False
    S = len(exp)
    score = np.array([-1.0 if exp[s] < 0 else state["cnt"][exp[s]] * 1e12 + state["last"][exp[s]] for s in range(S)])
    for e in needed:
        if slot_of[e] >= 0:
            score[slot_of[e]] = np.inf
    order = np.argsort(score, kind="stable")
    victims = order[: len(missing)]
    tie = len(missing) < S and score[order[len(missing) - 1]] == score[order[len(missing)]] and \
        score[order[len(missing) - 1]] >= 0
    evicted = []
    for e, s in zip(missing, victims):
        if exp[s] >= 0:
            evicted.append(int(exp[s]))
            slot_of[exp[s]] = -1
        exp[s] = e
        slot_of[e] = s
    return sorted(int(e) for e in missing), sorted(evicted), bool(tie)
