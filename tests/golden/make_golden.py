"""Golden vectors for the MoE block, written by the CPU oracle (test infrastructure only).

    python tests/golden/make_golden.py          # rewrites tests/golden/moe_golden.npz

The reference commits no vectors for this path (its tests draw data with mx.random at run time,
engine/tests/test_kernels.py:21-29, :68-75), so these fixtures are the oracle's outputs on small seeded inputs,
pinned in git so that a change to the oracle or to the seeded inputs shows up as a diff:

  tiny_*    the tiny MoE layer (8 experts, top-2, hidden 256, intermediate 512, 4 bf16 token rows ~ N(0, 1),
            router weight ~ N(0, 0.02) in bf16, bias 0, experts MXFP4-quantised from N(0, 0.02)): router logits,
            routes, group_routes, the distinct-expert decode output (kernels.py:176-199), the per-row M = 1
            output (model.py:173-182) and the prefill output (model.py:230-271).  The expert pool is rebuilt
            from its seed by `tiny_pool` and pinned by its SHA-256.
  sel_*     selection given logits (model.py:60-64) on 256 experts, top-8, with exact ties, NaN, +-inf and a
            bias: the canonical order (key descending, lower id first, NaN last) and the renormalised weights.
  disp_*    the prefill dispatch (model.py:235-242, :266-268) of 40 tokens x 2 routes over 8 slots.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import experts as ox, mxfp4 as oq, routing as orr   # noqa: E402

PATH = os.path.join(HERE, "moe_golden.npz")
TINY = dict(E=8, k=2, H=256, I=512, T=4, seed=1201)


def tiny_pool(E=TINY["E"], H=TINY["H"], I=TINY["I"], seed=TINY["seed"]):
    """Expert pool of the tiny layer: per projection [E, out, in] ~ N(0, 0.02), rounded to bf16, MXFP4-quantised
    by the oracle (the reference's make_pool, engine/tests/test_kernels.py:21-29).  Returns the pool dict."""
    rng = np.random.default_rng(seed)
    p = {}
    for name, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        w = oq.round_bf16((rng.standard_normal((E * o, i)) * 0.02).astype(np.float32))
        q, s = oq.quantize_mxfp4(w)
        p[f"{name}_w"] = q.reshape(E, o, i // 8)
        p[f"{name}_s"] = s.reshape(E, o, i // 32)
    return p


def pool_sha256(p):
    h = hashlib.sha256()
    for key in ("gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s"):
        h.update(np.ascontiguousarray(p[key]).tobytes())
    return h.hexdigest()


def tiny_inputs(seed=TINY["seed"]):
    rng = np.random.default_rng(seed + 1)
    x = oq.round_bf16(rng.standard_normal((TINY["T"], TINY["H"])).astype(np.float32))
    Wg = oq.round_bf16((rng.standard_normal((TINY["E"], TINY["H"])) * 0.02).astype(np.float32))
    bias = np.zeros(TINY["E"], np.float32)
    return x, Wg, bias


def selection_logits():
    """[6, 256] fp32 logits with the cases the canonical order has to settle."""
    rng = np.random.default_rng(77)
    lg = (rng.standard_normal((6, 256)) * 2.0).astype(np.float32)
    lg[0, [3, 9, 200, 17]] = np.float32(4.0)                # four-way exact tie at the top-8 boundary
    lg[1, :] = np.float32(0.5)                                # every logit equal: the bias, then the lower ids
    lg[2, [5, 6]] = np.nan                                    # NaN keys go last
    lg[2, 7] = np.inf
    lg[3, [1, 2, 3]] = -np.inf
    lg[3, 10] = np.float32(90.0)                              # sigmoid saturates to 1.0
    lg[3, 11] = np.float32(95.0)                              # tie with the one above after the sigmoid
    lg[4, :] = np.float32(-30.0)                              # tiny scores: the 1e-20 guard shows in the weights
    lg[5, 100:108] = np.float32(6.0)                          # an eight-way tie split by the bias below
    return lg


def selection_bias():
    b = np.zeros(256, np.float32)
    b[104] = np.float32(1e-3)
    b[101] = np.float32(-1e-3)
    b[42] = np.float32(0.25)
    return b


def dispatch_slots():
    rng = np.random.default_rng(5)
    s = np.stack([rng.choice(8, 2, replace=False) for _ in range(40)]).astype(np.int32)
    s[:6] = [[3, 1], [3, 1], [1, 3], [0, 7], [7, 0], [3, 7]]
    return s


def build():
    T, k = TINY["T"], TINY["k"]
    pool = ox.ExpertPool(tiny_pool())
    x, Wg, bias = tiny_inputs()
    logits, inds, w = orr.router(x, Wg, bias, k)
    uids, urows, ucnt, uw, gidx = orr.group_routes(inds, w, R=8)
    y_small, _, _ = ox.moe_experts(x, pool, uids, urows, ucnt, uw, gidx, k, R=8)
    y_m1 = np.stack([ox.gather_m1(x[t], pool, inds[t], w[t]) for t in range(T)])
    y_prefill = ox.moe_prefill(x, pool, inds, w)
    lg, b = selection_logits(), selection_bias()
    sel_inds, sel_w = orr.select_topk(lg, b, 8)
    dslots = dispatch_slots()
    perm, offsets, inv = orr.prefill_dispatch(dslots, 8)
    bits = lambda a: oq.f32_to_bf16_bits(a).astype(np.uint16)
    return {
        "tiny_pool_sha256": np.array(pool_sha256(pool.p)),
        "tiny_x": bits(x), "tiny_wg": bits(Wg), "tiny_bias": bias,
        "tiny_logits": logits, "tiny_inds": inds, "tiny_w": w,
        "tiny_uids": uids, "tiny_urows": urows, "tiny_ucnt": ucnt, "tiny_uw": uw, "tiny_gidx": gidx,
        "tiny_y_small": bits(y_small), "tiny_y_m1": bits(y_m1), "tiny_y_prefill": bits(y_prefill),
        "sel_logits": lg, "sel_bias": b, "sel_inds": sel_inds, "sel_w": sel_w,
        "disp_slots": dslots, "disp_perm": perm, "disp_offsets": offsets, "disp_inv": inv,
    }


if __name__ == "__main__":
    d = build()
    np.savez_compressed(PATH, **d)
    print(f"wrote {PATH} ({os.path.getsize(PATH)} bytes): " + ", ".join(sorted(d)))
