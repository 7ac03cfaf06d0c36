"""Expert compute and combine semantics (oracle; test infrastructure only).

Restated reference behaviour:
  * Kernel A (engine/mimo_stream/kernels.py:33-85): for every distinct expert u and each of its rows r,
      g = gate_u . x_row and up = up_u . x_row accumulated in fp32 (:50-77), gt = bf16(g), ut = bf16(up),
      h = bf16(bf16(gt * sigtab[gt]) * ut) (:79-82), with sigtab = bf16(sigmoid(bf16)) (:138-146).
  * Kernel B (kernels.py:88-123): part[u, r, m] = fp32(down_u[m] . h[u, r]) * uw[u, r] (:120), 0 for r >= cnt.
  * Combine (kernels.py:198-199): y[row] = bf16(sum over the row's k routes, in route order, of part).
  * M = 1 path _gather_m1 (engine/mimo_stream/model.py:173-182, :215): per expert a = bf16(gate.x),
      b = bf16(up.x), h = bf16(bf16(a * sig(a)) * b), y_e = bf16(down.h); y = bf16(sum_j fp32(y_e_j) * w_j).
  * Prefill _pair_outputs / _moe_prefill (model.py:221-228, :269-271): the same per (token, slot) pair as the
    M = 1 path, then the fixed-order weighted sum over k.

Dot products are accumulated in float64 over exactly dequantised weights and rounded once to fp32; the
reference accumulates in fp32 (Metal simd_sum / MLX gather_qmm order), so expert outputs are compared with a
stated tolerance while the rounding points above are reproduced exactly.
"""
import numpy as np
from . import mxfp4
from .routing import sigmoid_f32

_SIGTAB = None


def sigtab_bits():
    """uint16 [65536]: bf16(sigmoid(bf16 value with these bits)), sigmoid as routing.sigmoid_f32.
    Restates sigmoid_table (kernels.py:138-146) with the exactly specified sigmoid."""
    global _SIGTAB
    if _SIGTAB is None:
        vals = mxfp4.bf16_bits_to_f32(np.arange(1 << 16, dtype=np.uint32).astype(np.uint16))
        with np.errstate(invalid="ignore"):
            _SIGTAB = mxfp4.f32_to_bf16_bits(sigmoid_f32(vals))
    return _SIGTAB


def swiglu_bf16(g_f32, u_f32):
    """Kernel A epilogue (kernels.py:79-82): h = bf16(bf16(gt * sigtab[gt]) * ut), gt/ut = bf16(g/u)."""
    gt_bits = mxfp4.f32_to_bf16_bits(g_f32)
    gt = mxfp4.bf16_bits_to_f32(gt_bits)
    ut = mxfp4.round_bf16(u_f32)
    sig = mxfp4.bf16_bits_to_f32(sigtab_bits()[gt_bits])
    return mxfp4.round_bf16(mxfp4.round_bf16(gt * sig) * ut)


class ExpertPool:
    """Slot pool {gate_w, gate_s, up_w, up_s, down_w, down_s} (model.py:32-45) with exact dequantisation.

    cache=True keeps every dequantised projection (float64, 8 bytes per weight): for pools that are used many
    times; cache=False dequantises on each use (for sub-pools of many MiMo-sized experts, each used once)."""

    def __init__(self, pools, cache=True):
        self.p = {k: np.asarray(v) for k, v in pools.items()}
        self._cache = {} if cache else None

    def weights(self, name, slot):
        """float64 [out, in]: the exactly dequantised weights of one slot."""
        key = (name, int(slot))
        if self._cache is not None and key in self._cache:
            return self._cache[key]
        W = mxfp4.dequantize_mxfp4_f64(self.p[f"{name}_w"][slot], self.p[f"{name}_s"][slot])
        if self._cache is not None:
            self._cache[key] = W
        return W

    def dot(self, name, slot, rows):
        """rows float [n, in] -> fp32 [n, out]: float64 accumulation, one rounding to fp32."""
        W = self.weights(name, slot)
        return (np.asarray(rows, dtype=np.float64) @ W.T).astype(np.float32)


def kernel_a(x, pool, uslot, urows, ucnt, R):
    """h float32 (bf16 values) [U, R, N]; rows r >= ucnt[u] are 0.  kernels.py:33-85."""
    x = np.asarray(x, dtype=np.float32)
    U = len(uslot)
    N = pool.p["gate_w"].shape[1]
    h = np.zeros((U, R, N), np.float32)
    for u in range(U):
        c = int(ucnt[u])
        if c == 0:
            continue
        xr = x[np.asarray(urows[u][:c])]
        g = pool.dot("gate", uslot[u], xr)
        up = pool.dot("up", uslot[u], xr)
        h[u, :c] = swiglu_bf16(g, up)
    return h


def kernel_b(h, pool, uslot, ucnt, uw, round_expert_bf16=False):
    """part float32 [U, R, H] = fp32(down . h) * uw (kernels.py:88-123); rows r >= ucnt[u] are 0.
    round_expert_bf16 rounds the dot to bf16 first (the gather_qmm output of model.py:181, :228)."""
    U, R, _ = h.shape
    H = pool.p["down_w"].shape[1]
    part = np.zeros((U, R, H), np.float32)
    for u in range(U):
        c = int(ucnt[u])
        if c == 0:
            continue
        d = pool.dot("down", uslot[u], h[u, :c])
        if round_expert_bf16:
            d = mxfp4.round_bf16(d)
        part[u, :c] = (d * np.asarray(uw[u][:c], np.float32)[:, None]).astype(np.float32)
    return part


def combine(part, gidx, M, k):
    """y bf16-valued float32 [M, H]: sequential fp32 sum over each row's k routes in route order.
    kernels.py:198-199 (Y = part[gidx]; Y.sum(1).astype(bf16))."""
    U, R, H = part.shape
    flat = part.reshape(U * R, H)
    y = np.zeros((M, H), np.float32)
    for m in range(M):
        acc = np.zeros(H, np.float32)
        for j in range(k):
            acc = (acc + flat[int(gidx[m * k + j])]).astype(np.float32)
        y[m] = acc
    return mxfp4.round_bf16(y)


def moe_experts(x, pool, uslot, urows, ucnt, uw, gidx, k, R=8, round_expert_bf16=False):
    """moe_experts (kernels.py:176-199): Kernel A -> Kernel B -> fixed-order combine.  Returns (y, h, part)."""
    h = kernel_a(x, pool, uslot, urows, ucnt, R)
    part = kernel_b(h, pool, uslot, ucnt, uw, round_expert_bf16)
    y = combine(part, gidx, np.asarray(x).shape[0], k)
    return y, h, part


def pair_outputs(x, pool, tok, slot):
    """_pair_outputs (model.py:221-228): bf16 expert outputs for (token, slot) pairs -> float32 [P, H]."""
    x = np.asarray(x, dtype=np.float32)
    tok = np.asarray(tok)
    slot = np.asarray(slot)
    H = pool.p["down_w"].shape[1]
    out = np.zeros((len(tok), H), np.float32)

    def one(s):      # every slot's pairs are independent: slots run on a thread pool (numpy releases the GIL)
        sel = np.nonzero(slot == s)[0]
        xr = x[tok[sel]]
        h = swiglu_bf16(pool.dot("gate", s, xr), pool.dot("up", s, xr))
        out[sel] = mxfp4.round_bf16(pool.dot("down", s, h))

    slots = np.unique(slot)
    if len(slots) > 1:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(min(8, len(slots))) as ex:
            list(ex.map(one, slots))
    else:
        for s in slots:
            one(s)
    return out


def weighted_sum_bf16(Y, w):
    """y = bf16(sum_j fp32(Y[:, j]) * w[:, j]) with a sequential fp32 sum in j (model.py:182, :270-271)."""
    Y = np.asarray(Y, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    T, k, H = Y.shape
    acc = np.zeros((T, H), np.float32)
    for j in range(k):
        acc = (acc + (Y[:, j] * w[:, j, None]).astype(np.float32)).astype(np.float32)
    return mxfp4.round_bf16(acc)


def gather_m1(x_row, pool, slots, w):
    """_gather_m1 (model.py:173-182) + the caller's cast (:215): [H] bf16-valued float32."""
    Y = pair_outputs(np.asarray(x_row, np.float32).reshape(1, -1), pool, np.zeros(len(slots), np.int64), slots)
    return weighted_sum_bf16(Y[None], np.asarray(w, np.float32)[None])[0]


def moe_prefill(x, pool, slot_inds, w):
    """_moe_prefill with every expert resident (model.py:230-271): [T, H] bf16-valued float32."""
    x = np.asarray(x, dtype=np.float32)
    T, k = np.asarray(slot_inds).shape
    tok = np.repeat(np.arange(T), k)
    Y = pair_outputs(x, pool, tok, np.asarray(slot_inds).reshape(-1)).reshape(T, k, -1)
    return weighted_sum_bf16(Y, w)


def reference_fp32(x, pool, slot_inds, scores):
    """The reference test's own fp32 oracle (engine/tests/test_kernels.py:32-46): dequantised weights,
    fp32 SwiGLU g * sigmoid(g) * u with no bf16 rounding, weighted sum.  Returns float64 [M, H]."""
    x = np.asarray(x, dtype=np.float64)
    M = x.shape[0]
    H = pool.p["down_w"].shape[1]
    out = np.zeros((M, H))
    for m in range(M):
        for e, s in zip(slot_inds[m], scores[m]):
            g = pool.weights("gate", e) @ x[m]
            u = pool.weights("up", e) @ x[m]
            hh = (g / (1.0 + np.exp(-g))) * u
            out[m] += float(s) * (pool.weights("down", e) @ hh)
    return out


def rel_err(a, b):
    """max|a - b| / max|b| (engine/tests/test_kernels.py:54-56)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-9))
