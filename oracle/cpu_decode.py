"""The MoE block's one-row decode on the host CPU in fp32 with PyTorch on every core: the CPU baseline the
benchmark reports beside the GPU figure (oracle package: test and benchmark infrastructure only, never on the
product path).

It restates the same reference algorithm as oracle.routing / oracle.experts, as a CPU implementation would run
it rather than as a pin:
  Router.__call__ (engine/mimo_stream/model.py:58-65): logits = x.f32 @ W.f32^T, s = sigmoid(logits), top-8 of
    s + e_score_correction_bias, w = s[inds] / (sum + 1e-20);
  _gather_m1 (model.py:173-182): per selected expert the MXFP4 weights are dequantised (E2M1 nibbles low first,
    one E8M0 scale per 32, kernels.py:5-30), a = bf16(gate . x), b = bf16(up . x), h = bf16(bf16(a * sig(a)) * b)
    with sig the bf16 sigmoid table (kernels.py:79-82, :138-146), y_e = bf16(down . h), y = bf16(sum_j y_e_j * w_j).
Dot products accumulate in fp32 in PyTorch's order and torch.sigmoid gives the sigmoid, so results agree with the
oracle within the same bf16 tolerance as the GPU path (tests/test_oracle_cpu_decode.py).

Two ways to form each expert's matrix-vector products are kept: `gather_m1` dequantises the whole weight matrix
to fp32 and multiplies (the plain port), `gather_m1_grouped` never forms it: per block of rows it sums the
unscaled E2M1 values times x within each 32-element group and then multiplies the group sums by the group's
E8M0 scale (the order a CPU kernel for the format would use)."""
import torch

from .mxfp4 import E2M1_VALUES

_PAIRS = torch.stack([torch.from_numpy(E2M1_VALUES)[torch.arange(256) & 15],
                      torch.from_numpy(E2M1_VALUES)[torch.arange(256) >> 4]], 1).contiguous()   # [256, 2] fp32


def dequantize(q, s):
    """q int32 [out, in/8] (32-bit words of eight nibbles), s uint8 [out, in/32] -> fp32 [out, in]."""
    out_dim = q.shape[0]
    K = q.shape[1] * 8
    b = q.contiguous().view(torch.uint8).reshape(-1).to(torch.int32)          # little-endian bytes: low first
    v = torch.index_select(_PAIRS, 0, b).reshape(out_dim, K // 32, 32)
    sc = torch.ldexp(torch.ones((), dtype=torch.float32), s.to(torch.int32) - 127)
    sc = torch.where(s == 255, torch.full_like(sc, float("nan")), sc)
    return (v * sc.unsqueeze(-1)).reshape(out_dim, K)


def _bf16(t):
    return t.to(torch.bfloat16).to(torch.float32)


def route(x, W, bias, k):
    """x fp32 [H] (bf16 values), W fp32 [E, H], bias fp32 [E] -> (inds int64 [k], w fp32 [k])."""
    logits = W @ x
    s = torch.sigmoid(logits)
    _, inds = torch.topk(s + bias, k)
    sel = s[inds]
    return inds, sel / (sel.sum() + 1e-20)


def gather_m1(x, pools, inds, w):
    """x fp32 [H]; pools {gate_w, gate_s, up_w, up_s, down_w, down_s} CPU tensors indexed by expert ->
    y fp32 [H] holding bf16 values."""
    acc = torch.zeros(pools["down_w"].shape[1], dtype=torch.float32)
    for j in range(inds.numel()):
        e = int(inds[j])
        g = _bf16(dequantize(pools["gate_w"][e], pools["gate_s"][e]) @ x)
        u = _bf16(dequantize(pools["up_w"][e], pools["up_s"][e]) @ x)
        h = _bf16(_bf16(g * _bf16(torch.sigmoid(g))) * u)
        ye = _bf16(dequantize(pools["down_w"][e], pools["down_s"][e]) @ h)
        acc = acc + ye * w[j]
    return _bf16(acc)


def group_dot(q, s, x, rows=128):
    """q int32 [out, in/8], s uint8 [out, in/32], x fp32 [in] -> fp32 [out]: y[o] = sum over groups g of
    2^(s[o, g] - 127) * sum_j e2m1(q[o, 32 g + j]) * x[32 g + j] (scale 255: NaN), `rows` rows at a time, so no
    fp32 copy of the matrix is formed (only the unscaled values of one block of rows)."""
    out_dim, G = s.shape
    xg = x.reshape(G, 16, 2)
    sc = torch.ldexp(torch.ones((), dtype=torch.float32), s.to(torch.int32) - 127)
    sc = torch.where(s == 255, torch.full_like(sc, float("nan")), sc)
    y = torch.empty(out_dim, dtype=torch.float32)
    for r0 in range(0, out_dim, rows):
        b = q[r0:r0 + rows].contiguous().view(torch.uint8).reshape(-1).to(torch.int32)
        v = torch.index_select(_PAIRS, 0, b).reshape(-1, G, 16, 2)       # unscaled values, low nibble first
        part = (v * xg).sum((2, 3))                                        # [rows, G] group sums
        y[r0:r0 + rows] = (part * sc[r0:r0 + rows]).sum(1)
    return y


def gather_m1_grouped(x, pools, inds, w):
    """gather_m1 with every product formed by group_dot (no fp32 weight matrices)."""
    acc = torch.zeros(pools["down_w"].shape[1], dtype=torch.float32)
    for j in range(inds.numel()):
        e = int(inds[j])
        g = _bf16(group_dot(pools["gate_w"][e], pools["gate_s"][e], x))
        u = _bf16(group_dot(pools["up_w"][e], pools["up_s"][e], x))
        h = _bf16(_bf16(g * _bf16(torch.sigmoid(g))) * u)
        ye = _bf16(group_dot(pools["down_w"][e], pools["down_s"][e], h))
        acc = acc + ye * w[j]
    return _bf16(acc)


def decode_step(x, W, bias, pools, k=8, grouped=False):
    """One-row MoE-layer decode (router + 8 experts + combine): y fp32 [H] (bf16 values), inds, w."""
    inds, w = route(x, W, bias, k)
    return (gather_m1_grouped if grouped else gather_m1)(x, pools, inds, w), inds, w
