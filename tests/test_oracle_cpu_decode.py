"""The CPU baseline's decode (oracle.cpu_decode: PyTorch fp32 on the host, every core) computes the reference
algorithm: its dequantisation equals the oracle's exactly, its routes are the oracle's, and its output is within
the GPU path's bf16 tolerance of the oracle (CPU only)."""
import numpy as np
import torch

from helpers import assert_bf16_close, rand_bf16
from oracle import cpu_decode as cd, experts as ox, mxfp4 as oq, routing as orr


def _pool(rng, E, H, I):
    p = {}
    for name, (o, i) in {"gate": (I, H), "up": (I, H), "down": (H, I)}.items():
        q, s = oq.quantize_mxfp4(rand_bf16(rng, (E * o, i), 0.02))
        p[f"{name}_w"] = q.reshape(E, o, i // 8)
        p[f"{name}_s"] = s.reshape(E, o, i // 32)
    return p


def test_dequantize_equals_oracle():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 2 ** 32, (64, 32), dtype=np.uint64).astype(np.uint32)
    s = rng.integers(0, 256, (64, 8)).astype(np.uint8)
    s[0, 0], s[1, 1] = 0, 255
    got = cd.dequantize(torch.from_numpy(q.view(np.int32)), torch.from_numpy(s)).numpy()
    ref = oq.dequantize_mxfp4(q, s)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok], ref[ok])


def test_decode_step_matches_oracle():
    rng = np.random.default_rng(2)
    E, H, I, k = 16, 512, 256, 8
    p = _pool(rng, E, H, I)
    W = rand_bf16(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * 1e-3).astype(np.float32)
    tp = {n: torch.from_numpy(v.view(np.int32) if n.endswith("_w") else v) for n, v in p.items()}
    pool = ox.ExpertPool(p)
    for t in range(4):
        x = rand_bf16(rng, (1, H))
        y, inds, w = cd.decode_step(torch.from_numpy(x[0]), torch.from_numpy(W), torch.from_numpy(bias), tp, k)
        oi, ow = orr.select_topk(orr.router_logits(x, W), bias, k)
        assert sorted(inds.tolist()) == sorted(oi[0].tolist())
        order = np.argsort(inds.numpy(), kind="stable")
        ref_order = np.argsort(oi[0], kind="stable")
        np.testing.assert_allclose(w.numpy()[order], ow[0][ref_order], rtol=1e-5)
        oy = ox.gather_m1(x[0], pool, oi[0], ow[0])
        assert_bf16_close(y.numpy(), oy, what=f"cpu decode step {t}")


def test_group_dot_equals_dequantised_product():
    """group_dot (group sums times the group scale) against the oracle's dequantised matrix times x in float64,
    including scale bytes 0 (2^-127) and 255 (NaN rows), and row counts that are not a multiple of the block."""
    rng = np.random.default_rng(3)
    out_dim, in_dim = 300, 256
    q = rng.integers(0, 2 ** 32, (out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
    s = rng.integers(110, 135, (out_dim, in_dim // 32)).astype(np.uint8)
    s[5, 2], s[7, 0] = 0, 255
    x = rand_bf16(rng, (in_dim,))
    got = cd.group_dot(torch.from_numpy(q.view(np.int32)), torch.from_numpy(s), torch.from_numpy(x), rows=64).numpy()
    with np.errstate(over="ignore", invalid="ignore"):   # the NaN row's scale
        dq = oq.dequantize_mxfp4(q, s).astype(np.float64)
    ref = dq @ x.astype(np.float64)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    assert np.isnan(got[7]) and not np.isnan(got[5])
    ok = ~np.isnan(ref)
    scale = np.abs(dq[ok]) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got[ok] - ref[ok]) <= 1e-6 * scale + 1e-30)


def test_grouped_decode_step_matches_oracle():
    rng = np.random.default_rng(4)
    E, H, I, k = 16, 512, 256, 8
    p = _pool(rng, E, H, I)
    W = rand_bf16(rng, (E, H), 0.02)
    bias = (rng.standard_normal(E) * 1e-3).astype(np.float32)
    tp = {n: torch.from_numpy(v.view(np.int32) if n.endswith("_w") else v) for n, v in p.items()}
    pool = ox.ExpertPool(p)
    for t in range(3):
        x = rand_bf16(rng, (1, H))
        y, inds, w = cd.decode_step(torch.from_numpy(x[0]), torch.from_numpy(W), torch.from_numpy(bias), tp, k,
                                    grouped=True)
        oi, ow = orr.select_topk(orr.router_logits(x, W), bias, k)
        assert sorted(inds.tolist()) == sorted(oi[0].tolist())
        oy = ox.gather_m1(x[0], pool, oi[0], ow[0])
        assert_bf16_close(y.numpy(), oy, what=f"grouped cpu decode step {t}")
