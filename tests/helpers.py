"""Shared helpers for the GPU parity tests: device tensors <-> oracle numpy arrays."""
import numpy as np
import torch

from oracle import experts as ox, mxfp4 as oq


def bf16_np(t):
    """bf16 torch tensor -> float32 numpy (exact)."""
    return t.detach().to(torch.float32).cpu().numpy()


def bf16_bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_dev_bf16(a, device="cuda"):
    """float32 numpy holding bf16 values -> bf16 device tensor (exact)."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(device)


def pool_np(bank):
    """Device bank dict -> oracle ExpertPool (uint32 / uint8 numpy)."""
    p = {}
    for k, v in bank.items():
        a = v.cpu().numpy()
        p[k] = a.view(np.uint32) if k.endswith("_w") else a
    return ox.ExpertPool(p)


def rand_bf16(rng, shape, scale=1.0):
    return oq.round_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def zipf_routes(rng, T, E, k, s=1.1):
    """Per-token top-k without replacement from a Zipf(s) popularity over a seeded permutation of E experts."""
    perm = rng.permutation(E)
    p = 1.0 / np.arange(1, E + 1) ** s
    logp = np.log(p / p.sum())
    g = rng.gumbel(size=(T, E)) + logp[None, :]
    top = np.argsort(-g, axis=1)[:, :k]
    return perm[top].astype(np.int32)


def assert_bf16_close(got, ref, max_rel=1e-2, within_ulp=0.99, what=""):
    """GPU bf16 output vs the oracle.  Both apply the same bf16 rounding points; they differ only where the
    fp32 accumulation order moves a value across a bf16 rounding boundary, i.e. by one bf16 ulp (2^-8
    relative) of that element.  Checks max|got - ref| / max|ref| < max_rel and that at least `within_ulp` of
    the elements agree to one bf16 ulp of their magnitude.  Returns (rel_err, fraction within one ulp)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rel = float(np.abs(got - ref).max() / (np.abs(ref).max() + 1e-30))
    ulp = np.maximum(np.abs(ref), np.abs(got)) * 2.0 ** -7 + 1e-30
    frac = float(np.mean(np.abs(got - ref) <= ulp))
    assert rel < max_rel and frac >= within_ulp, f"{what}: rel_err {rel:.3e}, within one ulp {frac:.4f}"
    return rel, frac
