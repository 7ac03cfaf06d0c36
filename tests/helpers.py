"""Shared helpers for the GPU parity tests: device tensors <-> oracle numpy arrays."""
import os
import subprocess
import sys

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


def pool_np(bank, cache=True):
    """Device bank dict -> oracle ExpertPool (uint32 / uint8 numpy)."""
    p = {}
    for k, v in bank.items():
        a = v.cpu().numpy()
        p[k] = a.view(np.uint32) if k.endswith("_w") else a
    return ox.ExpertPool(p, cache=cache)


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
    fp32 accumulation order moves an intermediate (g, up, h) or the output across a bf16 rounding boundary:
    one ulp (2^-8 relative) of that value, and an h flip moves the downstream sums by a fraction of an ulp.
    Checks max|got - ref| / max|ref| < max_rel and that at least `within_ulp` of the elements agree to two
    bf16 ulps of their magnitude, with an absolute floor of 2^-10 of max|ref| for outputs that are sums of
    cancelling terms.  Returns (rel_err, fraction within that bound)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max() + 1e-30
    rel = float(np.abs(got - ref).max() / scale)
    ulp = np.maximum(np.abs(ref), np.abs(got)) * 2.0 ** -6 + scale * 2.0 ** -10
    frac = float(np.mean(np.abs(got - ref) <= ulp))
    dump = os.environ.get("MIMO_TEST_DUMP")
    if dump and not (rel < max_rel and frac >= within_ulp):
        np.savez(os.path.join(dump, f"fail_{what.replace(' ', '_')}.npz"), got=got, ref=ref)
    assert rel < max_rel and frac >= within_ulp, f"{what}: rel_err {rel:.3e}, within two ulps {frac:.4f}"
    return rel, frac


def shared_routes(rng, M, S, k):
    """M rows of k distinct experts out of S; row 1 shares its first k//2 experts with row 0 (the shared-
    expert case of engine/tests/test_kernels.py:73) without repeating an expert inside a row."""
    rows = [rng.choice(S, k, replace=False)]
    for r in range(1, M):
        if r == 1:
            keep = rows[0][: k // 2]
            rest = rng.choice(np.setdiff1d(np.arange(S), keep), k - k // 2, replace=False)
            rows.append(np.concatenate([keep, rest]))
        else:
            rows.append(rng.choice(S, k, replace=False))
    return np.stack(rows).astype(np.int32)


ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Preamble of child-process GPU checks: inputs made by torch alone (no library call), a bank of random E2M1
# codes (every code) with E8M0 scales 118..122.
CHILD_COMMON = r"""
import sys, numpy as np, torch
from mimo_stream import _lib, pools
torch.manual_seed(5)
dev = torch.device("cuda")

def torch_bank(E, H, I):
    # random E2M1 codes (every code) and E8M0 scales 118..122, made by torch only
    bank = {}
    for k, (o, i) in pools.shapes(H, I).items():
        bank[f"{k}_w"] = torch.randint(-2**31, 2**31 - 1, (E, o, i // 8), dtype=torch.int32, device=dev)
        bank[f"{k}_s"] = torch.randint(118, 123, (E, o, i // 32), dtype=torch.uint8, device=dev)
    return bank

def bf16(*shape, scale=1.0):
    return (torch.randn(*shape, device=dev) * scale).to(torch.bfloat16)

def say(msg):
    print(msg, flush=True)
"""


def run_child(code, marker, timeout=300):
    """Run a Python GPU check in a fresh process (library and package importable); it must exit 0 and print
    marker."""
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([ROOT, os.path.join(ROOT, "mimo-on-a-mac_amd"), env.get("PYTHONPATH", "")])
    p = subprocess.run([sys.executable, "-u", "-c", code], env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=timeout)
    assert p.returncode == 0 and marker in p.stdout, f"child exited {p.returncode}:\n{p.stdout[-3000:]}"


