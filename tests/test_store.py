"""The converted checkpoint's on-disk format (scripts/convert-mimo-v26-mlx.py:6-12, :67-131;
engine/mimo_stream/store.py:15-44): writing, header/offset checks, loading into slot banks.

CPU: files written by write_expert_layer parse with the safetensors library itself, keep the 16 KiB alignment
the format promises, and load back byte for byte (whole layers, slot orders, per-expert jobs); malformed files
are rejected.  GPU: a MoE block loaded from files gives bit-identical outputs to the block built from the
same bank in memory."""
import json
import os
import struct

import numpy as np
import pytest
import torch

from mimo_stream import pools, store

E_T, H_T, I_T = 8, 256, 512


def _random_bank(n, hidden, inter, seed):
    g = torch.Generator().manual_seed(seed)
    bank = pools.alloc_bank(n, hidden, inter, device="cpu")
    for k, v in bank.items():
        v.view(torch.uint8).copy_(torch.randint(0, 256, v.view(torch.uint8).shape, generator=g, dtype=torch.uint8))
    return bank


def test_written_file_matches_the_format(tmp_path):
    from safetensors.numpy import load_file
    bank = _random_bank(E_T, H_T, I_T, seed=1)
    path = store.expert_file(tmp_path, 3)
    store.write_expert_layer(path, 3, bank)
    base, hdr = store.read_header(path)
    assert base % store.ALIGN == 0
    names = [n for n in hdr if n != "__metadata__"]
    assert names == [store.tensor_name(3, p, s) for p in store.PROJ for s in ("weight", "scales")]
    assert hdr["__metadata__"] == {"format": "mlx"}
    arrays = load_file(path)                      # the safetensors library's own parser
    for proj, key in zip(store.PROJ, store.KEYS):
        w = arrays[store.tensor_name(3, proj, "weight")]
        s = arrays[store.tensor_name(3, proj, "scales")]
        assert w.dtype == np.uint32 and s.dtype == np.uint8
        np.testing.assert_array_equal(w.view(np.int32), bank[f"{key}_w"].numpy())
        np.testing.assert_array_equal(s, bank[f"{key}_s"].numpy())
    st = store.ExpertStore(tmp_path, [3])
    assert (st.n, st.hidden, st.inter) == (E_T, H_T, I_T)
    for (L, key, kind), (p, off, stride, shape) in st.loc.items():
        assert off % store.ALIGN == 0 and stride * st.n == int(np.prod(shape)) * (4 if kind == "w" else 1)


def test_load_bank_whole_order_and_jobs(tmp_path):
    bank = _random_bank(E_T, H_T, I_T, seed=2)
    store.write_expert_layer(store.expert_file(tmp_path, 1), 1, bank)
    st = store.ExpertStore(tmp_path, [1])
    got = st.load_bank(1, device="cpu", chunk=40000)          # chunk smaller than a tensor: several reads
    for k in bank:
        assert torch.equal(got[k], bank[k]), k
    order = [5, 2, 7]
    sub = st.load_bank(1, order=order, device="cpu", chunk=12345)
    for k in bank:
        assert torch.equal(sub[k], bank[k][order]), k
    slot = pools.alloc_bank(1, H_T, I_T, device="cpu")
    dst = {(key, kind): memoryview(slot[f"{key}_{kind}"].view(torch.uint8).numpy().reshape(-1))
           for key in store.KEYS for kind in ("w", "s")}
    for path, off, mv in st.jobs(1, 6, dst):
        with open(path, "rb") as f:
            f.seek(off)
            mv[:] = f.read(mv.nbytes)
    for k in bank:
        assert torch.equal(slot[k][0], bank[k][6]), k


def _rewrite_header(path, edit):
    base, hdr = store.read_header(path)
    with open(path, "rb") as f:
        f.seek(base)
        data = f.read()
    edit(hdr)
    hj = json.dumps(hdr, separators=(",", ":")).encode()
    hj += b" " * ((-(8 + len(hj))) % store.ALIGN)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)) + hj + data)


@pytest.mark.parametrize("case", ["dtype", "missing", "shape", "count", "misaligned_start"])
def test_malformed_files_are_rejected(tmp_path, case):
    bank = _random_bank(E_T, H_T, I_T, seed=3)
    path = store.expert_file(tmp_path, 2)
    store.write_expert_layer(path, 2, bank)
    name = store.tensor_name(2, "up_proj", "weight")
    if case == "dtype":
        _rewrite_header(path, lambda h: h[name].update(dtype="I32"))
    elif case == "missing":
        _rewrite_header(path, lambda h: h.pop(store.tensor_name(2, "down_proj", "scales")))
    elif case == "shape":
        _rewrite_header(path, lambda h: h[name].update(shape=[E_T, I_T, H_T // 8 * 2]))
    elif case == "count":
        _rewrite_header(path, lambda h: h[name].update(shape=[E_T // 2, I_T * 2, H_T // 8]))
    else:
        base, hdr = store.read_header(path)
        with open(path, "rb") as f:
            f.seek(base)
            data = f.read()
        hj = json.dumps(hdr, separators=(",", ":")).encode()
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", len(hj)) + hj + data)
    with pytest.raises(ValueError):
        store.ExpertStore(tmp_path, [2])


def test_write_refuses_unaligned_tensors(tmp_path):
    bank = _random_bank(3, H_T, I_T, seed=4)       # 3 x 256 x 16 scale bytes: not a multiple of 16 KiB
    with pytest.raises(ValueError):
        store.write_expert_layer(store.expert_file(tmp_path, 0), 0, bank)


def test_router_from_dense(tmp_path):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(5)
    W = (torch.randn(E_T, H_T, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(E_T, generator=g) * 1e-3
    wn, bn = store.router_names(4)
    save_file({wn: W, bn: b, "model.norm.weight": torch.ones(H_T)}, os.path.join(tmp_path, "dense.safetensors"))
    r = store.load_router(tmp_path, 4, device="cpu", n_experts=E_T, top_k=2)
    assert torch.equal(r.weight, W) and torch.equal(r.e_score_correction_bias, b) and r.top_k == 2
    with pytest.raises(ValueError):
        store.load_router(tmp_path, 4, device="cpu", n_experts=16)


@pytest.mark.gpu
def test_gpu_block_from_files_matches_bank(tmp_path):
    from safetensors.torch import save_file
    from mimo_stream import MoEBlock, Router
    H, I, n = 4096, 2048, 16
    bank = pools.random_bank(n, seed=9, hidden=H, inter=I)
    store.write_expert_layer(store.expert_file(tmp_path, 7), 7, bank)
    g = torch.Generator().manual_seed(6)
    W = (torch.randn(n, H, generator=g) * 0.02).to(torch.bfloat16)
    wn, bn = store.router_names(7)
    save_file({wn: W, bn: torch.zeros(n)}, os.path.join(tmp_path, "dense.safetensors"))
    blk = store.load_block(tmp_path, 7)
    for k in bank:
        assert torch.equal(blk.bank[k], bank[k]), k
    r = Router(H, n, 8)
    r.weight.copy_(W)
    ref = MoEBlock(r, bank)
    x = torch.randn(3, H, generator=g).to(torch.bfloat16).cuda()
    for rows in (x[:1], x):
        y, inds, _ = blk(rows, return_routes=True)
        y2, inds2, _ = ref(rows, return_routes=True)
        assert torch.equal(inds, inds2) and torch.equal(y, y2)
    x2 = torch.randn(40, H, generator=g).to(torch.bfloat16).cuda()          # prefill-sized block
    assert torch.equal(blk(x2), ref(x2))
    # a slot order: experts 9, 3, 12, 0 resident in slots 0..3, routes drawn among them
    order = [9, 3, 12, 0]
    sub = store.load_block(tmp_path, 7, order=order)
    for k in bank:
        assert torch.equal(sub.bank[k], bank[k][order]), k
    inds = torch.tensor([[9, 0, 3, 12], [3, 12, 0, 9]], dtype=torch.int32).cuda()
    w = torch.full((2, 4), 0.25).cuda()
    ys = sub._moe_prefill(x[:2], inds, w)
    yr = ref._moe_prefill(x[:2], inds, w)
    assert torch.equal(ys, yr)
