"""The MoE half of a decoder layer, around the MoE block (engine/mimo_stream/model.py:296-340):

    r = post_attention_layernorm(x)        (:299; nn.RMSNorm(hidden, eps=layernorm_epsilon), :75)
    inds, w = gate(r);  y = experts(r)     (:300-336)
    h = x + y                              (:340)

with the next-layer route prediction of :305-314 (the next MoE layer's router applied to its own norm of this
layer's residual x) and, for layers that keep fewer slots than experts, the prefetch of the predicted misses
(:320-329).

A resident block (MoEBlock) runs the whole layer as one library call, mimo_moe_layer_decode (T <= 8) or
mimo_moe_layer_prefill: the norm kernel, the block on r, and the residual added in the block's combine kernel.  A
streamed block (StreamedMoEBlock) needs the routes on the host between router and experts, and a router with the
vendored gate's options routes through its own selection, so those run mimo_rmsnorm, the block, then
mimo_residual_add.
"""
import json
import os

import numpy as np
import torch

from . import _lib, pools
from .model import MoEBlock
from .residency import StreamedMoEBlock


class MoELayer:
    def __init__(self, block, norm_weight, eps):
        self.block = block
        inner = block.block if isinstance(block, StreamedMoEBlock) else block
        if not isinstance(inner, MoEBlock):
            raise TypeError("block must be a MoEBlock or a StreamedMoEBlock")
        H = inner._bank_struct.hidden
        w = torch.as_tensor(norm_weight)
        if w.shape != (H,):
            raise ValueError(f"norm weight of shape {tuple(w.shape)} for hidden size {H}")
        dev = inner.router.weight.device
        self.norm_weight = w.to(device=dev, dtype=torch.bfloat16).contiguous()
        self.eps = float(eps)
        if not self.eps >= 0.0:
            raise ValueError("eps must be a non-negative number")
        self.hidden = H

    @property
    def _inner(self):
        return self.block.block if isinstance(self.block, StreamedMoEBlock) else self.block

    def norm(self, x):
        """post_attention_layernorm(x): bf16 [T, H] (model.py:299)."""
        x2 = self._rows(x)
        r = torch.empty_like(x2)
        if x2.shape[0] == 0:
            return r
        _lib.call("mimo_rmsnorm", _lib.ptr(x2), x2.shape[0], self.hidden, _lib.ptr(self.norm_weight), self.eps,
                  _lib.ptr(r), _lib.stream_ptr(x2.device))
        return r

    def _rows(self, x):
        _lib.require_cuda(x)
        if x.shape[-1] != self.hidden:
            raise ValueError(f"rows of {x.shape[-1]} for hidden size {self.hidden}")
        return x.reshape(-1, self.hidden).to(torch.bfloat16).contiguous()

    def __call__(self, x, return_routes=False, return_norm=False):
        """h = x + MoE(post_attention_layernorm(x)) for x bf16 [..., H] (model.py:299-340); T <= 8 rows take the
        decode path, more the prefill path.  Returns h (x's shape), plus (inds, w) and / or r when asked."""
        x2 = self._rows(x)
        T = x2.shape[0]
        dev = x2.device
        if T == 0:                          # an empty batch: h = x, nothing routed, no launch
            k = self._inner.router.top_k
            out = (x2.clone().reshape(x.shape),)
            if return_routes:
                out += (torch.empty((0, k), dtype=torch.int32, device=dev),
                        torch.empty((0, k), dtype=torch.float32, device=dev))
            if return_norm:
                out += (torch.empty_like(x2),)
            return out if len(out) > 1 else out[0]
        if isinstance(self.block, StreamedMoEBlock) or self._inner.router.gate_options is not None:
            r = self.norm(x2)
            y, inds, w = self.block(r, return_routes=True)
            h = torch.empty_like(x2)
            _lib.call("mimo_residual_add", _lib.ptr(x2), _lib.ptr(y), x2.numel(), _lib.ptr(h), _lib.stream_ptr(dev))
        else:
            blk = self.block
            b = blk._bank_struct
            rt = blk.router
            En, k = rt.weight.shape[0], rt.top_k
            h = torch.empty_like(x2)
            r = torch.empty_like(x2) if return_norm else None
            inds = torch.empty((T, k), dtype=torch.int32, device=dev)
            w = torch.empty((T, k), dtype=torch.float32, device=dev)
            head = (_lib.ptr(x2), T, _lib.ptr(self.norm_weight), self.eps, _lib.ptr(rt.weight),
                    _lib.ptr(rt.e_score_correction_bias), _lib.ptr(blk.slot_of), En, k, b)
            tail = (_lib.ptr(h), _lib.ptr(r), _lib.ptr(inds), _lib.ptr(w), _lib.ptr(blk.status))
            if T <= pools.VERIFY_MAX:
                nbytes = _lib.load().mimo_moe_layer_decode_workspace_size(T, En, k, b.hidden, b.inter)
                ws = _lib.workspace(nbytes, dev, "layer_decode")
                _lib.call("mimo_moe_layer_decode", *head, *tail, _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
            else:
                nbytes = _lib.load().mimo_moe_layer_prefill_workspace_size(T, En, k, b.n_slots, b.hidden, b.inter)
                ws = _lib.workspace(nbytes, dev, "layer_prefill")
                _lib.call("mimo_moe_layer_prefill", *head, *tail, _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
            if blk.partial:
                blk.check_status("MoELayer")
        h = h.reshape(x.shape)
        out = (h,)
        if return_routes:
            out += (inds, w)
        if return_norm:
            out += (r,)
        return out if len(out) > 1 else h

    def predict(self, x, top=None):
        """Expert ids this layer's router picks for the residual x of the layer before it (model.py:305-314):
        its router on its own norm of x.  top < k keeps the `top` highest-weight experts of the last row (as the
        reference's prefetch_k); otherwise every row's experts.  Returns a sorted numpy array of distinct ids."""
        r = self.norm(x)
        inds, w = self._inner.router(r)
        k = inds.shape[1]
        if top is not None and top < k:
            wl = w[-1]
            order = torch.argsort(-wl, stable=True)[:top]
            ids = inds[-1][order]
        else:
            ids = inds.reshape(-1)
        return np.unique(ids.cpu().numpy().astype(np.int64))

    def prefetch(self, experts):
        """Make predicted experts resident ahead of this layer's step (model.py:320-329): for a streamed block,
        the predicted misses are read and copied into slots without counting as uses; a resident block holds
        every expert already.  Returns the number of experts read."""
        if isinstance(self.block, StreamedMoEBlock):
            return self.block.prefetch(experts)
        return 0

    def prefetch_stage(self):
        """Before a long prefill chunk reaches this layer (model.py:273-285, :336-339): a streamed block streams
        all its non-resident experts into the next shared staging bank.  Returns the number of experts read."""
        if isinstance(self.block, StreamedMoEBlock):
            return self.block.prefetch_stage()
        return 0


def norm_name(L):
    return f"model.layers.{L}.post_attention_layernorm.weight"


def layernorm_epsilon(model_dir):
    """layernorm_epsilon of the checkpoint's config.json (model.py:86, :75)."""
    with open(os.path.join(model_dir, "config.json")) as f:
        cfg = json.load(f)
    if "layernorm_epsilon" not in cfg:
        raise ValueError("config.json: no layernorm_epsilon")
    return float(cfg["layernorm_epsilon"])


def load_norm(model_dir, L, device="cuda"):
    """Layer L's post_attention_layernorm weight from dense.safetensors (safetensors loader, no pickle)."""
    from safetensors import safe_open
    name = norm_name(L)
    with safe_open(os.path.join(model_dir, "dense.safetensors"), framework="pt") as f:
        if name not in set(f.keys()):
            raise ValueError(f"dense.safetensors: missing {name}")
        w = f.get_tensor(name)
    if w.dim() != 1:
        raise ValueError(f"{name}: shape {tuple(w.shape)}")
    return w.to(device=device, dtype=torch.bfloat16)


def load_layer(model_dir, L, block=None, device="cuda", eps=None):
    """MoELayer of layer L: its norm weight and epsilon from the checkpoint, around `block` (default: the fully
    resident MoEBlock of store.load_block)."""
    from .store import load_block
    if block is None:
        block = load_block(model_dir, L, device=device)
    eps = layernorm_epsilon(model_dir) if eps is None else eps
    return MoELayer(block, load_norm(model_dir, L, device=device), eps)
