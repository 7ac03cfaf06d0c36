"""mimo_stream: the MiMo-V2.6-Flash MoE block (router -> top-8 -> MXFP4 SwiGLU experts -> weighted combine)
on MI355X, behind the API of the reference's engine/mimo_stream package.

Compute runs in libmimo_moe.so (hand-written gfx950 HIP kernels, C ABI in include/mimo_moe.h); this package
holds the Python mirror of the reference interface over torch device tensors.
"""
from .pools import E, TOPK, VERIFY_MAX, SHAPES, EXPERT_BYTES, alloc_bank, random_bank, expert_bytes  # noqa: F401
from .cache import SlotCache  # noqa: F401
from .kernels import sigmoid_table, group_routes, moe_experts  # noqa: F401
from .model import Router, MoEBlock, select_from_logits, prefill_dispatch  # noqa: F401
from .store import ExpertStore, load_block, load_router, write_expert_layer  # noqa: F401
from .residency import StagingBanks, StreamedMoEBlock  # noqa: F401
from .layer import MoELayer, load_layer, load_norm, layernorm_epsilon  # noqa: F401
