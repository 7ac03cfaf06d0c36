"""CPU oracle for the MiMo-V2.6-Flash MoE block (router -> top-8 -> MXFP4 SwiGLU experts -> combine).

TEST INFRASTRUCTURE ONLY.  This package restates, in numpy, the algorithm of the reference engine's MoE
block (engine/mimo_stream/kernels.py, engine/mimo_stream/model.py:26-65, :173-271, engine/mimo_stream/cache.py,
engine/mimo_stream/mimo_v2.py:165-239).  It is the oracle the HIP implementation is compared against, and the
timed CPU baseline in bench.py.  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may
import it; the product path (mimo_stream + libmimo_moe.so) never does.

Modules:
  mxfp4    - E2M1 / E8M0 codec, OCP MX quantiser, the [S, out, in/8] u32 + [S, out, in/32] u8 packing.
  routing  - the exactly specified sigmoid, Router selection (top-k, renormalisation), group_routes,
             the prefill stable dispatch permutation.
  experts  - Kernel A / Kernel B semantics (bf16 rounding points), the M=1 gather_qmm path, the prefill
             pair path and the fixed-order combine.
  layer    - the decoder layer around the block: post-attention RMSNorm and the residual h = x + y.

Parity status per function is stated in each function's docstring ("pinned by ...").
"""
