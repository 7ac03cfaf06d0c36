/* libmimo_moe: MI355X (gfx950) MoE block of MiMo-V2.6-Flash behind a plain C ABI.
 *
 * Reference: cialanjcampbell-coder/mimo-on-a-mac, engine/mimo_stream (MLX + inline Metal).  The reference's
 * plugin boundary is mx.fast.metal_kernel (engine/mimo_stream/kernels.py:128-132); each entry point below
 * names the reference function or kernel it replaces.  All pointers are device pointers unless noted, all
 * calls are asynchronous on `stream` (a hipStream_t, 0 = default stream) and never synchronise the host.
 * bf16 tensors are passed as uint16_t bit patterns.  Return value: MIMO_OK or a negative MIMO_ERR_* code;
 * mimo_last_error() gives the message of the calling thread's last failure.
 *
 * Expert layout (engine/mimo_stream/model.py:28-45, kernels.py:5-12): per projection a slot pool of
 * E2M1 nibbles [S, out, in/8] uint32 (low nibble first) and E8M0 scales [S, out, in/32] uint8;
 * gate/up are [S, I, H/8] + [S, I, H/32], down is [S, H, I/8] + [S, H, I/32].  Kernels address experts by
 * slot; slot_of maps expert id -> slot (engine/mimo_stream/cache.py:16-17).
 *
 * Workspaces: entry points that take (ws, ws_bytes) need a caller-owned device buffer of at least the size
 * the matching *_workspace_size() returns; its contents need no initialisation (every kernel writes what it
 * later reads).  Calls that share one workspace must be ordered on one stream.
 *
 * Device status: the fused entry points (mimo_moe_decode, mimo_moe_prefill, mimo_moe_prefill_block,
 * mimo_moe_layer_decode, mimo_moe_layer_prefill) take an optional status_out, a device int32 [1] that the
 * call's own kernels overwrite with MIMO_OK or the failure they found: MIMO_ERR_SLOT when a selected
 * expert has no resident slot (slot_of entry outside [0, n_slots)) and MIMO_ERR_ROWS_PER_EXPERT when more
 * than 8 rows reach one slot (kernels.py:167-168).  Such a route is computed with slot 0 instead of being
 * read out of bounds, so the outputs of a call whose status is not MIMO_OK are not valid.  The word is
 * written on the stream like every output (read it after the stream's work, no host sync inside the call);
 * NULL keeps it in the workspace.
 *
 * Streams: the prefill entry points (mimo_moe_prefill, mimo_moe_prefill_staged, mimo_moe_prefill_block,
 * mimo_moe_layer_prefill) run part of each grouped GEMM on a side stream forked from and joined back to
 * `stream` with events; every (device, stream) pair has its own side stream, kept for the life of the
 * process (the first 64 pairs; prefills on further streams run that part on `stream` itself, after the
 * rest, with the same results).  A call therefore orders work only on its own `stream`: prefills on different
 * streams never wait for each other, and a prefill captured into a HIP graph captures only its own stream's
 * work.  No entry point builds anything on the device at first use (the sigmoid table is constant data), so
 * the first call of a process may itself be captured.
 */
#ifndef MIMO_MOE_H
#define MIMO_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIMO_ABI_VERSION 2

enum {
  MIMO_OK = 0,
  MIMO_ERR_SHAPE = -1,            /* unsupported or inconsistent sizes */
  MIMO_ERR_ALIGN = -2,            /* a pointer is not 16-byte aligned */
  MIMO_ERR_ROWS_PER_EXPERT = -3,  /* more than R rows routed to one expert (kernels.py:167-168) */
  MIMO_ERR_SLOT = -4,             /* an expert has no resident slot / slot id out of range */
  MIMO_ERR_WORKSPACE = -5,        /* workspace missing or too small */
  MIMO_ERR_HIP = -6,              /* a HIP runtime call or kernel launch failed */
  MIMO_ERR_ARG = -7               /* null pointer or invalid argument */
};

/* One MoE layer's expert slot pool (model.py:32-45 alloc_bank; pool dict keys of kernels.py:176-193). */
typedef struct mimo_bank {
  const uint32_t* gate_w;  /* [S, I, H/8] */
  const uint8_t* gate_s;   /* [S, I, H/32] */
  const uint32_t* up_w;    /* [S, I, H/8] */
  const uint8_t* up_s;     /* [S, I, H/32] */
  const uint32_t* down_w;  /* [S, H, I/8] */
  const uint8_t* down_s;   /* [S, H, I/32] */
  int32_t n_slots;         /* S */
  int32_t hidden;          /* H (4096 for MiMo) */
  int32_t inter;           /* I (2048 for MiMo) */
} mimo_bank;

int mimo_abi_version(void);
const char* mimo_last_error(void);

/* ---------------------------------------------------------------- codec (MXFP4 / activation split) */

/* bf16 [rows, cols] -> MXFP4 q [rows, cols/8] + s [rows, cols/32] (OCP MX rule, group 32).
 * Replaces mx.quantize(mode="mxfp4") used to build pools (engine/tests/test_kernels.py:26). */
int mimo_quantize_mxfp4(const uint16_t* w, int64_t rows, int64_t cols, uint32_t* q, uint8_t* s, void* stream);

/* MXFP4 -> fp32 [rows, cols].  Replaces mx.dequantize(mode="mxfp4") (engine/tests/test_kernels.py:34). */
int mimo_dequantize_mxfp4(const uint32_t* q, const uint8_t* s, int64_t rows, int64_t cols, float* out,
                          void* stream);

/* Seeded N(0, stddev) bf16 values, element i a pure function of (seed, i).  Together with
 * mimo_fill_random_mxfp4 this replaces make_pool's mx.random.normal(...) * 0.02 (test_kernels.py:25). */
int mimo_random_bf16(uint64_t seed, float stddev, int64_t n, uint16_t* out, void* stream);

/* quantize(random_bf16(seed, stddev)) for a [rows, cols] matrix without the bf16 intermediate
 * (bit-identical to the two calls above); used to initialise resident pools in place. */
int mimo_fill_random_mxfp4(uint64_t seed, float stddev, int64_t rows, int64_t cols, uint32_t* q, uint8_t* s,
                           void* stream);

/* Activation split for the block-scaled MFMA paths: bf16 x [rows, cols] -> hi, lo E4M3 codes [rows, cols]
 * with E8M0 block scales hs, ls [rows, cols/32]; x == hi + lo for every element within 2^14 of its block
 * maximum.  Internal step of mimo_moe_experts / mimo_moe_prefill (the reference multiplies bf16
 * activations directly, kernels.py:59-68), exported for parity tests. */
int mimo_quantize_fp8_hilo(const uint16_t* x, int64_t rows, int64_t cols, uint8_t* hi, uint8_t* hs,
                           uint8_t* lo, uint8_t* ls, void* stream);

/* bf16 sigmoid of every bf16 bit pattern, uint16 [65536] (kernels.py:138-146 sigmoid_table). */
int mimo_sigmoid_table(uint16_t* out, void* stream);

/* ---------------------------------------------------------------- router */

/* Selection given fp32 logits [T, E]: sigmoid, + bias, top-k, renormalise, * scaling
 * (model.py:60-64; mimo_v2.py:175-192 with n_group = 1).  inds int32 [T, k] in canonical order
 * (descending key, ties to the lower id), w fp32 [T, k].  Bit-exact entry point. */
int mimo_router_select(const float* logits, const float* bias, int T, int E, int k, float scaling,
                       int32_t* inds, float* w, void* stream);

/* group_expert_select of the vendored noaux-tc gate (mimo_v2.py:165-193), given fp32 logits [T, E]: keys =
 * sigmoid + bias; with n_group > 1 the keys of all but the topk_group groups with the largest sum of their two
 * largest keys are set to 0 (ties to the lower group index); top-k of the keys; weights = the sigmoid scores
 * of the chosen experts, renormalised when norm_topk_prob and k > 1, times routed_scaling_factor. */
int mimo_router_select_grouped(const float* logits, const float* bias, int T, int E, int k, int n_group,
                               int topk_group, int norm_topk_prob, float routed_scaling_factor, int32_t* inds,
                               float* w, void* stream);

/* Router.__call__ (model.py:58-65): logits = x.f32 @ Wg.f32^T then mimo_router_select.
 * x bf16 [T, H], Wg bf16 [E, H], bias fp32 [E]; logits fp32 [T, E] (output). */
int mimo_router(const uint16_t* x, const uint16_t* Wg, const float* bias, int T, int H, int E, int k,
                float* logits, int32_t* inds, float* w, void* stream);

/* ---------------------------------------------------------------- dispatch */

/* group_routes (kernels.py:149-173) on the device.  inds [M, k] expert ids; slot_of [E] (NULL = identity,
 * ids are slots); outputs padded to Umax = min(M*k, n_slots) entries: uids [Umax] ascending slots,
 * urows [Umax, R], ucnt [Umax], uw [Umax, R], gidx [M*k] = u*R + c, n_unique [1] = U.
 * status [1] receives MIMO_OK or MIMO_ERR_ROWS_PER_EXPERT / MIMO_ERR_SLOT (device-side check). */
int mimo_group_routes(const int32_t* inds, const float* scores, const int32_t* slot_of, int M, int k, int R,
                      int n_slots, int32_t* uids, int32_t* urows, int32_t* ucnt, float* uw, uint32_t* gidx,
                      int32_t* n_unique, int32_t* status, void* stream);

/* Prefill dispatch (model.py:235-242, :266-268): stable sort of the flat (token, k) routes by slot.
 * slot_inds [T, k] -> perm [T*k] (sorted position -> flat route), offsets [n_slots + 1], inv [T*k]. */
int mimo_prefill_dispatch(const int32_t* slot_inds, int T, int k, int n_slots, int32_t* perm,
                          int32_t* offsets, int32_t* inv, void* ws, size_t ws_bytes, void* stream);
size_t mimo_prefill_dispatch_workspace_size(int T, int k, int n_slots);

/* ---------------------------------------------------------------- experts */

/* moe_experts (kernels.py:176-199): Kernel A (gate/up + SwiGLU, bf16 rounding points of :79-82),
 * Kernel B (down, * router weight, fp32 partials :120) and the fixed-order combine (:198-199), for M <= 8
 * rows grouped by distinct expert (uslot/urows/ucnt/uw/gidx as from mimo_group_routes; n_unique may be
 * NULL, then all Umax entries are used).  round_expert_bf16 = 1 rounds each expert's down output to bf16
 * before weighting (the gather_qmm path of model.py:173-182).  y bf16 [M, H]; h_out bf16 [Umax, R, I] and
 * part_out fp32 [Umax, R, H] are optional copies of the intermediates (NULL to skip). */
int mimo_moe_experts(const uint16_t* x, int M, const mimo_bank* bank, const int32_t* uslot,
                     const int32_t* urows, const int32_t* ucnt, const float* uw, const int32_t* n_unique,
                     int Umax, int R, const uint32_t* gidx, int k, int round_expert_bf16, uint16_t* y,
                     uint16_t* h_out, float* part_out, void* ws, size_t ws_bytes, void* stream);
size_t mimo_moe_experts_workspace_size(int M, int Umax, int R, int H, int I);

/* One MoE block in decode (model.py:303-325 with _moe_small :184-219, every expert resident):
 * router -> grouping -> experts -> combine for M <= 8 rows, no host synchronisation.  M == 1 uses the
 * gather_qmm rounding (bf16 expert outputs, model.py:173-182), M >= 2 the distinct-expert kernels' fp32
 * partials (kernels.py:120).  inds_out / w_out (optional) receive the routes, status_out (optional) the
 * device status. */
int mimo_moe_decode(const uint16_t* x, int M, const uint16_t* Wg, const float* bias, const int32_t* slot_of,
                    int E, int k, const mimo_bank* bank, uint16_t* y, int32_t* inds_out, float* w_out,
                    int32_t* status_out, void* ws, size_t ws_bytes, void* stream);
size_t mimo_moe_decode_workspace_size(int M, int E, int k, int H, int I);

/* _moe_prefill (model.py:230-271) with every expert resident: slot_inds int32 [T, k] (slots), w fp32
 * [T, k]; sorted-by-slot grouped GEMMs on block-scaled MFMA, bf16 expert outputs, fixed-order weighted
 * combine.  y bf16 [T, H]; status_out (optional): MIMO_ERR_SLOT when a slot id is outside [0, n_slots). */
int mimo_moe_prefill(const uint16_t* x, int T, const int32_t* slot_inds, const float* w, int k,
                     const mimo_bank* bank, uint16_t* y, int32_t* status_out, void* ws, size_t ws_bytes,
                     void* stream);
size_t mimo_moe_prefill_workspace_size(int T, int k, int n_slots, int H, int I);

/* _moe_prefill with non-resident experts in a staging bank (model.py:230-271 with the staging banks of
 * :140-143): slot ids [0, bank->n_slots) address the resident bank, ids bank->n_slots + j slot j of `stage`
 * (same hidden / inter).  The reference runs the resident and the staged routes as two gather_qmm passes and
 * merges their bf16 outputs in (token, k) order before the fixed-order sum (:244-271); here one dispatch over
 * both banks writes the same bf16 route outputs, so y equals mimo_moe_prefill's on a bank holding every
 * expert.  Workspace: mimo_moe_prefill_workspace_size(T, k, bank->n_slots + stage->n_slots, H, I). */
int mimo_moe_prefill_staged(const uint16_t* x, int T, const int32_t* slot_inds, const float* w, int k,
                            const mimo_bank* bank, const mimo_bank* stage, uint16_t* y, int32_t* status_out,
                            void* ws, size_t ws_bytes, void* stream);

/* Router + _moe_prefill for one chunk (model.py:303, :335-336): y bf16 [T, H]; inds_out / w_out / status_out
 * optional. */
int mimo_moe_prefill_block(const uint16_t* x, int T, const uint16_t* Wg, const float* bias,
                           const int32_t* slot_of, int E, int k, const mimo_bank* bank, uint16_t* y,
                           int32_t* inds_out, float* w_out, int32_t* status_out, void* ws, size_t ws_bytes,
                           void* stream);
size_t mimo_moe_prefill_block_workspace_size(int T, int E, int k, int n_slots, int H, int I);

/* ---------------------------------------------------------------- the decoder layer around the block */

/* post_attention_layernorm (model.py:299, nn.RMSNorm(hidden, eps=layernorm_epsilon) :75): r = RMSNorm(x) * w
 * for T rows of H bf16 (H a multiple of 256, at most 8192), fp32 sum of squares in a fixed tree, inv =
 * 1 / sqrt(ss / H + eps), r = bf16(w * bf16(x * inv)).  r may not alias x; x, w, r 16-byte aligned. */
int mimo_rmsnorm(const uint16_t* x, int T, int H, const uint16_t* w, float eps, uint16_t* r, void* stream);

/* The layer residual h = x + y (model.py:340): h = bf16(x + y) elementwise over n bf16 values; h may alias x or
 * y.  Pointers 16-byte aligned. */
int mimo_residual_add(const uint16_t* x, const uint16_t* y, int64_t n, uint16_t* h, void* stream);

/* The MoE half of a decoder layer in decode (model.py:299-340 for T <= 8): r = RMSNorm(x) * norm_w (computed
 * inside the router kernel, bit-identical to mimo_rmsnorm), the decode block on r (as mimo_moe_decode),
 * h = bf16(x + y) in the block's combine.  h may alias x; r_out (optional, not aliasing x or h) receives r;
 * inds_out / w_out (optional) the routes, status_out (optional) the device status. */
int mimo_moe_layer_decode(const uint16_t* x, int M, const uint16_t* norm_w, float eps, const uint16_t* Wg,
                          const float* bias, const int32_t* slot_of, int E, int k, const mimo_bank* bank,
                          uint16_t* h, uint16_t* r_out, int32_t* inds_out, float* w_out, int32_t* status_out,
                          void* ws, size_t ws_bytes, void* stream);
size_t mimo_moe_layer_decode_workspace_size(int M, int E, int k, int H, int I);

/* The same for a prefill chunk (model.py:299-340 for T > 8): RMSNorm, the prefill block on r (as
 * mimo_moe_prefill_block), h = bf16(x + y) in the combine.  h may alias x. */
int mimo_moe_layer_prefill(const uint16_t* x, int T, const uint16_t* norm_w, float eps, const uint16_t* Wg,
                           const float* bias, const int32_t* slot_of, int E, int k, const mimo_bank* bank,
                           uint16_t* h, uint16_t* r_out, int32_t* inds_out, float* w_out, int32_t* status_out,
                           void* ws, size_t ws_bytes, void* stream);
size_t mimo_moe_layer_prefill_workspace_size(int T, int E, int k, int n_slots, int H, int I);

/* No counterpart in the reference: mimo_moe_layer_decode for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The same kernels, with the
 * workspace in a scratch array the library holds on each GPU (MIMO_NOALLOC_SCRATCH_BYTES, kept until the process
 * ends); the call itself allocates nothing (per-kernel event timing is skipped for it).  Batches whose workspace
 * (mimo_moe_layer_decode_workspace_size) exceeds the scratch are refused with MIMO_ERR_WORKSPACE; MiMo's largest,
 * 8 rows of 256 experts, needs about 2.3 MB.  Every call on one GPU uses that GPU's one scratch array: calls that
 * overlap on one GPU (two host threads, or two streams without an ordering between them) race. */
#define MIMO_NOALLOC_SCRATCH_BYTES (4u << 20)
int mimo_moe_layer_decode_noalloc(const uint16_t* x, int M, const uint16_t* norm_w, float eps, const uint16_t* Wg,
                                  const float* bias, const int32_t* slot_of, int E, int k, const mimo_bank* bank,
                                  uint16_t* h, uint16_t* r_out, int32_t* inds_out, float* w_out,
                                  int32_t* status_out, void* stream);

/* ---------------------------------------------------------------- measurement */

/* No counterpart in the reference: per-kernel timing for benchmarks.  While enabled, every kernel launch is
 * followed by a HIP event on its stream; the kernel's time runs from the previous kernel's event of the same
 * entry-point call (or from an event recorded just before it, for the first kernel of a call) to its own, so
 * back-to-back kernels add one event record each.  mimo_profile_enable also clears the records.  mimo_profile_read synchronises on the recorded events and returns the number of distinct
 * kernel names; for the first max_kernels of them it writes the name (64 bytes each, NUL-terminated, host
 * buffer), the total milliseconds and the launch count (host arrays). */
int mimo_profile_enable(int on);
int mimo_profile_read(int max_kernels, char* names, float* total_ms, int* launches);

#ifdef __cplusplus
}
#endif
#endif /* MIMO_MOE_H */
