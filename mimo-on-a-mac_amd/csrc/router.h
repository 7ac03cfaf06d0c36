// Launchers shared between the router, decode and prefill translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimo {

struct RouterSmallArgs {
  const uint16_t* x;       // [T, H] bf16
  const uint16_t* Wg;      // [E, H] bf16
  const float* bias;       // [E]
  int T, H, E, k, nlog;    // nlog = E logits blocks (set by the launcher)
  float* logits;           // [T, E]
  float* scores;           // [T, E] sigmoid (optional)
  float* keys;             // [T, E] sigmoid + bias (optional)
  uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;   // optional fp8 split of x: [T, H], [T, H/32]
  // optional RMSNorm of the rows first (the post-attention norm of a decoder layer): logits and split are then of
  // r = RMSNorm(x) * norm_w, and r itself goes to r_out when given (H a multiple of 256)
  const uint16_t* norm_w;  // [H] bf16
  float eps;
  uint16_t* r_out;         // [T, H] bf16 (optional)
};

int launch_router_logits_small(const RouterSmallArgs& a, hipStream_t st);   // logits, sigmoid, keys, x split

struct SelectGroupArgs {
  const float *scores, *keys;   // [T, E]
  int T, E, k;
  const int32_t* slot_of;
  int R, n_slots, Umax;
  int32_t* inds_out;
  float* w_out;
  int32_t *uids, *urows, *ucnt;
  float* uw;
  uint32_t* gidx;
  int32_t *n_unique, *status;
};
// top-k + renormalisation per row and grouping by slot (one block; T <= 8, T*k <= 64, Umax*R <= 512)
int launch_select_group(const float* scores, const float* keys, int T, int E, int k, const int32_t* slot_of, int R,
                        int n_slots, int Umax, int32_t* inds_out, float* w_out, int32_t* uids, int32_t* urows,
                        int32_t* ucnt, float* uw, uint32_t* gidx, int32_t* n_unique, int32_t* status,
                        hipStream_t st);
// zero_status (optional): a status word the launch clears (its first block), for the kernels queued after it
int launch_router_logits(const uint16_t* x, const uint16_t* W, int T, int H, int E, float* logits, hipStream_t st,
                         int32_t* zero_status = nullptr);
int launch_router_select(const float* logits, const float* bias, int T, int E, int k, float scaling, int32_t* inds,
                         float* w, const int32_t* slot_of, int32_t* slot_inds, int n_slots, int32_t* status,
                         hipStream_t st);
// Row tiles of the grouped GEMM: a slot with 1..narrow_max routes is one narrow tile; a larger one is split into
// ceil(count / wide_rows) wide tiles of near-equal whole unit-route chunks (wide_rows a multiple of unit).
// tiles[0] = (wide count, narrow count), wide tile t at tiles[1 + t], narrow tile t at tiles[1 + wcap + t], each
// (slot, first route, end route, 0).
struct TileSpec {
  int narrow_max, wide_rows, wcap, unit;
};
int launch_dispatch(const int32_t* slots, int n, int n_slots, int32_t* hist, int32_t* perm, int32_t* offsets,
                    int32_t* inv, const TileSpec* spec, int4* tiles, int32_t* status, hipStream_t st);
size_t dispatch_workspace(int n, int n_slots);
int launch_quantize_fp8_hilo(const uint16_t* x, int64_t rows, int64_t cols, uint8_t* hi, uint8_t* hs, uint8_t* lo,
                             uint8_t* ls, hipStream_t st, int32_t* zero_status = nullptr);

}  // namespace mimo
