// Route selection and distinct-expert grouping, shared by the router kernels and the fused decode kernel.
//
// Reference: Router.__call__ engine/mimo_stream/model.py:58-65 (selection and renormalisation) and
// group_routes engine/mimo_stream/kernels.py:149-173.  Canonical order: descending key (sigmoid + bias),
// ties to the lower expert id, NaN keys last; renormalisation sums in that order.
#pragma once
#include "device.h"
#include "../../include/mimo_moe.h"

namespace mimo {

// ------------------------------------------------------------------ selection (one wave per row)
// Lane l owns candidates e = l + 64 j (j < PER).  It sorts them once (descending key; ids increase with j, so
// the sort keeps the lower id first on equal keys); then each of the k rounds takes the maximum head key over
// the wave (DPP), the minimum id among lanes whose head carries it, and the winning lane shifts its list.
// Keys are fp32 mapped to an order-preserving uint32 plus one (0 = exhausted; NaN sorts lowest).
template <int PER>
__device__ inline void wave_select_row_t(const float* s_row, const float* key_row, int E, int k, float scaling,
                                         int32_t* inds_out, float* w_out, int* lds_sel) {
  const int lane = threadIdx.x & 63;
  float* lds_s = reinterpret_cast<float*>(lds_sel + 16);   // lds_sel has room for 32 entries
  uint32_t cv[PER], id[PER];
  float sc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + 64 * j;
    const bool ok = e < E;
    const float kv = key_row[ok ? e : 0];
    sc[j] = s_row[ok ? e : 0];
    cv[j] = ok ? key_to_ordered(kv) + 1u : 0u;
    id[j] = (uint32_t)e;
  }
  // odd-even transposition sort, descending by value, stable on equal values
#pragma unroll
  for (int pass = 0; pass < PER; ++pass) {
#pragma unroll
    for (int j = pass & 1; j + 1 < PER; j += 2) {
      if (cv[j + 1] > cv[j]) {
        uint32_t t = cv[j]; cv[j] = cv[j + 1]; cv[j + 1] = t;
        t = id[j]; id[j] = id[j + 1]; id[j + 1] = t;
        float f = sc[j]; sc[j] = sc[j + 1]; sc[j + 1] = f;
      }
    }
  }
  for (int r = 0; r < k; ++r) {
    const uint32_t kmax = dpp_max_u32(cv[0]);
    const uint32_t myid = (cv[0] == kmax) ? id[0] : 0xFFFFFFFFu;
    const uint32_t idmin = dpp_min_u32(myid);   // ties between lanes go to the lower expert id
    if (myid == idmin) {
      lds_sel[r] = (int)idmin;
      lds_s[r] = sc[0];
#pragma unroll
      for (int j = 0; j + 1 < PER; ++j) { cv[j] = cv[j + 1]; id[j] = id[j + 1]; sc[j] = sc[j + 1]; }
      cv[PER - 1] = 0u;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // renormalisation: sequential fp32 sum in selection order (lane 0), divisions on k lanes
  float denom = 0.0f;
  if (lane == 0) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    for (int r = 0; r < k; ++r) acc = acc + lds_s[r];
    denom = acc + 1e-20f;
  }
  denom = __shfl(denom, 0, 64);
  if (lane < k) {
#pragma clang fp contract(off)
    float wv = lds_s[lane] / denom;
    if (scaling != 1.0f) wv = wv * scaling;
    inds_out[lane] = lds_sel[lane];
    w_out[lane] = wv;
  }
  __builtin_amdgcn_wave_barrier();
}

__device__ inline void wave_select_row(const float* s_row, const float* key_row, int E, int k, float scaling,
                                       int32_t* inds_out, float* w_out, int* lds_sel) {
  if (E <= 64) wave_select_row_t<1>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel);
  else if (E <= 128) wave_select_row_t<2>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel);
  else if (E <= 256) wave_select_row_t<4>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel);
  else if (E <= 512) wave_select_row_t<8>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel);
  else wave_select_row_t<16>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel);
}

// ------------------------------------------------------------------ grouping (one wave, <= 64 routes)
// The same outputs as block_group_routes from shuffles only: route t on lane t; lower = earlier routes of its
// slot (= its row slot c), rank = distinct smaller slots (= u).  lurows/luw: LDS scratch of Umax*R entries.
__device__ inline void wave_group_routes(const int32_t* inds, const float* scores, const int32_t* slot_of, int M, int k,
                                  int R, int n_slots, int Umax, int32_t* uids, int32_t* urows, int32_t* ucnt,
                                  float* uw, uint32_t* gidx, int32_t* n_unique, int32_t* status, int* lurows,
                                  float* luw, uint32_t* bits) {
  const int lane = threadIdx.x & 63;
  const int nr = M * k;
  int bad = 0;
  int s = -1;
  float sc = 0.0f;
  if (lane < nr) {
    int e = inds[lane];
    s = slot_of ? ((e >= 0) ? slot_of[e] : -1) : e;
    if (s < 0 || s >= n_slots) { bad = MIMO_ERR_SLOT; s = 0; }
    sc = scores[lane];
  }
  // lanes holding the same slot: AND of per-bit ballots (slot ids < 1024)
  const uint64_t live = __ballot(lane < nr);
  uint64_t match = live;
#pragma unroll
  for (int b = 0; b < 10; ++b) {
    const uint64_t m = __ballot((s >> b) & 1);
    match &= ((s >> b) & 1) ? m : ~m;
  }
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int lower = __popcll(match & below);       // earlier routes of this slot = the route's row slot c
  const int same = __popcll(match);
  const int first = (lane < nr && lower == 0) ? 1 : 0;
  const int U = __popcll(__ballot(first));
  // rank of the slot among the distinct slots (= u): bitmap of present slots in LDS
  if (lane < 32) bits[lane] = 0u;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (first) atomicOr(&bits[s >> 5], 1u << (s & 31));
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  int rank = 0;
  const int sw = s >> 5;
#pragma unroll
  for (int w = 0; w < 32; ++w) {
    const uint32_t bw = bits[w];
    rank += w < sw ? __popc(bw) : (w == sw ? __popc(bw & ((1u << (s & 31)) - 1u)) : 0);
  }
  for (int e = lane; e < Umax * R; e += 64) { lurows[e] = 0; luw[e] = 0.0f; }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (lane < nr) {
    if (lower >= R) {
      bad = bad ? bad : MIMO_ERR_ROWS_PER_EXPERT;
    } else if (rank < Umax) {
      lurows[rank * R + lower] = lane / k;
      luw[rank * R + lower] = sc;
      gidx[lane] = (uint32_t)(rank * R + lower);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  for (int e = lane; e < Umax * R; e += 64) { urows[e] = lurows[e]; uw[e] = luw[e]; }
  for (int u = lane; u < Umax; u += 64) {
    ucnt[u] = 0;
    uids[u] = 0;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  if (first && rank < Umax) {
    ucnt[rank] = same > R ? R : same;
    uids[rank] = s;
  }
  // most severe code (most negative) over the wave
  const int worst = -(int)dpp_max_u32((uint32_t)(-bad));
  if (lane == 0) {
    n_unique[0] = U;
    status[0] = worst;
  }
}

}  // namespace mimo
