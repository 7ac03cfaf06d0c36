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
// Lane l owns candidates e = l + 64 j (j < PER), keyed by the fp32 key mapped to an order-preserving uint32
// plus one (0 = no candidate; NaN keys map to 1 and sort lowest).  A bisection on that key finds the k-th
// largest value T (count(key >= T) >= k > count(key > T)), each step one ballot per candidate slot and
// scalar popcounts, stopping early once exactly k keys reach the midpoint.  The selection is every key above
// T plus the lowest-id keys equal to T; its k entries are then ranked by (key descending, id ascending) in
// LDS.  Renormalisation sums the scores sequentially in that order.
constexpr int kSelLds = 80;   // ints of LDS scratch per selecting wave (k <= 16)

// The selected set of one row: take[j] says whether candidate lane + 64 j is among the top k (key order,
// ties to the lower id).  cv: the order-preserving keys.
template <int PER>
__device__ __forceinline__ void wave_select_set(const uint32_t (&cv)[PER], int k, bool (&take)[PER]) {
  const int lane = threadIdx.x & 63;
  // count(cv >= lo) >= k (every candidate has cv >= 1 and E >= k); count(cv >= hi) < k (cv < 2^32 - 1)
  uint32_t lo = 1u, hi = 0xFFFFFFFFu;
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    int c = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) c += __popcll(__ballot(cv[j] >= mid));
    if (c >= k) lo = mid; else hi = mid;
    if (c == k) break;
  }
  const uint32_t T = lo;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int ngt = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) ngt += __popcll(__ballot(cv[j] > T));
  const int need = k - ngt;                  // keys equal to T that are taken, lowest ids first
  int ties_before = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint64_t tie = __ballot(cv[j] == T);
    take[j] = cv[j] > T || (cv[j] == T && ties_before + (int)__popcll(tie & below) < need);
    ties_before += (int)__popcll(tie);
  }
}

// position of the n-th (0-based) set bit of m, n < popcount(m): a binary search on the halves' popcounts
__device__ __forceinline__ int nth_set_bit(uint64_t m, int n) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const uint64_t low = m & ((1ull << w) - 1ull);
    const int c = __popcll(low);
    if (n >= c) {
      n -= c;
      m >>= w;
      pos += w;
    } else {
      m = low;
    }
  }
  return pos;
}

template <int PER>
__device__ __forceinline__ void wave_load_keys(const float* key_row, int E, uint32_t (&cv)[PER]) {
  const int lane = threadIdx.x & 63;
  float kv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) kv[j] = key_row[(lane + 64 * j) < E ? lane + 64 * j : 0];
#pragma unroll
  for (int j = 0; j < PER; ++j) cv[j] = (lane + 64 * j) < E ? key_to_ordered(kv[j]) + 1u : 0u;
}

// The selected candidates of one row staged in LDS in (j, lane) order, which is ascending id: t_key, t_id, t_sc
// of lds_sel (positions 0 .. k - 1).
template <int PER>
__device__ __forceinline__ void wave_stage_selected(const uint32_t (&cv)[PER], const float (&sc)[PER],
                                                    const bool (&take)[PER], int* lds_sel) {
  const int lane = threadIdx.x & 63;
  uint32_t* t_key = reinterpret_cast<uint32_t*>(lds_sel);        // [16] selected, in (j, lane) order
  int* t_id = lds_sel + 16;
  float* t_sc = reinterpret_cast<float*>(lds_sel + 32);
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int sel_before = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint64_t sel = __ballot(take[j]);
    if (take[j]) {
      const int pos = sel_before + __popcll(sel & below);
      t_key[pos] = cv[j];
      t_id[pos] = lane + 64 * j;
      t_sc[pos] = sc[j];
    }
    sel_before += __popcll(sel);
  }
}

// Rank the k staged candidates by (key descending, id ascending) and write ids and weights in that order.
// renorm: divide the selected scores by their sum (model.py:64; mimo_v2.py:190-191 only when norm_topk_prob and
// k > 1); the weights are then multiplied by scaling (mimo_v2.py:192) unless it is 1.  LDS and registers only.
__device__ __forceinline__ void wave_rank_renorm(int k, float scaling, int32_t* inds_out, float* w_out, int* lds_sel,
                                                 bool renorm) {
  const int lane = threadIdx.x & 63;
  const uint32_t* t_key = reinterpret_cast<const uint32_t*>(lds_sel);
  const int* t_id = lds_sel + 16;
  const float* t_sc = reinterpret_cast<const float*>(lds_sel + 32);
  int* f_id = lds_sel + 48;                                        // [16] in canonical order
  float* f_sc = reinterpret_cast<float*>(lds_sel + 64);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (lane < k) {
    const uint32_t mk = t_key[lane];
    const int mi = t_id[lane];
    int rank = 0;
#pragma unroll
    for (int t = 0; t < 16; ++t) {            // k <= 16; reads batched, entries past k ignored
      const uint32_t ok = t_key[t];
      const int oi = t_id[t];
      rank += (t < k && (ok > mk || (ok == mk && oi < mi))) ? 1 : 0;
    }
    f_id[rank] = mi;
    f_sc[rank] = t_sc[lane];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // renormalisation: sequential fp32 sum in selection order (lane 0), divisions on k lanes
  float denom = 0.0f;
  if (lane == 0) {
#pragma clang fp contract(off)
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = f_sc[r];
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc = r < k ? acc + v[r] : acc;
    denom = acc + 1e-20f;
  }
  denom = __shfl(denom, 0, 64);
  if (lane < k) {
#pragma clang fp contract(off)
    float wv = renorm ? f_sc[lane] / denom : f_sc[lane];
    if (scaling != 1.0f) wv = wv * scaling;
    inds_out[lane] = f_id[lane];
    w_out[lane] = wv;
  }
  __builtin_amdgcn_wave_barrier();
}

template <int PER>
__device__ __forceinline__ void wave_select_row_t(const float* s_row, const float* key_row, int E, int k, float scaling,
                                                  int32_t* inds_out, float* w_out, int* lds_sel, bool renorm = true) {
  const int lane = threadIdx.x & 63;
  uint32_t cv[PER];
  float sc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) sc[j] = s_row[(lane + 64 * j) < E ? lane + 64 * j : 0];   // with the keys below
  wave_load_keys<PER>(key_row, E, cv);
  bool take[PER];
  wave_select_set<PER>(cv, k, take);
  wave_stage_selected<PER>(cv, sc, take, lds_sel);
  wave_rank_renorm(k, scaling, inds_out, w_out, lds_sel, renorm);
}

__device__ __forceinline__ void wave_select_row(const float* s_row, const float* key_row, int E, int k, float scaling,
                                       int32_t* inds_out, float* w_out, int* lds_sel, bool renorm = true) {
  if (E <= 64) wave_select_row_t<1>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel, renorm);
  else if (E <= 128) wave_select_row_t<2>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel, renorm);
  else if (E <= 256) wave_select_row_t<4>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel, renorm);
  else if (E <= 512) wave_select_row_t<8>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel, renorm);
  else wave_select_row_t<16>(s_row, key_row, E, k, scaling, inds_out, w_out, lds_sel, renorm);
}

// ------------------------------------------------------------------ grouping (one wave, <= 64 routes)
// The same outputs as block_group_routes from ballots only: route t on lane t.  One pass over the slot bits,
// high to low, keeps `match` = live lanes that agree with this lane's slot on the bits seen so far; a lane
// dropped at a bit where this lane has a 1 holds a smaller slot.  lower = earlier routes of the slot (= the
// route's row position c), rank = distinct smaller slots (= u).  lurows/luw: LDS scratch of Umax*R entries.
__device__ __forceinline__ void wave_group_routes(const int32_t* inds, const float* scores, const int32_t* slot_of,
                                                  int M, int k, int R, int n_slots, int Umax, int32_t* uids,
                                                  int32_t* urows, int32_t* ucnt, float* uw, uint32_t* gidx,
                                                  int32_t* n_unique, int32_t* status, int* lurows, float* luw) {
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
  const uint64_t live = __ballot(lane < nr);
  const int nbits = n_slots > 1 ? 32 - __clz(n_slots - 1) : 1;      // slot ids are < n_slots
  uint64_t match = live, smaller = 0ull;
  for (int b = nbits - 1; b >= 0; --b) {
    const bool one = (s >> b) & 1;
    const uint64_t m = __ballot(one);
    smaller |= one ? (match & ~m) : 0ull;
    match &= one ? m : ~m;
  }
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int lower = __popcll(match & below);       // earlier routes of this slot = the route's row slot c
  const int same = __popcll(match);
  const bool first = lane < nr && lower == 0;
  const uint64_t firsts = __ballot(first);
  const int U = __popcll(firsts);
  const int rank = __popcll(smaller & firsts);     // distinct slots below this one
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
