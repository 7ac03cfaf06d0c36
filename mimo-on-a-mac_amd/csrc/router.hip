// Router (gate linear, sigmoid + bias selection, top-k, renormalisation), distinct-expert grouping and the
// prefill counting-sort dispatch.
//
// Reference: Router.__call__ engine/mimo_stream/model.py:58-65; group_routes engine/mimo_stream/kernels.py:
// 149-173; prefill dispatch model.py:235-242, :266-268.  Selection order is canonical: descending key
// (sigmoid + bias), ties to the lower expert id, NaN keys last; weights are renormalised with a sequential
// fp32 sum in that order.  Everything here is integer or exactly specified fp32/fp64 arithmetic, so routes
// and permutations are bit-exact against the oracle given identical logits.
#include "device.h"
#include "host.h"
#include "layer.h"
#include "router.h"
#include "routing.h"

namespace mimo {

// ------------------------------------------------------------------ grouping (one block, <= 1024 routes)
// group_routes restated: uids ascending, urows/uw in route order per expert, gidx = u*R + c.
// Requires blockDim.x >= n_routes and LDS `present` of n_slots ints.
__device__ void block_group_routes(const int32_t* inds, const float* scores, const int32_t* slot_of, int M, int k,
                                   int R, int n_slots, int Umax, int32_t* uids, int32_t* urows, int32_t* ucnt,
                                   float* uw, uint32_t* gidx, int32_t* n_unique, int32_t* status, int* present,
                                   int* route_slot) {
  const int tid = threadIdx.x;
  const int nr = M * k;
  for (int i = tid; i < n_slots; i += blockDim.x) present[i] = 0;
  for (int i = tid; i < Umax * R; i += blockDim.x) { urows[i] = 0; uw[i] = 0.0f; }
  for (int i = tid; i < Umax; i += blockDim.x) { ucnt[i] = 0; uids[i] = 0; }
  __syncthreads();
  int bad = 0;
  if (tid < nr) {
    int e = inds[tid];
    int s = slot_of ? (e >= 0 ? slot_of[e] : -1) : e;
    if (s < 0 || s >= n_slots) { bad = MIMO_ERR_SLOT; s = 0; }
    route_slot[tid] = s;
    present[s] = 1;
  }
  __syncthreads();
  if (tid == 0) {          // ascending ranks of present slots (sequential, deterministic)
    int u = 0;
    for (int s = 0; s < n_slots; ++s) {
      if (present[s]) { present[s] = u + 1; ++u; }
    }
    n_unique[0] = u;
  }
  __syncthreads();
  if (tid < nr) {
    int s = route_slot[tid];
    int u = present[s] - 1;
    int c = 0;
    for (int t = 0; t < tid; ++t) c += (route_slot[t] == s);
    if (c >= R) {
      bad = MIMO_ERR_ROWS_PER_EXPERT;
    } else if (u < Umax) {
      urows[u * R + c] = tid / k;
      uw[u * R + c] = scores[tid];
      gidx[tid] = (uint32_t)(u * R + c);
      uids[u] = s;
      int total = c;
      for (int t = tid + 1; t < nr; ++t) total += (route_slot[t] == s);
      if (c == 0) ucnt[u] = total + 1 > R ? R : total + 1;
    }
  }
  // status: first nonzero code wins deterministically (lowest route index)
  __shared__ int s_bad;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  if (bad) atomicMin(&s_bad, bad);      // codes are negative: min = most severe, order independent
  __syncthreads();
  if (tid == 0) status[0] = s_bad;
}

// ------------------------------------------------------------------ small-T router (T <= 8)
// Two kernels, no cross-block synchronisation inside either:
//  router_logits_small_kernel: blocks [0, nlog = E) give one block per expert: T logits (fp32 FMA over bf16
//    products; each wave a quarter of the row, loaded in one batch with the T activation rows, summed through
//    DPP and then in LDS in a fixed order), then sigmoid and key by one thread per row;
//    blocks [nlog, ...) split x into hi/lo E4M3 halves for the expert kernels (one thread per 32-block).
//  router_select_group_kernel (one block): top-k per row (one wave per row) and the grouping by slot.
template <int NCH>
__global__ void __launch_bounds__(256) router_logits_small_kernel(RouterSmallArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q4 = a.H / 4;
  const bool norm = a.norm_w != nullptr;
  __shared__ float wsum[8][4];            // per row, the 4 wave sums of squares (norm only)
  if ((int)blockIdx.x >= a.nlog) {           // hi/lo split of x: one element per lane, 32 lanes per block
    if (!a.xq_hi && !a.r_out) return;
    const int64_t n = (int64_t)a.T * a.H;
    const int64_t idx = ((int64_t)(blockIdx.x - a.nlog) * blockDim.x + threadIdx.x);
    const bool live = idx < n;
    uint16_t xb = live ? a.x[idx] : (uint16_t)0;
    if (norm) {
      // the block's 256 elements lie in one row (H a multiple of 256): that row's inverse RMS, computed exactly as
      // the logits blocks and the norm kernel compute it
      const int64_t row = ((int64_t)(blockIdx.x - a.nlog) * blockDim.x) / a.H;
      const uint16_t wb = a.norm_w[live ? idx - row * a.H : 0];
      const uint16_t* xq = a.x + row * a.H + wave * q4;
      uint4 xv[NCH];
      bool ok[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int off = c * 512 + lane * 8;
        ok[c] = off < q4;
        xv[c] = *reinterpret_cast<const uint4*>(xq + (ok[c] ? off : 0));
      }
      float ss = 0.0f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) ss = ok[c] ? norm_sq_add8(xv[c], ss) : ss;
      ss = norm_wave_sum(ss);
      if (lane == 0) wsum[0][wave] = ss;
      __syncthreads();
      xb = norm_apply1(xb, wb, norm_inv(wsum[0], a.H, a.eps));
      if (live && a.r_out) a.r_out[idx] = xb;
      if (!a.xq_hi) return;
    }
    const float v = live ? bf16_to_f32(xb) : 0.0f;
    float amax = dpp_group_max16(fabsf(v));
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    const int X = fp8_block_exp(amax);
    float res;
    const uint32_t hc = e4m3_encode(v, X, &res);
    float ramax = dpp_group_max16(fabsf(res));
    ramax = fmaxf(ramax, __shfl_xor(ramax, 16, 64));
    const int Y = fp8_block_exp(ramax);
    float lres;   // the lo code's own residual, unused
    const uint32_t lc = e4m3_encode(res, Y, &lres);
    if (live) {
      a.xq_hi[idx] = (uint8_t)hc;
      a.xq_lo[idx] = (uint8_t)lc;
      if ((lane & 31) == 0) {
        a.xq_hs[idx >> 5] = (uint8_t)(X + 127);
        a.xq_ls[idx >> 5] = (uint8_t)(Y + 127);
      }
    }
    return;
  }
  // block e: expert e's logits for the T <= 8 rows.  Wave w covers elements [w H/4, (w+1) H/4): lane owns the
  // 8-element chunks c*512 + lane*8 of that range (c < NCH; chunks past it read element 0 and count 0).
  __shared__ float part[8][4];
  const int e = blockIdx.x;
  const uint16_t* wrow = a.Wg + (size_t)e * a.H + wave * q4;
  uint4 wq[NCH], xq[8][NCH], nw[NCH];
  bool ok[NCH];
  // the expert's selection bias comes in with the first batch: loaded after the logit stores below it would be
  // one more memory round trip at the end of every block (the compiler cannot move it above stores it may alias)
  const float bias_e = a.keys ? a.bias[e] : 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int off = c * 512 + lane * 8;
    ok[c] = off < q4;
    wq[c] = *reinterpret_cast<const uint4*>(wrow + (ok[c] ? off : 0));
    if (norm) nw[c] = *reinterpret_cast<const uint4*>(a.norm_w + wave * q4 + (ok[c] ? off : 0));
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const uint16_t* xrow = a.x + (size_t)(r < a.T ? r : 0) * a.H + wave * q4;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (r < a.T) xq[r][c] = *reinterpret_cast<const uint4*>(xrow + (ok[c] ? c * 512 + lane * 8 : 0));
  }
  __builtin_amdgcn_sched_barrier(0);     // every load is in flight before the arithmetic
  if (norm) {                            // rows -> r: sums of squares in the norm kernel's order, then r in place
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (r < a.T) {
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) ss = ok[c] ? norm_sq_add8(xq[r][c], ss) : ss;
        ss = norm_wave_sum(ss);
        if (lane == 0) wsum[r][wave] = ss;
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (r < a.T) {
        const float inv = norm_inv(wsum[r], a.H, a.eps);
#pragma unroll
        for (int c = 0; c < NCH; ++c) xq[r][c] = norm_apply8(xq[r][c], nw[c], inv);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (r < a.T) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // four independent chains, added in a fixed order
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const uint4 xv = ok[c] ? xq[r][c] : make_uint4(0, 0, 0, 0);
        const uint32_t xp[4] = {xv.x, xv.y, xv.z, xv.w};
        const uint32_t wp[4] = {wq[c].x, wq[c].y, wq[c].z, wq[c].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[j] = fmaf(__uint_as_float(xp[j] << 16), __uint_as_float(wp[j] << 16), acc[j]);
          acc[j] = fmaf(__uint_as_float(xp[j] & 0xFFFF0000u), __uint_as_float(wp[j] & 0xFFFF0000u), acc[j]);
        }
      }
      const float s = dpp_sum_f32((acc[0] + acc[1]) + (acc[2] + acc[3]));
      if (lane == 0) part[r][wave] = s;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < a.T) {     // one thread per row: the four quarters in order, sigmoid and selection key
    const int r = threadIdx.x;
    const float l = ((part[r][0] + part[r][1]) + part[r][2]) + part[r][3];
    const float s = sigmoid_spec(l);
    a.logits[r * a.E + e] = l;
    if (a.scores) a.scores[r * a.E + e] = s;
    if (a.keys) a.keys[r * a.E + e] = s + bias_e;
  }
}

// One block, one wave per row: top-k and renormalisation, then wave 0 groups the routes by slot.
__global__ void __launch_bounds__(512) router_select_group_kernel(SelectGroupArgs a) {
  const int wave = threadIdx.x >> 6;
  __shared__ int sel[8][kSelLds];
  __shared__ int32_t s_inds[64];
  __shared__ float s_w[64];
  __shared__ int lurows[512];
  __shared__ float luw[512];
  if (wave < a.T)
    wave_select_row(a.scores + wave * a.E, a.keys + wave * a.E, a.E, a.k, 1.0f, s_inds + wave * a.k, s_w + wave * a.k,
                    sel[wave]);
  __syncthreads();
  for (int i = threadIdx.x; i < a.T * a.k; i += blockDim.x) {
    if (a.inds_out) a.inds_out[i] = s_inds[i];
    if (a.w_out) a.w_out[i] = s_w[i];
  }
  if (wave == 0)
    wave_group_routes(s_inds, s_w, a.slot_of, a.T, a.k, a.R, a.n_slots, a.Umax, a.uids, a.urows, a.ucnt, a.uw,
                      a.gidx, a.n_unique, a.status, lurows, luw);
}

int launch_select_group(const float* scores, const float* keys, int T, int E, int k, const int32_t* slot_of, int R,
                        int n_slots, int Umax, int32_t* inds_out, float* w_out, int32_t* uids, int32_t* urows,
                        int32_t* ucnt, float* uw, uint32_t* gidx, int32_t* n_unique, int32_t* status,
                        hipStream_t st) {
  SelectGroupArgs a{scores, keys, T, E, k, slot_of, R, n_slots, Umax, inds_out, w_out, uids, urows, ucnt, uw, gidx,
                    n_unique, status};
  ProfScope p(st, "router_select_group");
  router_select_group_kernel<<<1, 512, 0, st>>>(a);
  return check_launch("router_select_group");
}

// ------------------------------------------------------------------ general-T logits: tiled fp32 GEMM
// logits[t, e] = sum_h x[t, h] * W[e, h]; block tile 32 tokens x 64 experts, K chunks of 64 through LDS.
__global__ void __launch_bounds__(256) router_logits_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ W,
                                                            int T, int H, int E, float* __restrict__ logits,
                                                            int32_t* zero_status) {
  if (zero_status && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *zero_status = 0;
  __shared__ float xs[32][65];
  __shared__ float ws[64][65];
  const int t0 = blockIdx.y * 32, e0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;   // 16 x 16 threads; each 2 tokens x 4 experts
  float acc[2][4] = {};
  for (int k0 = 0; k0 < H; k0 += 64) {
    for (int i = threadIdx.x; i < 32 * 64; i += 256) {
      int r = i >> 6, c = i & 63;
      int t = t0 + r;
      xs[r][c] = t < T ? bf16_to_f32(x[(size_t)t * H + k0 + c]) : 0.0f;
    }
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
      int r = i >> 6, c = i & 63;
      int e = e0 + r;
      ws[r][c] = e < E ? bf16_to_f32(W[(size_t)e * H + k0 + c]) : 0.0f;
    }
    __syncthreads();
#pragma unroll 8
    for (int c = 0; c < 64; ++c) {
      float xv0 = xs[ty * 2][c], xv1 = xs[ty * 2 + 1][c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float wv = ws[tx * 4 + j][c];
        acc[0][j] = fmaf(xv0, wv, acc[0][j]);
        acc[1][j] = fmaf(xv1, wv, acc[1][j]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int t = t0 + ty * 2 + i;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int e = e0 + tx * 4 + j;
      if (t < T && e < E) logits[(size_t)t * E + e] = acc[i][j];
    }
  }
}

// one wave per row: sigmoid, key, top-k, renormalise; optional expert -> slot mapping for the dispatch
__global__ void __launch_bounds__(256) router_select_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
                                                            int T, int E, int k, float scaling, int32_t* inds,
                                                            float* w, const int32_t* slot_of, int32_t* slot_inds,
                                                            int n_slots, int32_t* status) {
  extern __shared__ float sm[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* s_row = sm + wave * 2 * E;
  float* k_row = s_row + E;
  __shared__ int sel[4][kSelLds];
  __shared__ int32_t oi[4][16];
  __shared__ float ow[4][16];
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  if (E <= 256) {   // every logit and bias of the row requested at once, the four sigmoids interleaved
    float lg[4], bs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j < E ? lane + 64 * j : 0;
      lg[j] = logits[(size_t)t * E + e];
      bs[j] = bias[e];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = sigmoid_spec(lg[j]);
      if (lane + 64 * j < E) {
        s_row[lane + 64 * j] = s;
        k_row[lane + 64 * j] = s + bs[j];
      }
    }
  } else {
    for (int e = lane; e < E; e += 64) {
      float s = sigmoid_spec(logits[(size_t)t * E + e]);
      s_row[e] = s;
      k_row[e] = s + bias[e];
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  wave_select_row(s_row, k_row, E, k, scaling, oi[wave], ow[wave], sel[wave]);
  if (lane < k) {
    int e = oi[wave][lane];
    if (inds) inds[(size_t)t * k + lane] = e;
    if (w) w[(size_t)t * k + lane] = ow[wave][lane];
    if (slot_inds) {
      int s = slot_of ? slot_of[e] : e;
      if (s < 0 || s >= n_slots) { atomicMin(status, MIMO_ERR_SLOT); s = 0; }
      slot_inds[(size_t)t * k + lane] = s;
    }
  }
}

// Group-limited selection of the vendored noaux-tc gate (engine/mimo_stream/mimo_v2.py:165-193), one wave per
// row: s = sigmoid(logit), key = s + bias; with n_group > 1 the experts split into n_group consecutive groups of
// G = E / n_group, a group's score is the sum of its two largest keys (mx.topk(..., 2), :180), and all but the
// topk_group highest-scoring groups have their keys set to exactly 0 (:181-185; ties between group scores go to
// the lower group index, NaN keys never count among a group's two largest); then the top-k of the keys, weights
// s at the chosen experts renormalised when norm_topk_prob and k > 1 (:190-191), times scaling (:192).
__global__ void __launch_bounds__(256) router_select_grouped_kernel(const float* __restrict__ logits,
                                                                    const float* __restrict__ bias, int T, int E, int k,
                                                                    int n_group, int topk_group, int norm,
                                                                    float scaling, int32_t* inds, float* w) {
  extern __shared__ float sm[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* s_row = sm + wave * 2 * E;
  float* k_row = s_row + E;
  __shared__ int sel[4][kSelLds];
  __shared__ int keep[4][64];
  __shared__ int32_t oi[4][16];
  __shared__ float ow[4][16];
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  for (int e = lane; e < E; e += 64) {
    const float s = sigmoid_spec(logits[(size_t)t * E + e]);
    s_row[e] = s;
    k_row[e] = s + bias[e];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (n_group > 1) {
    const int G = E / n_group;
    float gs = -__builtin_inff();
    if (lane < n_group) {          // lane g: the two largest keys of group g, in one pass
      float m1 = -__builtin_inff(), m2 = -__builtin_inff();
      for (int e = lane * G; e < (lane + 1) * G; ++e) {
        const float v = k_row[e];
        if (v > m1) { m2 = m1; m1 = v; }
        else if (v > m2) m2 = v;
      }
      gs = m1 + m2;
      gs = gs == gs ? gs : -__builtin_inff();
    }
    int rank = 0;                   // groups ahead of this one: higher score, or equal score and lower index
    for (int h = 0; h < n_group; ++h) {
      const float o = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs), h));
      rank += (o > gs || (o == gs && h < lane)) ? 1 : 0;
    }
    if (lane < n_group) keep[wave][lane] = rank < topk_group;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    for (int e = lane; e < E; e += 64)
      if (!keep[wave][e / G]) k_row[e] = 0.0f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
  wave_select_row(s_row, k_row, E, k, scaling, oi[wave], ow[wave], sel[wave], norm != 0 && k > 1);
  if (lane < k) {
    inds[(size_t)t * k + lane] = oi[wave][lane];
    w[(size_t)t * k + lane] = ow[wave][lane];
  }
}

__global__ void group_routes_kernel(const int32_t* inds, const float* scores, const int32_t* slot_of, int M, int k,
                                    int R, int n_slots, int Umax, int32_t* uids, int32_t* urows, int32_t* ucnt,
                                    float* uw, uint32_t* gidx, int32_t* n_unique, int32_t* status) {
  __shared__ int present[1024];
  __shared__ int route_slot[1024];
  if (M * k <= 64 && Umax * R <= 1024) {
    if (threadIdx.x < 64)
      wave_group_routes(inds, scores, slot_of, M, k, R, n_slots, Umax, uids, urows, ucnt, uw, gidx, n_unique, status,
                        present, reinterpret_cast<float*>(route_slot));
    return;
  }
  block_group_routes(inds, scores, slot_of, M, k, R, n_slots, Umax, uids, urows, ucnt, uw, gidx, n_unique, status,
                     present, route_slot);
}

// ------------------------------------------------------------------ prefill dispatch (stable counting sort)
constexpr int DISPATCH_CHUNK = 1024;

// slot ids outside [0, n_slots) are counted as slot 0 and flagged in *status (never indexed out of bounds)
__device__ __forceinline__ int checked_slot(const int32_t* slots, int i, int n_slots, int32_t* status) {
  int s = slots[i];
  if (s < 0 || s >= n_slots) {
    if (status) atomicMin(status, MIMO_ERR_SLOT);
    s = 0;
  }
  return s;
}

__global__ void __launch_bounds__(1024) dispatch_hist_kernel(const int32_t* __restrict__ slots, int n, int n_slots,
                                                             int32_t* __restrict__ hist, int32_t* status) {
  extern __shared__ int h[];
  for (int i = threadIdx.x; i < n_slots; i += blockDim.x) h[i] = 0;
  __syncthreads();
  int i = blockIdx.x * DISPATCH_CHUNK + threadIdx.x;
  if (i < n) atomicAdd(&h[checked_slot(slots, i, n_slots, status)], 1);   // integer counts: order independent
  __syncthreads();
  for (int s = threadIdx.x; s < n_slots; s += blockDim.x) hist[(size_t)blockIdx.x * n_slots + s] = h[s];
}

// Scan and placement in one launch: block b (one per chunk) sums the chunk histograms per slot (one thread per
// slot, n_slots <= 1024), scans the totals over the slots (wave scans), and places its chunk's routes at
// offsets[s] + sum_{b' < b} hist[b'][s] + (rank among the chunk's routes of slot s).  Block 0 also writes
// offsets and, with a TileSpec, the row tiles of each slot (see TileSpec).  Ranks within the chunk: earlier
// waves' counts of the slot (per-wave counts in LDS) plus earlier lanes of the wave (ballots over the slot bits).
__global__ void __launch_bounds__(1024) dispatch_scan_place_kernel(const int32_t* __restrict__ slots, int n,
                                                                   const int32_t* __restrict__ hist, int nchunks,
                                                                   int n_slots, int32_t* __restrict__ offsets,
                                                                   TileSpec spec, int4* __restrict__ tiles,
                                                                   int32_t* __restrict__ perm, int32_t* __restrict__ inv) {
  extern __shared__ int dsp[];                   // base[n_slots], then wc[16 waves][n_slots] (counts <= 64)
  int* base = dsp;
  uint16_t* wc = reinterpret_cast<uint16_t*>(dsp + n_slots);
  __shared__ int wsum[3][16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int blk = blockIdx.x;
  for (int i = tid; i < 16 * n_slots; i += blockDim.x) wc[i] = 0;
  // per-slot total and the part of it in earlier chunks (integer sums: any order)
  constexpr int HB = 16;
  int c = 0, pre = 0;
  if (tid < n_slots)
    for (int b0 = 0; b0 < nchunks; b0 += HB) {
      int h[HB];
#pragma unroll
      for (int u = 0; u < HB; ++u) h[u] = b0 + u < nchunks ? hist[(size_t)(b0 + u) * n_slots + tid] : 0;
#pragma unroll
      for (int u = 0; u < HB; ++u) {
        c += h[u];
        pre += b0 + u < blk ? h[u] : 0;
      }
    }
  const bool tl = tiles != nullptr && blk == 0;
  const int nw = (tl && c > spec.narrow_max) ? (c + spec.wide_rows - 1) / spec.wide_rows : 0;
  const int ns = (tl && c >= 1 && c <= spec.narrow_max) ? 1 : 0;
  int v0 = c, v1 = nw, v2 = ns;                  // inclusive scans within the wave
  for (int d = 1; d < 64; d <<= 1) {
    const int u0 = __shfl_up(v0, d, 64), u1 = __shfl_up(v1, d, 64), u2 = __shfl_up(v2, d, 64);
    if (lane >= d) {
      v0 += u0;
      v1 += u1;
      v2 += u2;
    }
  }
  if (lane == 63) {
    wsum[0][wv] = v0;
    wsum[1][wv] = v1;
    wsum[2][wv] = v2;
  }
  __syncthreads();
  for (int w = 0; w < wv; ++w) {
    v0 += wsum[0][w];
    v1 += wsum[1][w];
    v2 += wsum[2][w];
  }
  if (tid < n_slots) {
    const int e0 = v0 - c, e1 = v1 - nw, e2 = v2 - ns;   // exclusive prefixes
    base[tid] = e0 + pre;
    if (blk == 0) {
      offsets[tid] = e0;
      if (tid == n_slots - 1) {
        offsets[n_slots] = v0;
        if (tiles) tiles[0] = make_int4(v1, v2, 0, 0);
      }
      if (nw) {
        const int chunks = (c + spec.unit - 1) / spec.unit;
        for (int q = 0; q < nw; ++q) {
          const int c0 = (int)((int64_t)q * chunks / nw), c1 = (int)((int64_t)(q + 1) * chunks / nw);
          tiles[1 + e1 + q] = make_int4(tid, e0 + spec.unit * c0, e0 + min(spec.unit * c1, c), 0);
        }
      }
      if (ns) tiles[1 + spec.wcap + e2] = make_int4(tid, e0, e0 + c, 0);
    }
  }
  // placement of this chunk's routes (slot ids were range-checked and flagged by dispatch_hist_kernel; clamped
  // identically here)
  const int i = blk * DISPATCH_CHUNK + tid;
  const int sl = i < n ? checked_slot(slots, i, n_slots, nullptr) : -1;
  uint64_t same = __ballot(sl >= 0);
#pragma unroll
  for (int bit = 0; bit < 10; ++bit) {           // lanes whose slot agrees with this lane's in every bit
    const uint64_t ones = __ballot(sl >= 0 && ((sl >> bit) & 1));
    same &= ((sl >> bit) & 1) ? ones : ~ones;
  }
  const int lower = __popcll(same & ((1ull << lane) - 1));
  if (sl >= 0 && lower == 0) wc[wv * n_slots + sl] = (uint16_t)__popcll(same);   // the slot's first lane records
  __syncthreads();
  if (sl >= 0) {
    int before = 0;
    for (int w = 0; w < wv; ++w) before += wc[w * n_slots + sl];
    const int pos = base[sl] + before + lower;
    perm[pos] = i;
    if (inv) inv[i] = pos;
  }
}

int launch_dispatch(const int32_t* slots, int n, int n_slots, int32_t* hist, int32_t* perm, int32_t* offsets,
                    int32_t* inv, const TileSpec* spec, int4* tiles, int32_t* status, hipStream_t st) {
  int nchunks = (n + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK;
  if (nchunks == 0) nchunks = 1;
  ProfScope p(st, "prefill_dispatch");
  dispatch_hist_kernel<<<nchunks, 1024, n_slots * sizeof(int), st>>>(slots, n, n_slots, hist, status);
  const TileSpec none{0, 1, 0, 1};
  dispatch_scan_place_kernel<<<nchunks, 1024, n_slots * (sizeof(int) + 16 * sizeof(uint16_t)), st>>>(
      slots, n, hist, nchunks, n_slots, offsets, spec ? *spec : none, spec ? tiles : nullptr, perm, inv);
  return check_launch("prefill dispatch");
}

size_t dispatch_workspace(int n, int n_slots) {
  int nchunks = (n + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK;
  if (nchunks == 0) nchunks = 1;
  return align256((size_t)nchunks * n_slots * sizeof(int32_t));
}

int launch_router_logits_small(const RouterSmallArgs& args, hipStream_t st) {
  RouterSmallArgs a = args;
  MIMO_REQUIRE(!a.norm_w || (a.H % 256 == 0 && aligned16(a.norm_w) && a.eps >= 0.0f && a.eps == a.eps),
               MIMO_ERR_ARG, "router: the fused norm needs H a multiple of 256, an aligned weight and eps >= 0");
  int nquant = (a.xq_hi || (a.norm_w && a.r_out)) ? (int)(((int64_t)a.T * a.H + 255) / 256) : 0;
  a.nlog = a.E;
  const int nch = (a.H / 4 + 511) / 512;
  ProfScope p(st, "router_logits_small");
  switch (nch) {
    case 2: router_logits_small_kernel<2><<<a.nlog + nquant, 256, 0, st>>>(a); break;
    default: router_logits_small_kernel<1><<<a.nlog + nquant, 256, 0, st>>>(a); break;
  }
  return check_launch("router_logits_small");
}

// logits[T, E] = x[T, H] . W[E, H]^T on bf16 MFMA (v_mfma_f32_16x16x32_bf16: bf16 products exact in fp32, fp32
// accumulation), for the prefill chunks (T > 8).  Block (512 threads, 8 waves): 32 tokens x 64 experts; wave w
// takes K-range w of 8 (H / 8 columns, a multiple of 32) for all of the block's 2 x 4 MFMA tiles, reading its
// operands straight from global memory: lane (i = l % 16, g = l / 16) of a 16 x 32 step loads 8 consecutive bf16
// of token row i and of expert row i at columns 8g .. 8g + 7 (the same columns for both operands, so the
// product pairs them correctly whatever order the unit sums in).  The 8 partial tiles are added in LDS in wave
// order.  Rows past T or E read the last valid row and are not written.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kRlTok = 32, kRlExp = 64, kRlSplit = 8;

__global__ void __launch_bounds__(512) router_logits_mfma_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ W, int T, int H, int E,
                                                                 float* __restrict__ logits, int32_t* zero_status) {
  if (zero_status && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *zero_status = 0;
  __shared__ float part[kRlSplit][kRlTok][kRlExp];   // 64 KB
  const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t0 = blockIdx.y * kRlTok, e0 = blockIdx.x * kRlExp;
  const int KW = H / kRlSplit, kb = wave * KW;
  const uint4* xa[2];
  const uint4* wb[4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
    xa[a] = reinterpret_cast<const uint4*>(x + (size_t)min(t0 + 16 * a + i, T - 1) * H + kb + 8 * g);
#pragma unroll
  for (int b = 0; b < 4; ++b)
    wb[b] = reinterpret_cast<const uint4*>(W + (size_t)min(e0 + 16 * b + i, E - 1) * H + kb + 8 * g);
  v4f acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // 4 K-steps of 32 per round: 24 loads in flight, then 32 MFMAs
  const int steps = KW / 32;
  int s = 0;
  for (; s + 4 <= steps; s += 4) {
    uint4 av[4][2], bv[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int a = 0; a < 2; ++a) av[u][a] = xa[a][4 * (s + u)];
#pragma unroll
      for (int b = 0; b < 4; ++b) bv[u][b] = wb[b][4 * (s + u)];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[u][a]),
                                                              __builtin_bit_cast(bf16x8, bv[u][b]), acc[a][b], 0, 0, 0);
  }
  for (; s < steps; ++s) {
    uint4 av[2], bv[4];
#pragma unroll
    for (int a = 0; a < 2; ++a) av[a] = xa[a][4 * s];
#pragma unroll
    for (int b = 0; b < 4; ++b) bv[b] = wb[b][4 * s];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[a]),
                                                            __builtin_bit_cast(bf16x8, bv[b]), acc[a][b], 0, 0, 0);
  }
  // D: lane l holds expert column l % 16 and token rows 4 (l / 16) .. + 3 of each tile
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) part[wave][16 * a + 4 * g + q][16 * b + i] = acc[a][b][q];
  __syncthreads();
  for (int o = threadIdx.x; o < kRlTok * kRlExp; o += 512) {
    const int r = o / kRlExp, c = o % kRlExp;
    float v = part[0][r][c];
#pragma unroll
    for (int w = 1; w < kRlSplit; ++w) v = v + part[w][r][c];
    const int t = t0 + r, e = e0 + c;
    if (t < T && e < E) logits[(size_t)t * E + e] = v;
  }
}

int launch_router_logits(const uint16_t* x, const uint16_t* W, int T, int H, int E, float* logits, hipStream_t st,
                         int32_t* zero_status) {
  ProfScope p(st, "router_logits");
  if (H % (kRlSplit * 32) == 0 && aligned16(x) && aligned16(W)) {
    dim3 grid((E + kRlExp - 1) / kRlExp, (T + kRlTok - 1) / kRlTok);
    router_logits_mfma_kernel<<<grid, 512, 0, st>>>(x, W, T, H, E, logits, zero_status);
  } else {
    dim3 grid((E + 63) / 64, (T + 31) / 32);
    router_logits_kernel<<<grid, 256, 0, st>>>(x, W, T, H, E, logits, zero_status);
  }
  return check_launch("router_logits");
}

int launch_router_select(const float* logits, const float* bias, int T, int E, int k, float scaling, int32_t* inds,
                         float* w, const int32_t* slot_of, int32_t* slot_inds, int n_slots, int32_t* status,
                         hipStream_t st) {
  int blocks = (T + 3) / 4;
  ProfScope p(st, "router_select");
  router_select_kernel<<<blocks, 256, 4 * 2 * E * sizeof(float), st>>>(logits, bias, T, E, k, scaling, inds, w,
                                                                         slot_of, slot_inds, n_slots, status);
  return check_launch("router_select");
}

}  // namespace mimo

using namespace mimo;

extern "C" {

int mimo_router_select(const float* logits, const float* bias, int T, int E, int k, float scaling, int32_t* inds,
                       float* w, void* stream) {
  MIMO_REQUIRE(logits && bias && inds && w, MIMO_ERR_ARG, "router_select: null pointer");
  MIMO_REQUIRE(T >= 0 && E >= 1 && E <= 1024 && k >= 1 && k <= 16 && k <= E, MIMO_ERR_SHAPE,
               "router_select: need 1 <= k <= min(16, E), E <= 1024");
  if (T == 0) return MIMO_OK;
  return launch_router_select(logits, bias, T, E, k, scaling, inds, w, nullptr, nullptr, 0, nullptr,
                              as_stream(stream));
}

int mimo_router_select_grouped(const float* logits, const float* bias, int T, int E, int k, int n_group,
                               int topk_group, int norm_topk_prob, float scaling, int32_t* inds, float* w,
                               void* stream) {
  MIMO_REQUIRE(logits && bias && inds && w, MIMO_ERR_ARG, "router_select_grouped: null pointer");
  MIMO_REQUIRE(T >= 0 && E >= 1 && E <= 1024 && k >= 1 && k <= 16 && k <= E, MIMO_ERR_SHAPE,
               "router_select_grouped: need 1 <= k <= min(16, E), E <= 1024");
  MIMO_REQUIRE(n_group >= 1 && n_group <= 64 && E % n_group == 0 && (n_group == 1 || E / n_group >= 2) &&
                   topk_group >= 1 && topk_group <= n_group,
               MIMO_ERR_SHAPE, "router_select_grouped: need n_group <= 64 dividing E into groups of >= 2, "
               "1 <= topk_group <= n_group");
  if (T == 0) return MIMO_OK;
  hipStream_t st = as_stream(stream);
  ProfScope p(st, "router_select_grouped");
  router_select_grouped_kernel<<<(T + 3) / 4, 256, 4 * 2 * E * sizeof(float), st>>>(
      logits, bias, T, E, k, n_group, topk_group, norm_topk_prob, scaling, inds, w);
  return check_launch("router_select_grouped");
}

int mimo_router(const uint16_t* x, const uint16_t* Wg, const float* bias, int T, int H, int E, int k, float* logits,
                int32_t* inds, float* w, void* stream) {
  MIMO_REQUIRE(x && Wg && bias && logits && inds && w, MIMO_ERR_ARG, "router: null pointer");
  MIMO_REQUIRE(T >= 0 && H >= 64 && H % 64 == 0 && E >= 1 && E <= 1024 && k >= 1 && k <= 16 && k <= E,
               MIMO_ERR_SHAPE, "router: need H %% 64 == 0, 1 <= k <= min(16, E), E <= 1024");
  if (T == 0) return MIMO_OK;
  hipStream_t st = as_stream(stream);
  int rc;
  if (T <= 8 && H <= 4096) {   // decode-sized batches: the fused decode's logits kernel, so both give the same bits
    RouterSmallArgs ra{};
    ra.x = x; ra.Wg = Wg; ra.bias = bias; ra.T = T; ra.H = H; ra.E = E; ra.k = k; ra.logits = logits;
    rc = launch_router_logits_small(ra, st);
  } else {
    rc = launch_router_logits(x, Wg, T, H, E, logits, st);
  }
  if (rc) return rc;
  return launch_router_select(logits, bias, T, E, k, 1.0f, inds, w, nullptr, nullptr, 0, nullptr, st);
}

int mimo_group_routes(const int32_t* inds, const float* scores, const int32_t* slot_of, int M, int k, int R,
                      int n_slots, int32_t* uids, int32_t* urows, int32_t* ucnt, float* uw, uint32_t* gidx,
                      int32_t* n_unique, int32_t* status, void* stream) {
  MIMO_REQUIRE(inds && scores && uids && urows && ucnt && uw && gidx && n_unique && status, MIMO_ERR_ARG,
               "group_routes: null pointer");
  MIMO_REQUIRE(M >= 1 && k >= 1 && M * k <= 1024 && R >= 1 && n_slots >= 1 && n_slots <= 1024, MIMO_ERR_SHAPE,
               "group_routes: need 1 <= M*k <= 1024, 1 <= n_slots <= 1024");
  int Umax = M * k < n_slots ? M * k : n_slots;
  group_routes_kernel<<<1, 1024, 0, as_stream(stream)>>>(inds, scores, slot_of, M, k, R, n_slots, Umax, uids, urows,
                                                         ucnt, uw, gidx, n_unique, status);
  return check_launch("group_routes");
}

size_t mimo_prefill_dispatch_workspace_size(int T, int k, int n_slots) {
  return dispatch_workspace(T * k, n_slots);
}

int mimo_prefill_dispatch(const int32_t* slot_inds, int T, int k, int n_slots, int32_t* perm, int32_t* offsets,
                          int32_t* inv, void* ws, size_t ws_bytes, void* stream) {
  MIMO_REQUIRE(slot_inds && perm && offsets, MIMO_ERR_ARG, "prefill_dispatch: null pointer");
  MIMO_REQUIRE(T >= 0 && k >= 1 && n_slots >= 1 && n_slots <= 1024, MIMO_ERR_SHAPE,
               "prefill_dispatch: need 1 <= n_slots <= 1024");
  MIMO_REQUIRE(ws && ws_bytes >= dispatch_workspace(T * k, n_slots), MIMO_ERR_WORKSPACE,
               "prefill_dispatch: workspace too small");
  return launch_dispatch(slot_inds, T * k, n_slots, static_cast<int32_t*>(ws), perm, offsets, inv, nullptr, nullptr,
                         nullptr, as_stream(stream));
}

}  // extern "C"
