// Small-batch (M <= 8 rows) MoE experts: distinct-expert gate/up + SwiGLU, down * router weight, fixed-order
// combine; and the fused decode block (router -> grouping -> experts -> combine) with no host sync.
//
// Reference: moe_experts engine/mimo_stream/kernels.py:176-199 (Kernel A :33-85, Kernel B :88-123, combine
// :198-199); _moe_small / _gather_m1 engine/mimo_stream/model.py:173-219.
//
// Each distinct expert's weights are streamed from HBM once and applied to every row routed to it.  The dot
// products run on gfx950 block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4): B = the expert's E2M1
// weights with their E8M0 scales, exactly as stored; A = the activations split into hi + lo E4M3 halves
// (each with its own E8M0 block scale) placed in MFMA rows 0-7 (hi) and 8-15 (lo), so one MFMA covers up to
// eight token rows at bf16 precision and the two halves are summed in fp32 afterwards.
//
// MFMA operand layout (16x16x128, lane l: g = l / 16, i = l % 16), measured on MI355X:
//   FP4 operand: lane holds K = 32g .. 32g+31 of row/column i (16 contiguous bytes).
//   FP8 operand: bytes 0-15 hold K = 16g .. 16g+15, bytes 16-31 hold K = 64+16g .. 64+16g+15.
//   scale of K-block b (32 wide) of row/column i comes from lane i + 16b (byte 0).
//   D: lane l holds column l % 16, rows 4g .. 4g+3.
#include <atomic>
#include <mutex>

#include "device.h"
#include "host.h"
#include "layer.h"
#include "router.h"
#include "routing.h"

namespace mimo {

struct ExpertsArgs {
  const uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;   // [M, H], [M, H/32]
  const uint32_t *gate_w, *up_w, *down_w;
  const uint8_t *gate_s, *up_s, *down_s;
  int H, I, R, Umax, k, M, S;
  const int32_t *uslot, *urows, *ucnt, *n_unique;
  const float* uw;
  const uint32_t* gidx;
  uint16_t* h;                              // [Umax, R, I] bf16
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;   // [Umax, R, I], [Umax, R, I/32]
  float* part;                              // [Umax, R, H]
  int round_bf16, zero_pad;
  uint16_t* y;                              // [M, H]
  // fused decode: the gate/up blocks select and group the routes themselves from the router's scores/keys
  const float *scores, *keys;               // [M, E]
  int E;
  const int32_t* slot_of;                   // [E] expert -> slot, or null (identity)
  int32_t* inds_out;                        // [M, k] routes (optional)
  float* w_out;                             // [M, k] weights (optional)
  int32_t *rt_uids, *rt_urows, *rt_ucnt;    // grouping written by block (0, 0) for the down kernel
  float* rt_uw;
  uint32_t* rt_gidx;
  int32_t *rt_nu, *rt_status;
  const uint16_t* resid;                    // [M, H] residual stream: y := bf16(resid + y) when given
};

// A operand (FP8 layout) for K-step k0 from a row of E4M3 codes; zero for padding rows.
__device__ __forceinline__ v8i a_operand(const uint8_t* row, int k0, int g, bool valid) {
  if (!valid) return v8i{0, 0, 0, 0, 0, 0, 0, 0};
  uint4 a0 = *reinterpret_cast<const uint4*>(row + k0 + 16 * g);
  uint4 a1 = *reinterpret_cast<const uint4*>(row + k0 + 64 + 16 * g);
  return v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
}
__device__ __forceinline__ v8i b_operand(uint4 b) { return v8i{(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0}; }

#define MFMA_F8xF4(A, B, C, SA, SB) __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4((A), (B), (C), 0, 4, 0, (SA), 0, (SB))

// ------------------------------------------------------------------ Kernel A: gate/up + SwiGLU
// Block (512 threads): one distinct expert u (blockIdx.y) x 32 outputs n (blockIdx.x).  Wave w: 16-output
// tile (w & 1) x K-range (w >> 1) of 4.  A wave's K-range is NS MFMA steps of K = 128 and its 2 x NS weight
// loads (16 B of gate and of up per lane and step) are issued in one straight-line batch and stay in
// registers, so a block keeps 8 x 16 KB of expert weights in flight.  Everything else the block reads is
// requested before that batch: the expert's activation rows go straight to LDS (global_load_lds) and the
// block's weight scales come in with one or two coalesced loads per thread; a load issued after the weight
// batch would queue behind it.  Loads never depend on the lane: padding rows read row 0 and are zeroed by
// selects.  K-range partials are summed in a fixed order through LDS; the epilogue applies the bf16 rounding
// points of kernels.py:79-82 and writes the hi/lo split of h (and h itself when the caller asked for it).
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int g) { return (w >> (8 * g)) & 0xFFu; }
// K split of the gate/up reduction: 4 ranges when H % 512 == 0, else 2; MFMA steps (K = 128) per range.
__host__ __device__ inline int gateup_ksplit(int H) { return H % 512 == 0 ? 4 : 2; }
__host__ __device__ inline int gateup_steps(int H) { return H / gateup_ksplit(H) / 128; }
__device__ __forceinline__ uint4 zero_if(uint4 v, bool keep) {
  return keep ? v : make_uint4(0, 0, 0, 0);
}
__host__ __device__ constexpr int align_up(int x, int a) { return (x + a - 1) / a * a; }

// Dynamic LDS of the gate/up kernel (bytes), for hidden size H and `rl` staged activation rows:
//   scales  2 x 32 rows x RS       gate then up scales of the block's rows, RS = H/32 + 16 (conflict-free reads)
//   a_hi    rl rows x RA           hi E4M3 codes of the staged rows, RA = H + 16 (rows 4 banks apart)
//   a_lo    rl rows x RA           lo codes, starting 128 bytes off a_hi's bank phase
//   a_sc    rl rows x 2 x H/32     [hi scales | lo scales] per row
// The K-range partials and the h tile reuse the activation region once the MFMA loop is done.
struct GateupLds {
  int RS, RA, a_hi, a_lo, a_sc, red, hl, total;
};
constexpr int kRedBytes = 4 * 2 * 2 * 32 * 4 * 4;   // [K-range][ntile][gate/up][lane][q] floats
__host__ __device__ inline GateupLds gateup_lds(int H, int rl) {
  GateupLds L;
  L.RS = H / 32 + 16;
  L.RA = H + 16;
  L.a_hi = 2 * 32 * L.RS;
  L.a_lo = align_up(L.a_hi + rl * L.RA, 256) + 128;
  L.a_sc = align_up(L.a_lo + rl * L.RA, 16);
  L.red = L.a_hi;
  L.hl = L.red + kRedBytes;
  const int a_end = L.a_sc + rl * 2 * (H / 32);
  const int e_end = L.hl + 8 * 32 * 4;
  L.total = a_end > e_end ? a_end : e_end;
  return L;
}

// Stage activation rows c0 .. c0 + n - 1 of the block's expert into LDS (rows 0 .. n - 1 there): per row, the
// hi and lo codes in 1 KB pieces and the [hi | lo] scales in one piece, spread over the block's NW waves,
// at most JMAX pieces per wave (n <= 8 rows of H <= 4096 need 9 with 8 waves).  Straight-line code: a loop here
// would make the compiler drain every outstanding load before entering it.
// tok: lane c holds the token of row c (wave-uniform reads through readlane).
template <int JMAX, int NW = 8>
__device__ __forceinline__ void stage_act_rows(const ExpertsArgs& a, uint8_t* lds, const GateupLds& L, int c0, int n,
                                               int tok, int wave, int lane) {
  const int nq = (a.H + 1023) >> 10;          // 1 KB pieces per half row
  const int per_row = 2 * nq + 1;
  const int hs = a.H / 32;
#pragma unroll
  for (int j = 0; j < JMAX; ++j) {
    const int t = wave + NW * j;
    if (t >= n * per_row) break;
    const int c = t / per_row, p = t - c * per_row;
    int token = __builtin_amdgcn_readlane(tok, c0 + c);
    token = (token < 0 || token >= a.M) ? 0 : token;
    if (p < 2 * nq) {
      const int half = p >= nq, q = half ? p - nq : p;
      const uint8_t* src = (half ? a.xq_lo : a.xq_hi) + (size_t)token * a.H + 1024 * q;
      const uint8_t* dst = lds + (half ? L.a_lo : L.a_hi) + c * L.RA + 1024 * q;
      if (1024 * q + 16 * lane < a.H) lds_copy16(src, 16 * lane, dst);
    } else {                                      // [hi scales | lo scales] of the row, 4 bytes per lane
      const uint8_t* dst = lds + L.a_sc + c * 2 * hs;
      if (4 * lane < hs) lds_copy4(a.xq_hs + (size_t)token * hs, 4 * lane, dst);
      else if (4 * lane < 2 * hs) lds_copy4(a.xq_ls + (size_t)token * hs - hs, 4 * lane, dst);
    }
  }
}

// Routes of one decode step for a block: wave r selects row r (top-k and renormalisation), wave 0 groups the
// routes by slot (E <= 256).
__device__ __forceinline__ void full_routing(const ExpertsArgs& a, int (*sel)[kSelLds], int32_t* s_inds, float* s_w,
                                             int* lurows, float* luw, int32_t* g_uids, int32_t* g_urows,
                                             int32_t* g_ucnt, float* g_uw, uint32_t* g_gidx, int32_t* g_nu, int wave) {
  if (wave < a.M)
    wave_select_row_t<4>(a.scores + wave * a.E, a.keys + wave * a.E, a.E, a.k, 1.0f, s_inds + wave * a.k,
                         s_w + wave * a.k, sel[wave]);
  __syncthreads();
  if (wave == 0)
    wave_group_routes(s_inds, s_w, a.slot_of, a.M, a.k, a.R, a.S, a.Umax, g_uids, g_urows, g_ucnt, g_uw, g_gidx,
                      &g_nu[0], &g_nu[1], lurows, luw);
  __syncthreads();
}

// Block (0, 0) of the routed gate/up kernel writes the step's routes and grouping for the down kernel (and the
// caller's inds/w), after its own loads: stores ahead of the weight loads would make them wait.
__device__ __forceinline__ void publish_routes(const ExpertsArgs& a, const int32_t* s_inds, const float* s_w,
                                               const int32_t* g_uids, const int32_t* g_urows, const int32_t* g_ucnt,
                                               const float* g_uw, const uint32_t* g_gidx, const int32_t* g_nu, int tid) {
  if (blockIdx.x != 0 || blockIdx.y != 0) return;
  const int nr = a.M * a.k;
  for (int e = tid; e < a.Umax * a.R; e += blockDim.x) { a.rt_urows[e] = g_urows[e]; a.rt_uw[e] = g_uw[e]; }
  for (int e = tid; e < a.Umax; e += blockDim.x) { a.rt_uids[e] = g_uids[e]; a.rt_ucnt[e] = g_ucnt[e]; }
  for (int e = tid; e < nr; e += blockDim.x) {
    a.rt_gidx[e] = g_gidx[e];
    if (a.inds_out) a.inds_out[e] = s_inds[e];
    if (a.w_out) a.w_out[e] = s_w[e];
  }
  if (tid == 0) { a.rt_nu[0] = g_nu[0]; a.rt_status[0] = g_nu[1]; }
}

// FAST2 (routed only; the launcher checks its conditions): two rows with expert ids as slots.
// HALF (the launcher uses it for one or two rows with expert ids as slots, where blocks take the fast selection):
// blocks of 256 threads and 16 outputs (wave w: K-range w), four per CU, so that a step's U x I / 16 blocks spread
// more evenly over the CUs than U x I / 32 larger ones; such a block writes h in bf16 and the down kernel splits
// it (an E8M0 block of h spans 32 outputs, two of these blocks).
template <int NS, bool ROUTED, bool FAST2, bool HALF = false>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) decode_gateup_kernel(ExpertsArgs a, int rl) {
  static_assert(!HALF || ROUTED, "16-output blocks only for the routed kernel");
  constexpr int NW = HALF ? 4 : 8;        // waves per block
  constexpr int NT = HALF ? 1 : 2;        // 16-output tiles per block
  constexpr int BO = 16 * NT;             // outputs per block
  extern __shared__ __align__(16) uint8_t lds[];
  // routed grouping (ROUTED only): kept for the publication at the end of block (0, 0)
  __shared__ int sel[ROUTED ? 8 : 1][kSelLds];
  __shared__ int32_t s_inds[ROUTED ? 64 : 1];
  __shared__ float s_w[ROUTED ? 64 : 1];
  __shared__ int lurows[ROUTED ? 512 : 1];
  __shared__ float luw[ROUTED ? 512 : 1];
  __shared__ int32_t g_uids[ROUTED ? 64 : 1], g_urows[ROUTED ? 512 : 1], g_ucnt[ROUTED ? 64 : 1], g_nu[2];
  __shared__ float g_uw[ROUTED ? 512 : 1];
  __shared__ uint32_t g_gidx[ROUTED ? 64 : 1];
  const int u = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar registers)
  int U, cnt_raw, slot, tok;          // tok: lane c < R holds the token of the expert's row c
  // one or two rows with expert ids as slots: a block needs only its expert, the u-th distinct selected id in
  // ascending order, and which rows chose it; the ranking and grouping are left to the publishing block
  const bool fast = ROUTED && (FAST2 || (a.M == 1 && a.slot_of == nullptr && a.S >= a.E));
  const bool publisher = ROUTED && blockIdx.x == 0 && blockIdx.y == 0;
  __shared__ uint64_t fast_mask[FAST2 ? 2 : 1][4];   // per row, the selection as ballot words (bit lane of word j)
  if (ROUTED && fast) {
    if (wave < (FAST2 ? 2 : 1)) {
      uint32_t cv[4];
      float sc[4];
      bool take[4];
      const int rb = wave * a.E;
#pragma unroll
      for (int j = 0; j < 4; ++j)                       // the scores only for the block that publishes the routes
        sc[j] = publisher ? a.scores[rb + ((lane + 64 * j) < a.E ? lane + 64 * j : 0)] : 0.0f;
      wave_load_keys<4>(a.keys + rb, a.E, cv);         // E <= 256 on this path
      wave_select_set<4>(cv, a.k, take);
      wave_stage_selected<4>(cv, sc, take, sel[wave]);  // ids in ascending order at sel[wave][16 ..]
      if constexpr (FAST2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint64_t m = __ballot(take[j]);
          if (lane == 0) fast_mask[wave][j] = m;
        }
      }
    }
    __syncthreads();
    if constexpr (!FAST2) {
      U = a.k;                                          // distinct experts, one row each
      cnt_raw = 1;
      slot = u < U ? sel[0][16 + u] : 0;
      tok = 0;
    } else {
      // distinct experts of the step in ascending id: the union of the two rows' selections
      uint64_t mu[4];
      int before = 0, jsel = 0, nsel = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        mu[j] = fast_mask[0][j] | fast_mask[1][j];
        const int c = __popcll(mu[j]);
        if (u >= before && u < before + c) { jsel = j; nsel = u - before; }
        before += c;
      }
      U = before;
      const int bit = u < U ? nth_set_bit(mu[jsel], nsel) : 0;
      slot = 64 * jsel + bit;
      const int in0 = (int)((fast_mask[0][jsel] >> bit) & 1ull);
      const int in1 = (int)((fast_mask[1][jsel] >> bit) & 1ull);
      cnt_raw = in0 + in1;
      tok = (lane == 0 && in0) ? 0 : 1;                 // the expert's first row: row 0 if it chose it, else row 1
    }
  } else if (ROUTED) {
    // routes of this step: wave r selects row r (top-k and renormalisation), wave 0 groups them by slot; every
    // block does this (it costs less than a separate launch) and block (0, 0) publishes the result at its end
    full_routing(a, sel, s_inds, s_w, lurows, luw, g_uids, g_urows, g_ucnt, g_uw, g_gidx, g_nu, wave);
    U = g_nu[0];
    cnt_raw = g_ucnt[u];
    slot = g_uids[u];
    tok = g_urows[u * a.R + min(lane, a.R - 1)];
  } else {
    // the routing metadata is loaded in one round trip (u < Umax, so every address is valid)
    U = a.n_unique ? *a.n_unique : a.Umax;
    cnt_raw = a.ucnt[u];
    slot = a.uslot[u];
    tok = a.urows[u * a.R + min(lane, a.R - 1)];
  }
  const int cnt = min(cnt_raw, a.R);
  // caller-supplied ids are range-checked; block (0, 0) of the routed kernel never returns here (expert 0 has a
  // row and a valid slot: the grouping maps invalid slots to 0 and flags them in the status)
  if (u >= U || cnt <= 0 || slot < 0 || slot >= a.S) return;
  wait_vm_all();   // the metadata loads are done; nothing the compiler tracks stays in flight past this point
  const GateupLds L = gateup_lds(a.H, rl);
  // the activation rows go first (they need only the metadata the weight addresses need as well)
  constexpr int JMAX = ROUTED ? (HALF ? 5 : 3) : 9;   // routed batches stage at most 2 rows at once, others 8
  stage_act_rows<JMAX, NW>(a, lds, L, 0, min(cnt, rl), tok, wave, lane);
  __builtin_amdgcn_sched_barrier(0);

  const int ntile = HALF ? 0 : (wave & 1), kr = HALF ? wave : (wave >> 1);
  const int nb = blockIdx.x * BO;
  const int n0 = nb + ntile * 16;
  const size_t brow = (size_t)slot * a.I + n0 + i;
  const int ksplit = gateup_ksplit(a.H);
  // with only two K-ranges (small H) waves 4-7 repeat K-range 0 and their partials are not used
  const int k0 = (kr < ksplit ? kr : 0) * NS * 128;
  const int b0 = k0 / 32;
  const uint4* gw = reinterpret_cast<const uint4*>(a.gate_w + brow * (a.H / 8)) + b0 + g;   // one uint4 per 32-block
  const uint4* upw = reinterpret_cast<const uint4*>(a.up_w + brow * (a.H / 8)) + b0 + g;
  // the block's gate and up scales (BO rows x H/32 bytes each, contiguous in the pools) in 8-byte pieces
  constexpr int LG_BO = HALF ? 4 : 5;
  const int lg_pr = __builtin_ctz(a.H / 256);             // pieces per scale row = H / 256
  const int npieces = (2 * BO) << lg_pr;
  const int p0 = tid, p1 = tid + 64 * NW;
  const int q0 = p0 < npieces ? p0 : 0, q1 = p1 < npieces ? p1 : 0;
  auto piece_src = [&](int p) {
    const int proj = p >> (LG_BO + lg_pr), row = (p >> lg_pr) & (BO - 1), c = p & ((1 << lg_pr) - 1);
    return reinterpret_cast<const uint2*>((proj ? a.up_s : a.gate_s) + ((size_t)slot * a.I + nb + row) * (a.H / 32)) + c;
  };
  auto piece_dst = [&](int p) {
    const int proj = p >> (LG_BO + lg_pr), row = (p >> lg_pr) & (BO - 1), c = p & ((1 << lg_pr) - 1);
    return reinterpret_cast<uint2*>(lds + (proj * 32 + row) * L.RS + 8 * c);
  };
  // the scale pieces, then the weight batch: the activation rows and the scales land first, so each MFMA step
  // can start as soon as its own weights arrive
  const uint2 sp0 = *piece_src(q0);
  const uint2 sp1 = *piece_src(q1);
  uint4 bg[NS], bu[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) { bg[s] = gw[4 * s]; bu[s] = upw[4 * s]; }
  __builtin_amdgcn_sched_barrier(0);
  if (ROUTED && fast && publisher && wave == 0) {
    // the step's full routing for the down kernel while this block's loads stream: ranking, renormalisation and
    // grouping of the staged selections touch only LDS and registers (workgroup fences wait on LDS only)
    for (int r = 0; r < a.M; ++r) {
      wave_rank_renorm(a.k, 1.0f, s_inds + r * a.k, s_w + r * a.k, sel[r], true);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
    wave_group_routes(s_inds, s_w, nullptr, a.M, a.k, a.R, a.S, a.Umax, g_uids, g_urows, g_ucnt, g_uw, g_gidx,
                      &g_nu[0], &g_nu[1], lurows, luw);
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vm_keep<2 * NS>();    // everything before the weight batch has landed: staged rows and scale pieces
  if (p0 < npieces) *piece_dst(p0) = sp0;
  if (p1 < npieces) *piece_dst(p1) = sp1;
  __syncthreads();

  v4f accg = {0.0f, 0.0f, 0.0f, 0.0f}, accu = {0.0f, 0.0f, 0.0f, 0.0f};
  const uint8_t* lrow = lds + (ntile * 16 + i) * L.RS + b0;   // this lane's gate scale row (up: + 32 rows)
  const int crow = i & 7;              // the expert's row c carried by this lane (hi rows 0-7, lo rows 8-15)
  // one pass over the staged rows: the operands of step s + 1 are read from LDS while step s multiplies
  auto run_pass = [&](int c0) {
    const bool avalid = crow >= c0 && crow < min(cnt, c0 + rl);
    const int lr = avalid ? crow - c0 : 0;
    const uint8_t* arow_p = lds + (i < 8 ? L.a_hi : L.a_lo) + lr * L.RA + k0 + 16 * g;
    const uint8_t* asc_p = lds + L.a_sc + lr * 2 * (a.H / 32) + (i < 8 ? 0 : a.H / 32) + b0;
    uint4 p = *reinterpret_cast<const uint4*>(arow_p), q = *reinterpret_cast<const uint4*>(arow_p + 64);
    uint32_t sw = *reinterpret_cast<const uint32_t*>(asc_p);
    uint32_t gs = *reinterpret_cast<const uint32_t*>(lrow), us = *reinterpret_cast<const uint32_t*>(lrow + 32 * L.RS);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint4 pc = zero_if(p, avalid), qc = zero_if(q, avalid);
      const int sa = avalid ? (int)byte_of(sw, g) : 127;
      const int sgc = (int)byte_of(gs, g), suc = (int)byte_of(us, g);
      if (s + 1 < NS) {
        p = *reinterpret_cast<const uint4*>(arow_p + 128 * (s + 1));
        q = *reinterpret_cast<const uint4*>(arow_p + 128 * (s + 1) + 64);
        sw = *reinterpret_cast<const uint32_t*>(asc_p + 4 * (s + 1));
        gs = *reinterpret_cast<const uint32_t*>(lrow + 4 * (s + 1));
        us = *reinterpret_cast<const uint32_t*>(lrow + 32 * L.RS + 4 * (s + 1));
      }
      v8i A = {(int)pc.x, (int)pc.y, (int)pc.z, (int)pc.w, (int)qc.x, (int)qc.y, (int)qc.z, (int)qc.w};
      accg = MFMA_F8xF4(A, b_operand(bg[s]), accg, sa, sgc);
      accu = MFMA_F8xF4(A, b_operand(bu[s]), accu, sa, suc);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  run_pass(0);
  for (int c0 = rl; c0 < cnt; c0 += rl) {   // rare: more rows routed to one expert than staged at once
    __syncthreads();
    stage_act_rows<JMAX, NW>(a, lds, L, c0, min(cnt - c0, rl), tok, wave, lane);
    wait_vm_all();
    __syncthreads();
    run_pass(c0);
  }
  mfma_f8f4_settle();
  float vg[4], vu[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {   // rows 4g+q (hi, g < 2) plus rows 8+4g+q (lo) of lane l + 32
    vg[q] = accg[q] + __shfl_xor(accg[q], 32, 64);
    vu[q] = accu[q] + __shfl_xor(accu[q], 32, 64);
  }
  __syncthreads();                 // the activation region is free: K-range partials and the h tile go there
  float (*red)[2][2][32][4] = reinterpret_cast<float (*)[2][2][32][4]>(lds + L.red);   // [K-range][ntile][g/u][lane][q]
  float (*hl)[32] = reinterpret_cast<float (*)[32]>(lds + L.hl);
  if (lane < 32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) { red[kr][ntile][0][lane][q] = vg[q]; red[kr][ntile][1][lane][q] = vu[q]; }
  }
  __syncthreads();
  // SwiGLU, one (row, output) per thread: K-range partials summed in a fixed order (0, 1, 2, 3)
  uint16_t hb = 0;
  const int e_q = tid & 3, e_l = (tid >> 2) & 31, e_nt = HALF ? 0 : ((tid >> 7) & 1);
  const int e_r = 4 * (e_l >> 4) + e_q, e_n = e_nt * 16 + (e_l & 15);
  if (tid < 128 * NT) {
    float gsum = red[0][e_nt][0][e_l][e_q], usum = red[0][e_nt][1][e_l][e_q];
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      const float pg = red[j][e_nt][0][e_l][e_q], pu = red[j][e_nt][1][e_l][e_q];
      gsum += j < ksplit ? pg : 0.0f;
      usum += j < ksplit ? pu : 0.0f;
    }
    const uint16_t gt = f32_to_bf16(gsum);
    const float gtf = bf16_to_f32(gt);
    const float ut = round_bf16(usum);
    const float sig = round_bf16(sigmoid_spec(gtf));   // the bf16 sigmoid table's entry for gt, computed in place
    const float hv = round_bf16(round_bf16(gtf * sig) * ut);
    hb = e_r < cnt ? f32_to_bf16(hv) : (uint16_t)0;
    if constexpr (!HALF) hl[e_r][e_n] = e_r < cnt ? hv : 0.0f;
  }
  if constexpr (HALF) {            // h in bf16 for the down kernel's split (and the padding rows when asked)
    if (tid < 128 && (e_r < cnt || (a.zero_pad && e_r < a.R)))
      a.h[((size_t)u * a.R + e_r) * a.I + nb + e_n] = hb;
    if (publisher) publish_routes(a, s_inds, s_w, g_uids, g_urows, g_ucnt, g_uw, g_gidx, g_nu, tid);
    return;
  }
  __syncthreads();
  if (a.zero_pad && tid < 256 && e_r < a.R)   // h itself only for callers that asked for the intermediates
    a.h[((size_t)u * a.R + e_r) * a.I + nb + e_n] = hb;
  if (tid < 256) {                 // hi/lo E4M3 split of h per (row, 32-block): one value per lane, a row per half-wave
    const int r = tid >> 5, nl = tid & 31;
    const float v = hl[r][nl];
    // max over the 32 lanes of the row: DPP within each 16-lane row, then one exchange between the two rows
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
    if (r < cnt) {
      const size_t row = (size_t)u * a.R + r;
      a.hq_hi[row * a.I + nb + nl] = (uint8_t)hc;
      a.hq_lo[row * a.I + nb + nl] = (uint8_t)lc;
      if (nl == 0) {
        a.hq_hs[row * (a.I / 32) + blockIdx.x] = (uint8_t)(X + 127);
        a.hq_ls[row * (a.I / 32) + blockIdx.x] = (uint8_t)(Y + 127);
      }
    }
  }
  if (publisher)   // block (0, 0) publishes the full routing for the down kernel
    publish_routes(a, s_inds, s_w, g_uids, g_urows, g_ucnt, g_uw, g_gidx, g_nu, tid);
}

// ------------------------------------------------------------------ Kernel B + combine (owner computes)
// Block (1024 threads, 16 waves) owns 16 outputs m (blockIdx.x) for every distinct expert.  Work item
// (u, K-half): wave w takes items w, w + 16, ...  Per item, the wave first sends the expert's h rows for its
// K-half straight to a wave-private LDS buffer (global_load_lds) and its weight scales to registers, then
// issues its NS = I / 256 weight steps in one batch; a load issued after that batch would queue behind it.
// The routing metadata and the combine inputs all come in with one round trip at the start.  The two K-half
// dot products of each route land in LDS (one row per route: expert u's rows start at the sum of the
// earlier experts' counts); the block adds them in a fixed order, applies the router weight (and the bf16
// rounding of the gather_qmm path when asked, model.py:181), sums each row's k routes in route order
// (kernels.py:198-199) and writes y.  No other block is waited for.

// Per-wave LDS buffer of the down kernel for `rw` staged h rows of one K-half (KH = I / 2 codes):
// hi rows (KH + 16 bytes each), lo rows (starting 128 bytes off the hi rows' bank phase), then per row the
// [hi | lo] scales (2 x KH / 32 bytes).
struct DownLds {
  int KH, RA, hi, lo, sc, wave_bytes, part, total;
};
__host__ __device__ inline DownLds down_lds(int I, int rw, int nroutes) {
  DownLds L;
  L.KH = I / 2;
  L.RA = L.KH + 16;
  L.hi = 0;
  L.lo = align_up(rw * L.RA, 256) + 128;
  L.sc = align_up(L.lo + rw * L.RA, 16);
  L.wave_bytes = align_up(L.sc + rw * 2 * (L.KH / 32), 256);
  L.part = 16 * L.wave_bytes;                       // [2][nroutes][16] floats
  L.total = L.part + 2 * nroutes * 16 * 4;
  return L;
}

// HSPLIT: h comes in bf16 (from the 16-output gate/up blocks) and each wave splits its item's rows into the hi/lo
// E4M3 planes itself while its weights stream, a lane pair per 32-block and the (at most rw <= 2) staged rows one
// after the other; the planes and scales are those the gate/up epilogue writes otherwise.
template <int NS, bool HSPLIT = false>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4))) decode_down_combine_kernel(ExpertsArgs a, int rw) {
  extern __shared__ __align__(16) uint8_t dl[];
  __shared__ uint32_t cgidx[64];      // combine indices and weights, loaded with the routing metadata
  __shared__ float cuw[1024];
  __shared__ int cpref[64], ccnt[64]; // first route row and row count of each distinct expert
  constexpr int SRS = NS + 4;         // dwords per staged scale row (16-byte aligned, conflict-free row reads)
  __shared__ __align__(16) uint32_t wsc[16][16 * SRS];   // per wave: the current item's 16 scale rows
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar registers)
  const int m0 = blockIdx.x * 16;
  const int UR = a.Umax * a.R;
  const int nr = a.M * a.k;
  const DownLds L = down_lds(a.I, rw, nr);
  // one round trip: per-expert counts and slots (lane j holds expert j), the combine inputs, the count
  const int ej = min(lane, a.Umax - 1);
  const int cntv = min(max(a.ucnt[ej], 0), a.R), slotv = a.uslot[ej];
  const uint32_t gi = a.gidx[min(tid, nr - 1)];
  const float wi = a.uw[min(tid, UR - 1)];
  const int U = a.n_unique ? min(*a.n_unique, a.Umax) : a.Umax;
  // the combine's residual element (thread tid < M * 16: row tid / 16, output m0 + tid % 16) comes in with them
  const uint16_t rres = (a.resid && tid < a.M * 16) ? a.resid[(size_t)(tid >> 4) * a.H + m0 + (tid & 15)] : (uint16_t)0;
  // first route row of expert j = sum of the earlier experts' counts (counts <= 8: four bit-plane ballots)
  int prefv = 0;
  {
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int c = lane < a.Umax ? cntv : 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) prefv += __popcll(__ballot((c >> b) & 1) & below) << b;
  }
  uint8_t* wb = dl + wave * L.wave_bytes;
  // h rows of the item staged at rows 0 .. n - 1 (n <= 3) of the wave's buffer: hi and lo codes of the K-half
  // (KH <= 1024 bytes, one piece each) and the [hi | lo] scales
  auto stage = [&](int u, int kh, int c0, int n) {
    const int sb = L.KH / 32;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      if (c >= n) break;
      const size_t row = (size_t)u * a.R + c0 + c;
      if (16 * lane < L.KH) {
        lds_copy16(a.hq_hi + row * a.I + kh * L.KH, 16 * lane, wb + L.hi + c * L.RA);
        lds_copy16(a.hq_lo + row * a.I + kh * L.KH, 16 * lane, wb + L.lo + c * L.RA);
      }
      const uint8_t* dst = wb + L.sc + c * 2 * sb;
      if (4 * lane < sb) lds_copy4(a.hq_hs + row * (a.I / 32) + kh * sb, 4 * lane, dst);
      else if (4 * lane < 2 * sb) lds_copy4(a.hq_ls + row * (a.I / 32) + kh * sb - sb, 4 * lane, dst);
    }
  };
  // HSPLIT: lane l holds bf16 values 16 l .. 16 l + 15 of the K-half (block l / 2) of staged rows c0 and c0 + 1
  auto hload = [&](int u, int kh, int c0, int n, bool active, uint4 (&hv)[2][2]) {
    const bool live = active && 16 * lane < L.KH;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const size_t row = (size_t)u * a.R + c0 + (c < n ? c : 0);
      const uint4* hp = reinterpret_cast<const uint4*>(a.h + row * a.I + kh * L.KH + 16 * (live ? lane : 0));
      hv[c][0] = hp[0];
      hv[c][1] = hp[1];
    }
    return live;
  };
  // every lane calls this (the pair exchanges its block maxima); rows c < n of the live lanes are written
  auto hsplit = [&](const uint4 (&hv)[2][2], int n, bool live) {
    const int sb = L.KH / 32;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      if (c >= n) break;                            // wave-uniform
      const uint32_t pw[8] = {hv[c][0].x, hv[c][0].y, hv[c][0].z, hv[c][0].w,
                              hv[c][1].x, hv[c][1].y, hv[c][1].z, hv[c][1].w};
      uint32_t hw[4], lw[4];
      int X, Y;
      quant_pair_fp8_hilo(pw, hw, lw, &X, &Y);
      if (live) {
        *reinterpret_cast<uint4*>(wb + L.hi + c * L.RA + 16 * lane) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *reinterpret_cast<uint4*>(wb + L.lo + c * L.RA + 16 * lane) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        if ((lane & 1) == 0) {
          wb[L.sc + c * 2 * sb + (lane >> 1)] = (uint8_t)(X + 127);
          wb[L.sc + c * 2 * sb + sb + (lane >> 1)] = (uint8_t)(Y + 127);
        }
      }
    }
  };
  // scale staging: lane L loads 8 bytes of row L / LPR of the item's K-half (NS * 4 bytes per row)
  constexpr int LPR = NS / 2;
  const int srow = min(lane / LPR, 15), spart = lane % LPR;
  const int crow = i & 7;
  float* part = reinterpret_cast<float*>(dl + L.part);
  for (int item = wave; item < 2 * U; item += 16) {
    const int u = item >> 1, kh = item & 1;
    const int cnt = __builtin_amdgcn_readlane(cntv, u);
    const int slot = __builtin_amdgcn_readlane(slotv, u);
    const int rbase = __builtin_amdgcn_readlane(prefv, u);
    const bool active = cnt > 0 && slot >= 0 && slot < a.S;
    uint4 hv[2][2];
    bool hlive = false;
    if constexpr (HSPLIT) hlive = hload(u, kh, 0, min(cnt, rw), active, hv);
    else if (active) stage(u, kh, 0, min(cnt, rw));
    const int b0 = kh * NS * 4;      // first 32-block of this K-half
    const size_t bslot = (size_t)(active ? slot : 0) * a.H + m0;
    const uint4* dw = reinterpret_cast<const uint4*>(a.down_w + (bslot + i) * (a.I / 8)) + b0 + g;
    const uint2 sraw = *(reinterpret_cast<const uint2*>(a.down_s + (bslot + srow) * (a.I / 32) + b0) + spart);
    uint4 bw[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) bw[s] = dw[4 * s];
    __builtin_amdgcn_sched_barrier(0);   // every weight load is in flight before anything waits
    wait_vm_keep<NS>();                  // the staged rows and the scales have landed; each MFMA step then waits
                                         // only for its own weights
    if constexpr (HSPLIT) hsplit(hv, min(cnt, rw), hlive);   // while the weights stream
    if (lane < 16 * LPR) *reinterpret_cast<uint2*>(&wsc[wave][srow * SRS + 2 * spart]) = sraw;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t* srow_p = &wsc[wave][i * SRS];
    // one pass over the staged rows: the operands of step s + 1 are read from LDS while step s multiplies
    auto run_pass = [&](int c0) {
      const bool avalid = crow >= c0 && crow < min(cnt, c0 + rw);
      const int lr = avalid ? crow - c0 : 0;
      const uint8_t* arow_p = wb + (i < 8 ? L.hi : L.lo) + lr * L.RA + 16 * g;
      const uint8_t* asc_p = wb + L.sc + lr * 2 * (L.KH / 32) + (i < 8 ? 0 : L.KH / 32);
      uint4 p = *reinterpret_cast<const uint4*>(arow_p), q = *reinterpret_cast<const uint4*>(arow_p + 64);
      uint32_t sw = *reinterpret_cast<const uint32_t*>(asc_p), bs = srow_p[0];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint4 pc = zero_if(p, avalid), qc = zero_if(q, avalid);
        const int sa = avalid ? (int)byte_of(sw, g) : 127;
        const int sb = (int)byte_of(bs, g);
        if (s + 1 < NS) {
          p = *reinterpret_cast<const uint4*>(arow_p + 128 * (s + 1));
          q = *reinterpret_cast<const uint4*>(arow_p + 128 * (s + 1) + 64);
          sw = *reinterpret_cast<const uint32_t*>(asc_p + 4 * (s + 1));
          bs = srow_p[s + 1];
        }
        v8i A = {(int)pc.x, (int)pc.y, (int)pc.z, (int)pc.w, (int)qc.x, (int)qc.y, (int)qc.z, (int)qc.w};
        acc = MFMA_F8xF4(A, b_operand(bw[s]), acc, sa, sb);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (active) run_pass(0);
    for (int c0 = rw; active && c0 < cnt; c0 += rw) {   // rare: more rows on one expert than the buffer holds
      __builtin_amdgcn_wave_barrier();
      if constexpr (HSPLIT) {
        uint4 hv2[2][2];
        const bool live2 = hload(u, kh, c0, min(cnt - c0, rw), true, hv2);
        wait_vm_all();
        hsplit(hv2, min(cnt - c0, rw), live2);
      } else {
        stage(u, kh, c0, min(cnt - c0, rw));
      }
      wait_vm_all();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      run_pass(c0);
    }
    __builtin_amdgcn_wave_barrier();     // the staged rows and scales are read before the next item overwrites them
    mfma_f8f4_settle();
    float dq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) dq[q] = acc[q] + __shfl_xor(acc[q], 32, 64);   // hi rows + lo rows
    if (lane < 32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 4 * g + q;
        if (r < cnt && rbase + r < nr) part[(kh * nr + rbase + r) * 16 + i] = dq[q];
      }
    }
  }
  if (tid < nr) cgidx[tid] = gi;
  if (tid < UR) cuw[tid] = wi;
  if (tid < 64) { cpref[tid] = prefv; ccnt[tid] = lane < a.Umax ? cntv : 0; }
  __syncthreads();
  // route row of a (u, c) index (u < U); -1 when it carries no route
  auto route_row = [&](uint32_t idx) -> int {
    const int u = (int)(idx / (uint32_t)a.R), c = (int)(idx % (uint32_t)a.R);
    const int row = cpref[u] + c;
    return (c < ccnt[u] && row < nr) ? row : -1;
  };
  if (a.zero_pad) {          // copy of the partials (kernels.py:120) for callers that asked for them
    for (int e = tid; e < U * a.R * 16; e += blockDim.x) {
      const int ur = e >> 4, mi = e & 15;
      const int u = ur / a.R, c = ur - u * a.R;
      (void)u; (void)c;
      float d = 0.0f;
      const int row = route_row((uint32_t)ur);
      if (row >= 0) d = part[row * 16 + mi] + part[(nr + row) * 16 + mi];
      if (a.round_bf16) d = round_bf16(d);
      a.part[(size_t)ur * a.H + m0 + mi] = d * cuw[ur];
    }
  }
  // combine: every (route, output) term d * w in parallel, then each output adds its k terms in route order
  const uint32_t nrows = (uint32_t)(U * a.R);
  __shared__ float cterm[1024];       // [M * k][16], M * k <= 64
  if (tid < nr * 16) {
    const int t = tid >> 4, mi = tid & 15;
    const uint32_t idx = cgidx[t];
    const int pr = idx < nrows ? route_row(idx) : -1;
    float term = 0.0f;
    if (pr >= 0) {
      float d = part[pr * 16 + mi] + part[(nr + pr) * 16 + mi];
      if (a.round_bf16) d = round_bf16(d);
      term = d * cuw[idx];
    }
    cterm[tid] = term;
  }
  __syncthreads();
  if (tid < a.M * 16) {
    const int row = tid >> 4, mi = tid & 15;
    float accy = 0.0f;
    for (int j = 0; j < a.k; ++j) accy = accy + cterm[(row * a.k + j) * 16 + mi];
    const uint16_t yb = f32_to_bf16(accy);
    a.y[(size_t)row * a.H + m0 + mi] = a.resid ? residual_bf16(rres, yb) : yb;
  }
}

// ------------------------------------------------------------------ host
struct ExpertsWs {
  uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;
  uint16_t* h;
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;
  float* part;
};
// intermediates: room for the bf16 h and the fp32 partials, written only when a caller of mimo_moe_experts asks
// for them (the fused decode never does); bf16_h: room for h alone (the two-row fused decode passes h in bf16)
static ExpertsWs carve_experts(Carve& c, int M, int Umax, int R, int H, int I, bool intermediates,
                               bool bf16_h = false) {
  ExpertsWs w{};
  w.xq_hi = c.take<uint8_t>((size_t)M * H);
  w.xq_lo = c.take<uint8_t>((size_t)M * H);
  w.xq_hs = c.take<uint8_t>((size_t)M * H / 32);
  w.xq_ls = c.take<uint8_t>((size_t)M * H / 32);
  if (intermediates || bf16_h) w.h = c.take<uint16_t>((size_t)Umax * R * I);
  w.hq_hi = c.take<uint8_t>((size_t)Umax * R * I);
  w.hq_lo = c.take<uint8_t>((size_t)Umax * R * I);
  w.hq_hs = c.take<uint8_t>((size_t)Umax * R * I / 32);
  w.hq_ls = c.take<uint8_t>((size_t)Umax * R * I / 32);
  if (intermediates) w.part = c.take<float>((size_t)Umax * R * H);
  return w;
}

static int check_bank(const mimo_bank* b) {
  MIMO_REQUIRE(b && b->gate_w && b->gate_s && b->up_w && b->up_s && b->down_w && b->down_s, MIMO_ERR_ARG,
               "bank: null pointer");
  const int H = b->hidden, ns = gateup_steps(H);
  const int nsd = b->inter / 256;
  MIMO_REQUIRE(b->n_slots >= 1 && (ns == 1 || ns == 2 || ns == 4 || ns == 8) && H % 256 == 0 && b->inter % 256 == 0 &&
                   (nsd == 2 || nsd == 4 || nsd == 8),
               MIMO_ERR_SHAPE, "bank: need hidden in {256, 512, 1024, 2048, 4096} and inter in {512, 1024, 2048} (got "
               "H=%d I=%d)", b->hidden, b->inter);
  MIMO_REQUIRE(((reinterpret_cast<uintptr_t>(b->gate_s) | reinterpret_cast<uintptr_t>(b->up_s) |
                 reinterpret_cast<uintptr_t>(b->down_s)) & 7) == 0,
               MIMO_ERR_ALIGN, "bank: scale pools must be 8-byte aligned");
  MIMO_REQUIRE(aligned16(b->gate_w) && aligned16(b->up_w) && aligned16(b->down_w), MIMO_ERR_ALIGN,
               "bank: weight pools must be 16-byte aligned");
  return MIMO_OK;
}

// Dynamic LDS above the default 64 KB has to be allowed per kernel once.  `allowed` (the largest size set so far)
// is read without a lock; raising it is serialised, so the attribute never drops below a size already allowed.
static std::mutex g_lds_attr_mu;
static int allow_lds(const void* fn, size_t bytes, std::atomic<int>* allowed) {
  if ((int)bytes <= 65536 || (int)bytes <= allowed->load(std::memory_order_acquire)) return MIMO_OK;
  std::lock_guard<std::mutex> lk(g_lds_attr_mu);
  if ((int)bytes <= allowed->load(std::memory_order_relaxed)) return MIMO_OK;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess)
    return set_error(MIMO_ERR_HIP, "hipFuncSetAttribute(%zu bytes of LDS): %s", bytes, hipGetErrorString(e));
  allowed->store((int)bytes, std::memory_order_release);
  return MIMO_OK;
}

template <int NS, bool ROUTED, bool FAST2>
static int launch_gateup(const ExpertsArgs& a, int rl, hipStream_t st) {
  static std::atomic<int> allowed{0};
  const size_t lds = (size_t)gateup_lds(a.H, rl).total;
  int rc = allow_lds(reinterpret_cast<const void*>(&decode_gateup_kernel<NS, ROUTED, FAST2>), lds, &allowed);
  if (rc) return rc;
  decode_gateup_kernel<NS, ROUTED, FAST2><<<dim3(a.I / 32, a.Umax), 512, lds, st>>>(a, rl);
  return MIMO_OK;
}

template <int NS, bool HSPLIT = false>
static int launch_down(const ExpertsArgs& a, int rw, hipStream_t st) {
  static std::atomic<int> allowed{0};
  const size_t lds = (size_t)down_lds(a.I, rw, a.M * a.k).total;
  int rc = allow_lds(reinterpret_cast<const void*>(&decode_down_combine_kernel<NS, HSPLIT>), lds, &allowed);
  if (rc) return rc;
  decode_down_combine_kernel<NS, HSPLIT><<<a.H / 16, 1024, lds, st>>>(a, rw);
  return MIMO_OK;
}

// one or two rows, expert ids as slots: 16-output gate/up blocks (h in bf16), the down kernel splitting h
template <int NS, bool FAST2>
static int launch_gateup_half(const ExpertsArgs& a, int rl, hipStream_t st) {
  static std::atomic<int> allowed{0};
  const size_t lds = (size_t)gateup_lds(a.H, rl).total;
  int rc = allow_lds(reinterpret_cast<const void*>(&decode_gateup_kernel<NS, true, FAST2, true>), lds, &allowed);
  if (rc) return rc;
  decode_gateup_kernel<NS, true, FAST2, true><<<dim3(a.I / 16, a.Umax), 256, lds, st>>>(a, rl);
  return MIMO_OK;
}

static int run_experts(const ExpertsArgs& base, int M, int round_bf16, hipStream_t st) {
  ExpertsArgs a = base;
  a.round_bf16 = round_bf16;
  const int ns = gateup_steps(a.H);    // MFMA steps per wave
  // activation rows staged at once: a row picks an expert at most once, so an expert gets at most M rows;
  // more (a slot table mapping two experts of a row to one slot) costs extra passes, not wrong results
  const bool fused_select = a.scores && a.Umax <= 16 && a.E <= 256;   // small batches: every block selects
  const int rl = min(a.R, fused_select ? min(M, 2) : M);   // the routed kernel stages at most 2 rows at once
  const int rw = min(min(a.R, M), 3);
  if (a.scores && !fused_select) {
    int rc = launch_select_group(a.scores, a.keys, a.M, a.E, a.k, a.slot_of, a.R, a.S, a.Umax, a.inds_out, a.w_out,
                                 a.rt_uids, a.rt_urows, a.rt_ucnt, a.rt_uw, a.rt_gidx, a.rt_nu, a.rt_status, st);
    if (rc) return rc;
  }
  int rc;
  bool half = false;   // 16-output gate/up blocks, h split by the down kernel
  {
    ProfScope p(st, "decode_gateup");
    // two rows with expert ids as slots (E <= 256 for a fused selection): each block finds its own expert from
    // the two threshold searches alone (one row does the same inside the general routed kernel)
    const bool fast2 = fused_select && a.slot_of == nullptr && a.S >= a.E && M == 2;
    const bool fast1 = fused_select && a.slot_of == nullptr && a.S >= a.E && M == 1;
    half = (fast1 || fast2) && a.h != nullptr && rw <= 2 && !a.zero_pad;
    if (half) {
      switch (ns * 2 + (fast2 ? 1 : 0)) {
        case 17: rc = launch_gateup_half<8, true>(a, rl, st); break;
        case 16: rc = launch_gateup_half<8, false>(a, rl, st); break;
        case 9: rc = launch_gateup_half<4, true>(a, rl, st); break;
        case 8: rc = launch_gateup_half<4, false>(a, rl, st); break;
        case 5: rc = launch_gateup_half<2, true>(a, rl, st); break;
        case 4: rc = launch_gateup_half<2, false>(a, rl, st); break;
        case 3: rc = launch_gateup_half<1, true>(a, rl, st); break;
        default: rc = launch_gateup_half<1, false>(a, rl, st); break;
      }
    } else if (fused_select) {   // cheaper than a separate selection launch
      switch (ns * 2 + (fast2 ? 1 : 0)) {
        case 17: rc = launch_gateup<8, true, true>(a, rl, st); break;
        case 16: rc = launch_gateup<8, true, false>(a, rl, st); break;
        case 9: rc = launch_gateup<4, true, true>(a, rl, st); break;
        case 8: rc = launch_gateup<4, true, false>(a, rl, st); break;
        case 5: rc = launch_gateup<2, true, true>(a, rl, st); break;
        case 4: rc = launch_gateup<2, true, false>(a, rl, st); break;
        case 3: rc = launch_gateup<1, true, true>(a, rl, st); break;
        default: rc = launch_gateup<1, true, false>(a, rl, st); break;
      }
    } else {
      switch (ns) {
        case 8: rc = launch_gateup<8, false, false>(a, rl, st); break;
        case 4: rc = launch_gateup<4, false, false>(a, rl, st); break;
        case 2: rc = launch_gateup<2, false, false>(a, rl, st); break;
        default: rc = launch_gateup<1, false, false>(a, rl, st); break;
      }
    }
  }
  if (rc) return rc;
  {
    ProfScope p(st, "decode_down_combine");
    switch (a.I / 256 + (half ? 16 : 0)) {
      case 24: rc = launch_down<8, true>(a, rw, st); break;
      case 20: rc = launch_down<4, true>(a, rw, st); break;
      case 18: rc = launch_down<2, true>(a, rw, st); break;
      case 8: rc = launch_down<8>(a, rw, st); break;
      case 4: rc = launch_down<4>(a, rw, st); break;
      default: rc = launch_down<2>(a, rw, st); break;
    }
  }
  if (rc) return rc;
  return check_launch("moe experts");
}

}  // namespace mimo

using namespace mimo;

extern "C" {

size_t mimo_moe_experts_workspace_size(int M, int Umax, int R, int H, int I) {
  Carve c(nullptr, 0);
  carve_experts(c, M, Umax, R, H, I, true);
  return c.off;
}

int mimo_moe_experts(const uint16_t* x, int M, const mimo_bank* bank, const int32_t* uslot, const int32_t* urows,
                     const int32_t* ucnt, const float* uw, const int32_t* n_unique, int Umax, int R,
                     const uint32_t* gidx, int k, int round_expert_bf16, uint16_t* y, uint16_t* h_out,
                     float* part_out, void* ws, size_t ws_bytes, void* stream) {
  ProfChain chain;   // per-kernel timing (when enabled) back to back within this call
  int rc = check_bank(bank);
  if (rc) return rc;
  MIMO_REQUIRE(x && uslot && urows && ucnt && uw && gidx && y, MIMO_ERR_ARG, "moe_experts: null pointer");
  MIMO_REQUIRE(M >= 1 && M <= 8 && R >= 1 && R <= 8 && k >= 1 && M * k <= 64 && Umax >= 1 && Umax <= M * k &&
                   Umax * R <= 1024,
               MIMO_ERR_SHAPE, "moe_experts: need 1 <= M <= 8, 1 <= R <= 8, M*k <= 64, 1 <= Umax <= M*k, "
               "Umax*R <= 1024");
  MIMO_REQUIRE(aligned16(x) && aligned16(y) && (!part_out || aligned16(part_out)), MIMO_ERR_ALIGN,
               "moe_experts: x, y, part_out must be 16-byte aligned");
  const int H = bank->hidden, I = bank->inter;
  Carve c(ws, ws_bytes);
  ExpertsWs w = carve_experts(c, M, Umax, R, H, I, true);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_experts: workspace too small (need %zu)", c.off);
  hipStream_t st = as_stream(stream);
  rc = launch_quantize_fp8_hilo(x, M, H, w.xq_hi, w.xq_hs, w.xq_lo, w.xq_ls, st);
  if (rc) return rc;
  ExpertsArgs a{};
  a.xq_hi = w.xq_hi; a.xq_lo = w.xq_lo; a.xq_hs = w.xq_hs; a.xq_ls = w.xq_ls;
  a.gate_w = bank->gate_w; a.up_w = bank->up_w; a.down_w = bank->down_w;
  a.gate_s = bank->gate_s; a.up_s = bank->up_s; a.down_s = bank->down_s;
  a.H = H; a.I = I; a.R = R; a.Umax = Umax; a.k = k; a.M = M; a.S = bank->n_slots;
  a.uslot = uslot; a.urows = urows; a.ucnt = ucnt; a.n_unique = n_unique; a.uw = uw; a.gidx = gidx;
  a.h = h_out ? h_out : w.h;
  a.hq_hi = w.hq_hi; a.hq_lo = w.hq_lo; a.hq_hs = w.hq_hs; a.hq_ls = w.hq_ls;
  a.part = part_out ? part_out : w.part;
  a.zero_pad = (h_out || part_out) ? 1 : 0;
  a.y = y;
  return run_experts(a, M, round_expert_bf16, st);
}

static void carve_decode(Carve& c, int M, int E, int k, int Umax, int R, float** logits, float** scores, float** keys,
                         int32_t** inds, float** w, int32_t** uids, int32_t** urows, int32_t** ucnt,
                         float** uw, uint32_t** gidx, int32_t** nu, int32_t** status) {
  *logits = c.take<float>((size_t)M * E);
  *scores = c.take<float>((size_t)M * E);
  *keys = c.take<float>((size_t)M * E);
  *inds = c.take<int32_t>((size_t)M * k);
  *w = c.take<float>((size_t)M * k);
  *uids = c.take<int32_t>(Umax);
  *urows = c.take<int32_t>((size_t)Umax * R);
  *ucnt = c.take<int32_t>(Umax);
  *uw = c.take<float>((size_t)Umax * R);
  *gidx = c.take<uint32_t>((size_t)M * k);
  *nu = c.take<int32_t>(1);
  *status = c.take<int32_t>(1);
}

static const int kDecodeR = 8;   // VERIFY_MAX (model.py:27): rows per distinct expert

size_t mimo_moe_decode_workspace_size(int M, int E, int k, int H, int I) {
  Carve c(nullptr, 0);
  // the call carves min(M * k, n_slots) distinct-expert entries; the bank's slot count is not an argument here,
  // so size for M * k, which covers every bank
  const int Umax = M * k;
  float *l, *s, *kk, *w, *uw;
  int32_t *inds, *uids, *urows, *ucnt, *nu, *st;
  uint32_t* gidx;
  carve_decode(c, M, E, k, Umax, kDecodeR, &l, &s, &kk, &inds, &w, &uids, &urows, &ucnt, &uw, &gidx, &nu, &st);
  carve_experts(c, M, Umax, kDecodeR, H, I, false, M <= 2);
  return c.off;
}

}  // extern "C"

namespace mimo {
// The fused decode block on rows x (router logits + hi/lo split, experts, combine); resid: optional residual
// stream added in the combine; norm_w: optional RMSNorm of the rows inside the router kernel (r to r_out if given).
static int decode_impl(const uint16_t* x, int M, const uint16_t* Wg, const float* bias, const int32_t* slot_of, int E,
                       int k, const mimo_bank* bank, uint16_t* y, int32_t* inds_out, float* w_out,
                       const uint16_t* resid, const uint16_t* norm_w, float eps, uint16_t* r_out,
                       int32_t* status_out, void* ws, size_t ws_bytes, hipStream_t st) {
  int rc = check_bank(bank);
  if (rc) return rc;
  MIMO_REQUIRE(x && Wg && bias && y, MIMO_ERR_ARG, "moe_decode: null pointer");
  MIMO_REQUIRE(M >= 1 && M <= 8 && k >= 1 && k <= 8 && E >= k && E <= 1024 && bank->n_slots <= 1024, MIMO_ERR_SHAPE,
               "moe_decode: need 1 <= M <= 8, 1 <= k <= 8, k <= E <= 1024");
  MIMO_REQUIRE(aligned16(x) && aligned16(Wg) && aligned16(y), MIMO_ERR_ALIGN, "moe_decode: 16-byte alignment");
  MIMO_REQUIRE(bank->hidden <= 4096, MIMO_ERR_SHAPE, "moe_decode: the fused router keeps a row in registers: H <= 4096");
  const int H = bank->hidden, I = bank->inter, S = bank->n_slots;
  const int Umax = M * k < S ? M * k : S;
  Carve c(ws, ws_bytes);
  float *logits, *scores, *keys, *w, *uw;
  int32_t *inds, *uids, *urows, *ucnt, *nu, *status;
  uint32_t* gidx;
  carve_decode(c, M, E, k, Umax, kDecodeR, &logits, &scores, &keys, &inds, &w, &uids, &urows, &ucnt, &uw,
               &gidx, &nu, &status);
  ExpertsWs ew = carve_experts(c, M, Umax, kDecodeR, H, I, false, M <= 2);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_decode: workspace too small (need %zu)", c.off);

  RouterSmallArgs ra{};
  ra.x = x; ra.Wg = Wg; ra.bias = bias; ra.T = M; ra.H = H; ra.E = E; ra.k = k;
  ra.logits = logits; ra.scores = scores; ra.keys = keys;
  ra.xq_hi = ew.xq_hi; ra.xq_lo = ew.xq_lo; ra.xq_hs = ew.xq_hs; ra.xq_ls = ew.xq_ls;
  ra.norm_w = norm_w; ra.eps = eps; ra.r_out = r_out;
  rc = launch_router_logits_small(ra, st);
  if (rc) return rc;

  ExpertsArgs a{};
  a.xq_hi = ew.xq_hi; a.xq_lo = ew.xq_lo; a.xq_hs = ew.xq_hs; a.xq_ls = ew.xq_ls;
  a.gate_w = bank->gate_w; a.up_w = bank->up_w; a.down_w = bank->down_w;
  a.gate_s = bank->gate_s; a.up_s = bank->up_s; a.down_s = bank->down_s;
  a.H = H; a.I = I; a.R = kDecodeR; a.Umax = Umax; a.k = k; a.M = M; a.S = S;
  a.uslot = uids; a.urows = urows; a.ucnt = ucnt; a.n_unique = nu; a.uw = uw; a.gidx = gidx;
  a.h = ew.h; a.hq_hi = ew.hq_hi; a.hq_lo = ew.hq_lo; a.hq_hs = ew.hq_hs; a.hq_ls = ew.hq_ls;
  a.part = ew.part; a.zero_pad = 0; a.y = y;
  a.scores = scores; a.keys = keys; a.E = E; a.slot_of = slot_of;
  a.inds_out = inds_out ? inds_out : inds;
  a.w_out = w_out ? w_out : w;
  a.rt_uids = uids; a.rt_urows = urows; a.rt_ucnt = ucnt; a.rt_uw = uw; a.rt_gidx = gidx; a.rt_nu = nu;
  a.rt_status = status_out ? status_out : status;   // written on every call (block (0, 0) or the selection launch)
  a.resid = resid;
  // M == 1 follows _gather_m1 (bf16 expert outputs, model.py:173-182); M >= 2 the distinct-expert kernels
  return run_experts(a, M, M == 1 ? 1 : 0, st);
}
}  // namespace mimo

extern "C" {

int mimo_moe_decode(const uint16_t* x, int M, const uint16_t* Wg, const float* bias, const int32_t* slot_of, int E,
                    int k, const mimo_bank* bank, uint16_t* y, int32_t* inds_out, float* w_out, int32_t* status_out,
                    void* ws, size_t ws_bytes, void* stream) {
  ProfChain chain;   // per-kernel timing (when enabled) back to back within this call
  return decode_impl(x, M, Wg, bias, slot_of, E, k, bank, y, inds_out, w_out, nullptr, nullptr, 0.0f, nullptr,
                     status_out, ws, ws_bytes, as_stream(stream));
}

// The layer step normalises the rows inside the router kernel: no rows of r are kept unless r_out asks for them,
// so the workspace is the decode block's.
size_t mimo_moe_layer_decode_workspace_size(int M, int E, int k, int H, int I) {
  return mimo_moe_decode_workspace_size(M, E, k, H, I);
}

int mimo_moe_layer_decode(const uint16_t* x, int M, const uint16_t* norm_w, float eps, const uint16_t* Wg,
                          const float* bias, const int32_t* slot_of, int E, int k, const mimo_bank* bank, uint16_t* h,
                          uint16_t* r_out, int32_t* inds_out, float* w_out, int32_t* status_out, void* ws,
                          size_t ws_bytes, void* stream) {
  ProfChain chain;
  MIMO_REQUIRE(x && norm_w && h && bank, MIMO_ERR_ARG, "moe_layer_decode: null pointer");
  MIMO_REQUIRE(M >= 1 && M <= 8, MIMO_ERR_SHAPE, "moe_layer_decode: need 1 <= M <= 8");
  MIMO_REQUIRE(aligned16(x) && aligned16(h) && aligned16(norm_w) && (!r_out || aligned16(r_out)), MIMO_ERR_ALIGN,
               "moe_layer_decode: 16-byte alignment");
  MIMO_REQUIRE(r_out != x && r_out != h, MIMO_ERR_ARG, "moe_layer_decode: r_out may not alias x or h");
  MIMO_REQUIRE(eps >= 0.0f && eps == eps, MIMO_ERR_ARG, "moe_layer_decode: eps must be a non-negative number");
  return decode_impl(x, M, Wg, bias, slot_of, E, k, bank, h, inds_out, w_out, x, norm_w, eps, r_out, status_out, ws,
                     ws_bytes, as_stream(stream));
}

}  // extern "C"

// ------------------------------------------------------------------ layer decode without a caller workspace
// The workspace of mimo_moe_layer_decode_noalloc: a file-scope device array, one copy per GPU, held until the
// process ends.  Host code never passes `scratch` itself to a kernel (in host code it names a host-side
// stand-in); it uses the device address that hipGetSymbolAddress returns for the current device.
namespace mimo {
constexpr size_t kNoAllocScratchBytes = MIMO_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// Device address of this GPU's scratch array, looked up once per device (with that device current).
static int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(MIMO_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  MIMO_REQUIRE(dev >= 0 && dev < 64, MIMO_ERR_HIP, "device %d: at most 64 devices", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(MIMO_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MIMO_OK;
}
}  // namespace mimo

extern "C" {

int mimo_moe_layer_decode_noalloc(const uint16_t* x, int M, const uint16_t* norm_w, float eps, const uint16_t* Wg,
                                  const float* bias, const int32_t* slot_of, int E, int k, const mimo_bank* bank,
                                  uint16_t* h, uint16_t* r_out, int32_t* inds_out, float* w_out, int32_t* status_out,
                                  void* stream) {
  ProfSuspend no_events;   // event timing would create events: this entry point allocates nothing
  MIMO_REQUIRE(bank, MIMO_ERR_ARG, "moe_layer_decode_noalloc: null bank");
  MIMO_REQUIRE(M >= 1 && M <= 8 && k >= 1 && k <= 8 && E >= 1 && E <= 1024, MIMO_ERR_SHAPE,
               "moe_layer_decode_noalloc: need 1 <= M <= 8, 1 <= k <= 8, E <= 1024");
  const size_t need = mimo_moe_layer_decode_workspace_size(M, E, k, bank->hidden, bank->inter);
  MIMO_REQUIRE(need <= kNoAllocScratchBytes, MIMO_ERR_WORKSPACE,
               "moe_layer_decode_noalloc: M=%d, E=%d, k=%d, hidden %d, intermediate %d need %zu bytes of scratch; "
               "the built-in scratch holds %zu (use mimo_moe_layer_decode with a workspace)", M, E, k, bank->hidden,
               bank->inter, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  int rc = scratch_address(&ws);
  if (rc) return rc;
  return mimo_moe_layer_decode(x, M, norm_w, eps, Wg, bias, slot_of, E, k, bank, h, r_out, inds_out, w_out,
                               status_out, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"
