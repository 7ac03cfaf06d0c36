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
#include "device.h"
#include "host.h"
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
  const uint16_t* sigtab;
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
// tile (w & 1) x K-range (w >> 1) of 4.  A wave's K-range is NS MFMA steps of K = 128; all of its loads (16 B
// of gate and of up weights per lane and step, the activation halves and the scale words) are issued in one
// straight-line batch before the first MFMA, so a block keeps 8 x 16 KB of expert weights in flight.  Loads
// never depend on the lane: padding rows read row 0 and are zeroed by selects.  K-range partials are summed
// in a fixed order through LDS; the epilogue applies the bf16 rounding points of kernels.py:79-82 and writes
// h and its hi/lo split.
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int g) { return (w >> (8 * g)) & 0xFFu; }
// K split of the gate/up reduction: 4 ranges when H % 512 == 0, else 2; MFMA steps (K = 128) per range.
__host__ __device__ inline int gateup_ksplit(int H) { return H % 512 == 0 ? 4 : 2; }
__host__ __device__ inline int gateup_steps(int H) { return H / gateup_ksplit(H) / 128; }
__device__ __forceinline__ uint4 zero_if(uint4 v, bool keep) {
  return keep ? v : make_uint4(0, 0, 0, 0);
}

template <int NS, bool ROUTED>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) decode_gateup_kernel(ExpertsArgs a) {
  const int u = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int arow = min(i & 7, a.R - 1);
  int U, cnt_raw, slot, token;
  if (ROUTED) {
    // routes of this step: wave r selects row r (top-k and renormalisation), wave 0 groups them by slot; every
    // block does this (it costs less than a separate launch) and block (0, 0) publishes the result
    __shared__ int sel[8][32];
    __shared__ int32_t s_inds[64];
    __shared__ float s_w[64];
    __shared__ int lurows[512];
    __shared__ float luw[512];
    __shared__ uint32_t bits[32];
    __shared__ int32_t g_uids[64], g_urows[512], g_ucnt[64], g_nu[2];
    __shared__ float g_uw[512];
    __shared__ uint32_t g_gidx[64];
    if (wave < a.M)
      wave_select_row(a.scores + wave * a.E, a.keys + wave * a.E, a.E, a.k, 1.0f, s_inds + wave * a.k,
                      s_w + wave * a.k, sel[wave]);
    __syncthreads();
    if (wave == 0)
      wave_group_routes(s_inds, s_w, a.slot_of, a.M, a.k, a.R, a.S, a.Umax, g_uids, g_urows, g_ucnt, g_uw, g_gidx,
                        &g_nu[0], &g_nu[1], lurows, luw, bits);
    __syncthreads();
    if (blockIdx.x == 0 && blockIdx.y == 0) {
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
    U = g_nu[0];
    cnt_raw = g_ucnt[u];
    slot = g_uids[u];
    token = g_urows[u * a.R + arow];
  } else {
    // the routing metadata is loaded in one round trip (u < Umax, so every address is valid)
    U = a.n_unique ? *a.n_unique : a.Umax;
    cnt_raw = a.ucnt[u];
    slot = a.uslot[u];
    token = a.urows[u * a.R + arow];
  }
  if (u >= U) return;
  const int cnt = min(cnt_raw, a.R);
  if (cnt <= 0 || slot < 0 || slot >= a.S) return;     // caller-supplied ids are range-checked
  const int ntile = wave & 1, kr = wave >> 1;
  const int nb = blockIdx.x * 32;
  const int n0 = nb + ntile * 16;
  const bool avalid = (i & 7) < cnt;
  token = (!avalid || token < 0 || token >= a.M) ? 0 : token;
  const uint8_t* abase = (i < 8 ? a.xq_hi : a.xq_lo) + (size_t)token * a.H;
  const uint8_t* ascl = (i < 8 ? a.xq_hs : a.xq_ls) + (size_t)token * (a.H / 32);
  const size_t brow = (size_t)slot * a.I + n0 + i;
  const bool kactive = kr < gateup_ksplit(a.H);     // wave-uniform
  const int k0 = (kactive ? kr : 0) * NS * 128;
  const int b0 = k0 / 32;
  const uint4* gw = reinterpret_cast<const uint4*>(a.gate_w + brow * (a.H / 8)) + b0 + g;   // one uint4 per 32-block
  const uint4* upw = reinterpret_cast<const uint4*>(a.up_w + brow * (a.H / 8)) + b0 + g;
  const uint32_t* gs = reinterpret_cast<const uint32_t*>(a.gate_s + brow * (a.H / 32) + b0);
  const uint32_t* us = reinterpret_cast<const uint32_t*>(a.up_s + brow * (a.H / 32) + b0);
  const uint4* xr = reinterpret_cast<const uint4*>(abase + k0) + g;        // 16-byte units
  const uint32_t* xs = reinterpret_cast<const uint32_t*>(ascl + b0);
  v4f accg = {0.0f, 0.0f, 0.0f, 0.0f}, accu = {0.0f, 0.0f, 0.0f, 0.0f};
  if (kactive) {
    // weights (the HBM stream) for every step stay in registers; activations (L2-resident) are loaded
    // PF steps ahead of their MFMA
    constexpr int PF = NS < 4 ? NS : 4;
    uint4 bg[NS], bu[NS], xa[PF], xb[PF];
    uint32_t sgw[NS], suw[NS], saw[PF];
#pragma unroll
    for (int s = 0; s < NS; ++s) { bg[s] = gw[4 * s]; bu[s] = upw[4 * s]; }
#pragma unroll
    for (int s = 0; s < NS; ++s) { sgw[s] = gs[s]; suw[s] = us[s]; }
#pragma unroll
    for (int s = 0; s < PF; ++s) { xa[s] = xr[8 * s]; xb[s] = xr[8 * s + 4]; saw[s] = xs[s]; }
    __builtin_amdgcn_sched_barrier(0);   // every weight load is in flight before the first MFMA
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint4 p = zero_if(xa[s % PF], avalid), q = zero_if(xb[s % PF], avalid);
      const int sa = avalid ? (int)byte_of(saw[s % PF], g) : 127;
      if (s + PF < NS) { xa[s % PF] = xr[8 * (s + PF)]; xb[s % PF] = xr[8 * (s + PF) + 4]; saw[s % PF] = xs[s + PF]; }
      v8i A = {(int)p.x, (int)p.y, (int)p.z, (int)p.w, (int)q.x, (int)q.y, (int)q.z, (int)q.w};
      accg = MFMA_F8xF4(A, b_operand(bg[s]), accg, sa, (int)byte_of(sgw[s], g));
      accu = MFMA_F8xF4(A, b_operand(bu[s]), accu, sa, (int)byte_of(suw[s], g));
    }
  }
  float vg[4], vu[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {   // rows 4g+q (hi, g < 2) plus rows 8+4g+q (lo) of lane l + 32
    vg[q] = accg[q] + __shfl_xor(accg[q], 32, 64);
    vu[q] = accu[q] + __shfl_xor(accu[q], 32, 64);
  }
  __shared__ float red[3][2][2][32][4];   // [K-range 1..3][ntile][gate/up][lane][q]
  __shared__ float hl[8][32];
  if (kr > 0 && lane < 32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) { red[kr - 1][ntile][0][lane][q] = vg[q]; red[kr - 1][ntile][1][lane][q] = vu[q]; }
  }
  __syncthreads();
  if (kr == 0 && lane < 32) {
    const int n = n0 + i;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 4 * g + q;
      float gsum = vg[q], usum = vu[q];
#pragma unroll
      for (int j = 0; j < 3; ++j) { gsum += red[j][ntile][0][lane][q]; usum += red[j][ntile][1][lane][q]; }
      uint16_t gt = f32_to_bf16(gsum);
      float gtf = bf16_to_f32(gt);
      float ut = round_bf16(usum);
      float sig = bf16_to_f32(a.sigtab[gt]);
      float hv = round_bf16(round_bf16(gtf * sig) * ut);
      if (r < cnt) a.h[((size_t)u * a.R + r) * a.I + n] = f32_to_bf16(hv);
      else if (a.zero_pad && r < a.R) a.h[((size_t)u * a.R + r) * a.I + n] = 0;
      hl[r][ntile * 16 + i] = r < cnt ? hv : 0.0f;
    }
  }
  __syncthreads();
  if (wave == 0) {                 // hi/lo E4M3 split of h per (row, 32-block): 8 lanes per row, 4 values each
    const int r = lane >> 3, nl = (lane & 7) * 4;
    float v[4];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[j] = hl[r][nl + j]; amax = fmaxf(amax, fabsf(v[j])); }
    amax = group_max(amax, 8);
    const int X = fp8_block_exp(amax);
    uint32_t hw = 0, lw = 0;
    float res[4], ramax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float dec;
      hw |= e4m3_encode(v[j], X, &dec) << (8 * j);
      res[j] = v[j] - dec;
      ramax = fmaxf(ramax, fabsf(res[j]));
    }
    ramax = group_max(ramax, 8);
    const int Y = fp8_block_exp(ramax);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float dec;
      lw |= e4m3_encode(res[j], Y, &dec) << (8 * j);
    }
    if (r < cnt) {
      const size_t row = (size_t)u * a.R + r;
      *reinterpret_cast<uint32_t*>(a.hq_hi + row * a.I + nb + nl) = hw;
      *reinterpret_cast<uint32_t*>(a.hq_lo + row * a.I + nb + nl) = lw;
      if ((lane & 7) == 0) {
        a.hq_hs[row * (a.I / 32) + blockIdx.x] = (uint8_t)(X + 127);
        a.hq_ls[row * (a.I / 32) + blockIdx.x] = (uint8_t)(Y + 127);
      }
    }
  }
}

// ------------------------------------------------------------------ Kernel B + combine (owner computes)
// Block (1024 threads, 16 waves) owns 16 outputs m (blockIdx.x) for every distinct expert.  Work item
// (u, K-half): wave w takes items w, w + 16, ...; per item its NS = I / 256 weight steps are loaded in one
// batch, the activations a few steps ahead of their MFMA.  The two K-half dot products of each (expert,
// row) land in LDS; the block adds them in a fixed order, applies the router weight (and the bf16 rounding
// of the gather_qmm path when asked, model.py:181), sums each row's k routes in route order
// (kernels.py:198-199) and writes y.  No other block is waited for.
template <int NS>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4))) decode_down_combine_kernel(ExpertsArgs a) {
  extern __shared__ float plds[];     // [2][Umax * R][16] K-half dot products
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int m0 = blockIdx.x * 16;
  const int arow = i & 7;
  const int UR = a.Umax * a.R;
  // the first item's metadata is loaded together with the expert count (one round trip)
  int nxt_cnt = a.ucnt[min(wave >> 1, a.Umax - 1)], nxt_slot = a.uslot[min(wave >> 1, a.Umax - 1)];
  const int U = a.n_unique ? min(*a.n_unique, a.Umax) : a.Umax;
  for (int item = wave; item < 2 * U; item += 16) {
    const int u = item >> 1, kh = item & 1;
    const int cnt = min(nxt_cnt, a.R);
    const int slot = nxt_slot;
    if (item + 16 < 2 * U) { nxt_cnt = a.ucnt[(item + 16) >> 1]; nxt_slot = a.uslot[(item + 16) >> 1]; }
    const bool active = cnt > 0 && slot >= 0 && slot < a.S;
    const bool avalid = active && arow < cnt;
    const size_t hrow = (size_t)u * a.R + (avalid ? arow : 0);
    const int b0 = kh * NS * 4;      // first 32-block of this K-half
    const uint4* xr = reinterpret_cast<const uint4*>((i < 8 ? a.hq_hi : a.hq_lo) + hrow * a.I + b0 * 32) + g;
    const uint32_t* xs = reinterpret_cast<const uint32_t*>((i < 8 ? a.hq_hs : a.hq_ls) + hrow * (a.I / 32) + b0);
    const size_t brow = (size_t)(active ? slot : 0) * a.H + m0 + i;
    const uint4* dw = reinterpret_cast<const uint4*>(a.down_w + brow * (a.I / 8)) + b0 + g;
    const uint32_t* dsw = reinterpret_cast<const uint32_t*>(a.down_s + brow * (a.I / 32) + b0);
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    {
      constexpr int PF = NS < 4 ? NS : 4;
      uint4 bw[NS], xa[PF], xb[PF];
      uint32_t sbw[NS], saw[PF];
#pragma unroll
      for (int s = 0; s < NS; ++s) bw[s] = dw[4 * s];
#pragma unroll
      for (int s = 0; s < NS; ++s) sbw[s] = dsw[s];
#pragma unroll
      for (int s = 0; s < PF; ++s) { xa[s] = xr[8 * s]; xb[s] = xr[8 * s + 4]; saw[s] = xs[s]; }
      __builtin_amdgcn_sched_barrier(0);   // every weight load is in flight before the first MFMA
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint4 p = zero_if(xa[s % PF], avalid), q = zero_if(xb[s % PF], avalid);
        const int sa = avalid ? (int)byte_of(saw[s % PF], g) : 127;
        if (s + PF < NS) { xa[s % PF] = xr[8 * (s + PF)]; xb[s % PF] = xr[8 * (s + PF) + 4]; saw[s % PF] = xs[s + PF]; }
        v8i A = {(int)p.x, (int)p.y, (int)p.z, (int)p.w, (int)q.x, (int)q.y, (int)q.z, (int)q.w};
        acc = MFMA_F8xF4(A, b_operand(bw[s]), acc, sa, (int)byte_of(sbw[s], g));
      }
    }
    float dq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) dq[q] = acc[q] + __shfl_xor(acc[q], 32, 64);   // hi rows + lo rows
    if (lane < 32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 4 * g + q;
        if (r < a.R) plds[(kh * UR + u * a.R + r) * 16 + i] = (active && r < cnt) ? dq[q] : 0.0f;
      }
    }
  }
  __syncthreads();
  if (a.zero_pad) {          // copy of the partials (kernels.py:120) for callers that asked for them
    for (int e = tid; e < U * a.R * 16; e += blockDim.x) {
      const int row = e >> 4, mi = e & 15;
      float d = plds[row * 16 + mi] + plds[(UR + row) * 16 + mi];
      if (a.round_bf16) d = round_bf16(d);
      a.part[(size_t)row * a.H + m0 + mi] = d * a.uw[row];
    }
  }
  const uint32_t nrows = (uint32_t)(U * a.R);
  for (int e = tid; e < a.M * 16; e += blockDim.x) {
    const int row = e >> 4, mi = e & 15;
    float accy = 0.0f;
    for (int j = 0; j < a.k; ++j) {
      const uint32_t idx = a.gidx[row * a.k + j];
      if (idx < nrows) {
        float d = plds[idx * 16 + mi] + plds[(UR + idx) * 16 + mi];
        if (a.round_bf16) d = round_bf16(d);
        accy = accy + d * a.uw[idx];
      }
    }
    a.y[(size_t)row * a.H + m0 + mi] = f32_to_bf16(accy);
  }
}

// ------------------------------------------------------------------ host
struct ExpertsWs {
  uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;
  uint16_t* h;
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;
  float* part;
};
static ExpertsWs carve_experts(Carve& c, int M, int Umax, int R, int H, int I) {
  ExpertsWs w;
  w.xq_hi = c.take<uint8_t>((size_t)M * H);
  w.xq_lo = c.take<uint8_t>((size_t)M * H);
  w.xq_hs = c.take<uint8_t>((size_t)M * H / 32);
  w.xq_ls = c.take<uint8_t>((size_t)M * H / 32);
  w.h = c.take<uint16_t>((size_t)Umax * R * I);
  w.hq_hi = c.take<uint8_t>((size_t)Umax * R * I);
  w.hq_lo = c.take<uint8_t>((size_t)Umax * R * I);
  w.hq_hs = c.take<uint8_t>((size_t)Umax * R * I / 32);
  w.hq_ls = c.take<uint8_t>((size_t)Umax * R * I / 32);
  w.part = c.take<float>((size_t)Umax * R * H);
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
                 reinterpret_cast<uintptr_t>(b->down_s)) & 3) == 0,
               MIMO_ERR_ALIGN, "bank: scale pools must be 4-byte aligned");
  MIMO_REQUIRE(aligned16(b->gate_w) && aligned16(b->up_w) && aligned16(b->down_w), MIMO_ERR_ALIGN,
               "bank: weight pools must be 16-byte aligned");
  return MIMO_OK;
}

static int run_experts(const ExpertsArgs& base, int M, int round_bf16, hipStream_t st) {
  ExpertsArgs a = base;
  a.round_bf16 = round_bf16;
  dim3 g1(a.I / 32, a.Umax);
  const int ns = gateup_steps(a.H);    // MFMA steps per wave
  if (a.scores && a.Umax > 16) {
    int rc = launch_select_group(a.scores, a.keys, a.M, a.E, a.k, a.slot_of, a.R, a.S, a.Umax, a.inds_out, a.w_out,
                                 a.rt_uids, a.rt_urows, a.rt_ucnt, a.rt_uw, a.rt_gidx, a.rt_nu, a.rt_status, st);
    if (rc) return rc;
  }
  {
    ProfScope p(st, "decode_gateup");
    if (a.scores && a.Umax <= 16) {   // small batches: every block selects (cheaper than a launch)
      switch (ns) {
        case 8: decode_gateup_kernel<8, true><<<g1, 512, 0, st>>>(a); break;
        case 4: decode_gateup_kernel<4, true><<<g1, 512, 0, st>>>(a); break;
        case 2: decode_gateup_kernel<2, true><<<g1, 512, 0, st>>>(a); break;
        default: decode_gateup_kernel<1, true><<<g1, 512, 0, st>>>(a); break;
      }
    } else {
      switch (ns) {
        case 8: decode_gateup_kernel<8, false><<<g1, 512, 0, st>>>(a); break;
        case 4: decode_gateup_kernel<4, false><<<g1, 512, 0, st>>>(a); break;
        case 2: decode_gateup_kernel<2, false><<<g1, 512, 0, st>>>(a); break;
        default: decode_gateup_kernel<1, false><<<g1, 512, 0, st>>>(a); break;
      }
    }
  }
  const size_t lds = 2 * (size_t)a.Umax * a.R * 16 * sizeof(float);
  {
    ProfScope p(st, "decode_down_combine");
    switch (a.I / 256) {
      case 8: decode_down_combine_kernel<8><<<a.H / 16, 1024, lds, st>>>(a); break;
      case 4: decode_down_combine_kernel<4><<<a.H / 16, 1024, lds, st>>>(a); break;
      default: decode_down_combine_kernel<2><<<a.H / 16, 1024, lds, st>>>(a); break;
    }
  }
  return check_launch("moe experts");
}

}  // namespace mimo

using namespace mimo;

extern "C" {

size_t mimo_moe_experts_workspace_size(int M, int Umax, int R, int H, int I) {
  Carve c(nullptr, 0);
  carve_experts(c, M, Umax, R, H, I);
  return c.off;
}

int mimo_moe_experts(const uint16_t* x, int M, const mimo_bank* bank, const int32_t* uslot, const int32_t* urows,
                     const int32_t* ucnt, const float* uw, const int32_t* n_unique, int Umax, int R,
                     const uint32_t* gidx, int k, int round_expert_bf16, uint16_t* y, uint16_t* h_out,
                     float* part_out, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_bank(bank);
  if (rc) return rc;
  MIMO_REQUIRE(x && uslot && urows && ucnt && uw && gidx && y, MIMO_ERR_ARG, "moe_experts: null pointer");
  MIMO_REQUIRE(M >= 1 && M <= 8 && R >= 1 && R <= 8 && k >= 1 && Umax >= 1 && Umax <= M * k && Umax * R <= 1024,
               MIMO_ERR_SHAPE, "moe_experts: need 1 <= M <= 8, 1 <= R <= 8, 1 <= Umax <= M*k, Umax*R <= 1024");
  MIMO_REQUIRE(aligned16(x) && aligned16(y) && (!part_out || aligned16(part_out)), MIMO_ERR_ALIGN,
               "moe_experts: x, y, part_out must be 16-byte aligned");
  const int H = bank->hidden, I = bank->inter;
  Carve c(ws, ws_bytes);
  ExpertsWs w = carve_experts(c, M, Umax, R, H, I);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_experts: workspace too small (need %zu)", c.off);
  int err;
  const uint16_t* sig = sigtab_device(&err);
  if (!sig) return err;
  hipStream_t st = as_stream(stream);
  rc = launch_quantize_fp8_hilo(x, M, H, w.xq_hi, w.xq_hs, w.xq_lo, w.xq_ls, st);
  if (rc) return rc;
  ExpertsArgs a{};
  a.xq_hi = w.xq_hi; a.xq_lo = w.xq_lo; a.xq_hs = w.xq_hs; a.xq_ls = w.xq_ls;
  a.gate_w = bank->gate_w; a.up_w = bank->up_w; a.down_w = bank->down_w;
  a.gate_s = bank->gate_s; a.up_s = bank->up_s; a.down_s = bank->down_s;
  a.H = H; a.I = I; a.R = R; a.Umax = Umax; a.k = k; a.M = M; a.S = bank->n_slots;
  a.uslot = uslot; a.urows = urows; a.ucnt = ucnt; a.n_unique = n_unique; a.uw = uw; a.gidx = gidx;
  a.sigtab = sig;
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
  int Umax = M * k < E ? M * k : E;
  float *l, *s, *kk, *w, *uw;
  int32_t *inds, *uids, *urows, *ucnt, *nu, *st;
  uint32_t* gidx;
  carve_decode(c, M, E, k, Umax, kDecodeR, &l, &s, &kk, &inds, &w, &uids, &urows, &ucnt, &uw, &gidx, &nu, &st);
  carve_experts(c, M, Umax, kDecodeR, H, I);
  return c.off;
}

int mimo_moe_decode(const uint16_t* x, int M, const uint16_t* Wg, const float* bias, const int32_t* slot_of, int E,
                    int k, const mimo_bank* bank, uint16_t* y, int32_t* inds_out, float* w_out, void* ws,
                    size_t ws_bytes, void* stream) {
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
  ExpertsWs ew = carve_experts(c, M, Umax, kDecodeR, H, I);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_decode: workspace too small (need %zu)", c.off);
  int err;
  const uint16_t* sig = sigtab_device(&err);
  if (!sig) return err;
  hipStream_t st = as_stream(stream);

  RouterSmallArgs ra{};
  ra.x = x; ra.Wg = Wg; ra.bias = bias; ra.T = M; ra.H = H; ra.E = E; ra.k = k; ra.nlog = (E + 3) / 4;
  ra.logits = logits; ra.scores = scores; ra.keys = keys;
  ra.xq_hi = ew.xq_hi; ra.xq_lo = ew.xq_lo; ra.xq_hs = ew.xq_hs; ra.xq_ls = ew.xq_ls;
  rc = launch_router_logits_small(ra, st);
  if (rc) return rc;

  ExpertsArgs a{};
  a.xq_hi = ew.xq_hi; a.xq_lo = ew.xq_lo; a.xq_hs = ew.xq_hs; a.xq_ls = ew.xq_ls;
  a.gate_w = bank->gate_w; a.up_w = bank->up_w; a.down_w = bank->down_w;
  a.gate_s = bank->gate_s; a.up_s = bank->up_s; a.down_s = bank->down_s;
  a.H = H; a.I = I; a.R = kDecodeR; a.Umax = Umax; a.k = k; a.M = M; a.S = S;
  a.uslot = uids; a.urows = urows; a.ucnt = ucnt; a.n_unique = nu; a.uw = uw; a.gidx = gidx;
  a.sigtab = sig;
  a.h = ew.h; a.hq_hi = ew.hq_hi; a.hq_lo = ew.hq_lo; a.hq_hs = ew.hq_hs; a.hq_ls = ew.hq_ls;
  a.part = ew.part; a.zero_pad = 0; a.y = y;
  a.scores = scores; a.keys = keys; a.E = E; a.slot_of = slot_of;
  a.inds_out = inds_out ? inds_out : inds;
  a.w_out = w_out ? w_out : w;
  a.rt_uids = uids; a.rt_urows = urows; a.rt_ucnt = ucnt; a.rt_uw = uw; a.rt_gidx = gidx; a.rt_nu = nu;
  a.rt_status = status;
  // M == 1 follows _gather_m1 (bf16 expert outputs, model.py:173-182); M >= 2 the distinct-expert kernels
  return run_experts(a, M, M == 1 ? 1 : 0, st);
}

}  // extern "C"
