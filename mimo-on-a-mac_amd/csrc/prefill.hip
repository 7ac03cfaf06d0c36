// Prefill MoE: (token, k) routes sorted by slot, grouped gate/up + SwiGLU and down GEMMs on block-scaled
// MFMA, bf16 expert outputs, fixed-order weighted combine back to token order.
//
// Reference: _moe_prefill engine/mimo_stream/model.py:230-271 and _pair_outputs :221-228 (three sorted
// gather_qmm calls, bf16 SwiGLU intermediate, bf16 expert outputs, inverse permutation, (Y.f32 * w).sum(1)).
//
// Tiling: a row tile is up to 64 consecutive sorted routes of one slot (the dispatch writes the tile table).
// A block (8 waves) owns one row tile and 128 gate + 128 up outputs (gate/up) or 256 outputs (down).  The K
// loop runs in steps of 128 through a 4-stage LDS ring filled by global_load_lds: per step 16 KB of
// activation codes (hi and lo E4M3 planes of the 64 routes), 16 KB of E2M1 weights (256 rows x 64 B) and the
// E8M0 scales; three steps are in flight while the fourth is multiplied.  Wave w takes route half w & 1 (four
// 8-route chunks) and output group w >> 1 (four 16-output weight tiles): 16 MFMAs per step, chunks past the
// tile's routes skipped.  Same operand layout as the decode kernels: the hi and lo halves of 8 routes fill
// rows 0-7 and 8-15 of one MFMA.
#include "device.h"
#include "host.h"
#include "router.h"

namespace mimo {

struct PrefillArgs {
  const uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;   // [T, H], [T, H/32]
  const int32_t *perm, *offsets, *tile_off, *inv;
  const int4* tiles;                              // (slot, first route, end route, 0) per row tile
  const float* w;
  int T, k, S, H, I, P;
  const uint32_t *gate_w, *up_w, *down_w;
  const uint8_t *gate_s, *up_s, *down_s;
  const uint16_t* sigtab;
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;         // [P, I], [P, I/32] in sorted route order
  uint16_t* Y;                                    // [P, H] bf16 expert outputs, sorted route order
  uint16_t* y;                                    // [T, H]
};

constexpr int PF_ROWS = 64;        // routes per row tile
constexpr int PF_STAGES = 4;
// Per-stage LDS layout (bytes).  A: two planes (hi, lo) of 64 routes x 128 codes, the 16-byte chunk q of route
// r stored at slot q ^ (r & 7); the lo plane starts 128 bytes off the hi plane's bank phase.  B: 256 weight
// rows x 64 bytes, chunk g of row r at slot (g + (r & 15) / 4) & 3.  Both layouts make the MFMA operand
// reads conflict-free.
constexpr int PF_A_LO = 8192 + 128;
constexpr int PF_B = 16640;
constexpr int PF_AS = PF_B + 16384;       // [2 planes][64 routes] scale words (4 K-blocks)
constexpr int PF_BS = PF_AS + 512;        // [256 rows] scale words
constexpr int PF_DUMMY = PF_BS + 1024;    // target of the copies that keep every wave's count equal
constexpr int PF_STAGE = PF_DUMMY + 256;  // 34816
constexpr int PF_LDS = PF_STAGES * PF_STAGE;
constexpr int PF_COPIES = 5;              // global -> LDS copies per wave and stage

__device__ __forceinline__ void wait_vm_le(int n) {   // s_waitcnt vmcnt(n), n in {0, 5, 10}
  if (n >= 10) __builtin_amdgcn_s_waitcnt(0x0F7A);
  else if (n >= 5) __builtin_amdgcn_s_waitcnt(0x0F75);
  else __builtin_amdgcn_s_waitcnt(0x0F70);
}
#define PF_MFMA(A, B, C, SA, SB) __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4((A), (B), (C), 0, 4, 0, (SA), 0, (SB))
__device__ __forceinline__ uint32_t pf_byte(uint32_t w, int g) { return (w >> (8 * g)) & 0xFFu; }

// GATEUP: A = the routes' token activations, B = gate rows 0-127 and up rows 128-255 of the block's outputs;
// epilogue SwiGLU and the hi/lo split of h.  !GATEUP: A = the routes' h rows, B = down rows of 256 outputs;
// epilogue bf16 expert outputs.
template <bool GATEUP>
__global__ void __launch_bounds__(512) prefill_gemm_kernel(PrefillArgs a) {
  extern __shared__ __align__(256) uint8_t pl[];
  __shared__ int s_tok[PF_ROWS];
  // XCD-aware order: workgroups go to the 8 XCDs round robin, so hardware block b runs on XCD b % 8.  XCD x
  // takes the contiguous range [x * per, (x + 1) * per) of the used (tile, output block) pairs, output blocks
  // fastest: a tile's activation rows and an expert's weights are then re-read from that XCD's L2.
  const int ntiles = a.tile_off[a.S];
  const int nblk = GATEUP ? a.I / 128 : a.H / 256;   // output blocks per tile
  const int used = ntiles * nblk;
  const int per = (used + 7) / 8;                    // the 1-D grid has at least 8 * per blocks
  const int hw = blockIdx.x;
  const int xcd = hw & 7, j = hw >> 3;
  const int logical = xcd * per + j;
  if (j >= per || logical >= used) return;
  const int tile = logical / nblk;
  const int4 tt = a.tiles[tile];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = __builtin_amdgcn_readfirstlane(tt.x);
  const int beg = __builtin_amdgcn_readfirstlane(tt.y);
  const int nvalid = __builtin_amdgcn_readfirstlane(tt.z) - beg;
  const int K = GATEUP ? a.H : a.I;             // reduction length
  const int nK = K / 128;
  const int ncol = GATEUP ? a.I : a.H;          // weight rows per slot
  const int n0 = (logical - tile * nblk) * (GATEUP ? 128 : 256);
  // activation row of each route (padding routes repeat the tile's first route)
  if (tid < PF_ROWS) {
    const int p = beg + min(tid, nvalid - 1);
    s_tok[tid] = GATEUP ? a.perm[p] / a.k : p;
  }
  __syncthreads();
  const bool a_pad = 8 * wave + (lane >> 3) >= nvalid;   // this lane copies a padding route
  const uint8_t* a_hi = GATEUP ? a.xq_hi : a.hq_hi;
  const uint8_t* a_lo = GATEUP ? a.xq_lo : a.hq_lo;
  const uint8_t* a_hs = GATEUP ? a.xq_hs : a.hq_hs;
  const uint8_t* a_ls = GATEUP ? a.xq_ls : a.hq_ls;
  // this wave's copies: A planes (routes 8w .. 8w+7), B rows 32w .. 32w+31, one scale or dummy row of 64 words
  const int ar = 8 * wave + (lane >> 3);
  // padding lanes all read the same 16 bytes (their rows are never used)
  const uint32_t a_off = a_pad ? (uint32_t)s_tok[0] * (uint32_t)K
                               : (uint32_t)s_tok[ar] * (uint32_t)K + 16u * (uint32_t)((lane & 7) ^ (lane >> 3));
  const bool up_half = GATEUP && wave >= 4;     // B rows 128-255 are the up projection
  const uint32_t* bw = GATEUP ? (up_half ? a.up_w : a.gate_w) : a.down_w;
  const uint8_t* bw_base = reinterpret_cast<const uint8_t*>(bw) + ((size_t)slot * ncol + n0) * (K / 2);
  const int brow0 = 32 * wave - (up_half ? 128 : 0);   // first weight row of the wave's copies in its projection
  const uint32_t b_off0 = (uint32_t)(brow0 + (lane >> 2)) * (uint32_t)(K / 2) + 16u * (uint32_t)(((lane & 3) - (lane >> 4)) & 3);
  const uint32_t b_off1 = b_off0 + 16u * (uint32_t)(K / 2);
  // scale copies: wave 0 A hi, wave 1 A lo, waves 2-5 B rows 64 (w - 2) .. + 63, waves 6-7 a dummy repeat of wave 0's
  const uint8_t* sc_base;
  uint32_t sc_off;
  int sc_dst;
  if (wave < 2 || wave >= 6) {
    sc_base = (wave == 1) ? a_ls : a_hs;
    sc_off = (uint32_t)s_tok[lane < nvalid ? lane : 0] * (uint32_t)(K / 32);
    sc_dst = wave == 0 ? PF_AS : (wave == 1 ? PF_AS + 256 : PF_DUMMY);
  } else {
    const int r = 64 * (wave - 2) + lane;          // B row of the block, 0..255
    const bool up_r = GATEUP && r >= 128;
    const uint8_t* s_pool = GATEUP ? (up_r ? a.up_s : a.gate_s) : a.down_s;
    sc_base = s_pool + ((size_t)slot * ncol + n0) * (K / 32);
    sc_off = (uint32_t)(r - (up_r ? 128 : 0)) * (uint32_t)(K / 32);
    sc_dst = PF_BS + 256 * (wave - 2);
  }
  auto issue = [&](int s) {                        // the five copies of K-step s into ring slot s % 4
    uint8_t* st = pl + (s & 3) * PF_STAGE;
    const uint32_t k0 = (uint32_t)s * 128u;
    lds_copy16(a_hi, a_off + k0, st + 1024 * wave);
    lds_copy16(a_lo, a_off + k0, st + PF_A_LO + 1024 * wave);
    lds_copy16(bw_base, b_off0 + k0 / 2, st + PF_B + 2048 * wave);
    lds_copy16(bw_base, b_off1 + k0 / 2, st + PF_B + 2048 * wave + 1024);
    lds_copy4(sc_base, sc_off + k0 / 32, st + sc_dst);
  };
  const int rh = wave & 1, ng = wave >> 1;
  v4f acc[4][4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[c][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // weight tile t of this wave: GATEUP t = 2 p + b (p gate/up, b 16-output half), else t = 16-output quarter
  int brow[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) brow[t] = GATEUP ? (t >> 1) * 128 + 32 * ng + 16 * (t & 1) + i : 64 * ng + 16 * t + i;
  const int bslot = 16 * ((g + (i >> 2)) & 3);
  int nch = 0;                                     // active 8-route chunks of this wave
#pragma unroll
  for (int c = 0; c < 4; ++c) nch += (8 * (4 * rh + c) < nvalid) ? 1 : 0;

  for (int s = 0; s < PF_STAGES - 1 && s < nK; ++s) issue(s);
  for (int s = 0; s < nK; ++s) {
    wait_vm_le(PF_COPIES * min(PF_STAGES - 2, nK - 1 - s));
    __syncthreads();                               // step s landed everywhere; step s - 1 is no longer read
    if (s + PF_STAGES - 1 < nK) issue(s + PF_STAGES - 1);
    const uint8_t* st = pl + (s & 3) * PF_STAGE;
    v8i B[4];
    int sb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint4 v = *reinterpret_cast<const uint4*>(st + PF_B + brow[t] * 64 + bslot);
      B[t] = v8i{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
      sb[t] = (int)pf_byte(*reinterpret_cast<const uint32_t*>(st + PF_BS + 4 * brow[t]), g);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c < nch) {
        const int r = 8 * (4 * rh + c) + (i & 7);
        const uint8_t* ab = st + (i < 8 ? 0 : PF_A_LO) + 128 * r;
        const uint4 lo16 = *reinterpret_cast<const uint4*>(ab + 16 * (g ^ (i & 7)));
        const uint4 hi16 = *reinterpret_cast<const uint4*>(ab + 16 * ((4 + g) ^ (i & 7)));
        const int sa = (int)pf_byte(*reinterpret_cast<const uint32_t*>(st + PF_AS + (i < 8 ? 0 : 256) + 4 * r), g);
        const v8i A = {(int)lo16.x, (int)lo16.y, (int)lo16.z, (int)lo16.w, (int)hi16.x, (int)hi16.y, (int)hi16.z, (int)hi16.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[c][t] = PF_MFMA(A, B[t], acc[c][t], sa, sb[t]);
      }
    }
  }

  // epilogue: lanes < 32 hold routes 8 chunk + 4 g + q (hi + lo rows summed) at output column i of each tile
  if constexpr (GATEUP) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= nch) continue;
      const int chunk = 4 * rh + c;
      float gv[2][4], uv[2][4];
      uint16_t gt[2][4];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          gv[b][q] = acc[c][b][q] + __shfl_xor(acc[c][b][q], 32, 64);
          uv[b][q] = acc[c][2 + b][q] + __shfl_xor(acc[c][2 + b][q], 32, 64);
          gt[b][q] = f32_to_bf16(gv[b][q]);
        }
      float sg[2][4];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) sg[b][q] = bf16_to_f32(a.sigtab[gt[b][q]]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float hv[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const float gtf = bf16_to_f32(gt[b][q]);
          hv[b] = round_bf16(round_bf16(gtf * sg[b][q]) * round_bf16(uv[b][q]));
        }
        // the wave's 32 outputs of this route are one E8M0 block of h: max over b and the 16 lanes of the row
        const float am = dpp_group_max16(fmaxf(fabsf(hv[0]), fabsf(hv[1])));
        const int X = fp8_block_exp(am);
        uint32_t hc[2], lc[2];
        float res[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          float dec;
          hc[b] = e4m3_encode(hv[b], X, &dec);
          res[b] = hv[b] - dec;
        }
        const float ram = dpp_group_max16(fmaxf(fabsf(res[0]), fabsf(res[1])));
        const int Yx = fp8_block_exp(ram);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          float dec;
          lc[b] = e4m3_encode(res[b], Yx, &dec);
        }
        const int r = 8 * chunk + 4 * g + q;
        if (lane < 32 && r < nvalid) {
          const size_t p = (size_t)(beg + r);
          const int n = n0 + 32 * ng;
          a.hq_hi[p * a.I + n + i] = (uint8_t)hc[0];
          a.hq_hi[p * a.I + n + 16 + i] = (uint8_t)hc[1];
          a.hq_lo[p * a.I + n + i] = (uint8_t)lc[0];
          a.hq_lo[p * a.I + n + 16 + i] = (uint8_t)lc[1];
          if (i == 0) {
            a.hq_hs[p * (a.I / 32) + n / 32] = (uint8_t)(X + 127);
            a.hq_ls[p * (a.I / 32) + n / 32] = (uint8_t)(Yx + 127);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c >= nch) continue;
      const int chunk = 4 * rh + c;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float v = acc[c][t][q] + __shfl_xor(acc[c][t][q], 32, 64);
          const int r = 8 * chunk + 4 * g + q;
          if (lane < 32 && r < nvalid) a.Y[(size_t)(beg + r) * a.H + n0 + 64 * ng + 16 * t + i] = f32_to_bf16(v);
        }
    }
  }
}

// ------------------------------------------------------------------ weighted combine in route order
// y[t] = bf16(sum_j fp32(Y[inv[t*k + j]]) * w[t, j]), j ascending (model.py:269-271).
__global__ void __launch_bounds__(256) prefill_combine_kernel(const uint16_t* __restrict__ Y, const int32_t* __restrict__ inv,
                                                              const float* __restrict__ w, int k, int H,
                                                              uint16_t* __restrict__ y) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int m = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (m >= H) return;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int j = 0; j < k; ++j) {
    const int p = inv[t * k + j];
    const float wj = w[t * k + j];
    const uint2 v = *reinterpret_cast<const uint2*>(Y + (size_t)p * H + m);
    float f[4] = {__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16),
                  __uint_as_float(v.y & 0xFFFF0000u)};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float prod = f[q] * wj;
      acc[q] = acc[q] + prod;
    }
  }
  uint2 o;
  o.x = (uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
  o.y = (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
  *reinterpret_cast<uint2*>(y + (size_t)t * H + m) = o;
}

// ------------------------------------------------------------------ host
struct PrefillWs {
  int32_t *hist, *perm, *inv, *offsets, *tile_off, *status, *slot_inds;
  int4* tiles;
  float *logits, *w;
  int32_t* inds;
  uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;
  uint16_t* Y;
};

static PrefillWs carve_prefill(Carve& c, int T, int k, int S, int H, int I, int E) {
  PrefillWs w{};
  const size_t P = (size_t)T * k;
  w.status = c.take<int32_t>(1);
  w.hist = reinterpret_cast<int32_t*>(c.take<char>(dispatch_workspace((int)P, S)));
  w.perm = c.take<int32_t>(P);
  w.inv = c.take<int32_t>(P);
  w.offsets = c.take<int32_t>(S + 1);
  w.tile_off = c.take<int32_t>(S + 1);
  w.tiles = c.take<int4>(P / PF_ROWS + S + 1);      // bound on sum_s ceil(count_s / PF_ROWS), plus one
  if (E > 0) {
    w.logits = c.take<float>((size_t)T * E);
    w.inds = c.take<int32_t>(P);
    w.w = c.take<float>(P);
    w.slot_inds = c.take<int32_t>(P);
  }
  w.xq_hi = c.take<uint8_t>((size_t)T * H);
  w.xq_lo = c.take<uint8_t>((size_t)T * H);
  w.xq_hs = c.take<uint8_t>((size_t)T * H / 32);
  w.xq_ls = c.take<uint8_t>((size_t)T * H / 32);
  w.hq_hi = c.take<uint8_t>(P * I);
  w.hq_lo = c.take<uint8_t>(P * I);
  w.hq_hs = c.take<uint8_t>(P * I / 32);
  w.hq_ls = c.take<uint8_t>(P * I / 32);
  w.Y = c.take<uint16_t>(P * H);
  return w;
}

__global__ void reset_status_kernel(int32_t* status) { status[0] = 0; }

static int run_prefill(const uint16_t* x, int T, const int32_t* slot_inds, const float* wts, int k, const mimo_bank* bank,
                       uint16_t* y, const PrefillWs& ws, hipStream_t st) {
  const int H = bank->hidden, I = bank->inter, S = bank->n_slots;
  const int P = T * k;
  // the GEMM kernels address activation and h rows with 32-bit offsets
  MIMO_REQUIRE((int64_t)T * H < (int64_t)1 << 31 && (int64_t)P * I < (int64_t)1 << 31, MIMO_ERR_SHAPE,
               "moe_prefill: T * hidden and T * k * inter must stay below 2^31");
  int err;
  const uint16_t* sig = sigtab_device(&err);
  if (!sig) return err;
  int rc = launch_dispatch(slot_inds, P, S, ws.hist, ws.perm, ws.offsets, ws.inv, PF_ROWS, ws.tile_off, ws.tiles,
                           ws.status, st);
  if (rc) return rc;
  rc = launch_quantize_fp8_hilo(x, T, H, ws.xq_hi, ws.xq_hs, ws.xq_lo, ws.xq_ls, st);
  if (rc) return rc;
  PrefillArgs a{};
  a.xq_hi = ws.xq_hi; a.xq_lo = ws.xq_lo; a.xq_hs = ws.xq_hs; a.xq_ls = ws.xq_ls;
  a.perm = ws.perm; a.offsets = ws.offsets; a.tile_off = ws.tile_off; a.inv = ws.inv; a.w = wts; a.tiles = ws.tiles;
  a.T = T; a.k = k; a.S = S; a.H = H; a.I = I; a.P = P;
  a.gate_w = bank->gate_w; a.up_w = bank->up_w; a.down_w = bank->down_w;
  a.gate_s = bank->gate_s; a.up_s = bank->up_s; a.down_s = bank->down_s;
  a.sigtab = sig;
  a.hq_hi = ws.hq_hi; a.hq_lo = ws.hq_lo; a.hq_hs = ws.hq_hs; a.hq_ls = ws.hq_ls;
  a.Y = ws.Y; a.y = y;
  const int max_tiles = P / PF_ROWS + S;     // bound on sum_s ceil(count_s / PF_ROWS)
  static int allowed_gu = 0, allowed_dn = 0;
  if (!allowed_gu) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_gemm_kernel<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, PF_LDS);
    if (e != hipSuccess) return set_error(MIMO_ERR_HIP, "prefill LDS attribute: %s", hipGetErrorString(e));
    allowed_gu = 1;
  }
  if (!allowed_dn) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_gemm_kernel<false>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, PF_LDS);
    if (e != hipSuccess) return set_error(MIMO_ERR_HIP, "prefill LDS attribute: %s", hipGetErrorString(e));
    allowed_dn = 1;
  }
  // 1-D grids: 8 x ceil(bound / 8) blocks, so every XCD has an index for each of its (tile, output block)
  // pairs; blocks past the used pairs exit at once
  const int grid_gu = 8 * ((max_tiles * (I / 128) + 7) / 8);
  const int grid_dn = 8 * ((max_tiles * (H / 256) + 7) / 8);
  { ProfScope p(st, "prefill_gateup"); prefill_gemm_kernel<true><<<grid_gu, 512, PF_LDS, st>>>(a); }
  { ProfScope p(st, "prefill_down"); prefill_gemm_kernel<false><<<grid_dn, 512, PF_LDS, st>>>(a); }
  { ProfScope p(st, "prefill_combine");
    prefill_combine_kernel<<<dim3((H + 1023) / 1024, T), 256, 0, st>>>(ws.Y, ws.inv, wts, k, H, y); }
  return check_launch("moe prefill");
}

static int check_prefill_bank(const mimo_bank* b) {
  MIMO_REQUIRE(b && b->gate_w && b->gate_s && b->up_w && b->up_s && b->down_w && b->down_s, MIMO_ERR_ARG,
               "bank: null pointer");
  MIMO_REQUIRE(b->n_slots >= 1 && b->n_slots <= 1024 && b->hidden % 256 == 0 && b->hidden >= 256 &&
                   b->inter % 128 == 0 && b->inter >= 128,
               MIMO_ERR_SHAPE, "prefill bank: need hidden a multiple of 256, inter of 128, n_slots <= 1024");
  MIMO_REQUIRE(((reinterpret_cast<uintptr_t>(b->gate_s) | reinterpret_cast<uintptr_t>(b->up_s) |
                 reinterpret_cast<uintptr_t>(b->down_s)) & 3) == 0,
               MIMO_ERR_ALIGN, "bank: scale pools must be 4-byte aligned");
  MIMO_REQUIRE(aligned16(b->gate_w) && aligned16(b->up_w) && aligned16(b->down_w), MIMO_ERR_ALIGN,
               "bank: weight pools must be 16-byte aligned");
  return MIMO_OK;
}

}  // namespace mimo

using namespace mimo;

extern "C" {

size_t mimo_moe_prefill_workspace_size(int T, int k, int n_slots, int H, int I) {
  Carve c(nullptr, 0);
  carve_prefill(c, T, k, n_slots, H, I, 0);
  return c.off;
}

int mimo_moe_prefill(const uint16_t* x, int T, const int32_t* slot_inds, const float* w, int k, const mimo_bank* bank,
                     uint16_t* y, void* ws, size_t ws_bytes, void* stream) {
  ProfChain chain;   // per-kernel timing (when enabled) back to back within this call
  int rc = check_prefill_bank(bank);
  if (rc) return rc;
  MIMO_REQUIRE(x && slot_inds && w && y, MIMO_ERR_ARG, "moe_prefill: null pointer");
  MIMO_REQUIRE(T >= 1 && k >= 1 && (int64_t)T * k < (1 << 30), MIMO_ERR_SHAPE, "moe_prefill: bad T or k");
  MIMO_REQUIRE(aligned16(x) && aligned16(y), MIMO_ERR_ALIGN, "moe_prefill: 16-byte alignment");
  Carve c(ws, ws_bytes);
  PrefillWs pw = carve_prefill(c, T, k, bank->n_slots, bank->hidden, bank->inter, 0);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_prefill: workspace too small (need %zu)", c.off);
  reset_status_kernel<<<1, 1, 0, as_stream(stream)>>>(pw.status);
  return run_prefill(x, T, slot_inds, w, k, bank, y, pw, as_stream(stream));
}

size_t mimo_moe_prefill_block_workspace_size(int T, int E, int k, int n_slots, int H, int I) {
  Carve c(nullptr, 0);
  carve_prefill(c, T, k, n_slots, H, I, E);
  return c.off;
}

int mimo_moe_prefill_block(const uint16_t* x, int T, const uint16_t* Wg, const float* bias, const int32_t* slot_of,
                           int E, int k, const mimo_bank* bank, uint16_t* y, int32_t* inds_out, float* w_out, void* ws,
                           size_t ws_bytes, void* stream) {
  ProfChain chain;   // per-kernel timing (when enabled) back to back within this call
  int rc = check_prefill_bank(bank);
  if (rc) return rc;
  MIMO_REQUIRE(x && Wg && bias && y, MIMO_ERR_ARG, "moe_prefill_block: null pointer");
  MIMO_REQUIRE(T >= 1 && k >= 1 && k <= 16 && E >= k && E <= 1024 && bank->hidden % 64 == 0, MIMO_ERR_SHAPE,
               "moe_prefill_block: need 1 <= k <= min(16, E), E <= 1024");
  MIMO_REQUIRE(aligned16(x) && aligned16(Wg) && aligned16(y), MIMO_ERR_ALIGN, "moe_prefill_block: alignment");
  Carve c(ws, ws_bytes);
  PrefillWs pw = carve_prefill(c, T, k, bank->n_slots, bank->hidden, bank->inter, E);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_prefill_block: workspace too small (need %zu)", c.off);
  hipStream_t st = as_stream(stream);
  int32_t* inds = inds_out ? inds_out : pw.inds;
  float* wts = w_out ? w_out : pw.w;
  reset_status_kernel<<<1, 1, 0, st>>>(pw.status);
  rc = launch_router_logits(x, Wg, T, bank->hidden, E, pw.logits, st);
  if (rc) return rc;
  rc = launch_router_select(pw.logits, bias, T, E, k, 1.0f, inds, wts, slot_of, pw.slot_inds, bank->n_slots, pw.status,
                            st);
  if (rc) return rc;
  return run_prefill(x, T, pw.slot_inds, wts, k, bank, y, pw, st);
}

}  // extern "C"
