// Prefill MoE: (token, k) routes sorted by slot, grouped gate/up + SwiGLU and down GEMMs on block-scaled
// MFMA, bf16 expert outputs, fixed-order weighted combine back to token order.
//
// Reference: _moe_prefill engine/mimo_stream/model.py:230-271 and _pair_outputs :221-228 (three sorted
// gather_qmm calls, bf16 SwiGLU intermediate, bf16 expert outputs, inverse permutation, (Y.f32 * w).sum(1)).
//
// Tiling: the dispatch cuts each slot's sorted routes into row tiles (narrow: a slot of at most 32 routes;
// wide: up to 64 routes) and writes the tile table.  A block (8 waves) owns one row tile and 256 weight rows
// (gate/up blocks take half of their rows from each projection).  Each GEMM is two launches that run
// concurrently: the narrow tiles (HBM-bound) on a side stream, one workgroup per CU with a 3-slot LDS ring, and
// the wide tiles (MFMA work of popular experts) on the caller's stream, two workgroups per CU with a 2-slot ring,
// so one workgroup's MFMAs run while the other waits at its barrier.  The K loop runs through the ring in steps
// of 256 codes (narrow) or 128 (wide), filled by global_load_lds (activation hi and lo E4M3 planes of the tile's
// routes, the block's E2M1 weight rows; E8M0 scales once per epoch); each wave multiplies 16-route chunks by
// four 16-row weight tiles, the hi and lo planes accumulating into the same tile.  The epilogue stages results in
// LDS and writes 16-byte pieces.
#include <atomic>
#include <memory>
#include <mutex>

#include "device.h"
#include "host.h"
#include "keyed_once.h"
#include "layer.h"
#include "router.h"

namespace mimo {

struct PrefillArgs {
  const uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;   // [T, H], [T, H/32]
  const int32_t *perm, *offsets, *inv;
  const int4* tiles;      // [0] = (wide tiles, narrow tiles); wide at 1 + t, narrow at 1 + wcap + t: (slot, beg, end, 0)
  int wcap;
  const float* w;
  int T, k, S, H, I, P;
  // slots [0, S0) address the bank's pools, slots [S0, S) the staging bank's (pool index 1, slot - S0)
  int S0;
  const uint32_t *gate_w[2], *up_w[2], *down_w[2];
  const uint8_t *gate_s[2], *up_s[2], *down_s[2];
  const uint16_t* sigtab;
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;         // [P, I], [P, I/32] in sorted route order
  uint16_t* Y;                                    // [P, H] bf16 expert outputs, sorted route order
  uint16_t* y;                                    // [T, H]
};

// Row tiles.  The dispatch cuts each slot's sorted routes into tiles of one of two shapes:
//   narrow: a slot with at most 32 routes (2 chunks of 16) is one tile, multiplied by 256 weight rows per block
//           (gate/up: 128 outputs of each projection; down: 256 outputs).  These blocks stream weights at the
//           HBM rate with little MFMA work.  Their K loop moves 256 codes per step, so each weight row is read
//           128 contiguous bytes (one whole cache line) at a time: a copy probe streamed weight rows at 4.9 TB/s
//           in 64-byte pieces and at 6.1 TB/s in 128-byte pieces.  49 KB per step through a 3-slot ring (two
//           steps in flight); 156 KB of LDS, one workgroup per CU.
//   wide:   a larger slot is split into ceil(count / 64) tiles of near-equal whole 16-route chunks (at most 4),
//           multiplied by 256 weight rows per block (128 + 128 outputs, or 256 down outputs).  128 codes (32 KB)
//           per step through a 2-slot ring; 77 KB of LDS, two workgroups per CU.  The tiles of a popular slot
//           share each weight block through L2.
// An MFMA multiplies 16 routes of one activation plane by 16 weight rows over 128 codes (a sub-step); the hi
// and lo planes accumulate into the same tile, so each accumulator lane holds finished sums for 4 routes.
// The E8M0 scales of an epoch of 4 sub-steps (16 bytes per row) are copied at once into one of two epoch
// buffers, one 4-byte word per lane, so scale traffic costs one request per row per epoch.
constexpr int PF_NARROW_MAX = 32;
constexpr int PF_WIDE_ROWS = 64;
constexpr int PF_UNIT = 16;                          // routes per MFMA chunk

// Stage layout (KSUB sub-steps of 128 codes per step): per sub-step, A planes of R routes x 128 codes, the
// 16-byte chunk q of route r at slot q ^ (r & 7), the lo plane 128 bytes off the hi plane's bank phase; then B
// rows of 64 KSUB bytes: with KSUB 1, chunk g of row r at slot (g + (r & 15) / 2) & 3; with KSUB 2, chunk q of row
// r at slot q ^ (r & 7).  These make the MFMA operand reads conflict-free (gfx950 LDS, measured with the
// bank-conflict counter).  Copies per wave and step: KSUB ACOP for A (one per 8-route block of a plane and
// sub-step) and BCOP for B (16 / KSUB weight rows each), up to ECOP of the NCOPY epoch copies per epoch.  A wave
// multiplies 4 weight tiles (64 rows) by NJ 16-route chunks spaced CSTEP apart; TGW waves cover the N rows.
// The ring holds STAGES steps of STAGE bytes, then two epoch buffers of SC_ROWS rows (2R + N used); STG bytes
// per wave stage the outputs after the K loop.
template <bool WIDE> struct PfShape;
template <> struct PfShape<false> {
  static constexpr int R = 32, CB = 4, N = 256, A_PL = 4224, KSUB = 2, B_OFF = 16896;
  static constexpr int ACOP = 1, BCOP = 4, NCOPY = 20, ECOP = 3, NJ = 1, CSTEP = 1, TGW = 4;
  static constexpr int STAGES = 3, STAGE = 49664, EPOCH = 4, SC_ROWS = 320, STG = 6144, BLOCKS_PER_CU = 1;
};
template <> struct PfShape<true> {
  static constexpr int R = 64, CB = 8, N = 256, A_PL = 8320, KSUB = 1, B_OFF = 16640;
  static constexpr int ACOP = 2, BCOP = 2, NCOPY = 24, ECOP = 3, NJ = 2, CSTEP = 2, TGW = 4;
  static constexpr int STAGES = 2, STAGE = 33024, EPOCH = 4, SC_ROWS = 384, STG = 4096, BLOCKS_PER_CU = 2;
};
template <bool W> constexpr int pf_lds_bytes() {
  using Sh = PfShape<W>;
  static_assert(Sh::B_OFF == Sh::KSUB * 2 * Sh::A_PL && Sh::B_OFF + Sh::N * 64 * Sh::KSUB <= Sh::STAGE &&
                    2 * Sh::R + Sh::N <= Sh::SC_ROWS, "stage layout");
  static_assert(Sh::TGW * 64 == Sh::N && 8 * Sh::NJ * 16 == Sh::TGW * Sh::R && Sh::BCOP * 128 == Sh::N * Sh::KSUB,
                "wave roles");
  static_assert(Sh::EPOCH % Sh::KSUB == 0 && Sh::EPOCH / Sh::KSUB >= Sh::STAGES - 1, "epoch buffers reused in time");
  static_assert(Sh::SC_ROWS * 4 * Sh::EPOCH == 256 * Sh::NCOPY && 8 * Sh::ECOP >= Sh::NCOPY, "epoch copies");
  static_assert(8 * Sh::STG <= Sh::STAGES * Sh::STAGE, "output staging inside the ring");
  return Sh::STAGES * Sh::STAGE + 2 * Sh::SC_ROWS * 4 * Sh::EPOCH;
}
static_assert(PfShape<true>::BLOCKS_PER_CU * (pf_lds_bytes<true>() + 4 * PfShape<true>::R) <= 163840 &&
              PfShape<false>::BLOCKS_PER_CU * (pf_lds_bytes<false>() + 4 * PfShape<false>::R) <= 163840,
              "workgroups per CU within 160 KB of LDS");
constexpr int PF_GROUP = 4;                          // wide tiles whose blocks of one output block run together

// s_waitcnt vmcnt(n), n in [0, 15] (wave-uniform); a larger n waits for everything
__device__ __forceinline__ void pf_wait(int n) {
  switch (n) {
#define PF_W(c) case c: __builtin_amdgcn_s_waitcnt(0x0F70 | c); break;
    PF_W(1) PF_W(2) PF_W(3) PF_W(4) PF_W(5) PF_W(6) PF_W(7) PF_W(8) PF_W(9) PF_W(10) PF_W(11) PF_W(12) PF_W(13)
    PF_W(14) PF_W(15)
#undef PF_W
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
}
// Epoch buffer rows: A hi [0, R), A lo [R, 2R), B [2R, 2R + N), 16 bytes each (the words of 4 sub-steps).  Row q
// keeps sub-step k's word at position k ^ pf_swz(q): without it the MFMAs' byte-wide scale reads conflicted
// (0.27 conflicts per LDS access in the wide launches against 0.03 with it, on the bank-conflict counter).
__device__ __forceinline__ int pf_swz(int q) { return (q >> 3) & 3; }
#define PF_MFMA(A, B, C, SA, SB) __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4((A), (B), (C), 0, 4, 0, (SA), 0, (SB))

// One (row tile, output block).  GATEUP: A = the routes' token activations, B = gate rows [0, N/2) and up rows
// [N/2, N) of the block's N/2 outputs; epilogue SwiGLU and the hi/lo split of h.  !GATEUP: A = the routes' h
// rows, B = down rows of N outputs; epilogue bf16 expert outputs.
template <bool GATEUP, bool WIDE>
__device__ __forceinline__ void pf_tile(const PrefillArgs& a, uint8_t* pl, int* s_tok, int slot, int beg, int nvalid,
                                        int ob) {
  using Sh = PfShape<WIDE>;
  constexpr int R = Sh::R, N = Sh::N, NJ = Sh::NJ, EP = Sh::EPOCH;
  constexpr int PF_SC = Sh::STAGES * Sh::STAGE;
  constexpr int SCB = Sh::SC_ROWS * 4 * EP;      // bytes of one epoch buffer
  constexpr int HALF = GATEUP ? N / 2 : N;       // block rows of one projection
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = GATEUP ? a.H : a.I;              // reduction length
  const int nK = K / 128;
  const int KS = K / 32;                         // scale bytes per row
  const int ncol = GATEUP ? a.I : a.H;           // weight rows per slot and projection
  const int n0 = ob * HALF;                      // first output of the block
  // activation row of each route (padding routes repeat the tile's last route)
  if (tid < R) {
    const int p = beg + min(tid, nvalid - 1);
    s_tok[tid] = GATEUP ? a.perm[p] / a.k : p;
  }
  __syncthreads();
  const uint8_t* a_hi = GATEUP ? a.xq_hi : a.hq_hi;
  const uint8_t* a_lo = GATEUP ? a.xq_lo : a.hq_lo;
  const uint8_t* a_hs = GATEUP ? a.xq_hs : a.hq_hs;
  const uint8_t* a_ls = GATEUP ? a.xq_ls : a.hq_ls;
  // A copies: 8-route block b = ACOP wave + c of plane b / NCH; padding lanes all read the same 16 bytes
  // (bases and LDS offsets are chosen here, once: the copy loops below index these arrays with constants only)
  uint32_t a_off[Sh::ACOP];
  const uint8_t* a_src[Sh::ACOP];
  int a_dst[Sh::ACOP];
#pragma unroll
  for (int c = 0; c < Sh::ACOP; ++c) {
    const int b = Sh::ACOP * wave + c;
    const int r = 8 * (b % Sh::CB) + (lane >> 3);
    a_off[c] = r < nvalid ? (uint32_t)s_tok[r] * (uint32_t)K + 16u * (uint32_t)((lane & 7) ^ (r & 7))
                          : (uint32_t)s_tok[0] * (uint32_t)K;
    a_src[c] = b >= Sh::CB ? a_lo : a_hi;
    a_dst[c] = (b >= Sh::CB ? Sh::A_PL : 0) + 1024 * (b % Sh::CB);
  }
  // B copies of 16 / KSUB rows each: KSUB 1, rows brow_c + 16 c + lane / 4, the lane's slot lane & 3 holding
  // chunk (slot - row / 2) & 3; KSUB 2, rows brow_c + 8 c + lane / 8, slot lane & 7 holding chunk slot ^ (row & 7)
  const bool up_half = GATEUP && wave >= 4;
  const int pool = slot >= a.S0;                 // tile-uniform: the bank or the staging bank
  const size_t ps = (size_t)(slot - (pool ? a.S0 : 0));
  const uint32_t* bw = GATEUP ? (up_half ? a.up_w[pool] : a.gate_w[pool]) : a.down_w[pool];
  const uint8_t* bw_base = reinterpret_cast<const uint8_t*>(bw) + (ps * ncol + n0) * (K / 2);
  const int brow_c = (N / 8) * wave;
  constexpr int BRC = 16 / Sh::KSUB;             // weight rows per B copy
  const uint32_t b_off =
      Sh::KSUB == 1 ? (uint32_t)(brow_c - (up_half ? HALF : 0) + (lane >> 2)) * (uint32_t)(K / 2) +
                          16u * (uint32_t)(((lane & 3) - (lane >> 3)) & 3)
                    : (uint32_t)(brow_c - (up_half ? HALF : 0) + (lane >> 3)) * (uint32_t)(K / 2) +
                          16u * (uint32_t)((lane & 7) ^ (lane >> 3));
  // scale copies: copy c covers epoch rows (64 / EP) (ECOP wave + c) .., EP lanes (words) per row
  const uint8_t* bs_base = (GATEUP ? a.gate_s[pool] : a.down_s[pool]) + (ps * ncol + n0) * KS;
  const uint8_t* us_base = a.up_s[pool] + (ps * ncol + n0) * KS;
  // The 16 rows of a copy lie in one region (region bounds are multiples of 16).  Row offsets are computed at
  // each epoch rather than kept: a route row's from its token in s_tok, a weight row's as a wave-uniform part
  // plus the lane's row.
  static_assert(EP == 4 && R % 16 == 0 && HALF % 16 == 0, "16-byte epoch rows, 16-row copies");
  auto issue_epoch = [&](int e) __attribute__((always_inline)) {
    uint8_t* dst = pl + PF_SC + (e & 1) * SCB;
    // the lane's word of row q: sub-step (lane % EP) ^ pf_swz(q) of the epoch; words past the row's end read
    // the row's first word instead (they are never used)
    auto wsw = [&](int q) {
      const uint32_t kk = 4u * EP * (uint32_t)e + 4u * (uint32_t)((lane % EP) ^ pf_swz(q));
      return kk < (uint32_t)KS ? kk : 0u;
    };
#pragma unroll
    for (int c = 0; c < Sh::ECOP; ++c) {
      const int cc = Sh::ECOP * wave + c;        // wave-uniform
      if (cc >= Sh::NCOPY) continue;
      const int q0 = (64 / EP) * cc;
      if (q0 < 2 * R) {
        const int r = (q0 < R ? q0 : q0 - R) + lane / EP;
        lds_copy4(q0 < R ? a_hs : a_ls, (uint32_t)s_tok[r < nvalid ? r : 0] * (uint32_t)KS + wsw(q0 + lane / EP),
                  dst + 256 * cc);
      } else if (q0 < 2 * R + N) {
        const int br0 = q0 - 2 * R;
        const bool up = GATEUP && br0 >= HALF;
        lds_copy4(up ? us_base : bs_base,
                  (uint32_t)(br0 - (up ? HALF : 0) + lane / EP) * (uint32_t)KS + wsw(q0 + lane / EP), dst + 256 * cc);
      } else {
        lds_copy4(bs_base, wsw(0), dst + 256 * cc);   // padding rows of the buffer: never read
      }
    }
  };
  // step s (sub-steps KSUB s ..) into ring slot s % STAGES, with the scales of the epoch it opens
  auto issue = [&](int s) __attribute__((always_inline)) {
    if ((Sh::KSUB * s) % EP == 0) issue_epoch(Sh::KSUB * s / EP);
    uint8_t* st = pl + (s % Sh::STAGES) * Sh::STAGE;
    const uint32_t k0 = (uint32_t)s * (128u * Sh::KSUB);
#pragma unroll
    for (int u = 0; u < Sh::KSUB; ++u)
#pragma unroll
      for (int c = 0; c < Sh::ACOP; ++c)
        lds_copy16(a_src[c], a_off[c] + k0 + 128u * u, st + 2 * Sh::A_PL * u + a_dst[c]);
#pragma unroll
    for (int c = 0; c < Sh::BCOP; ++c)
      lds_copy16(bw_base, b_off + (uint32_t)(BRC * c) * (uint32_t)(K / 2) + k0 / 2u,
                 st + Sh::B_OFF + 64 * Sh::KSUB * (brow_c + BRC * c));
  };

  // the wave's tiles: weight rows 64 tg .. (GATEUP t = 2 p + b: projection p, 16-output half b), chunks
  // cb + CSTEP j (routes 16 chunk ..) for the live j
  const int tg = wave % Sh::TGW;
  const int cb = wave / Sh::TGW;
  uint32_t live = 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) live |= (PF_UNIT * (cb + Sh::CSTEP * j) < nvalid) ? 1u << j : 0u;
  live = __builtin_amdgcn_readfirstlane(live);
  // row of tile t = brow0 + bdt(t), bdt a compile-time constant, so the tiles' LDS addresses share one register
  auto bdt = [](int t) constexpr { return GATEUP ? (t >> 1) * HALF + 16 * (t & 1) : 16 * t; };
  const int brow0 = (GATEUP ? 32 : 64) * tg + i;
  const int bsc0 = 4 * EP * (2 * R + brow0) + g;
  // B operand of sub-step u: chunk 4 u + g of the row (KSUB 2) or chunk g (KSUB 1), at its swizzled slot
  int bslot[Sh::KSUB];
#pragma unroll
  for (int u = 0; u < Sh::KSUB; ++u) bslot[u] = Sh::KSUB == 1 ? 16 * ((g + (i >> 1)) & 3) : 16 * ((4 * u + g) ^ (i & 7));
  // A operand of chunk j, plane p: route row r = 16 chunk + i, chunks g and 4 + g of its 128 codes
  int aoff[NJ], asc[NJ][2];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int r = PF_UNIT * (cb + Sh::CSTEP * j) + i;
    aoff[j] = 128 * r;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      asc[j][p] = 4 * EP * (p * R + r) + g;
    }
  }
  const int sw_lo = 16 * (g ^ (i & 7)), sw_hi = 16 * ((4 + g) ^ (i & 7));
  v4f acc[NJ][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[j][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  constexpr int AHEAD = Sh::STAGES - 1;          // steps in flight while one is multiplied
  const int nS = nK / Sh::KSUB;
  const int n_ecop = __builtin_amdgcn_readfirstlane(max(0, min(Sh::ECOP, Sh::NCOPY - Sh::ECOP * wave)));
  issue(0);
  if (AHEAD == 2 && nS > 1) issue(1);
  for (int s = 0; s < nS; ++s) {
    // copies issued after step s's: AHEAD 2: step s + 1's, with its epoch's scales when it opens one; AHEAD 1: none
    if constexpr (AHEAD == 2)
      pf_wait(s + 1 < nS ? Sh::KSUB * Sh::ACOP + Sh::BCOP + ((Sh::KSUB * (s + 1)) % EP == 0 ? n_ecop : 0) : 0);
    else pf_wait(0);
    __syncthreads();                             // step s landed everywhere; step s - 1's slot is free
    if (s + AHEAD < nS) issue(s + AHEAD);
    const uint8_t* st = pl + (s % Sh::STAGES) * Sh::STAGE;
#pragma unroll
    for (int u = 0; u < Sh::KSUB; ++u) {
      if (!live) break;                          // wave-uniform: no chunk of this wave holds routes
      const int ss = Sh::KSUB * s + u;           // sub-step: 128 codes
      const uint8_t* sc = pl + PF_SC + ((ss / EP) & 1) * SCB;
      const int kw = ss % EP;
      const uint8_t* sa_st = st + 2 * Sh::A_PL * u;
      v8i B[4];
      int sb[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint4 v = *reinterpret_cast<const uint4*>(st + Sh::B_OFF + brow0 * (64 * Sh::KSUB) + bslot[u] +
                                                        bdt(t) * (64 * Sh::KSUB));
        B[t] = v8i{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
        sb[t] = sc[bsc0 + 4 * (kw ^ pf_swz(2 * R + brow0 + bdt(t))) + 4 * EP * bdt(t)];
      }
      v8i A[NJ][2];
      int sa[NJ][2];
#pragma unroll
      for (int j = 0; j < NJ; ++j)               // read unconditionally: fixed LDS counts let each MFMA group
#pragma unroll                                   // wait for its own operands only
        for (int p = 0; p < 2; ++p) {
          const uint8_t* ab = sa_st + p * Sh::A_PL + aoff[j];
          const uint4 lo16 = *reinterpret_cast<const uint4*>(ab + sw_lo);
          const uint4 hi16 = *reinterpret_cast<const uint4*>(ab + sw_hi);
          A[j][p] = v8i{(int)lo16.x, (int)lo16.y, (int)lo16.z, (int)lo16.w, (int)hi16.x, (int)hi16.y, (int)hi16.z, (int)hi16.w};
          sa[j][p] = sc[asc[j][p] + 4 * (kw ^ pf_swz(p * R + PF_UNIT * (cb + Sh::CSTEP * j) + i))];
        }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (live & (1u << j)) {
#pragma unroll
          for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[j][t] = PF_MFMA(A[j][p], B[t], acc[j][t], sa[j][p], sb[t]);
        }
      }
    }
  }

  // epilogue: lane (i, g) holds routes 16 chunk + 4 g + q at output column i of each tile.  Results go through
  // a per-wave LDS staging area (the ring is free once every wave has left the K loop) so that the global
  // stores are 16 bytes per lane.
  mfma_f8f4_settle();
  __syncthreads();
  uint8_t* stg = pl + Sh::STG * wave;
  if constexpr (GATEUP) {
    // staging: [16 NJ routes][hi 32 bytes | lo 32 bytes], then the routes' (hi, lo) scale bytes
    uint8_t* ssc = stg + 64 * PF_UNIT * NJ;
    uint16_t gt[NJ][2][4], sgv[NJ][2][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) gt[j][b][q] = f32_to_bf16(acc[j][b][q]);
#pragma unroll
    for (int j = 0; j < NJ; ++j)                 // every sigmoid lookup in flight before the first use
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) sgv[j][b][q] = a.sigtab[gt[j][b][q]];   // any 16-bit index is in the table
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (!(live & (1u << j))) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float hv[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const float gtf = bf16_to_f32(gt[j][b][q]);
          hv[b] = round_bf16(round_bf16(gtf * bf16_to_f32(sgv[j][b][q])) * round_bf16(acc[j][2 + b][q]));
        }
        // the wave's 32 outputs of this route are one E8M0 block of h: max over b and the 16 lanes of the row
        const float am = dpp_group_max16(fmaxf(fabsf(hv[0]), fabsf(hv[1])));
        const int X = fp8_block_exp(am);
        // hi = E4M3 of hv / 2^X, lo = E4M3 of the exact residual / 2^Yx (scalings by powers of two are exact)
        const uint32_t hc = e4m3_pack2(hv[0] * exp2i(-X), hv[1] * exp2i(-X));
        const v2f hd = e4m3_unpack2(hc);
        const float res[2] = {__builtin_fmaf(-hd.x, exp2i(X), hv[0]), __builtin_fmaf(-hd.y, exp2i(X), hv[1])};
        const float ram = dpp_group_max16(fmaxf(fabsf(res[0]), fabsf(res[1])));
        const int Yx = fp8_block_exp(ram);
        const uint32_t lc = e4m3_pack2(res[0] * exp2i(-Yx), res[1] * exp2i(-Yx));
        const int rl = PF_UNIT * j + 4 * g + q;  // route of the wave's staging
        uint8_t* row = stg + 64 * rl;
        row[i] = (uint8_t)hc;
        row[16 + i] = (uint8_t)(hc >> 8);
        row[32 + i] = (uint8_t)lc;
        row[48 + i] = (uint8_t)(lc >> 8);
        if (i == 0) {
          ssc[2 * rl] = (uint8_t)(X + 127);
          ssc[2 * rl + 1] = (uint8_t)(Yx + 127);
        }
      }
    }
    const int n = n0 + 32 * tg;                  // the wave's 32 outputs
#pragma unroll
    for (int k = 0; k < NJ; ++k) {               // 16 routes x 4 pieces of 16 bytes per pass
      const int rl = PF_UNIT * k + (lane >> 2), part = lane & 3;
      const int r = PF_UNIT * (cb + Sh::CSTEP * k) + (lane >> 2);
      if ((live & (1u << k)) && r < nvalid) {
        const uint4 v = *reinterpret_cast<const uint4*>(stg + 64 * rl + 16 * part);
        uint8_t* dst = (part >> 1) ? a.hq_lo : a.hq_hi;
        *reinterpret_cast<uint4*>(dst + (size_t)(beg + r) * a.I + n + 16 * (part & 1)) = v;
        if (part == 0) {
          a.hq_hs[(size_t)(beg + r) * (a.I / 32) + n / 32] = ssc[2 * rl];
          a.hq_ls[(size_t)(beg + r) * (a.I / 32) + n / 32] = ssc[2 * rl + 1];
        }
      }
    }
  } else {
    // staging: [16 NJ routes][64 outputs] bf16
    uint16_t* stg16 = reinterpret_cast<uint16_t*>(stg);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (!(live & (1u << j))) continue;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) stg16[64 * (PF_UNIT * j + 4 * g + q) + 16 * t + i] = f32_to_bf16(acc[j][t][q]);
    }
#pragma unroll
    for (int k = 0; k < 2 * NJ; ++k) {           // 8 routes x 8 pieces of 16 bytes per pass
      const int rl = 8 * k + (lane >> 3), part = lane & 7;
      const int j = rl >> 4;
      const int r = PF_UNIT * (cb + Sh::CSTEP * j) + (rl & 15);
      if ((live & (1u << j)) && r < nvalid) {
        const uint4 v = *reinterpret_cast<const uint4*>(stg + 128 * rl + 16 * part);
        *reinterpret_cast<uint4*>(a.Y + (size_t)(beg + r) * a.H + n0 + 64 * tg + 8 * part) = v;
      }
    }
  }
}

// One launch per tile shape.  Workgroups go to the 8 XCDs round robin (hardware block b runs on XCD b % 8); XCD x
// takes the x-th eighth of the shape's (tile, output block) list.  The 1-D grid has 8 ceil(bound / 8) blocks;
// those past the used pairs exit at once.
// (The second launch bound is the minimum number of waves per SIMD: 8 waves per block x BLOCKS_PER_CU over 4 SIMDs,
// so the wide kernel must fit two blocks' waves in the register file: at most 128 VGPRs.)
template <bool GATEUP, bool WIDE>
__global__ void __launch_bounds__(512, 2 * PfShape<WIDE>::BLOCKS_PER_CU) prefill_gemm_kernel(PrefillArgs a) {
  using Sh = PfShape<WIDE>;
  extern __shared__ __align__(256) uint8_t pl[];
  __shared__ int s_tok[Sh::R];
  const int4 hdr = a.tiles[0];                   // (wide tiles, narrow tiles)
  const int nt = __builtin_amdgcn_readfirstlane(WIDE ? hdr.x : hdr.y);
  const int obn = GATEUP ? a.I / (Sh::N / 2) : a.H / Sh::N;   // output blocks per tile
  const int used = nt * obn, per = (used + 7) / 8;
  const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
  if (j >= max(0, min(per, used - x * per))) return;
  const int l = x * per + j;
  int tile, ob;
  if constexpr (WIDE) {
    // groups of PF_GROUP consecutive tiles (a popular slot's tiles are consecutive), output block, then tile, so
    // the blocks that run together on an XCD share each weight block between PF_GROUP tiles and each tile's
    // activations between the group's output blocks; the last group may hold fewer tiles
    const int grp = l / (PF_GROUP * obn), rem = l - grp * PF_GROUP * obn;
    const int ng = min(PF_GROUP, nt - grp * PF_GROUP);
    ob = rem / ng;
    tile = grp * PF_GROUP + (rem - ob * ng);
  } else {
    tile = l / obn;                              // output blocks fastest
    ob = l - tile * obn;
  }
  const int4 tt = a.tiles[1 + (WIDE ? 0 : a.wcap) + tile];
  pf_tile<GATEUP, WIDE>(a, pl, s_tok, __builtin_amdgcn_readfirstlane(tt.x), __builtin_amdgcn_readfirstlane(tt.y),
                        __builtin_amdgcn_readfirstlane(tt.z - tt.y), ob);
}

// ------------------------------------------------------------------ weighted combine in route order
// y[t] = bf16(sum_j fp32(Y[inv[t*k + j]]) * w[t, j]), j ascending (model.py:269-271).  A thread owns 8 outputs
// (16-byte loads); all k route rows are requested before the sum.
__global__ void __launch_bounds__(256) prefill_combine_kernel(const uint16_t* __restrict__ Y, const int32_t* __restrict__ inv,
                                                              const float* __restrict__ w, int k, int H,
                                                              const uint16_t* resid, uint16_t* y) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int m = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (m >= H) return;
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int KB = 8;                          // routes whose rows are in flight at once
  for (int j0 = 0; j0 < k; j0 += KB) {
    uint4 v[KB];
    float wj[KB];
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) {
      const int j = j0 + jj < k ? j0 + jj : j0;
      v[jj] = *reinterpret_cast<const uint4*>(Y + (size_t)inv[t * k + j] * H + m);
      wj[jj] = w[t * k + j];
    }
#pragma unroll
    for (int jj = 0; jj < KB; ++jj) {
      if (j0 + jj >= k) break;
      const uint32_t u[4] = {v[jj].x, v[jj].y, v[jj].z, v[jj].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = __uint_as_float(u[q] << 16), hi = __uint_as_float(u[q] & 0xFFFF0000u);
        const float plo = lo * wj[jj], phi = hi * wj[jj];
        acc[2 * q] = acc[2 * q] + plo;
        acc[2 * q + 1] = acc[2 * q + 1] + phi;
      }
    }
  }
  uint16_t yb[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) yb[q] = f32_to_bf16(acc[q]);
  if (resid) {                       // h = x + y of the decoder layer (resid may alias y: read before the write)
    const uint4 rv = *reinterpret_cast<const uint4*>(resid + (size_t)t * H + m);
    const uint32_t r[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      yb[2 * q] = residual_bf16((uint16_t)r[q], yb[2 * q]);
      yb[2 * q + 1] = residual_bf16((uint16_t)(r[q] >> 16), yb[2 * q + 1]);
    }
  }
  uint4 o;
  o.x = (uint32_t)yb[0] | ((uint32_t)yb[1] << 16);
  o.y = (uint32_t)yb[2] | ((uint32_t)yb[3] << 16);
  o.z = (uint32_t)yb[4] | ((uint32_t)yb[5] << 16);
  o.w = (uint32_t)yb[6] | ((uint32_t)yb[7] << 16);
  *reinterpret_cast<uint4*>(y + (size_t)t * H + m) = o;
}

// ------------------------------------------------------------------ host
struct PrefillWs {
  int32_t *hist, *perm, *inv, *offsets, *status, *slot_inds;
  int4* tiles;
  float *logits, *w;
  int32_t* inds;
  uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;
  uint16_t* Y;
};

// Tile capacities: a wide tile holds more than narrow_max routes (or, with narrow tiles off, at least one), so
// sum_s ceil(count_s / 64) <= P / 64 + #{s : count_s > narrow_max}; at most one narrow tile per slot.
struct PfTiling {
  int narrow_max, wcap, scap;
};
static PfTiling pf_tiling(int64_t P, int S, int I) {
  PfTiling t;
  const bool narrow = I % 256 == 0;    // narrow blocks: 128 (gate/up) or 256 (down) outputs, K-steps of 256
  t.narrow_max = narrow ? PF_NARROW_MAX : 0;
  t.wcap = (int)(P / PF_WIDE_ROWS + std::min<int64_t>(S, P / (t.narrow_max + 1)) + 1);
  t.scap = narrow ? (int)std::min<int64_t>(S, P) : 0;
  return t;
}

static PrefillWs carve_prefill(Carve& c, int T, int k, int S, int H, int I, int E) {
  PrefillWs w{};
  const size_t P = (size_t)T * k;
  const PfTiling tl = pf_tiling((int64_t)P, S, I);
  w.status = c.take<int32_t>(1);
  w.hist = reinterpret_cast<int32_t*>(c.take<char>(dispatch_workspace((int)P, S)));
  w.perm = c.take<int32_t>(P);
  w.inv = c.take<int32_t>(P);
  w.offsets = c.take<int32_t>(S + 1);
  w.tiles = c.take<int4>(1 + (size_t)tl.wcap + tl.scap);
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

// stage (optional): a second bank whose slots follow the bank's (slot ids bank->n_slots ...)
// The narrow tiles of a GEMM run on a side stream concurrently with the wide tiles on the caller's stream: the
// narrow launch waits for the work queued on the caller's stream, and the caller's stream waits for the narrow
// launch before its next work.  Each (device, caller stream) pair has a side stream of its own (default priority,
// created with its two events on the pair's first prefill and kept for the life of the process), so a prefill
// waits only for work of its own caller stream: calls on different streams create no ordering between those
// streams, and a capture on one stream never joins another stream's work.  The fork and join of one call are
// enqueued under the pair's lock, so host threads sharing a caller stream never wait on each other's events.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  std::mutex mu;
};
// At most kMaxSideStreams pairs get one; a prefill on any other caller stream (or one whose side stream could not
// be created) runs both tile launches on the caller's stream, one after the other: the same results, without the
// overlap.
constexpr size_t kMaxSideStreams = 64;
static SideStream* side_stream(hipStream_t caller) {
  static KeyedOnce<std::pair<int, hipStream_t>, SideStream> per;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  return per.get(std::make_pair(dev, caller), []() -> std::unique_ptr<SideStream> {
    std::unique_ptr<SideStream> ss(new SideStream);
    if (hipStreamCreateWithFlags(&ss->s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&ss->fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ss->join, hipEventDisableTiming) != hipSuccess) {
      if (ss->fork) (void)hipEventDestroy(ss->fork);
      (void)hipStreamDestroy(ss->s);
      return nullptr;
    }
    return ss;
  }, kMaxSideStreams);
}

template <bool GATEUP, bool WIDE> static int pf_allow_lds() {
  static std::atomic<int> allowed{0};   // host threads may race to set the attribute; setting it twice is harmless
  if (allowed.load(std::memory_order_acquire)) return MIMO_OK;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_gemm_kernel<GATEUP, WIDE>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, pf_lds_bytes<WIDE>());
  if (e != hipSuccess) return set_error(MIMO_ERR_HIP, "prefill LDS attribute: %s", hipGetErrorString(e));
  allowed.store(1, std::memory_order_release);
  return MIMO_OK;
}

// zero_status: the status word has not been cleared yet in this call (the activation split, queued first,
// clears it before the dispatch may flag bad slots)
static int run_prefill(const uint16_t* x, int T, const int32_t* slot_inds, const float* wts, int k, const mimo_bank* bank,
                       const mimo_bank* stage, uint16_t* y, const PrefillWs& ws, hipStream_t st, bool zero_status,
                       const uint16_t* resid = nullptr) {
  const int H = bank->hidden, I = bank->inter, S = bank->n_slots + (stage ? stage->n_slots : 0);
  const int P = T * k;
  // the GEMM kernels address activation and h rows with 32-bit offsets
  MIMO_REQUIRE((int64_t)T * H < (int64_t)1 << 31 && (int64_t)P * I < (int64_t)1 << 31, MIMO_ERR_SHAPE,
               "moe_prefill: T * hidden and T * k * inter must stay below 2^31");
  int err;
  const uint16_t* sig = sigtab_device(&err);
  if (!sig) return err;
  const PfTiling tl = pf_tiling(P, S, I);
  const TileSpec spec{tl.narrow_max, PF_WIDE_ROWS, tl.wcap, PF_UNIT};
  int rc = launch_quantize_fp8_hilo(x, T, H, ws.xq_hi, ws.xq_hs, ws.xq_lo, ws.xq_ls, st,
                                    zero_status ? ws.status : nullptr);
  if (rc) return rc;
  rc = launch_dispatch(slot_inds, P, S, ws.hist, ws.perm, ws.offsets, ws.inv, &spec, ws.tiles, ws.status, st);
  if (rc) return rc;
  PrefillArgs a{};
  a.xq_hi = ws.xq_hi; a.xq_lo = ws.xq_lo; a.xq_hs = ws.xq_hs; a.xq_ls = ws.xq_ls;
  a.perm = ws.perm; a.offsets = ws.offsets; a.inv = ws.inv; a.w = wts; a.tiles = ws.tiles; a.wcap = tl.wcap;
  a.T = T; a.k = k; a.S = S; a.H = H; a.I = I; a.P = P;
  a.S0 = bank->n_slots;
  const mimo_bank* pools[2] = {bank, stage ? stage : bank};
  for (int i = 0; i < 2; ++i) {
    a.gate_w[i] = pools[i]->gate_w; a.up_w[i] = pools[i]->up_w; a.down_w[i] = pools[i]->down_w;
    a.gate_s[i] = pools[i]->gate_s; a.up_s[i] = pools[i]->up_s; a.down_s[i] = pools[i]->down_s;
  }
  a.sigtab = sig;
  a.hq_hi = ws.hq_hi; a.hq_lo = ws.hq_lo; a.hq_hs = ws.hq_hs; a.hq_ls = ws.hq_ls;
  a.Y = ws.Y; a.y = y;
  int rc2 = pf_allow_lds<true, true>();
  if (!rc2) rc2 = pf_allow_lds<true, false>();
  if (!rc2) rc2 = pf_allow_lds<false, true>();
  if (!rc2) rc2 = pf_allow_lds<false, false>();
  if (rc2) return rc2;
  // 1-D grids of 8 ceil(bound / 8) blocks per shape, so every XCD has an index for each of its (tile, output
  // block) pairs; blocks past the used pairs exit at once.
  auto grid_of = [&](int cap, int obn) { return 8 * (int)(((int64_t)cap * obn + 7) / 8); };
  using NS = PfShape<false>;
  using WS = PfShape<true>;
  SideStream* ss = tl.scap ? side_stream(st) : nullptr;
  // one GEMM: narrow tiles on the side stream, wide tiles on st, joined before st's next work (without a side
  // stream, both on st)
  auto gemm = [&](auto narrow_kernel, auto wide_kernel, int obn_narrow, int obn_wide) -> int {
    if (!ss) {
      if (tl.scap) narrow_kernel<<<grid_of(tl.scap, obn_narrow), 512, pf_lds_bytes<false>(), st>>>(a);
      wide_kernel<<<grid_of(tl.wcap, obn_wide), 512, pf_lds_bytes<true>(), st>>>(a);
      return MIMO_OK;
    }
    std::lock_guard<std::mutex> g(ss->mu);
    MIMO_HIP(hipEventRecord(ss->fork, st));
    MIMO_HIP(hipStreamWaitEvent(ss->s, ss->fork, 0));
    narrow_kernel<<<grid_of(tl.scap, obn_narrow), 512, pf_lds_bytes<false>(), ss->s>>>(a);
    wide_kernel<<<grid_of(tl.wcap, obn_wide), 512, pf_lds_bytes<true>(), st>>>(a);
    MIMO_HIP(hipEventRecord(ss->join, ss->s));
    MIMO_HIP(hipStreamWaitEvent(st, ss->join, 0));
    return MIMO_OK;
  };
  {
    ProfScope p(st, "prefill_gateup");
    int rc3 = gemm(prefill_gemm_kernel<true, false>, prefill_gemm_kernel<true, true>, I / (NS::N / 2), I / (WS::N / 2));
    if (rc3) return rc3;
  }
  {
    ProfScope p(st, "prefill_down");
    int rc3 = gemm(prefill_gemm_kernel<false, false>, prefill_gemm_kernel<false, true>, H / NS::N, H / WS::N);
    if (rc3) return rc3;
  }
  { ProfScope p(st, "prefill_combine");
    prefill_combine_kernel<<<dim3((H + 2047) / 2048, T), 256, 0, st>>>(ws.Y, ws.inv, wts, k, H, resid, y); }
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
                     uint16_t* y, int32_t* status_out, void* ws, size_t ws_bytes, void* stream) {
  ProfChain chain;   // per-kernel timing (when enabled) back to back within this call
  int rc = check_prefill_bank(bank);
  if (rc) return rc;
  MIMO_REQUIRE(x && slot_inds && w && y, MIMO_ERR_ARG, "moe_prefill: null pointer");
  MIMO_REQUIRE(T >= 1 && k >= 1 && (int64_t)T * k < (1 << 30), MIMO_ERR_SHAPE, "moe_prefill: bad T or k");
  MIMO_REQUIRE(aligned16(x) && aligned16(y), MIMO_ERR_ALIGN, "moe_prefill: 16-byte alignment");
  Carve c(ws, ws_bytes);
  PrefillWs pw = carve_prefill(c, T, k, bank->n_slots, bank->hidden, bank->inter, 0);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_prefill: workspace too small (need %zu)", c.off);
  if (status_out) pw.status = status_out;
  return run_prefill(x, T, slot_inds, w, k, bank, nullptr, y, pw, as_stream(stream), true);
}

int mimo_moe_prefill_staged(const uint16_t* x, int T, const int32_t* slot_inds, const float* w, int k,
                            const mimo_bank* bank, const mimo_bank* stage, uint16_t* y, int32_t* status_out, void* ws,
                            size_t ws_bytes, void* stream) {
  ProfChain chain;
  int rc = check_prefill_bank(bank);
  if (rc) return rc;
  rc = check_prefill_bank(stage);
  if (rc) return rc;
  MIMO_REQUIRE(stage->hidden == bank->hidden && stage->inter == bank->inter, MIMO_ERR_SHAPE,
               "moe_prefill_staged: staging bank of another expert shape");
  MIMO_REQUIRE(bank->n_slots + stage->n_slots <= 1024, MIMO_ERR_SHAPE,
               "moe_prefill_staged: at most 1024 slots in the bank and the staging bank together");
  MIMO_REQUIRE(x && slot_inds && w && y, MIMO_ERR_ARG, "moe_prefill_staged: null pointer");
  MIMO_REQUIRE(T >= 1 && k >= 1 && (int64_t)T * k < (1 << 30), MIMO_ERR_SHAPE, "moe_prefill_staged: bad T or k");
  MIMO_REQUIRE(aligned16(x) && aligned16(y), MIMO_ERR_ALIGN, "moe_prefill_staged: 16-byte alignment");
  Carve c(ws, ws_bytes);
  PrefillWs pw = carve_prefill(c, T, k, bank->n_slots + stage->n_slots, bank->hidden, bank->inter, 0);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_prefill_staged: workspace too small (need %zu)", c.off);
  if (status_out) pw.status = status_out;
  return run_prefill(x, T, slot_inds, w, k, bank, stage, y, pw, as_stream(stream), true);
}

size_t mimo_moe_prefill_block_workspace_size(int T, int E, int k, int n_slots, int H, int I) {
  Carve c(nullptr, 0);
  carve_prefill(c, T, k, n_slots, H, I, E);
  return c.off;
}

}  // extern "C"

namespace mimo {
// Router + grouped GEMMs + combine on rows x; resid: optional residual stream added in the combine.
static int prefill_block_impl(const uint16_t* x, int T, const uint16_t* Wg, const float* bias, const int32_t* slot_of,
                              int E, int k, const mimo_bank* bank, uint16_t* y, int32_t* inds_out, float* w_out,
                              const uint16_t* resid, int32_t* status_out, void* ws, size_t ws_bytes, hipStream_t st) {
  int rc = check_prefill_bank(bank);
  if (rc) return rc;
  MIMO_REQUIRE(x && Wg && bias && y, MIMO_ERR_ARG, "moe_prefill_block: null pointer");
  MIMO_REQUIRE(T >= 1 && k >= 1 && k <= 16 && E >= k && E <= 1024 && bank->hidden % 64 == 0, MIMO_ERR_SHAPE,
               "moe_prefill_block: need 1 <= k <= min(16, E), E <= 1024");
  MIMO_REQUIRE(aligned16(x) && aligned16(Wg) && aligned16(y), MIMO_ERR_ALIGN, "moe_prefill_block: alignment");
  Carve c(ws, ws_bytes);
  PrefillWs pw = carve_prefill(c, T, k, bank->n_slots, bank->hidden, bank->inter, E);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_prefill_block: workspace too small (need %zu)", c.off);
  int32_t* inds = inds_out ? inds_out : pw.inds;
  float* wts = w_out ? w_out : pw.w;
  if (status_out) pw.status = status_out;
  rc = launch_router_logits(x, Wg, T, bank->hidden, E, pw.logits, st, pw.status);   // clears the status word
  if (rc) return rc;
  rc = launch_router_select(pw.logits, bias, T, E, k, 1.0f, inds, wts, slot_of, pw.slot_inds, bank->n_slots, pw.status,
                            st);
  if (rc) return rc;
  return run_prefill(x, T, pw.slot_inds, wts, k, bank, nullptr, y, pw, st, false, resid);
}
}  // namespace mimo

extern "C" {

int mimo_moe_prefill_block(const uint16_t* x, int T, const uint16_t* Wg, const float* bias, const int32_t* slot_of,
                           int E, int k, const mimo_bank* bank, uint16_t* y, int32_t* inds_out, float* w_out,
                           int32_t* status_out, void* ws, size_t ws_bytes, void* stream) {
  ProfChain chain;   // per-kernel timing (when enabled) back to back within this call
  return prefill_block_impl(x, T, Wg, bias, slot_of, E, k, bank, y, inds_out, w_out, nullptr, status_out, ws, ws_bytes,
                            as_stream(stream));
}

// The normalised rows r (T x H bf16) go first in the layer workspace, 256-byte aligned.
static size_t prefill_rows_bytes(int T, int H) { return ((size_t)T * H * 2 + 255) / 256 * 256; }

size_t mimo_moe_layer_prefill_workspace_size(int T, int E, int k, int n_slots, int H, int I) {
  return prefill_rows_bytes(T, H) + mimo_moe_prefill_block_workspace_size(T, E, k, n_slots, H, I);
}

int mimo_moe_layer_prefill(const uint16_t* x, int T, const uint16_t* norm_w, float eps, const uint16_t* Wg,
                           const float* bias, const int32_t* slot_of, int E, int k, const mimo_bank* bank, uint16_t* h,
                           uint16_t* r_out, int32_t* inds_out, float* w_out, int32_t* status_out, void* ws,
                           size_t ws_bytes, void* stream) {
  ProfChain chain;
  MIMO_REQUIRE(x && norm_w && h && bank, MIMO_ERR_ARG, "moe_layer_prefill: null pointer");
  MIMO_REQUIRE(T >= 1, MIMO_ERR_SHAPE, "moe_layer_prefill: need T >= 1");
  MIMO_REQUIRE(aligned16(x) && aligned16(h) && (!r_out || aligned16(r_out)), MIMO_ERR_ALIGN,
               "moe_layer_prefill: 16-byte alignment");
  MIMO_REQUIRE(r_out != x && r_out != h, MIMO_ERR_ARG, "moe_layer_prefill: r_out may not alias x or h");
  const int H = bank->hidden;
  const size_t rb = prefill_rows_bytes(T, H);
  MIMO_REQUIRE(ws && ws_bytes >= rb, MIMO_ERR_WORKSPACE, "moe_layer_prefill: workspace too small (need %zu)",
               mimo_moe_layer_prefill_workspace_size(T, E, k, bank->n_slots, H, bank->inter));
  hipStream_t st = as_stream(stream);
  uint16_t* r = r_out ? r_out : static_cast<uint16_t*>(ws);
  int rc = launch_rmsnorm(x, T, H, norm_w, eps, r, st);
  if (rc) return rc;
  return prefill_block_impl(r, T, Wg, bias, slot_of, E, k, bank, h, inds_out, w_out, x, status_out,
                            static_cast<uint8_t*>(ws) + rb, ws_bytes - rb, st);
}

}  // extern "C"
