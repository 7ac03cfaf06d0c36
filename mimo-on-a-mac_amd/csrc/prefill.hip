// Prefill MoE: (token, k) routes sorted by slot, grouped gate/up + SwiGLU and down GEMMs on block-scaled
// MFMA, bf16 expert outputs, fixed-order weighted combine back to token order.
//
// Reference: _moe_prefill engine/mimo_stream/model.py:230-271 and _pair_outputs :221-228 (three sorted
// gather_qmm calls, bf16 SwiGLU intermediate, bf16 expert outputs, inverse permutation, (Y.f32 * w).sum(1)).
//
// Tiling: a "row tile" is up to 32 consecutive sorted routes of one slot (the dispatch builds the per-slot
// row-tile offsets).  Each block owns one row tile and 128 outputs; each wave 32 outputs.  Per K-step of 128
// a wave issues 4 (8-route chunks) x 2 (16-output tiles) MFMAs per projection, the chunk's hi and lo E4M3
// activation halves sharing one MFMA in rows 0-7 / 8-15 (same operand layout as the decode kernels).
#include "device.h"
#include "host.h"
#include "router.h"

namespace mimo {

struct PrefillArgs {
  const uint8_t *xq_hi, *xq_lo, *xq_hs, *xq_ls;   // [T, H], [T, H/32]
  const int32_t *perm, *offsets, *tile_off, *inv;
  const float* w;
  int T, k, S, H, I, P;
  const uint32_t *gate_w, *up_w, *down_w;
  const uint8_t *gate_s, *up_s, *down_s;
  const uint16_t* sigtab;
  uint8_t *hq_hi, *hq_lo, *hq_hs, *hq_ls;         // [P, I], [P, I/32] in sorted route order
  uint16_t* Y;                                    // [P, H] bf16 expert outputs, sorted route order
  uint16_t* y;                                    // [T, H]
};

constexpr int PF_ROWS = 32;

__device__ __forceinline__ v8i pf_a(const uint8_t* row, int k0, int g, bool valid) {
  if (!valid) return v8i{0, 0, 0, 0, 0, 0, 0, 0};
  uint4 a0 = *reinterpret_cast<const uint4*>(row + k0 + 16 * g);
  uint4 a1 = *reinterpret_cast<const uint4*>(row + k0 + 64 + 16 * g);
  return v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
}
__device__ __forceinline__ v8i pf_b(uint4 b) { return v8i{(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0}; }
#define PF_MFMA(A, B, C, SA, SB) __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4((A), (B), (C), 0, 4, 0, (SA), 0, (SB))

// row tile rt -> slot s and its sorted-route range [beg, end)
__device__ __forceinline__ bool find_tile(const PrefillArgs& a, int rt, int* s_out, int* beg, int* end) {
  if (rt >= a.tile_off[a.S]) return false;
  int lo = 0, hi = a.S;                        // tile_off[lo] <= rt < tile_off[hi]
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (a.tile_off[mid] <= rt) lo = mid; else hi = mid;
  }
  *s_out = lo;
  *beg = a.offsets[lo] + (rt - a.tile_off[lo]) * PF_ROWS;
  int e = *beg + PF_ROWS;
  *end = e < a.offsets[lo + 1] ? e : a.offsets[lo + 1];
  return true;
}

// ------------------------------------------------------------------ gate/up + SwiGLU + hi/lo split of h
__global__ void __launch_bounds__(256) prefill_gateup_kernel(PrefillArgs a) {
  int s, beg, end;
  if (!find_tile(a, blockIdx.y, &s, &beg, &end)) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int n0 = blockIdx.x * 128 + wave * 32;
  const uint8_t* arow[4];
  const uint8_t* ascl[4];
  bool av[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int p = beg + c * 8 + (i & 7);
    av[c] = p < end;
    int tok = av[c] ? a.perm[p] / a.k : 0;
    arow[c] = (i < 8 ? a.xq_hi : a.xq_lo) + (size_t)tok * a.H;
    ascl[c] = (i < 8 ? a.xq_hs : a.xq_ls) + (size_t)tok * (a.H / 32);
  }
  const uint32_t* gw[2];
  const uint32_t* uwp[2];
  const uint8_t* gs[2];
  const uint8_t* us[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const size_t brow = (size_t)s * a.I + n0 + b * 16 + i;
    gw[b] = a.gate_w + brow * (a.H / 8);
    uwp[b] = a.up_w + brow * (a.H / 8);
    gs[b] = a.gate_s + brow * (a.H / 32);
    us[b] = a.up_s + brow * (a.H / 32);
  }
  v4f accg[4][2], accu[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int b = 0; b < 2; ++b) { accg[c][b] = v4f{0, 0, 0, 0}; accu[c][b] = v4f{0, 0, 0, 0}; }
  for (int k0 = 0; k0 < a.H; k0 += 128) {
    const int blk = k0 / 32 + g;
    v8i Bg[2], Bu[2];
    int sg[2], su[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      Bg[b] = pf_b(*reinterpret_cast<const uint4*>(gw[b] + k0 / 8 + 4 * g));
      Bu[b] = pf_b(*reinterpret_cast<const uint4*>(uwp[b] + k0 / 8 + 4 * g));
      sg[b] = gs[b][blk];
      su[b] = us[b][blk];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      v8i A = pf_a(arow[c], k0, g, av[c]);
      int sa = av[c] ? (int)ascl[c][blk] : 127;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        accg[c][b] = PF_MFMA(A, Bg[b], accg[c][b], sa, sg[b]);
        accu[c][b] = PF_MFMA(A, Bu[b], accu[c][b], sa, su[b]);
      }
    }
  }
  // epilogue per 8-route chunk: lanes < 32 hold routes c*8 + 4g + q at outputs n0 + 16b + i
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float hv[2][4];
    float amax[4] = {0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float gsum = accg[c][b][q] + __shfl_xor(accg[c][b][q], 32, 64);
        float usum = accu[c][b][q] + __shfl_xor(accu[c][b][q], 32, 64);
        uint16_t gt = f32_to_bf16(gsum);
        float gtf = bf16_to_f32(gt);
        float ut = round_bf16(usum);
        float sig = bf16_to_f32(a.sigtab[gt]);
        hv[b][q] = round_bf16(round_bf16(gtf * sig) * ut);
        amax[q] = fmaxf(amax[q], fabsf(hv[b][q]));
      }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // the 32 outputs of this wave form one E8M0 block of h: reduce over the 16 lanes of the group
      float am = group_max(amax[q], 16);
      const int X = fp8_block_exp(am);
      uint32_t hc[2], lc[2];
      float res[2];
      float ram = 0.0f;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float dec;
        hc[b] = e4m3_encode(hv[b][q], X, &dec);
        res[b] = hv[b][q] - dec;
        ram = fmaxf(ram, fabsf(res[b]));
      }
      ram = group_max(ram, 16);
      const int Yx = fp8_block_exp(ram);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float dec;
        lc[b] = e4m3_encode(res[b], Yx, &dec);
      }
      const int p = beg + c * 8 + 4 * g + q;
      if (lane < 32 && p < end) {
        uint8_t* hrow = a.hq_hi + (size_t)p * a.I + n0;
        uint8_t* lrow = a.hq_lo + (size_t)p * a.I + n0;
        hrow[i] = (uint8_t)hc[0];
        hrow[16 + i] = (uint8_t)hc[1];
        lrow[i] = (uint8_t)lc[0];
        lrow[16 + i] = (uint8_t)lc[1];
        if (i == 0) {
          a.hq_hs[(size_t)p * (a.I / 32) + n0 / 32] = (uint8_t)(X + 127);
          a.hq_ls[(size_t)p * (a.I / 32) + n0 / 32] = (uint8_t)(Yx + 127);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ down: bf16 expert outputs
__global__ void __launch_bounds__(256) prefill_down_kernel(PrefillArgs a) {
  int s, beg, end;
  if (!find_tile(a, blockIdx.y, &s, &beg, &end)) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int m0 = blockIdx.x * 128 + wave * 32;
  const uint8_t* arow[4];
  const uint8_t* ascl[4];
  bool av[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int p = beg + c * 8 + (i & 7);
    av[c] = p < end;
    const size_t pr = av[c] ? (size_t)p : 0;
    arow[c] = (i < 8 ? a.hq_hi : a.hq_lo) + pr * a.I;
    ascl[c] = (i < 8 ? a.hq_hs : a.hq_ls) + pr * (a.I / 32);
  }
  const uint32_t* dw[2];
  const uint8_t* dsc[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const size_t brow = (size_t)s * a.H + m0 + b * 16 + i;
    dw[b] = a.down_w + brow * (a.I / 8);
    dsc[b] = a.down_s + brow * (a.I / 32);
  }
  v4f acc[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[c][b] = v4f{0, 0, 0, 0};
  for (int k0 = 0; k0 < a.I; k0 += 128) {
    const int blk = k0 / 32 + g;
    v8i B[2];
    int sb[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      B[b] = pf_b(*reinterpret_cast<const uint4*>(dw[b] + k0 / 8 + 4 * g));
      sb[b] = dsc[b][blk];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      v8i A = pf_a(arow[c], k0, g, av[c]);
      int sa = av[c] ? (int)ascl[c][blk] : 127;
#pragma unroll
      for (int b = 0; b < 2; ++b) acc[c][b] = PF_MFMA(A, B[b], acc[c][b], sa, sb[b]);
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v = acc[c][b][q] + __shfl_xor(acc[c][b][q], 32, 64);
        const int p = beg + c * 8 + 4 * g + q;
        if (lane < 32 && p < end) a.Y[(size_t)p * a.H + m0 + b * 16 + i] = f32_to_bf16(v);
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
  int err;
  const uint16_t* sig = sigtab_device(&err);
  if (!sig) return err;
  int rc = launch_dispatch(slot_inds, P, S, ws.hist, ws.perm, ws.offsets, ws.inv, PF_ROWS, ws.tile_off, ws.status, st);
  if (rc) return rc;
  rc = launch_quantize_fp8_hilo(x, T, H, ws.xq_hi, ws.xq_hs, ws.xq_lo, ws.xq_ls, st);
  if (rc) return rc;
  PrefillArgs a{};
  a.xq_hi = ws.xq_hi; a.xq_lo = ws.xq_lo; a.xq_hs = ws.xq_hs; a.xq_ls = ws.xq_ls;
  a.perm = ws.perm; a.offsets = ws.offsets; a.tile_off = ws.tile_off; a.inv = ws.inv; a.w = wts;
  a.T = T; a.k = k; a.S = S; a.H = H; a.I = I; a.P = P;
  a.gate_w = bank->gate_w; a.up_w = bank->up_w; a.down_w = bank->down_w;
  a.gate_s = bank->gate_s; a.up_s = bank->up_s; a.down_s = bank->down_s;
  a.sigtab = sig;
  a.hq_hi = ws.hq_hi; a.hq_lo = ws.hq_lo; a.hq_hs = ws.hq_hs; a.hq_ls = ws.hq_ls;
  a.Y = ws.Y; a.y = y;
  const int max_tiles = (P + PF_ROWS - 1) / PF_ROWS + S;     // bound on sum_s ceil(count_s / PF_ROWS)
  { ProfScope p(st, "prefill_gateup"); prefill_gateup_kernel<<<dim3(I / 128, max_tiles), 256, 0, st>>>(a); }
  { ProfScope p(st, "prefill_down"); prefill_down_kernel<<<dim3(H / 128, max_tiles), 256, 0, st>>>(a); }
  { ProfScope p(st, "prefill_combine");
    prefill_combine_kernel<<<dim3((H + 1023) / 1024, T), 256, 0, st>>>(ws.Y, ws.inv, wts, k, H, y); }
  return check_launch("moe prefill");
}

static int check_prefill_bank(const mimo_bank* b) {
  MIMO_REQUIRE(b && b->gate_w && b->gate_s && b->up_w && b->up_s && b->down_w && b->down_s, MIMO_ERR_ARG,
               "bank: null pointer");
  MIMO_REQUIRE(b->n_slots >= 1 && b->n_slots <= 1024 && b->hidden % 128 == 0 && b->hidden >= 128 &&
                   b->inter % 128 == 0 && b->inter >= 128,
               MIMO_ERR_SHAPE, "prefill bank: need hidden, inter multiples of 128 and n_slots <= 1024");
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
