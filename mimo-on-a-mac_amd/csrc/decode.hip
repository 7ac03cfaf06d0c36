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
// Block: one distinct expert u (blockIdx.y) x 32 outputs n (blockIdx.x).  Waves: 2 n-tiles x 2 K-halves.
// Writes h (bf16, rounding points of kernels.py:79-82) and its hi/lo E4M3 split for the down projection.
__global__ void __launch_bounds__(256) decode_gateup_kernel(ExpertsArgs a) {
  const int u = blockIdx.y;
  const int U = a.n_unique ? *a.n_unique : a.Umax;
  if (u >= U) return;
  const int cnt = min(a.ucnt[u], a.R);
  const int slot = a.uslot[u];
  if (cnt <= 0 || slot < 0 || slot >= a.S) return;     // caller-supplied ids are range-checked
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int ntile = wave & 1, khalf = wave >> 1;
  const int nb = blockIdx.x * 32;
  const int n0 = nb + ntile * 16;
  const int arow = i & 7;
  const bool avalid = arow < cnt;
  int token = avalid ? a.urows[u * a.R + arow] : 0;
  token = (token < 0 || token >= a.M) ? 0 : token;
  const uint8_t* abase = (i < 8 ? a.xq_hi : a.xq_lo) + (size_t)token * a.H;
  const uint8_t* ascl = (i < 8 ? a.xq_hs : a.xq_ls) + (size_t)token * (a.H / 32);
  const size_t brow = (size_t)slot * a.I + n0 + i;
  const uint32_t* gw = a.gate_w + brow * (a.H / 8);
  const uint32_t* upw = a.up_w + brow * (a.H / 8);
  const uint8_t* gs = a.gate_s + brow * (a.H / 32);
  const uint8_t* us = a.up_s + brow * (a.H / 32);
  const int kspan = a.H / 2;
  const int kbeg = khalf * kspan;
  v4f accg = {0.0f, 0.0f, 0.0f, 0.0f}, accu = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
  for (int k0 = kbeg; k0 < kbeg + kspan; k0 += 128) {
    const int blk = k0 / 32 + g;
    uint4 bg = *reinterpret_cast<const uint4*>(gw + k0 / 8 + 4 * g);
    uint4 bu = *reinterpret_cast<const uint4*>(upw + k0 / 8 + 4 * g);
    int sg = gs[blk], su = us[blk];
    v8i A = a_operand(abase, k0, g, avalid);
    int sa = avalid ? (int)ascl[blk] : 127;
    accg = MFMA_F8xF4(A, b_operand(bg), accg, sa, sg);
    accu = MFMA_F8xF4(A, b_operand(bu), accu, sa, su);
  }
  float vg[4], vu[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {   // rows 4g+q (hi, g < 2) plus rows 8+4g+q (lo) of lane l + 32
    vg[q] = accg[q] + __shfl_xor(accg[q], 32, 64);
    vu[q] = accu[q] + __shfl_xor(accu[q], 32, 64);
  }
  __shared__ float red[2][2][32][4];
  __shared__ float hl[8][32];
  if (khalf == 1 && lane < 32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) { red[ntile][0][lane][q] = vg[q]; red[ntile][1][lane][q] = vu[q]; }
  }
  __syncthreads();
  if (khalf == 0 && lane < 32) {
    const int n = n0 + i;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 4 * g + q;
      float gsum = vg[q] + red[ntile][0][lane][q];
      float usum = vu[q] + red[ntile][1][lane][q];
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

// ------------------------------------------------------------------ Kernel B: down * router weight
// Block: one distinct expert u (blockIdx.y) x 64 outputs m (blockIdx.x); one wave per 16 outputs, full K.
__global__ void __launch_bounds__(256) decode_down_kernel(ExpertsArgs a) {
  const int u = blockIdx.y;
  const int U = a.n_unique ? *a.n_unique : a.Umax;
  if (u >= U) return;
  const int cnt = min(a.ucnt[u], a.R);
  const int slot = a.uslot[u];
  if (cnt <= 0 || slot < 0 || slot >= a.S) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
  const int m0 = blockIdx.x * 64 + wave * 16;
  const int arow = i & 7;
  const bool avalid = arow < cnt;
  const size_t hrow = (size_t)u * a.R + arow;
  const uint8_t* abase = (i < 8 ? a.hq_hi : a.hq_lo) + hrow * a.I;
  const uint8_t* ascl = (i < 8 ? a.hq_hs : a.hq_ls) + hrow * (a.I / 32);
  const size_t brow = (size_t)slot * a.H + m0 + i;
  const uint32_t* dw = a.down_w + brow * (a.I / 8);
  const uint8_t* dsc = a.down_s + brow * (a.I / 32);
  v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
  for (int k0 = 0; k0 < a.I; k0 += 128) {
    const int blk = k0 / 32 + g;
    uint4 b = *reinterpret_cast<const uint4*>(dw + k0 / 8 + 4 * g);
    int sb = dsc[blk];
    v8i A = a_operand(abase, k0, g, avalid);
    int sa = avalid ? (int)ascl[blk] : 127;
    acc = MFMA_F8xF4(A, b_operand(b), acc, sa, sb);
  }
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = acc[q] + __shfl_xor(acc[q], 32, 64);
  if (lane < 32) {
    const int m = m0 + i;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 4 * g + q;
      if (r < cnt) {
        float d = v[q];
        if (a.round_bf16) d = round_bf16(d);
        a.part[((size_t)u * a.R + r) * a.H + m] = d * a.uw[u * a.R + r];
      } else if (a.zero_pad && r < a.R) {
        a.part[((size_t)u * a.R + r) * a.H + m] = 0.0f;
      }
    }
  }
}

// ------------------------------------------------------------------ fixed-order combine
// y[row] = bf16(sum_j part[gidx[row*k + j]]), j ascending (kernels.py:198-199).
__global__ void __launch_bounds__(256) decode_combine_kernel(const float* __restrict__ part, const uint32_t* __restrict__ gidx,
                                                             int k, int H, uint32_t nrows, uint16_t* __restrict__ y) {
  const int row = blockIdx.y;
  const int m = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (m >= H) return;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int j = 0; j < k; ++j) {
    const uint32_t idx = gidx[row * k + j];
    if (idx >= nrows) continue;                  // caller-supplied gather index out of range
    const float4 p = *reinterpret_cast<const float4*>(part + (size_t)idx * H + m);
    acc.x = acc.x + p.x;
    acc.y = acc.y + p.y;
    acc.z = acc.z + p.z;
    acc.w = acc.w + p.w;
  }
  uint2 o;
  o.x = (uint32_t)f32_to_bf16(acc.x) | ((uint32_t)f32_to_bf16(acc.y) << 16);
  o.y = (uint32_t)f32_to_bf16(acc.z) | ((uint32_t)f32_to_bf16(acc.w) << 16);
  *reinterpret_cast<uint2*>(y + (size_t)row * H + m) = o;
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
  MIMO_REQUIRE(b->n_slots >= 1 && b->hidden >= 256 && b->hidden % 256 == 0 && b->inter >= 128 && b->inter % 128 == 0,
               MIMO_ERR_SHAPE, "bank: need hidden %% 256 == 0 and inter %% 128 == 0 (got H=%d I=%d)", b->hidden,
               b->inter);
  MIMO_REQUIRE(aligned16(b->gate_w) && aligned16(b->up_w) && aligned16(b->down_w), MIMO_ERR_ALIGN,
               "bank: weight pools must be 16-byte aligned");
  return MIMO_OK;
}

static int run_experts(const ExpertsArgs& base, int M, int round_bf16, hipStream_t st) {
  ExpertsArgs a = base;
  a.round_bf16 = round_bf16;
  dim3 g1(a.I / 32, a.Umax), g2(a.H / 64, a.Umax), g3((a.H + 1023) / 1024, M);
  { ProfScope p(st, "decode_gateup"); decode_gateup_kernel<<<g1, 256, 0, st>>>(a); }
  { ProfScope p(st, "decode_down"); decode_down_kernel<<<g2, 256, 0, st>>>(a); }
  { ProfScope p(st, "decode_combine");
    decode_combine_kernel<<<g3, 256, 0, st>>>(a.part, a.gidx, a.k, a.H, (uint32_t)(a.Umax * a.R), a.y); }
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
  MIMO_REQUIRE(M >= 1 && M <= 8 && R >= 1 && R <= 8 && k >= 1 && Umax >= 1 && Umax <= M * k, MIMO_ERR_SHAPE,
               "moe_experts: need 1 <= M <= 8, 1 <= R <= 8, 1 <= Umax <= M*k");
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
                         int** counter, int32_t** inds, float** w, int32_t** uids, int32_t** urows, int32_t** ucnt,
                         float** uw, uint32_t** gidx, int32_t** nu, int32_t** status) {
  *counter = c.take<int>(1);
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
  int* cnt;
  int32_t *inds, *uids, *urows, *ucnt, *nu, *st;
  uint32_t* gidx;
  carve_decode(c, M, E, k, Umax, kDecodeR, &l, &s, &kk, &cnt, &inds, &w, &uids, &urows, &ucnt, &uw, &gidx, &nu, &st);
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
  const int H = bank->hidden, I = bank->inter, S = bank->n_slots;
  const int Umax = M * k < S ? M * k : S;
  Carve c(ws, ws_bytes);
  float *logits, *scores, *keys, *w, *uw;
  int* counter;
  int32_t *inds, *uids, *urows, *ucnt, *nu, *status;
  uint32_t* gidx;
  carve_decode(c, M, E, k, Umax, kDecodeR, &logits, &scores, &keys, &counter, &inds, &w, &uids, &urows, &ucnt, &uw,
               &gidx, &nu, &status);
  ExpertsWs ew = carve_experts(c, M, Umax, kDecodeR, H, I);
  MIMO_REQUIRE(ws && c.fits(), MIMO_ERR_WORKSPACE, "moe_decode: workspace too small (need %zu)", c.off);
  int err;
  const uint16_t* sig = sigtab_device(&err);
  if (!sig) return err;
  hipStream_t st = as_stream(stream);

  RouterSmallArgs ra{};
  ra.x = x; ra.Wg = Wg; ra.bias = bias; ra.T = M; ra.H = H; ra.E = E; ra.k = k; ra.nlog = (E + 3) / 4;
  ra.logits = logits; ra.scores = scores; ra.keys = keys; ra.counter = counter;
  ra.inds_out = inds_out ? inds_out : inds;
  ra.w_out = w_out ? w_out : w;
  ra.xq_hi = ew.xq_hi; ra.xq_lo = ew.xq_lo; ra.xq_hs = ew.xq_hs; ra.xq_ls = ew.xq_ls;
  ra.slot_of = slot_of; ra.R = kDecodeR; ra.n_slots = S; ra.Umax = Umax;
  ra.uids = uids; ra.urows = urows; ra.ucnt = ucnt; ra.uw = uw; ra.gidx = gidx; ra.n_unique = nu; ra.status = status;
  rc = launch_router_small(ra, st);
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
  // M == 1 follows _gather_m1 (bf16 expert outputs, model.py:173-182); M >= 2 the distinct-expert kernels
  return run_experts(a, M, M == 1 ? 1 : 0, st);
}

}  // extern "C"
