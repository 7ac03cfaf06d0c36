// Device helpers shared by the MoE kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimo {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// round-to-nearest-even float -> bf16 bits; NaN stays a quiet NaN with its high payload bits, i.e.
// ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 for numbers, (u >> 16) | 0x40 for NaN.  The hardware conversion
// (v_cvt_pk_bf16_f32) gives exactly these bits for every one of the 2^32 inputs (checked on MI355X).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ------------------------------------------------------------------ E2M1 / E8M0
// E2M1 magnitude code for y >= 0 already divided by the block scale: nearest-even on
// {0, .5, 1, 1.5, 2, 3, 4, 6}, saturating at 6 (OCP MX v1.0).
__device__ __forceinline__ uint32_t e2m1_mag_code(float y) {
  float v;
  if (y < 2.0f) v = rintf(y * 2.0f) * 0.5f;
  else if (y < 4.0f) v = rintf(y);
  else v = rintf(y * 0.5f) * 2.0f;
  // v in {0,.5,1,1.5,2,3,4,6,8}
  if (v >= 6.0f) return 7u;
  if (v >= 4.0f) return 6u;
  if (v >= 3.0f) return 5u;
  if (v >= 2.0f) return 4u;
  return (uint32_t)(v * 2.0f);  // 0, 1, 2, 3
}

// ------------------------------------------------------------------ E4M3 (activation hi/lo split)
// magnitude code for 0 <= y <= 448 (y exactly representable scaling of a bf16 value), nearest-even.
__device__ __forceinline__ uint32_t e4m3_mag_code(float y) {
  // below 2^-6: subnormal, quantum 2^-9 (a result of 8 is the smallest normal, same encoding)
  const uint32_t sub = (uint32_t)rintf(y * 512.0f);
  const uint32_t u = __float_as_uint(y);
  int e = (int)((u >> 23) & 0xFF) - 127;
  const uint32_t f = u & 0x7FFFFFu;
  uint32_t q = f >> 20;
  const uint32_t rem = f & 0xFFFFFu;
  q += (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ? 1u : 0u;
  e += q == 8u ? 1 : 0;
  q = q == 8u ? 0u : q;
  uint32_t code = ((uint32_t)(e + 7) << 3) | q;
  code = code > 0x7Eu ? 0x7Eu : code;
  return y < 0.015625f ? sub : code;
}
__device__ __forceinline__ float e4m3_decode_mag(uint32_t c) {
  uint32_t e = (c >> 3) & 0xF, m = c & 7;
  return e == 0 ? (float)m * 0.001953125f : __uint_as_float(((e + 120u) << 23) | (m << 20));
}
// E8M0 exponent X for an E4M3 block with maximum magnitude amax: amax / 2^X in (224, 448].
__device__ __forceinline__ int fp8_block_exp(float amax) {
  if (amax == 0.0f) return 0;
  uint32_t u = __float_as_uint(amax);
  int E = (int)((u >> 23) & 0xFF);
  int e = E == 0 ? -127 : E - 127;
  int X = (u & 0x7FFFFFu) > 0x600000u ? e - 7 : e - 8;
  return X < -127 ? -127 : (X > 127 ? 127 : X);
}
__device__ __forceinline__ float exp2i(int X) {   // 2^X for -127 <= X <= 127, exact
  return X >= -126 ? __uint_as_float((uint32_t)(X + 127) << 23) : __uint_as_float(0x00400000u);
}
// Signed E4M3 code of v / 2^X (positive zero for a zero magnitude); writes the residual v - code * 2^X, computed
// as one fused multiply-add: the difference is exact and the product, which can pass the fp32 range for the
// largest blocks (448 * 2^120), is never rounded on its own.
// A non-finite v (NaN or +-inf; E4M3 has no infinity) gets the E4M3 NaN code 0x7F and a NaN residual, as the
// hardware conversion gives, so every product of its row is NaN.
__device__ __forceinline__ uint32_t e4m3_encode(float v, int X, float* res) {
  float inv = exp2i(-X);        // exact when -X in range; X >= -127 so -X <= 127
  float y = fabsf(v) * inv;
  uint32_t mag = e4m3_mag_code(y);
  float dm = e4m3_decode_mag(mag);
  uint32_t sgn = (mag != 0u && v < 0.0f) ? 0x80u : 0u;
  const bool finite = fabsf(v) <= 3.40282347e38f;
  const float r = __builtin_fmaf(sgn ? dm : -dm, exp2i(X), v);
  *res = finite ? r : __uint_as_float(0x7FC00000u);
  return finite ? (mag | sgn) : 0x7Fu;
}

// Two E4M3 codes (bits 0-7 and 8-15) of values already divided by their block scale (|y| <= 448) from the
// hardware conversion (OCP E4M3, round to nearest even, checked against the oracle on every bf16 input), with
// the sign of zero codes cleared: the codes e4m3_encode gives.
__device__ __forceinline__ uint32_t e4m3_pack2(float y0, float y1) {
  const uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y0, y1, 0, false) & 0xFFFFu;
  const uint32_t t = w & 0x7F7Fu;
  return t | (w & ((t + 0x7F7Fu) & 0x8080u));   // bit 7 of each byte kept only where the magnitude is nonzero
}
typedef float v2f __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v2f e4m3_unpack2(uint32_t w) { return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false); }

// ------------------------------------------------------------------ the specified sigmoid
// exp(x) for |x| <= 200: Cody-Waite reduction by ln 2 (fdlibm split) and a degree-13 Taylor polynomial in
// Horner form, every step one correctly rounded IEEE double operation (no contraction), so the result is
// reproducible bit for bit on any IEEE platform that evaluates the same sequence.
__device__ __forceinline__ double exp_spec(double x) {
#pragma clang fp contract(off)
  const double LN2_HI = 0x1.62e42feep-1;
  const double LN2_LO = 0x1.a39ef35793c76p-33;
  const double INV_LN2 = 0x1.71547652b82fep+0;
  double n = __builtin_rint(x * INV_LN2);
  double r = (x - n * LN2_HI) - n * LN2_LO;
  double p = 1.0 / 6227020800.0;             // 1/13!
  p = p * r + 1.0 / 479001600.0;             // 1/12!
  p = p * r + 1.0 / 39916800.0;
  p = p * r + 1.0 / 3628800.0;
  p = p * r + 1.0 / 362880.0;
  p = p * r + 1.0 / 40320.0;
  p = p * r + 1.0 / 5040.0;
  p = p * r + 1.0 / 720.0;
  p = p * r + 1.0 / 120.0;
  p = p * r + 1.0 / 24.0;
  p = p * r + 1.0 / 6.0;
  p = p * r + 0.5;
  p = p * r + 1.0;
  p = p * r + 1.0;
  return __builtin_ldexp(p, (int)n);
}
// fp32 sigmoid = fp32(1 / (1 + exp_spec(-x))), input clamped to [-200, 200]; NaN -> canonical quiet NaN.
// Branch-free, so that independent evaluations interleave.
__device__ __forceinline__ float sigmoid_spec(float xf) {
#pragma clang fp contract(off)
  const bool nan = xf != xf;
  double x = nan ? 0.0 : (double)xf;
  x = x < -200.0 ? -200.0 : x;
  x = x > 200.0 ? 200.0 : x;
  const double e = exp_spec(-x);
  float s = (float)(1.0 / (1.0 + e));
  asm volatile("" : "+v"(s));   // evaluated for every lane: keeps the compiler from branching around it
  return nan ? __uint_as_float(0x7FC00000u) : s;
}

// 32 bf16-valued floats -> hi / lo E4M3 words (4 codes per word, element order) and E8M0 bytes: hi = E4M3 block
// quantisation of v, lo = the same of the exact residual v - hi.  Codes from the hardware conversion
// (v_cvt_pk_fp8_f32: OCP E4M3, round to nearest even, checked against e4m3_encode on every bf16 input;
// e4m3_pack2 clears the sign of zero codes); the scalings by 2^-X and 2^-Y are exact, and the residual is one
// fused multiply-add (exact, with no overflow of the product for the largest blocks).
__device__ __forceinline__ void quant_block_fp8_hilo(const float* v, uint32_t* hw, uint32_t* lw, uint8_t* hsb,
                                                        uint8_t* lsb) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  const int X = fp8_block_exp(amax);
  const float sx = exp2i(-X), dx = exp2i(X);
  float r[32];
  float ramax = 0.0f;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const uint32_t c01 = e4m3_pack2(v[4 * w] * sx, v[4 * w + 1] * sx);
    const uint32_t c23 = e4m3_pack2(v[4 * w + 2] * sx, v[4 * w + 3] * sx);
    hw[w] = c01 | (c23 << 16);
    const v2f d01 = e4m3_unpack2(c01), d23 = e4m3_unpack2(c23);
    r[4 * w] = __builtin_fmaf(-d01.x, dx, v[4 * w]);          // exact residuals, no overflow of the product
    r[4 * w + 1] = __builtin_fmaf(-d01.y, dx, v[4 * w + 1]);
    r[4 * w + 2] = __builtin_fmaf(-d23.x, dx, v[4 * w + 2]);
    r[4 * w + 3] = __builtin_fmaf(-d23.y, dx, v[4 * w + 3]);
#pragma unroll
    for (int j = 0; j < 4; ++j) ramax = fmaxf(ramax, fabsf(r[4 * w + j]));
  }
  const int Y = fp8_block_exp(ramax);
  const float sy = exp2i(-Y);
#pragma unroll
  for (int w = 0; w < 8; ++w)
    lw[w] = e4m3_pack2(r[4 * w] * sy, r[4 * w + 1] * sy) | (e4m3_pack2(r[4 * w + 2] * sy, r[4 * w + 3] * sy) << 16);
  *hsb = (uint8_t)(X + 127);
  *lsb = (uint8_t)(Y + 127);
}

// The same split of a 32-value block held by two adjacent lanes (lane pair l, l ^ 1: values 16 (l & 1) .. of the
// block), 16 bf16 values per lane packed two per word (element 2 j in the low half of p[j]).  Every lane of the
// wave calls it (the block maxima are exchanged between the pair); per element the operations are those of
// quant_block_fp8_hilo, so the codes and exponents are the same.  hw, lw: 4 words of codes each; X, Y: the
// block's hi and lo exponents (E8M0 byte = exponent + 127).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ void quant_pair_fp8_hilo(const uint32_t (&p)[8], uint32_t (&hw)[4], uint32_t (&lw)[4],
                                                    int* Xo, int* Yo) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(p[j])), fabsf(bf16_hi(p[j]))));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  const int X = fp8_block_exp(amax);
  const float sx = exp2i(-X), dx = exp2i(X);
  float ramax = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float v0 = bf16_lo(p[2 * w]), v1 = bf16_hi(p[2 * w]), v2 = bf16_lo(p[2 * w + 1]), v3 = bf16_hi(p[2 * w + 1]);
    const uint32_t c01 = e4m3_pack2(v0 * sx, v1 * sx);
    const uint32_t c23 = e4m3_pack2(v2 * sx, v3 * sx);
    hw[w] = c01 | (c23 << 16);
    const v2f d01 = e4m3_unpack2(c01), d23 = e4m3_unpack2(c23);
    ramax = fmaxf(ramax, fabsf(__builtin_fmaf(-d01.x, dx, v0)));
    ramax = fmaxf(ramax, fabsf(__builtin_fmaf(-d01.y, dx, v1)));
    ramax = fmaxf(ramax, fabsf(__builtin_fmaf(-d23.x, dx, v2)));
    ramax = fmaxf(ramax, fabsf(__builtin_fmaf(-d23.y, dx, v3)));
  }
  ramax = fmaxf(ramax, __shfl_xor(ramax, 1, 64));
  const int Y = fp8_block_exp(ramax);
  const float sy = exp2i(-Y);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float v0 = bf16_lo(p[2 * w]), v1 = bf16_hi(p[2 * w]), v2 = bf16_lo(p[2 * w + 1]), v3 = bf16_hi(p[2 * w + 1]);
    const v2f d01 = e4m3_unpack2(hw[w] & 0xFFFFu), d23 = e4m3_unpack2(hw[w] >> 16);
    const float r0 = __builtin_fmaf(-d01.x, dx, v0), r1 = __builtin_fmaf(-d01.y, dx, v1);
    const float r2 = __builtin_fmaf(-d23.x, dx, v2), r3 = __builtin_fmaf(-d23.y, dx, v3);
    lw[w] = e4m3_pack2(r0 * sy, r1 * sy) | (e4m3_pack2(r2 * sy, r3 * sy) << 16);
  }
  *Xo = X;
  *Yo = Y;
}

// ------------------------------------------------------------------ wave reductions (wave64)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}
// max over groups of `width` consecutive lanes (width a power of two <= 64)
__device__ __forceinline__ float group_max(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// max over each group of 8 consecutive lanes through DPP (xor 1, xor 2 within quads, then the half-row mirror)
__device__ __forceinline__ float dpp_group_max8(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x141, 0xF, 0xF, false)));
  return v;
}

// max over each group of 16 consecutive lanes (a DPP row): the 8-lane steps, then the row mirror
__device__ __forceinline__ float dpp_group_max16(float v) {
  v = dpp_group_max8(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x140, 0xF, 0xF, false)));
  return v;
}

// wave64 sum through DPP row operations (xor 1, xor 2, half-row and row mirrors, then row_bcast15 / 31 into
// rows 1-3); the total is read from lane 63 and returned to every lane
__device__ __forceinline__ float dpp_sum_f32(float v) {
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// wave64 max / min of a uint32 through DPP row operations (xor 1, xor 2, half-row and row mirrors, then the
// row_bcast15 / row_bcast31 steps across rows); every lane receives the result read from lane 63.
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t dpp_min_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// order-preserving map of an fp32 key to uint32 (NaN lowest, -0 treated as +0)
__device__ __forceinline__ uint32_t key_to_ordered(float k) {
  const uint32_t u = __float_as_uint(k == 0.0f ? 0.0f : k);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return k != k ? 0u : o;
}

// ------------------------------------------------------------------ global -> LDS copies
// global_load_lds: lane l's 16 (or 4) bytes at gbase + voff land at lds_dst + 16 l (or 4 l), without passing
// through registers.  gbase and lds_dst must be wave-uniform (they go to SGPRs and M0).  Issued from inline
// assembly so that the compiler's wait-counter bookkeeping does not pin the address registers (it would wait
// for every outstanding load before reusing them); the caller waits with wait_vm_all() before any wave reads
// the data.  M0 is only a launch-time scratch register on gfx950 (ordinary LDS instructions do not use it).
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
// The LDS byte offset of a pointer into LDS: the low 32 bits of its generic address (the LDS aperture puts the
// offset there).  No address-space cast: its null check, folded against the aperture base in divergent code,
// made the gfx950 backend emit an invalid compare.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
// The base address operands of these copies are SGPRs that are often written by v_readfirstlane just before
// the asm; a VMEM instruction reading an SGPR that a VALU instruction wrote needs 5 wait states, which the
// compiler does not supply inside inline assembly: each asm starts with them (s_nop 4 = 5 wait states).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"     // M0 is declared clobbered on purpose
__device__ __forceinline__ void lds_copy16(const void* gbase, uint32_t voff, const void* lds_dst) {
  const uint64_t b = uniform_u64((uint64_t)gbase);
  const uint32_t m = lds_addr(lds_dst);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(b), "s"(m)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void* gbase, uint32_t voff, const void* lds_dst) {
  const uint64_t b = uniform_u64((uint64_t)gbase);
  const uint32_t m = lds_addr(lds_dst);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(b), "s"(m)
               : "memory", "m0");
}
// 16 bytes per lane global -> VGPRs, not tracked by the compiler's wait counting: the caller waits for it with
// an explicit s_waitcnt before any use (and pins the use below that wait)
__device__ __forceinline__ void gload16(v4i& dst, const void* gbase, uint32_t voff) {
  const uint64_t b = uniform_u64((uint64_t)gbase);
  asm volatile("s_nop 4\n\tglobal_load_dwordx4 %0, %1, %2" : "=v"(dst) : "v"(voff), "s"(b) : "memory");
}
#pragma clang diagnostic pop
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): every global load of the wave has landed,
// including the global -> LDS copies above
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt vmcnt(N): at most the N most recent vector memory loads still in flight (loads, including the LDS
// copies above, complete in issue order, so everything issued before them has landed)
template <int N>
__device__ __forceinline__ void wait_vm_keep() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}

// ------------------------------------------------------------------ MFMA result reads
// The block-scaled fp8 x fp4 MFMA (v_mfma_scale_f32_16x16x128_f8f6f4 with an E4M3 A operand) runs 16 passes, but
// the compiler pads a read of its result as if it took fewer: an epilogue that read the accumulator 12 wait
// states after the last MFMA got values the MFMA had not finished writing (found on MI355X in a kernel whose
// second MFMA was followed by a short epilogue).  Placed after a chain of these MFMAs and before anything reads
// the accumulators, this waits 20 states and keeps the scheduler from moving instructions across it.
__device__ __forceinline__ void mfma_f8f4_settle() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// ------------------------------------------------------------------ misc
__device__ __forceinline__ uint32_t load_u8x4(const uint8_t* p) { return *(const uint32_t*)p; }

}  // namespace mimo
