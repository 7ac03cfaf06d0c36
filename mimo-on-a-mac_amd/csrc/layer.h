// The decoder-layer pieces around the MoE block: the post-attention RMSNorm and the residual add.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.h"

namespace mimo {

// r = RMSNorm(x) * w, rows of H bf16 (H a multiple of 256, at most 8192, 16-byte aligned); r may not alias x.
int launch_rmsnorm(const uint16_t* x, int T, int H, const uint16_t* w, float eps, uint16_t* r, hipStream_t st);

// RMSNorm arithmetic shared by the norm kernel and the decode router kernel, which normalises its rows itself.
// In a 256-thread block, thread (wave w, lane l) owns the 8-element chunks of a row that start at
// w H/4 + 512 c + 8 l for c = 0, 1, ... (chunks at or past (w + 1) H/4 are empty).  Rounding points:
//   ss  = fp32 sum of x^2 (a bf16 square is exact in fp32): each thread adds the squares of its chunks in
//         (chunk, element) order; each wave's 64 partials combine by a butterfly (xor 32, 16, 8, 4, 2, 1); the
//         4 wave sums as (s0 + s1) + (s2 + s3)
//   inv = 1 / sqrt(ss / H + eps)             (IEEE fp32 division and square root)
//   r_j = bf16(w_j * bf16(x_j * inv))        (normalise, round, scale: the w product is exact in fp32)

// ss + x_0^2 + ... + x_7^2 over the 8 bf16 of v in element order
__device__ __forceinline__ float norm_sq_add8(uint4 v, float ss) {
#pragma clang fp contract(off)
  const uint32_t p[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float lo = __uint_as_float(p[q] << 16), hi = __uint_as_float(p[q] & 0xFFFF0000u);
    ss = ss + lo * lo;
    ss = ss + hi * hi;
  }
  return ss;
}

// the wave's butterfly sum (every lane ends with the same value: fp32 addition is commutative)
__device__ __forceinline__ float norm_wave_sum(float ss) {
#pragma clang fp contract(off)
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) ss = ss + __shfl_xor(ss, s, 64);
  return ss;
}

__device__ __forceinline__ float norm_inv(const float* wsum4, int H, float eps) {
#pragma clang fp contract(off)
  const float tot = (wsum4[0] + wsum4[1]) + (wsum4[2] + wsum4[3]);
  return 1.0f / sqrtf(tot / (float)H + eps);
}

// r for the 8 bf16 of x with weights w
__device__ __forceinline__ uint4 norm_apply8(uint4 x, uint4 w, float inv) {
#pragma clang fp contract(off)
  const uint32_t xp[4] = {x.x, x.y, x.z, x.w}, wp[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float nlo = round_bf16(__uint_as_float(xp[q] << 16) * inv);
    const float nhi = round_bf16(__uint_as_float(xp[q] & 0xFFFF0000u) * inv);
    const uint16_t rlo = f32_to_bf16(__uint_as_float(wp[q] << 16) * nlo);
    const uint16_t rhi = f32_to_bf16(__uint_as_float(wp[q] & 0xFFFF0000u) * nhi);
    o[q] = (uint32_t)rlo | ((uint32_t)rhi << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ uint16_t norm_apply1(uint16_t x, uint16_t w, float inv) {
#pragma clang fp contract(off)
  return f32_to_bf16(bf16_to_f32(w) * round_bf16(bf16_to_f32(x) * inv));
}

// h = bf16(x + y) for bf16 x and y (the residual of a decoder layer): one fp32 addition, rounded to nearest even.
__device__ __forceinline__ uint16_t residual_bf16(uint16_t x, uint16_t y) {
  return f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(y));
}

}  // namespace mimo
