// The MoE half of a decoder layer around the block (engine/mimo_stream/model.py:296-340):
//   r = post_attention_layernorm(x)          (:299, nn.RMSNorm with the checkpoint's layernorm_epsilon, :75)
//   routes and experts on r                  (:300-336, the router / decode / prefill entry points)
//   h = x + y                                (:340)
// This file holds the RMSNorm kernel and the standalone residual add; the fused layer entry points (norm, block,
// residual in the combine kernels) sit with the decode and prefill paths.
//
// RMSNorm rounding points (one row per 256-thread block, H = 256 n):
//   ss  = fp32 sum of x^2 (a bf16 square is exact in fp32): thread t adds x[t + 256 j]^2 for j = 0, 1, ... in
//         order; each wave's 64 partials combine by a butterfly (xor 32, 16, 8, 4, 2, 1); the 4 wave sums as
//         (s0 + s1) + (s2 + s3)
//   inv = 1 / sqrt(ss / H + eps)             (IEEE fp32 division and square root)
//   r_j = bf16(w_j * bf16(x_j * inv))        (normalise, round, scale: the w product is exact in fp32)
// mlx.core.fast.rms_norm (the reference's nn.RMSNorm) applies the same rounding points with its own fp32 sum
// order, so the two agree to within a bf16 rounding flip where inv differs in its last bits.
#include "device.h"
#include "host.h"
#include "layer.h"

namespace mimo {

constexpr int kNormMaxPer = 32;   // bf16 elements per thread: H <= 8192

// PER >= H / 256 elements per thread; every load is issued before any is used (indices past the row repeat the
// thread's first element), so the row arrives in one round trip.
template <int PER>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x, int H,
                                                      const uint16_t* __restrict__ w, float eps,
                                                      uint16_t* __restrict__ r) {
#pragma clang fp contract(off)
  __shared__ float wsum[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint16_t* xr = x + (size_t)blockIdx.x * H;
  uint16_t* rr = r + (size_t)blockIdx.x * H;
  const int n = H >> 8;
  uint16_t xb[PER], wb[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = t + 256 * (j < n ? j : 0);
    xb[j] = xr[e];
    wb[j] = w[e];
  }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float v = bf16_to_f32(xb[j]);
    ss = j < n ? ss + v * v : ss;
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) ss = ss + __shfl_xor(ss, s, 64);
  if (lane == 0) wsum[wave] = ss;
  __syncthreads();
  const float tot = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (j < n) {
      const float nv = bf16_to_f32(f32_to_bf16(bf16_to_f32(xb[j]) * inv));
      rr[t + 256 * j] = f32_to_bf16(bf16_to_f32(wb[j]) * nv);
    }
  }
}

// h = bf16(x + y), 8 elements per thread (n a multiple of 8, 16-byte aligned rows) or one per thread otherwise.
__global__ void __launch_bounds__(256) residual_add_kernel(const uint16_t* x, const uint16_t* y, int64_t n, uint16_t* h) {
#pragma clang fp contract(off)
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i + 8 <= n) {
    const uint4 a = *reinterpret_cast<const uint4*>(x + i);
    const uint4 b = *reinterpret_cast<const uint4*>(y + i);
    const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint16_t lo = residual_bf16((uint16_t)av[q], (uint16_t)bv[q]);
      const uint16_t hi = residual_bf16((uint16_t)(av[q] >> 16), (uint16_t)(bv[q] >> 16));
      o[q] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<uint4*>(h + i) = make_uint4(o[0], o[1], o[2], o[3]);
  } else {
    for (int64_t e = i; e < n && e < i + 8; ++e) h[e] = residual_bf16(x[e], y[e]);
  }
}

int launch_rmsnorm(const uint16_t* x, int T, int H, const uint16_t* w, float eps, uint16_t* r, hipStream_t st) {
  MIMO_REQUIRE(x && w && r, MIMO_ERR_ARG, "rmsnorm: null pointer");
  MIMO_REQUIRE(T >= 1 && H >= 256 && H % 256 == 0 && H <= 256 * kNormMaxPer, MIMO_ERR_SHAPE,
               "rmsnorm: need T >= 1 and H a multiple of 256 up to %d (got T=%d H=%d)", 256 * kNormMaxPer, T, H);
  MIMO_REQUIRE(eps >= 0.0f && eps == eps, MIMO_ERR_ARG, "rmsnorm: eps must be a non-negative number");
  const int n = H / 256;
  {
    ProfScope p(st, "rmsnorm");
    if (n <= 1) rmsnorm_kernel<1><<<T, 256, 0, st>>>(x, H, w, eps, r);
    else if (n <= 2) rmsnorm_kernel<2><<<T, 256, 0, st>>>(x, H, w, eps, r);
    else if (n <= 4) rmsnorm_kernel<4><<<T, 256, 0, st>>>(x, H, w, eps, r);
    else if (n <= 8) rmsnorm_kernel<8><<<T, 256, 0, st>>>(x, H, w, eps, r);
    else if (n <= 16) rmsnorm_kernel<16><<<T, 256, 0, st>>>(x, H, w, eps, r);
    else rmsnorm_kernel<32><<<T, 256, 0, st>>>(x, H, w, eps, r);
  }
  return check_launch("rmsnorm");
}

}  // namespace mimo

using namespace mimo;

extern "C" {

int mimo_rmsnorm(const uint16_t* x, int T, int H, const uint16_t* w, float eps, uint16_t* r, void* stream) {
  MIMO_REQUIRE(x != r, MIMO_ERR_ARG, "rmsnorm: r may not alias x");
  return launch_rmsnorm(x, T, H, w, eps, r, as_stream(stream));
}

int mimo_residual_add(const uint16_t* x, const uint16_t* y, int64_t n, uint16_t* h, void* stream) {
  MIMO_REQUIRE(x && y && h, MIMO_ERR_ARG, "residual_add: null pointer");
  MIMO_REQUIRE(n >= 0, MIMO_ERR_SHAPE, "residual_add: n must be >= 0");
  MIMO_REQUIRE(aligned16(x) && aligned16(y) && aligned16(h), MIMO_ERR_ALIGN, "residual_add: 16-byte alignment");
  if (n == 0) return MIMO_OK;
  const int64_t blocks = (n + 2047) / 2048;
  MIMO_REQUIRE(blocks < (1ll << 31), MIMO_ERR_SHAPE, "residual_add: n too large");
  residual_add_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(x, y, n, h);
  return check_launch("residual_add");
}

}  // extern "C"
