// The MoE half of a decoder layer around the block (engine/mimo_stream/model.py:296-340):
//   r = post_attention_layernorm(x)          (:299, nn.RMSNorm with the checkpoint's layernorm_epsilon, :75)
//   routes and experts on r                  (:300-336, the router / decode / prefill entry points)
//   h = x + y                                (:340)
// This file holds the RMSNorm kernel and the standalone residual add; the fused layer entry points (norm, block,
// residual in the combine kernels) sit with the decode and prefill paths.
//
// RMSNorm: the rounding points and the fp32 summation order are those of layer.h (norm_*).  mlx.core.fast.rms_norm
// (the reference's nn.RMSNorm) applies the same rounding points with its own fp32 sum order, so the two agree to
// within a bf16 rounding flip where inv differs in its last bits.
#include "device.h"
#include "host.h"
#include "layer.h"

namespace mimo {

// One row per 256-thread block; NCH = ceil(H / 2048) chunks of 8 elements per thread, all loaded before any is used
// (a thread's empty chunks re-read its wave's first chunk and are not counted), so the row arrives in one round trip.
template <int NCH>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x, int H,
                                                      const uint16_t* __restrict__ w, float eps,
                                                      uint16_t* __restrict__ r) {
  __shared__ float wsum[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q4 = H >> 2;
  const size_t rowq = (size_t)blockIdx.x * H + wave * q4;
  uint4 xv[NCH], wv[NCH];
  bool ok[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int off = c * 512 + 8 * lane;
    ok[c] = off < q4;
    const int o = ok[c] ? off : 0;
    xv[c] = *reinterpret_cast<const uint4*>(x + rowq + o);
    wv[c] = *reinterpret_cast<const uint4*>(w + wave * q4 + o);
  }
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) ss = ok[c] ? norm_sq_add8(xv[c], ss) : ss;
  ss = norm_wave_sum(ss);
  if (lane == 0) wsum[wave] = ss;
  __syncthreads();
  const float inv = norm_inv(wsum, H, eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (ok[c]) *reinterpret_cast<uint4*>(r + rowq + c * 512 + 8 * lane) = norm_apply8(xv[c], wv[c], inv);
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
  MIMO_REQUIRE(T >= 1 && H >= 256 && H % 256 == 0 && H <= 8192, MIMO_ERR_SHAPE,
               "rmsnorm: need T >= 1 and H a multiple of 256 up to 8192 (got T=%d H=%d)", T, H);
  MIMO_REQUIRE(aligned16(x) && aligned16(w) && aligned16(r), MIMO_ERR_ALIGN, "rmsnorm: 16-byte alignment");
  MIMO_REQUIRE(eps >= 0.0f && eps == eps, MIMO_ERR_ARG, "rmsnorm: eps must be a non-negative number");
  const int nch = (H / 4 + 511) / 512;
  {
    ProfScope p(st, "rmsnorm");
    switch (nch) {
      case 1: rmsnorm_kernel<1><<<T, 256, 0, st>>>(x, H, w, eps, r); break;
      case 2: rmsnorm_kernel<2><<<T, 256, 0, st>>>(x, H, w, eps, r); break;
      case 3: rmsnorm_kernel<3><<<T, 256, 0, st>>>(x, H, w, eps, r); break;
      default: rmsnorm_kernel<4><<<T, 256, 0, st>>>(x, H, w, eps, r); break;
    }
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
