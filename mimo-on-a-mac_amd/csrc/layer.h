// The decoder-layer pieces around the MoE block: the post-attention RMSNorm and the residual add.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.h"

namespace mimo {

// r = RMSNorm(x) * w, rows of H bf16 (H a multiple of 256, at most 8192); r may not alias x.
int launch_rmsnorm(const uint16_t* x, int T, int H, const uint16_t* w, float eps, uint16_t* r, hipStream_t st);

// h = bf16(x + y) for bf16 x and y (the residual of a decoder layer): one fp32 addition, rounded to nearest even.
__device__ __forceinline__ uint16_t residual_bf16(uint16_t x, uint16_t y) {
  return f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(y));
}

}  // namespace mimo
