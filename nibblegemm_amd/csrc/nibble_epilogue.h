// Output epilogues of the weight-streaming kernels: fused forms of what a
// caller would otherwise run as separate elementwise ops on the fp16 product.
// Shared by the decode GEMV (gemv.hip) and the persistent decode chain
// (chain.hip), which must give the same bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace nibble {

constexpr int kEpilogueNone = 0;
constexpr int kEpilogueBias = 1;    // Y = fp16(fp16(X W) + bias)
constexpr int kEpilogueSwiglu = 2;  // W = [gate | up] in 16-column blocks; Y = silu(G) * U
constexpr int kSwigluBlock = 16;    // columns of one gate or up block of that layout

// The fp16 arithmetic of the unfused composition, step by step: the two
// products rounded to fp16, silu(g) = g / (1 + e^-g) evaluated in fp32 and
// rounded, then the fp32 product of the two fp16 values (rounded at the
// store).
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float g16 = static_cast<float>(static_cast<_Float16>(g));
  const float u16 = static_cast<float>(static_cast<_Float16>(u));
  const float s16 = static_cast<float>(static_cast<_Float16>(g16 / (1.0f + expf(-g16))));
  return s16 * u16;
}

}  // namespace nibble
