// Fixed-order reductions shared by the kernels that must agree bit for bit:
// the RMSNorm kernel and the GEMV's fused-RMSNorm prologue compute the same
// row scale with the same instructions in the same order.
#pragma once

#include "nibble_decode.h"

namespace nibble {

// Cross-lane reductions on DPP moves (VALU latency, no LDS round trip).
// Within each 16-lane row: partners lane ^ 1, lane ^ 2 (quad permutes), then
// the mirrored lane of the 8-lane half and of the row, so after four steps
// every lane of the row holds the row's total -- the same bits in every lane,
// since each step adds the same two values in either lane.  A wave's total
// adds its four row totals in row order (readlane).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each 16 lanes

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return ((lane_value(v, 0) + lane_value(v, 16)) + lane_value(v, 32)) + lane_value(v, 48);
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Sum over a 256-thread workgroup (4 waves) of one value per thread: each
// wave's total, then the four in wave order.  `part` is 4 floats of LDS.
// Callers that reuse `part` place a barrier before its next write.
__device__ __forceinline__ float block256_sum(float v, float* part) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((part[0] + part[1]) + part[2]) + part[3];
}

// RMSNorm of a row held as 16-byte chunks: chunk c of thread t covers columns
// (256 c + t) * 8 .. + 7.  The squares are accumulated chunk by chunk, element
// by element, with fma; the scale is 1 / sqrt(total / cols + eps).
constexpr int kRmsThreads = 256;

__device__ __forceinline__ float sumsq_chunk(h8_t v, float ss) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float f = static_cast<float>(v[i]);
    ss = __builtin_fmaf(f, f, ss);
  }
  return ss;
}

__device__ __forceinline__ float rms_scale(float total, int cols, float eps) {
  return 1.0f / sqrtf(total / static_cast<float>(cols) + eps);
}

// fp16(x * r * w): the normalised, weighted value, rounded once.
__device__ __forceinline__ h8_t rms_apply(h8_t x, h8_t w, float r) {
  h8_t y;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    y[i] = static_cast<_Float16>(static_cast<float>(x[i]) * r * static_cast<float>(w[i]));
  return y;
}

}  // namespace nibble
