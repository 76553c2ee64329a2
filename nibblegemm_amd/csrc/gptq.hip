// GPTQ's column loop for one quantisation group, on the GPU.
//
// Reference: python/nibblegemm/gptq.py:65-134 (gptq_quantize), after Frantar
// et al., "GPTQ: Accurate Post-Training Quantization for Generative
// Pre-trained Transformers" (2023).  Within a group of G input channels the
// reference walks the channels in order; for each one it rounds every output
// row's weight with the group's scale, and spreads the row's rounding error
// over the row's later channels through the upper Cholesky factor of H^-1:
//
//   scale_n = max(amax_n(W1) * fp32(1/7), 1e-8);  inv_n = 1 / scale_n
//   for i in 0..G-1:
//     q     = clamp(rint(W1[n, i] * inv_n), -8, 7)
//     err   = (W1[n, i] - q * scale_n) / U[i, i]
//     W1[n, j] -= err * U[i, j]         for j > i
//
// Every output row is independent, so one thread takes one row: the group's
// G x G factor sits in LDS (read as broadcasts), the workgroup's 64 rows in
// LDS (padded rows: conflict-free), and the whole G-step loop runs in one
// launch instead of G small elementwise launches per group.  The arithmetic
// is the reference's op for op, each product and difference rounded on its
// own (no fused multiply-add), the division true, and the scale's division
// by 7 a multiply by fp32(1/7) -- how PyTorch divides a GPU tensor by a
// Python scalar, which is what the reference does where its weights live.
// The update of the channels after the group (a GEMM) stays with the caller.
#include "nibble_common.h"

namespace nibble {

namespace {

constexpr int kGptqRows = 64;  // output rows (threads) per workgroup

template <int G>
__global__ __launch_bounds__(kGptqRows) void gptq_group_kernel(
    const float* __restrict__ W, int64_t ldw, int N, const float* __restrict__ U, int64_t ldu,
    uint8_t* __restrict__ Q, int64_t ldq, float* __restrict__ E, float* __restrict__ scales) {
#pragma clang fp contract(off)
  __shared__ float u[G][G];
  __shared__ float w[kGptqRows][G + 1];
  const int t = threadIdx.x;
  const int row0 = blockIdx.x * kGptqRows;
  for (int e = t; e < G * G; e += kGptqRows) u[e / G][e % G] = U[(e / G) * ldu + e % G];
  for (int e = t; e < kGptqRows * G; e += kGptqRows) {
    const int r = e / G, c = e % G;
    w[r][c] = row0 + r < N ? W[static_cast<size_t>(row0 + r) * ldw + c] : 0.0f;
  }
  __syncthreads();
  const int n = row0 + t;
  if (n >= N) return;
  float amax = 0.0f;
  for (int j = 0; j < G; ++j) amax = fmaxf(amax, fabsf(w[t][j]));
  constexpr float kInv7 = 1.0f / 7.0f;
  const float scale = fmaxf(amax * kInv7, 1e-8f);
  const float inv = 1.0f / scale;
  for (int i = 0; i < G; ++i) {
    const float wi = w[t][i];
    const float q = fminf(fmaxf(rintf(wi * inv), -8.0f), 7.0f);
    const float qs = q * scale;
    const float err = (wi - qs) / u[i][i];
    Q[static_cast<size_t>(n) * ldq + i] = static_cast<uint8_t>(static_cast<int>(q) + 8);
    E[static_cast<size_t>(n) * G + i] = err;
    for (int j = i + 1; j < G; ++j) {
      const float d = err * u[i][j];
      w[t][j] = w[t][j] - d;
    }
  }
  scales[n] = scale;
}

}  // namespace

}  // namespace nibble

using namespace nibble;

extern "C" int nibble_gptq_group_f32(const void* W, int64_t ldw, int64_t N, int64_t G,
                                     const void* U, int64_t ldu, void* Q, int64_t ldq, void* E,
                                     void* scales, void* stream_) {
  NIBBLE_CHECK(G == 64 || G == 128, "group size must be 64 or 128, got %lld", (long long)G);
  NIBBLE_CHECK(N >= 0 && N < (int64_t(1) << 31), "N out of range");
  NIBBLE_CHECK(ldw >= G && ldu >= G && ldq >= G, "leading dimensions must be >= G");
  if (N == 0) return ok();
  NIBBLE_CHECK(W != nullptr && U != nullptr && Q != nullptr && E != nullptr && scales != nullptr,
               "null pointer");
  NIBBLE_CHECK(aligned(W, 4) && aligned(U, 4) && aligned(E, 4) && aligned(scales, 4),
               "fp32 operands must be 4-byte aligned");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  const dim3 grid(static_cast<unsigned>(ceil_div(N, kGptqRows)));
  const auto* w = static_cast<const float*>(W);
  const auto* u = static_cast<const float*>(U);
  auto* q = static_cast<uint8_t*>(Q);
  auto* e = static_cast<float*>(E);
  auto* s = static_cast<float*>(scales);
  if (G == 128)
    gptq_group_kernel<128><<<grid, kGptqRows, 0, stream>>>(w, ldw, static_cast<int>(N), u, ldu, q,
                                                           ldq, e, s);
  else
    gptq_group_kernel<64><<<grid, kGptqRows, 0, stream>>>(w, ldw, static_cast<int>(N), u, ldu, q,
                                                          ldq, e, s);
  NIBBLE_HIP(hipGetLastError());
  return ok();
}
