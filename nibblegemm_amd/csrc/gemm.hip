// Prefill-regime W4A16 matmul on CDNA4 MFMA: Y[M,N] = X[M,K] @ dequant(Wq, S).
//
// Reference: csrc/gemm_w4a16.cu (tile staging :66-146, kernels :151-377, host
// checks :379-429).  The reference decodes B into shared memory and feeds
// wmma / mma.sync; here the tile is fed to v_mfma_f32_16x16x32_f16.
//
// Tile: BM x BN x 32 per workgroup of 4 wave64s (2 x 2), each wave owning a
// (BM/2) x (BN/2) block of 16 x 16 MFMA tiles.  Per K step:
//   * A (X, fp16) rows are copied global -> LDS with 16-byte loads, rows past
//     M zero-filled;
//   * B: every packed word is exactly 8 consecutive k of one column, i.e. one
//     MFMA B-operand lane's worth.  Words are loaded a K step ahead into
//     registers, decoded with the magic-exponent trick, multiplied by the group
//     scale (one RNE rounding, so the LDS tile holds exactly dequantize()'s fp16
//     values) and stored n-major (k contiguous) with one 16-byte store;
//   * each wave reads its A and B operands with ds_read_b128 and issues
//     (BM/32) x (BN/32) MFMAs with fp32 accumulation.
// The epilogue converts to fp16 and stores with row/column masks.
//
// MFMA operand layout (16x16x32 f16): lane l supplies row (A) / column (B)
// l % 16 and the 8 k of block l / 16; the f32 result tile gives lane l column
// l % 16 and rows 4 * (l / 16) + {0,1,2,3}.
#include <algorithm>

#include "nibble_common.h"
#include "nibble_decode.h"
#include "stream_matmul.h"

namespace nibble {

namespace {

constexpr int BK = 32;
constexpr int kPad = 8;           // fp16 elements of padding per LDS row
constexpr int LDK = BK + kPad;    // LDS row pitch in fp16 elements
constexpr int kGemmThreads = 256; // 4 waves as 2 x 2

template <int BM, int BN>
struct TileCfg {
  static constexpr int WM = BM / 2, WN = BN / 2;     // wave tile
  static constexpr int FM = WM / 16, FN = WN / 16;   // MFMA tiles per wave
  static constexpr int A_CHUNKS = BM * (BK / 8);     // 16-byte chunks of A per K step
  static constexpr int A_ITERS = A_CHUNKS / kGemmThreads;
  static constexpr int B_WORDS = BN * (BK / 8);      // packed words of B per K step
  static constexpr int B_ITERS = B_WORDS / kGemmThreads;
  static_assert(A_CHUNKS % kGemmThreads == 0, "A tile must split evenly");
  static_assert(B_WORDS % kGemmThreads == 0, "B tile must split evenly");
};

template <int BM, int BN, int GROUP>
__global__ __launch_bounds__(kGemmThreads) void gemm_mfma_kernel(const _Float16* __restrict__ X,
                                                                 const uint32_t* __restrict__ Wq,
                                                                 const _Float16* __restrict__ S,
                                                                 _Float16* __restrict__ Y, int M,
                                                                 int K, int N) {
  using C = TileCfg<BM, BN>;
  __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * C::WM;
  const int wn = (wave & 1) * C::WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;

  f4_t acc[C::FM][C::FN];
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // B prefetch registers: word and scale for each (packed row, column) this
  // thread stages.  Element e = tid + it * threads: r8 = e / BN, c = e % BN.
  uint32_t bq[C::B_ITERS];
  _Float16 bs[C::B_ITERS];
  auto prefetch_b = [&](int k0) {
#pragma unroll
    for (int it = 0; it < C::B_ITERS; ++it) {
      const int e = tid + it * kGemmThreads;
      const int r8 = e / BN, c = e % BN;
      const int n = n0 + c;
      const bool ok = n < N;
      bq[it] = ok ? Wq[static_cast<size_t>(k0 / 8 + r8) * N + n] : 0u;
      bs[it] = ok ? S[static_cast<size_t>((k0 + r8 * 8) / GROUP) * N + n] : (_Float16)0.0f;
    }
  };
  auto commit_b = [&]() {
#pragma unroll
    for (int it = 0; it < C::B_ITERS; ++it) {
      const int e = tid + it * kGemmThreads;
      const int r8 = e / BN, c = e % BN;
      h2_t w[4];
      const h2_t s2 = {bs[it], bs[it]};
      decode8_scaled(bq[it], s2, w);
      h8_t v = {w[0][0], w[0][1], w[1][0], w[1][1], w[2][0], w[2][1], w[3][0], w[3][1]};
      *reinterpret_cast<h8_t*>(&Bs[c * LDK + r8 * 8]) = v;
    }
  };
  auto load_a = [&](int k0) {
#pragma unroll
    for (int it = 0; it < C::A_ITERS; ++it) {
      const int e = tid + it * kGemmThreads;
      const int row = e / (BK / 8), col = (e % (BK / 8)) * 8;
      const int gm = m0 + row;
      h8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (gm < M) v = *reinterpret_cast<const h8_t*>(X + static_cast<size_t>(gm) * K + k0 + col);
      *reinterpret_cast<h8_t*>(&As[row * LDK + col]) = v;
    }
  };

  const int ntiles = K / BK;
  prefetch_b(0);
  for (int t = 0; t < ntiles; ++t) {
    load_a(t * BK);
    commit_b();
    if (t + 1 < ntiles) prefetch_b((t + 1) * BK);
    __syncthreads();

    const int kb = (lane >> 4) * 8;
    const int r = lane & 15;
    h8_t a[C::FM], b[C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
      a[i] = *reinterpret_cast<const h8_t*>(&As[(wm + i * 16 + r) * LDK + kb]);
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
      b[j] = *reinterpret_cast<const h8_t*>(&Bs[(wn + j * 16 + r) * LDK + kb]);
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  // Epilogue: lane l holds column l % 16, rows 4 * (l / 16) + q.
  const int col_in = lane & 15;
  const int row_in = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int gn = n0 + wn + j * 16 + col_in;
      if (gn >= N) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int gm = m0 + wm + i * 16 + row_in + q;
        if (gm < M) Y[static_cast<size_t>(gm) * N + gn] = (_Float16)acc[i][j][q];
      }
    }
  }
}

template <int BM, int BN>
hipError_t launch_tile(const _Float16* x, const uint32_t* w, const _Float16* s, _Float16* y,
                       int64_t M, int64_t K, int64_t N, int64_t G, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(ceil_div(N, BN)), static_cast<unsigned>(ceil_div(M, BM)));
  if (G == 128)
    gemm_mfma_kernel<BM, BN, 128><<<grid, kGemmThreads, 0, stream>>>(x, w, s, y, (int)M, (int)K, (int)N);
  else
    gemm_mfma_kernel<BM, BN, 64><<<grid, kGemmThreads, 0, stream>>>(x, w, s, y, (int)M, (int)K, (int)N);
  return hipGetLastError();
}

}  // namespace

// Mirrors the reference's host checks (csrc/gemm_w4a16.cu:381-400); pure host.
int validate_gemm(const void* X, int64_t x_rows, int64_t x_cols, const void* Wq, int64_t wq_rows,
                  int64_t wq_cols, const void* S, int64_t s_rows, int64_t s_cols, int64_t group_size,
                  int64_t version, const void* Y) {
  NIBBLE_CHECK(x_rows >= 0 && x_cols >= 0 && wq_rows >= 0 && wq_cols >= 0 && s_rows >= 0 &&
                   s_cols >= 0,
               "negative dimension");
  const int64_t M = x_rows, K = x_cols, N = wq_cols;
  NIBBLE_CHECK(wq_rows * 8 == K, "packed weight rows disagree with K");
  NIBBLE_CHECK(K % BK == 0, "K must be a multiple of %d", BK);
  NIBBLE_CHECK(N % 2 == 0, "N must be even");
  NIBBLE_CHECK(group_size == 64 || group_size == 128, "group_size must be 64 or 128");
  NIBBLE_CHECK(s_rows * group_size == K, "scale rows disagree with K/group_size");
  NIBBLE_CHECK(s_cols == N, "scale columns disagree with N");
  NIBBLE_CHECK(version == 6 || version == 7, "gemm version must be 6 or 7, got %lld",
               (long long)version);
  const int64_t lim = int64_t(1) << 31;
  NIBBLE_CHECK(M * N < lim && M * K < lim && K * N < lim,
               "shape too large for 32-bit indexing in the prefill kernel");
  NIBBLE_CHECK(ceil_div(M, 64) < 65536, "M too large");
  // Only operands that hold elements are dereferenced (empty tensors may
  // carry a null data pointer).
  const bool x_used = M * K > 0 && N > 0;
  const bool w_used = K * N > 0 && M > 0;
  const bool y_used = M * N > 0;
  NIBBLE_CHECK((!x_used || X != nullptr) && (!w_used || (Wq != nullptr && S != nullptr)) &&
                   (!y_used || Y != nullptr),
               "null pointer");
  NIBBLE_CHECK((!x_used || aligned(X, 16)) && (!w_used || (aligned(Wq, 4) && aligned(S, 2))) &&
                   (!y_used || aligned(Y, 2)),
               "misaligned pointer (X needs 16-byte alignment)");
  return NIBBLE_OK;
}

}  // namespace nibble

using namespace nibble;

namespace {
// Small batches go to the weight-streaming kernel: each weight byte is read
// once and multiplied against all M rows (one or two 16-row MFMA tiles),
// where a 64/128-row tile would leave most of the device idle and re-decode
// the weights per row tile.  Measured on MI355X at K=4096, N=14336: M=16
// takes 82 us through the tile kernel, ~9 us streaming.
bool gemm_streams(int64_t M, int64_t K, int64_t N, int64_t G) {
  return M >= 1 && M <= kStreamMaxM && K > 0 && N > 0 && N % 4 == 0 && K % G == 0;
}
}  // namespace

extern "C" size_t nibble_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                              int64_t version, void* stream) {
  (void)stream;
  if ((version != 6 && version != 7) || (group_size != 64 && group_size != 128)) return 0;
  if (!gemm_streams(M, K, N, group_size)) return 0;
  StreamPlan p;
  if (plan_stream(M, K, N, group_size, true, 0, 0, &p) != NIBBLE_OK) return 0;
  return p.workspace_bytes;
}

extern "C" size_t nibble_gemm_counter_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                            int64_t version, void* stream) {
  (void)stream;
  if ((version != 6 && version != 7) || (group_size != 64 && group_size != 128)) return 0;
  if (!gemm_streams(M, K, N, group_size)) return 0;
  StreamPlan p;
  if (plan_stream(M, K, N, group_size, true, 0, 0, &p) != NIBBLE_OK) return 0;
  return p.counter_bytes;
}

extern "C" int nibble_gemm_w4a16(const void* X, int64_t x_rows, int64_t x_cols, const void* Wq,
                                 int64_t wq_rows, int64_t wq_cols, const void* S, int64_t s_rows,
                                 int64_t s_cols, int64_t group_size, int64_t version, void* Y,
                                 void* workspace, size_t workspace_bytes, void* stream_) {
  int rc = validate_gemm(X, x_rows, x_cols, Wq, wq_rows, wq_cols, S, s_rows, s_cols, group_size,
                         version, Y);
  if (rc != NIBBLE_OK) return rc;
  const int64_t M = x_rows, K = x_cols, N = wq_cols;
  if (M == 0 || N == 0) return ok();
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  if (K == 0) {
    NIBBLE_HIP(fill_zero_f16(Y, M * N, stream));
    return ok();
  }
  if (gemm_streams(M, K, N, group_size) && stream_supported(X, Wq, S, Y, M, K, N, group_size)) {
    StreamPlan p;
    rc = plan_stream(M, K, N, group_size, true, 0, 0, &p);
    if (rc != NIBBLE_OK) return rc;
    rc = launch_stream(X, Wq, S, Y, M, K, N, group_size, p, workspace, workspace_bytes, stream,
                       "gemm (streaming) kernel launch");
    return rc == NIBBLE_OK ? ok() : rc;
  }
  const auto* x = static_cast<const _Float16*>(X);
  const auto* w = static_cast<const uint32_t*>(Wq);
  const auto* s = static_cast<const _Float16*>(S);
  auto* y = static_cast<_Float16*>(Y);
  hipError_t e;
  if (version == 7)
    e = launch_tile<64, 128>(x, w, s, y, M, K, N, group_size, stream);
  else
    e = launch_tile<128, 128>(x, w, s, y, M, K, N, group_size, stream);
  if (e != hipSuccess) return hip_fail(e, "gemm kernel launch");
  return ok();
}
