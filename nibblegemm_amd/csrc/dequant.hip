// Standalone dequantisation: packed INT4 + fp16 group scales -> dense fp16 W.
//
// Reference: csrc/dequant_kernel.cu:18-74 (fast and scalar kernels, host
// checks) and the semantics of python/nibblegemm/quant.py:199-204.
//
// The kernel is HBM-bound and write-dominated: it reads K*N/2 + (K/G)*N*2 bytes
// and writes 2*K*N.  Each thread takes one packed row (8 k) of COLS adjacent
// columns: COLS/4 dwordx4 weight loads, one COLS-wide scale load and 8
// COLS*2-byte stores, so a wave64 writes 64*COLS*2 contiguous bytes per output
// row (1 KiB at COLS = 8).  Both decodes produce fp16_rne((n - 8) * s) bit for
// bit: the fast one builds the exact n - 8 with the magic-exponent trick and
// rounds once in v_pk_mul_f16; the scalar one forms the exact product in fp32
// and rounds once on conversion.
#include <hip/hip_fp16.h>

#include "nibble_common.h"
#include "nibble_decode.h"
#include "stream_matmul.h"

namespace nibble {

namespace {

// One wave per workgroup: 4096 x 14336 26.6 us against 26.9 / 29.5 / 30.9
// at 256 / 512 / 1024 threads (MI355X, graph replay, the stores below).
constexpr int kDequantThreads = 64;

// Cache policy of the 8-column stores: non-temporal at system scope (nt, sc0
// and sc1), measured against the plain non-temporal store (nt alone): 26.6
// vs 27.6 us at 4096 x 14336, 7.8 vs 7.8 at 4096 x 4096, 30.0 vs 30.8 at
// 8192 x 8192; cached stores 31.3.  Results are visible to later kernels
// and the host either way once the kernel completes.
constexpr int kStoreAux = 1 | 2 | 16;

// STRIPS: the weights are in a strip-major layout `L` (strips of at least 16
// columns, so a thread's 8 columns lie in one strip; every offset below
// 2^31, host-checked); otherwise in the packed [K / 8, N] layout.
template <int COLS, bool FAST, bool BUFFER_STORES, bool STRIPS = false>
__global__ __launch_bounds__(kDequantThreads) void dequant_kernel(
    const uint32_t* __restrict__ Wq, const _Float16* __restrict__ S, _Float16* __restrict__ out,
    int N, int group_size, WeightLayout L = WeightLayout()) {
  const int col_chunk = blockIdx.x * kDequantThreads + threadIdx.x;
  const int n0 = col_chunk * COLS;
  const int r8 = blockIdx.y;  // packed row
  if (n0 >= N) return;

  const size_t in_off = static_cast<size_t>(r8) * N + n0;
  const size_t s_off = static_cast<size_t>((r8 * 8) / group_size) * N + n0;
  const size_t out_row0 = static_cast<size_t>(r8) * 8 * N + n0;

  uint32_t q[COLS];
  _Float16 sc[COLS];
  if constexpr (STRIPS) {
    static_assert(COLS == 8, "strip-major weights are read 8 columns at a time");
    const char* wp = reinterpret_cast<const char*>(Wq) + r8 * L.w_row + L.wcol(n0);
    const char* sp = reinterpret_cast<const char*>(S) + ((r8 * 8) / group_size) * L.s_row +
                     L.scol(n0);
    const u4_t a = *reinterpret_cast<const u4_t*>(wp);
    const u4_t b = *reinterpret_cast<const u4_t*>(wp + 16);
    const h8_t s = *reinterpret_cast<const h8_t*>(sp);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      q[c] = a[c];
      q[4 + c] = b[c];
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) sc[c] = s[c];
  } else if constexpr (COLS == 8) {
    const u4_t a = *reinterpret_cast<const u4_t*>(Wq + in_off);
    const u4_t b = *reinterpret_cast<const u4_t*>(Wq + in_off + 4);
    const h8_t s = *reinterpret_cast<const h8_t*>(S + s_off);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      q[c] = a[c];
      q[4 + c] = b[c];
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) sc[c] = s[c];
  } else if constexpr (COLS == 4) {
    const u4_t a = *reinterpret_cast<const u4_t*>(Wq + in_off);
    const h4_t s = *reinterpret_cast<const h4_t*>(S + s_off);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      q[c] = a[c];
      sc[c] = s[c];
    }
  } else {
    q[0] = Wq[in_off];
    sc[0] = S[s_off];
  }

  // vals[k][c]: row k of the 8, column c.
  _Float16 vals[8][COLS];
#pragma unroll
  for (int c = 0; c < COLS; ++c) {
    if constexpr (FAST) {
      h2_t w[4];
      const h2_t s2 = {sc[c], sc[c]};
      decode8_scaled(q[c], s2, w);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        vals[2 * t][c] = w[t][0];
        vals[2 * t + 1][c] = w[t][1];
      }
    } else {
      const float s = static_cast<float>(sc[c]);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        vals[k][c] = static_cast<_Float16>(static_cast<float>(nibble_value(q[c], k)) * s);
    }
  }

  // BUFFER_STORES (the host checks 16 * N < 2^31): a resource over this
  // workgroup's 8 output rows, 16 * N bytes, with 32-bit lane offsets.
  _Float16* const rows8 = out + static_cast<size_t>(r8) * 8 * N;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    _Float16* dst = out + out_row0 + static_cast<size_t>(k) * N;
    if constexpr (COLS == 8) {
      h8_t v;
#pragma unroll
      for (int c = 0; c < 8; ++c) v[c] = vals[k][c];
      if constexpr (BUFFER_STORES)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4_t, v),
                                               make_rsrc(rows8, static_cast<uint32_t>(16 * N)),
                                               static_cast<uint32_t>((k * N + n0) * 2), 0,
                                               kStoreAux);
      else
        __builtin_nontemporal_store(v, reinterpret_cast<h8_t*>(dst));
    } else if constexpr (COLS == 4) {
      h4_t v;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = vals[k][c];
      __builtin_nontemporal_store(v, reinterpret_cast<h4_t*>(dst));
    } else {
      dst[0] = vals[k][0];
    }
  }
}

template <int COLS>
hipError_t launch(const uint32_t* w, const _Float16* s, _Float16* o, int64_t rows, int64_t N,
                  int64_t g, bool fast, hipStream_t stream) {
  const int64_t chunks = ceil_div(N, COLS);
  dim3 grid(static_cast<unsigned>(ceil_div(chunks, kDequantThreads)), static_cast<unsigned>(rows));
  if (COLS == 8 && 16 * N < (int64_t(1) << 31)) {
    if (fast)
      dequant_kernel<COLS, true, true><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)g);
    else
      dequant_kernel<COLS, false, true><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)g);
  } else if (fast) {
    dequant_kernel<COLS, true, false><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)g);
  } else {
    dequant_kernel<COLS, false, false><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)g);
  }
  return hipGetLastError();
}

}  // namespace

// Host validation shared by the launcher; pure host code, no HIP calls.
int validate_dequant(const void* Wq, int64_t wq_rows, int64_t wq_cols, const void* S,
                     int64_t s_rows, int64_t s_cols, int64_t group_size, const void* W) {
  NIBBLE_CHECK(wq_rows >= 0 && wq_cols >= 0, "packed weight shape must be non-negative");
  NIBBLE_CHECK(group_size > 0 && group_size % 8 == 0,
               "group_size must be a positive multiple of 8 (got %lld)", (long long)group_size);
  const int64_t K = wq_rows * 8, N = wq_cols;
  NIBBLE_CHECK(K % group_size == 0, "K=%lld must be divisible by group_size=%lld", (long long)K,
               (long long)group_size);
  NIBBLE_CHECK(s_rows * group_size == K, "scale rows disagree with K/group_size");
  NIBBLE_CHECK(s_cols == N, "scale columns disagree with N");
  NIBBLE_CHECK(K * N < (int64_t(1) << 40), "tensor too large");
  NIBBLE_CHECK(wq_rows < 65536 * 1024, "too many packed rows");
  NIBBLE_CHECK(N < (int64_t(1) << 31), "N too large");
  if (K * N > 0) {
    NIBBLE_CHECK(Wq != nullptr && S != nullptr && W != nullptr, "null pointer");
    NIBBLE_CHECK(aligned(Wq, 4) && aligned(S, 2) && aligned(W, 2), "misaligned pointer");
  }
  return NIBBLE_OK;
}

}  // namespace nibble

extern "C" int nibble_dequant_w4(const void* Wq, int64_t wq_rows, int64_t wq_cols, const void* S,
                                 int64_t s_rows, int64_t s_cols, int64_t group_size, int fast,
                                 void* W, void* stream_) {
  using namespace nibble;
  int rc = validate_dequant(Wq, wq_rows, wq_cols, S, s_rows, s_cols, group_size, W);
  if (rc != NIBBLE_OK) return rc;
  if (wq_rows == 0 || wq_cols == 0) return ok();
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));

  const auto* w = static_cast<const uint32_t*>(Wq);
  const auto* s = static_cast<const _Float16*>(S);
  auto* o = static_cast<_Float16*>(W);
  const int64_t N = wq_cols;
  const bool vec_ok = aligned(Wq, 16) && aligned(S, 16) && aligned(W, 16);
  hipError_t e;
  if (vec_ok && N % 8 == 0)
    e = launch<8>(w, s, o, wq_rows, N, group_size, fast != 0, stream);
  else if (vec_ok && N % 4 == 0)
    e = launch<4>(w, s, o, wq_rows, N, group_size, fast != 0, stream);
  else
    e = launch<1>(w, s, o, wq_rows, N, group_size, fast != 0, stream);
  if (e != hipSuccess) return hip_fail(e, "dequant kernel launch");
  return ok();
}

// dequant_w4 of strip-major weights (no counterpart in the reference): the
// same [K, N] fp16 output, bit for bit, as the packed call on the weight the
// strips were packed from.
extern "C" int nibble_dequant_w4_strip_major(const void* Wt, const void* St, int64_t K, int64_t N,
                                             int64_t group_size, int64_t strip_cols, int fast,
                                             void* W, void* stream_) {
  using namespace nibble;
  NIBBLE_CHECK(K >= 0 && N >= 0 && K % 8 == 0, "bad dimension (K a multiple of 8)");
  NIBBLE_CHECK(strip_cols == 16 || strip_cols == 32 || strip_cols == 64,
               "strip_cols must be 16, 32 or 64, got %lld", (long long)strip_cols);
  NIBBLE_CHECK(N % strip_cols == 0, "N=%lld is not a multiple of strip_cols=%lld", (long long)N,
               (long long)strip_cols);
  int rc = validate_dequant(Wt, K / 8, N, St, group_size > 0 ? K / group_size : 0, N, group_size,
                            W);
  if (rc != NIBBLE_OK) return rc;
  NIBBLE_CHECK(group_size == 64 || group_size == 128, "group_size must be 64 or 128");
  NIBBLE_CHECK(strip_cols != 16 || group_size == 128, "16-column strips need group_size 128");
  NIBBLE_CHECK(K / 8 * N * 4 < (int64_t(1) << 31), "weights beyond 32-bit offsets");
  if (K == 0 || N == 0) return ok();
  NIBBLE_CHECK(aligned(Wt, 16) && aligned(St, 16) && aligned(W, 16),
               "strip-major dequant needs 16-byte aligned weights, scales and output");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  const WeightLayout L = strip_major_layout(K, N, group_size, strip_cols);
  const auto* w = static_cast<const uint32_t*>(Wt);
  const auto* s = static_cast<const _Float16*>(St);
  auto* o = static_cast<_Float16*>(W);
  const dim3 grid(static_cast<unsigned>(ceil_div(N / 8, kDequantThreads)),
                  static_cast<unsigned>(K / 8));
  const bool bufs = 16 * N < (int64_t(1) << 31);
  if (fast && bufs)
    dequant_kernel<8, true, true, true><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)group_size, L);
  else if (fast)
    dequant_kernel<8, true, false, true><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)group_size, L);
  else if (bufs)
    dequant_kernel<8, false, true, true><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)group_size, L);
  else
    dequant_kernel<8, false, false, true><<<grid, kDequantThreads, 0, stream>>>(w, s, o, (int)N, (int)group_size, L);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "strip-major dequant kernel launch");
  return ok();
}
