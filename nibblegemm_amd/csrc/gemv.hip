// Decode-regime W4A16 matmul (M <= 8): Y[M,N] = X[M,K] @ dequant(Wq, S).
//
// Reference: csrc/gemv_w4a16.cu (kernels v0-v4 :30-244, host :251-425).
//
// The streaming kernel (versions 2, 3, 4) is one launch:
//
//  * Workgroup = WAVES wave64s over one 256-column slab (each lane owns 4
//    adjacent columns, i.e. one 16-byte word quad per packed row, so a wave
//    reads 1 KiB contiguous per row) and one K split of whole quant groups.
//  * Wave w of the workgroup takes groups gb+w, gb+w+WAVES, ... of its split.
//    Per group it issues all GROUP/8 dwordx4 buffer loads up front (SGPR row
//    offsets, no per-load VALU address math), then decodes each word with the
//    0x6400 magic-exponent trick (v_and_or_b32) and accumulates x*w with
//    v_dot2_f32_f16 into fp32 group sums.  X is wave-uniform and is read with
//    scalar loads.  The group scale multiplies the fp32 group sum.
//  * Waves are reduced through LDS in wave order.  With one split the
//    workgroup writes fp16 Y directly.  With several, each workgroup writes an
//    fp32 partial [split, M, N], and the last workgroup of each slab to finish
//    (agent-scope counter) sums the partials in split order and writes Y --
//    deterministic, and no second launch (the reference ran reduce_splits as a
//    separate kernel, :237-244, :418-423).  That workgroup resets the counter
//    to zero, so the counter region stays zero between calls.
//
// Versions 0 and 1 are scalar fp32 kernels, one thread per output (the
// reference's v0/v1, :30-72): an on-device reference, not a fast path.
#include <algorithm>

#include "nibble_common.h"
#include "nibble_decode.h"

namespace nibble {

namespace {

constexpr int kSlabCols = 256;  // 64 lanes x 4 columns

struct GemvArgs {
  const _Float16* X;
  const uint32_t* Wq;
  const _Float16* S;
  _Float16* Y;
  float* partial;      // [splits, M, N] fp32, used when splits > 1
  uint32_t* counters;  // [slabs], zero on entry and on exit
  int M, K, N;
  int groups_per_split;
  int splits;
};

template <int MT, int GROUP, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_stream_kernel(GemvArgs a) {
  constexpr int WORDS = GROUP / 8;  // packed rows per quant group
  __shared__ f4_t red[WAVES][MT][64];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slab = blockIdx.x;
  const int split = blockIdx.y;
  const int n0 = slab * kSlabCols + lane * 4;
  const bool active = n0 < a.N;
  const int total_groups = a.K / GROUP;
  const int gb = split * a.groups_per_split;
  const int ge = min(gb + a.groups_per_split, total_groups);
  const uint32_t row_bytes = static_cast<uint32_t>(a.N) * 4u;
  // Inactive lanes (past N in the last slab) point outside the buffer
  // resource, so their loads return zero without touching memory.
  const uint32_t voff = active ? static_cast<uint32_t>(n0) * 4u : 0x80000000u;

  float acc[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;

  for (int g = gb + wave; g < ge; g += WAVES) {
    const uint32_t* gbase = a.Wq + static_cast<size_t>(g) * WORDS * a.N;
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(gbase, WORDS * row_bytes);
    u4_t w[WORDS];
#pragma unroll
    for (int j = 0; j < WORDS; ++j)
      w[j] = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, j * row_bytes, 0));

    h4_t sc = {0, 0, 0, 0};
    if (active) sc = *reinterpret_cast<const h4_t*>(a.S + static_cast<size_t>(g) * a.N + n0);

    float gs[MT][4];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) gs[m][c] = 0.0f;

#pragma unroll
    for (int j = 0; j < WORDS; ++j) {
      h2_t d[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) decode8(w[j][c], d[c]);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < a.M) {
          const h8_t xv = *reinterpret_cast<const h8_t*>(a.X + static_cast<size_t>(m) * a.K +
                                                         g * GROUP + j * 8);
          const h2_t xp[4] = {{xv[0], xv[1]}, {xv[2], xv[3]}, {xv[4], xv[5]}, {xv[6], xv[7]}};
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < 4; ++t)
              gs[m][c] = __builtin_amdgcn_fdot2(d[c][t], xp[t], gs[m][c], false);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[m][c] = __builtin_fmaf(gs[m][c], (float)sc[c], acc[m][c]);
  }

  // Cross-wave reduction in LDS, summed in wave order.
#pragma unroll
  for (int m = 0; m < MT; ++m) red[wave][m][lane] = f4_t{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
  __syncthreads();

  const bool direct = a.splits == 1;
  for (int it = threadIdx.x; it < MT * 64; it += WAVES * 64) {
    const int m = it >> 6, l = it & 63;
    const int col = slab * kSlabCols + l * 4;
    if (m >= a.M || col >= a.N) continue;
    f4_t s = red[0][m][l];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      const f4_t v = red[w][m][l];
      s[0] += v[0];
      s[1] += v[1];
      s[2] += v[2];
      s[3] += v[3];
    }
    if (direct) {
      const h4_t y = {(_Float16)s[0], (_Float16)s[1], (_Float16)s[2], (_Float16)s[3]};
      *reinterpret_cast<h4_t*>(a.Y + static_cast<size_t>(m) * a.N + col) = y;
    } else {
      *reinterpret_cast<f4_t*>(a.partial + (static_cast<size_t>(split) * a.M + m) * a.N + col) = s;
    }
  }
  if (direct) return;

  // Publish this split's partial; the last workgroup of the slab reduces.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(a.counters + slab, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == static_cast<uint32_t>(a.splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  for (int it = threadIdx.x; it < MT * 64; it += WAVES * 64) {
    const int m = it >> 6, l = it & 63;
    const int col = slab * kSlabCols + l * 4;
    if (m >= a.M || col >= a.N) continue;
    f4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp = 0; sp < a.splits; ++sp) {
      const f4_t v =
          *reinterpret_cast<const f4_t*>(a.partial + (static_cast<size_t>(sp) * a.M + m) * a.N + col);
      s[0] += v[0];
      s[1] += v[1];
      s[2] += v[2];
      s[3] += v[3];
    }
    const h4_t y = {(_Float16)s[0], (_Float16)s[1], (_Float16)s[2], (_Float16)s[3]};
    *reinterpret_cast<h4_t*>(a.Y + static_cast<size_t>(m) * a.N + col) = y;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(a.counters + slab, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Versions 0 and 1: one thread per (m, n), scalar decode, fp32 weights
// (n - 8) * s and fp32 accumulation.  REUSE = false reloads the packed word for
// every k (v0), REUSE = true uses each word for its 8 k (v1).
template <bool REUSE>
__global__ __launch_bounds__(256) void gemv_scalar_kernel(const _Float16* __restrict__ X,
                                                          const uint32_t* __restrict__ Wq,
                                                          const _Float16* __restrict__ S,
                                                          _Float16* __restrict__ Y, int M, int K,
                                                          int N, int group_size) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  float acc = 0.0f;
  const _Float16* x = X + static_cast<size_t>(m) * K;
  if (REUSE) {
    for (int k8 = 0; k8 < K / 8; ++k8) {
      const uint32_t q = Wq[static_cast<size_t>(k8) * N + n];
      const float s = (float)S[static_cast<size_t>((k8 * 8) / group_size) * N + n];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += (float)x[k8 * 8 + j] * ((float)nibble_value(q, j) * s);
    }
  } else {
    for (int k = 0; k < K; ++k) {
      const uint32_t q = Wq[static_cast<size_t>(k / 8) * N + n];
      const float s = (float)S[static_cast<size_t>(k / group_size) * N + n];
      acc += (float)x[k] * ((float)nibble_value(q, k % 8) * s);
    }
  }
  Y[static_cast<size_t>(m) * N + n] = (_Float16)acc;
}

// Launch geometry of the streaming kernel.
struct Plan {
  int mt = 1;
  int waves = 4;
  int slabs = 0;
  int splits = 1;
  int groups_per_split = 0;
  size_t counter_bytes = 0;
  size_t workspace_bytes = 0;
};

int mt_for(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

// Largest wave count the LDS reduction buffer allows for MT rows (<= 32 KiB).
int max_waves_for(int mt) { return std::min(16, 32 / mt); }

int default_waves(int mt) { return std::min(4, max_waves_for(mt)); }

// Split heuristic for MI355X: aim for ~8 resident waves per CU in total
// (counted in wave-groups: one wave streams one quant group at a time), with
// the K range of each split a whole number of waves' worth of groups.
int plan_stream(int64_t M, int64_t K, int64_t N, int64_t G, int64_t version, int64_t splits_override,
                int64_t threads_override, int cus, Plan* p) {
  p->mt = mt_for(M);
  if (threads_override > 0) {
    p->waves = static_cast<int>(threads_override / 64);
    if (p->waves > max_waves_for(p->mt))
      return fail(NIBBLE_ERR_UNSUPPORTED, "block_threads=%lld too large for M=%lld (max %d)",
                  (long long)threads_override, (long long)M, max_waves_for(p->mt) * 64);
  } else {
    p->waves = default_waves(p->mt);
  }
  p->slabs = static_cast<int>(ceil_div(N, kSlabCols));
  const int groups = static_cast<int>(K / G);
  int gps = groups;  // groups per split
  if (version == 4 && splits_override > 0) {
    // Floor, then trim empty splits (csrc/gemv_w4a16.cu:398-401).
    const int want = static_cast<int>(std::min<int64_t>(splits_override, groups));
    gps = std::max(1, groups / want);
  } else if (version == 4) {
    const int64_t target_waves = static_cast<int64_t>(cus) * 8;
    const int64_t per_split = static_cast<int64_t>(p->slabs) * p->waves;
    int64_t want = ceil_div(target_waves, per_split);
    want = std::max<int64_t>(1, std::min<int64_t>(want, ceil_div(groups, p->waves)));
    // A whole number of waves' worth of groups per split.
    int64_t g = ceil_div(groups, want);
    g = ceil_div(g, p->waves) * p->waves;
    gps = static_cast<int>(std::min<int64_t>(g, groups));
  }
  const int splits = static_cast<int>(ceil_div(groups, gps));
  p->splits = splits;
  p->groups_per_split = gps;
  if (splits > 1) {
    p->counter_bytes = align_up(static_cast<size_t>(p->slabs) * 4, 256);
    p->workspace_bytes = p->counter_bytes + static_cast<size_t>(splits) * M * N * 4;
  } else {
    p->counter_bytes = 0;
    p->workspace_bytes = 0;
  }
  return NIBBLE_OK;
}

template <int MT, int GROUP>
hipError_t launch_mt(const GemvArgs& a, const Plan& p, hipStream_t stream) {
  dim3 grid(p.slabs, p.splits);
  switch (p.waves) {
    case 1: gemv_stream_kernel<MT, GROUP, 1><<<grid, 64, 0, stream>>>(a); break;
    case 2: gemv_stream_kernel<MT, GROUP, 2><<<grid, 128, 0, stream>>>(a); break;
    case 4: gemv_stream_kernel<MT, GROUP, 4><<<grid, 256, 0, stream>>>(a); break;
    case 8:
      if constexpr (MT <= 4) {
        gemv_stream_kernel<MT, GROUP, 8><<<grid, 512, 0, stream>>>(a);
        break;
      } else {
        return hipErrorInvalidValue;
      }
    case 16:
      if constexpr (MT <= 2) {
        gemv_stream_kernel<MT, GROUP, 16><<<grid, 1024, 0, stream>>>(a);
        break;
      } else {
        return hipErrorInvalidValue;
      }
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int GROUP>
hipError_t launch_group(const GemvArgs& a, const Plan& p, hipStream_t stream) {
  switch (p.mt) {
    case 1: return launch_mt<1, GROUP>(a, p, stream);
    case 2: return launch_mt<2, GROUP>(a, p, stream);
    case 4: return launch_mt<4, GROUP>(a, p, stream);
    default: return launch_mt<8, GROUP>(a, p, stream);
  }
}

}  // namespace

// Mirrors check_inputs (csrc/gemv_w4a16.cu:251-265) on shapes; pure host code.
int validate_gemv(const void* X, int64_t x_rows, int64_t x_cols, const void* Wq, int64_t wq_rows,
                  int64_t wq_cols, const void* S, int64_t s_rows, int64_t s_cols, int64_t group_size,
                  int64_t version, int64_t splits_override, int64_t threads_override,
                  const void* Y) {
  NIBBLE_CHECK(threads_override == 0 || threads_override == 64 || threads_override == 128 ||
                   threads_override == 256 || threads_override == 512 || threads_override == 1024,
               "block_threads must be 0 (heuristic) or 64, 128, 256, 512, 1024 (a wave is 64 lanes), "
               "got %lld",
               (long long)threads_override);
  NIBBLE_CHECK(splits_override >= 0, "splits must be >= 0");
  NIBBLE_CHECK(x_rows >= 0 && x_cols >= 0 && wq_rows >= 0 && wq_cols >= 0 && s_rows >= 0 &&
                   s_cols >= 0,
               "negative dimension");
  const int64_t K = x_cols, N = wq_cols;
  NIBBLE_CHECK(wq_rows * 8 == K, "packed weight rows disagree with K");
  NIBBLE_CHECK(s_rows * group_size == K, "scale rows disagree with K/group_size");
  NIBBLE_CHECK(s_cols == N, "scale columns disagree with N");
  NIBBLE_CHECK(N % 4 == 0, "N must be a multiple of 4 for 128-bit weight loads");
  NIBBLE_CHECK(group_size == 64 || group_size == 128, "group_size must be 64 or 128");
  NIBBLE_CHECK(version >= 0 && version <= 4, "version must be 0..4, got %lld", (long long)version);
  NIBBLE_CHECK(K < (int64_t(1) << 31) && N < (int64_t(1) << 31) && x_rows < (int64_t(1) << 31),
               "dimension too large");
  NIBBLE_CHECK((K / 8) * N * 4 < (int64_t(1) << 32) || version <= 1,
               "packed weights too large for 32-bit buffer offsets");
  if (x_rows * K > 0 || x_rows * N > 0) {
    NIBBLE_CHECK(X != nullptr && Wq != nullptr && S != nullptr && Y != nullptr, "null pointer");
    NIBBLE_CHECK(aligned(X, 16) && aligned(Wq, 16) && aligned(S, 8) && aligned(Y, 8),
                 "misaligned pointer (X and Wq need 16-byte, S and Y 8-byte alignment)");
  }
  return NIBBLE_OK;
}

}  // namespace nibble

using namespace nibble;

namespace {
int gemv_plan(int64_t M, int64_t K, int64_t N, int64_t G, int64_t version, int64_t splits_override,
              int64_t threads_override, hipStream_t stream, Plan* p) {
  int cus = 256;
  if (version == 4 && splits_override <= 0) {
    int dev = 0;
    NIBBLE_HIP(stream_device(stream, &dev));
    NIBBLE_HIP(cu_count(dev, &cus));
  }
  return plan_stream(M, K, N, G, version, splits_override, threads_override, cus, p);
}
}  // namespace

extern "C" size_t nibble_gemv_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                              int64_t version, int64_t splits_override,
                                              int64_t threads_override, void* stream) {
  if (version < 2 || version > 4 || M <= 0 || M > 8 || N <= 0 || K <= 0) return 0;
  if (group_size != 64 && group_size != 128) return 0;
  if (K % group_size != 0) return 0;
  Plan p;
  if (gemv_plan(M, K, N, group_size, version, splits_override, threads_override,
                static_cast<hipStream_t>(stream), &p) != NIBBLE_OK)
    return 0;
  return p.workspace_bytes;
}

extern "C" size_t nibble_gemv_counter_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                            int64_t version, int64_t splits_override,
                                            int64_t threads_override, void* stream) {
  if (version < 2 || version > 4 || M <= 0 || M > 8 || N <= 0 || K <= 0) return 0;
  if (group_size != 64 && group_size != 128) return 0;
  if (K % group_size != 0) return 0;
  Plan p;
  if (gemv_plan(M, K, N, group_size, version, splits_override, threads_override,
                static_cast<hipStream_t>(stream), &p) != NIBBLE_OK)
    return 0;
  return p.counter_bytes;
}

extern "C" int nibble_gemv_w4a16(const void* X, int64_t x_rows, int64_t x_cols, const void* Wq,
                                 int64_t wq_rows, int64_t wq_cols, const void* S, int64_t s_rows,
                                 int64_t s_cols, int64_t group_size, int64_t version,
                                 int64_t splits_override, int64_t threads_override, void* Y,
                                 void* workspace, size_t workspace_bytes, void* stream_) {
  int rc = validate_gemv(X, x_rows, x_cols, Wq, wq_rows, wq_cols, S, s_rows, s_cols, group_size,
                         version, splits_override, threads_override, Y);
  if (rc != NIBBLE_OK) return rc;
  const int64_t M = x_rows, K = x_cols, N = wq_cols;
  if (version >= 3 && M > 8)
    return fail(NIBBLE_ERR_UNSUPPORTED,
                "gemv path supports M <= 8; use gemm_w4a16 for larger M (got M=%lld)", (long long)M);
  if (M == 0 || N == 0) return ok();
  hipStream_t stream = static_cast<hipStream_t>(stream_);

  if (K == 0) {
    // Empty reduction: Y is all zeros (the reference's kernels write 0 too).
    DeviceGuard guard;
    int dev = 0;
    NIBBLE_HIP(guard.enter(stream, &dev));
    NIBBLE_HIP(fill_zero_f16(Y, M * N, stream));
    return ok();
  }

  if (version <= 1) {
    DeviceGuard guard;
    int dev = 0;
    NIBBLE_HIP(guard.enter(stream, &dev));
    dim3 grid(static_cast<unsigned>(ceil_div(N, 256)), static_cast<unsigned>(M));
    if (grid.y > 65535) return fail(NIBBLE_ERR_UNSUPPORTED, "M too large for versions 0/1");
    const auto* x = static_cast<const _Float16*>(X);
    const auto* w = static_cast<const uint32_t*>(Wq);
    const auto* s = static_cast<const _Float16*>(S);
    auto* y = static_cast<_Float16*>(Y);
    if (version == 0)
      gemv_scalar_kernel<false><<<grid, 256, 0, stream>>>(x, w, s, y, (int)M, (int)K, (int)N,
                                                          (int)group_size);
    else
      gemv_scalar_kernel<true><<<grid, 256, 0, stream>>>(x, w, s, y, (int)M, (int)K, (int)N,
                                                         (int)group_size);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "gemv scalar kernel launch");
    return ok();
  }

  // Version 2 has no row limit in the reference: it is served in blocks of 8
  // rows by the single-split streaming kernel.
  if (version == 2 && M > 8) {
    const size_t xrow = static_cast<size_t>(K) * 2, yrow = static_cast<size_t>(N) * 2;
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
      const int64_t mb = std::min<int64_t>(8, M - m0);
      rc = nibble_gemv_w4a16(static_cast<const char*>(X) + m0 * xrow, mb, K, Wq, wq_rows, wq_cols, S,
                             s_rows, s_cols, group_size, 2, 0, threads_override,
                             static_cast<char*>(Y) + m0 * yrow, nullptr, 0, stream_);
      if (rc != NIBBLE_OK) return rc;
    }
    return ok();
  }

  Plan p;
  rc = gemv_plan(M, K, N, group_size, version, splits_override, threads_override, stream, &p);
  if (rc != NIBBLE_OK) return rc;
  if (p.workspace_bytes > 0) {
    if (workspace == nullptr || workspace_bytes < p.workspace_bytes)
      return fail(NIBBLE_ERR_WORKSPACE, "gemv needs %zu bytes of workspace, got %zu",
                  p.workspace_bytes, workspace == nullptr ? size_t(0) : workspace_bytes);
    if (!aligned(workspace, 256)) return fail(NIBBLE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }

  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));

  GemvArgs a;
  a.X = static_cast<const _Float16*>(X);
  a.Wq = static_cast<const uint32_t*>(Wq);
  a.S = static_cast<const _Float16*>(S);
  a.Y = static_cast<_Float16*>(Y);
  a.counters = p.splits > 1 ? static_cast<uint32_t*>(workspace) : nullptr;
  a.partial = p.splits > 1
                  ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.counter_bytes)
                  : nullptr;
  a.M = static_cast<int>(M);
  a.K = static_cast<int>(K);
  a.N = static_cast<int>(N);
  a.groups_per_split = p.groups_per_split;
  a.splits = p.splits;
  hipError_t e = group_size == 128 ? launch_group<128>(a, p, stream) : launch_group<64>(a, p, stream);
  if (e != hipSuccess) return hip_fail(e, "gemv kernel launch");
  return ok();
}
