// Decode-regime W4A16 matmul (M <= 8): Y[M,N] = X[M,K] @ dequant(Wq, S).
//
// Reference: csrc/gemv_w4a16.cu (kernels v0-v4 :30-244, host :251-425).
//
// The streaming kernel (versions 2, 3, 4) runs the dot products on CDNA4
// matrix cores (v_mfma_f32_16x16x32_f16) and is one launch:
//
//  * A workgroup owns a 64-column strip and one K split (whole quant groups);
//    its WAVES waves take the split's groups round-robin.  Per 32-k chunk a
//    lane issues one dwordx4 buffer load: 4 adjacent columns of one packed
//    row, so a wave reads 4 rows x 256 contiguous bytes.  Lane l's word for
//    column 4*(l%16)+j is exactly the B operand of MFMA j in B-column slot
//    l%16 and k block l/16 -- no shuffles.
//  * Each word is decoded with the 0x6400 magic-exponent trick, one
//    v_and_or_b32 per half2 (1024 + n or 1024 + 16n, see decode8_biased).  The
//    bias and the 1/16 are not removed per weight: activations are pre-scaled
//    (x/16 at k % 8 in {2,3,6,7}) and one extra MFMA per chunk against a
//    constant correction adds -1032 / -1152 times the activations, which is
//    the same for every column.  5 VALU ops per packed word, whatever M is.
//  * Row m of the MFMA A operand is activation row m (rows >= M read as
//    zero), so M = 1..8 costs the same matrix-core work as M = 1.
//  * Per quant group the fp32 MFMA tile is scaled by the column's fp16 scale
//    into fp32 totals; loads of the next group are in flight meanwhile
//    (double-buffered registers).
//  * Waves are summed through LDS in wave order.  With one split the
//    workgroup writes fp16 Y directly.  With several, each workgroup writes
//    an fp32 partial [split, M, N] with device-coherent stores, and the last
//    workgroup of the strip (agent-scope counter) sums the partials in split
//    order and writes Y -- deterministic, and no second launch (the reference
//    ran reduce_splits as a separate kernel, :237-244, :418-423).  That
//    workgroup resets the counter, so the counter region stays zero between
//    calls.
//
// Versions 0 and 1 are scalar fp32 kernels, one thread per output (the
// reference's v0/v1, :30-72): an on-device reference, not a fast path.
#include <algorithm>
#include <cmath>

#include "nibble_common.h"
#include "nibble_decode.h"
#include "nibble_reduce.h"
#include "stream_matmul.h"

namespace nibble {

namespace {

constexpr int kStripCols = 64;  // 16 lanes x 4 columns

struct GemvArgs {
  const _Float16* X;
  const uint32_t* Wq;
  const _Float16* S;
  _Float16* Y;
  float* partial;      // [splits, M, N] fp32, used when splits > 1
  uint32_t* counters;  // [strips], zero on entry and on exit
  int M, K, N;
  int groups_per_split;
  int splits;
  int epilogue;           // kEpilogueNone / kEpilogueBias / kEpilogueSwiglu
  const _Float16* bias;   // [N] for kEpilogueBias
  const _Float16* norm_w; // [K]: the activations are RMSNorm(X) * norm_w (fused prologue), or null
  float norm_eps;
};

// Output epilogues of the streaming kernel (fused forms of what a caller
// would otherwise run as separate elementwise kernels on the fp16 result).
constexpr int kEpilogueNone = 0;
constexpr int kEpilogueBias = 1;    // Y = fp16(fp16(X W) + bias)
constexpr int kEpilogueSwiglu = 2;  // W = [gate | up] in 32-column blocks; Y = silu(G) * U

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

__device__ __forceinline__ f4_t mfma16(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Writes a strip's outputs from `total(r, qq)`, the fp32 sums of column quad
// qq of row r, through the launch's epilogue.
template <int MT, int THREADS, typename Total>
__device__ __forceinline__ void emit_outputs(const GemvArgs& a, int strip, int m_base, int mrows,
                                             Total total) {
  if (a.epilogue == kEpilogueSwiglu) {
    const int nout = a.N / 2;
    for (int e = threadIdx.x; e < MT * 8; e += THREADS) {
      const int r = e >> 3, qq = e & 7;
      const int ocol = strip * (kStripCols / 2) + 4 * qq;
      if (r >= mrows || ocol >= nout) continue;
      const f4_t g = total(r, qq), u = total(r, qq + 8);
      const h4_t y = {(_Float16)silu_mul(g[0], u[0]), (_Float16)silu_mul(g[1], u[1]),
                      (_Float16)silu_mul(g[2], u[2]), (_Float16)silu_mul(g[3], u[3])};
      *reinterpret_cast<h4_t*>(a.Y + static_cast<size_t>(m_base + r) * nout + ocol) = y;
    }
    return;
  }
  for (int e = threadIdx.x; e < MT * 16; e += THREADS) {
    const int r = e >> 4, qq = e & 15;
    const int ocol = strip * kStripCols + 4 * qq;
    if (r >= mrows || ocol >= a.N) continue;
    const f4_t sum = total(r, qq);
    h4_t y = {(_Float16)sum[0], (_Float16)sum[1], (_Float16)sum[2], (_Float16)sum[3]};
    if (a.epilogue == kEpilogueBias) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        y[c] = (_Float16)(static_cast<float>(y[c]) + static_cast<float>(a.bias[ocol + c]));
    }
    *reinterpret_cast<h4_t*>(a.Y + static_cast<size_t>(m_base + r) * a.N + ocol) = y;
  }
}

// STREAM: the launch reads every weight exactly once (a single row block), so
// packed words and scales are loaded with the non-temporal hint -- measured
// 1-2% faster at M <= 32; launches of several row blocks re-read the weights
// from cache and keep the default policy.
// NORM: the activations are RMSNorm rows of X, fp16(x * r * norm_w) with r
// the row's 1 / sqrt(mean(x^2) + eps).  A prologue computes r exactly as the
// RMSNorm kernel does (same chunking, same fixed-order reduction, so the
// same bits), writes the normalised rows of the workgroup's block to LDS
// once, and the loop reads its activation chunks from there instead of X.
template <int MT, int GROUP, int WAVES, bool STREAM, bool NORM = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_mfma_kernel(GemvArgs a) {
  constexpr int kWPolicy = STREAM ? 2 : 0;  // buffer-load cache policy: 2 = nt
  constexpr int CPG = GROUP / 32;                  // 32-k chunks per quant group
  constexpr int TILES = (MT + 15) / 16;            // 16-row MFMA A tiles
  constexpr int LANE_ROWS = MT < 4 ? MT : 4;       // output rows a lane holds per tile
  constexpr int THREADS = WAVES * 64;
  __shared__ f4_t red[WAVES][MT][16];              // [wave][row][column quad]
  __shared__ int s_last;
  extern __shared__ __attribute__((aligned(16))) _Float16 xnorm[];  // NORM: [MT][K]
  static_assert(!NORM || THREADS == kRmsThreads, "the RMSNorm prologue runs on 256 threads");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = blockIdx.x;
  const int split = blockIdx.y;
  // Rows [m_base, m_base + mrows) of X and Y belong to this workgroup: one
  // block of MT rows per grid z (batches above 32 rows run several blocks,
  // each streaming the weights; repeats hit the Infinity Cache).
  const int m_base = blockIdx.z * MT;
  const int mrows = min(MT, a.M - m_base);
  const int q = lane & 15;   // B column slot (column quad) and A row within a tile
  const int kb = lane >> 4;  // 8-k block within a 32-k chunk
  const int col = strip * kStripCols + 4 * q;
  const bool col_ok = col < a.N;
  const uint32_t row_bytes = static_cast<uint32_t>(a.N) * 4u;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.Wq, static_cast<uint32_t>(a.K / 8) * row_bytes);
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(a.X, static_cast<uint32_t>(a.M) * static_cast<uint32_t>(a.K) * 2u);
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(a.S, static_cast<uint32_t>(a.K / GROUP) * static_cast<uint32_t>(a.N) * 2u);
  const uint32_t voff_w = col_ok ? kb * row_bytes + static_cast<uint32_t>(col) * 4u : kOutOfRange;
  const uint32_t voff_s = col_ok ? static_cast<uint32_t>(col) * 2u : kOutOfRange;
  uint32_t voff_x[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const int m = 16 * t + q;
    voff_x[t] = m < mrows ? (static_cast<uint32_t>(m_base + m) * a.K + 8u * kb) * 2u : kOutOfRange;
  }

  struct Stage {
    h8_t x[TILES][CPG];
    h4_t s;
    u4_t w[CPG];
    int g;
  };
  // Loads of group g.  A prefetch past the split re-reads the split's last
  // group (just loaded, so an L2 hit) instead of being predicated off: the
  // loads stay unconditional and identical on every path, which lets the
  // compiler keep exact in-order wait counts across the loop back-edge
  // (a per-lane "disabled" offset made it drain every load at the top of
  // each iteration).
  const int total_groups = a.K / GROUP;
  const int gb = split * a.groups_per_split;
  const int ge = min(gb + a.groups_per_split, total_groups);
  auto load = [&](Stage& st, int g, bool enabled) {
    g = enabled ? g : ge - 1;
    const uint32_t kx = static_cast<uint32_t>(g) * GROUP * 2u;
    const uint32_t kw = static_cast<uint32_t>(g) * (GROUP / 8) * row_bytes;
    st.g = g;
    if constexpr (!NORM) {
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int c = 0; c < CPG; ++c)
          st.x[t][c] = __builtin_bit_cast(
              h8_t, __builtin_amdgcn_raw_buffer_load_b128(rx, voff_x[t], kx + c * 64, 0));
    }
    st.s = __builtin_bit_cast(
        h4_t, __builtin_amdgcn_raw_buffer_load_b64(rs, voff_s, static_cast<uint32_t>(g) * a.N * 2u,
                                                   kWPolicy));
#pragma unroll
    for (int c = 0; c < CPG; ++c)
      st.w[c] = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, voff_w, kw + c * 4 * row_bytes, kWPolicy));
  };

  f4_t tot[TILES][4];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) tot[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const DecodeConsts dk = decode_consts();
  const h8_t xscale = biased_x_scale();
  const h8_t bcorr = biased_correction();
  auto compute = [&](const Stage& st) {
    h8_t xs[TILES][CPG];
    f4_t acc[TILES][4];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      if constexpr (NORM) {
        // Lane (q, kb) takes row 16 t + q, k = g GROUP + 32 c + 8 kb + 0..7.
        const int m = 16 * t + q;
#pragma unroll
        for (int c = 0; c < CPG; ++c)
          xs[t][c] = (m < mrows ? *reinterpret_cast<const h8_t*>(
                                      &xnorm[m * a.K + st.g * GROUP + 32 * c + 8 * kb])
                                : h8_t{}) *
                     xscale;
      } else {
#pragma unroll
        for (int c = 0; c < CPG; ++c) xs[t][c] = st.x[t][c] * xscale;
      }
      f4_t corr = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < CPG; ++c) corr = mfma16(xs[t][c], bcorr, corr);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][j] = corr;
    }
    // One decode per word serves every tile.
#pragma unroll
    for (int c = 0; c < CPG; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h8_t b = decode8_biased(st.w[c][j], dk);
#pragma unroll
        for (int t = 0; t < TILES; ++t) acc[t][j] = mfma16(xs[t][c], b, acc[t][j]);
      }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sj = static_cast<float>(st.s[j]);
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int i = 0; i < LANE_ROWS; ++i)
          tot[t][j][i] = __builtin_fmaf(sj, acc[t][j][i], tot[t][j][i]);
    }
  };

  Stage s0, s1;
  int g = gb + wave;
  if constexpr (NORM) {
    // The first group's weights do not depend on the activations: their
    // loads go out before the prologue, which their latency then covers.
    if (g < ge) load(s0, g, true);
    // Rows of this block, normalised into LDS.  Thread t holds chunks
    // (256 c + t) * 8 of a row (K <= 16384: at most 8), x and the weight
    // loaded before the reduction, as in the RMSNorm kernel.
    __shared__ float part[kRmsThreads / 64];
    constexpr int kMaxChunks = 8;
    const int tid = threadIdx.x;
    for (int r = 0; r < mrows; ++r) {
      const _Float16* xr = a.X + static_cast<size_t>(m_base + r) * a.K;
      h8_t v[kMaxChunks], w[kMaxChunks];
      float ss = 0.0f;
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        const int col = (c * kRmsThreads + tid) * 8;
        v[c] = col < a.K ? *reinterpret_cast<const h8_t*>(xr + col) : h8_t{};
        w[c] = col < a.K ? *reinterpret_cast<const h8_t*>(a.norm_w + col) : h8_t{};
        ss = sumsq_chunk(v[c], ss);
      }
      const float rr = rms_scale(block256_sum(ss, part), a.K, a.norm_eps);
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        const int col = (c * kRmsThreads + tid) * 8;
        if (col < a.K) *reinterpret_cast<h8_t*>(&xnorm[r * a.K + col]) = rms_apply(v[c], w[c], rr);
      }
      __syncthreads();  // before `part` is written again, and before the loop reads xnorm
    }
  }

  // Groups gb + wave, gb + wave + WAVES, ... with the next group's loads in
  // flight while the current one is computed.  The scheduling barriers keep
  // the compiler from sinking the prefetch below the compute it is meant to
  // overlap.
  if (g < ge) {
    if constexpr (!NORM) load(s0, g, true);
    while (true) {
      const int g1 = g + WAVES;
      load(s1, g1, g1 < ge);
      __builtin_amdgcn_sched_barrier(0);
      compute(s0);
      __builtin_amdgcn_sched_barrier(0);
      if (g1 >= ge) break;
      const int g2 = g1 + WAVES;
      load(s0, g2, g2 < ge);
      __builtin_amdgcn_sched_barrier(0);
      compute(s1);
      __builtin_amdgcn_sched_barrier(0);
      if (g2 >= ge) break;
      g = g2;
    }
  }

  // Lane (q, kb) holds rows 16*t + 4*kb + i of columns col + j.  Sum the
  // waves in LDS in wave order.
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int i = 0; i < LANE_ROWS; ++i) {
      const int r = 16 * t + 4 * kb + i;
      if (r < MT) red[wave][r][q] = f4_t{tot[t][0][i], tot[t][1][i], tot[t][2][i], tot[t][3][i]};
    }
  __syncthreads();

  // Thread e of the workgroup owns (row e / 16, column quad e % 16) -- or,
  // with the SwiGLU epilogue, (row e / 8, output quad e % 8), reading gate
  // quad e % 8 and up quad e % 8 + 8 of the strip.
  const bool direct = a.splits == 1;
  auto wave_sum = [&](int r, int qq) {
    f4_t sum = red[0][r][qq];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      const f4_t v = red[w][r][qq];
      sum[0] += v[0];
      sum[1] += v[1];
      sum[2] += v[2];
      sum[3] += v[3];
    }
    return sum;
  };
  if (direct) {
    emit_outputs<MT, THREADS>(a, strip, m_base, mrows, wave_sum);
    return;
  }
  for (int e = threadIdx.x; e < MT * 16; e += THREADS) {
    const int r = e >> 4, qq = e & 15;
    const int ocol = strip * kStripCols + 4 * qq;
    if (r >= mrows || ocol >= a.N) continue;
    const int gr = m_base + r;
    const f4_t sum = wave_sum(r, qq);
    float* dst = a.partial + (static_cast<size_t>(split) * a.M + gr) * a.N + ocol;
#pragma unroll
    for (int c = 0; c < 4; ++c) store_coherent(dst + c, sum[c]);
  }

  // Publish this split's partial; the last workgroup of the strip reduces.
  // The partials were written with device-coherent stores; waiting for them
  // to complete orders them before the counter update without the whole-L2
  // write-back / invalidate an agent-scope fence costs on a multi-XCD device.
  wait_vm_stores();
  __syncthreads();
  uint32_t* counter = a.counters + blockIdx.z * gridDim.x + strip;
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == static_cast<uint32_t>(a.splits - 1));
  }
  __syncthreads();
  if (!s_last) return;

  auto split_sum = [&](int r, int qq) {
    const int ocol = strip * kStripCols + 4 * qq;
    f4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp = 0; sp < a.splits; ++sp) {
      const float* src = a.partial + (static_cast<size_t>(sp) * a.M + m_base + r) * a.N + ocol;
#pragma unroll
      for (int c = 0; c < 4; ++c) sum[c] += load_coherent(src + c);
    }
    return sum;
  };
  emit_outputs<MT, THREADS>(a, strip, m_base, mrows, split_sum);
  if (threadIdx.x == 0)
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

int mt_for(int64_t M) {
  return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : M <= 16 ? 16 : 32;
}

// Largest workgroup the LDS reduction buffer (waves x rows x 256 B) allows
// within 64 KiB.
int max_waves_for(int mt) { return std::min(16, 256 / mt); }

constexpr int kDefaultWaves = 4;
// Quant groups per wave a split aims for.  Measured on MI355X at M = 1 and 4:
// one split is best up to K = 32 * 128 (the cross-workgroup reduction costs
// more than it spreads), and larger K is split so each wave streams about
// eight groups -- 14336 x 4096 is fastest at 4 splits, 8192 x 8192 at 2.
constexpr int kGroupsPerWave = 8;

template <int MT, int GROUP, bool STREAM>
hipError_t launch_mts(const GemvArgs& a, const StreamPlan& p, hipStream_t stream) {
  dim3 grid(p.strips, p.splits, p.mblocks);
  if (a.norm_w != nullptr) {
    // The fused-RMSNorm form: one row block of at most 8 rows, 4 waves
    // (validated on the host), the block's normalised rows in dynamic LDS.
    if constexpr (MT <= 8) {
      if (p.waves != 4 || p.mblocks != 1) return hipErrorInvalidValue;
      const size_t lds = static_cast<size_t>(MT) * a.K * sizeof(_Float16);
      gemv_mfma_kernel<MT, GROUP, 4, STREAM, true><<<grid, 256, lds, stream>>>(a);
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
  switch (p.waves) {
    case 1: gemv_mfma_kernel<MT, GROUP, 1, STREAM><<<grid, 64, 0, stream>>>(a); break;
    case 2: gemv_mfma_kernel<MT, GROUP, 2, STREAM><<<grid, 128, 0, stream>>>(a); break;
    case 4: gemv_mfma_kernel<MT, GROUP, 4, STREAM><<<grid, 256, 0, stream>>>(a); break;
    case 8: gemv_mfma_kernel<MT, GROUP, 8, STREAM><<<grid, 512, 0, stream>>>(a); break;
    case 16:
      if constexpr (MT <= 16) {
        gemv_mfma_kernel<MT, GROUP, 16, STREAM><<<grid, 1024, 0, stream>>>(a);
        break;
      } else {
        return hipErrorInvalidValue;
      }
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Row blocks of fewer than 32 rows always fit one block; 32-row blocks take
// the non-temporal loads only when the batch is a single block.
template <int MT, int GROUP>
hipError_t launch_mt(const GemvArgs& a, const StreamPlan& p, hipStream_t stream) {
  if constexpr (MT < 32) {
    return launch_mts<MT, GROUP, true>(a, p, stream);
  } else {
    return p.mblocks == 1 ? launch_mts<MT, GROUP, true>(a, p, stream)
                          : launch_mts<MT, GROUP, false>(a, p, stream);
  }
}

template <int GROUP>
hipError_t launch_group(const GemvArgs& a, const StreamPlan& p, hipStream_t stream) {
  switch (p.mt) {
    case 1: return launch_mt<1, GROUP>(a, p, stream);
    case 2: return launch_mt<2, GROUP>(a, p, stream);
    case 4: return launch_mt<4, GROUP>(a, p, stream);
    case 8: return launch_mt<8, GROUP>(a, p, stream);
    case 16: return launch_mt<16, GROUP>(a, p, stream);
    default: return launch_mt<32, GROUP>(a, p, stream);
  }
}

}  // namespace

// Split heuristic: whole K in one workgroup per 64-column strip unless a wave
// would have to stream more than kGroupsPerWave groups, in which case K is
// split evenly.  Overrides follow the reference: splits are floor-then-trimmed
// (csrc/gemv_w4a16.cu:398-401).
int plan_stream(int64_t M, int64_t K, int64_t N, int64_t G, bool split_k, int64_t splits_override,
                int64_t threads_override, StreamPlan* p) {
  if (M < 1 || M > kStreamMaxM || K <= 0 || N <= 0 || (G != 64 && G != 128) || K % G != 0)
    return fail(NIBBLE_ERR_INVALID_ARGUMENT, "no streaming plan for M=%lld K=%lld N=%lld G=%lld",
                (long long)M, (long long)K, (long long)N, (long long)G);
  p->mt = mt_for(std::min<int64_t>(M, 32));
  p->mblocks = static_cast<int>(ceil_div(M, p->mt));
  // A 32-thread block (accepted by the reference, csrc/gemv_w4a16.cu:384-385)
  // runs as one wave64.
  p->waves = threads_override > 0 ? std::max(1, static_cast<int>(threads_override / 64))
                                  : kDefaultWaves;
  if (p->waves > max_waves_for(p->mt))
    return fail(NIBBLE_ERR_UNSUPPORTED, "block_threads=%lld too large for M=%lld (max %d)",
                (long long)threads_override, (long long)M, max_waves_for(p->mt) * 64);
  p->strips = static_cast<int>(ceil_div(N, kStripCols));
  const int groups = static_cast<int>(K / G);
  int gps = groups;  // groups per split
  if (split_k && splits_override > 0) {
    const int want = static_cast<int>(std::min<int64_t>(splits_override, groups));
    gps = std::max(1, groups / want);
  } else if (split_k) {
    const int want = static_cast<int>(ceil_div(groups, kGroupsPerWave * p->waves));
    gps = static_cast<int>(ceil_div(groups, std::max(1, want)));
  }
  const int splits = static_cast<int>(ceil_div(groups, gps));
  p->splits = splits;
  p->groups_per_split = gps;
  if (splits > 1) {
    p->counter_bytes = align_up(static_cast<size_t>(p->strips) * p->mblocks * 4, 256);
    p->workspace_bytes = p->counter_bytes + static_cast<size_t>(splits) * M * N * 4;
  } else {
    p->counter_bytes = 0;
    p->workspace_bytes = 0;
  }
  return NIBBLE_OK;
}

bool stream_supported(const void* X, const void* Wq, const void* S, const void* Y, int64_t M,
                      int64_t K, int64_t N, int64_t G) {
  const int64_t lim = int64_t(1) << 31;
  return N % 4 == 0 && aligned(X, 16) && aligned(Wq, 16) && aligned(S, 8) && aligned(Y, 8) &&
         (K / 8) * N * 4 < lim && M * K * 2 < lim && (K / G) * N * 2 < lim;
}

int launch_stream(const void* X, const void* Wq, const void* S, void* Y, int64_t M, int64_t K,
                  int64_t N, int64_t G, const StreamPlan& p, void* workspace,
                  size_t workspace_bytes, hipStream_t stream, const char* who, int epilogue,
                  const void* bias, const void* norm_w, float norm_eps) {
  if (p.workspace_bytes > 0) {
    if (workspace == nullptr || workspace_bytes < p.workspace_bytes)
      return fail(NIBBLE_ERR_WORKSPACE, "%s needs %zu bytes of workspace, got %zu", who,
                  p.workspace_bytes, workspace == nullptr ? size_t(0) : workspace_bytes);
    if (!aligned(workspace, 256))
      return fail(NIBBLE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }
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
  a.epilogue = epilogue;
  a.bias = static_cast<const _Float16*>(bias);
  a.norm_w = static_cast<const _Float16*>(norm_w);
  a.norm_eps = norm_eps;
  hipError_t e = G == 128 ? launch_group<128>(a, p, stream) : launch_group<64>(a, p, stream);
  if (e != hipSuccess) return hip_fail(e, who);
  return NIBBLE_OK;
}

namespace {
}  // namespace

// Mirrors check_inputs (csrc/gemv_w4a16.cu:251-265) on shapes; pure host code.
int validate_gemv(const void* X, int64_t x_rows, int64_t x_cols, const void* Wq, int64_t wq_rows,
                  int64_t wq_cols, const void* S, int64_t s_rows, int64_t s_cols, int64_t group_size,
                  int64_t version, int64_t splits_override, int64_t threads_override,
                  const void* Y) {
  NIBBLE_CHECK(threads_override == 0 || threads_override == 32 || threads_override == 64 ||
                   threads_override == 128 || threads_override == 256 ||
                   threads_override == 512 || threads_override == 1024,
               "block_threads must be 0 (heuristic) or 32, 64, 128, 256, 512, 1024 (32 runs as one "
               "64-lane wave), got %lld",
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
  // The streaming kernel addresses each operand through a buffer resource
  // with 32-bit offsets and keeps 2^31 and up as its "read nothing" offset.
  const int64_t lim = int64_t(1) << 31;
  NIBBLE_CHECK(version <= 1 || ((K / 8) * N * 4 < lim && std::min<int64_t>(x_rows, 8) * K * 2 < lim &&
                                (K / group_size) * N * 2 < lim),
               "operands too large for 32-bit buffer offsets");
  // Only operands that hold elements are dereferenced (empty tensors may
  // carry a null data pointer).
  const bool x_used = x_rows * K > 0 && x_rows * N > 0;
  const bool w_used = K * N > 0 && x_rows > 0;
  const bool y_used = x_rows * N > 0;
  NIBBLE_CHECK((!x_used || X != nullptr) && (!w_used || (Wq != nullptr && S != nullptr)) &&
                   (!y_used || Y != nullptr),
               "null pointer");
  NIBBLE_CHECK((!x_used || aligned(X, 16)) && (!w_used || (aligned(Wq, 16) && aligned(S, 8))) &&
                   (!y_used || aligned(Y, 8)),
               "misaligned pointer (X and Wq need 16-byte, S and Y 8-byte alignment)");
  return NIBBLE_OK;
}

}  // namespace nibble

using namespace nibble;

namespace {
// The streaming plan for a gemv call (versions 2-4, M <= 8).
int gemv_plan(int64_t M, int64_t K, int64_t N, int64_t G, int64_t version, int64_t splits_override,
              int64_t threads_override, StreamPlan* p) {
  return plan_stream(M, K, N, G, version == 4, splits_override, threads_override, p);
}

bool gemv_plannable(int64_t M, int64_t K, int64_t N, int64_t G, int64_t version) {
  return version >= 2 && version <= 4 && M > 0 && M <= 8 && N > 0 && K > 0 &&
         (G == 64 || G == 128) && K % G == 0;
}
}  // namespace

extern "C" size_t nibble_gemv_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                              int64_t version, int64_t splits_override,
                                              int64_t threads_override, void* stream) {
  (void)stream;
  StreamPlan p;
  if (!gemv_plannable(M, K, N, group_size, version) ||
      gemv_plan(M, K, N, group_size, version, splits_override, threads_override, &p) != NIBBLE_OK)
    return 0;
  return p.workspace_bytes;
}

extern "C" size_t nibble_gemv_counter_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                            int64_t version, int64_t splits_override,
                                            int64_t threads_override, void* stream) {
  (void)stream;
  StreamPlan p;
  if (!gemv_plannable(M, K, N, group_size, version) ||
      gemv_plan(M, K, N, group_size, version, splits_override, threads_override, &p) != NIBBLE_OK)
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

  StreamPlan p;
  rc = gemv_plan(M, K, N, group_size, version, splits_override, threads_override, &p);
  if (rc != NIBBLE_OK) return rc;
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  rc = launch_stream(X, Wq, S, Y, M, K, N, group_size, p, workspace, workspace_bytes, stream,
                     "gemv kernel launch");
  return rc == NIBBLE_OK ? ok() : rc;
}

// ---------------------------------------------------------------------------
// Streaming matmul with a fused output epilogue (no counterpart in the
// reference, whose QuantLinear adds the bias as a separate fp16 op,
// python/nibblegemm/ops.py:131-135).

namespace {
int validate_fused(const void* X, int64_t x_rows, int64_t x_cols, const void* Wq, int64_t wq_rows,
                   int64_t wq_cols, const void* S, int64_t s_rows, int64_t s_cols,
                   int64_t group_size, int64_t epilogue, const void* bias, const void* norm_w,
                   float norm_eps, const void* Y) {
  NIBBLE_CHECK(x_rows >= 0 && x_cols > 0 && wq_rows >= 0 && wq_cols > 0 && s_rows >= 0 && s_cols >= 0,
               "bad dimension (K and N must be positive)");
  const int64_t M = x_rows, K = x_cols, N = wq_cols;
  NIBBLE_CHECK(M <= kStreamMaxM, "fused matmul supports M <= %d, got %lld", kStreamMaxM,
               (long long)M);
  NIBBLE_CHECK(wq_rows * 8 == K, "packed weight rows disagree with K");
  NIBBLE_CHECK(group_size == 64 || group_size == 128, "group_size must be 64 or 128");
  NIBBLE_CHECK(s_rows * group_size == K, "scale rows disagree with K/group_size");
  NIBBLE_CHECK(s_cols == N, "scale columns disagree with N");
  NIBBLE_CHECK(N % 4 == 0, "N must be a multiple of 4");
  NIBBLE_CHECK(epilogue == kEpilogueNone || epilogue == kEpilogueBias ||
                   epilogue == kEpilogueSwiglu,
               "epilogue must be 0 (none), 1 (bias) or 2 (swiglu), got %lld", (long long)epilogue);
  NIBBLE_CHECK(epilogue != kEpilogueSwiglu || N % kStripCols == 0,
               "swiglu needs N (gate|up interleaved in 32-column blocks) to be a multiple of 64");
  NIBBLE_CHECK(epilogue != kEpilogueBias || M == 0 || bias != nullptr, "null bias");
  NIBBLE_CHECK(epilogue != kEpilogueBias || aligned(bias, 2), "misaligned bias");
  if (norm_w != nullptr) {
    NIBBLE_CHECK(M <= kNormMaxM, "the fused RMSNorm supports M <= %d, got %lld", kNormMaxM,
                 (long long)M);
    NIBBLE_CHECK(K <= kNormMaxK, "the fused RMSNorm supports K <= %d, got %lld", kNormMaxK,
                 (long long)K);
    // The block's normalised rows live in LDS: mt x K fp16 within 64 KiB.
    NIBBLE_CHECK(M == 0 || mt_for(M) * K * 2 <= 65536,
                 "the fused RMSNorm needs %lld rows x K=%lld fp16 of LDS, above 64 KiB",
                 (long long)mt_for(M), (long long)K);
    NIBBLE_CHECK(aligned(norm_w, 16), "norm weight must be 16-byte aligned");
    NIBBLE_CHECK(std::isfinite(norm_eps) && norm_eps >= 0.0f, "norm eps must be finite and >= 0");
  }
  if (M == 0) return NIBBLE_OK;
  NIBBLE_CHECK(X != nullptr && Wq != nullptr && S != nullptr && Y != nullptr, "null pointer");
  NIBBLE_CHECK(stream_supported(X, Wq, S, Y, M, K, N, group_size),
               "operands must be aligned (X, Wq 16-byte; S, Y 8-byte) and within 32-bit offsets");
  return NIBBLE_OK;
}
}  // namespace

extern "C" size_t nibble_matmul_fused_workspace_bytes(int64_t M, int64_t K, int64_t N,
                                                      int64_t group_size, void* stream) {
  (void)stream;
  StreamPlan p;
  if (M < 1 || M > kStreamMaxM || K <= 0 || N <= 0 || (group_size != 64 && group_size != 128) ||
      K % group_size != 0 || plan_stream(M, K, N, group_size, true, 0, 0, &p) != NIBBLE_OK)
    return 0;
  return p.workspace_bytes;
}

extern "C" size_t nibble_matmul_fused_counter_bytes(int64_t M, int64_t K, int64_t N,
                                                    int64_t group_size, void* stream) {
  (void)stream;
  StreamPlan p;
  if (M < 1 || M > kStreamMaxM || K <= 0 || N <= 0 || (group_size != 64 && group_size != 128) ||
      K % group_size != 0 || plan_stream(M, K, N, group_size, true, 0, 0, &p) != NIBBLE_OK)
    return 0;
  return p.counter_bytes;
}

extern "C" int nibble_matmul_w4a16_fused(const void* X, int64_t x_rows, int64_t x_cols,
                                         const void* Wq, int64_t wq_rows, int64_t wq_cols,
                                         const void* S, int64_t s_rows, int64_t s_cols,
                                         int64_t group_size, int64_t epilogue, const void* bias,
                                         const void* norm_weight, float norm_eps, void* Y,
                                         void* workspace, size_t workspace_bytes, void* stream_) {
  int rc = validate_fused(X, x_rows, x_cols, Wq, wq_rows, wq_cols, S, s_rows, s_cols, group_size,
                          epilogue, bias, norm_weight, norm_eps, Y);
  if (rc != NIBBLE_OK) return rc;
  const int64_t M = x_rows, K = x_cols, N = wq_cols;
  if (M == 0) return ok();
  StreamPlan p;
  rc = plan_stream(M, K, N, group_size, true, 0, 0, &p);
  if (rc != NIBBLE_OK) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  rc = launch_stream(X, Wq, S, Y, M, K, N, group_size, p, workspace, workspace_bytes, stream,
                     "fused matmul kernel launch", static_cast<int>(epilogue), bias, norm_weight,
                     norm_eps);
  return rc == NIBBLE_OK ? ok() : rc;
}
