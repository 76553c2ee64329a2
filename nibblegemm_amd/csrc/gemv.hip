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
#include <mutex>

#include "nibble_common.h"
#include "nibble_decode.h"
#include "nibble_epilogue.h"
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
  int strips;             // strip kernel: column strips of the launch
  int strips_per_xcd;     // strip kernel: strips run by each XCD's workgroups
  int stage_x;            // strip kernel: copy the activations to LDS (if they fit 64 KiB)
  // Where the weights and scales of a column live (packed or strip-major).
  WeightLayout L;
  // Strip kernel at M = 1 only (diagnostics): per wave 8 uint64, the
  // timeline that nibble_gemv_timeline documents; null when off.
  unsigned long long* stamps = nullptr;
};

// Whether a kernel that rebuilds the weight layout from w_row and the strip
// shift (the strip kernel) sees the call's layout: every layout has
// s_row = w_row / 2, w_strip = (K / 8) w_row and s_strip = (K / GROUP) s_row.
inline bool layout_rebuilds(const GemvArgs& a, int group) {
  const uint32_t K = static_cast<uint32_t>(a.K);
  const bool packed = a.L.strip_shift == 31;  // one strip: the strip strides are unused
  return a.L.s_row == a.L.w_row / 2 && (packed || a.L.w_strip == (K / 8) * a.L.w_row) &&
         (packed || a.L.s_strip == (K / static_cast<uint32_t>(group)) * a.L.s_row);
}

__device__ __forceinline__ f4_t mfma16(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Writes a strip's outputs from `total(r, qq)`, the fp32 sums of column quad
// qq of row r, through the launch's epilogue.  SW is the strip width in
// columns; the SwiGLU epilogue needs strips of whole gate|up block pairs.
template <int MT, int THREADS, int SW = kStripCols, typename Total>
__device__ __forceinline__ void emit_outputs(const GemvArgs& a, int strip, int m_base, int mrows,
                                             Total total) {
  constexpr int QUADS = SW / 4;
  if constexpr (SW >= 2 * kSwigluBlock) {
    if (a.epilogue == kEpilogueSwiglu) {
      // The strip holds SW / 32 pairs of 16 gate columns and the matching 16
      // up columns; output quad o reads gate quad 8 (o / 4) + o % 4 and the
      // up quad 4 columns later.
      const int nout = a.N / 2;
      for (int e = threadIdx.x; e < MT * (QUADS / 2); e += THREADS) {
        const int r = e / (QUADS / 2), o = e % (QUADS / 2);
        const int gq = 8 * (o / 4) + o % 4;
        const int ocol = strip * (SW / 2) + 4 * o;
        if (r >= mrows || ocol >= nout) continue;
        const f4_t g = total(r, gq), u = total(r, gq + 4);
        const h4_t y = {(_Float16)silu_mul(g[0], u[0]), (_Float16)silu_mul(g[1], u[1]),
                        (_Float16)silu_mul(g[2], u[2]), (_Float16)silu_mul(g[3], u[3])};
        *reinterpret_cast<h4_t*>(a.Y + static_cast<size_t>(m_base + r) * nout + ocol) = y;
      }
      return;
    }
  }
  for (int e = threadIdx.x; e < MT * QUADS; e += THREADS) {
    const int r = e / QUADS, qq = e % QUADS;
    const int ocol = strip * SW + 4 * qq;
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

// The fused-RMSNorm prologue: rows [m_base, m_base + mrows) of X, normalised
// into `xnorm` ([rows][K] fp16 in LDS) as fp16(x * r * norm_w), with r
// computed exactly as the RMSNorm kernel does -- the first 256 threads hold
// chunks (256 c + t) * 8 of the row (K <= 16384: at most 8), x and the weight
// loaded before the reduction, the squares reduced in the same fixed order --
// so the fused launch has the two-step composition's bits.  Threads past the
// first 256 only pass the same barriers.
template <int THREADS>
__device__ __forceinline__ void norm_rows_to_lds(const GemvArgs& a, int m_base, int mrows,
                                                 _Float16* xnorm) {
  static_assert(THREADS % kRmsThreads == 0, "the RMSNorm prologue runs on 256-thread multiples");
  __shared__ float part[kRmsThreads / 64];
  constexpr int kMaxChunks = kNormMaxK / (kRmsThreads * 8);
  const int tid = threadIdx.x;
  const bool active = THREADS == kRmsThreads || tid < kRmsThreads;
  for (int r = 0; r < mrows; ++r) {
    const _Float16* xr = a.X + static_cast<size_t>(m_base + r) * a.K;
    h8_t v[kMaxChunks], w[kMaxChunks];
    float ss = 0.0f;
    if (active) {
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        const int col = (c * kRmsThreads + tid) * 8;
        v[c] = col < a.K ? *reinterpret_cast<const h8_t*>(xr + col) : h8_t{};
        w[c] = col < a.K ? *reinterpret_cast<const h8_t*>(a.norm_w + col) : h8_t{};
        ss = sumsq_chunk(v[c], ss);
      }
      ss = wave_sum(ss);
      if ((tid & 63) == 0) part[tid >> 6] = ss;
    }
    __syncthreads();
    const float total = ((part[0] + part[1]) + part[2]) + part[3];
    if (active) {
      const float rr = rms_scale(total, a.K, a.norm_eps);
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        const int col = (c * kRmsThreads + tid) * 8;
        if (col < a.K) *reinterpret_cast<h8_t*>(&xnorm[r * a.K + col]) = rms_apply(v[c], w[c], rr);
      }
    }
    __syncthreads();  // before `part` is written again, and before the loop reads xnorm
  }
}

// norm_rows_to_lds for rows already copied to LDS: `xs` holds the raw
// activation rows [mrows][K] and `ws` the norm weight [K]; each row is
// normalised in place with norm_rows_to_lds's chunking and arithmetic (the
// same bits).  All rows at once: the workgroup's 256-thread groups take
// every (THREADS / 256)-th row, each row's sum of squares is formed as in
// the RMSNorm kernel, and one barrier separates the sums from the
// normalisation.  Measured against rows one at a time (two barriers each):
// 4096 x 6144 M = 1 / 2 / 4 / 8 5.9 / 6.3 / 7.6 / 9.9 us against 6.1 / 7.3 /
// 9.6 / 13.8; 4096 x 4096 M = 1 5.5 against 5.3 (code layout), M = 8 9.8
// against 13.8.
template <int THREADS, int MT>
__device__ __forceinline__ void norm_rows_in_lds(const GemvArgs& a, int mrows, _Float16* xs,
                                                 const _Float16* ws) {
  static_assert(THREADS % kRmsThreads == 0, "the RMSNorm prologue runs on 256-thread multiples");
  constexpr int GROUPS = THREADS / kRmsThreads;
  constexpr int RPG = (MT + GROUPS - 1) / GROUPS;  // rows per 256-thread group
  constexpr int kMaxChunks = kNormMaxK / (kRmsThreads * 8);
  __shared__ float part[MT][kRmsThreads / 64];
  const int tid = threadIdx.x % kRmsThreads;
  const int grp = threadIdx.x / kRmsThreads;
#pragma unroll
  for (int i = 0; i < RPG; ++i) {
    const int r = grp + GROUPS * i;
    if (r < mrows) {  // uniform across each wave
      float ss = 0.0f;
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        const int col = (c * kRmsThreads + tid) * 8;
        if (col < a.K) ss = sumsq_chunk(*reinterpret_cast<const h8_t*>(&xs[r * a.K + col]), ss);
      }
      ss = wave_sum(ss);
      if ((tid & 63) == 0) part[r][tid >> 6] = ss;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RPG; ++i) {
    const int r = grp + GROUPS * i;
    if (r < mrows) {
      const float total = ((part[r][0] + part[r][1]) + part[r][2]) + part[r][3];
      const float rr = rms_scale(total, a.K, a.norm_eps);
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        const int col = (c * kRmsThreads + tid) * 8;
        if (col < a.K) {
          _Float16* const x = &xs[r * a.K + col];
          *reinterpret_cast<h8_t*>(x) = rms_apply(*reinterpret_cast<const h8_t*>(x),
                                                 *reinterpret_cast<const h8_t*>(&ws[col]), rr);
        }
      }
    }
  }
  __syncthreads();  // before the loop reads xs
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
  const uint32_t row_bytes = a.L.w_row;

  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(a.Wq, static_cast<uint32_t>(a.K / 8) * static_cast<uint32_t>(a.N) * 4u);
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(a.X, static_cast<uint32_t>(a.M) * static_cast<uint32_t>(a.K) * 2u);
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(a.S, static_cast<uint32_t>(a.K / GROUP) * static_cast<uint32_t>(a.N) * 2u);
  const uint32_t voff_w = col_ok ? kb * row_bytes + a.L.wcol(col) : kOutOfRange;
  const uint32_t voff_s = col_ok ? a.L.scol(col) : kOutOfRange;
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
        h4_t, __builtin_amdgcn_raw_buffer_load_b64(rs, voff_s, static_cast<uint32_t>(g) * a.L.s_row,
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
    norm_rows_to_lds<THREADS>(a, m_base, mrows, xnorm);
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
    f4_t v[WAVES];
#pragma unroll
    for (int w = 0; w < WAVES; ++w) v[w] = red[w][r][qq];
    __builtin_amdgcn_sched_barrier(0);  // every read ahead of the adds
    f4_t sum = v[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      sum[0] += v[w][0];
      sum[1] += v[w][1];
      sum[2] += v[w][2];
      sum[3] += v[w][3];
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
  // Relies on gfx950 hardware ordering: see "HARDWARE ASSUMPTION" in
  // nibble_decode.h.
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

  // The partials of up to kSplitBatch splits are loaded in one round and then
  // added in split order: one memory round trip per batch instead of one per
  // split.  Loads past the last split re-read split 0 and are not added.
  auto split_sum = [&](int r, int qq) {
    constexpr int kSplitBatch = 8;
    const int ocol = strip * kStripCols + 4 * qq;
    f4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp0 = 0; sp0 < a.splits; sp0 += kSplitBatch) {
      f4_t v[kSplitBatch];
#pragma unroll
      for (int b = 0; b < kSplitBatch; ++b) {
        const int sp = sp0 + b < a.splits ? sp0 + b : 0;
        const float* src = a.partial + (static_cast<size_t>(sp) * a.M + m_base + r) * a.N + ocol;
#pragma unroll
        for (int c = 0; c < 4; ++c) v[b][c] = load_coherent(src + c);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < kSplitBatch; ++b)
        if (sp0 + b < a.splits) {
#pragma unroll
          for (int c = 0; c < 4; ++c) sum[c] += v[b][c];
        }
    }
    return sum;
  };
  emit_outputs<MT, THREADS>(a, strip, m_base, mrows, split_sum);
  if (threadIdx.x == 0)
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The staging wave's copy of one activation window: COPIES LDS-DMA loads of
// 16 bytes a lane, load j landing at dst + 1 KiB j.  Lane unit j reads
// activation k = k0 + dma_k[j] of the row at byte dma_row[j]; rows past M
// (dma_row[j] == kOutOfRange) and k past K take the out-of-range offset: no
// memory access.  (The resource is built here from X and its byte extent:
// the host pass cannot take a buffer resource as a template function's
// parameter.)
template <int COPIES>
__device__ __forceinline__ void copy_window(const void* X, uint32_t xbytes, unsigned char* dst,
                                            uint32_t k0, uint32_t K, const uint32_t* dma_k,
                                            const uint32_t* dma_row) {
  using lds_ptr = __attribute__((address_space(3))) void*;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(X, xbytes);
#pragma unroll
  for (int j = 0; j < COPIES; ++j) {
    const uint32_t k = k0 + dma_k[j];
    const uint32_t off = dma_row[j] == kOutOfRange || k >= K ? kOutOfRange : dma_row[j] + 2u * k;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(dst + j * 1024), 16, off, 0, 0, 0);
  }
}

// Batch kernel: 12 to 64 activation rows (small batches through gemm) in one
// block of MT = 16, 32 or 64 rows.  The split kernel's geometry -- one
// workgroup per 64-column strip and K split, its 4 waves taking the split's
// quant groups round-robin (SPW = 2: a workgroup takes two adjacent strips,
// 4 waves each, sharing the activation copies) -- and its arithmetic: per
// group the same pre-scaled activations, correction MFMA, decode and MFMA
// sequence, the same per-group scaling into fp32 totals, the same wave and
// split reduction order.  A launch with the split kernel's plan returns the
// split kernel's bits.
//
// What differs is where the activations come from.  The split kernel loads
// a 16-byte activation chunk per lane per MFMA -- 2 x GROUP / 32 loads per
// group beside GROUP / 32 weight loads, each touching 16 rows -- and holds
// them in registers for the two groups in flight.  Here the 4 groups the
// waves take in one step form one K window of the activations, which
// STAGERS staging waves (waves 4..) copy once into an LDS ring slot by
// LDS-DMA (1 KiB per instruction, whole rows; rows past M are not read); the
// MFMA operands are ds_read_b128s, and the registers hold DEPTH steps of
// weight loads.  The copies are the staging waves' only vector-memory
// operations, so the compute waves' waits cover their own weight loads
// alone (vmcnt completes in order: copies interleaved with the weight loads
// would make every wait for a copy also wait for the older weight loads).
//
// Ring protocol, per step i (one workgroup barrier a step):
//   barrier B(i) -- a staging wave arrives once its copies of step i have
//     landed, the compute waves once they are done with step i - 1's slot;
//   staging waves: their copies of step i + RING - 1 into step i - 1's slot
//     (past the last step: out-of-range offsets), then wait until only their
//     newest RING - 2 slots' copies are in flight (step i + 1's have landed);
//   compute waves: step i from its slot and the weights loaded DEPTH steps
//     ago, then the weight loads of step i + DEPTH (past the last step:
//     out-of-range offsets, no memory access).
// A slot row is the window's 4 x GROUP k; 16-byte unit u of row r is stored
// at unit u ^ (r % 16), so the 16 rows a ds_read_b128 quarter-wave reads
// fall in 16 different bank groups.  After the loop the ring holds the wave
// totals.  Rows past M hold whatever the ring held: MFMA row m of the output
// depends on activation row m alone, and those rows are never written.
//
// Moving the activations into a CU costs about as much per byte as the
// weight stream, by either path (per-lane loads or LDS-DMA): measured with
// the split kernel at 4096 x 14336, M = 32, the texture-address unit was
// 64-78% busy, half of that stalled by the L1.  The copies here are whole
// 1 KiB rows issued by STAGERS waves that do nothing else, so they flow
// beside the weight loads instead of in the compute waves' own queues.
template <int MT, int GROUP, int DEPTH, int RING, int STAGERS, bool STREAM, int SPW = 1>
__global__ __launch_bounds__((4 * SPW + STAGERS) * 64) void gemv_batch_kernel(GemvArgs a) {
  static_assert(MT == 16 || MT == 32 || MT == 64, "16-row MFMA tiles");
  static_assert(SPW == 1 || (SPW == 2 && MT != 64), "strips per workgroup: 1, or 2 below 64 rows");
  constexpr int kWaves = 4;                // group waves: the quant groups of one step
  constexpr int kCompute = kWaves * SPW;   // compute waves: kWaves per strip
  constexpr int THREADS = (kCompute + STAGERS) * 64;
  constexpr int kWPolicy = STREAM ? 2 : 0;
  constexpr int kPolicySc1 = 16;                  // agent-coherent: misses a stale L2 line
  constexpr int CPG = GROUP / 32;
  constexpr int TILES = MT / 16;
  constexpr uint32_t UPR = kWaves * GROUP / 8;    // 16-byte units per slot row
  constexpr uint32_t SLOT_BYTES = MT * UPR * 16;
  constexpr int COPIES = MT * UPR / 64 / STAGERS;  // each staging wave's loads per slot
  constexpr int WAIT_X = (RING - 2) * COPIES;
  constexpr int QUADS = kStripCols / 4;
  static_assert(UPR >= 16 && (MT * UPR) % (64 * STAGERS) == 0, "swizzle within a row, whole copies");
  static_assert(RING >= 2 && WAIT_X <= 63, "vmcnt range");
  static_assert(SPW * kWaves * MT * 16 * 16 <= RING * SLOT_BYTES, "the wave totals fit the ring");
  extern __shared__ __attribute__((aligned(16))) unsigned char ring[];
  __shared__ int s_last;

  const uint32_t lane = threadIdx.x & 63u;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool stager = wave >= kCompute;
  // Compute wave w takes group slot gw of every step in strip sp of the
  // workgroup's SPW adjacent strips; the activation window is copied once for
  // all of them.
  const int gw = wave % kWaves, sp = stager ? 0 : wave / kWaves;
  const int tile = blockIdx.x;
  const int strip = tile * SPW + sp;
  const int split = blockIdx.y;
  const int m_base = blockIdx.z * MT;
  const int mrows = min(MT, a.M - m_base);
  const uint32_t K = static_cast<uint32_t>(a.K);
  const uint32_t q = lane & 15u, kb = lane >> 4;
  const int col = strip * kStripCols + 4 * static_cast<int>(q);
  const bool col_ok = col < a.N;
  const uint32_t row_bytes = a.L.w_row;

  const int total_groups = a.K / GROUP;
  const int gb = split * a.groups_per_split;
  const int ge = min(gb + a.groups_per_split, total_groups);
  const int steps = (ge - gb + kWaves - 1) / kWaves;

  f4_t tot[TILES][4];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) tot[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  if (stager) {
    // Lane unit of copy j: slot row r, window unit u stored at u ^ (r % 16).
    const uint32_t xbytes = static_cast<uint32_t>(a.M) * K * 2u;
    uint32_t dma_k[COPIES], dma_row[COPIES];
#pragma unroll
    for (int j = 0; j < COPIES; ++j) {
      const uint32_t e = static_cast<uint32_t>((wave - kCompute) * COPIES + j) * 64u + lane;
      const uint32_t r = e / UPR, pos = e % UPR;
      dma_k[j] = 8u * (pos ^ (r & 15u));
      dma_row[j] = static_cast<int>(r) < mrows ? (static_cast<uint32_t>(m_base) + r) * K * 2u
                                               : kOutOfRange;
    }
    auto copy = [&](int step, uint32_t slot) {
      copy_window<COPIES>(a.X, xbytes, ring + slot * SLOT_BYTES + (wave - kCompute) * COPIES * 1024,
                          static_cast<uint32_t>(gb + step * kWaves) * GROUP, K, dma_k, dma_row);
    };
#pragma unroll
    for (int s = 0; s < RING - 1; ++s) copy(s, s);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(WAIT_X));
    uint32_t slot = 0;
    for (int i = 0; i < steps; ++i) {
      lds_barrier();  // B(i)
      copy(i + RING - 1, slot == 0 ? RING - 1 : slot - 1);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(WAIT_X));
      slot = slot == RING - 1 ? 0 : slot + 1;
    }
    // Every copy (including those past the last step) has landed before the
    // ring is reused for the totals.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  } else {
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(a.Wq, static_cast<uint32_t>(a.K / 8) * static_cast<uint32_t>(a.N) * 4u);
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(a.S, static_cast<uint32_t>(a.K / GROUP) * static_cast<uint32_t>(a.N) * 2u);
    const uint32_t voff_w = col_ok ? kb * row_bytes + a.L.wcol(col) : kOutOfRange;
    const uint32_t voff_s = col_ok ? a.L.scol(col) : kOutOfRange;
    struct WStage {
      u4_t w[CPG];
      h4_t s;
    };
    auto load = [&](WStage& st, int step) {
      const int g = gb + step * kWaves + gw;
      const bool in = step < steps && g < ge;
      const uint32_t vw = in ? voff_w : kOutOfRange;
      const uint32_t kw = in ? static_cast<uint32_t>(g) * (GROUP / 8) * row_bytes : 0u;
#pragma unroll
      for (int c = 0; c < CPG; ++c)
        st.w[c] = __builtin_bit_cast(
            u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, vw, kw + c * 4 * row_bytes, kWPolicy));
      st.s = __builtin_bit_cast(
          h4_t, __builtin_amdgcn_raw_buffer_load_b64(rs, in ? voff_s : kOutOfRange,
                                                     in ? static_cast<uint32_t>(g) * a.L.s_row : 0u,
                                                     kWPolicy));
    };
    const DecodeConsts dk = decode_consts();
    const h8_t xscale = biased_x_scale();
    const h8_t bcorr = biased_correction();
    // gemv_mfma_kernel's compute, the activations read from the slot.  With
    // 64 rows (4 row tiles) the activations of every chunk and tile would
    // not fit the registers beside the accumulators: chunks are taken one
    // at a time, the correction accumulated apart and added before the
    // group's scaling (the sums' order differs from the 32-row form, which
    // serves the split kernel's plans; nothing else runs 64-row blocks).
    auto compute64 = [&](const WStage& st, const unsigned char* base) {
      f4_t acc[TILES][4], corr[TILES];
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        corr[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int c = 0; c < CPG; ++c) {
        h8_t xs[TILES];
        const uint32_t u = static_cast<uint32_t>(gw * (GROUP / 8) + 4 * c) + kb;
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
          const uint32_t r = 16u * t + q;
          xs[t] = *reinterpret_cast<const h8_t*>(base + (r * UPR + (u ^ q)) * 16u) * xscale;
          corr[t] = mfma16(xs[t], bcorr, corr[t]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const h8_t b = decode8_biased(st.w[c][j], dk);
#pragma unroll
          for (int t = 0; t < TILES; ++t) acc[t][j] = mfma16(xs[t], b, acc[t][j]);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float sj = static_cast<float>(st.s[j]);
#pragma unroll
        for (int t = 0; t < TILES; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            tot[t][j][i] = __builtin_fmaf(sj, acc[t][j][i] + corr[t][i], tot[t][j][i]);
      }
    };
    auto compute = [&](const WStage& st, const unsigned char* base) {
      if constexpr (MT == 64) {
        compute64(st, base);
        return;
      }
      h8_t xs[TILES][CPG];
      f4_t acc[TILES][4];
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const uint32_t r = 16u * t + q;
        f4_t corr = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < CPG; ++c) {
          const uint32_t u = static_cast<uint32_t>(gw * (GROUP / 8) + 4 * c) + kb;
          xs[t][c] = *reinterpret_cast<const h8_t*>(base + (r * UPR + (u ^ q)) * 16u) * xscale;
          corr = mfma16(xs[t][c], bcorr, corr);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][j] = corr;
      }
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
          for (int i = 0; i < 4; ++i) tot[t][j][i] = __builtin_fmaf(sj, acc[t][j][i], tot[t][j][i]);
      }
    };

    WStage st[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      load(st[d], d);
      __builtin_amdgcn_sched_barrier(0);
    }
    uint32_t slot = 0;  // step i's slot: i % RING
    auto step = [&](WStage& sd, int i) {
      lds_barrier();  // B(i)
      if (gb + i * kWaves + gw < ge) compute(sd, ring + slot * SLOT_BYTES);
      __builtin_amdgcn_sched_barrier(0);
      load(sd, i + DEPTH);
      slot = slot == RING - 1 ? 0 : slot + 1;
    };
    // Whole blocks of DEPTH steps, then the rest: a loop whose body could
    // leave early would reach its head with stage 0's loads possibly the
    // newest, and the compiler would then drain every load there.
    int i0 = 0;
    for (; i0 + DEPTH <= steps; i0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) step(st[d], i0 + d);
    }
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d)
      if (i0 + d < steps) step(st[d], i0 + d);
  }
  lds_barrier();  // every copy has landed and every slot read is done

  // Lane (q, kb) of compute wave (sp, gw) holds rows 16 t + 4 kb + i of
  // columns 4 q + j of strip sp: red[sp][gw][row][q], summed over gw in order.
  f4_t* const red = reinterpret_cast<f4_t*>(ring);
  if (!stager) {
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * t + 4 * static_cast<int>(kb) + i;
        red[((sp * kWaves + gw) * MT + r) * 16 + q] =
            f4_t{tot[t][0][i], tot[t][1][i], tot[t][2][i], tot[t][3][i]};
      }
  }
  __syncthreads();
  auto wave_sum = [&](int s, int r, int qq) {
    f4_t v[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v[w] = red[((s * kWaves + w) * MT + r) * 16 + qq];
    __builtin_amdgcn_sched_barrier(0);
    f4_t sum = v[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      sum[0] += v[w][0];
      sum[1] += v[w][1];
      sum[2] += v[w][2];
      sum[3] += v[w][3];
    }
    return sum;
  };
  if (a.splits == 1) {
#pragma unroll
    for (int s = 0; s < SPW; ++s)
      emit_outputs<MT, THREADS>(a, tile * SPW + s, m_base, mrows,
                                [&](int r, int qq) { return wave_sum(s, r, qq); });
    return;
  }
  // The split kernel's publication and last-workgroup reduction ("HARDWARE
  // ASSUMPTION" in nibble_decode.h), with 16-byte agent-coherent accesses;
  // the last workgroup issues every split's loads before the first add.
  const uint32_t pbytes = static_cast<uint32_t>(a.splits) * static_cast<uint32_t>(a.M) *
                          static_cast<uint32_t>(a.N) * 4u;
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partial, pbytes);
  // Element e of the workgroup's outputs: strip e / (MT QUADS), then row and
  // column quad.
  auto poff = [&](int spl, int e) {
    const int s = e / (MT * QUADS), r = e % (MT * QUADS) / QUADS, qq = e % QUADS;
    return ((static_cast<uint32_t>(spl) * a.M + m_base + r) * static_cast<uint32_t>(a.N) +
            (tile * SPW + s) * kStripCols + 4 * qq) * 4u;
  };
  auto in_range = [&](int e) {
    const int s = e / (MT * QUADS), r = e % (MT * QUADS) / QUADS, qq = e % QUADS;
    return e < SPW * MT * QUADS && r < mrows && (tile * SPW + s) * kStripCols + 4 * qq < a.N;
  };
  for (int e = threadIdx.x; e < SPW * MT * QUADS; e += THREADS) {
    if (!in_range(e)) continue;
    const int s = e / (MT * QUADS), r = e % (MT * QUADS) / QUADS, qq = e % QUADS;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4_t, wave_sum(s, r, qq)), rp,
                                           poff(split, e), 0, kPolicySc1);
  }
  wait_vm_stores();
  __syncthreads();
  uint32_t* counter = a.counters + blockIdx.z * gridDim.x + tile;
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == static_cast<uint32_t>(a.splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  constexpr int PER = (SPW * MT * QUADS + THREADS - 1) / THREADS;
  constexpr int kSplitBatch = 8;
  f4_t* const sums = red;  // [SPW][MT][QUADS]
  f4_t acc[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) acc[k] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (int sp0 = 0; sp0 < a.splits; sp0 += kSplitBatch) {
    f4_t v[PER][kSplitBatch];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = threadIdx.x + k * THREADS;
      const bool ok = in_range(e);
#pragma unroll
      for (int b = 0; b < kSplitBatch; ++b)
        v[k][b] = __builtin_bit_cast(
            f4_t, __builtin_amdgcn_raw_buffer_load_b128(
                      rp, ok && sp0 + b < a.splits ? poff(sp0 + b, e) : kOutOfRange, 0,
                      kPolicySc1));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < PER; ++k)
#pragma unroll
      for (int b = 0; b < kSplitBatch; ++b)
        if (sp0 + b < a.splits) {
          acc[k][0] += v[k][b][0];
          acc[k][1] += v[k][b][1];
          acc[k][2] += v[k][b][2];
          acc[k][3] += v[k][b][3];
        }
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = threadIdx.x + k * THREADS;
    if (e < SPW * MT * QUADS) sums[e] = acc[k];
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < SPW; ++s)
    emit_outputs<MT, THREADS>(a, tile * SPW + s, m_base, mrows,
                              [&](int r, int qq) { return sums[(s * MT + r) * QUADS + qq]; });
  if (threadIdx.x == 0)
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Column-strip decode kernel (M <= 8, one launch, no cross-workgroup
// exchange).  A workgroup owns SW columns (16, 32 or 64) over the whole of K;
// its WAVES waves take contiguous ranges of quant groups, and every wave
// keeps the weight loads of DEPTH groups in flight (a register ring; ONEPASS
// when no wave has more groups than that, so every load is issued before
// the first wait).  Workgroups are numbered so that each XCD (workgroup id %
// 8 on a multi-XCD part) runs a contiguous run of strips.
//
// MFMA mapping.  A wave load is one dwordx4 per lane: lane l reads columns
// 4 c .. 4 c + 3 (c = l % LPR, LPR = SW / 4 lanes per packed row) of packed
// row r = l / LPR, so one load covers RPL = 64 / LPR packed rows (8 RPL k).
// In v_mfma_f32_16x16x32_f16 terms lane l supplies B column slot n = l % 16
// and k block b = l / 16, i.e. column 4 (n % LPR) + j of packed row
// P b + n / LPR, with P = RPL / 4 phases.  Column slots of different phases
// read different packed rows, so the A operand is laid out block-diagonally:
// A row m' = RPT p + mm (RPT = 16 / P rows per phase) holds activation row mm
// at the packed rows of phase p, and only the C entries with m' / RPT ==
// n / LPR are kept.  For SW = 64 (one phase) this is the plain mapping of
// gemv_mfma_kernel.  Phase-major rows put activation row mm of every phase in
// accumulator element mm % 4 of a lane, so at M = 1 each lane carries one
// live element per column word and the per-group scaling touches only that.
// A 16-row A tile holds RPT activation rows, so M <= 8 takes one tile for
// SW >= 32 and two for SW = 16.  The per-lane decode, the pre-scaled
// activations and the correction MFMA are those of gemv_mfma_kernel; waves
// and phases are summed in LDS in a fixed order.
//
// STAGED: the activation rows ([MT][K] fp16) and the strip's scales
// ([K / GROUP][SW] fp16) are copied into LDS once per workgroup by LDS-DMA
// buffer loads issued ahead of the weights, and the MFMA operands are read
// from there.  Per group a wave then issues only its weight loads: a
// per-lane activation load would cost a whole 64-lane address-unit pass for
// the few lanes that hold real rows at M <= 8, and a per-lane scale load the
// same for 8-byte scale quads.  NORM (RMSNorm prologue) fills the activation
// rows itself and implies STAGED.
//
// Kernel arguments.  The body takes the fields the prologue needs before its
// first weight load as scalars.  The packed-weight entry (gemv_strip_kernel)
// receives them as its first 14 scalar dwords (gfx950's limit), and the
// library is built with kernel-argument preloading, so the command processor
// writes them into SGPRs at wave launch: the copies and weight loads issue
// without a kernel-argument fetch.  The strip-major entry
// (gemv_strip_kernel_block) reads them from its argument block.  The rest of the
// call (outputs, epilogue, timeline buffer) stays in the GemvArgs block,
// which is fetched while the weights stream.  The weight layout is rebuilt
// from its row stride and strip shift (every layout has s_row = w_row / 2,
// w_strip = (K / 8) w_row and s_strip = (K / GROUP) s_row; the launcher
// checks that).  4096 x 14336 M = 1: 7.29 -> 7.00-7.07 us.  The split and
// batch kernels take the block alone: preloading their prologue fields the
// same way measured no change (14336 x 4096 M = 16..32, the 224-launch 8B
// step).
template <int MT, int GROUP, int SW, int WAVES, int DEPTH, bool NORM, bool ONEPASS, bool STAGED,
          bool TIMELINE>
__device__ __forceinline__ void strip_body(
    const _Float16* Xp, const uint32_t* Wqp, const _Float16* Sp,
    const _Float16* norm_wp, uint32_t Mp, uint32_t Kp, uint32_t Np, uint32_t strips_p,
    uint32_t w_row_p, uint32_t strip_shift_p, const GemvArgs& a) {
  // TIMELINE: s_memrealtime ticks (100 MHz) at the points nibble_gemv_timeline
  // lists; only that instantiation has them.
  unsigned long long tl[7] = {};
  if constexpr (TIMELINE) tl[0] = __builtin_amdgcn_s_memrealtime();
  constexpr int LPR = SW / 4;            // lanes per packed row
  constexpr int RPL = 64 / LPR;          // packed rows per wave load
  constexpr int P = RPL / 4;             // phases
  constexpr int KPL = 8 * RPL;           // k per wave load
  constexpr int CPG = GROUP / KPL;       // wave loads per quant group
  constexpr int RPT = 16 / P;            // activation rows per 16-row A tile
  constexpr int TILES = (MT + RPT - 1) / RPT;
  // Accumulator elements that can hold a real row: element i of row block q
  // is A row 4 q + i, activation row (4 q + i) % RPT < MT.
  constexpr int LANE_ROWS = MT < 4 ? MT : 4;
  constexpr int THREADS = WAVES * 64;
  static_assert(SW == 16 || SW == 32 || SW == 64, "strip width");
  static_assert(CPG >= 1 && GROUP % KPL == 0, "a wave load must not straddle quant groups");
  static_assert(!NORM || STAGED, "the RMSNorm prologue leaves the activations in LDS");
  static_assert(DEPTH >= 2, "the ring prepares the next stage while computing this one");
  constexpr int kWPolicy = 2;            // non-temporal: the launch reads each weight once
  __shared__ __attribute__((aligned(16))) float red[WAVES][P][MT][SW];
  // STAGED: [MT][K] activation rows, (NORM) the [K] norm weight, then
  // [K / GROUP][SW] scales.
  extern __shared__ __attribute__((aligned(16))) _Float16 xnorm[];

  // The grid is rounded up to whole XCD runs; a workgroup past the last
  // strip finds every column out of range (its loads read zeros, its stores
  // are skipped).  It does not return early: that test would need the
  // strip count before the operand pointers, two dependent kernel-argument
  // fetches ahead of the first weight load instead of one.
  // Unsigned index arithmetic throughout (divisions by powers of two become
  // shifts); every kernel argument the weight loads need is read up front.
  const uint32_t K = Kp, N = Np;
  WeightLayout L;
  L.strip_shift = strip_shift_p;
  L.w_row = w_row_p;
  L.s_row = w_row_p >> 1;
  L.w_strip = (K >> 3) * w_row_p;
  L.s_strip = (K / GROUP) * L.s_row;
  const uint32_t strip = (blockIdx.x & 7u) * ((strips_p + 7u) >> 3) + (blockIdx.x >> 3);
  const uint32_t lane = threadIdx.x & 63u;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int mrows = min(MT, static_cast<int>(Mp));
  const uint32_t total_groups = K / GROUP;

  // B side: lane (c, r).
  const uint32_t c = lane % LPR, r = lane / LPR;
  const uint32_t col = strip * SW + 4 * c;
  const bool col_ok = strip < strips_p && col < N;
  const uint32_t row_bytes = L.w_row, s_row = L.s_row;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(Wqp, (K / 8) * N * 4u);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(Xp, Mp * K * 2u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(Sp, total_groups * N * 2u);
  const uint32_t voff_w = col_ok ? r * row_bytes + L.wcol(col) : kOutOfRange;
  const uint32_t voff_s = col_ok ? L.scol(col) : kOutOfRange;
  // A side: lane (m', kb) holds row m' = RPT p + mm of each tile at k block
  // kb, i.e. the 8 k of packed row P kb + p of a wave load.
  const uint32_t mq = lane & 15u, kb = lane >> 4;
  const uint32_t ph = mq / RPT, mm = mq % RPT;
  const uint32_t kx_lane = (kb * P + ph) * 8u;
  uint32_t voff_x[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const uint32_t m = t * RPT + mm;
    voff_x[t] = m < static_cast<uint32_t>(mrows) ? (m * K + kx_lane) * 2u : kOutOfRange;
  }
  _Float16* const wn_lds = xnorm + MT * K;                     // NORM weight
  _Float16* const s_lds = wn_lds + (NORM ? K : 0u);              // STAGED scales

  // STAGED: LDS-DMA copies of the activation rows and the strip's scales,
  // 16 bytes per lane, block i of a region landing at byte 1024 i; lanes
  // past the end are masked off.
  auto stage_to_lds = [&]() {
    using lds_ptr = __attribute__((address_space(3))) void*;
    {
      const uint32_t chunks = static_cast<uint32_t>(mrows) * K / 8;
      for (uint32_t blk = wave; blk * 64 < chunks; blk += WAVES) {
        const uint32_t ch = blk * 64 + lane;
        if (ch < chunks)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(xnorm + blk * 512), 16, ch * 16u,
                                                   0, 0, 0);
      }
    }
    if constexpr (NORM) {
      const __amdgpu_buffer_rsrc_t rn = make_rsrc(norm_wp, K * 2u);
      const uint32_t chunks = K / 8;
      for (uint32_t blk = wave; blk * 64 < chunks; blk += WAVES) {
        const uint32_t ch = blk * 64 + lane;
        if (ch < chunks)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rn, (lds_ptr)(wn_lds + blk * 512), 16, ch * 16u,
                                                   0, 0, 0);
      }
    }
    // Scales: row g of the strip is SW / 8 chunks of 8 columns.
    constexpr uint32_t kRowChunks = SW / 8;
    const uint32_t chunks = total_groups * kRowChunks;
    for (uint32_t blk = wave; blk * 64 < chunks; blk += WAVES) {
      const uint32_t ch = blk * 64 + lane;
      const uint32_t g = ch / kRowChunks, part = ch % kRowChunks;
      const uint32_t scol = strip * SW + 8 * part;
      if (ch < chunks)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_ptr)(s_lds + blk * 512), 16,
            strip < strips_p && scol < N ? L.scol(scol) + g * s_row
                                                                : kOutOfRange,
            0, 0, 0);
    }
    // Rows past M read as zeros from LDS (no masking in the loop).
    for (uint32_t e = threadIdx.x; e < static_cast<uint32_t>(MT - mrows) * K / 8; e += THREADS)
      *reinterpret_cast<h8_t*>(xnorm + mrows * K + 8 * e) = h8_t{};
  };

  // This wave's quant groups [g0, g0 + n).
  const int g0 = static_cast<int>((wave * total_groups) / WAVES);
  const int n = static_cast<int>(((wave + 1) * total_groups) / WAVES) - g0;

  struct Stage {
    h8_t x[TILES][CPG];  // unstaged: loaded with the weights; staged: read from LDS by prep
    u4_t w[CPG];
    h4_t s;
    f4_t corr[TILES];
    int g;
  };
  // Loads of the wave's i-th group; past the range every lane takes the
  // out-of-range offset (zeros, no memory access), so the load sequence is
  // the same on every path and the compiler's wait counts stay exact.
  auto load = [&](Stage& st, int i) {
    const bool in = i < n;
    const int g = in ? g0 + i : g0;
    const uint32_t vw = in ? voff_w : kOutOfRange;
    st.g = g;
    if constexpr (!STAGED) {
      const uint32_t kx = static_cast<uint32_t>(g) * GROUP * 2u;
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int cc = 0; cc < CPG; ++cc)
          st.x[t][cc] = __builtin_bit_cast(
              h8_t, __builtin_amdgcn_raw_buffer_load_b128(rx, in ? voff_x[t] : kOutOfRange,
                                                          kx + cc * KPL * 2, 0));
    }
    const uint32_t kw = static_cast<uint32_t>(g) * (GROUP / 8) * row_bytes;
#pragma unroll
    for (int cc = 0; cc < CPG; ++cc)
      st.w[cc] = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, vw, kw + cc * RPL * row_bytes, kWPolicy));
    if constexpr (!STAGED)
      st.s = __builtin_bit_cast(
          h4_t, __builtin_amdgcn_raw_buffer_load_b64(rs, in ? voff_s : kOutOfRange,
                                                     static_cast<uint32_t>(g) * s_row, kWPolicy));
  };

  f4_t tot[TILES][4];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) tot[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const DecodeConsts dk = decode_consts();
  const h8_t xscale = biased_x_scale();
  const h8_t bcorr = biased_correction();
  // The activations of a group (pre-scaled) and its correction term
  // sum_k x~ * correction, which does not depend on the weights: staged
  // launches compute it ahead of the weight MFMAs, off their dependency
  // chain.
  auto prep = [&](Stage& st) {
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      f4_t corr = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int cc = 0; cc < CPG; ++cc) {
        if constexpr (STAGED)
          st.x[t][cc] = *reinterpret_cast<const h8_t*>(
              &xnorm[(t * RPT + mm) * K + st.g * GROUP + cc * KPL + kx_lane]);
        st.x[t][cc] = st.x[t][cc] * xscale;
        corr = mfma16(st.x[t][cc], bcorr, corr);
      }
      st.corr[t] = corr;
    }
    // The group's scales, read a stage ahead of their use.
    if constexpr (STAGED) st.s = *reinterpret_cast<const h4_t*>(&s_lds[st.g * SW + 4 * c]);
  };
  auto compute = [&](const Stage& st) {
    f4_t acc[TILES][4];
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][j] = st.corr[t];
#pragma unroll
    for (int cc = 0; cc < CPG; ++cc)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h8_t b = decode8_biased(st.w[cc][j], dk);
#pragma unroll
        for (int t = 0; t < TILES; ++t) acc[t][j] = mfma16(st.x[t][cc], b, acc[t][j]);
      }
    const h4_t sc = st.s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sj = static_cast<float>(sc[j]);
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int i = 0; i < LANE_ROWS; ++i)
          tot[t][j][i] = __builtin_fmaf(sj, acc[t][j][i], tot[t][j][i]);
    }
  };

  // The prologue's loads are issued stage by stage, in the order the loop
  // body issues them: with the scheduler free to interleave them, the wait
  // counts at the loop head could not be matched across the back edge and
  // the compiler drained every load there.
  // The LDS-DMA copies go first: the barrier before the first compute then
  // waits for them alone (wait counts are in issue order), not for every
  // weight load in flight.  Issuing the first group's weights ahead of the
  // copies (the barrier then waits for that group, which the first compute
  // needs anyway) measured slower: 4096 x 14336 M = 1 7.17 against 7.00 us,
  // the copies landing ~0.6 us after the barrier is reached.  So did a fifth
  // wave issuing the copies while the four compute waves issue their weights
  // at entry (8.17 us): a CU returns the copies' data behind the weights
  // already queued, 1.3 us after issue.  Workgroup-uniform address bases with
  // 24-bit row products left the prologue's ~0.8 us (mostly the issue of 44
  // 1 KiB requests per CU) unchanged.
  if constexpr (STAGED) {
    stage_to_lds();
    __builtin_amdgcn_sched_barrier(0);
  }
  Stage st[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    load(st[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  // Every wave's LDS-DMA copies have landed (each waits for its own, the
  // barrier for the others').  The RMSNorm prologue then normalises the
  // staged rows in place: its inputs were copied ahead of the weight loads,
  // so its wait does not include them.
  if constexpr (TIMELINE) tl[1] = __builtin_amdgcn_s_memrealtime();
  if constexpr (STAGED) __syncthreads();
  if constexpr (TIMELINE) tl[2] = __builtin_amdgcn_s_memrealtime();
  if constexpr (NORM) norm_rows_in_lds<THREADS, MT>(a, mrows, xnorm, wn_lds);
  if constexpr (ONEPASS) {
    // Every group of the wave is already in flight (n <= DEPTH).
    if constexpr (STAGED) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d)
        if (d < n) prep(st[d]);
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      __builtin_amdgcn_sched_barrier(0);
      if (d < n) {
        if constexpr (!STAGED) prep(st[d]);
        compute(st[d]);
        if constexpr (TIMELINE)
          if (d == 0) tl[3] = __builtin_amdgcn_s_memrealtime();
      }
    }
  } else {
    if constexpr (STAGED) prep(st[0]);
    for (int i0 = 0; i0 < n; i0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        __builtin_amdgcn_sched_barrier(0);
        if (i0 + d < n) {
          if constexpr (STAGED) {
            // the next group's activations and correction, then this group
            if (i0 + d + 1 < n) prep(st[(d + 1) % DEPTH]);
          } else {
            prep(st[d]);
          }
          compute(st[d]);
          if constexpr (TIMELINE)
            if (i0 + d == 0) tl[3] = __builtin_amdgcn_s_memrealtime();
        }
        __builtin_amdgcn_sched_barrier(0);
        load(st[d], i0 + d + DEPTH);
      }
    }
  }
  if constexpr (TIMELINE) tl[4] = __builtin_amdgcn_s_memrealtime();

  // Lane (n = lane % 16, row block lane / 16) holds C rows 4 (lane / 16) + i
  // of each tile; it keeps the entries of its own phase.
  const int nslot = lane & 15;
  const int my_phase = nslot / LPR;
  const int ccol = 4 * (nslot % LPR);
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int i = 0; i < LANE_ROWS; ++i) {
      const int mp = 4 * (lane >> 4) + i;
      const int m = t * RPT + mp % RPT;
      if (mp / RPT == my_phase && m < MT) {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[wave][my_phase][m][ccol + j] = tot[t][j][i];
      }
    }
  __syncthreads();
  if constexpr (TIMELINE) tl[5] = __builtin_amdgcn_s_memrealtime();
  // Sum the WAVES * P partials of an output quad in (wave, phase) order.  The
  // reads go out in batches of up to 16 ahead of their adds (a scheduling
  // barrier keeps the compiler from interleaving each read with its add,
  // which exposed the LDS latency once per partial).
  auto strip_sum = [&](int row, int qq) {
    constexpr int E = WAVES * P;
    constexpr int BATCH = E < 16 ? E : 16;
    static_assert(E % BATCH == 0, "whole batches");
    f4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e0 = 0; e0 < E; e0 += BATCH) {
      f4_t v[BATCH];
#pragma unroll
      for (int b = 0; b < BATCH; ++b)
        v[b] = *reinterpret_cast<const f4_t*>(&red[(e0 + b) / P][(e0 + b) % P][row][4 * qq]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
        sum[0] += v[b][0];
        sum[1] += v[b][1];
        sum[2] += v[b][2];
        sum[3] += v[b][3];
      }
    }
    return sum;
  };
  emit_outputs<MT, THREADS, SW>(a, strip, 0, mrows, strip_sum);
  if constexpr (TIMELINE) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's output stores acknowledged
    tl[6] = __builtin_amdgcn_s_memrealtime();
    const unsigned hw_id = __builtin_amdgcn_s_getreg((31 << 11) | 4);  // HW_REG_HW_ID
    const unsigned xcc = __builtin_amdgcn_s_getreg((15 << 11) | 20);   // HW_REG_XCC_ID
    if (lane == 0) {
      unsigned long long* const out = a.stamps + (static_cast<size_t>(blockIdx.x) * WAVES + wave) * 8;
#pragma unroll
      for (int k = 0; k < 7; ++k) out[k] = tl[k];
      out[7] = (static_cast<unsigned long long>(blockIdx.x) << 40) |
               (static_cast<unsigned long long>(wave) << 36) |
               (static_cast<unsigned long long>(xcc & 0xFu) << 32) | hw_id;
    }
  }
}

// The strip kernel on packed weights: its prologue's fields preloaded.
template <int MT, int GROUP, int SW, int WAVES, int DEPTH, bool NORM, bool ONEPASS, bool STAGED,
          bool TIMELINE = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_strip_kernel(
    const _Float16* Xp, const uint32_t* Wqp, const _Float16* Sp,
    const _Float16* norm_wp, uint32_t Mp, uint32_t Kp, uint32_t Np, uint32_t strips_p,
    uint32_t w_row_p, uint32_t strip_shift_p, GemvArgs a) {
  strip_body<MT, GROUP, SW, WAVES, DEPTH, NORM, ONEPASS, STAGED, TIMELINE>(
      Xp, Wqp, Sp, norm_wp, Mp, Kp, Np, strips_p, w_row_p, strip_shift_p, a);
}

// The strip kernel on strip-major weights: every field from the argument
// block, as its waves fetch it.  Measured on MI355X (graph replay, M = 1,
// same-box A/B against the kernel before preloading): preloaded fields gain
// on packed weights (4096 x 14336 7.40-7.46 -> 7.24-7.28 us, 8192 x 8192
// 9.09-9.10 -> 8.79-8.84, 4096 x 6144 5.43-5.52 -> 5.32-5.42) but cost the
// strip-major 8192 x 8192 plan 8% (7.96-8.02 -> 8.61-8.71; through this entry
// 7.88-7.94), the other strip-major shapes within noise either way.
//
// The operand pointers carry no __restrict__: with it the compiler treated
// the buffer loads as invariant and re-issued the first group's loads inside
// the one-pass compute branch, draining the ring there (strip-major 4096 x
// 4096 4.0 -> 4.35 us).
template <int MT, int GROUP, int SW, int WAVES, int DEPTH, bool NORM, bool ONEPASS, bool STAGED,
          bool TIMELINE = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_strip_kernel_block(GemvArgs a) {
  strip_body<MT, GROUP, SW, WAVES, DEPTH, NORM, ONEPASS, STAGED, TIMELINE>(
      a.X, a.Wq, a.S, a.norm_w, static_cast<uint32_t>(a.M), static_cast<uint32_t>(a.K),
      static_cast<uint32_t>(a.N), static_cast<uint32_t>(a.strips), a.L.w_row, a.L.strip_shift, a);
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
// Batch kernel geometry: weight loads of 2 steps in flight per wave, 3 LDS
// activation slots (96 KiB at GROUP = 128), 4 staging waves.  Measured on
// MI355X, M = 17..32, graph replay, against the same kernel with 1 / 2 / 8
// staging waves (32 / 16 / 4 copies each per slot): 14336 x 4096 M = 32
// 12.3 us against 15.8 / 14.4 / 15.5, 4096 x 4096 8.4 against 9.9 / 9.2 /
// 9.1 -- one wave issuing the copies (an LDS-DMA load each, at most 63 in
// flight) was the bound; 8 staging waves put two on a compute wave's SIMD.
// 3 steps of weights were 1-6% slower than 2, 2 slots 5-10% slower than 3.
// It serves single blocks of 12..32 rows outside the strip kernel's plans
// (kBatchWorkgroups: the grid a plan aims for, one workgroup per CU of an
// MI355X; the plan is host arithmetic, the same on any device).
constexpr int kBatchDepth = 2;
constexpr int kBatchRing = 3;
constexpr int kBatchStagers = 4;
constexpr int kBatchWorkgroups = 256;
constexpr int kBatchMaxSplits = 8;
// 33..64 rows run one 64-row block only when its grid fills the CUs in one
// round (224..256 workgroups).  Measured on MI355X against gemm's 64-row
// tiles, M = 33 / 64: 4096 x 14336 17.1 / 17.6 us against 19.2 / 19.7,
// 14336 x 4096 17.4 / 18.8 against 20.0 / 21.6, 4096 x 4096 11.0 / 11.0
// against 11.9 / 12.4; 192 workgroups (4096 x 6144) 12.9 against 12.3, two
// rounds (4096 x 28672) 29.9 against 26.2.
constexpr int kBatch64MinWorkgroups = 224;
// 16-row blocks run the batch kernel from this many rows: at 9 rows the
// split kernel, whose activation loads scale with the rows, is as fast or
// faster (4096 x 4096 7.0 against 7.7 us, 14336 x 4096 10.4 against 10.5).
constexpr int kBatchMinRows = 12;
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

// The strip kernel's preloaded scalar arguments, then the argument block.
#define NIBBLE_STRIP_ARGS(a)                                                                   \
  (a).X, (a).Wq, (a).S, (a).norm_w, static_cast<uint32_t>((a).M), static_cast<uint32_t>((a).K), \
      static_cast<uint32_t>((a).N), static_cast<uint32_t>((a).strips), (a).L.w_row,            \
      (a).L.strip_shift, (a)

// A strip-kernel launch: the preloaded-argument entry on packed weights,
// the argument-block entry on strip-major weights.
template <int MT, int GROUP, int SW, int WAVES, int DEPTH, bool NORM, bool ONEPASS, bool STAGED,
          bool TIMELINE = false>
void launch_strip_kernel(dim3 grid, int threads, size_t lds, hipStream_t stream, const GemvArgs& a) {
  if (a.L.strip_shift == 31)
    gemv_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, NORM, ONEPASS, STAGED, TIMELINE>
        <<<grid, threads, lds, stream>>>(NIBBLE_STRIP_ARGS(a));
  else
    gemv_strip_kernel_block<MT, GROUP, SW, WAVES, DEPTH, NORM, ONEPASS, STAGED, TIMELINE>
        <<<grid, threads, lds, stream>>>(a);
}

// The strip kernel at one geometry.  The grid is rounded up to a whole
// number of XCD runs (8 workgroups per strip-per-XCD).
template <int MT, int GROUP, int SW, int WAVES, int DEPTH>
hipError_t launch_strip_geometry(const GemvArgs& a, hipStream_t stream) {
  if constexpr (SW == 16 && GROUP != 128) {
    return hipErrorInvalidValue;  // a 16-column wave load spans 128 k
  } else if constexpr (MT > 16) {
    return hipErrorInvalidValue;
  } else {
    // The kernel rebuilds the layout from w_row and the strip shift, and
    // derives the per-XCD strip count from the strip count.
    if (!layout_rebuilds(a, GROUP) || a.strips_per_xcd != (a.strips + 7) / 8)
      return hipErrorInvalidValue;
    const dim3 grid(8 * a.strips_per_xcd);
    // A dispatch asking for more LDS than a workgroup can hold (160 KiB on
    // gfx950) aborts the queue: every launch below is checked against it.
    // Static LDS is the partials buffer, WAVES x phases x MT x SW floats, plus
    // a few words.
    constexpr size_t kLdsMax = 160 * 1024;
    constexpr size_t kStaticLds = sizeof(float) * WAVES * (64 / SW) * MT * SW + 256;
    // One pass when no wave has more groups than the ring holds; activations
    // and scales staged in LDS when the rows fit 64 KiB, or, for 16-row
    // blocks, wherever they fit beside the partials (the RMSNorm prologue
    // always stages, and is only planned when they fit).
    const bool onepass = (a.K / GROUP + WAVES - 1) / WAVES <= DEPTH;
    const size_t xbytes = static_cast<size_t>(MT) * a.K * sizeof(_Float16);
    const size_t nbytes = a.norm_w != nullptr ? static_cast<size_t>(a.K) * sizeof(_Float16) : 0;
    const size_t lds = xbytes + nbytes + static_cast<size_t>(a.K / GROUP) * SW * sizeof(_Float16);
    const bool staged = a.norm_w != nullptr ||
                        (a.stage_x && (xbytes <= 65536 || (MT == 16 && kStaticLds + lds <= kLdsMax)));
    if (kStaticLds + (staged ? lds : 0) > kLdsMax) return hipErrorInvalidValue;
    if constexpr (MT == 1) {
      if (a.stamps != nullptr && a.norm_w == nullptr) {
        if (staged) {
          if (onepass)
            launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, true, true, true>(grid, WAVES * 64, lds, stream, a);
          else
            launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, false, true, true>(grid, WAVES * 64, lds, stream, a);
        } else {
          if (onepass)
            launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, true, false, true>(grid, WAVES * 64, 0, stream, a);
          else
            launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, false, false, true>(grid, WAVES * 64, 0, stream, a);
        }
        return hipGetLastError();
      }
    }
    if (a.norm_w != nullptr) {
      if (onepass)
        launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, true, true, true>(grid, WAVES * 64, lds, stream, a);
      else
        launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, true, false, true>(grid, WAVES * 64, lds, stream, a);
    } else if (staged) {
      if (onepass)
        launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, true, true>(grid, WAVES * 64, lds, stream, a);
      else
        launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, false, true>(grid, WAVES * 64, lds, stream, a);
    } else {
      if (onepass)
        launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, true, false>(grid, WAVES * 64, 0, stream, a);
      else
        launch_strip_kernel<MT, GROUP, SW, WAVES, DEPTH, false, false, false>(grid, WAVES * 64, 0, stream, a);
    }
    return hipGetLastError();
  }
}

// The strip geometries compiled into the library; plan_strip only picks
// these.
template <int MT, int GROUP>
hipError_t launch_strip_mt(const GemvArgs& a, const StreamPlan& p, hipStream_t stream) {
  const int key = p.strip_cols * 10000 + p.waves * 100 + p.depth;
  switch (key) {
    case 16 * 10000 + 8 * 100 + 4: return launch_strip_geometry<MT, GROUP, 16, 8, 4>(a, stream);
    case 32 * 10000 + 8 * 100 + 2: return launch_strip_geometry<MT, GROUP, 32, 8, 2>(a, stream);
    case 32 * 10000 + 16 * 100 + 2: return launch_strip_geometry<MT, GROUP, 32, 16, 2>(a, stream);
    case 64 * 10000 + 4 * 100 + 2: return launch_strip_geometry<MT, GROUP, 64, 4, 2>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int GROUP>
hipError_t launch_strip_group(const GemvArgs& a, const StreamPlan& p, hipStream_t stream) {
  switch (p.mt) {
    case 1: return launch_strip_mt<1, GROUP>(a, p, stream);
    case 2: return launch_strip_mt<2, GROUP>(a, p, stream);
    case 4: return launch_strip_mt<4, GROUP>(a, p, stream);
    case 8: return launch_strip_mt<8, GROUP>(a, p, stream);
    case 16: return launch_strip_mt<16, GROUP>(a, p, stream);
    default: return hipErrorInvalidValue;
  }
}

// The batch kernel: 4 compute waves per strip (SPW strips per workgroup) and
// kBatchStagers staging waves, RING activation slots of MT rows x (4 x GROUP)
// k in dynamic LDS (96 KiB at 32 rows and GROUP = 128).
template <int MT, int GROUP, int SPW = 1>
hipError_t launch_batch_rows(const GemvArgs& a, const StreamPlan& p, hipStream_t stream) {
  // 64-row slots (64 KiB at GROUP = 128) leave room for 2.
  constexpr int kRing = MT == 64 ? 2 : kBatchRing;
  constexpr size_t kSlots = static_cast<size_t>(kRing) * MT * (4 * GROUP / 8) * 16;
  constexpr size_t kTotals = static_cast<size_t>(SPW) * 4 * MT * 16 * 16;
  constexpr size_t kLds = kSlots > kTotals ? kSlots : kTotals;
  static_assert(kLds + 256 <= 160 * 1024, "a workgroup holds at most 160 KiB of LDS");
  const dim3 grid(static_cast<unsigned>(ceil_div(p.strips, SPW)), p.splits, p.mblocks);
  constexpr int kThreads = (4 * SPW + kBatchStagers) * 64;
  if (p.mblocks == 1)
    gemv_batch_kernel<MT, GROUP, kBatchDepth, kRing, kBatchStagers, true, SPW>
        <<<grid, kThreads, kLds, stream>>>(a);
  else
    gemv_batch_kernel<MT, GROUP, kBatchDepth, kRing, kBatchStagers, false, SPW>
        <<<grid, kThreads, kLds, stream>>>(a);
  return hipGetLastError();
}

template <int GROUP>
hipError_t launch_batch_group(const GemvArgs& a, const StreamPlan& p, hipStream_t stream) {
  if (p.waves != 4 || p.depth != kBatchDepth || p.ring != kBatchRing) return hipErrorInvalidValue;
  if (p.pair == 2) {
    // Two strips' totals need the 128-row-group ring (planned at GROUP = 128 only).
    if constexpr (GROUP == 128) {
      if (p.splits != 1 || p.mblocks != 1) return hipErrorInvalidValue;
      if (p.mt == 16) return launch_batch_rows<16, GROUP, 2>(a, p, stream);
      if (p.mt == 32) return launch_batch_rows<32, GROUP, 2>(a, p, stream);
    }
    return hipErrorInvalidValue;
  }
  switch (p.mt) {
    case 16: return launch_batch_rows<16, GROUP>(a, p, stream);
    case 32: return launch_batch_rows<32, GROUP>(a, p, stream);
    case 64: return launch_batch_rows<64, GROUP>(a, p, stream);
    default: return hipErrorInvalidValue;
  }
}

// Split heuristic: whole K in one workgroup per 64-column strip unless a wave
// would have to stream more than kGroupsPerWave groups, in which case K is
// split evenly.  Overrides follow the reference: splits are floor-then-trimmed
// (csrc/gemv_w4a16.cu:398-401).
int plan_split_kernel(int64_t M, int64_t K, int64_t N, int64_t G, bool split_k,
                      int64_t splits_override, int64_t threads_override, StreamPlan* p) {
  if (M < 1 || M > kStreamMaxM || K <= 0 || N <= 0 || (G != 64 && G != 128) || K % G != 0)
    return fail(NIBBLE_ERR_INVALID_ARGUMENT, "no streaming plan for M=%lld K=%lld N=%lld G=%lld",
                (long long)M, (long long)K, (long long)N, (long long)G);
  *p = StreamPlan();
  p->kernel = kSplitKernel;
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

}  // namespace

// The strip kernel serves M <= 8 up to K = 8192.  Its geometry depends on
// (M, K, N) only -- never on the epilogue or the RMSNorm prologue -- so the
// fused and unfused launches of one shape sum every output in the same order
// and give the same bits.  Measured on MI355X (graph replay, weights streamed
// from HBM, M = 1, against the split kernel's plan):
//  * N >= 12288: 64-column strips, 4 waves -- 4096 x 14336 7.6 us (7.8;
//    32-column strips 9.0), 4096 x 28672 13.3 us (14.0);
//  * narrower: 32-column strips, 8 waves (16 at K = 8192) -- 4096 x 1024
//    4.4 us (5.5), 4096 x 4096 4.7 (5.8), 4096 x 6144 5.5 (6.7), 8192 x 8192
//    9.2 (9.4); 16-column strips were no faster and 64-column ones slower;
//  * two groups of loads in flight per wave (deeper rings measured slower);
//  * longer K keeps the split kernel: 14336 x 4096 9.5 us there, 10.0 us at
//    the best strip geometry.
constexpr int64_t kStripMaxK = 8192;
constexpr int64_t kStripWideN = 12288;
// 9 <= M <= 16 (batches through gemm): 16-row blocks on 64-column strips
// with the activations staged in LDS (128 KiB at K = 4096, beside 16 KiB of
// partials).  Measured on MI355X against the split kernel, graph replay:
// 4096 x 14336 M = 9 / 12 / 16 8.66 / 8.64 / 8.74 us (8.73 / 9.28 / 9.67),
// 4096 x 28672 M = 12 / 16 16.1 / 16.4 (16.3 / 17.6).  Narrower N keeps the
// split kernel (4096 x 4096, 64 strips: 7.7-7.8 against 6.9-8.1).
constexpr int64_t kStrip16MaxK = 4096;

bool plan_strip(int64_t M, int64_t K, int64_t N, int64_t G, StreamFusion fusion, StreamPlan* p) {
  (void)fusion;
  if (M < 1 || M > 16 || K <= 0 || K > kStripMaxK || N <= 0 || (G != 64 && G != 128) ||
      K % G != 0)
    return false;
  if (M > 8 && (K > kStrip16MaxK || N < kStripWideN)) return false;
  StreamPlan q;
  q.kernel = kStripKernel;
  q.mt = mt_for(M);
  q.mblocks = 1;
  q.splits = 1;
  q.groups_per_split = static_cast<int>(K / G);
  q.depth = 2;
  if (N >= kStripWideN) {
    q.strip_cols = 64;
    q.waves = 4;
  } else {
    q.strip_cols = 32;
    q.waves = K <= 4096 ? 8 : 16;
  }
  q.strips = static_cast<int>(ceil_div(N, q.strip_cols));
  q.counter_bytes = 0;
  q.workspace_bytes = 0;
  *p = q;
  return true;
}

namespace {
// K splits of a batch-kernel plan: the split kernel's count, raised where the
// strips alone leave CUs idle (at most kBatchMaxSplits, at least 4 groups a
// split).
int batch_splits(int strips, int groups, int heuristic) {
  const int fill = std::min({kBatchMaxSplits, kBatchWorkgroups / std::max(1, strips), groups / 4});
  return std::max(heuristic, fill);
}
}  // namespace

int batch_block_rows(int64_t M, int64_t K, int64_t N, int64_t G) {
  if (M < kBatchMinRows || M > 64 || K <= 0 || N <= 0 || (G != 64 && G != 128) || K % G != 0)
    return 0;
  if (M <= 16) {
    StreamPlan strip;
    return plan_strip(M, K, N, G, StreamFusion(), &strip) ? 0 : 16;
  }
  if (M <= 32) return 32;
  // 33..64 rows: one 64-row block where its grid is one full round of the
  // CUs; otherwise the tiles (or 32-row passes) of gemm's own plan.
  StreamPlan sp;
  if (plan_split_kernel(M, K, N, G, true, 0, 0, &sp) != NIBBLE_OK) return 0;
  const int64_t grid = static_cast<int64_t>(sp.strips) *
                       batch_splits(sp.strips, static_cast<int>(K / G), sp.splits);
  return grid >= kBatch64MinWorkgroups && grid <= kBatchWorkgroups ? 64 : 0;
}

int plan_stream(int64_t M, int64_t K, int64_t N, int64_t G, bool split_k, int64_t splits_override,
                int64_t threads_override, StreamPlan* p, StreamFusion fusion) {
  if (split_k && splits_override == 0 && threads_override == 0 &&
      plan_strip(M, K, N, G, fusion, p))
    return NIBBLE_OK;
  const int rc = plan_split_kernel(M, K, N, G, split_k, splits_override, threads_override, p);
  if (rc != NIBBLE_OK || !split_k || splits_override != 0 || threads_override != 0 || p->waves != 4)
    return rc;
  const int rows = batch_block_rows(M, K, N, G);
  if (rows == 0) return rc;
  p->mt = rows;
  p->mblocks = 1;
  // 12..32 rows (those the strip kernel does not take) run the batch kernel
  // in one block of 16 or 32 rows (the split kernel's bits for the same
  // plan), with K split further where the strips alone leave CUs idle (at
  // most kBatchMaxSplits, at least 4 groups a split).  Measured on MI355X,
  // graph replay, against the split kernel's own plan: M = 17 / 32 4096 x
  // 14336 10.8 / 11.1 us against 11.0 / 13.5; 14336 x 4096 11.9 / 12.3
  // against 14.0 / 18.4; 4096 x 4096 (4 splits) 8.2 / 8.4 against 9.3 /
  // 12.4; 4096 x 1024 (8 splits) 6.9 / 7.1 against 9.0 / 11.9; M = 12 / 16
  // 14336 x 4096 10.5 / 10.6 against 11.1 / 12.2, 8192 x 8192 10.7 / 10.8
  // against 11.8 / 13.1.
  const int groups = static_cast<int>(K / G);
  const int fill = batch_splits(p->strips, groups, p->splits);
  if (fill > p->splits) {
    p->groups_per_split = static_cast<int>(ceil_div(groups, fill));
    p->splits = static_cast<int>(ceil_div(groups, p->groups_per_split));
  }
  p->counter_bytes = p->splits > 1 ? align_up(static_cast<size_t>(p->strips) * 4, 256) : 0;
  p->workspace_bytes =
      p->splits > 1 ? p->counter_bytes + static_cast<size_t>(p->splits) * M * N * 4 : 0;
  p->kernel = kBatchKernel;
  p->depth = kBatchDepth;
  p->ring = kBatchRing;
  // Where pairs of adjacent strips still make one round of the CUs without a
  // K split, a workgroup takes a pair and copies the activation window once
  // for both (same arithmetic per output, so the same bits).  Measured on
  // MI355X, graph replay, 4096 x 28672: M = 17 / 32 18.9 / 20.4 -> 16.7 /
  // 17.5 us.  Where the pairs would need a K split to fill the CUs, the split
  // epilogue costs more than the halved copies save (4096 x 14336 M = 32
  // 11.1 -> 14.0 us with 2 splits).
  const int64_t pairs = ceil_div(p->strips, 2);
  if (p->splits == 1 && rows != 64 && G == 128 && pairs >= kBatch64MinWorkgroups &&
      pairs <= kBatchWorkgroups)
    p->pair = 2;
  return rc;
}

// Strip width for strip-major weights (the layout fixes it, so it is chosen
// once, when the weight is packed).  Measured on MI355X, M = 1, graph replay,
// strip-major against the packed layout's own plan: 14336 x 4096 7.6 us with
// 16-column strips (split kernel 9.5); 4096 x 1024 3.7 (4.3); 4096 x 4096
// 4.1 with 16-column strips reading the activations per lane (4.7; 4.5 with
// 32-column strips); 4096 x 6144 4.8 (5.5); 4096 x 14336 7.2 (7.3);
// 4096 x 28672 12.1 (13.0); 8192 x 8192 8.0 (9.2).  Narrow strips of the
// packed layout read 64 or 128 contiguous bytes per packed row, 4 N bytes
// apart, which HBM serves at a fraction of its streaming rate; a strip-major
// strip is one contiguous run.
int64_t strip_major_cols(int64_t K, int64_t N, int64_t G) {
  if (K <= 0 || N <= 0 || (G != 64 && G != 128) || K % G != 0) return 0;
  if (N >= kStripWideN && N % 64 == 0) return 64;
  const bool narrow = G == 128 && N % 16 == 0;  // a 16-column wave load spans 128 k
  // Too few 32-column strips to fill the chip, or (K <= 4096, N <= 4096)
  // 16-column strips measured faster.
  if (narrow && (N <= 2048 || K >= 12288 || (K <= 4096 && N <= 4096))) return 16;
  if (N % 32 == 0) return 32;
  return narrow ? 16 : 0;
}

bool plan_strip_major(int64_t M, int64_t K, int64_t N, int64_t G, int64_t SW, StreamPlan* p) {
  if (M < 1 || M > 8 || K <= 0 || N <= 0 || (G != 64 && G != 128) || K % G != 0) return false;
  if ((SW != 16 && SW != 32 && SW != 64) || N % SW != 0 || (SW == 16 && G != 128)) return false;
  StreamPlan q;
  q.kernel = kStripKernel;
  q.mt = mt_for(M);
  q.mblocks = 1;
  q.splits = 1;
  q.groups_per_split = static_cast<int>(K / G);
  q.strip_cols = static_cast<int>(SW);
  // 16-column strips keep 4 groups of loads in flight per wave (1 KiB each);
  // wider strips hold enough bytes with 2.
  q.waves = SW == 64 ? 4 : 8;
  q.depth = SW == 16 ? 4 : 2;
  // 16-column strips over a short K read their activations per lane with
  // the weights: at 4096 x 4096 4.1 us against 4.4 staged (equal at
  // 4096 x 1024; staging wins from K = 14336: 7.6 against 8.3).
  q.stage_x = !(SW == 16 && K <= 4096);
  q.strips = static_cast<int>(N / SW);
  q.counter_bytes = 0;
  q.workspace_bytes = 0;
  *p = q;
  return true;
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
                  const void* bias, const void* norm_w, float norm_eps, int64_t strip_cols) {
  if (p.workspace_bytes > 0) {
    if (workspace == nullptr || workspace_bytes < p.workspace_bytes)
      return fail(NIBBLE_ERR_WORKSPACE, "%s needs %zu bytes of workspace, got %zu", who,
                  p.workspace_bytes, workspace == nullptr ? size_t(0) : workspace_bytes);
    if (!aligned(workspace, 256))
      return fail(NIBBLE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }
  void* counters = p.workspace_bytes > 0 ? workspace : nullptr;
  void* partials =
      p.workspace_bytes > 0 ? static_cast<char*>(workspace) + p.counter_bytes : nullptr;
  return launch_stream_split(X, Wq, S, Y, M, K, N, G, p, counters, partials, stream, who,
                             epilogue, bias, norm_w, norm_eps, strip_cols);
}

// nibble_gemv_timeline's buffer for this host thread's launches (off: null).
thread_local unsigned long long* t_timeline = nullptr;
thread_local int64_t t_timeline_bytes = 0;

int launch_stream_split(const void* X, const void* Wq, const void* S, void* Y, int64_t M,
                        int64_t K, int64_t N, int64_t G, const StreamPlan& p, void* counters,
                        void* partials, hipStream_t stream, const char* who, int epilogue,
                        const void* bias, const void* norm_w, float norm_eps,
                        int64_t strip_cols) {
  GemvArgs a;
  a.L = layout_for(K, N, G, strip_cols);
  a.X = static_cast<const _Float16*>(X);
  a.Wq = static_cast<const uint32_t*>(Wq);
  a.S = static_cast<const _Float16*>(S);
  a.Y = static_cast<_Float16*>(Y);
  a.counters = p.splits > 1 ? static_cast<uint32_t*>(counters) : nullptr;
  a.partial = p.splits > 1 ? static_cast<float*>(partials) : nullptr;
  a.M = static_cast<int>(M);
  a.K = static_cast<int>(K);
  a.N = static_cast<int>(N);
  a.groups_per_split = p.groups_per_split;
  a.splits = p.splits;
  a.epilogue = epilogue;
  a.bias = static_cast<const _Float16*>(bias);
  a.norm_w = static_cast<const _Float16*>(norm_w);
  a.norm_eps = norm_eps;
  hipError_t e;
  if (p.kernel == kStripKernel) {
    a.strips = p.strips;
    a.strips_per_xcd = static_cast<int>(ceil_div(p.strips, 8));
    a.stage_x = p.stage_x ? 1 : 0;
    if (t_timeline != nullptr && M == 1 && norm_w == nullptr) {
      const int64_t need = int64_t(8) * a.strips_per_xcd * p.waves * 8 * 8;
      NIBBLE_CHECK(need <= t_timeline_bytes,
                   "%s: the timeline of this launch needs %lld bytes, the buffer holds %lld", who,
                   (long long)need, (long long)t_timeline_bytes);
      a.stamps = t_timeline;
    }
    e = G == 128 ? launch_strip_group<128>(a, p, stream) : launch_strip_group<64>(a, p, stream);
  } else if (p.kernel == kBatchKernel) {
    e = G == 128 ? launch_batch_group<128>(a, p, stream) : launch_batch_group<64>(a, p, stream);
  } else {
    e = G == 128 ? launch_group<128>(a, p, stream) : launch_group<64>(a, p, stream);
  }
  if (e != hipSuccess) return hip_fail(e, who);
  return NIBBLE_OK;
}

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

extern "C" int nibble_gemv_timeline(void* stamps, int64_t bytes) {
  NIBBLE_CHECK(stamps == nullptr || bytes > 0, "a timeline buffer needs a positive size");
  NIBBLE_CHECK(stamps == nullptr || reinterpret_cast<uintptr_t>(stamps) % 8 == 0,
               "the timeline buffer needs 8-byte alignment");
  t_timeline = static_cast<unsigned long long*>(stamps);
  t_timeline_bytes = stamps != nullptr ? bytes : 0;
  return NIBBLE_OK;
}

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
  NIBBLE_CHECK(epilogue != kEpilogueSwiglu || N % (2 * kSwigluBlock) == 0,
               "swiglu needs N (gate|up interleaved in 16-column blocks) to be a multiple of 32");
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

// The workspace a fused launch may need does not depend on its epilogue: the
// query answers for the split kernel, the larger of the two plans (the strip
// kernel needs none), so one buffer serves every epilogue and prologue.
namespace {
// The fused entry's workspace covers both streaming plans of these operands
// (the split kernel's, and the heuristic plan the launch takes), so one
// buffer serves every epilogue and prologue: a counter region as large as
// either plan's, then room for either plan's partials.  The launch lays the
// workspace out that way too (fused_layout), so a caller that keys buffers
// by the reported counter region never finds partials inside it.
bool fused_plan_bytes(int64_t M, int64_t K, int64_t N, int64_t G, size_t* ws, size_t* counters) {
  StreamPlan a, b;
  if (M < 1 || M > kStreamMaxM || K <= 0 || N <= 0 || (G != 64 && G != 128) || K % G != 0 ||
      plan_split_kernel(M, K, N, G, true, 0, 0, &a) != NIBBLE_OK ||
      plan_stream(M, K, N, G, true, 0, 0, &b) != NIBBLE_OK)
    return false;
  *counters = std::max(a.counter_bytes, b.counter_bytes);
  const size_t partials = std::max(a.workspace_bytes - a.counter_bytes,
                                   b.workspace_bytes - b.counter_bytes);
  *ws = partials > 0 ? *counters + partials : 0;
  return true;
}

// A split plan of the fused entry takes the reported layout: its counters
// at the start of a region of the reported size, its partials after it.
void fused_layout(int64_t M, int64_t K, int64_t N, int64_t G, StreamPlan* p) {
  size_t ws = 0, counters = 0;
  if (p->workspace_bytes == 0 || !fused_plan_bytes(M, K, N, G, &ws, &counters)) return;
  p->workspace_bytes = counters + (p->workspace_bytes - p->counter_bytes);
  p->counter_bytes = counters;
}
}  // namespace

extern "C" size_t nibble_matmul_fused_workspace_bytes(int64_t M, int64_t K, int64_t N,
                                                      int64_t group_size, void* stream) {
  (void)stream;
  size_t ws = 0, counters = 0;
  return fused_plan_bytes(M, K, N, group_size, &ws, &counters) ? ws : 0;
}

extern "C" size_t nibble_matmul_fused_counter_bytes(int64_t M, int64_t K, int64_t N,
                                                    int64_t group_size, void* stream) {
  (void)stream;
  size_t ws = 0, counters = 0;
  return fused_plan_bytes(M, K, N, group_size, &ws, &counters) ? counters : 0;
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
  StreamFusion fusion;
  fusion.epilogue = static_cast<int>(epilogue);
  fusion.norm = norm_weight != nullptr;
  StreamPlan p;
  rc = plan_stream(M, K, N, group_size, true, 0, 0, &p, fusion);
  if (rc != NIBBLE_OK) return rc;
  fused_layout(M, K, N, group_size, &p);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  rc = launch_stream(X, Wq, S, Y, M, K, N, group_size, p, workspace, workspace_bytes, stream,
                     "fused matmul kernel launch", static_cast<int>(epilogue), bias, norm_weight,
                     norm_eps);
  return rc == NIBBLE_OK ? ok() : rc;
}

// ---------------------------------------------------------------------------
// nibble_gemv_w4a16 without a caller workspace.  No counterpart in the
// reference; for callers that cannot allocate (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).  The split-K counters
// and partials live in `scratch`, a file-scope device array: every GPU the
// library runs on holds one copy until the process ends, and every call on a
// GPU shares it, so calls that overlap on one GPU (concurrent streams or
// threads) race.  The first kScratchCounterBytes are split counters: zeroed
// by a fill kernel when a device first uses the array, and returned to zero
// by every call; the fp32 partials follow them.  Requests whose plan needs
// more are refused before anything is launched.

namespace {
constexpr size_t kScratchBytes = size_t(4) << 20;          // the whole array
constexpr size_t kScratchCounterBytes = size_t(64) << 10;  // counter region at its start
constexpr int kScratchDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mutex;
void* g_scratch_addr[kScratchDevices];  // this device's `scratch` (null until set up)

__global__ void zero_words_kernel(uint32_t* __restrict__ p, uint32_t n) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The device address of `scratch` on `device` (which must be current), set
// up on the device's first use: the address comes from the runtime (in host
// code the array's name only stands for the symbol), and the counter region
// is cleared by a kernel on `stream` that completes before the address is
// published, so every later call on any stream of the device finds it zero.
// That first use cannot be captured into a graph (the clearing would exist
// only inside the graph): it is refused while `stream` is capturing.
int scratch_on(int device, hipStream_t stream, void** addr) {
  if (device < 0 || device >= kScratchDevices)
    return fail(NIBBLE_ERR_UNSUPPORTED, "no-alloc scratch: device %d out of range", device);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_addr[device] == nullptr) {
    hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
    NIBBLE_HIP(hipStreamIsCapturing(stream, &capturing));
    if (capturing != hipStreamCaptureStatusNone)
      return fail(NIBBLE_ERR_UNSUPPORTED,
                  "nibble_gemv_w4a16_noalloc: the first split-K call on device %d sets up the "
                  "static scratch and cannot run under graph capture; make one such call "
                  "outside the capture first",
                  device);
    void* p = nullptr;
    NIBBLE_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    const uint32_t words = static_cast<uint32_t>(kScratchCounterBytes / 4);
    zero_words_kernel<<<(words + 255) / 256, 256, 0, stream>>>(static_cast<uint32_t*>(p), words);
    NIBBLE_HIP(hipGetLastError());
    NIBBLE_HIP(hipStreamSynchronize(stream));
    g_scratch_addr[device] = p;
  }
  *addr = g_scratch_addr[device];
  return NIBBLE_OK;
}
}  // namespace

extern "C" int nibble_gemv_w4a16_noalloc(const void* X, int64_t x_rows, int64_t x_cols,
                                         const void* Wq, int64_t wq_rows, int64_t wq_cols,
                                         const void* S, int64_t s_rows, int64_t s_cols,
                                         int64_t group_size, int64_t version,
                                         int64_t splits_override, int64_t threads_override,
                                         void* Y, void* stream_) {
  int rc = validate_gemv(X, x_rows, x_cols, Wq, wq_rows, wq_cols, S, s_rows, s_cols, group_size,
                         version, splits_override, threads_override, Y);
  if (rc != NIBBLE_OK) return rc;
  const int64_t M = x_rows, K = x_cols, N = wq_cols;
  StreamPlan p;
  const bool needs_workspace =
      gemv_plannable(M, K, N, group_size, version) &&
      gemv_plan(M, K, N, group_size, version, splits_override, threads_override, &p) ==
          NIBBLE_OK &&
      p.workspace_bytes > 0;
  // Every other request (no split, or one the launcher rejects) is exactly
  // nibble_gemv_w4a16 without a workspace.
  if (!needs_workspace)
    return nibble_gemv_w4a16(X, x_rows, x_cols, Wq, wq_rows, wq_cols, S, s_rows, s_cols,
                             group_size, version, splits_override, threads_override, Y, nullptr,
                             0, stream_);
  const size_t partial_bytes = p.workspace_bytes - p.counter_bytes;
  if (p.counter_bytes > kScratchCounterBytes ||
      partial_bytes > kScratchBytes - kScratchCounterBytes)
    return fail(NIBBLE_ERR_UNSUPPORTED,
                "nibble_gemv_w4a16_noalloc: M=%lld K=%lld N=%lld splits into %d and needs %zu "
                "bytes of split counters and %zu of partials; its static scratch holds %zu and "
                "%zu (use nibble_gemv_w4a16 with a workspace)",
                (long long)M, (long long)K, (long long)N, p.splits, p.counter_bytes,
                partial_bytes, kScratchCounterBytes, kScratchBytes - kScratchCounterBytes);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  void* base = nullptr;
  rc = scratch_on(dev, stream, &base);
  if (rc != NIBBLE_OK) return rc;
  rc = launch_stream_split(X, Wq, S, Y, M, K, N, group_size, p, base,
                           static_cast<char*>(base) + kScratchCounterBytes, stream,
                           "gemv (no-alloc) kernel launch");
  return rc == NIBBLE_OK ? ok() : rc;
}

// ---------------------------------------------------------------------------
// Strip-major weights for the decode GEMV.  No counterpart in the reference,
// which has only the packed [K / 8, N] layout (python/nibblegemm/quant.py:
// 28-50).  The layout splits the N columns into strips of `strip_cols` and
// stores each strip's packed rows (and group scales) contiguously, so a
// workgroup of the strip kernel streams one contiguous run instead of short
// pieces of every packed row.

namespace {
// One 16-byte chunk per thread iteration: packed words (4 columns) of the
// source row-major [rows, n] array go to strip n / sw, row r, column n % sw;
// scale chunks hold 8 columns.
__global__ __launch_bounds__(256) void pack_strip_major_kernel(const u4_t* __restrict__ wq,
                                                               const u4_t* __restrict__ s,
                                                               u4_t* __restrict__ wt,
                                                               u4_t* __restrict__ st,
                                                               uint32_t rows, uint32_t srows,
                                                               uint32_t n, uint32_t sw) {
  const uint32_t wq_row = n / 4, s_row = n / 8;
  const uint32_t wchunks = rows * wq_row, total = wchunks + srows * s_row;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    if (i < wchunks) {
      const uint32_t r = i / wq_row, col = (i % wq_row) * 4u;
      wt[((col / sw) * rows + r) * (sw / 4u) + (col % sw) / 4u] = wq[i];
    } else {
      const uint32_t e = i - wchunks;
      const uint32_t g = e / s_row, col = (e % s_row) * 8u;
      st[((col / sw) * srows + g) * (sw / 8u) + (col % sw) / 8u] = s[e];
    }
  }
}

bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
  const char *pa = static_cast<const char*>(a), *pb = static_cast<const char*>(b);
  return pa < pb + bn && pb < pa + an;
}

int check_strip_cols(int64_t N, int64_t G, int64_t SW) {
  NIBBLE_CHECK(SW == 16 || SW == 32 || SW == 64, "strip_cols must be 16, 32 or 64, got %lld",
               (long long)SW);
  NIBBLE_CHECK(N % SW == 0, "N=%lld is not a multiple of strip_cols=%lld", (long long)N,
               (long long)SW);
  NIBBLE_CHECK(SW != 16 || G == 128, "16-column strips need group_size 128");
  return NIBBLE_OK;
}
}  // namespace

extern "C" int64_t nibble_strip_major_cols(int64_t K, int64_t N, int64_t group_size) {
  return strip_major_cols(K, N, group_size);
}

extern "C" int nibble_pack_strip_major(const void* Wq, int64_t wq_rows, int64_t wq_cols,
                                       const void* S, int64_t s_rows, int64_t s_cols,
                                       int64_t group_size, int64_t strip_cols, void* Wt,
                                       void* St, void* stream_) {
  NIBBLE_CHECK(wq_rows > 0 && wq_cols > 0 && s_rows > 0 && s_cols > 0,
               "bad dimension (K and N must be positive)");
  const int64_t K = wq_rows * 8, N = wq_cols;
  NIBBLE_CHECK(group_size == 64 || group_size == 128, "group_size must be 64 or 128");
  NIBBLE_CHECK(s_rows * group_size == K, "scale rows disagree with K/group_size");
  NIBBLE_CHECK(s_cols == N, "scale columns disagree with N");
  int rc = check_strip_cols(N, group_size, strip_cols);
  if (rc != NIBBLE_OK) return rc;
  NIBBLE_CHECK(Wq != nullptr && S != nullptr && Wt != nullptr && St != nullptr, "null pointer");
  NIBBLE_CHECK(aligned(Wq, 16) && aligned(S, 16) && aligned(Wt, 16) && aligned(St, 16),
               "weights and scales must be 16-byte aligned");
  const size_t wbytes = static_cast<size_t>(K / 8) * N * 4;
  const size_t sbytes = static_cast<size_t>(s_rows) * N * 2;
  NIBBLE_CHECK(wbytes < (size_t(1) << 31) && sbytes < (size_t(1) << 31),
               "weights beyond 32-bit offsets");
  NIBBLE_CHECK(!overlaps(Wt, wbytes, Wq, wbytes) && !overlaps(Wt, wbytes, S, sbytes) &&
                   !overlaps(St, sbytes, Wq, wbytes) && !overlaps(St, sbytes, S, sbytes) &&
                   !overlaps(Wt, wbytes, St, sbytes),
               "the strip-major outputs must not overlap the inputs or each other");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  const int64_t chunks = (K / 8) * (N / 4) + s_rows * (N / 8);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(chunks, 256), 8192));
  pack_strip_major_kernel<<<blocks, 256, 0, stream>>>(
      static_cast<const u4_t*>(Wq), static_cast<const u4_t*>(S), static_cast<u4_t*>(Wt),
      static_cast<u4_t*>(St), static_cast<uint32_t>(K / 8), static_cast<uint32_t>(s_rows),
      static_cast<uint32_t>(N), static_cast<uint32_t>(strip_cols));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "strip-major pack kernel launch");
  return ok();
}

extern "C" int nibble_gemv_w4a16_strip_major(const void* X, int64_t x_rows, int64_t x_cols,
                                             const void* Wt, const void* St, int64_t K, int64_t N,
                                             int64_t group_size, int64_t strip_cols,
                                             int64_t epilogue, const void* bias,
                                             const void* norm_weight, float norm_eps, void* Y,
                                             void* stream_) {
  NIBBLE_CHECK(x_rows >= 0 && K > 0 && N > 0, "bad dimension (K and N must be positive)");
  NIBBLE_CHECK(x_cols == K, "activation columns (%lld) disagree with K=%lld", (long long)x_cols,
               (long long)K);
  const int64_t M = x_rows;
  NIBBLE_CHECK(M <= 8, "strip-major gemv supports M <= 8, got %lld", (long long)M);
  NIBBLE_CHECK(group_size == 64 || group_size == 128, "group_size must be 64 or 128");
  NIBBLE_CHECK(K % group_size == 0, "K=%lld is not a multiple of group_size=%lld", (long long)K,
               (long long)group_size);
  int rc = check_strip_cols(N, group_size, strip_cols);
  if (rc != NIBBLE_OK) return rc;
  NIBBLE_CHECK(epilogue == kEpilogueNone || epilogue == kEpilogueBias ||
                   epilogue == kEpilogueSwiglu,
               "epilogue must be 0 (none), 1 (bias) or 2 (swiglu), got %lld", (long long)epilogue);
  NIBBLE_CHECK(epilogue != kEpilogueSwiglu || strip_cols >= 2 * kSwigluBlock,
               "swiglu needs strips of at least 32 columns (gate|up 16-column blocks)");
  NIBBLE_CHECK(epilogue != kEpilogueBias || M == 0 || bias != nullptr, "null bias");
  NIBBLE_CHECK(epilogue != kEpilogueBias || aligned(bias, 2), "misaligned bias");
  if (norm_weight != nullptr) {
    NIBBLE_CHECK(K <= kNormMaxK, "the fused RMSNorm supports K <= %d, got %lld", kNormMaxK,
                 (long long)K);
    NIBBLE_CHECK(M == 0 || mt_for(M) * K * 2 <= 65536,
                 "the fused RMSNorm needs %lld rows x K=%lld fp16 of LDS, above 64 KiB",
                 (long long)mt_for(M), (long long)K);
    NIBBLE_CHECK(aligned(norm_weight, 16), "norm weight must be 16-byte aligned");
    NIBBLE_CHECK(std::isfinite(norm_eps) && norm_eps >= 0.0f, "norm eps must be finite and >= 0");
  }
  if (M == 0) return ok();
  NIBBLE_CHECK(X != nullptr && Wt != nullptr && St != nullptr && Y != nullptr, "null pointer");
  NIBBLE_CHECK(stream_supported(X, Wt, St, Y, M, K, N, group_size),
               "operands must be aligned (X, Wt 16-byte; St, Y 8-byte) and within 32-bit offsets");
  StreamPlan p;
  if (!plan_strip_major(M, K, N, group_size, strip_cols, &p))
    return fail(NIBBLE_ERR_UNSUPPORTED, "no strip-major plan for M=%lld K=%lld N=%lld",
                (long long)M, (long long)K, (long long)N);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  rc = launch_stream_split(X, Wt, St, Y, M, K, N, group_size, p, nullptr, nullptr, stream,
                           "strip-major gemv kernel launch", static_cast<int>(epilogue), bias,
                           norm_weight, norm_eps, strip_cols);
  return rc == NIBBLE_OK ? ok() : rc;
}
