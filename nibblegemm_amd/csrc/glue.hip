// Decode-step glue of a Llama-shaped layer at batch 1, around the W4A16
// projections: RMSNorm and grouped-query attention over a KV cache.
//
// In the reference these are PyTorch / transformers operations of the model
// that bench/bench_model.py decodes token by token with its Linear layers
// swapped for QuantLinear (decode_tokens_per_s, bench/bench_model.py:177-188;
// the swap, :131-154).  Here they are kernels, so that a whole decode step --
// norms, projections, attention, residual adds -- is captured in one HIP
// graph.  The residual adds need no kernel of their own: at M = 1 the residual
// is a bias vector of the o and down projections (the fused bias epilogue of
// the matmul).
//
// Both kernels are memory-latency work of a few hundred KB; they are written
// for short, dependency-free loads (16-byte rows, no LDS staging of the
// cache) and deterministic reductions (fixed orders, no float atomics).
#include <cmath>

#include "nibble_common.h"
#include "nibble_decode.h"
#include "nibble_reduce.h"

namespace nibble {

namespace {

constexpr int kHeadDim = 128;
constexpr int kRopeHalf = kHeadDim / 2;
constexpr int kChunk = 128;  // cached tokens per attention workgroup
constexpr int kGlueThreads = 256;
constexpr int kRmsMaxCols = kRmsThreads * 8 * 8;
constexpr int kAttnMaxSeq = 1 << 16;
constexpr int kAttnMaxChunks = kAttnMaxSeq / kChunk;

// y = fp16(x * r * w) with r = 1 / sqrt(mean(x^2) + eps), in fp32 (the
// transformers LlamaRMSNorm computes the same in fp32 and rounds x * r to
// fp16 before the weight; this rounds once).  One workgroup per row; each
// thread holds CH 16-byte chunks of the row.  The sum of squares is reduced
// per wave (DPP rows, then rows in order) and across waves in wave order:
// deterministic.
template <int CH>
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_kernel(const _Float16* __restrict__ X,
                                                              const _Float16* __restrict__ W,
                                                              _Float16* __restrict__ Y, int cols,
                                                              float eps) {
  __shared__ float part[kRmsThreads / 64];
  const int tid = threadIdx.x;
  const size_t base = static_cast<size_t>(blockIdx.x) * cols;
  h8_t v[CH], w[CH];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * kRmsThreads + tid) * 8;
    v[c] = col < cols ? *reinterpret_cast<const h8_t*>(X + base + col) : h8_t{};
    w[c] = col < cols ? *reinterpret_cast<const h8_t*>(W + col) : h8_t{};  // before the reduction
    ss = sumsq_chunk(v[c], ss);
  }
  const float r = rms_scale(block256_sum(ss, part), cols, eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * kRmsThreads + tid) * 8;
    if (col < cols) *reinterpret_cast<h8_t*>(Y + base + col) = rms_apply(v[c], w[c], r);
  }
}

struct AttnArgs {
  const _Float16* qkv;     // [n_heads * 128 | n_kv * 128 | n_kv * 128]: q, k, v of this token
  _Float16* k_cache;       // [n_kv][max_seq][128]
  _Float16* v_cache;       // [n_kv][max_seq][128]
  const float* rope_cos;   // [max_seq][64], or null: no rotary embedding
  const float* rope_sin;   // [max_seq][64]
  _Float16* out;           // [n_heads * 128]
  float* partial;          // [n_kv][chunks][QPK][2 + 128] when chunks > 1
  uint32_t* counters;      // [n_kv], zero on entry and on exit
  int n_kv, max_seq, pos, chunks;
};

// Element d of the rotary embedding of a 128-vector x at position pos, in the
// rotate-half pairing of transformers' apply_rotary_pos_emb (d with d +- 64),
// from xd = x[d], its partner xp = x[d ^ 64] and the position's cos / sin of
// d mod 64:
//   d <  64: x[d] cos - x[d + 64] sin;   d >= 64: x[d] cos + x[d - 64] sin.
__device__ __forceinline__ float rotate_half(_Float16 xd, _Float16 xp, float c, float s, int d) {
  const float v = static_cast<float>(xd);
  return d < kRopeHalf ? v * c - static_cast<float>(xp) * s : v * c + static_cast<float>(xp) * s;
}

// Grouped-query attention of one decode token: QPK query heads share each
// kv head.  Workgroup (h, c) takes kv head h, its QPK query heads and cached
// tokens [128 c, min(128 c + 128, pos + 1)).  Token pos is the current one:
// its k (rotated, rounded to fp16 as the cache holds it) and v come from qkv
// and are written into the caches by the workgroup of the last chunk.
//
// 16 groups of 16 lanes each take every 16th token of the chunk; lane j of a
// group holds dims 8j..8j+7 of the token's rows (one 16-byte load each).  All
// of a lane's k and v rows are loaded at entry, before anything else: they
// depend on nothing, so the chunk costs one memory round trip instead of one
// per token.
//   1. scores: per token, QPK dot products summed over the 16-lane group
//      (one DPP row);
//   2. softmax within the chunk: max, exp, sum per head (one wave a head);
//   3. P V: each lane accumulates QPK x 8 outputs, then the 16 groups are
//      summed in LDS in group order.
// With one chunk the output is written directly.  Otherwise each workgroup
// publishes (max, sum, unnormalised P V) with device-coherent stores and the
// last workgroup of the kv head (agent-scope counter) combines the chunks:
// per head, the global max, the chunk weights exp(max_c - max) and the total
// are formed in LDS (fixed order), then every output sums its chunks in chunk
// order.  The first 8 to 32 chunks' partial outputs are loaded in the same
// round as the maxima and sums.  Deterministic, one launch.
template <int QPK>
__global__ __launch_bounds__(kGlueThreads) void attention_decode_kernel(AttnArgs a) {
  constexpr int HD = kHeadDim;
  constexpr int TPG = kChunk / 16;  // tokens per 16-lane group
  constexpr float kScale = 0.08838834764831845f;  // 1 / sqrt(128)
  __shared__ float qs[QPK][HD];
  __shared__ __attribute__((aligned(16))) _Float16 knew[HD];
  __shared__ __attribute__((aligned(16))) _Float16 vnew[HD];
  __shared__ float sc[QPK][kChunk];
  __shared__ float red[16][QPK][HD];
  __shared__ float mrow[QPK], lrow[QPK];
  __shared__ float wchunk[kAttnMaxChunks][QPK];  // chunk max, then chunk weight
  __shared__ float lchunk[kAttnMaxChunks][QPK];  // chunk sum
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = blockIdx.x;
  const int c = blockIdx.y;
  const int n_heads = a.n_kv * QPK;
  const int t0 = c * kChunk;
  const int t1 = min(t0 + kChunk, a.pos + 1);
  const size_t row0 = static_cast<size_t>(h) * a.max_seq;  // cache row of token 0
  const int g16 = tid >> 4;
  const int j = tid & 15;

  // Every load of the prologue is issued before any of them is used, so the
  // prologue costs one memory round trip: this thread's q elements with their
  // rotary partners and cos / sin, the new token's k and v, then the cached
  // rows (issued last: the rotary work waits only for the loads before them).
  // Buffer loads without branches: a lane with nothing to load passes an
  // offset beyond the resource (it reads zero), and without rotary tables the
  // cos / sin resources are empty.
  constexpr int QE = (QPK * HD + kGlueThreads - 1) / kGlueThreads;  // q elements per thread
  const bool rope = a.rope_cos != nullptr;
  const uint32_t rope_bytes = rope ? static_cast<uint32_t>(a.max_seq) * kRopeHalf * 4u : 0u;
  const auto rq = make_rsrc(a.qkv, static_cast<uint32_t>(n_heads + 2 * a.n_kv) * HD * 2u);
  const auto rcos = make_rsrc(a.rope_cos, rope_bytes);
  const auto rsin = make_rsrc(a.rope_sin, rope_bytes);
  const uint32_t rope_row = static_cast<uint32_t>(a.pos) * kRopeHalf * 4u;
  const bool writer = t1 == a.pos + 1 && tid < HD;  // writes the new token's k and v
  auto ld16 = [&](uint32_t off) {
    return __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rq, off, 0, 0));
  };
  auto ld32 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  };
  _Float16 qx[QE], qp[QE];
  float qc[QE], qn[QE];
#pragma unroll
  for (int u = 0; u < QE; ++u) {
    const int e = tid + u * kGlueThreads;
    const int d = e % HD;
    const uint32_t base = e < QPK * HD ? static_cast<uint32_t>(h * QPK * HD + e - d) * 2u
                                       : kOutOfRange;
    const uint32_t rot = e < QPK * HD ? rope_row + static_cast<uint32_t>(d & (kRopeHalf - 1)) * 4u
                                      : kOutOfRange;
    qx[u] = ld16(base + static_cast<uint32_t>(d) * 2u);
    qp[u] = ld16(base + static_cast<uint32_t>(d ^ kRopeHalf) * 2u);
    qc[u] = ld32(rcos, rot);
    qn[u] = ld32(rsin, rot);
  }
  const uint32_t kbase = writer ? static_cast<uint32_t>((n_heads + h) * HD) * 2u : kOutOfRange;
  const uint32_t vbase = writer ? static_cast<uint32_t>((n_heads + a.n_kv + h) * HD) * 2u
                                : kOutOfRange;
  const uint32_t krot = writer ? rope_row + static_cast<uint32_t>(tid & (kRopeHalf - 1)) * 4u
                               : kOutOfRange;
  const _Float16 kx0 = ld16(kbase + static_cast<uint32_t>(tid) * 2u);
  const _Float16 kxp = ld16(kbase + static_cast<uint32_t>(tid ^ kRopeHalf) * 2u);
  const _Float16 vx0 = ld16(vbase + static_cast<uint32_t>(tid) * 2u);
  const float kc = ld32(rcos, krot);
  const float kn_s = ld32(rsin, krot);
  // This kv head's cache rows (max_seq x 128 fp16 each, under 2^31 bytes:
  // max_seq is bounded on the host); rows outside the chunk and the current
  // token's (not written yet) read as zero.
  const uint32_t head_bytes = static_cast<uint32_t>(a.max_seq) * HD * 2u;
  const auto rk = make_rsrc(a.k_cache + row0 * HD, head_bytes);
  const auto rv = make_rsrc(a.v_cache + row0 * HD, head_bytes);
  h8_t kr[TPG], vr[TPG];
#pragma unroll
  for (int u = 0; u < TPG; ++u) {
    const int t = t0 + g16 + 16 * u;
    const uint32_t off = t < t1 && t != a.pos ? static_cast<uint32_t>(t * HD + 8 * j) * 2u
                                              : kOutOfRange;
    kr[u] = __builtin_bit_cast(h8_t, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
    vr[u] = __builtin_bit_cast(h8_t, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
  }

#pragma unroll
  for (int u = 0; u < QE; ++u) {
    const int e = tid + u * kGlueThreads;
    if (e < QPK * HD) {
      const int hq = e / HD, d = e % HD;
      const float v = rope ? rotate_half(qx[u], qp[u], qc[u], qn[u], d) : static_cast<float>(qx[u]);
      qs[hq][d] = v * kScale;
    }
  }
  if (writer) {
    const _Float16 kn = static_cast<_Float16>(
        rope ? rotate_half(kx0, kxp, kc, kn_s, tid) : static_cast<float>(kx0));
    knew[tid] = kn;
    vnew[tid] = vx0;
    a.k_cache[(row0 + a.pos) * HD + tid] = kn;
    a.v_cache[(row0 + a.pos) * HD + tid] = vx0;
  }
  __syncthreads();

  float qr[QPK][8];
#pragma unroll
  for (int hq = 0; hq < QPK; ++hq)
#pragma unroll
    for (int i = 0; i < 8; ++i) qr[hq][i] = qs[hq][8 * j + i];
#pragma unroll
  for (int u = 0; u < TPG; ++u) {
    const int t = t0 + g16 + 16 * u;
    if (t == a.pos) {
      kr[u] = *reinterpret_cast<const h8_t*>(&knew[8 * j]);
      vr[u] = *reinterpret_cast<const h8_t*>(&vnew[8 * j]);
    }
    // The whole 16-lane group (a DPP row) shares t, so all its lanes take
    // part in the row sum.
    if (t < t1) {
      float s[QPK];
#pragma unroll
      for (int hq = 0; hq < QPK; ++hq) {
        s[hq] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          s[hq] = __builtin_fmaf(qr[hq][i], static_cast<float>(kr[u][i]), s[hq]);
        s[hq] = row16_sum(s[hq]);
      }
      if (j == 0) {
#pragma unroll
        for (int hq = 0; hq < QPK; ++hq) sc[hq][t - t0] = s[hq];
      }
    }
  }
  __syncthreads();

  const int nt = t1 - t0;  // >= 1: the host sizes the grid so every chunk has a token
  for (int hq = wave; hq < QPK; hq += kGlueThreads / 64) {
    float m = -INFINITY;
    for (int t = lane; t < nt; t += 64) m = fmaxf(m, sc[hq][t]);
    m = wave_max(m);
    float l = 0.0f;
    for (int t = lane; t < nt; t += 64) {
      const float p = __expf(sc[hq][t] - m);
      sc[hq][t] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      mrow[hq] = m;
      lrow[hq] = l;
    }
  }
  __syncthreads();

  float acc[QPK][8];
#pragma unroll
  for (int hq = 0; hq < QPK; ++hq)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[hq][i] = 0.0f;
#pragma unroll
  for (int u = 0; u < TPG; ++u) {
    const int t = t0 + g16 + 16 * u;
    if (t < t1) {
#pragma unroll
      for (int hq = 0; hq < QPK; ++hq) {
        const float p = sc[hq][t - t0];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          acc[hq][i] = __builtin_fmaf(p, static_cast<float>(vr[u][i]), acc[hq][i]);
      }
    }
  }
#pragma unroll
  for (int hq = 0; hq < QPK; ++hq)
#pragma unroll
    for (int i = 0; i < 8; ++i) red[g16][hq][8 * j + i] = acc[hq][i];
  __syncthreads();

  const bool direct = a.chunks == 1;
  for (int e = tid; e < QPK * HD; e += kGlueThreads) {
    const int hq = e / HD, d = e % HD;
    float o = 0.0f;
#pragma unroll
    for (int g = 0; g < 16; ++g) o += red[g][hq][d];
    if (direct) {
      a.out[static_cast<size_t>(h * QPK + hq) * HD + d] = static_cast<_Float16>(o / lrow[hq]);
    } else {
      float* P = a.partial + ((static_cast<size_t>(h) * a.chunks + c) * QPK + hq) * (HD + 2);
      store_coherent(P + 2 + d, o);
      if (d == 0) {
        store_coherent(P, mrow[hq]);
        store_coherent(P + 1, lrow[hq]);
      }
    }
  }
  if (direct) return;

  // Last-arriver exchange; relies on gfx950 hardware ordering: see
  // "HARDWARE ASSUMPTION" in nibble_decode.h.
  wait_vm_stores();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(a.counters + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == static_cast<uint32_t>(a.chunks - 1);
  }
  __syncthreads();
  if (!s_last) return;

  auto chunk_part = [&](int cc, int hq) {
    return a.partial + ((static_cast<size_t>(h) * a.chunks + cc) * QPK + hq) * (HD + 2);
  };
  // One round of loads for up to PRE chunks: every chunk's (max, sum) into
  // LDS, and this thread's partial outputs of the first PRE chunks into
  // registers, all issued together.
  constexpr int OUTS = (QPK * HD + kGlueThreads - 1) / kGlueThreads;  // outputs per thread
  constexpr int PRE = 32 / OUTS;
  float pv[OUTS][PRE];
#pragma unroll
  for (int k = 0; k < OUTS; ++k) {
    const int e = tid + k * kGlueThreads;
#pragma unroll
    for (int u = 0; u < PRE; ++u)
      pv[k][u] = e < QPK * HD && u < a.chunks
                     ? load_coherent(chunk_part(u, e / HD) + 2 + e % HD)
                     : 0.0f;
  }
  for (int e = tid; e < a.chunks * QPK; e += kGlueThreads) {
    const float* P = chunk_part(e / QPK, e % QPK);
    const float mx = load_coherent(P);
    const float sm = load_coherent(P + 1);
    __builtin_amdgcn_sched_barrier(0);  // both loads in flight before either store waits
    wchunk[e / QPK][e % QPK] = mx;
    lchunk[e / QPK][e % QPK] = sm;
  }
  __syncthreads();
  // Per head, over the chunks in order: the global max M, the chunk weights
  // exp(max_c - M), and the total L = sum_c sum_c * weight_c.
  if (tid < QPK) {
    float M = -INFINITY;
    for (int cc = 0; cc < a.chunks; ++cc) M = fmaxf(M, wchunk[cc][tid]);
    mrow[tid] = M;
  }
  __syncthreads();
  for (int e = tid; e < a.chunks * QPK; e += kGlueThreads) {
    const int cc = e / QPK, hq = e % QPK;
    wchunk[cc][hq] = __expf(wchunk[cc][hq] - mrow[hq]);
  }
  __syncthreads();
  if (tid < QPK) {
    float L = 0.0f;
    for (int cc = 0; cc < a.chunks; ++cc) L += lchunk[cc][tid] * wchunk[cc][tid];
    lrow[tid] = L;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < OUTS; ++k) {
    const int e = tid + k * kGlueThreads;
    if (e >= QPK * HD) continue;
    const int hq = e / HD, d = e % HD;
    float o = 0.0f;
#pragma unroll
    for (int u = 0; u < PRE; ++u)
      if (u < a.chunks) o += pv[k][u] * wchunk[u][hq];
    for (int c0 = PRE; c0 < a.chunks; c0 += 8) {  // beyond the prefetch: eight loads a round
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = c0 + u < a.chunks ? load_coherent(chunk_part(c0 + u, hq) + 2 + d) : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (c0 + u < a.chunks) o += v[u] * wchunk[c0 + u][hq];
    }
    a.out[static_cast<size_t>(h * QPK + hq) * HD + d] = static_cast<_Float16>(o / lrow[hq]);
  }
  if (tid == 0) __hip_atomic_store(a.counters + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int attn_chunks(int64_t pos) { return static_cast<int>(ceil_div(pos + 1, kChunk)); }

struct AttnPlan {
  int qpk = 0, chunks = 0;
  size_t counter_bytes = 0, workspace_bytes = 0;
};

int plan_attention(int64_t n_heads, int64_t n_kv, int64_t head_dim, int64_t max_seq, int64_t pos,
                   AttnPlan* p) {
  NIBBLE_CHECK(head_dim == kHeadDim, "head_dim must be %d, got %lld", kHeadDim,
               (long long)head_dim);
  NIBBLE_CHECK(n_kv >= 1 && n_kv <= 65535, "n_kv_heads must be in [1, 65535], got %lld",
               (long long)n_kv);
  NIBBLE_CHECK(n_heads >= n_kv && n_heads % n_kv == 0,
               "n_heads (%lld) must be a multiple of n_kv_heads (%lld)", (long long)n_heads,
               (long long)n_kv);
  const int64_t qpk = n_heads / n_kv;
  NIBBLE_CHECK(qpk == 1 || qpk == 2 || qpk == 4 || qpk == 8,
               "query heads per kv head must be 1, 2, 4 or 8, got %lld", (long long)qpk);
  NIBBLE_CHECK(pos >= 0 && pos < max_seq, "pos (%lld) must be in [0, max_seq = %lld)",
               (long long)pos, (long long)max_seq);
  // The combine keeps every chunk's (max, sum) in LDS: at most 512 chunks.
  NIBBLE_CHECK(max_seq <= kAttnMaxSeq, "max_seq above %d", kAttnMaxSeq);
  p->qpk = static_cast<int>(qpk);
  p->chunks = attn_chunks(pos);
  if (p->chunks > 1) {
    p->counter_bytes = align_up(static_cast<size_t>(n_kv) * 4, 256);
    p->workspace_bytes = p->counter_bytes + static_cast<size_t>(n_kv) * p->chunks * qpk *
                                                (kHeadDim + 2) * sizeof(float);
  }
  return NIBBLE_OK;
}

template <int QPK>
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(a.n_kv), static_cast<unsigned>(a.chunks));
  attention_decode_kernel<QPK><<<grid, kGlueThreads, 0, stream>>>(a);
  return hipGetLastError();
}

template <int CH>
hipError_t launch_rmsnorm(const _Float16* X, const _Float16* W, _Float16* Y, int64_t rows,
                          int cols, float eps, hipStream_t stream) {
  rmsnorm_kernel<CH><<<dim3(static_cast<unsigned>(rows)), kGlueThreads, 0, stream>>>(X, W, Y, cols,
                                                                                    eps);
  return hipGetLastError();
}

}  // namespace

}  // namespace nibble

using namespace nibble;

extern "C" int nibble_rmsnorm_f16(const void* X, int64_t rows, int64_t cols, const void* W,
                                  float eps, void* Y, void* stream_) {
  NIBBLE_CHECK(rows >= 0 && rows <= 0x7fffffff, "rows must be in [0, 2^31), got %lld",
               (long long)rows);
  NIBBLE_CHECK(cols > 0 && cols % 8 == 0 && cols <= kRmsMaxCols,
               "cols must be a positive multiple of 8 up to %d, got %lld", kRmsMaxCols,
               (long long)cols);
  NIBBLE_CHECK(std::isfinite(eps) && eps >= 0.0f, "eps must be finite and >= 0");
  if (rows == 0) return ok();
  NIBBLE_CHECK(X != nullptr && W != nullptr && Y != nullptr, "null pointer");
  NIBBLE_CHECK(aligned(X, 16) && aligned(W, 16) && aligned(Y, 16),
               "X, W and Y must be 16-byte aligned");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  const auto* x = static_cast<const _Float16*>(X);
  const auto* w = static_cast<const _Float16*>(W);
  auto* y = static_cast<_Float16*>(Y);
  const int c = static_cast<int>(cols);
  const int ch = static_cast<int>(ceil_div(cols, kGlueThreads * 8));
  hipError_t e = ch <= 1   ? launch_rmsnorm<1>(x, w, y, rows, c, eps, stream)
                 : ch <= 2 ? launch_rmsnorm<2>(x, w, y, rows, c, eps, stream)
                 : ch <= 4 ? launch_rmsnorm<4>(x, w, y, rows, c, eps, stream)
                           : launch_rmsnorm<8>(x, w, y, rows, c, eps, stream);
  NIBBLE_HIP(e);
  return ok();
}

extern "C" size_t nibble_attention_decode_workspace_bytes(int64_t n_heads, int64_t n_kv_heads,
                                                          int64_t head_dim, int64_t max_seq,
                                                          int64_t pos, void* stream) {
  (void)stream;
  AttnPlan p;
  if (plan_attention(n_heads, n_kv_heads, head_dim, max_seq, pos, &p) != NIBBLE_OK) return 0;
  return p.workspace_bytes;
}

extern "C" size_t nibble_attention_decode_counter_bytes(int64_t n_heads, int64_t n_kv_heads,
                                                        int64_t head_dim, int64_t max_seq,
                                                        int64_t pos, void* stream) {
  (void)stream;
  AttnPlan p;
  if (plan_attention(n_heads, n_kv_heads, head_dim, max_seq, pos, &p) != NIBBLE_OK) return 0;
  return p.counter_bytes;
}

extern "C" int nibble_attention_decode_f16(const void* QKV, int64_t n_heads, int64_t n_kv_heads,
                                           int64_t head_dim, void* K_cache, void* V_cache,
                                           int64_t max_seq, int64_t pos, const void* rope_cos,
                                           const void* rope_sin, void* Out, void* workspace,
                                           size_t workspace_bytes, void* stream_) {
  AttnPlan p;
  int rc = plan_attention(n_heads, n_kv_heads, head_dim, max_seq, pos, &p);
  if (rc != NIBBLE_OK) return rc;
  NIBBLE_CHECK(QKV != nullptr && K_cache != nullptr && V_cache != nullptr && Out != nullptr,
               "null pointer");
  NIBBLE_CHECK(aligned(QKV, 16) && aligned(K_cache, 16) && aligned(V_cache, 16) &&
                   aligned(Out, 16),
               "qkv, caches and output must be 16-byte aligned");
  NIBBLE_CHECK((rope_cos == nullptr) == (rope_sin == nullptr),
               "rope_cos and rope_sin must both be given or both be null");
  NIBBLE_CHECK(rope_cos == nullptr || (aligned(rope_cos, 4) && aligned(rope_sin, 4)),
               "rope tables must be 4-byte aligned");
  if (p.workspace_bytes > 0) {
    if (workspace == nullptr || workspace_bytes < p.workspace_bytes)
      return fail(NIBBLE_ERR_WORKSPACE, "attention needs %zu bytes of workspace, got %zu",
                  p.workspace_bytes, workspace == nullptr ? size_t(0) : workspace_bytes);
    if (!aligned(workspace, 256))
      return fail(NIBBLE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  AttnArgs a;
  a.qkv = static_cast<const _Float16*>(QKV);
  a.k_cache = static_cast<_Float16*>(K_cache);
  a.v_cache = static_cast<_Float16*>(V_cache);
  a.rope_cos = static_cast<const float*>(rope_cos);
  a.rope_sin = static_cast<const float*>(rope_sin);
  a.out = static_cast<_Float16*>(Out);
  a.counters = p.chunks > 1 ? static_cast<uint32_t*>(workspace) : nullptr;
  a.partial = p.chunks > 1
                  ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.counter_bytes)
                  : nullptr;
  a.n_kv = static_cast<int>(n_kv_heads);
  a.max_seq = static_cast<int>(max_seq);
  a.pos = static_cast<int>(pos);
  a.chunks = p.chunks;
  hipError_t e = p.qpk == 1   ? launch_attention<1>(a, stream)
                 : p.qpk == 2 ? launch_attention<2>(a, stream)
                 : p.qpk == 4 ? launch_attention<4>(a, stream)
                              : launch_attention<8>(a, stream);
  NIBBLE_HIP(e);
  return ok();
}
