// Prefill-regime W4A16 matmul on CDNA4 MFMA: Y[M,N] = X[M,K] @ dequant(Wq, S).
//
// Reference: csrc/gemm_w4a16.cu (tile staging :66-146, kernels :151-377, host
// checks :379-429).  The reference decodes B into shared memory and feeds
// wmma / mma.sync; here the tile feeds v_mfma_f32_32x32x16_f16.
//
// Two kernels share the tile arithmetic.  gemm_pc64_kernel (further down)
// runs wherever its 16-byte B loads apply: four waves multiply while four
// others load and decode the next 64-k step.  gemm_tile_kernel, described
// here, serves the remaining operands (N % 4 != 0, under-aligned weights).
//
// Tile: BM x BN x 32 per workgroup of 4 wave64s (2 x 2), each wave owning a
// (BM/2) x (BN/2) block of 32 x 32 MFMA tiles.  Per 32-k step:
//   * A (X, fp16): 16-byte global loads into registers, rows past M read as
//     zero, then stored to LDS;
//   * B: each thread loads BN/64 adjacent packed words of one packed row (a
//     wave covers one packed row of the tile, 4*BN contiguous bytes).  Every
//     word is exactly 8 consecutive k of one column: it is decoded with the
//     magic-exponent trick and multiplied by the group scale (one RNE
//     rounding, so the LDS tile holds exactly dequantize()'s fp16 values, as
//     the reference's does, gemm_w4a16.cu:137-146) and stored n-major
//     (k contiguous) with one 16-byte LDS store -- one MFMA B-operand lane;
//   * the next step's global loads are issued before the current step's
//     MFMAs and written to the other LDS buffer after them: one barrier per
//     step;
//   * each wave reads its operands with ds_read_b128 (the swizzled layout of
//     lds_unit keeps reads and stores free of bank conflicts) and issues
//     (BM/64) x (BN/64) MFMAs per 16 k with fp32 accumulation.
//
// MFMA operand layout (32x32x16 f16): lane l supplies row (A) / column (B)
// l % 32 and the 8 k of block l / 32; result register r of lane l holds
// column l % 32, row 8 * (r / 4) + 4 * (l / 32) + r % 4.
#include <algorithm>
#include <type_traits>

#include "nibble_common.h"
#include "nibble_decode.h"
#include "stream_matmul.h"

namespace nibble {

namespace {

typedef float f16_t __attribute__((ext_vector_type(16)));

constexpr int BK = 32;
// LDS tile layout.  A tile row (an A row or a B column) holds BK = 32 fp16
// as four 16-byte units, rows 64 bytes apart with no padding.  Rows are
// permuted within aligned groups of four and the units of a row XOR-swizzled,
// both by low row bits, so that every 16-lane phase of the three access
// patterns touches 16 distinct units -- all 64 banks once -- (and every
// 8-lane phase all of 32 banks once):
//   * operand reads: 16 consecutive rows, one unit each;
//   * A stores: 4 consecutive rows, all 4 units each;
//   * B stores: 16 rows 1 or 2 apart (a lane's 1 or 2 adjacent columns), one
//     unit each -- with a 64-byte pitch, rows of one parity alone cover only
//     half the banks, hence the row permutation.
// Found by exhaustive search over linear (XOR) maps of the row bits.
__device__ __forceinline__ int lds_unit(int r, int c) {
  const int p0 = (r ^ (r >> 3) ^ (r >> 4)) & 1;
  const int p1 = ((r >> 1) ^ (r >> 3)) & 1;
  const int f = ((r >> 1) & 1) | (((r >> 2) & 1) << 1);
  return 4 * ((r & ~3) + p0 + 2 * p1) + (c ^ f);
}
constexpr int LDK = BK;  // fp16 elements per tile row
constexpr int kGemmThreads = 256;  // 4 waves as 2 x 2
constexpr int kStages = 4;         // 32-k steps of global loads in flight

template <int BM, int BN>
struct TileCfg {
  static constexpr int WM = BM / 2, WN = BN / 2;    // wave tile
  static constexpr int TM = WM / 32, TN = WN / 32;  // 32 x 32 MFMA tiles per wave
  static constexpr int A_ITERS = BM * (BK / 8) / kGemmThreads;  // 16-byte A chunks per thread
  static constexpr int VB = BN / 64;                // packed words per thread per step
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32 x 32 MFMA tile");
  static_assert(A_ITERS >= 1, "A tile must give every thread a chunk");
  static_assert(VB == 1 || VB == 2 || VB == 4, "B words per thread");
};

// VB adjacent packed words (and their fp16 scales) of one packed row, as one
// buffer load each.
template <int VB>
struct BWords;
template <>
struct BWords<4> {
  using word_t = u4_t;
  using scale_t = h4_t;
  static __device__ __forceinline__ word_t load_w(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(r, v, s, 0));
  }
  static __device__ __forceinline__ scale_t load_s(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_bit_cast(h4_t, __builtin_amdgcn_raw_buffer_load_b64(r, v, s, 0));
  }
  static __device__ __forceinline__ uint32_t word(word_t w, int j) { return w[j]; }
  static __device__ __forceinline__ _Float16 scale(scale_t x, int j) { return x[j]; }
};
template <>
struct BWords<2> {
  using word_t = u2_t;
  using scale_t = h2_t;
  static __device__ __forceinline__ word_t load_w(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_bit_cast(u2_t, __builtin_amdgcn_raw_buffer_load_b64(r, v, s, 0));
  }
  static __device__ __forceinline__ scale_t load_s(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_raw_buffer_load_b32(r, v, s, 0));
  }
  static __device__ __forceinline__ uint32_t word(word_t w, int j) { return w[j]; }
  static __device__ __forceinline__ _Float16 scale(scale_t x, int j) { return x[j]; }
};
template <>
struct BWords<1> {
  using word_t = uint32_t;
  using scale_t = _Float16;
  static __device__ __forceinline__ word_t load_w(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, v, s, 0);
  }
  static __device__ __forceinline__ scale_t load_s(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    return __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, v, s, 0));
  }
  static __device__ __forceinline__ uint32_t word(word_t w, int) { return w; }
  static __device__ __forceinline__ _Float16 scale(scale_t x, int) { return x; }
};

__device__ __forceinline__ f16_t mfma32(h8_t a, h8_t b, f16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

struct TileArgs {
  const _Float16* X;
  const uint32_t* Wq;
  const _Float16* S;
  _Float16* Y;
  float* partial;      // [splits, M, N] fp32 when splits > 1
  uint32_t* counters;  // [tiles], zero on entry and on exit
  int M, K, N;
  int steps_per_split;  // 32-k steps per K split
  int splits;
  WeightLayout L;       // where a column's words and scales live (packed or strip-major)
};

// Last-arriver sum of a split output tile [m0, m0 + BM) x [n0, n0 + BN) by
// the whole workgroup: each thread takes 16-byte chunks of 4 columns and
// loads the chunk's partial of every split (up to 4 in one round, with the
// same device-coherent cache policy as load_coherent) before adding them in
// split order, then stores the 4 fp16 results.  Chunks go two at a time, so
// a thread has at most 8 loads in flight and the kernels keep their
// register budget.  Needs N % 4 == 0 (16-byte partial rows, 8-byte output
// stores) and M * N * 4 < 2^31 (32-bit buffer offsets; the plans split only
// grids of a few hundred tiles).
template <int THREADS, int BM, int BN>
__device__ __forceinline__ void tile_sum_splits(const TileArgs& args, int m0, int n0) {
  constexpr int QUADS = BN / 4;
  constexpr int CHUNKS = BM * QUADS;
  constexpr int kPair = 2, kBatch = 4;
  constexpr bool kWholeRounds = CHUNKS % (THREADS * kPair) == 0;
  constexpr uint32_t kCoherent = 16;  // sc1: the cache policy of an agent-scope load
  const int M = args.M, N = args.N;
  const uint32_t plane = static_cast<uint32_t>(M) * static_cast<uint32_t>(N);
  // The ABI asks only 2-byte alignment of Y: 8-byte stores when it has more.
  const bool y_quads = (reinterpret_cast<uintptr_t>(args.Y) & 7u) == 0;
#pragma nounroll
  for (int c0 = 0; c0 < CHUNKS; c0 += THREADS * kPair) {
    uint32_t off[kPair];
    bool ok[kPair];
#pragma unroll
    for (int u = 0; u < kPair; ++u) {
      const int c = c0 + u * THREADS + static_cast<int>(threadIdx.x);
      const int gm = m0 + c / QUADS, gn = n0 + 4 * (c % QUADS);
      ok[u] = gm < M && gn < N && (kWholeRounds || c < CHUNKS);
      off[u] = ok[u] ? (static_cast<uint32_t>(gm) * N + gn) * 4u : kOutOfRange;
    }
    f4_t sum[kPair] = {};
    for (int sp0 = 0; sp0 < args.splits; sp0 += kBatch) {
      f4_t v[kBatch][kPair];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int sp = sp0 + b < args.splits ? sp0 + b : 0;
        const __amdgpu_buffer_rsrc_t rp =
            make_rsrc(args.partial + static_cast<size_t>(sp) * plane, plane * 4u);
#pragma unroll
        for (int u = 0; u < kPair; ++u)
          v[b][u] = __builtin_bit_cast(
              f4_t, __builtin_amdgcn_raw_buffer_load_b128(rp, off[u], 0, kCoherent));
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
        if (sp0 + b < args.splits) {
#pragma unroll
          for (int u = 0; u < kPair; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[u][e] += v[b][u][e];
        }
    }
#pragma unroll
    for (int u = 0; u < kPair; ++u)
      if (ok[u]) {
        const h4_t y = {(_Float16)sum[u][0], (_Float16)sum[u][1], (_Float16)sum[u][2],
                        (_Float16)sum[u][3]};
        _Float16* dst = args.Y + off[u] / 4;
        if (y_quads) {
          *reinterpret_cast<h4_t*>(dst) = y;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[e] = y[e];
        }
      }
  }
}

template <int BM, int BN, int GROUP>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void
gemm_tile_kernel(TileArgs args) {
  using C = TileCfg<BM, BN>;
  constexpr int VB = C::VB;
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDK];
  __shared__ int s_last;
  const _Float16* __restrict__ X = args.X;
  const uint32_t* __restrict__ Wq = args.Wq;
  const _Float16* __restrict__ S = args.S;
  _Float16* __restrict__ Y = args.Y;
  const int M = args.M, K = args.K, N = args.N;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * C::WM;
  const int wn = (wave & 1) * C::WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;

  f16_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Staging registers for one 32-k step.  kStages steps are in flight at
  // once (rotating register sets, indexed only by compile-time constants);
  // the LDS holds two steps (the one being multiplied and the next).  All
  // staging is in vector values (no small arrays the compiler could move to
  // memory), and every load is an unpredicated buffer load: rows past M and
  // columns past N use an offset outside the buffer and read zero.
  using BVec = typename BWords<VB>::word_t;
  using SVec = typename BWords<VB>::scale_t;
  struct Stage {
    h8_t a[C::A_ITERS];
    BVec b;
    SVec s;
  };
  // B: thread tid loads packed row (tid / 64) of the step, columns
  // n0 + VB * (tid % 64) .. + VB - 1.
  const int b_row = tid >> 6;
  const int b_col = n0 + VB * (tid & 63);
  // This workgroup's K split: steps [step0, step0 + ntiles) of 32 k.
  const int step0 = blockIdx.z * args.steps_per_split;
  const int ntiles = min(args.steps_per_split, K / BK - step0);
  const uint32_t row_bytes = args.L.w_row;
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(X, static_cast<uint32_t>(M) * static_cast<uint32_t>(K) * 2u);
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(Wq, static_cast<uint32_t>(K / 8) * static_cast<uint32_t>(N) * 4u);
  const __amdgpu_buffer_rsrc_t rsc =
      make_rsrc(S, static_cast<uint32_t>(K / GROUP) * static_cast<uint32_t>(N) * 2u);
  uint32_t voff_a[C::A_ITERS];
#pragma unroll
  for (int it = 0; it < C::A_ITERS; ++it) {
    const int e = tid + it * kGemmThreads;
    const int gm = m0 + (e >> 2);
    voff_a[it] = gm < M ? (static_cast<uint32_t>(gm) * K + (e & 3) * 8) * 2u : kOutOfRange;
  }
  const bool b_ok = b_col < N;
  const uint32_t voff_b = b_ok ? b_row * row_bytes + args.L.wcol(b_col) : kOutOfRange;
  const uint32_t voff_s = b_ok ? args.L.scol(b_col) : kOutOfRange;

  // Loads of step `step`, clamped to the last step: a prefetch past the end
  // re-reads it (an L2 hit) rather than being skipped, so the loads are the
  // same on every path and the compiler's in-order wait counts stay exact.
  auto load_step = [&](Stage& st, int step) {
    const uint32_t k0 = static_cast<uint32_t>((step0 + min(step, ntiles - 1)) * BK);
#pragma unroll
    for (int it = 0; it < C::A_ITERS; ++it)
      st.a[it] = __builtin_bit_cast(h8_t, __builtin_amdgcn_raw_buffer_load_b128(rx, voff_a[it], k0 * 2u, 0));
    st.b = BWords<VB>::load_w(rw, voff_b, (k0 / 8) * row_bytes);
    st.s = BWords<VB>::load_s(rsc, voff_s, (k0 / GROUP) * args.L.s_row);
  };
  // LDS offsets (fp16 elements).  Rows 64 apart share the swizzle of their
  // low 5 bits, so each offset is a per-thread constant plus a row multiple.
  // A stores: thread tid writes row tid / 4 + 64 it, unit tid % 4.
  const int a_st = lds_unit(tid >> 2, tid & 3) * 8;
  // B stores: columns VB * (tid % 64) + j, unit b_row.
  int b_st[VB];
#pragma unroll
  for (int j = 0; j < VB; ++j) b_st[j] = lds_unit(VB * (tid & 63) + j, b_row) * 8;
  auto store_step = [&](const Stage& st, int buf) {
#pragma unroll
    for (int it = 0; it < C::A_ITERS; ++it)
      *reinterpret_cast<h8_t*>(&As[buf][a_st + it * 64 * LDK]) = st.a[it];
#pragma unroll
    for (int j = 0; j < VB; ++j) {
      h2_t w[4];
      const _Float16 sj = BWords<VB>::scale(st.s, j);
      const h2_t s2 = {sj, sj};
      decode8_scaled(BWords<VB>::word(st.b, j), s2, w);
      const h8_t v = {w[0][0], w[0][1], w[1][0], w[1][1], w[2][0], w[2][1], w[3][0], w[3][1]};
      *reinterpret_cast<h8_t*>(&Bs[buf][b_st[j]]) = v;
    }
  };
  // Operand reads: row (32 i + lane % 32) of a wave's 32-row block, unit
  // 2 ks + lane / 32 (the lane's 8 k of the 16-k MFMA step ks).
  const int r32 = lane & 31;
  int rd[BK / 16];
#pragma unroll
  for (int ks = 0; ks < BK / 16; ++ks) rd[ks] = lds_unit(r32, 2 * ks + (lane >> 5)) * 8;
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      h8_t a[C::TM], b[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
        a[i] = *reinterpret_cast<const h8_t*>(&As[buf][(wm + 32 * i) * LDK + rd[ks]]);
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        b[j] = *reinterpret_cast<const h8_t*>(&Bs[buf][(wn + 32 * j) * LDK + rd[ks]]);
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    }
  };

  Stage R[kStages];
#pragma unroll
  for (int i = 0; i < kStages; ++i) load_step(R[i], i);
  store_step(R[0], 0);
  __syncthreads();
  // Step t: refill the register set that held step t (already in LDS) with
  // step t + kStages, multiply step t from LDS, then move step t + 1 from its
  // registers into the other LDS buffer.
  auto iter = [&](auto u_const, int t) {
    constexpr int u = decltype(u_const)::value;
    load_step(R[u], t + kStages);
    __builtin_amdgcn_sched_barrier(0);  // keep the refill ahead of the MFMAs
    compute(t & 1);
    __builtin_amdgcn_sched_barrier(0);
    store_step(R[(u + 1) % kStages], (t + 1) & 1);
    __syncthreads();
  };
  // Whole rounds of kStages steps with no exit in the middle (an exit after
  // each step makes the compiler keep a copy of the accumulators per exit),
  // then the remaining 0..kStages-1 steps once.
  int t = 0;
  for (; t + kStages <= ntiles; t += kStages) {
    iter(std::integral_constant<int, 0>{}, t);
    iter(std::integral_constant<int, 1>{}, t + 1);
    iter(std::integral_constant<int, 2>{}, t + 2);
    iter(std::integral_constant<int, 3>{}, t + 3);
  }
  const int rem = ntiles - t;
  if (rem > 0) iter(std::integral_constant<int, 0>{}, t);
  if (rem > 1) iter(std::integral_constant<int, 1>{}, t + 1);
  if (rem > 2) iter(std::integral_constant<int, 2>{}, t + 2);

  // Epilogue: register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4,
  // column l % 32 of each 32 x 32 tile.
  const int rq = (lane >> 5) * 4;
  if (args.splits == 1) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        const int gn = n0 + wn + 32 * j + r32;
        if (gn >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = m0 + wm + 32 * i + 8 * (r >> 2) + rq + (r & 3);
          if (gm < M) Y[static_cast<size_t>(gm) * N + gn] = (_Float16)acc[i][j][r];
        }
      }
    }
    return;
  }

  // K split: publish this split's fp32 tile with device-coherent stores; the
  // last workgroup of the tile (agent-scope counter) sums the splits in
  // split order and writes Y -- deterministic, one launch.
  float* part = args.partial + static_cast<size_t>(blockIdx.z) * M * N;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int gn = n0 + wn + 32 * j + r32;
      if (gn >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + wm + 32 * i + 8 * (r >> 2) + rq + (r & 3);
        if (gm < M) store_coherent(part + static_cast<size_t>(gm) * N + gn, acc[i][j][r]);
      }
    }
  // Last-arriver exchange; relies on gfx950 hardware ordering: see
  // "HARDWARE ASSUMPTION" in nibble_decode.h.
  wait_vm_stores();
  __syncthreads();
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  if (tid == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(args.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == static_cast<uint32_t>(args.splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  if (N % 4 == 0) {
    tile_sum_splits<kGemmThreads, BM, BN>(args, m0, n0);
  } else {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        const int gn = n0 + wn + 32 * j + r32;
        if (gn >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = m0 + wm + 32 * i + 8 * (r >> 2) + rq + (r & 3);
          if (gm >= M) continue;
          const size_t off = static_cast<size_t>(gm) * N + gn;
          float sum = 0.0f;
          for (int sp = 0; sp < args.splits; ++sp)
            sum += load_coherent(args.partial + static_cast<size_t>(sp) * M * N + off);
          Y[off] = (_Float16)sum;
        }
      }
  }
  if (tid == 0)
    __hip_atomic_store(args.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Epilogue of the producer/consumer kernels: the consumer waves hold the
// results (wave block top-left (mw, nw), the tile kernel's register layout);
// every wave passes the barriers of the K-split exchange.
template <int TM, int TN, int THREADS, int BM, int BN, bool CAN_SPLIT = true>
__device__ __forceinline__ void pc_epilogue(const f16_t (&acc)[TM][TN], const TileArgs& args,
                                            bool producer, int mw, int nw, int& s_last) {
  const int M = args.M, N = args.N;
  const int lane = threadIdx.x & 63;
  const int r32 = lane & 31;
  const int rq = (lane >> 5) * 4;
  _Float16* __restrict__ Y = args.Y;
  // The large-tile kernel never splits K (CAN_SPLIT false): only this path.
  if (!CAN_SPLIT || args.splits == 1) {
    if (producer) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int gn = nw + 32 * j + r32;
        if (gn >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = mw + 32 * i + 8 * (r >> 2) + rq + (r & 3);
          if (gm < M) Y[static_cast<size_t>(gm) * N + gn] = (_Float16)acc[i][j][r];
        }
      }
    return;
  }
  float* part = args.partial + static_cast<size_t>(blockIdx.z) * M * N;
  if (!producer) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int gn = nw + 32 * j + r32;
        if (gn >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = mw + 32 * i + 8 * (r >> 2) + rq + (r & 3);
          if (gm < M) store_coherent(part + static_cast<size_t>(gm) * N + gn, acc[i][j][r]);
        }
      }
  }
  // Last-arriver exchange; relies on gfx950 hardware ordering: see
  // "HARDWARE ASSUMPTION" in nibble_decode.h.
  wait_vm_stores();
  __syncthreads();
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(args.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == static_cast<uint32_t>(args.splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  // Every wave (producers too) sums the tile: N % 4 == 0 for these kernels.
  tile_sum_splits<THREADS, BM, BN>(args, static_cast<int>(blockIdx.y) * BM,
                                   static_cast<int>(blockIdx.x) * BN);
  if (threadIdx.x == 0)
    __hip_atomic_store(args.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS layout of the 64-k producer/consumer kernel: rows of 64 fp16 (eight
// 16-byte units, 128 bytes, no padding), rows paired and XOR-swizzled by row
// bits 0..5 so that the operand reads (16 consecutive rows, one unit),
// A stores (2 rows x 8 units) and B stores (rows 4 apart, one unit) of every
// 16-lane phase cover all 64 banks once (and every 8-lane phase all 32).
__device__ __forceinline__ int lds_unit64(int r, int c) {
  const int s0 = (r ^ (r >> 5)) & 1;
  const int f = ((r ^ (r >> 3)) & 1) | (((r >> 1) ^ (r >> 4)) & 1) << 1 | ((r >> 2) & 1) << 2;
  return 8 * ((r & ~1) | s0) + (c ^ f);
}

// Producer/consumer form of the tile kernel, with 64-k steps: four producer
// waves and CWAVES (4 or 8) consumer waves.
//
// In the tile kernel above every wave loads, decodes and stores its share of
// the next step, waits at the barrier and then multiplies, so its MFMA pipe
// idles while it does the rest (busy about a quarter of a wave's lifetime at
// M = 2048).  Here the consumer waves only read operands from LDS and issue
// MFMAs (a 64 x 64 or 32 x 64 wave tile, 16 or 8 MFMAs per wave per step),
// while the four producer waves run the global-load pipeline and the decode,
// storing step t + 1 into the other LDS buffer while step t is multiplied.
// Consumers and producers share the SIMDs, so the decode VALU work and the
// memory waits overlap the MFMAs.  Both roles pass the same barriers, ntiles
// + 1 of them, one per step.
//  * CWAVES = 4 (eight waves, 2 x 2 consumers): BM = 64 or 128; two
//    workgroups per CU; PSTAGES = 4 steps of loads in flight.
//  * CWAVES = 8 (twelve waves, 4 x 2 consumers of 64 x 64): BM = 256, one
//    workgroup per CU (96 KiB of LDS).  Each decoded B tile then serves 256
//    rows, which halves the decode work and the B stores per FLOP; A's LDS
//    traffic per FLOP is unchanged.  PSTAGES = 2 (3 and 4 spill or measured
//    slower, 1 exposes the load latency).
//
// Producers: thread tid loads BM / 32 16-byte A chunks (rows tid / 8 + 32 it,
// unit tid % 8) and one dwordx4 of B -- packed row tid / 32 of the step,
// columns 4 (tid % 32) .. + 3 -- with its four scales.  BN = 128.
template <int BM, int GROUP, int CWAVES = 4, int PSTAGES = kStages>
__global__ __launch_bounds__((CWAVES + 4) * 64) void gemm_pc64_kernel(TileArgs args) {
  constexpr int BN = 128;
  constexpr int PBK = 64;
  constexpr int THREADS = (CWAVES + 4) * 64;
  constexpr int WROWS = CWAVES / 2;                  // consumer waves as WROWS x 2
  constexpr int WM = BM / WROWS, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;          // 32 x 32 MFMA tiles per wave
  constexpr int A_IT = BM * (PBK / 8) / kGemmThreads;
  static_assert(CWAVES == 4 || CWAVES == 8, "four or eight consumer waves");
  static_assert(TM >= 1 && PSTAGES >= 1 && PSTAGES <= 4, "wave tile and load ring");
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * PBK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * PBK];
  __shared__ int s_last;
  const int M = args.M, K = args.K, N = args.N;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const bool producer = wave >= CWAVES;
  const int tid = static_cast<int>(threadIdx.x) - (producer ? CWAVES * 64 : 0);
  const int lane = tid & 63;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int step0 = blockIdx.z * args.steps_per_split;
  const int ntiles = min(args.steps_per_split, K / PBK - step0);
  const int wm = (wave >> 1) % WROWS * WM;
  const int wn = (wave & 1) * WN;
  const int r32 = lane & 31;

  f16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  if (producer) {
    struct Stage {
      h8_t a[A_IT];
      u4_t b;
      h4_t s;
    };
    const int prow = tid >> 5;
    const int b_col = n0 + 4 * (tid & 31);
    const uint32_t row_bytes = args.L.w_row;
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(args.X, static_cast<uint32_t>(M) * static_cast<uint32_t>(K) * 2u);
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(args.Wq, static_cast<uint32_t>(K / 8) * static_cast<uint32_t>(N) * 4u);
    const __amdgpu_buffer_rsrc_t rsc =
        make_rsrc(args.S, static_cast<uint32_t>(K / GROUP) * static_cast<uint32_t>(N) * 2u);
    uint32_t voff_a[A_IT];
    int a_st[A_IT];
#pragma unroll
    for (int it = 0; it < A_IT; ++it) {
      const int row = (tid >> 3) + 32 * it;
      const int gm = m0 + row;
      voff_a[it] = gm < M ? (static_cast<uint32_t>(gm) * K + (tid & 7) * 8) * 2u : kOutOfRange;
      a_st[it] = lds_unit64(row, tid & 7) * 8;
    }
    const bool b_ok = b_col < N;  // N % 4 == 0: the quad is wholly inside or outside
    const uint32_t voff_b = b_ok ? prow * row_bytes + args.L.wcol(b_col) : kOutOfRange;
    const uint32_t voff_s = b_ok ? args.L.scol(b_col) : kOutOfRange;
    int b_st[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b_st[j] = lds_unit64(4 * (tid & 31) + j, prow) * 8;
    auto load_step = [&](Stage& st, int step) {
      const uint32_t k0 = static_cast<uint32_t>((step0 + min(step, ntiles - 1)) * PBK);
#pragma unroll
      for (int it = 0; it < A_IT; ++it)
        st.a[it] = __builtin_bit_cast(
            h8_t, __builtin_amdgcn_raw_buffer_load_b128(rx, voff_a[it], k0 * 2u, 0));
      st.b = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, voff_b, (k0 / 8) * row_bytes, 0));
      st.s = __builtin_bit_cast(
          h4_t, __builtin_amdgcn_raw_buffer_load_b64(
                    rsc, voff_s, (k0 / GROUP) * args.L.s_row, 0));
    };
    auto store_step = [&](const Stage& st, int buf) {
#pragma unroll
      for (int it = 0; it < A_IT; ++it) *reinterpret_cast<h8_t*>(&As[buf][a_st[it]]) = st.a[it];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h2_t w[4];
        const h2_t s2 = {st.s[j], st.s[j]};
        decode8_scaled(st.b[j], s2, w);
        const h8_t v = {w[0][0], w[0][1], w[1][0], w[1][1], w[2][0], w[2][1], w[3][0], w[3][1]};
        *reinterpret_cast<h8_t*>(&Bs[buf][b_st[j]]) = v;
      }
    };
    // Ring of PSTAGES register stages: stage u holds step i while
    // i % PSTAGES == u (each index is a compile-time constant).
    Stage R[PSTAGES];
#pragma unroll
    for (int i = 0; i < PSTAGES; ++i) load_step(R[i], i);
    auto piter = [&](auto u_const, int i) {
      constexpr int u = decltype(u_const)::value;
      store_step(R[u], i & 1);
      load_step(R[u], i + PSTAGES);
      __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, (PSTAGES > 1 ? 1 : 0)>;
    using I2 = std::integral_constant<int, (PSTAGES > 2 ? 2 : 0)>;
    using I3 = std::integral_constant<int, (PSTAGES > 3 ? 3 : 0)>;
    int i = 0;
    for (; i + PSTAGES <= ntiles; i += PSTAGES) {
      piter(I0{}, i);
      if constexpr (PSTAGES > 1) piter(I1{}, i + 1);
      if constexpr (PSTAGES > 2) piter(I2{}, i + 2);
      if constexpr (PSTAGES > 3) piter(I3{}, i + 3);
    }
    const int rem = ntiles - i;  // < PSTAGES
    if constexpr (PSTAGES > 1) {
      if (rem > 0) piter(I0{}, i);
    }
    if constexpr (PSTAGES > 2) {
      if (rem > 1) piter(I1{}, i + 1);
    }
    if constexpr (PSTAGES > 3) {
      if (rem > 2) piter(I2{}, i + 2);
    }
    __syncthreads();
  } else {
    int rda[TM][PBK / 16], rdb[TN][PBK / 16];
#pragma unroll
    for (int ks = 0; ks < PBK / 16; ++ks) {
#pragma unroll
      for (int i = 0; i < TM; ++i) rda[i][ks] = lds_unit64(wm + 32 * i + r32, 2 * ks + (lane >> 5)) * 8;
#pragma unroll
      for (int j = 0; j < TN; ++j) rdb[j][ks] = lds_unit64(wn + 32 * j + r32, 2 * ks + (lane >> 5)) * 8;
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
      const int buf = t & 1;
#pragma unroll
      for (int ks = 0; ks < PBK / 16; ++ks) {
        h8_t a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const h8_t*>(&As[buf][rda[i][ks]]);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = *reinterpret_cast<const h8_t*>(&Bs[buf][rdb[j][ks]]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
      }
      __syncthreads();
    }
  }
  // The twelve-wave form is planned without a K split.
  pc_epilogue<TM, TN, THREADS, BM, BN, CWAVES == 4>(acc, args, producer, m0 + wm, n0 + wn, s_last);
}

template <int BM>
hipError_t launch_pc64(const TileArgs& a, int64_t G, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(ceil_div(a.N, 128)), static_cast<unsigned>(ceil_div(a.M, BM)),
            static_cast<unsigned>(a.splits));
  if (G == 128)
    gemm_pc64_kernel<BM, 128><<<grid, 2 * kGemmThreads, 0, stream>>>(a);
  else
    gemm_pc64_kernel<BM, 64><<<grid, 2 * kGemmThreads, 0, stream>>>(a);
  return hipGetLastError();
}

// 256-row tiles, eight consumer waves; never split over K.
hipError_t launch_pc256(const TileArgs& a, int64_t G, hipStream_t stream) {
  if (a.splits != 1) return hipErrorInvalidValue;
  dim3 grid(static_cast<unsigned>(ceil_div(a.N, 128)), static_cast<unsigned>(ceil_div(a.M, 256)), 1);
  if (G == 128)
    gemm_pc64_kernel<256, 128, 8, 2><<<grid, 12 * 64, 0, stream>>>(a);
  else
    gemm_pc64_kernel<256, 64, 8, 2><<<grid, 12 * 64, 0, stream>>>(a);
  return hipGetLastError();
}

// Large-tile form for big batches: 256 x 256 output tiles, four waves (one
// per SIMD), each wave a (BM/2) x (BN/2) block of 32 x 32 MFMA tiles held in
// registers (256 accumulators per lane).  Every wave loads, decodes, stores
// and multiplies, like the tile kernel, but an operand read from LDS now
// feeds four MFMAs instead of two, halving the LDS traffic per FLOP of the
// 128 x 128 producer/consumer kernel.  64-k steps, LDS double buffered
// (2 x 64 KiB), global loads two steps ahead in registers, one barrier per
// step.  The template also builds 256 x 128 and 128 x 256 tiles; measured on
// MI355X they lost to the 128 x 128 producer/consumer kernel wherever they
// were the largest tile to fill the chip (14336 x 4096, M = 2048: 267 and
// 250 us against 242 us), so the planner does not use them.
//
// Loads per thread and step: BM / 32 16-byte A chunks (rows tid / 8 + 32 it,
// unit tid % 8) and BN / 128 dwordx4 of packed B (columns 4 q .. 4 q + 3,
// q = tid % (BN / 4), packed rows tid / (BN / 4) apart by 256 / (BN / 4))
// with their four scales.
template <int BM, int BN, int GROUP>
__global__ __launch_bounds__(kGemmThreads) void gemm_big_kernel(TileArgs args) {
  constexpr int PBK = 64;
  constexpr int TM = BM / 64, TN = BN / 64;                   // 32 x 32 tiles per wave
  constexpr int A_IT = BM * (PBK / 8) / kGemmThreads;          // 16-byte A chunks per thread
  constexpr int QUADS = BN / 4;                                // column quads per packed row
  constexpr int B_IT = (PBK / 8) * QUADS / kGemmThreads;       // packed quads per thread
  constexpr int PR_STEP = kGemmThreads / QUADS;                // packed rows apart
  static_assert(GROUP % PBK == 0, "one scale per column per step");
  static_assert(B_IT >= 1 && A_IT >= 1, "tile too small for the loaders");
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * PBK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * PBK];
  __shared__ int s_last;
  const int M = args.M, K = args.K, N = args.N;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int step0 = blockIdx.z * args.steps_per_split;
  const int ntiles = min(args.steps_per_split, K / PBK - step0);
  const int wm = (wave >> 1) * (BM / 2);
  const int wn = (wave & 1) * (BN / 2);
  const int r32 = lane & 31;

  struct Stage {
    h8_t a[A_IT];
    u4_t b[B_IT];
    h4_t s;
  };
  const uint32_t row_bytes = args.L.w_row;
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(args.X, static_cast<uint32_t>(M) * static_cast<uint32_t>(K) * 2u);
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(args.Wq, static_cast<uint32_t>(K / 8) * static_cast<uint32_t>(N) * 4u);
  const __amdgpu_buffer_rsrc_t rsc =
      make_rsrc(args.S, static_cast<uint32_t>(K / GROUP) * static_cast<uint32_t>(N) * 2u);
  uint32_t voff_a[A_IT];
  int a_st[A_IT];
#pragma unroll
  for (int it = 0; it < A_IT; ++it) {
    const int row = (tid >> 3) + 32 * it;
    const int gm = m0 + row;
    voff_a[it] = gm < M ? (static_cast<uint32_t>(gm) * K + (tid & 7) * 8) * 2u : kOutOfRange;
    a_st[it] = lds_unit64(row, tid & 7) * 8;
  }
  const int quad = tid % QUADS;
  const int b_col = n0 + 4 * quad;
  const bool b_ok = b_col < N;  // N % 4 == 0: the quad is wholly inside or outside
  uint32_t voff_b[B_IT];
  int b_st[B_IT][4];
#pragma unroll
  for (int it = 0; it < B_IT; ++it) {
    const int pr = tid / QUADS + PR_STEP * it;
    voff_b[it] = b_ok ? pr * row_bytes + args.L.wcol(b_col) : kOutOfRange;
#pragma unroll
    for (int j = 0; j < 4; ++j) b_st[it][j] = lds_unit64(4 * quad + j, pr) * 8;
  }
  const uint32_t voff_s = b_ok ? args.L.scol(b_col) : kOutOfRange;

  auto load_step = [&](Stage& st, int step) {
    const uint32_t k0 = static_cast<uint32_t>((step0 + min(step, ntiles - 1)) * PBK);
#pragma unroll
    for (int it = 0; it < A_IT; ++it)
      st.a[it] = __builtin_bit_cast(
          h8_t, __builtin_amdgcn_raw_buffer_load_b128(rx, voff_a[it], k0 * 2u, 0));
#pragma unroll
    for (int it = 0; it < B_IT; ++it)
      st.b[it] = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, voff_b[it], (k0 / 8) * row_bytes, 0));
    st.s = __builtin_bit_cast(
        h4_t, __builtin_amdgcn_raw_buffer_load_b64(
                  rsc, voff_s, (k0 / GROUP) * args.L.s_row, 0));
  };
  auto store_step = [&](const Stage& st, int buf) {
#pragma unroll
    for (int it = 0; it < A_IT; ++it) *reinterpret_cast<h8_t*>(&As[buf][a_st[it]]) = st.a[it];
#pragma unroll
    for (int it = 0; it < B_IT; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h2_t w[4];
        const h2_t s2 = {st.s[j], st.s[j]};
        decode8_scaled(st.b[it][j], s2, w);
        const h8_t v = {w[0][0], w[0][1], w[1][0], w[1][1], w[2][0], w[2][1], w[3][0], w[3][1]};
        *reinterpret_cast<h8_t*>(&Bs[buf][b_st[it][j]]) = v;
      }
  };

  f16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  int rda[TM][PBK / 16], rdb[TN][PBK / 16];
#pragma unroll
  for (int ks = 0; ks < PBK / 16; ++ks) {
#pragma unroll
    for (int i = 0; i < TM; ++i) rda[i][ks] = lds_unit64(wm + 32 * i + r32, 2 * ks + (lane >> 5)) * 8;
#pragma unroll
    for (int j = 0; j < TN; ++j) rdb[j][ks] = lds_unit64(wn + 32 * j + r32, 2 * ks + (lane >> 5)) * 8;
  }
  auto compute_step = [&](int buf) {
    h8_t a[2][TM], b[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[0][i] = *reinterpret_cast<const h8_t*>(&As[buf][rda[i][0]]);
#pragma unroll
    for (int j = 0; j < TN; ++j) b[0][j] = *reinterpret_cast<const h8_t*>(&Bs[buf][rdb[j][0]]);
#pragma unroll
    for (int ks = 0; ks < PBK / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < PBK / 16) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          a[cur ^ 1][i] = *reinterpret_cast<const h8_t*>(&As[buf][rda[i][ks + 1]]);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          b[cur ^ 1][j] = *reinterpret_cast<const h8_t*>(&Bs[buf][rdb[j][ks + 1]]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(a[cur][i], b[cur][j], acc[i][j]);
    }
  };

  Stage R0, R1;
  load_step(R0, 0);
  load_step(R1, 1);
  store_step(R0, 0);
  load_step(R0, 2);
  __syncthreads();
  int t = 0;
  for (; t + 2 <= ntiles; t += 2) {
    compute_step(0);
    store_step(R1, 1);
    load_step(R1, t + 3);
    __syncthreads();
    compute_step(1);
    store_step(R0, 0);
    load_step(R0, t + 4);
    __syncthreads();
  }
  if (t < ntiles) {
    compute_step(0);
    __syncthreads();
  }
  pc_epilogue<TM, TN, kGemmThreads, BM, BN, false>(acc, args, false, m0 + wm, n0 + wn, s_last);
}

template <int BM, int BN>
hipError_t launch_big(const TileArgs& a, int64_t G, hipStream_t stream) {
  if (a.splits != 1) return hipErrorInvalidValue;  // the kernel sums all of K
  dim3 grid(static_cast<unsigned>(ceil_div(a.N, BN)), static_cast<unsigned>(ceil_div(a.M, BM)),
            static_cast<unsigned>(a.splits));
  if (G == 128)
    gemm_big_kernel<BM, BN, 128><<<grid, kGemmThreads, 0, stream>>>(a);
  else
    gemm_big_kernel<BM, BN, 64><<<grid, kGemmThreads, 0, stream>>>(a);
  return hipGetLastError();
}


template <int BM, int BN>
hipError_t launch_tile(const TileArgs& a, int64_t G, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(ceil_div(a.N, BN)), static_cast<unsigned>(ceil_div(a.M, BM)),
            static_cast<unsigned>(a.splits));
  if (G == 128)
    gemm_tile_kernel<BM, BN, 128><<<grid, kGemmThreads, 0, stream>>>(a);
  else
    gemm_tile_kernel<BM, BN, 64><<<grid, kGemmThreads, 0, stream>>>(a);
  return hipGetLastError();
}

struct TileChoice {
  int bm, bn;
  bool pc = false;   // the producer/consumer kernel (BN = 128, 64-k steps)
  bool big = false;  // the 256 x 256 large-tile kernel (64-k steps)
};

// Batches from this many rows up may run the twelve-wave producer/consumer
// kernel (256 x 128 tiles, version 6).
constexpr int64_t kPc256MinM = 2048;

// The device the plans are made for: MI355X, 256 CUs.  Planning with a fixed
// count keeps the workspace query pure host code and equal to the launch.
constexpr int kPlanCUs = 256;

// A grid of one-workgroup-per-CU tiles that fills whole rounds of the CUs,
// the last at least 7/8 full.
bool whole_rounds(int64_t tiles) {
  const int64_t last = tiles % kPlanCUs;
  return tiles >= kPlanCUs && (last == 0 || 8 * last >= 7 * kPlanCUs);
}

// Batches from this many rows up may run the large-tile kernel (version 6).
constexpr int64_t kBigMinM = 1024;

// The widest B vector aligned operands of this N allow (the plan the
// workspace query assumes).
int nominal_bn_max(int64_t N) { return N % 4 == 0 ? 256 : N % 2 == 0 ? 128 : 64; }

// k per pipeline step of the kernel a choice runs.
int step_k(TileChoice t) { return t.pc || t.big ? 64 : BK; }

// Widest B vector (BN / 64 packed words per thread) the operands allow.
int max_bn(int64_t N, const void* w, const void* s) {
  if (N % 4 == 0 && aligned(w, 16) && aligned(s, 8)) return 256;
  if (N % 2 == 0 && aligned(w, 8) && aligned(s, 4)) return 128;
  return 64;
}

// Tile choice of the tile kernel (the shapes the producer/consumer kernel
// does not take), measured on MI355X over M = 64..2048 at 4096 x 14336 and
// 14336 x 4096: 128 x 128 (2 waves per SIMD, so one workgroup's barrier
// wait overlaps another's MFMAs) is fastest whenever its grid gives every CU
// a workgroup; otherwise 64 x 128, whose doubled grid wins (e.g. 126 us vs
// 165 us at M = 512, 14336 x 4096).  256-wide tiles of this kernel, one
// workgroup per CU, were slower at every shape.  Narrower B vectors serve N
// not a multiple of 2 or operands without 8-byte alignment.
TileChoice choose_tile(int64_t M, int64_t N, int bn_max) {
  const int bn = std::min(128, bn_max);
  if (ceil_div(M, 128) * ceil_div(N, bn) >= kPlanCUs) return {128, bn};
  return {64, bn};
}

// Launch plan of the tile kernel.  Long reductions (K >= 8192) with few
// output tiles split K so the grid reaches two workgroups per CU, at most 4
// ways.  Measured at 14336 x 4096 (64 x 128 tiles): M = 128 from 126 us to
// 70 us (4 splits), M = 512 from 129 us to 117 us (2 splits).  At K = 4096
// every split measured slower: the partial round trip outweighs the extra
// parallelism.
struct TilePlan {
  TileChoice t;
  int splits = 1;
  int steps_per_split = 0;
  size_t counter_bytes = 0;
  size_t workspace_bytes = 0;
};

TilePlan plan_tile(int64_t M, int64_t K, int64_t N, int64_t version, int bn_max) {
  TilePlan p;
  int64_t tiles = 0;
  int splits = 1;
  // 256 x 256 tiles when the grid is one round over the CUs, at least 7/8
  // full; never split over K.  Measured on MI355X against the 128 x 128
  // producer/consumer kernel, graph replays interleaved with each other and
  // with hipBLASLt: 1024 x 4096 x 14336 (224 tiles) 128 vs 133 us,
  // 4096 x 14336 x 4096 (256 tiles) 414 vs 464 us.  Grids of several rounds
  // lost under that load: 2048 and 4096 x 4096 x 14336 (448 and 896 tiles,
  // 1.75 and 3.5 rounds) 254 vs 242 and 495 vs 474 us.  Their last round is
  // part-empty, and with one workgroup per CU no other workgroup's MFMAs
  // overlap a tile's prologue and epilogue.
  const int64_t t256 = ceil_div(M, 256) * ceil_div(N, 256);
  const bool big = version == 6 && M >= kBigMinM && K % 64 == 0 && bn_max >= 256 &&
                   8 * t256 >= 7 * kPlanCUs && t256 <= kPlanCUs;
  if (M <= kStreamMaxM && K % 64 == 0 && bn_max >= 256) {
    // Small batches that do not stream (gemm_streams): 64-row tiles of the
    // producer/consumer kernel, K split so that the grid nears one round of
    // the CUs -- the largest of 1, 2, 4, 8 ways keeping it within 320
    // workgroups.  Both versions take this plan (so they agree to the bit).
    p.t = TileChoice{64, 128, true};
    tiles = ceil_div(M, 64) * ceil_div(N, 128);
    while (splits < 8 && tiles * splits * 2 <= 320 && K / 64 >= 2 * splits) splits *= 2;
  } else if (big) {
    p.t = TileChoice{256, 256, false, true};
    tiles = t256;
  } else if (version == 6 && M >= kPc256MinM && K % 64 == 0 && bn_max >= 256 &&
             whole_rounds(ceil_div(M, 256) * ceil_div(N, 128))) {
    // 256 x 128 tiles with eight consumer waves, one workgroup per CU, where
    // their grid makes whole rounds of the CUs (the last at least 7/8 full);
    // never split over K.  Measured on MI355X against the 128 x 128 kernel
    // (graph replays interleaved with hipBLASLt): 2048 x 14336 x 4096 (256
    // tiles, one round) 232 vs 245 us; 4096 x 4096 x 14336 (1792 tiles,
    // seven rounds) 470 vs 491.  With a part-filled last round the 128 x 128
    // kernel's two workgroups per CU balance better: 2048 and 3072 x 4096 x
    // 14336 (3.5 and 5.25 rounds) 254 vs 248 and 385 vs 378, 3072 x 14336 x
    // 4096 (1.5 rounds) 405 vs 365.
    p.t = TileChoice{256, 128, true};
    tiles = ceil_div(M, 256) * ceil_div(N, 128);
  } else if (K % 64 == 0 && bn_max >= 256) {
    // The producer/consumer kernel wherever it applies (whole 64-k steps,
    // 16-byte packed-word loads).  Measured on MI355X, graph replay:
    //  * K < 8192 (no split): 128-row tiles once the launch has ~192 of them
    //    (4096 x 14336 from M = 160), 64-row tiles below;
    //  * K >= 8192: 128-row tiles, split over K by the tile count -- at
    //    14336 x 4096, M = 160 (64 tiles) 4 ways: 41 us (64-row tiles,
    //    2 ways: 58); M = 384 / 512 (96 / 128 tiles) 2 ways: 74 / 76 us
    //    (97 / 101); M = 768 / 1024 (192 / 256 tiles) unsplit; M = 1536
    //    (384 tiles, a round and a half) 2 ways: 202 us (242 unsplit);
    //    M = 2048 (512 tiles) unsplit.  The split's partials are summed by
    //    the whole last workgroup of each tile (tile_sum_splits);
    //  * 4096 <= K < 8192 with at most 160 64-row tiles: 4 ways -- 4096 x
    //    4096, M = 129 / 192 / 256 (96 / 96 / 128 tiles) 16.7 / 17.4 /
    //    19.3 us unsplit 25.0 / 25.3 / 25.0; 4096 x 6144, M = 129 / 160 /
    //    192 (144 tiles) 21.2 / 22.5 / 23.7 unsplit 25.6 / 25.3 / 25.0; at
    //    192 tiles (4096 x 6144, M = 256) unsplit is ahead, 25.5 vs 27.4.
    const int64_t t128 = ceil_div(M, 128) * ceil_div(N, 128);
    p.t = TileChoice{version == 7 || K >= 8192 || t128 >= 192 ? 128 : 64, 128, true};
    tiles = ceil_div(M, p.t.bm) * ceil_div(N, 128);
    if (K >= 8192) {
      if (tiles <= 64)
        splits = 4;
      else if (tiles <= 128)
        splits = 2;
      else if (tiles > kPlanCUs && tiles < 2 * kPlanCUs)
        splits = 2;
    } else if (p.t.bm == 64 && K >= 4096 && tiles <= 160) {
      splits = 4;
    }
  } else {
    p.t = version == 7 ? TileChoice{128, std::min(128, bn_max)} : choose_tile(M, N, bn_max);
    tiles = ceil_div(M, p.t.bm) * ceil_div(N, p.t.bn);
    if (K >= 8192 && tiles < 2 * kPlanCUs)
      splits = static_cast<int>(std::min<int64_t>(ceil_div(2 * kPlanCUs, tiles), 4));
  }
  const int steps = static_cast<int>(K / step_k(p.t));
  p.steps_per_split = static_cast<int>(ceil_div(steps, splits));
  p.splits = static_cast<int>(ceil_div(steps, p.steps_per_split));
  if (p.splits > 1) {
    p.counter_bytes = align_up(static_cast<size_t>(tiles) * 4, 256);
    p.workspace_bytes = p.counter_bytes + static_cast<size_t>(p.splits) * M * N * 4;
  }
  return p;
}

hipError_t launch_choice(TileChoice t, const TileArgs& a, int64_t G, hipStream_t stream) {
  if (t.big) {
    return launch_big<256, 256>(a, G, stream);
  }
  if (t.pc) {
    if (t.bm == 256) return launch_pc256(a, G, stream);
    return t.bm == 128 ? launch_pc64<128>(a, G, stream) : launch_pc64<64>(a, G, stream);
  }
  if (t.bm == 128 && t.bn == 128) return launch_tile<128, 128>(a, G, stream);
  if (t.bm == 64 && t.bn == 128) return launch_tile<64, 128>(a, G, stream);
  if (t.bm == 128 && t.bn == 64) return launch_tile<128, 64>(a, G, stream);
  return launch_tile<64, 64>(a, G, stream);
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
// Small batches go to the weight-streaming kernel: each pass reads every
// weight byte once and multiplies it against up to 32 rows (one or two
// 16-row MFMA tiles), where a 64/128-row tile would leave most of the device
// idle.  Measured on MI355X at K=4096, N=14336: M=16 takes 82 us through the
// tile kernel and 11 us streaming.  Above 32 rows streaming takes one pass
// per 32 rows; once those passes would move 48 MiB or more, 64-row tiles of
// the producer/consumer kernel with a K split win (plan_tile).  Measured,
// graph replay, streaming against tiles: 4096 x 14336 M = 48 / 64 / 128
// 21.0 / 23.7 / 41.9 us against 19.6 / 20.1 / 26.5; 14336 x 4096 M = 33 /
// 64 / 128 23.1 / 31.6 / 56.6 against 20.6 / 21.9 / 29.3; 8192 x 8192
// M = 33 25.0 against 19.6; 4096 x 6144 M = 128 22.0 against 19.0.  Below
// that streaming stays ahead: 4096 x 4096 M = 33..128 12.4-12.6 us against
// 12.9-14.4, 4096 x 6144 M = 64 12.7 against 14.0.
bool gemm_streams(int64_t M, int64_t K, int64_t N, int64_t G) {
  if (!(M >= 1 && M <= kStreamMaxM && K > 0 && N > 0 && N % 4 == 0 && K % G == 0)) return false;
  const int64_t pass_bytes = K * N / 2;
  return M <= 32 || K % 64 != 0 || ceil_div(M, 32) * pass_bytes < (int64_t(48) << 20) ||
         batch_block_rows(M, K, N, G) == 64;  // 33..64 rows in one 64-row block
}
}  // namespace

namespace {
// The plan a call with these arguments runs (streaming for small batches,
// tiles otherwise), assuming operands aligned for the widest loads.
void gemm_plan_bytes(int64_t M, int64_t K, int64_t N, int64_t G, int64_t version, size_t* ws,
                     size_t* counters) {
  *ws = 0;
  *counters = 0;
  if ((version != 6 && version != 7) || (G != 64 && G != 128) || M <= 0 || N <= 0 || K <= 0 ||
      K % BK != 0 || K % G != 0)
    return;
  if (gemm_streams(M, K, N, G)) {
    StreamPlan p;
    if (plan_stream(M, K, N, G, true, 0, 0, &p) != NIBBLE_OK) return;
    *ws = p.workspace_bytes;
    *counters = p.counter_bytes;
    return;
  }
  const TilePlan p = plan_tile(M, K, N, version, nominal_bn_max(N));
  *ws = p.workspace_bytes;
  *counters = p.counter_bytes;
}
}  // namespace

extern "C" size_t nibble_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                              int64_t version, void* stream) {
  (void)stream;
  size_t ws, counters;
  gemm_plan_bytes(M, K, N, group_size, version, &ws, &counters);
  return ws;
}

extern "C" int nibble_gemm_streams(int64_t M, int64_t K, int64_t N, int64_t group_size) {
  return (group_size == 64 || group_size == 128) && K % BK == 0 && gemm_streams(M, K, N, group_size)
             ? 1
             : 0;
}

extern "C" size_t nibble_gemm_counter_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                            int64_t version, void* stream) {
  (void)stream;
  size_t ws, counters;
  gemm_plan_bytes(M, K, N, group_size, version, &ws, &counters);
  return counters;
}

namespace {
// The body of nibble_gemm_w4a16 for validated operands, the weights in the
// packed layout (strip_cols 0) or the strip-major layout of that width: the
// plans depend on (M, K, N, group_size, version) and pointer alignment only,
// so both layouts run the same kernels in the same order and give the same
// bits.
int gemm_run(const void* X, int64_t M, int64_t K, int64_t N, const void* Wq, const void* S,
             int64_t group_size, int64_t version, void* Y, void* workspace,
             size_t workspace_bytes, void* stream_, int64_t strip_cols) {
  int rc = NIBBLE_OK;
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
                       "gemm (streaming) kernel launch", 0, nullptr, nullptr, 0.0f, strip_cols);
    return rc == NIBBLE_OK ? ok() : rc;
  }
  const auto* x = static_cast<const _Float16*>(X);
  auto* y = static_cast<_Float16*>(Y);
  // Version 6 picks the tile for the shape; version 7 runs 128-row tiles.
  // Every tile accumulates each output over k in the same order, so without
  // a K split the two give identical bits (as the reference's v6 and v7 do).
  const int bn_max = max_bn(N, Wq, S);
  TilePlan p = plan_tile(M, K, N, version, bn_max);
  // The kernel addresses X through a buffer resource with 32-bit offsets:
  // tall activations are run in row blocks that stay below 2^31 bytes (such
  // grids are far too large to need a K split).
  const int64_t rows_max = std::max<int64_t>(256, ((int64_t(1) << 31) - 1) / (K * 2) / 256 * 256);
  // The workspace query plans for aligned operands; when the pointers force
  // another kernel than that plan's (tiles where the query planned the
  // streaming kernel, or another tile), the call runs without a split, as do
  // row-blocked tall launches.
  const TilePlan nominal = plan_tile(M, K, N, version, nominal_bn_max(N));
  if (M > rows_max || gemm_streams(M, K, N, group_size) || p.t.pc != nominal.t.pc ||
      p.t.big != nominal.t.big || p.t.bm != nominal.t.bm || p.t.bn != nominal.t.bn)
    p.splits = 1;
  if (p.splits > 1) {
    if (workspace == nullptr || workspace_bytes < p.workspace_bytes)
      return fail(NIBBLE_ERR_WORKSPACE, "gemm needs %zu bytes of workspace, got %zu",
                  p.workspace_bytes, workspace == nullptr ? size_t(0) : workspace_bytes);
    if (!aligned(workspace, 256)) return fail(NIBBLE_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  } else {
    p.steps_per_split = static_cast<int>(K / step_k(p.t));
  }
  TileArgs a;
  a.Wq = static_cast<const uint32_t*>(Wq);
  a.S = static_cast<const _Float16*>(S);
  a.K = static_cast<int>(K);
  a.N = static_cast<int>(N);
  a.steps_per_split = p.steps_per_split;
  a.splits = p.splits;
  a.counters = p.splits > 1 ? static_cast<uint32_t*>(workspace) : nullptr;
  a.partial = p.splits > 1
                  ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.counter_bytes)
                  : nullptr;
  a.L = layout_for(K, N, group_size, strip_cols);
  hipError_t e = hipSuccess;
  for (int64_t m0 = 0; m0 < M && e == hipSuccess; m0 += rows_max) {
    a.X = x + m0 * K;
    a.Y = y + m0 * N;
    a.M = static_cast<int>(std::min(rows_max, M - m0));
    e = launch_choice(p.t, a, group_size, stream);
  }
  if (e != hipSuccess) return hip_fail(e, "gemm kernel launch");
  return ok();
}
}  // namespace

extern "C" int nibble_gemm_w4a16(const void* X, int64_t x_rows, int64_t x_cols, const void* Wq,
                                 int64_t wq_rows, int64_t wq_cols, const void* S, int64_t s_rows,
                                 int64_t s_cols, int64_t group_size, int64_t version, void* Y,
                                 void* workspace, size_t workspace_bytes, void* stream_) {
  const int rc = validate_gemm(X, x_rows, x_cols, Wq, wq_rows, wq_cols, S, s_rows, s_cols,
                               group_size, version, Y);
  if (rc != NIBBLE_OK) return rc;
  return gemm_run(X, x_rows, x_cols, wq_cols, Wq, S, group_size, version, Y, workspace,
                  workspace_bytes, stream_, 0);
}

// nibble_gemm_w4a16 for batches of 9 rows and more on strip-major weights
// (no counterpart in the reference): the same plans, kernels and bits as the
// packed call; batches of at most 8 rows take the strip-major GEMV.
extern "C" int nibble_gemm_w4a16_strip_major(const void* X, int64_t x_rows, int64_t x_cols,
                                             const void* Wt, const void* St, int64_t K, int64_t N,
                                             int64_t group_size, int64_t strip_cols,
                                             int64_t version, void* Y, void* workspace,
                                             size_t workspace_bytes, void* stream) {
  NIBBLE_CHECK(x_cols == K, "activation columns (%lld) disagree with K=%lld", (long long)x_cols,
               (long long)K);
  NIBBLE_CHECK(K > 0 && N > 0, "bad dimension (K and N must be positive)");
  NIBBLE_CHECK(group_size == 64 || group_size == 128, "group_size must be 64 or 128");
  NIBBLE_CHECK(K % group_size == 0, "K=%lld is not a multiple of group_size=%lld", (long long)K,
               (long long)group_size);
  NIBBLE_CHECK(strip_cols == 16 || strip_cols == 32 || strip_cols == 64,
               "strip_cols must be 16, 32 or 64, got %lld", (long long)strip_cols);
  NIBBLE_CHECK(N % strip_cols == 0, "N=%lld is not a multiple of strip_cols=%lld", (long long)N,
               (long long)strip_cols);
  NIBBLE_CHECK(strip_cols != 16 || group_size == 128, "16-column strips need group_size 128");
  NIBBLE_CHECK(x_rows == 0 || x_rows > 8,
               "batches of at most 8 rows take nibble_gemv_w4a16_strip_major (got M=%lld)",
               (long long)x_rows);
  NIBBLE_CHECK(Wt == nullptr || (aligned(Wt, 16) && aligned(St, 16)),
               "strip-major weights and scales must be 16-byte aligned");
  const int rc = validate_gemm(X, x_rows, x_cols, Wt, K / 8, N, St, K / group_size, N, group_size,
                               version, Y);
  if (rc != NIBBLE_OK) return rc;
  return gemm_run(X, x_rows, K, N, Wt, St, group_size, version, Y, workspace, workspace_bytes,
                  stream, strip_cols);
}
