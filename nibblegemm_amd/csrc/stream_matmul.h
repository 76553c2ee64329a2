// The weight-streaming MFMA matmul (gemv.hip) as used by both entry points:
// nibble_gemv_w4a16 (M <= 8) and nibble_gemm_w4a16 for small batches
// (M <= kStreamMaxM), where streaming the weights beats tiling: up to 32 rows
// share one pass over the weights, larger batches take one pass per 32 rows.
#pragma once

#include "nibble_common.h"

namespace nibble {

constexpr int kStreamMaxM = 128;

// Where column n's packed words and scales live, for either weight layout
// (byte offsets within the words / scales):
//   packed [K / 8, N] (the reference's format): word (r, n) at r w_row + 4 n
//     with w_row = 4 N, scale (g, n) at g s_row + 2 n with s_row = 2 N --
//     one strip (strip_shift 31);
//   strip-major of width SW = 2^strip_shift (nibble_pack_strip_major): the
//     words of strip n / SW are one run of w_strip bytes, row r of it at
//     r w_row (w_row = 4 SW), column n % SW at 4 (n % SW) within the row;
//     the scales likewise (s_strip, s_row = 2 SW).
// Every kernel reading weights computes a lane's column offset once with
// wcol / scol and steps along K by w_row / s_row, so it reads either layout
// and loads the same values from both.
struct WeightLayout {
  uint32_t strip_shift = 31;
  uint32_t w_row = 0, w_strip = 0;
  uint32_t s_row = 0, s_strip = 0;
  __host__ __device__ uint32_t wcol(uint32_t n) const {
    return (n >> strip_shift) * w_strip + (n & ((1u << strip_shift) - 1u)) * 4u;
  }
  __host__ __device__ uint32_t scol(uint32_t n) const {
    return (n >> strip_shift) * s_strip + (n & ((1u << strip_shift) - 1u)) * 2u;
  }
};

inline WeightLayout packed_layout(int64_t N) {
  WeightLayout l;
  l.strip_shift = 31;
  l.w_row = static_cast<uint32_t>(N) * 4u;
  l.s_row = static_cast<uint32_t>(N) * 2u;
  return l;
}

// SW must be 16, 32 or 64 (the caller checks).
inline WeightLayout strip_major_layout(int64_t K, int64_t N, int64_t G, int64_t SW) {
  (void)N;
  WeightLayout l;
  l.strip_shift = SW == 16 ? 4u : SW == 32 ? 5u : 6u;
  l.w_row = static_cast<uint32_t>(SW) * 4u;
  l.w_strip = static_cast<uint32_t>(K / 8 * SW * 4);
  l.s_row = static_cast<uint32_t>(SW) * 2u;
  l.s_strip = static_cast<uint32_t>(K / G * SW * 2);
  return l;
}

// The layout of a call: packed when strip_cols is 0, else strip-major.
inline WeightLayout layout_for(int64_t K, int64_t N, int64_t G, int64_t strip_cols) {
  return strip_cols > 0 ? strip_major_layout(K, N, G, strip_cols) : packed_layout(N);
}

// Two kernels serve the plan.  kSplitKernel: 64-column strips, K split
// across workgroups when a wave would stream too many groups, partials
// reduced by the last workgroup of a strip (any M up to kStreamMaxM).
// kStripKernel (M <= 8): `strip_cols`-column strips over the whole of K,
// `waves` waves per workgroup on contiguous group ranges with `depth` groups
// of loads in flight per wave; no workspace.
// kBatchKernel (one block of 12..64 rows): the split kernel's geometry and
// arithmetic (so its bits), with each step's activation window copied once
// into an LDS ring by staging waves and `depth` steps of weight loads in
// flight per wave.
constexpr int kSplitKernel = 0;
constexpr int kStripKernel = 1;
constexpr int kBatchKernel = 2;

// Launch geometry.  The split-K workspace (split kernel, splits > 1) is
// `counter_bytes` of uint32 counters, one per (row block, strip), zero on
// entry and left zero, followed by fp32 partials [splits, M, N];
// `workspace_bytes` is the total.
struct StreamPlan {
  int kernel = kSplitKernel;
  int mt = 1;      // compiled row count: 1, 2, 4, 8, 16 or 32 (64: batch kernel)
  int mblocks = 1; // blocks of mt rows (grid.z); more than one only above 32 rows
  int waves = 4;   // wave64s per workgroup
  int strips = 0;  // column strips (grid.x for the split kernel)
  int splits = 1;  // K splits (grid.y)
  int groups_per_split = 0;
  int strip_cols = 64;  // strip kernel: 16, 32 or 64
  int depth = 2;        // strip / batch kernel: groups (steps) of weight loads in flight per wave
  int ring = 3;         // batch kernel: LDS activation slots
  int pair = 1;         // batch kernel: adjacent strips per workgroup (1 or 2)
  bool stage_x = true;  // strip kernel: activations copied to LDS (when they fit 64 KiB)
  size_t counter_bytes = 0;
  size_t workspace_bytes = 0;
};

// What a launch asks of the kernel besides the matmul: the output epilogue
// (0 none, 1 bias, 2 SwiGLU) and whether the RMSNorm prologue is fused.
struct StreamFusion {
  int epilogue = 0;
  bool norm = false;
};

// Pure host arithmetic.  split_k = false forces one split of the split
// kernel (gemv versions 2 and 3); splits_override / threads_override of 0
// mean "heuristic", and only the heuristic path may choose the strip kernel.
int plan_stream(int64_t M, int64_t K, int64_t N, int64_t G, bool split_k, int64_t splits_override,
                int64_t threads_override, StreamPlan* p, StreamFusion fusion = StreamFusion());

// The strip kernel's plan for these operands, if it serves them (M <= 8,
// and the fusion it supports); returns false otherwise.  Pure host arithmetic.
bool plan_strip(int64_t M, int64_t K, int64_t N, int64_t G, StreamFusion fusion, StreamPlan* p);

// Rows of the one block the batch kernel takes these operands in (16, 32 or
// 64), or 0 when the plan is another kernel's: 12..16 rows outside the strip
// kernel's plans, 17..32 rows, and 33..64 rows where the 64-row block's grid
// fills the CUs in one round.  Pure host arithmetic.
int batch_block_rows(int64_t M, int64_t K, int64_t N, int64_t G);

// Whether the streaming kernel can take these operands: N a multiple of 4,
// 16-byte X and Wq, 8-byte S and Y, offsets within 31 bits.
bool stream_supported(const void* X, const void* Wq, const void* S, const void* Y, int64_t M,
                      int64_t K, int64_t N, int64_t G);

// Checks the workspace against the plan and launches on `stream` (whose
// device must be current).  `epilogue` 0 writes X W; 1 adds `bias` ([N]
// fp16) in fp16; 2 reads W as gate|up interleaved in 32-column blocks and
// writes silu(gate) * up ([M, N/2]).  A non-null `norm_w` ([K] fp16)
// multiplies by the RMSNorm rows of X instead of X (M <= 8, K <= 16384, the
// default 4-wave plan).  Returns a NIBBLE_* status.
int launch_stream(const void* X, const void* Wq, const void* S, void* Y, int64_t M, int64_t K,
                  int64_t N, int64_t G, const StreamPlan& p, void* workspace,
                  size_t workspace_bytes, hipStream_t stream, const char* who, int epilogue = 0,
                  const void* bias = nullptr, const void* norm_w = nullptr,
                  float norm_eps = 0.0f, int64_t strip_cols = 0);

// launch_stream with the split-K workspace given as its two parts: the
// counter region (zero on entry, left zero) and the fp32 partials.  The plan
// must fit whatever those point at; no checks are made here.  A non-zero
// `strip_cols` reads Wq and S in the strip-major layout of that width (any
// plan; the plan's geometry, and so the bits, are the packed layout's).
int launch_stream_split(const void* X, const void* Wq, const void* S, void* Y, int64_t M,
                        int64_t K, int64_t N, int64_t G, const StreamPlan& p, void* counters,
                        void* partials, hipStream_t stream, const char* who, int epilogue = 0,
                        const void* bias = nullptr, const void* norm_w = nullptr,
                        float norm_eps = 0.0f, int64_t strip_cols = 0);

// Strip width recommended for strip-major weights of this shape (0: none
// fits), and the strip kernel's plan for a strip-major weight of width SW.
// Pure host arithmetic.
int64_t strip_major_cols(int64_t K, int64_t N, int64_t G);
bool plan_strip_major(int64_t M, int64_t K, int64_t N, int64_t G, int64_t SW, StreamPlan* p);

// Largest K the fused-RMSNorm prologue takes (8 chunks of 256 x 8 columns).
constexpr int kNormMaxK = 16384;
constexpr int kNormMaxM = 8;

}  // namespace nibble
