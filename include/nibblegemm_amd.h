/*
 * nibblegemm_amd.h -- C ABI of the MI355X (gfx950) W4A16 kernel library.
 *
 * This is the drop-in boundary.  It replaces the reference's pybind11 module
 * `nibblegemm_cuda` (csrc/bindings.cpp:11-22 in arvindcr4/nibblegemm), whose
 * three functions took and returned torch tensors.  Here every entry point takes
 * plain device pointers, shapes and a HIP stream, and returns a status code:
 *
 *   nibble_gemv_w4a16   <- gemv_w4a16(X, Wq, S, group_size, version=4,
 *                                     splits_override=0, threads_override=0)
 *                          csrc/bindings.cpp:12-15, csrc/gemv_w4a16.cu:341-425
 *   nibble_gemm_w4a16   <- gemm_w4a16(X, Wq, S, group_size, version=6)
 *                          csrc/bindings.cpp:16-19, csrc/gemm_w4a16.cu:379-429
 *   nibble_dequant_w4   <- dequant_w4(Wq, S, group_size, fast=True)
 *                          csrc/bindings.cpp:20-21, csrc/dequant_kernel.cu:48-74
 *
 * Tensor-shape arguments are passed as the reference's tensors would report
 * them (rows and columns of X, Wq and S), so the library can apply exactly the
 * reference's host checks (csrc/gemv_w4a16.cu:251-265, csrc/gemm_w4a16.cu:
 * 381-400, csrc/dequant_kernel.cu:49-52) before any HIP call.  dtype, device
 * and contiguity are properties of tensors, not of pointers; the caller checks
 * those (the Python layer in nibblegemm_amd/ops.py does).
 *
 * Data layout (all row-major, contiguous):
 *   X   fp16  [M, K]        activations
 *   Wq  int32 [K/8, N]      packed nibbles, slot order {0,4,1,5,2,6,3,7} along K,
 *                           stored value = q + 8 (implicit zero-point 8)
 *   S   fp16  [K/G, N]      one scale per group of G rows along K
 *   Y   fp16  [M, N]        output (caller-allocated)
 *   W   fp16  [K, N]        dequant output (caller-allocated)
 *
 * Ownership: inputs are borrowed; outputs and workspace are caller-allocated
 * (the reference allocated them inside the call, gemv_w4a16.cu:350, :403-408).
 * The library allocates no device memory and keeps no mutable global state
 * beyond per-device attribute caches, so calls on different streams and
 * threads are independent -- except that calls sharing one workspace must be
 * ordered on one stream.
 *
 * Errors: a non-zero status.  nibble_last_error() returns this thread's message
 * for the most recent failing call (the reference raised c10::Error, seen in
 * Python as RuntimeError).  Validation failures never touch the GPU.
 */
#ifndef NIBBLEGEMM_AMD_H_
#define NIBBLEGEMM_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NIBBLE_ABI_VERSION 14

#if defined(__GNUC__) || defined(__clang__)
#define NIBBLE_API __attribute__((visibility("default")))
#else
#define NIBBLE_API
#endif

enum {
  NIBBLE_OK = 0,
  NIBBLE_ERR_INVALID_ARGUMENT = 1, /* a reference TORCH_CHECK would have fired */
  NIBBLE_ERR_UNSUPPORTED = 2,      /* valid request this kernel does not serve (e.g. gemv M > 8) */
  NIBBLE_ERR_WORKSPACE = 3,        /* workspace missing, too small or misaligned */
  NIBBLE_ERR_HIP = 4               /* a HIP runtime call or kernel launch failed */
};

/* Version of this header the library was built from (NIBBLE_ABI_VERSION). */
NIBBLE_API int nibble_abi_version(void);

/* Message for the last failing call on the calling thread ("" if none). */
NIBBLE_API const char* nibble_last_error(void);

/*
 * Decode-regime matmul Y = X @ dequant(Wq, S), M <= 8 for versions 3 and 4.
 *
 * version           0 = scalar fp32 reference kernel (one thread per output);
 *                   1 = scalar decode, packed word reused for its 8 k;
 *                   2, 3 = the streaming kernel with one K split;
 *                   4 = the streaming kernel with split-K (default).
 * splits_override   0 = heuristic; else the number of K splits (version 4).
 * threads_override  0 = heuristic; else workgroup size in {32,64,128,256,512,1024}
 *                   (32, which the reference accepts, runs as one 64-lane wave).
 * workspace         version 4 with more than one K split (K above 8192, or an
 *                   explicit splits_override / threads_override) needs
 *                   nibble_gemv_workspace_bytes(...) bytes, 256-byte aligned.
 *                   Its first nibble_gemv_counter_bytes(...) bytes must be zero
 *                   before the first call; every call leaves them zero again.
 *                   May be NULL when the query returns 0.
 * stream            hipStream_t (NULL = the null stream of the current device).
 */
NIBBLE_API int nibble_gemv_w4a16(const void* X, int64_t x_rows, int64_t x_cols,
                      const void* Wq, int64_t wq_rows, int64_t wq_cols,
                      const void* S, int64_t s_rows, int64_t s_cols,
                      int64_t group_size, int64_t version, int64_t splits_override,
                      int64_t threads_override, void* Y, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * nibble_gemv_w4a16 that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Arguments, results and errors are nibble_gemv_w4a16's.  When
 * the plan splits K across workgroups, the split counters and partials live
 * in a static device array of the library (4 MiB per GPU, held until the
 * process ends: 64 KiB of counters, zeroed when a GPU first uses it, then the
 * fp32 partials [splits, M, N]); a request needing more than that fails with
 * NIBBLE_ERR_UNSUPPORTED before anything is launched.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams or
 * threads) race and must be serialised by the caller.  The first split-K
 * call on a GPU clears the counters and waits for that to finish, so it
 * cannot itself be captured into a graph: under capture it fails with
 * NIBBLE_ERR_UNSUPPORTED (make one such call before capturing).
 */
NIBBLE_API int nibble_gemv_w4a16_noalloc(const void* X, int64_t x_rows, int64_t x_cols,
                      const void* Wq, int64_t wq_rows, int64_t wq_cols,
                      const void* S, int64_t s_rows, int64_t s_cols,
                      int64_t group_size, int64_t version, int64_t splits_override,
                      int64_t threads_override, void* Y, void* stream);

/* Bytes of workspace nibble_gemv_w4a16 needs for these arguments (0 if none,
 * and 0 for arguments the launcher would reject).  Pure host computation:
 * `stream` is accepted for symmetry with the launcher and is not used. */
NIBBLE_API size_t nibble_gemv_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                   int64_t version, int64_t splits_override,
                                   int64_t threads_override, void* stream);

/* Leading bytes of that workspace that must be zero on entry (split counters). */
NIBBLE_API size_t nibble_gemv_counter_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                 int64_t version, int64_t splits_override,
                                 int64_t threads_override, void* stream);

/*
 * Diagnostics; no counterpart in the reference (which has no in-kernel
 * timing).  While `stamps` is non-NULL, every launch of this host thread that
 * runs the strip kernel at M = 1 without the RMSNorm prologue (the decode
 * GEMV, whichever entry point plans it) writes its timeline into `stamps` (device memory, `bytes` long, 8-byte
 * aligned): per wave w of workgroup b, 8 uint64 at index (b * waves + w) * 8
 * -- s_memrealtime ticks (100 MHz) at kernel entry, after the prologue's
 * loads are issued, after the activation/scale copies have landed (workgroup
 * barrier), after the first quant group is computed, after the last, after
 * the partials are in LDS, after this wave's output stores are acknowledged
 * -- then (b << 40) | (w << 36) | (XCC_ID << 32) | HW_ID.  Such a launch
 * needs grid * waves * 64 bytes (grid = 8 * ceil(strips / 8)); a smaller
 * buffer makes it fail with NIBBLE_ERR_INVALID_ARGUMENT before anything is
 * launched.  NULL turns it off.  Other launches are unchanged; the outputs
 * are the same bits either way.
 */
NIBBLE_API int nibble_gemv_timeline(void* stamps, int64_t bytes);

/*
 * Prefill-regime matmul on CDNA4 MFMA (any M >= 1).  version 6 (default) or 7
 * (alternate tile shape; same numerics).  Requires K % 32 == 0, N even,
 * group_size in {64, 128} and M*N, M*K, K*N < 2^31 (the reference's checks).
 * Batches of M <= 128 (with N % 4 == 0) run the weight-streaming kernel of
 * the GEMV, larger ones the tile kernel; either may split K across
 * workgroups.  `workspace` follows the same rules as for nibble_gemv_w4a16,
 * sized by nibble_gemm_workspace_bytes(...) (NULL allowed when that is 0).
 */
NIBBLE_API int nibble_gemm_w4a16(const void* X, int64_t x_rows, int64_t x_cols,
                      const void* Wq, int64_t wq_rows, int64_t wq_cols,
                      const void* S, int64_t s_rows, int64_t s_cols,
                      int64_t group_size, int64_t version, void* Y,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Workspace nibble_gemm_w4a16 needs (0 if none) and its leading zeroed
 * counter bytes.  Pure host computation; `stream` is not used. */
NIBBLE_API size_t nibble_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                   int64_t version, void* stream);
NIBBLE_API size_t nibble_gemm_counter_bytes(int64_t M, int64_t K, int64_t N, int64_t group_size,
                                 int64_t version, void* stream);
/* 1 when nibble_gemm_w4a16 runs these sizes on the streaming kernel (given
 * operands aligned as nibble_matmul_w4a16_fused requires), so that its result
 * has the bits of nibble_matmul_w4a16_fused's epilogue 0; 0 when it takes
 * tiles.  No counterpart in the reference, whose gemm_w4a16 has one kernel.
 * Callers that compose a bias or activation themselves use it to choose
 * between the fused entry and nibble_gemm_w4a16 + separate ops with the same
 * bits either way. */
NIBBLE_API int nibble_gemm_streams(int64_t M, int64_t K, int64_t N, int64_t group_size);

/*
 * Streaming matmul (1 <= M <= 128) with a fused output epilogue.  No
 * counterpart in the reference: its QuantLinear adds the bias as a separate
 * fp16 op (python/nibblegemm/ops.py:131-135), and gate/up activations run as
 * separate ops after the matmul.  For callers that want one launch per
 * layer projection (decode steps, HIP graphs):
 *   epilogue 0  Y [M, N] = X @ W, as nibble_gemm_w4a16 writes it where
 *               nibble_gemm_streams(M, K, N, group_size) is 1 (within
 *               tolerance of it elsewhere: different split sums);
 *   epilogue 1  Y [M, N] = fp16(fp16(X @ W) + bias), bias fp16 [N] -- the
 *               same bits as the separate fp16 add;
 *   epilogue 2  W is [gate | up] interleaved in 16-column blocks (N a
 *               multiple of 32, nibblegemm_amd.quant.interleave_swiglu);
 *               Y [M, N/2] = silu(G) * U with G, U and silu(G) rounded to
 *               fp16 as the unfused fp16 ops would.
 * A non-null `norm_weight` (fp16 [K], 16-byte aligned) fuses an RMSNorm
 * prologue: the product is taken with fp16(x * r * norm_weight) per row of X,
 * r = 1 / sqrt(mean(x^2) + norm_eps) -- the same bits as nibble_rmsnorm_f16
 * followed by this call without it.  It needs M <= 8, K <= 16384 and the
 * normalised row block (M rounded up to 1, 2, 4 or 8 rows, times K fp16)
 * within 64 KiB.
 * Requires N % 4 == 0, group_size in {64, 128}, X and Wq 16-byte and S, Y
 * 8-byte aligned (NIBBLE_ERR_INVALID_ARGUMENT otherwise; there is no other
 * kernel to fall back to).  `workspace` as for nibble_gemv_w4a16, sized by
 * nibble_matmul_fused_workspace_bytes(...).
 */
NIBBLE_API int nibble_matmul_w4a16_fused(const void* X, int64_t x_rows, int64_t x_cols,
                      const void* Wq, int64_t wq_rows, int64_t wq_cols,
                      const void* S, int64_t s_rows, int64_t s_cols,
                      int64_t group_size, int64_t epilogue, const void* bias,
                      const void* norm_weight, float norm_eps, void* Y,
                      void* workspace, size_t workspace_bytes, void* stream);
NIBBLE_API size_t nibble_matmul_fused_workspace_bytes(int64_t M, int64_t K, int64_t N,
                                           int64_t group_size, void* stream);
NIBBLE_API size_t nibble_matmul_fused_counter_bytes(int64_t M, int64_t K, int64_t N,
                                         int64_t group_size, void* stream);

/*
 * Strip-major weights for the decode GEMV (M <= 8).  No counterpart in the
 * reference, which keeps only the packed layout above (python/nibblegemm/
 * quant.py:28-50); this is an MI355X layout for decode-bound callers that can
 * hold a second copy of a weight (or convert once at load).  The N columns
 * are cut into strips of `strip_cols` (16, 32 or 64; 16 needs group_size 128)
 * and each strip is stored whole, so one workgroup of the decode kernel
 * streams one contiguous run:
 *   Wt  int32 [N/strip_cols, K/8, strip_cols]   Wt[s][r][j] = Wq[r][s*strip_cols + j]
 *   St  fp16  [N/strip_cols, K/G, strip_cols]   St[s][g][j] = S[g][s*strip_cols + j]
 * Same bytes as Wq and S; the nibble format within a word is unchanged.
 *
 * nibble_strip_major_cols: the strip width this library measures fastest for
 * a [K, N] weight (0 when none fits: N not a multiple of 16, or of 32 with
 * group_size 64).  Pure host computation.
 *
 * nibble_pack_strip_major: writes Wt and St from Wq and S on `stream` (an
 * exact permutation).  Wq, S, Wt, St 16-byte aligned; the outputs must not
 * overlap the inputs.
 *
 * nibble_gemv_w4a16_strip_major: Y = X @ dequant(W) for M = x_rows <= 8 from
 * Wt and St packed with this `strip_cols`, with nibble_matmul_w4a16_fused's
 * epilogue (0 none, 1 fp16 bias, 2 SwiGLU of a gate|up interleaved weight,
 * strip_cols >= 32) and optional RMSNorm prologue (same arithmetic and
 * limits).  No workspace.  The result agrees with nibble_gemv_w4a16 on the
 * packed weight within fp32 summation order (the two may sum in a different
 * order); it is deterministic.
 */
NIBBLE_API int64_t nibble_strip_major_cols(int64_t K, int64_t N, int64_t group_size);
NIBBLE_API int nibble_pack_strip_major(const void* Wq, int64_t wq_rows, int64_t wq_cols,
                      const void* S, int64_t s_rows, int64_t s_cols,
                      int64_t group_size, int64_t strip_cols, void* Wt, void* St,
                      void* stream);
NIBBLE_API int nibble_gemv_w4a16_strip_major(const void* X, int64_t x_rows, int64_t x_cols,
                      const void* Wt, const void* St, int64_t K, int64_t N,
                      int64_t group_size, int64_t strip_cols, int64_t epilogue,
                      const void* bias, const void* norm_weight, float norm_eps,
                      void* Y, void* stream);

/*
 * Dense fp16 W [K, N] from packed weights, bit-exact with the reference's
 * dequantize(): W[k][n] = fp16_rne((nibble - 8) * S[k / G][n]).
 * fast != 0 selects the magic-exponent decode, fast == 0 the scalar
 * shift/mask/convert decode; both give identical bits.  K = wq_rows * 8.
 */
NIBBLE_API int nibble_dequant_w4(const void* Wq, int64_t wq_rows, int64_t wq_cols,
                      const void* S, int64_t s_rows, int64_t s_cols,
                      int64_t group_size, int fast, void* W, void* stream);

/*
 * Decode-step glue.  No counterpart in the reference's extension: its model
 * decode (bench/bench_model.py:177-188, a transformers Llama with its Linear
 * layers swapped for QuantLinear, :131-154) runs these as PyTorch ops.  For
 * callers that capture a whole batch-1 decode step in one HIP graph.
 *
 * RMSNorm of each row: Y[r, :] = fp16(X[r, :] * r_r * W) with
 * r_r = 1 / sqrt(mean_c(X[r, c]^2) + eps), all in fp32.  X, Y fp16
 * [rows, cols], W fp16 [cols]; cols a multiple of 8 up to 16384; all three
 * 16-byte aligned.
 */
NIBBLE_API int nibble_rmsnorm_f16(const void* X, int64_t rows, int64_t cols, const void* W,
                                  float eps, void* Y, void* stream);

/*
 * Grouped-query attention of one decode token at position `pos`.
 * QKV fp16 [n_heads * 128 | n_kv_heads * 128 | n_kv_heads * 128] is the
 * token's q, k and v (the q|k|v projection's output row).  K_cache and
 * V_cache fp16 [n_kv_heads][max_seq][128] hold tokens 0 .. pos - 1; the call
 * writes the token's k (rotated) and v at row `pos` and returns
 * Out fp16 [n_heads * 128] = softmax(q k^T / sqrt(128)) v over tokens
 * 0 .. pos, query head i reading kv head i / (n_heads / n_kv_heads).
 * rope_cos / rope_sin fp32 [max_seq][64] (both or neither) apply the
 * rotary embedding to q and k in the rotate-half pairing; NULL skips it.
 * head_dim must be 128, n_heads / n_kv_heads 1, 2, 4 or 8, and
 * 0 <= pos < max_seq <= 65536.  Positions
 * beyond 127 split across workgroups: `workspace` (256-byte aligned, its
 * leading nibble_attention_decode_counter_bytes(...) zero before the first
 * call, restored to zero by each call) must then hold
 * nibble_attention_decode_workspace_bytes(...) bytes; NULL when that is 0.
 */
NIBBLE_API int nibble_attention_decode_f16(const void* QKV, int64_t n_heads, int64_t n_kv_heads,
                                           int64_t head_dim, void* K_cache, void* V_cache,
                                           int64_t max_seq, int64_t pos, const void* rope_cos,
                                           const void* rope_sin, void* Out, void* workspace,
                                           size_t workspace_bytes, void* stream);
NIBBLE_API size_t nibble_attention_decode_workspace_bytes(int64_t n_heads, int64_t n_kv_heads,
                                                          int64_t head_dim, int64_t max_seq,
                                                          int64_t pos, void* stream);
NIBBLE_API size_t nibble_attention_decode_counter_bytes(int64_t n_heads, int64_t n_kv_heads,
                                                        int64_t head_dim, int64_t max_seq,
                                                        int64_t pos, void* stream);

/*
 * Strip-major weights for every batch size (no counterpart in the
 * reference): nibble_gemm_w4a16 and nibble_dequant_w4 on the strip-major
 * copy (Wt, St) of a weight, so that a model can keep that one copy.
 * nibble_gemm_w4a16_strip_major takes batches of more than 8 rows (at most 8
 * take nibble_gemv_w4a16_strip_major) and runs the packed call's plans and
 * kernels, so it returns the packed call's bits and needs the same
 * workspace (nibble_gemm_workspace_bytes / nibble_gemm_counter_bytes).
 * nibble_dequant_w4_strip_major writes the packed call's [K, N] output.
 * Wt and St 16-byte aligned; strip_cols 16, 32 or 64 dividing N.
 */
NIBBLE_API int nibble_gemm_w4a16_strip_major(const void* X, int64_t x_rows, int64_t x_cols,
                                             const void* Wt, const void* St, int64_t K, int64_t N,
                                             int64_t group_size, int64_t strip_cols,
                                             int64_t version, void* Y, void* workspace,
                                             size_t workspace_bytes, void* stream);
NIBBLE_API int nibble_dequant_w4_strip_major(const void* Wt, const void* St, int64_t K, int64_t N,
                                             int64_t group_size, int64_t strip_cols, int fast,
                                             void* W, void* stream);

/*
 * Persistent decode chain: a list of strip-major decode GEMVs ("stages") run
 * by ONE launch, each stage optionally waiting for an earlier one.  No
 * counterpart in the reference, whose decode step is one launch per
 * projection (bench/bench_model.py:70-86) and whose optimisation log names
 * fewer launches as the fix for the launch-bound small projections
 * (docs/OPTIMIZATION_LOG.md:159-163).  Every output has the bits of
 * nibble_gemv_w4a16_strip_major with the same operands and epilogue.
 *
 * A stage is Y = X @ W (epilogue 0), fp16(fp16(X @ W) + bias) (1) or the
 * SwiGLU of an interleave_swiglu weight (2, strips of >= 32 columns), with
 * X [M, K] fp16 and Y [M, N] fp16 ([M, N / 2] for SwiGLU).  W is either
 * strip-major (layout 0: nibble_pack_strip_major at `strip_cols`) or the
 * packed [K/8, N] words and [K/G, N] scales of nibble_gemv_w4a16 (layout 1),
 * read as strips of `strip_cols` columns; the two give the same bits (256-
 * byte row pieces at 64 columns read as fast as contiguous strips).  No
 * counterpart in the reference for the layout choice: its decode reads the
 * packed layout, which layout 1 takes unconverted.  `after` names an earlier stage
 * (index) that must have finished before this one reads its X and bias, or
 * is -1.  Whatever a stage reads that another stage writes, and whatever two
 * stages both write, must be ordered by `after` links (directly or through a
 * chain of them); nibble_chain_create checks this, and that no stage writes
 * weights.  All stages share M (1..8) and group_size.
 */
typedef struct nibble_chain_stage {
  const void* X;
  const void* Wt;
  const void* St;
  void* Y;
  const void* bias;
  int64_t K, N, group_size, strip_cols, epilogue;
  int64_t after;
  int64_t layout;  /* 0 strip-major, 1 packed */
} nibble_chain_stage;

/* Validates the stages, plans the launch (one workgroup per CU; every
 * workgroup gets an ordered list of strips, balanced by bytes) and copies
 * the plan to the device of `stream` (allocates; not for graph capture).
 * The pointers are recorded: the buffers must outlive the chain. */
NIBBLE_API int nibble_chain_create(const nibble_chain_stage* stages, int64_t n_stages, int64_t M,
                                   void* stream, void** chain);
/* One run of every stage on `stream` (allocates nothing; graph-capturable).
 * Runs of one chain must not overlap (they share its counters).
 * `timestamps`: NULL, or n_stages + 1 uint64 the caller has set to 0 (and
 * the last to UINT64_MAX): per stage the s_memrealtime (100 MHz) tick at
 * which its last round ended, and the tick the first workgroup started. */
NIBBLE_API int nibble_chain_run(void* chain, void* timestamps, void* stream);
/* Synchronises `stream`, then reports whether a run gave up waiting for a
 * stage (bounded waits; e.g. when not every workgroup could be resident):
 * NIBBLE_ERR_HIP with a message if so (the flag is then cleared). */
NIBBLE_API int nibble_chain_check(void* chain, void* stream);
/* 0: workgroups, 1: rounds, 2: dynamic LDS bytes, 3: stages; -1 otherwise. */
NIBBLE_API int64_t nibble_chain_info(void* chain, int64_t what);
NIBBLE_API int nibble_chain_destroy(void* chain);
/* The strip width at which a chain of independent M-row stages streams a
 * [K, N] weight fastest: the widest of 64 and 32 columns for which a
 * one-stage chain of it has a plan (the LDS of the chain grows with K and
 * the strip's scales), else nibble_strip_major_cols's width; 0 when none has
 * a chain plan.  A chain round costs a fixed allowance besides its bytes, so
 * a chain of many stages wants fewer, wider strips than the per-projection
 * launches, which want a workgroup per CU (a chain of one narrow weight may
 * want more strips than this gives).  A weight converted at either width
 * serves both.  Pure host computation. */
NIBBLE_API int64_t nibble_chain_strip_cols(int64_t K, int64_t N, int64_t group_size, int64_t M);

/*
 * Measurement: a streaming read of `bytes` (a positive multiple of 16) from
 * `src` (16-byte aligned) by `workgroups` workgroups of 256 threads, each
 * folding its contiguous slice into one word of `sink` (4 bytes per
 * workgroup, nibble_read_probe_sink_bytes(...)).  The achievable HBM read
 * bandwidth the decode GEMV is compared with.  No counterpart in the
 * reference, whose harness times a device copy (bench/harness.py:189-200).
 */
NIBBLE_API int nibble_read_probe(const void* src, size_t bytes, int64_t workgroups, void* sink,
                                 void* stream);
NIBBLE_API size_t nibble_read_probe_sink_bytes(size_t bytes, int64_t workgroups);

#ifdef __cplusplus
}
#endif

#endif /* NIBBLEGEMM_AMD_H_ */
