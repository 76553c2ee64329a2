// INT4 -> fp16 decode primitives for gfx950.
//
// Packed format: one 32-bit word holds 8 consecutive k of one column.  Logical
// offset k lives in nibble slot {0,4,1,5,2,6,3,7}[k] (even k in slots 0..3, odd
// k in slots 4..7; python/nibblegemm/quant.py:28-50 in the reference), and the
// stored value is q + 8.
//
// Fast decode (the fp16 magic-exponent method): 0x6400 is fp16 1024.0 and the
// ten mantissa bits below it count in units of 1, so OR-ing a nibble n into the
// low mantissa bits gives exactly 1024 + n; OR-ing it one nibble higher gives
// 1024 + 16n.  One v_and_or_b32 ((a & mask) | 0x64006400) extracts two nibbles
// that sit 16 bits apart straight into a packed half2.  Because of the slot
// interleave, the four masks/shifts below hand back k = (0,1), (2,3), (4,5),
// (6,7) in that order:
//
//   (q      & 0x000f000f) | magic -> slots 0,4 -> k 0,1  as 1024 + n
//   (q      & 0x00f000f0) | magic -> slots 1,5 -> k 2,3  as 1024 + 16n
//   (q >> 8 & 0x000f000f) | magic -> slots 2,6 -> k 4,5  as 1024 + n
//   (q >> 8 & 0x00f000f0) | magic -> slots 3,7 -> k 6,7  as 1024 + 16n
//
// The bias 1024 and the zero-point 8 come off in one v_pk_add_f16 (-1032) for
// the low pairs and one v_pk_fma_f16 (x/16 - 72) for the high pairs.  Every
// intermediate is an integer <= 1264, exactly representable in fp16, so the
// result is the exact n - 8.  9 VALU ops decode 8 weights.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nibble {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kMaskLo = 0x000f000fu;
constexpr uint32_t kMaskHi = 0x00f000f0u;
constexpr uint32_t kMagic = 0x64006400u;  // two copies of fp16 1024.0

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
__device__ __forceinline__ uint32_t as_u32(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// (a & mask) | magic -- selected as one v_and_or_b32 when the mask and the
// magic are register operands.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
  return (a & mask) | magic;
}

// The decode constants as opaque register values.  gfx9 VOP3 encodings take
// no 32-bit literal, so with the constants visible the compiler splits every
// and-or into a v_and_b32 and a v_or_b32 with literal operands; hiding them
// behind empty asm statements (which emit nothing) leaves it an SGPR mask and
// a VGPR magic, and it selects the single v_and_or_b32 itself -- with the
// usual hazard tracking towards the MFMAs that consume the result.
struct DecodeConsts {
  uint32_t lo, hi, magic;
};
__device__ __forceinline__ DecodeConsts decode_consts() {
  DecodeConsts c;
  asm("" : "=s"(c.lo) : "0"(kMaskLo));
  asm("" : "=s"(c.hi) : "0"(kMaskHi));
  asm("" : "=v"(c.magic) : "0"(kMagic));
  return c;
}

// The four raw magic-biased pairs of one word: k (0,1) and (4,5) as 1024 + n,
// k (2,3) and (6,7) as 1024 + 16n.
__device__ __forceinline__ void decode8_raw(uint32_t q, uint32_t (&r)[4],
                                            const DecodeConsts& k = decode_consts()) {
  const uint32_t qh = q >> 8;
  r[0] = and_or(q, k.lo, k.magic);
  r[1] = and_or(q, k.hi, k.magic);
  r[2] = and_or(qh, k.lo, k.magic);
  r[3] = and_or(qh, k.hi, k.magic);
}

// Exact (n - 8) for k = 0..7 as four half2 in ascending k.
__device__ __forceinline__ void decode8(uint32_t q, h2_t (&out)[4]) {
  uint32_t r[4];
  decode8_raw(q, r);
  const h2_t bias_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
  const h2_t mul_hi = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2_t bias_hi = {(_Float16)-72.0f, (_Float16)-72.0f};
  out[0] = as_h2(r[0]) - bias_lo;
  out[1] = __builtin_elementwise_fma(as_h2(r[1]), mul_hi, bias_hi);
  out[2] = as_h2(r[2]) - bias_lo;
  out[3] = __builtin_elementwise_fma(as_h2(r[3]), mul_hi, bias_hi);
}

// decode8 followed by one round-to-nearest-even fp16 multiply by the group
// scale: fp16((n - 8) * s), bit-identical to the reference dequantize().
__device__ __forceinline__ void decode8_scaled(uint32_t q, h2_t scale2, h2_t (&out)[4]) {
  decode8(q, out);
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = out[i] * scale2;
}

// The four magic-biased pairs of one word as eight fp16 in ascending k, i.e.
// one MFMA B-operand lane: k (0,1) and (4,5) hold 1024 + n, k (2,3) and (6,7)
// hold 1024 + 16n.  5 VALU ops for 8 weights.
__device__ __forceinline__ h8_t decode8_biased(uint32_t q, const DecodeConsts& k) {
  uint32_t r[4];
  decode8_raw(q, r, k);
  const u4_t v = {r[0], r[1], r[2], r[3]};
  return __builtin_bit_cast(h8_t, v);
}

// Companions of decode8_biased for an MFMA dot product.  With activations
// pre-scaled by kBiasedXScale (x/16 at k % 8 in {2,3,6,7}), the biased weights
// plus kBiasedCorrection give back exactly x * (n - 8) per element:
//   k in {0,1,4,5}:  x    * ((1024 + n)   - 1032) = x * (n - 8)
//   k in {2,3,6,7}:  x/16 * ((1024 + 16n) - 1152) = x * (n - 8)
// so sum_k x~ * biased + sum_k x~ * correction is the exact-weight dot
// product; the second sum does not depend on the column, so one MFMA
// against the constant correction serves every column of a chunk.
__device__ __forceinline__ h8_t biased_x_scale() {
  const _Float16 a = (_Float16)1.0f, b = (_Float16)0.0625f;
  return h8_t{a, a, b, b, a, a, b, b};
}
__device__ __forceinline__ h8_t biased_correction() {
  const _Float16 a = (_Float16)-1032.0f, b = (_Float16)-1152.0f;
  return h8_t{a, a, b, b, a, a, b, b};
}

// Scalar decode of logical offset k (0..7): shift, mask, subtract the
// zero-point.  Slot formula from csrc/dequant.cuh:94-99 in the reference.
__device__ __forceinline__ int nibble_value(uint32_t q, int k) {
  const int slot = (k & 1) ? (4 + (k >> 1)) : (k >> 1);
  return static_cast<int>((q >> (4 * slot)) & 0xFu) - 8;
}

// Cross-workgroup exchange ("last arriver reduces").  Every split-K reduction
// in this library (gemv.hip split kernel, gemm.hip split-K epilogues,
// glue.hip attention splits) follows one protocol:
//   1. each workgroup writes its partials with store_coherent();
//   2. wait_vm_stores(), then __syncthreads();
//   3. one thread does a relaxed agent-scope fetch_add on the tile's counter;
//      the workgroup that sees count == splits - 1 is the last;
//   4. the last workgroup reads every partial with load_coherent(), writes
//      the output and stores the counter back to zero.
// HARDWARE ASSUMPTION (gfx950 / CDNA4; not true of the C++ memory model in
// general): the ordering between 1 and 3 comes from the hardware, not from a
// release/acquire pair.  On gfx9 a vector store counts in vmcnt until it has
// been acknowledged by the memory side, an agent-scope store is written
// through past the issuing XCD's L2 (and an agent-scope load misses in it),
// and the counter atomic is performed at the device's coherence point.  So
// once step 2 has waited vmcnt to zero, every partial is visible to an
// agent-scope load from any XCD before the counter can show this workgroup's
// increment.  This replaces the agent-scope release/acquire fences, which on
// a multi-XCD device write back and invalidate the whole L2 (measured at
// several microseconds per decode launch).  A port to another target has to
// re-establish the ordering with __ATOMIC_RELEASE / __ATOMIC_ACQUIRE on the
// counter; the #error in nibble_common.h stops a build for any other target.

// Device-coherent (agent-scope, relaxed) accesses for data exchanged between
// workgroups of one launch.  On a multi-XCD device each XCD has its own L2;
// these bypass its non-coherent copy instead of writing back / invalidating
// the whole L2 the way an agent-scope fence does.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until every outstanding vector-memory access of this wave (loads and
// stores; gfx9 counts both in vmcnt) has completed.  A compiler barrier on
// both sides keeps memory operations from moving across it.
__device__ __forceinline__ void wait_vm_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Buffer resource for raw buffer loads on gfx9: base, stride 0, byte extent,
// and the gfx9 data-format dword.  Loads past `bytes` return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// A lane offset no buffer resource of this library reaches (every resource is
// < 2^31 bytes, checked on the host): loads through it return zero without
// touching memory.
constexpr uint32_t kOutOfRange = 0x80000000u;

// s_waitcnt immediate that waits for all but the newest n vector-memory
// operations of the wave (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4],
// lgkmcnt[11:8]; the counters not named are left at their maxima), and the
// one that waits for every LDS / scalar-memory operation (lgkmcnt 0).
constexpr int waitcnt_vm(int n) { return (n & 0xF) | ((n >> 4) << 14) | 0x70 | 0xF00; }
constexpr int kWaitLgkm0 = 0xC07F;

// A workgroup barrier that orders LDS only: each arriving wave's own LDS
// accesses are complete (lgkmcnt 0).  __syncthreads() would also wait for
// every vector-memory access of the wave (vmcnt 0), draining whatever weight
// loads it keeps in flight.  LDS written by LDS-DMA is ordered by explicit
// vmcnt waits before the barrier instead.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace nibble
