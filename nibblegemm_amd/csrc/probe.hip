// Streaming-read probe: the HBM read bandwidth a plain kernel reaches, the
// denominator the decode GEMV (a read-dominated kernel) is compared with next
// to the device copy.  No counterpart in the reference, whose harness measures
// a copy only (bench/harness.py:189-200).
//
// Each workgroup streams a contiguous slice with 16-byte loads, four in flight
// per thread, and folds them into one word it writes out, so the loads are
// not dead; the sink takes 4 bytes per workgroup.
#include "nibble_common.h"
#include "nibble_decode.h"

namespace nibble {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const u4_t* __restrict__ src,
                                                                    uint64_t n16, uint64_t per_wg,
                                                                    uint32_t* __restrict__ sink) {
  const uint64_t begin = static_cast<uint64_t>(blockIdx.x) * per_wg;
  const uint64_t end = begin + per_wg < n16 ? begin + per_wg : n16;
  uint32_t acc = 0;
  for (uint64_t i = begin + threadIdx.x; i < end; i += kProbeThreads * kProbeUnroll) {
    u4_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const uint64_t j = i + static_cast<uint64_t>(u) * kProbeThreads;
      v[u] = j < end ? __builtin_nontemporal_load(src + j) : u4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  __shared__ uint32_t part[kProbeThreads / 64];
  acc = __builtin_amdgcn_readfirstlane(acc) ^ __builtin_amdgcn_readlane(acc, 63);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

}  // namespace
}  // namespace nibble

using namespace nibble;

extern "C" size_t nibble_read_probe_sink_bytes(size_t bytes, int64_t workgroups) {
  (void)bytes;
  return workgroups > 0 ? static_cast<size_t>(workgroups) * 4 : 0;
}

extern "C" int nibble_read_probe(const void* src, size_t bytes, int64_t workgroups, void* sink,
                                 void* stream_) {
  NIBBLE_CHECK(src != nullptr && sink != nullptr, "null pointer");
  NIBBLE_CHECK(aligned(src, 16) && aligned(sink, 4), "src must be 16-byte and sink 4-byte aligned");
  NIBBLE_CHECK(bytes % 16 == 0 && bytes > 0, "bytes must be a positive multiple of 16");
  NIBBLE_CHECK(workgroups >= 1 && workgroups <= (int64_t(1) << 20),
               "workgroups must be in [1, 2^20], got %lld", (long long)workgroups);
  const uint64_t n16 = bytes / 16;
  uint64_t per = (n16 + workgroups - 1) / workgroups;
  per = (per + kProbeThreads - 1) / kProbeThreads * kProbeThreads;
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  DeviceGuard guard;
  int dev = 0;
  NIBBLE_HIP(guard.enter(stream, &dev));
  read_probe_kernel<<<static_cast<unsigned>(workgroups), kProbeThreads, 0, stream>>>(
      static_cast<const u4_t*>(src), n16, per, static_cast<uint32_t*>(sink));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "read probe launch");
  return ok();
}
