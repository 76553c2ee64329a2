// ABI-wide entry points and the host plumbing declared in nibble_common.h.
#include <atomic>
#include <cstdio>
#include <string>

#include "nibble_common.h"

namespace nibble {

namespace {
thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];
}  // namespace

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return NIBBLE_OK;
}

int hip_fail(hipError_t err, const char* what) {
  return fail(NIBBLE_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(err), (int)err);
}

hipError_t stream_device(hipStream_t stream, int* device) {
  if (stream == nullptr) return hipGetDevice(device);
  return hipStreamGetDevice(stream, device);
}

hipError_t DeviceGuard::enter(hipStream_t stream, int* device) {
  hipError_t e = stream_device(stream, device);
  if (e != hipSuccess) return e;
  int cur = -1;
  e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  if (cur != *device) {
    e = hipSetDevice(*device);
    if (e != hipSuccess) return e;
    restore_ = cur;
  }
  return hipSuccess;
}

namespace {
__global__ void fill_zero_kernel(_Float16* __restrict__ y, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) y[i] = (_Float16)0.0f;
}
}  // namespace

hipError_t fill_zero_f16(void* y, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  fill_zero_kernel<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(static_cast<_Float16*>(y), n);
  return hipGetLastError();
}

hipError_t cu_count(int device, int* out) {
  if (device >= 0 && device < kMaxDevices) {
    const int cached = g_cu_count[device].load(std::memory_order_relaxed);
    if (cached > 0) {
      *out = cached;
      return hipSuccess;
    }
  }
  int v = 0;
  hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return e;
  if (v <= 0) v = 1;
  if (device >= 0 && device < kMaxDevices) g_cu_count[device].store(v, std::memory_order_relaxed);
  *out = v;
  return hipSuccess;
}

}  // namespace nibble

extern "C" {

int nibble_abi_version(void) { return NIBBLE_ABI_VERSION; }

const char* nibble_last_error(void) { return nibble::g_last_error.c_str(); }

}  // extern "C"
