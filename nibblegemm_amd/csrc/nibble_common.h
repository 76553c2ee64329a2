// Host-side plumbing shared by every entry point of the C ABI: the per-thread
// error message, status helpers, the device guard and cached device attributes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>

#include "../../include/nibblegemm_amd.h"

// Every kernel of this library is written for gfx950 (CDNA4) alone: MFMA
// shapes, LDS size, the 8-XCD workgroup mapping and the cross-workgroup
// ordering described in nibble_decode.h ("HARDWARE ASSUMPTION") all assume it.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "nibblegemm_amd is built for gfx950 only"
#endif

namespace nibble {

// Records a printf-style message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears this thread's last error and returns NIBBLE_OK.
int ok();

// Maps a failed HIP call to NIBBLE_ERR_HIP with the runtime's message.
int hip_fail(hipError_t err, const char* what);

#define NIBBLE_CHECK(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::nibble::fail(NIBBLE_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define NIBBLE_HIP(expr)                                          \
  do {                                                            \
    hipError_t e_ = (expr);                                       \
    if (e_ != hipSuccess) return ::nibble::hip_fail(e_, #expr);   \
  } while (0)

// Makes the stream's device current for the lifetime of the guard (the
// reference used a CUDAGuard on X's device, csrc/gemv_w4a16.cu:344).
class DeviceGuard {
 public:
  DeviceGuard() = default;
  ~DeviceGuard() {
    if (restore_ >= 0) (void)hipSetDevice(restore_);
  }
  hipError_t enter(hipStream_t stream, int* device);

 private:
  int restore_ = -1;
};

// Writes n fp16 zeros to y on `stream` with a kernel (not a memset, so the
// call stays safe to record into a HIP graph).  Used for empty reductions.
hipError_t fill_zero_f16(void* y, int64_t n, hipStream_t stream);

// Compute-unit count of `device`, cached after the first query.
hipError_t cu_count(int device, int* out);

// Device of `stream` (the current device for the null stream).
hipError_t stream_device(hipStream_t stream, int* device);

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace nibble
