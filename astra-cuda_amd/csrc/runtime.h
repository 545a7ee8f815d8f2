// runtime.h -- shared by the engine's translation units: error reporting in the
// C ABI's style, and the runtime calls the device build makes on HIP and the
// host-emulation build (-DASTRA_HOST_EMULATION) makes on host memory.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "astra_market.h"

#define ASTRA_HD __host__ __device__ __forceinline__

namespace astra_rt {

// Message of the last failed ABI call on this host thread (astra_last_error).
inline thread_local std::string g_last_error;

inline int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

#ifdef ASTRA_HOST_EMULATION
inline hipError_t rt_device_count(int *n) {
  *n = 1;
  return hipSuccess;
}
inline hipError_t rt_memcpy(void *d, const void *s, size_t n, hipStream_t) {
  std::memmove(d, s, n);
  return hipSuccess;
}
inline hipError_t rt_sync(hipStream_t) { return hipSuccess; }
inline hipError_t rt_last_error() { return hipSuccess; }
// The host build stands in for gfx950: 256 CUs with 160 KB of LDS each, all of
// which one workgroup may use.
inline hipError_t rt_lds_per_block(int, int *bytes) {
  *bytes = 160 * 1024;
  return hipSuccess;
}
inline hipError_t rt_lds_per_cu(int, int *bytes) {
  *bytes = 160 * 1024;
  return hipSuccess;
}
inline hipError_t rt_cu_count(int, int *n) {
  *n = 256;
  return hipSuccess;
}
struct DeviceGuard {
  bool ok = true;
  explicit DeviceGuard(int) {}
};
inline void rt_device_sync(int) {}
struct StreamMark {
  hipEvent_t ev = nullptr;
  hipError_t record(hipStream_t) { return hipSuccess; }
  hipError_t wait() { return hipSuccess; }
};
#else
inline hipError_t rt_device_count(int *n) { return hipGetDeviceCount(n); }
inline hipError_t rt_memcpy(void *d, const void *s, size_t n, hipStream_t st) {
  return hipMemcpyAsync(d, s, n, hipMemcpyDefault, st);
}
inline hipError_t rt_sync(hipStream_t st) { return hipStreamSynchronize(st); }
inline hipError_t rt_last_error() { return hipGetLastError(); }
inline hipError_t rt_lds_per_block(int dev, int *bytes) {
  return hipDeviceGetAttribute(bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
}
inline hipError_t rt_lds_per_cu(int dev, int *bytes) {
  return hipDeviceGetAttribute(bytes, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev);
}
inline hipError_t rt_cu_count(int dev, int *n) {
  return hipDeviceGetAttribute(n, hipDeviceAttributeMultiprocessorCount, dev);
}
// Restores the calling thread's current device when it goes out of scope.
struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};
inline void rt_device_sync(int dev) {
  DeviceGuard g(dev);
  (void)hipDeviceSynchronize();
}
// A point in a stream the host can wait for while later work on the stream
// runs (one cached event per host thread and device).
// An event recorded on a stream and waited for: `ev` if the caller set one,
// else one created on first use per host thread and device and kept.
struct StreamMark {
  hipEvent_t ev = nullptr;
  hipError_t record(hipStream_t st) {
    if (ev) return hipEventRecord(ev, st);
    static thread_local hipEvent_t cache[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!cache[dev] && (e = hipEventCreateWithFlags(&cache[dev], hipEventDisableTiming)) != hipSuccess)
      return e;
    ev = cache[dev];
    return hipEventRecord(ev, st);
  }
  hipError_t wait() { return hipEventSynchronize(ev); }
};
#endif

}  // namespace astra_rt

// Mirrors ASTRA_CHECK_OP's text (src/utils/astra_utils.h:116-131); ASTRA_SRC_NAME
// is the including file's name.
#define ASTRA_ABI_CHECK(x_exp, op, y_exp)                                               \
  do {                                                                                  \
    long long x_ = (long long)(x_exp), y_ = (long long)(y_exp);                         \
    if (!(x_ op y_))                                                                    \
      return astra_rt::fail(ASTRA_ERR_INVALID_ARGUMENT,                                 \
                            std::string(ASTRA_SRC_NAME ":") + std::to_string(__LINE__) + \
                                " " #x_exp " " #op " " #y_exp "\n" #x_exp " = " +       \
                                std::to_string(x_) + ", " #y_exp " = " +                \
                                std::to_string(y_));                                    \
  } while (false)

#define ASTRA_HIP_CHECK(call, what)                                                     \
  do {                                                                                  \
    hipError_t e_ = (call);                                                             \
    if (e_ != hipSuccess)                                                               \
      return astra_rt::fail(ASTRA_ERR_HIP, std::string("HIP error in ") + (what) + ": " + \
                                               hipGetErrorString(e_));                  \
  } while (false)
