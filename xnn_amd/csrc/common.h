// Host-side helpers of the C ABI: thread-local error text and launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "xnn_amd.h"

namespace xnn {

void set_error(const char* fmt, ...);

inline hipStream_t as_hip(xnn_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int grid_1d(int64_t n, int block) { return (int)((n + block - 1) / block); }

// wave-local ordering of LDS traffic (lanes of one wave exchange through LDS)
__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace xnn

#define XNN_REQUIRE(cond, ...)      \
  do {                              \
    if (!(cond)) {                  \
      ::xnn::set_error(__VA_ARGS__); \
      return XNN_EINVAL;            \
    }                               \
  } while (0)

#define XNN_LAUNCH_CHECK()                                               \
  do {                                                                   \
    hipError_t err_ = hipGetLastError();                                 \
    if (err_ != hipSuccess) {                                            \
      ::xnn::set_error("HIP launch failed: %s", hipGetErrorString(err_)); \
      return XNN_EHIP;                                                   \
    }                                                                    \
  } while (0)

#define XNN_HIP_CHECK(expr)                                                     \
  do {                                                                          \
    hipError_t err_ = (expr);                                                   \
    if (err_ != hipSuccess) {                                                   \
      ::xnn::set_error("%s failed: %s", #expr, hipGetErrorString(err_));         \
      return XNN_EHIP;                                                          \
    }                                                                           \
  } while (0)
