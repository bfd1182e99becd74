/*
 * vx_hip_common.h -- error handling and numeric helpers shared by the HIP
 * dispatch library and its kernels.
 *
 * A device or runtime error is fatal, as in every Vx dispatch library
 * (reference runtime/cuda_dispatch.cpp:188-325): the message names the call
 * and the library, goes to stderr (stdout belongs to the program), and the
 * process aborts.
 */
#ifndef VX_AMD_HIP_COMMON_H
#define VX_AMD_HIP_COMMON_H

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define VX_HIP_CHECK(call)                                                     \
  do {                                                                         \
    hipError_t vx_err_ = (call);                                               \
    if (vx_err_ != hipSuccess) {                                               \
      fprintf(stderr, "[Vx HIP] FATAL: %s failed: %s (%s:%d)\n", #call,        \
              hipGetErrorString(vx_err_), __FILE__, __LINE__);                 \
      abort();                                                                 \
    }                                                                          \
  } while (0)

namespace vxk {

/* bf16 <-> f32. bf16 is the top half of an f32; narrowing rounds to nearest
 * even, and a NaN stays a quiet NaN. */
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  union {
    uint32_t u;
    float f;
  } v;
  v.u = (uint32_t)h << 16;
  return v.f;
}

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  union {
    uint32_t u;
    float f;
  } v;
  v.f = f;
  if ((v.u & 0x7f800000u) == 0x7f800000u && (v.u & 0x007fffffu)) {
    return (uint16_t)((v.u >> 16) | 0x40);
  }
  uint32_t round = 0x7fffu + ((v.u >> 16) & 1u);
  return (uint16_t)((v.u + round) >> 16);
}

__host__ __device__ inline float f16_to_f32(uint16_t h) {
  _Float16 x;
  __builtin_memcpy(&x, &h, 2);
  return (float)x;
}

__host__ __device__ inline uint16_t f32_to_f16(float f) {
  _Float16 x = (_Float16)f;
  uint16_t h;
  __builtin_memcpy(&h, &x, 2);
  return h;
}

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

/* Compute units of the device current at the first call (256 if it cannot
 * be read); launch shapes are sized by it. */
inline int device_cu_count() {
  static std::atomic<int> cached{0};
  int n = cached.load();
  if (n == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    n = hipGetDevice(&dev) == hipSuccess &&
                hipGetDeviceProperties(&prop, dev) == hipSuccess
            ? prop.multiProcessorCount
            : 256;
    cached.store(n);
  }
  return n;
}

} // namespace vxk

#endif /* VX_AMD_HIP_COMMON_H */
