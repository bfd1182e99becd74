/*
 * Device images for the payload-image launch tests, written the way the
 * MLIR GPU lowering emits a region's kernel: every memref argument exploded
 * into (allocated pointer, aligned pointer, offset, sizes..., strides...) and
 * every scalar passed by value, in the order of the dispatch's arguments.
 * The build compiles this file into a bare gfx950 code object and into a
 * clang offload bundle; the tests put either in a payload's binary section.
 */
#include <hip/hip_runtime.h>
#include <cstdint>

#define MEMREF1(T, n) T *n##_alloc, T *n, int64_t n##_off, int64_t n##_size, int64_t n##_stride
#define MEMREF2(T, n)                                                                      \
  T *n##_alloc, T *n, int64_t n##_off, int64_t n##_rows, int64_t n##_cols,                 \
      int64_t n##_rstride, int64_t n##_cstride

/* y = a x + y over x's extent, grid-strided (`launch=` sizes the grid). */
extern "C" __global__ void vx_img_axpy(MEMREF1(float, x), MEMREF1(float, y), float a) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < x_size; i += step) {
    y[y_off + i * y_stride] = a * x[x_off + i * x_stride] + y[y_off + i * y_stride];
  }
}

/* Block b scales row b: m[b][j] = 2 m[b][j] + add (`grid=$0`, `block=`). */
extern "C" __global__ void vx_img_rows(MEMREF2(float, m), int32_t add) {
  const int64_t row = blockIdx.x + (int64_t)blockIdx.y * gridDim.x;
  if (row >= m_rows) {
    return;
  }
  for (int64_t j = threadIdx.x; j < m_cols; j += blockDim.x) {
    float *p = m + m_off + row * m_rstride + j * m_cstride;
    *p = 2.0f * *p + (float)add;
  }
}

/* Sets the assert flag (the extra last parameter) when an element is
 * negative; writes |x| either way. */
extern "C" __global__ void vx_img_check(MEMREF1(float, x), int *assert_flag) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < x_size; i += step) {
    float *p = x + x_off + i * x_stride;
    if (*p < 0.0f) {
      *assert_flag = 1;
    }
    *p = fabsf(*p);
  }
}

/* Reverses each block's slice of x through dynamic LDS (`shared=` bytes). */
extern "C" __global__ void vx_img_reverse(MEMREF1(float, x)) {
  extern __shared__ float tile[];
  const int64_t base = (int64_t)blockIdx.x * blockDim.x;
  const int t = threadIdx.x;
  const int64_t n = x_size - base < (int64_t)blockDim.x ? x_size - base : blockDim.x;
  if (t < n) {
    tile[t] = x[x_off + (base + t) * x_stride];
  }
  __syncthreads();
  if (t < n) {
    x[x_off + (base + t) * x_stride] = tile[n - 1 - t];
  }
}
