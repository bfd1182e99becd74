/*
 * gemv_i8.hip -- int8 weight-only GEMV / skinny GEMM, HBM-streaming, no MFMA.
 *
 * y[b, r] = scale[r] * sum_c w[r, c] * x[b, c], w int8 [rows, cols], x bf16
 * [batch, cols], f32 sums.
 *
 * The weights are the traffic: every byte of W is read exactly once, with
 * 16-byte loads that a wave issues as 1 KiB of one row. A workgroup of 4
 * waves owns 4 * kRows consecutive rows; x is staged into LDS in column
 * chunks once per workgroup and reused by all its rows. Each lane converts
 * its 16 weight bytes to f32 once per row (one v_cvt per byte) and applies
 * them to every batch row of x, so the convert cost is shared across the
 * batch. A wave reduces its 64 partial sums per (row, batch) with
 * cross-lane shuffles and lane 0 applies the scale.
 */
#include "../vx_hip_common.h"
#include "../vx_ops_kernels.h"

namespace vxk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kChunk = 2048; /* columns of x per LDS stage */

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v += __shfl_xor(v, off, 64);
  }
  return v;
}

__device__ __forceinline__ void bytes_to_f32(u32x4 w, float out[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[q * 4 + j] = (float)(int8_t)(w[q] >> (8 * j));
    }
  }
}

__device__ __forceinline__ void bf16x16_to_f32(u32x4 lo, u32x4 hi,
                                               float out[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    out[2 * q] = __uint_as_float(lo[q] << 16);
    out[2 * q + 1] = __uint_as_float(lo[q] & 0xffff0000u);
    out[8 + 2 * q] = __uint_as_float(hi[q] << 16);
    out[8 + 2 * q + 1] = __uint_as_float(hi[q] & 0xffff0000u);
  }
}

template <int kB, int kRows>
__global__ __launch_bounds__(kThreads) void gemv_i8_kernel(
    const int8_t *__restrict__ W, const float *__restrict__ scale,
    const uint16_t *__restrict__ X, float *__restrict__ Y, int rows,
    int cols) {
  __shared__ u32x4 xs[kB * kChunk / 8];
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int row0 = (blockIdx.x * 4 + wave) * kRows;

  float acc[kRows][kB];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      acc[r][b] = 0.0f;
    }
  }

  for (int c0 = 0; c0 < cols; c0 += kChunk) {
    const int kc = min(kChunk, cols - c0);
    const int vecs = kc / 8;
    for (int i = t; i < kB * vecs; i += kThreads) {
      const int b = i / vecs;
      const int v = i - b * vecs;
      xs[b * (kChunk / 8) + v] = *reinterpret_cast<const u32x4 *>(
          X + (int64_t)b * cols + c0 + v * 8);
    }
    __syncthreads();
    for (int cc = lane * 16; cc < kc; cc += 64 * 16) {
      u32x4 wv[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const int row = row0 + r;
        wv[r] = row < rows ? __builtin_nontemporal_load(
                                 reinterpret_cast<const u32x4 *>(
                                     W + (int64_t)row * cols + c0 + cc))
                           : u32x4{0, 0, 0, 0};
      }
      float wf[kRows][16];
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        bytes_to_f32(wv[r], wf[r]);
      }
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        float xf[16];
        bf16x16_to_f32(xs[b * (kChunk / 8) + cc / 8],
                       xs[b * (kChunk / 8) + cc / 8 + 1], xf);
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            acc[r][b] += wf[r][j] * xf[j];
          }
        }
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int row = row0 + r;
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const float s = wave_sum(acc[r][b]);
      if (lane == 0 && row < rows) {
        Y[(int64_t)b * rows + row] = scale[row] * s;
      }
    }
  }
}

template <int kB>
void launch_b(const int8_t *w, const float *s, const uint16_t *x, float *y,
              int rows, int cols, hipStream_t stream) {
  constexpr int kRows = kB <= 4 ? 2 : 4;
  const int groups = (rows + 4 * kRows - 1) / (4 * kRows);
  hipLaunchKernelGGL((gemv_i8_kernel<kB, kRows>), dim3(groups), dim3(kThreads),
                     0, stream, w, s, x, y, rows, cols);
}

} // namespace

bool gemv_i8_launch(const int8_t *w, const float *scale, const uint16_t *x,
                    float *y, int64_t rows, int64_t cols, int64_t batch,
                    hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || cols % 16 != 0 || rows > INT32_MAX ||
      cols > INT32_MAX || batch < 1 || batch > 16 ||
      (reinterpret_cast<uintptr_t>(w) & 15) ||
      (reinterpret_cast<uintptr_t>(x) & 15)) {
    return false;
  }
  const int r = (int)rows, c = (int)cols;
  switch (batch) {
#define VX_GEMV_CASE(n)                                                        \
  case n:                                                                      \
    launch_b<n>(w, scale, x, y, r, c, stream);                                 \
    break;
    VX_GEMV_CASE(1)
    VX_GEMV_CASE(2)
    VX_GEMV_CASE(3)
    VX_GEMV_CASE(4)
    VX_GEMV_CASE(5)
    VX_GEMV_CASE(6)
    VX_GEMV_CASE(7)
    VX_GEMV_CASE(8)
    VX_GEMV_CASE(9)
    VX_GEMV_CASE(10)
    VX_GEMV_CASE(11)
    VX_GEMV_CASE(12)
    VX_GEMV_CASE(13)
    VX_GEMV_CASE(14)
    VX_GEMV_CASE(15)
    VX_GEMV_CASE(16)
#undef VX_GEMV_CASE
  default:
    return false;
  }
  VX_HIP_CHECK(hipGetLastError());
  return true;
}

} // namespace vxk
