/*
 * gemv_i8.hip -- int8 weight-only GEMV / skinny GEMM, HBM-streaming.
 *
 * y[b, r] = scale[r] * sum_c w[r, c] * x[b, c], w int8 [rows, cols], x bf16
 * [batch, cols], f32 sums.
 *
 * The weights are the traffic: every byte of W is read once, with 16-byte
 * non-temporal loads. The int8 weights become bf16 pairs exactly (|w| <= 127
 * fits bf16's mantissa: a byte-to-f32 convert, then the high halves of two
 * floats) and meet x either in v_dot2_f32_bf16 (gemv_i8_rows: batch 1, and
 * batches up to 4 over at most 4096 columns) or in v_mfma_f32_16x16x32_bf16
 * (gemv_i8_lds: the rest); the products are exact either way and every
 * batch row reuses one conversion.
 */
#include "../vx_hip_common.h"
#include "../vx_ops_kernels.h"

#include <algorithm>
#include <atomic>

namespace vxk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kGroupCols = kThreads * 16; /* columns one pass of a WG covers */
constexpr int kMaxRows = 64;              /* rows per workgroup, at most */
constexpr int kMaxGrid = 2048;

/* int8 bytes of `w` as 8 bf16 pairs (exact). */
__device__ __forceinline__ void bytes_to_bf16x2(u32x4 w, uint32_t out[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float f0 = (float)(int8_t)(w[q]);
    const float f1 = (float)(int8_t)(w[q] >> 8);
    const float f2 = (float)(int8_t)(w[q] >> 16);
    const float f3 = (float)(int8_t)(w[q] >> 24);
    out[2 * q] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0),
                                       0x07060302u);
    out[2 * q + 1] = __builtin_amdgcn_perm(__float_as_uint(f3),
                                           __float_as_uint(f2), 0x07060302u);
  }
}

__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                         __builtin_bit_cast(bf16x2, x), acc,
                                         false);
}

constexpr int log2i(int n) { return n <= 1 ? 0 : 1 + log2i(n / 2); }

/* Lane exchange across the wave with VALU data movement (no LDS
 * crossbar): the two 32-lane halves and the 16-lane rows trade through
 * v_permlane32_swap / v_permlane16_swap, lanes within a row through DPP. */
__device__ __forceinline__ void swap32(float &x, float &y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                  __float_as_uint(y), false,
                                                  false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}

__device__ __forceinline__ void swap16(float &x, float &y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x),
                                                  __float_as_uint(y), false,
                                                  false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}

/* DPP controls pairing lane i of a 16-lane row with the lane differing in
 * bit 3 (rotate by 8), bit 2 (mirror within 8: i <-> 7-i), bit 1 and bit 0
 * (quad permutes). */
template <int kO> constexpr int dpp_partner() {
  return kO == 8 ? 0x128 : kO == 4 ? 0x141 : kO == 2 ? 0x4e : 0xb1;
}

template <int kO> __device__ __forceinline__ float from_partner(float v) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(
      0u, __float_as_uint(v), dpp_partner<kO>(), 0xf, 0xf, false));
}

/* Sum v[b] over the 64 lanes for every b, as a reduce-scatter: at each of
 * the first log2(kB) exchange steps (partners across 32, 16, 8, 4, 2, 1
 * lanes) a lane keeps the sums of half of its values and hands the other
 * half to its partner; the remaining steps are plain sums. Returns the
 * batch index whose total this lane holds in v[0]; lanes whose low
 * 6 - log2(kB) bits are zero are the ones to read. */
template <int kB, int kStep>
__device__ __forceinline__ void rs_step(float (&v)[kB], int lane, int &b) {
  constexpr int kP = log2i(kB);
  constexpr int kO = 32 >> kStep;
  if constexpr (kStep < kP) {
    constexpr int kHalf = kB >> (kStep + 1);
    const bool up = (lane & kO) != 0;
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      if constexpr (kO >= 16) {
        float x = v[i], y = v[i + kHalf];
        kO == 32 ? swap32(x, y) : swap16(x, y);
        v[i] = x + y;
      } else {
        const float lo = v[i] + from_partner<kO>(v[i]);
        const float hi = v[i + kHalf] + from_partner<kO>(v[i + kHalf]);
        v[i] = up ? hi : lo;
      }
    }
    b += up ? kHalf : 0;
  } else {
    if constexpr (kO >= 16) {
      float x = v[0], y = v[0];
      kO == 32 ? swap32(x, y) : swap16(x, y);
      v[0] = x + y;
    } else {
      v[0] += from_partner<kO>(v[0]);
    }
  }
}

template <int kB>
__device__ __forceinline__ int wave_reduce_scatter(float (&v)[kB], int lane) {
  int b = 0;
  rs_step<kB, 0>(v, lane, b);
  rs_step<kB, 1>(v, lane, b);
  rs_step<kB, 2>(v, lane, b);
  rs_step<kB, 3>(v, lane, b);
  rs_step<kB, 4>(v, lane, b);
  rs_step<kB, 5>(v, lane, b);
  return b;
}

/* y[b, r] for batches of 3 and 4 over at most 4096 columns: kB batch rows
 * (nb of them real, the rest padding), kU weight rows in flight per pass.
 *
 * Workgroup g owns rows g, g + G, g + 2G, ... (G = gridDim.x), so at any
 * moment the whole grid reads a contiguous band of W. Thread t owns columns
 * t*16 + j*4096 of every row; for each such column group j it holds its 16
 * columns of x for every batch row in registers and sweeps its rows, kU at
 * a time, with 16-byte non-temporal loads (1 KiB per wave instruction, 4 KiB
 * per row per workgroup). A row's partial sums go through the wave
 * reduce-scatter and land in LDS, one slot per (row, batch, wave), summed
 * over the column groups; the 4 waves' slots are added once at the end. */
template <int kB, int kU>
__global__ __launch_bounds__(kThreads) void gemv_i8_kernel(
    const int8_t *__restrict__ W, const float *__restrict__ scale,
    const uint16_t *__restrict__ X, float *__restrict__ Y, int rows, int cols,
    int nb) {
  __shared__ float red[kMaxRows][kB][kWaves];
  constexpr int kP = log2i(kB);
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int grid = gridDim.x;
  const int nk = (rows - (int)blockIdx.x + grid - 1) / grid; /* my rows */
  const bool writer = (lane & ((64 >> kP) - 1)) == 0;

  for (int c0 = 0; c0 < cols; c0 += kGroupCols) {
    const int c = c0 + t * 16;
    const bool live = c < cols;
    u32x4 xl[kB], xh[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const bool ok = live && b < nb;
      const uint16_t *xp = X + (int64_t)b * cols + c;
      xl[b] = ok ? *reinterpret_cast<const u32x4 *>(xp) : u32x4{0, 0, 0, 0};
      xh[b] = ok ? *reinterpret_cast<const u32x4 *>(xp + 8) : u32x4{0, 0, 0, 0};
    }
    for (int k0 = 0; k0 < nk; k0 += kU) {
      u32x4 wv[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int r = (int)blockIdx.x + (k0 + u) * grid;
        wv[u] = (live && k0 + u < nk)
                    ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(
                          W + (int64_t)r * cols + c))
                    : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        uint32_t wp[8];
        bytes_to_bf16x2(wv[u], wp);
        float v[kB];
#pragma unroll
        for (int b = 0; b < kB; ++b) {
          float a = 0.0f;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            a = dot2(wp[p], xl[b][p], a);
          }
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            a = dot2(wp[4 + p], xh[b][p], a);
          }
          v[b] = a;
        }
        const int b = wave_reduce_scatter<kB>(v, lane);
        if (writer && k0 + u < nk) {
          float &slot = red[k0 + u][b][wave];
          slot = c0 == 0 ? v[0] : slot + v[0];
        }
      }
    }
  }
  __syncthreads();
  for (int i = t; i < nk * nb; i += kThreads) {
    const int k = i / nb;
    const int b = i % nb;
    const int r = (int)blockIdx.x + k * grid;
    float v = red[k][b][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      v += red[k][b][w];
    }
    Y[(int64_t)b * rows + r] = scale[r] * v;
  }
}

/* y[b, r] for kB batch rows (nb of them real, the rest zero padding).
 *
 * Workgroup g owns the kR consecutive rows kR g .. kR g + kR - 1: one
 * contiguous stretch of W. It walks the columns in passes of 4096 (thread t
 * takes columns 16 t .. 16 t + 15 of each pass), kP passes at a time, and
 * issues every load of those kP passes -- its x columns for each batch row,
 * then its 16 bytes of each of the kR rows -- before it waits for any: the
 * workgroup is one burst of reads, and the hardware keeps the CU full by
 * starting the next workgroup as one ends. Buffer loads return zeros past
 * the workgroup's rows, past the last column and past batch row nb, so the
 * ragged edges need no branch (a branch around a load would make the
 * compiler wait for it before issuing the next). The kR * kB partial sums
 * go through one wave reduce-scatter and meet across the 4 waves in LDS. */
template <int kB, int kR, int kP>
__global__ __launch_bounds__(kThreads) void gemv_i8_rows(
    const int8_t *__restrict__ W, const float *__restrict__ scale,
    const uint16_t *__restrict__ X, float *__restrict__ Y, int rows, int cols,
    int nb) {
  constexpr int kV = kR * kB;
  constexpr int kLog = log2i(kV);
  static_assert((1 << kLog) == kV && kV <= 64, "kR * kB: a power of two");
  constexpr uint32_t kOut = 0x80000000u; /* past every range */
  __shared__ float red[kWaves][kV];
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int r0 = (int)blockIdx.x * kR;
  const int my_rows = min(kR, rows - r0);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(W + (int64_t)r0 * cols), (short)0, my_rows * cols, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)X, (short)0, nb * cols * 2, 0x00020000);
  float v[kV];
#pragma unroll
  for (int i = 0; i < kV; ++i) {
    v[i] = 0.0f;
  }
  for (int c0 = 0; c0 < cols; c0 += kGroupCols * kP) {
    u32x4 xl[kP][kB], xh[kP][kB], wv[kP][kR];
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      const int c = c0 + p * kGroupCols + t * 16;
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const uint32_t off = c < cols ? (uint32_t)((b * cols + c) * 2) : kOut;
        xl[p][b] = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0);
        xh[p][b] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (int)(c < cols ? off + 16 : kOut), 0, 0);
      }
    }
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      const int c = c0 + p * kGroupCols + t * 16;
#pragma unroll
      for (int u = 0; u < kR; ++u) {
        const uint32_t off = c < cols ? (uint32_t)(u * cols + c) : kOut;
        wv[p][u] = __builtin_amdgcn_raw_buffer_load_b128(wr, (int)off, 0, 2);
      }
    }
#pragma unroll
    for (int p = 0; p < kP; ++p) {
#pragma unroll
      for (int u = 0; u < kR; ++u) {
        uint32_t wp[8];
        bytes_to_bf16x2(wv[p][u], wp);
#pragma unroll
        for (int b = 0; b < kB; ++b) {
          float a = v[u * kB + b];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            a = dot2(wp[q], xl[p][b][q], a);
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            a = dot2(wp[4 + q], xh[p][b][q], a);
          }
          v[u * kB + b] = a;
        }
      }
    }
  }
  const int i = wave_reduce_scatter<kV>(v, lane);
  if ((lane & ((64 >> kLog) - 1)) == 0) {
    red[wave][i] = v[0];
  }
  __syncthreads();
  if (t < kV) {
    const int u = t / kB, b = t % kB;
    if (u < my_rows && b < nb) {
      float sum = red[0][t];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) {
        sum += red[w][t];
      }
      Y[(int64_t)b * rows + r0 + u] = scale[r0 + u] * sum;
    }
  }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma_bf16(const uint32_t *a, u32x4 b, f32x4 c) {
  const u32x4 av = {a[0], a[1], a[2], a[3]};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                 __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

/* MFMA GEMV with contiguous weight loads. Each wave owns a private LDS tile
 * of 16 kR rows x kCols bytes: it loads the tile with 16-byte non-temporal
 * buffer loads in which every wave instruction covers 1 KiB of W (1024 /
 * kCols rows of kCols contiguous bytes: the shape that streams HBM best),
 * writes it to the tile, and reads it back in the MFMA operand order (lane
 * l: row l % 16 of each 16-row block, 16 bytes at column 16 (l / 16) of each
 * 64-column step). Tile rows are padded by 16 bytes so those reads hit
 * distinct banks. The tile is private to its wave, whose LDS operations
 * complete in order, so only wave-scope ordering is needed between the
 * writes and the reads.
 *
 * Loads retire in issue order, so each pass issues this tile's x loads,
 * then writes the tile (waiting for its weights), then issues the next
 * tile's weight loads, and only then waits for x. Buffer loads return zero
 * past the end of their range, which covers the last rows, the last columns
 * and the batch rows past nb without a branch.
 *
 * kXl (16-row tiles): x goes through the wave's LDS as well. The wave
 * loads its x columns as whole 128-byte lines of each batch row (in operand
 * order a load instruction touches 16 half lines), writes them to an x
 * tile beside the weight tile and reads the MFMA operands from there; and
 * the next tile's weights are requested with no branch around the loads (a
 * tile past the last has every column past `cols`), so the multiply waits
 * for x alone (behind a branch the compiler's waits at the join count the
 * prefetch as possibly absent, and each tile's last MFMA waited for it).
 * The launch takes it with 128-column tiles (measured faster than 256 with
 * the x tile) when the grid fits one round, for batches of 8 and more
 * (below, most of the tile is zeros and its LDS round trip cost more than
 * the whole lines saved). The branch-free prefetch alone, or on 64-row
 * tiles without the x tile, measured slower.
 *
 * Workgroup g owns rows 16 kR g ..; its kW waves take the column tiles w,
 * w + kW, ...; their accumulators meet in LDS at the end. */
template <int kW, int kCols, int kR, bool kXl>
__global__ __launch_bounds__(kW * 64) void gemv_i8_lds(
    const int8_t *__restrict__ W, const float *__restrict__ scale,
    const uint16_t *__restrict__ X, float *__restrict__ Y, int rows, int cols,
    int nb) {
  constexpr int kRows = 16 * kR;
  constexpr int kStride = kCols + 16;
  constexpr int kLanesPerRow = kCols / 16;
  constexpr int kRowsPerInst = 64 / kLanesPerRow;
  constexpr int kInst = kRows / kRowsPerInst;
  constexpr int kSteps = kCols / 64;
  constexpr uint32_t kOut = 0x80000000u; /* past every range */
  /* x tile (kXl): 16 batch rows of kCols bf16, rows padded by 16 bytes;
   * each load instruction covers 64 * 16 bytes of it in whole lines. */
  constexpr int kXStride = kCols * 2 + 16;
  constexpr int kXLanesPerRow = kCols * 2 / 16;
  constexpr int kXRowsPerInst = 64 / kXLanesPerRow;
  constexpr int kXInst = kXl ? 16 / kXRowsPerInst : 1;
  constexpr int kWaveBytes = kRows * kStride + (kXl ? 16 * kXStride : 0);
  static_assert(!kXl || (kXLanesPerRow <= 64 && 64 % kXLanesPerRow == 0), "x tile shape");
  /* The waves' tiles and, once every wave is past its last tile, the
   * partial sums share one LDS block. */
  constexpr int kTileBytes = kW * kWaveBytes;
  constexpr int kRedBytes = kW * kRows * 17 * 4;
  __shared__ __attribute__((aligned(16)))
  int8_t smem[kTileBytes > kRedBytes ? kTileBytes : kRedBytes];
  auto tile = reinterpret_cast<int8_t (*)[kWaveBytes]>(smem);
  auto red = reinterpret_cast<float (*)[kRows][17]>(smem);
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int m = lane & 15, g = lane >> 4;
  const int r0 = (int)blockIdx.x * kRows;
  const int lr = lane / kLanesPerRow;        /* row within an instruction */
  const int lc = (lane % kLanesPerRow) * 16; /* byte column within the tile */
  const int my_rows = min(kRows, rows - r0);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(W + (int64_t)r0 * cols), (short)0, my_rows * cols, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)X, (short)0, nb * cols * 2, 0x00020000);
  int8_t *my = tile[wave];
  int8_t *myx = my + kRows * kStride; /* kXl: this wave's x tile */
  const int ntiles = (cols + kCols - 1) / kCols;

  u32x4 cur[kInst];
  auto load_w = [&](int s) {
    const int c = s * kCols + lc;
#pragma unroll
    for (int j = 0; j < kInst; ++j) {
      const uint32_t off = c < cols ? (uint32_t)((j * kRowsPerInst + lr) * cols + c) : kOut;
      cur[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, (int)off, 0, 2);
    }
  };
  f32x4 acc[kR];
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  u32x4 xa[kSteps], xb[kSteps];
  u32x4 xl[kXInst];
  auto load_x = [&](int s) {
    if constexpr (kXl) {
      /* lane l of instruction i: batch row i * kXRowsPerInst + l /
       * kXLanesPerRow, 8 columns at (l % kXLanesPerRow) * 8 */
      const int c = s * kCols + (lane % kXLanesPerRow) * 8;
#pragma unroll
      for (int i = 0; i < kXInst; ++i) {
        const int n = i * kXRowsPerInst + lane / kXLanesPerRow;
        const uint32_t off = (uint32_t)((n * cols + c) * 2);
        xl[i] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (int)(n < nb && c < cols ? off : kOut), 0, 0);
      }
    } else {
#pragma unroll
      for (int jj = 0; jj < kSteps; ++jj) {
        const int c = s * kCols + 64 * jj + 8 * g;
        const uint32_t off = (uint32_t)((m * cols + c) * 2);
        xa[jj] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (int)(m < nb && c < cols ? off : kOut), 0, 0);
        xb[jj] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (int)(m < nb && c + 32 < cols ? off + 64 : kOut), 0, 0);
      }
    }
  };
  int s = wave;
  if (kXl || s < ntiles) {
    load_w(s);
  }
  for (; s < ntiles; s += kW) {
    load_x(s);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kInst; ++j) {
      *reinterpret_cast<u32x4 *>(my + (j * kRowsPerInst + lr) * kStride + lc) = cur[j];
    }
    __builtin_amdgcn_sched_barrier(0);
    if (kXl || s + kW < ntiles) {
      load_w(s + kW);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kXl) {
#pragma unroll
      for (int i = 0; i < kXInst; ++i) {
        const int n = i * kXRowsPerInst + lane / kXLanesPerRow;
        *reinterpret_cast<u32x4 *>(myx + n * kXStride + (lane % kXLanesPerRow) * 16) = xl[i];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if constexpr (kXl) {
      /* operand order: batch row m, columns 64 jj + 8 g (and + 32) */
#pragma unroll
      for (int jj = 0; jj < kSteps; ++jj) {
        const int8_t *px = myx + m * kXStride + 128 * jj + 16 * g;
        xa[jj] = *reinterpret_cast<const u32x4 *>(px);
        xb[jj] = *reinterpret_cast<const u32x4 *>(px + 64);
      }
    }
#pragma unroll
    for (int jj = 0; jj < kSteps; ++jj) {
#pragma unroll
      for (int i = 0; i < kR; ++i) {
        const int8_t *p = my + (16 * i + m) * kStride + 64 * jj + 8 * g;
        const uint2 lo = *reinterpret_cast<const uint2 *>(p);
        const uint2 hi = *reinterpret_cast<const uint2 *>(p + 32);
        uint32_t wp[8];
        bytes_to_bf16x2(u32x4{lo.x, lo.y, hi.x, hi.y}, wp);
        acc[i] = mfma_bf16(wp, xa[jj], acc[i]);
        acc[i] = mfma_bf16(wp + 4, xb[jj], acc[i]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __syncthreads(); /* every wave is done with its tile */
  /* Accumulator lane l holds batch row l % 16 of rows 4 (l / 16) + q. */
#pragma unroll
  for (int i = 0; i < kR; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      red[wave][16 * i + 4 * g + q][m] = acc[i][q];
    }
  }
  __syncthreads();
  for (int i = t; i < kRows * nb; i += kW * 64) {
    const int rr = i % kRows, b = i / kRows;
    if (rr < my_rows) {
      float v = red[0][rr][b];
#pragma unroll
      for (int w = 1; w < kW; ++w) {
        v += red[w][rr][b];
      }
      Y[(int64_t)b * rows + r0 + rr] = scale[r0 + rr] * v;
    }
  }
}

/* Waves per workgroup and tile width of the 16-row kernel (kR = 1). Sweep
 * on the config-5 shapes at batches 4, 8 and 16: 4, 8 and 16 waves with
 * 128-, 256- and 512-column tiles all within 5% of each other. */
#ifndef VX_GEMV_LDS_W
#define VX_GEMV_LDS_W 8
#endif
#ifndef VX_GEMV_LDS_COLS
#define VX_GEMV_LDS_COLS 256
#endif
/* x through LDS (kXl above): batches of 8 and more on 16-row tiles whose
 * grid fits one round, and the 48-row tiles. */
#ifndef VX_GEMV_XLDS
#define VX_GEMV_XLDS 1
#endif

template <int kR>
void launch_lds(const int8_t *w, const float *s, const uint16_t *x, float *y,
                int rows, int cols, int nb, hipStream_t stream) {
  const int grid = (rows + 16 * kR - 1) / (16 * kR);
  constexpr int kW = kR == 1 ? VX_GEMV_LDS_W : 8;
  constexpr int kCols = kR == 1 ? VX_GEMV_LDS_COLS : 256;
  /* x through LDS, 128-column tiles: 16-row tiles (53 KiB of LDS) for
   * batches of 8 and more when the grid fits one round of the CUs; 48-row
   * tiles (88 KiB; the caller sends them only grids of one round) */
  if (VX_GEMV_XLDS && kR == 3) {
    hipLaunchKernelGGL((gemv_i8_lds<8, 128, 3, true>), dim3(grid), dim3(8 * 64), 0,
                       stream, w, s, x, y, rows, cols, nb);
  } else if (VX_GEMV_XLDS && kR == 1 && nb >= 8 && grid <= device_cu_count()) {
    hipLaunchKernelGGL((gemv_i8_lds<kW, 128, 1, true>), dim3(grid), dim3(kW * 64), 0,
                       stream, w, s, x, y, rows, cols, nb);
  } else {
    hipLaunchKernelGGL((gemv_i8_lds<kW, kCols, kR, false>), dim3(grid), dim3(kW * 64), 0,
                       stream, w, s, x, y, rows, cols, nb);
  }
}

/* Batches of 3 and 4: 8 rows per workgroup, 4 in flight per thread. A
 * workgroup loads its slice of x once and reuses it for all of its rows. */
void launch_b4(const int8_t *w, const float *s, const uint16_t *x, float *y,
               int rows, int cols, int nb, hipStream_t stream) {
  int grid = std::min(kMaxGrid, (rows + 7) / 8);
  grid = std::max(grid, (rows + kMaxRows - 1) / kMaxRows);
  hipLaunchKernelGGL((gemv_i8_kernel<4, 4>), dim3(grid), dim3(kThreads), 0,
                     stream, w, s, x, y, rows, cols, nb);
}

/* gemv_i8_rows with kR rows per workgroup; one load group covers up to three
 * 4096-column passes. Measured best: 4 rows for batch 1 (against 1, 2, 8 and
 * 16) and 16 for batch 2 (against 4 and 8): x costs the workgroup 2 * kB
 * bytes per column, the weights kR. */
/* Rows per workgroup at batch 1, for rows of at most kGroupCols columns and
 * for longer ones. */
#ifndef VX_GEMV_B1_R
#define VX_GEMV_B1_R 4
#endif
#ifndef VX_GEMV_B1_RLONG
#define VX_GEMV_B1_RLONG 4
#endif

template <int kB, int kR>
void launch_rows(const int8_t *w, const float *s, const uint16_t *x, float *y,
                 int rows, int cols, int nb, hipStream_t stream) {
  const dim3 grid((unsigned)((rows + kR - 1) / kR));
  if (cols <= kGroupCols) {
    hipLaunchKernelGGL((gemv_i8_rows<kB, kR, 1>), grid, dim3(kThreads), 0,
                       stream, w, s, x, y, rows, cols, nb);
  } else if (cols <= 2 * kGroupCols) {
    hipLaunchKernelGGL((gemv_i8_rows<kB, kR, 2>), grid, dim3(kThreads), 0,
                       stream, w, s, x, y, rows, cols, nb);
  } else {
    hipLaunchKernelGGL((gemv_i8_rows<kB, kR, 3>), grid, dim3(kThreads), 0,
                       stream, w, s, x, y, rows, cols, nb);
  }
}

std::atomic<int> forced_gemv{0};

/* Batches of 3 and more over 8192 rows and more go to 48-row MFMA tiles
 * with x through LDS while their grid fits one round of the CUs. */
bool tall_tiles(int rows, int nb) {
  return VX_GEMV_XLDS && nb >= 3 && rows >= 8192 && (rows + 47) / 48 <= device_cu_count();
}

/* The automatic choice, from sweeps of every kernel over 4096 x 4096,
 * 11008 x 4096 and 4096 x 11008: gemv_i8_rows (dot2; each workgroup one
 * burst of loads) for batch 1 at any width and batch 2 over at most 4096
 * columns; the grid-stride dot2 kernel, whose work per weight byte grows
 * with the batch but overlaps the stream, for batches 3 and 4 over at most
 * 4096 columns, except over 8192 rows and more, where 48-row MFMA tiles
 * with x through LDS take batches from 3 while their grid fits one round;
 * otherwise the MFMA kernel, whose cost beyond the weight stream is the x
 * operand, read once per 16 (or 48, or for batches of 8 and more over 8192
 * rows and more 64) rows. */
GemvKernel gemv_pick(int rows, int cols, int nb) {
  if (nb == 1 || (nb == 2 && cols <= kGroupCols)) {
    return GEMV_ROWS;
  }
  if (nb <= 4 && cols <= kGroupCols && !tall_tiles(rows, nb)) {
    return GEMV_DOT2_B4;
  }
  return GEMV_LDS;
}

} // namespace

void gemv_i8_force(GemvKernel which) { forced_gemv.store((int)which); }

bool gemv_i8_launch(const int8_t *w, const float *scale, const uint16_t *x,
                    float *y, int64_t rows, int64_t cols, int64_t batch,
                    hipStream_t stream) {
  /* Buffer ranges are 31-bit byte counts: 64 rows of W and all of x. */
  if (rows <= 0 || cols <= 0 || cols % 16 != 0 || rows > INT32_MAX ||
      cols > kGemvMaxCols || batch < 1 || batch > 16 ||
      (reinterpret_cast<uintptr_t>(w) & 15) ||
      (reinterpret_cast<uintptr_t>(x) & 15)) {
    return false;
  }
  const int r = (int)rows, c = (int)cols, nb = (int)batch;
  GemvKernel which = (GemvKernel)forced_gemv.load();
  if (which == GEMV_AUTO) {
    which = gemv_pick(r, c, nb);
  }
  switch (which) {
  case GEMV_ROWS:
    if (nb > 2) {
      return false;
    }
    if (nb == 1) {
      if (c > kGroupCols) {
        launch_rows<1, VX_GEMV_B1_RLONG>(w, scale, x, y, r, c, nb, stream);
      } else {
        launch_rows<1, VX_GEMV_B1_R>(w, scale, x, y, r, c, nb, stream);
      }
    } else {
      launch_rows<2, 16>(w, scale, x, y, r, c, nb, stream);
    }
    break;
  case GEMV_DOT2_B4:
    if (nb > 4 || c > kGroupCols) {
      return false;
    }
    launch_b4(w, scale, x, y, r, c, nb, stream);
    break;
  case GEMV_LDS:
    if (tall_tiles(r, nb)) {
      /* 48-row tiles, one round (one workgroup per CU) */
      launch_lds<3>(w, scale, x, y, r, c, nb, stream);
    } else if (nb >= 8 && r >= 8192) {
      launch_lds<4>(w, scale, x, y, r, c, nb, stream);
    } else {
      launch_lds<1>(w, scale, x, y, r, c, nb, stream);
    }
    break;
  default:
    return false;
  }
  VX_HIP_CHECK(hipGetLastError());
  return true;
}

} // namespace vxk
