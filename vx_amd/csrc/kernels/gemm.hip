/*
 * gemm.hip -- the routed `a @ b` on gfx950.
 *
 * Two kernels:
 *
 *  - gemm_mfma_256: 16-bit inputs (bf16 or f16), f32 accumulate, f32 or
 *    16-bit output. One 256-thread workgroup (4 waves, 2x2) owns a 256x256
 *    tile of C and walks K in steps of 64. Each wave owns 128x128 of the tile
 *    as 4x4 v_mfma_f32_32x32x16 accumulators. A and B stages go through
 *    registers into a double-buffered LDS ring (2 x 64 KiB), one barrier per
 *    step. B arrives row-major (k-major), while the MFMA B operand wants
 *    8 consecutive k per lane, so each thread loads an 8x8 block of B and
 *    transposes it in registers before the LDS write; both LDS planes then
 *    hold 16-byte k-chunks per row, XOR-swizzled so ds_read_b128 of 16 rows
 *    at one k-chunk touch distinct banks. Workgroups are renumbered so that
 *    the 32 consecutive tiles each XCD receives form a 4x8 patch of C, which
 *    keeps each XCD's A and B panels in its own L2.
 *
 *  - gemm_tiled: every supported type pair, any shape and row stride. 64x64
 *    tiles, 16-deep K stages through LDS, one multiply and one add per term
 *    with contraction off, k in order: for f32 this is the same arithmetic,
 *    term for term, as the reference CPU loop nest
 *    (runtime/host_dispatch_common.h:65-79), and for bf16 -> f32 the same as
 *    the outlined linalg.matmul (extend, f32 multiply, f32 add, k sequential;
 *    src/codegen/flat/emit/tensor.rs:1600-1647).
 */
#include "../../../include/vx_hardware_runtime.h"
#include "../vx_hip_common.h"
#include "../vx_kernels.h"

#include <type_traits>

namespace vxk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileM = 256;
constexpr int kTileN = 256;
constexpr int kStageK = 64;
constexpr int kChunks = kStageK / 8; /* 16-byte k-chunks per LDS row */
constexpr int kThreads = 256;
constexpr int kGroupM = 4; /* tile rows per launch-order group */

/* Physical chunk of logical k-chunk `c` in LDS row `row`. A permutation of
 * 0..7 per row; 16 consecutive rows at one logical chunk land on 16 distinct
 * (row parity, chunk) pairs, so a 16-lane ds_read_b128 phase is conflict-free
 * whether the LDS is 32 or 64 banks wide. */
__device__ __forceinline__ int swz(int row, int c) {
  return c ^ (row & 7) ^ ((row >> 3) & 1);
}

template <bool kBf16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
        0);
  }
}

template <int kOut>
__device__ __forceinline__ void put(void *c, int64_t at, float v) {
  if constexpr (kOut == VX_DTYPE_F32) {
    static_cast<float *>(c)[at] = v;
  } else if constexpr (kOut == VX_DTYPE_BF16) {
    static_cast<uint16_t *>(c)[at] = f32_to_bf16(v);
  } else {
    static_cast<uint16_t *>(c)[at] = f32_to_f16(v);
  }
}

template <bool kBf16, int kOut>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_256(
    const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
    void *__restrict__ C, int K, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n) {
  __shared__ u32x4 lds[2][2][kTileM * kChunks]; /* [stage][A|B][row*8+chunk] */

  const int t = threadIdx.x;

  /* Launch order -> tile. Workgroup i runs on XCD i % 8; renumber so each
   * XCD's workgroups are consecutive, then walk tiles in groups of kGroupM
   * tile rows so consecutive numbers share A and B panels. */
  int id = blockIdx.x;
  const int nwg = gridDim.x;
  if ((nwg & 7) == 0) {
    id = (id & 7) * (nwg >> 3) + (id >> 3);
  }
  const int group_size = kGroupM * tiles_n;
  const int first_m = (id / group_size) * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int in_group = id % group_size;
  const int tm = first_m + in_group % rows_in_group;
  const int tn = in_group / rows_in_group;
  const int64_t m0 = (int64_t)tm * kTileM;
  const int64_t n0 = (int64_t)tn * kTileN;

  /* A stage: 8 passes of 32 rows x 8 chunks. */
  const uint16_t *a_src = A + (m0 + (t >> 3)) * lda + (t & 7) * 8;
  const int64_t a_pass = 32 * lda;
  /* B stage: thread owns the 8x8 block at k-chunk kc, n-block nb. */
  const int kc = t & 7;
  const int nb = t >> 3;
  const uint16_t *b_src = B + (int64_t)(kc * 8) * ldb + n0 + nb * 8;

  u32x4 areg[8], breg[8];

  auto fetch = [&](int step) {
    const uint16_t *ap = a_src + (int64_t)step * kStageK;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      areg[p] = *reinterpret_cast<const u32x4 *>(ap + p * a_pass);
    }
    const uint16_t *bp = b_src + (int64_t)step * kStageK * ldb;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      breg[r] = *reinterpret_cast<const u32x4 *>(bp + r * ldb);
    }
  };

  auto stash = [&](int s) {
    u32x4 *la = lds[s][0];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int row = p * 32 + (t >> 3);
      la[row * kChunks + swz(row, t & 7)] = areg[p];
    }
    /* 8x8 transpose: word w of row r holds columns 2w (low) and 2w+1 (high);
     * column j's k-chunk packs rows (2q, 2q+1) into word q. */
    u32x4 col[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t x = breg[2 * q][w];
        const uint32_t y = breg[2 * q + 1][w];
        col[2 * w][q] = (x & 0xffffu) | (y << 16);
        col[2 * w + 1][q] = (x >> 16) | (y & 0xffff0000u);
      }
    }
    u32x4 *lb = lds[s][1];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = nb * 8 + j;
      lb[row * kChunks + swz(row, kc)] = col[j];
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
      }
    }
  }

  const int wave = t >> 6;
  const int lane = t & 63;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int lrow = lane & 31;
  const int lk = lane >> 5;

  const int steps = K / kStageK;
  fetch(0);
  stash(0);
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int s = step & 1;
    if (step + 1 < steps) {
      fetch(step + 1);
    }
    const u32x4 *la = lds[s][0];
    const u32x4 *lb = lds[s][1];
#pragma unroll
    for (int ks = 0; ks < kStageK / 16; ++ks) {
      const int c = ks * 2 + lk;
      u32x4 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wm * 128 + i * 32 + lrow;
        af[i] = la[row * kChunks + swz(row, c)];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = wn * 128 + j * 32 + lrow;
        bfr[j] = lb[row * kChunks + swz(row, c)];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j] = mfma32<kBf16>(af[i], bfr[j], acc[i][j]);
        }
      }
    }
    if (step + 1 < steps) {
      stash(s ^ 1);
    }
    __syncthreads();
  }

  /* 32x32 accumulator layout: lane l, element r holds row
   * 8*(r/4) + 4*(l/32) + r%4, column l%32. */
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn * 128 + j * 32 + lrow;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row =
            m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        put<kOut>(C, row * ldc + col, acc[i][j][r]);
      }
    }
  }
}

/* Software-pipelined variant of the same 256x256x64 tile, for kWavesM x
 * kWavesN waves (4 = one wave per SIMD, 8 = two).
 *
 * Per stage (K step of 64) the wave walks 4 k-substeps of 16. The MFMA
 * operands of substep s+1 are read from LDS into a second register set
 * before the MFMAs of substep s issue (sched_barrier keeps that order), so
 * LDS latency hides behind MFMA work instead of stalling it. The global
 * loads of the stage after next are issued after substep 2 and land in
 * registers; they are written into the idle LDS buffer after substep 1 of
 * the following stage, leaving a whole stage for the loads to arrive. One
 * barrier per stage. B's 8-row blocks are kNB columns wide (8 for 256
 * threads, 4 for 512) so each thread owns exactly one block. */
template <int kWavesM, int kWavesN, bool kBf16, int kOut>
__global__ __launch_bounds__(64 * kWavesM * kWavesN, 1) void gemm_mfma_pipe(
    const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
    void *__restrict__ C, int K, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n) {
  constexpr int kT = 64 * kWavesM * kWavesN;
  constexpr int kTM = kTileM / kWavesM / 32; /* 32x32 tiles per wave in m */
  constexpr int kTN = kTileN / kWavesN / 32;
  constexpr int kALoads = kTileM * kChunks / kT;
  constexpr int kNB = kTileN * kChunks / kT; /* B block width: 8 or 4 */
  static_assert(kNB == 8 || kNB == 4, "one B block per thread");
  __shared__ u32x4 lds[2][2][kTileM * kChunks];

  const int t = threadIdx.x;
  int id = blockIdx.x;
  const int nwg = gridDim.x;
  if ((nwg & 7) == 0) {
    id = (id & 7) * (nwg >> 3) + (id >> 3);
  }
  const int group_size = kGroupM * tiles_n;
  const int first_m = (id / group_size) * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int in_group = id % group_size;
  const int tm = first_m + in_group % rows_in_group;
  const int tn = in_group / rows_in_group;
  const int64_t m0 = (int64_t)tm * kTileM;
  const int64_t n0 = (int64_t)tn * kTileN;

  const uint16_t *a_src = A + (m0 + (t >> 3)) * lda + (t & 7) * 8;
  const int64_t a_pass = (int64_t)(kT / 8) * lda;
  const int kc = t & 7;
  const int nb = t >> 3;
  const uint16_t *b_src = B + (int64_t)(kc * 8) * ldb + n0 + nb * kNB;

  using BRow = typename std::conditional<kNB == 8, u32x4, u32x2>::type;
  u32x4 areg[kALoads];
  BRow breg[8]; /* one row of the thread's 8 x kNB block of B */

  auto fetch = [&](int step) {
    const uint16_t *ap = a_src + (int64_t)step * kStageK;
#pragma unroll
    for (int p = 0; p < kALoads; ++p) {
      areg[p] = *reinterpret_cast<const u32x4 *>(ap + p * a_pass);
    }
    const uint16_t *bp = b_src + (int64_t)step * kStageK * ldb;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      breg[r] = *reinterpret_cast<const BRow *>(bp + r * ldb);
    }
  };

  auto stash = [&](int s) {
    u32x4 *la = lds[s][0];
#pragma unroll
    for (int p = 0; p < kALoads; ++p) {
      const int row = p * (kT / 8) + (t >> 3);
      la[row * kChunks + swz(row, t & 7)] = areg[p];
    }
    u32x4 *lb = lds[s][1];
#pragma unroll
    for (int w = 0; w < kNB / 2; ++w) {
      u32x4 lo, hi;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t x = breg[2 * q][w];
        const uint32_t y = breg[2 * q + 1][w];
        lo[q] = (x & 0xffffu) | (y << 16);
        hi[q] = (x >> 16) | (y & 0xffff0000u);
      }
      const int row = nb * kNB + 2 * w;
      lb[row * kChunks + swz(row, kc)] = lo;
      lb[(row + 1) * kChunks + swz(row + 1, kc)] = hi;
    }
  };

  f32x16 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
      }
    }
  }

  const int wave = t >> 6;
  const int lane = t & 63;
  const int wm = wave / kWavesN;
  const int wn = wave % kWavesN;
  const int lrow = lane & 31;
  const int lk = lane >> 5;
  const int a_row0 = wm * (kTileM / kWavesM) + lrow;
  const int b_row0 = wn * (kTileN / kWavesN) + lrow;

  u32x4 fa[2][kTM], fb[2][kTN];
  auto frags = [&](int s, int ks, u32x4 *af, u32x4 *bfr) {
    const u32x4 *la = lds[s][0];
    const u32x4 *lb = lds[s][1];
    const int c = ks * 2 + lk;
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      const int row = a_row0 + i * 32;
      af[i] = la[row * kChunks + swz(row, c)];
    }
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int row = b_row0 + j * 32;
      bfr[j] = lb[row * kChunks + swz(row, c)];
    }
  };

  const int steps = K / kStageK;
  fetch(0);
  stash(0);
  if (steps > 1) {
    fetch(1);
  }
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int s = step & 1;
    frags(s, 0, fa[0], fb[0]);
#pragma unroll
    for (int ks = 0; ks < kStageK / 16; ++ks) {
      if (ks + 1 < kStageK / 16) {
        frags(s, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kTM; ++i) {
#pragma unroll
        for (int j = 0; j < kTN; ++j) {
          acc[i][j] = mfma32<kBf16>(fa[ks & 1][i], fb[ks & 1][j], acc[i][j]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (ks == 1 && step + 1 < steps) {
        stash(s ^ 1);
      }
      if (ks == 2 && step + 2 < steps) {
        fetch(step + 2);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < kTM; ++i) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int64_t col = n0 + wn * (kTileN / kWavesN) + j * 32 + lrow;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * (kTileM / kWavesM) + i * 32 + 8 * (r >> 2) +
                            4 * lk + (r & 3);
        put<kOut>(C, row * ldc + col, acc[i][j][r]);
      }
    }
  }
}

template <int kIn>
__device__ __forceinline__ auto load_in(const void *p, int64_t at) {
  if constexpr (kIn == VX_DTYPE_F64) {
    return static_cast<const double *>(p)[at];
  } else if constexpr (kIn == VX_DTYPE_F32) {
    return static_cast<const float *>(p)[at];
  } else if constexpr (kIn == VX_DTYPE_BF16) {
    return bf16_to_f32(static_cast<const uint16_t *>(p)[at]);
  } else {
    return f16_to_f32(static_cast<const uint16_t *>(p)[at]);
  }
}

template <int kOut, typename Acc>
__device__ __forceinline__ void put_any(void *c, int64_t at, Acc v) {
  if constexpr (kOut == VX_DTYPE_F64) {
    static_cast<double *>(c)[at] = v;
  } else {
    put<kOut>(c, at, (float)v);
  }
}

template <int kIn, int kOut>
__global__ __launch_bounds__(256) void gemm_tiled(const void *__restrict__ A,
                                                  const void *__restrict__ B,
                                                  void *__restrict__ C,
                                                  int64_t M, int64_t N,
                                                  int64_t K, int64_t lda,
                                                  int64_t ldb, int64_t ldc) {
#pragma clang fp contract(off)
  using Acc = decltype(load_in<kIn>(nullptr, 0));
  __shared__ Acc As[16][65]; /* [k][m] */
  __shared__ Acc Bs[16][65]; /* [k][n] */
  const int t = threadIdx.x;
  const int tx = t & 15;
  const int ty = t >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * 64;
  const int64_t n0 = (int64_t)blockIdx.x * 64;
  Acc acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = Acc(0);
    }
  }
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = t + e * 256;
      const int am = idx >> 4, ak = idx & 15;
      const int64_t gm = m0 + am, gk = k0 + ak;
      As[ak][am] = (gm < M && gk < K) ? load_in<kIn>(A, gm * lda + gk) : Acc(0);
      const int bk = idx >> 6, bn = idx & 63;
      const int64_t hk = k0 + bk, hn = n0 + bn;
      Bs[bk][bn] = (hk < K && hn < N) ? load_in<kIn>(B, hk * ldb + hn) : Acc(0);
    }
    __syncthreads();
    const int kk_end = (K - k0) < 16 ? (int)(K - k0) : 16;
    for (int kk = 0; kk < kk_end; ++kk) {
      Acc a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = As[kk][ty * 4 + i];
        b[i] = Bs[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          Acc prod = a[i] * b[j];
          acc[i][j] = acc[i][j] + prod;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t gm = m0 + ty * 4 + i;
    if (gm >= M) {
      continue;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + tx * 4 + j;
      if (gn < N) {
        put_any<kOut>(C, gm * ldc + gn, acc[i][j]);
      }
    }
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

bool mfma_takes(const GemmArgs &g) {
  const bool sixteen = g.in_dtype == VX_DTYPE_BF16 || g.in_dtype == VX_DTYPE_F16;
  const bool out_ok = g.out_dtype == VX_DTYPE_F32 || g.out_dtype == g.in_dtype;
  return sixteen && out_ok && g.m > 0 && g.n > 0 && g.k > 0 &&
         g.m % kTileM == 0 && g.n % kTileN == 0 && g.k % kStageK == 0 &&
         g.k <= INT32_MAX && (g.m / kTileM) * (g.n / kTileN) <= INT32_MAX &&
         g.lda % 8 == 0 && g.ldb % 8 == 0 && g.lda >= g.k && g.ldb >= g.n &&
         g.ldc >= g.n && aligned16(g.a) && aligned16(g.b);
}

bool tiled_takes(const GemmArgs &g) {
  if (g.m <= 0 || g.n <= 0 || g.k <= 0 || g.lda < g.k || g.ldb < g.n ||
      g.ldc < g.n) {
    return false;
  }
  if ((g.m + 63) / 64 > 65535) {
    return false; /* grid.y limit */
  }
  switch (g.in_dtype) {
  case VX_DTYPE_F32:
  case VX_DTYPE_F64:
    return g.out_dtype == g.in_dtype;
  case VX_DTYPE_BF16:
  case VX_DTYPE_F16:
    return g.out_dtype == g.in_dtype || g.out_dtype == VX_DTYPE_F32;
  default:
    return false;
  }
}

template <bool kBf16, int kOut>
void launch_mfma(const GemmArgs &g, hipStream_t s) {
  const int tiles_m = (int)(g.m / kTileM), tiles_n = (int)(g.n / kTileN);
  hipLaunchKernelGGL((gemm_mfma_256<kBf16, kOut>), dim3(tiles_m * tiles_n),
                     dim3(kThreads), 0, s, static_cast<const uint16_t *>(g.a),
                     static_cast<const uint16_t *>(g.b), g.c, (int)g.k, g.lda,
                     g.ldb, g.ldc, tiles_m, tiles_n);
}

template <int kWM, int kWN, bool kBf16, int kOut>
void launch_pipe(const GemmArgs &g, hipStream_t s) {
  const int tiles_m = (int)(g.m / kTileM), tiles_n = (int)(g.n / kTileN);
  hipLaunchKernelGGL((gemm_mfma_pipe<kWM, kWN, kBf16, kOut>),
                     dim3(tiles_m * tiles_n), dim3(64 * kWM * kWN), 0, s,
                     static_cast<const uint16_t *>(g.a),
                     static_cast<const uint16_t *>(g.b), g.c, (int)g.k, g.lda,
                     g.ldb, g.ldc, tiles_m, tiles_n);
}

template <int kWM, int kWN>
void launch_pipe_any(const GemmArgs &g, hipStream_t s) {
  const bool bf = g.in_dtype == VX_DTYPE_BF16;
  if (g.out_dtype == VX_DTYPE_F32) {
    bf ? launch_pipe<kWM, kWN, true, VX_DTYPE_F32>(g, s)
       : launch_pipe<kWM, kWN, false, VX_DTYPE_F32>(g, s);
  } else if (bf) {
    launch_pipe<kWM, kWN, true, VX_DTYPE_BF16>(g, s);
  } else {
    launch_pipe<kWM, kWN, false, VX_DTYPE_F16>(g, s);
  }
}

template <int kIn, int kOut>
void launch_tiled(const GemmArgs &g, hipStream_t s) {
  dim3 grid((unsigned)((g.n + 63) / 64), (unsigned)((g.m + 63) / 64));
  hipLaunchKernelGGL((gemm_tiled<kIn, kOut>), grid, dim3(256), 0, s, g.a, g.b,
                     g.c, g.m, g.n, g.k, g.lda, g.ldb, g.ldc);
}

} // namespace

GemmKernel gemm_pick(const GemmArgs &g) {
  if (mfma_takes(g)) {
    return GEMM_MFMA_PIPE4;
  }
  if (tiled_takes(g)) {
    return GEMM_TILED;
  }
  return GEMM_NONE;
}

bool gemm_launch_kernel(GemmKernel which, const GemmArgs &g,
                        hipStream_t stream) {
  if (which == GEMM_MFMA_256) {
    if (!mfma_takes(g)) {
      return false;
    }
    const bool bf = g.in_dtype == VX_DTYPE_BF16;
    if (g.out_dtype == VX_DTYPE_F32) {
      bf ? launch_mfma<true, VX_DTYPE_F32>(g, stream)
         : launch_mfma<false, VX_DTYPE_F32>(g, stream);
    } else if (bf) {
      launch_mfma<true, VX_DTYPE_BF16>(g, stream);
    } else {
      launch_mfma<false, VX_DTYPE_F16>(g, stream);
    }
  } else if (which == GEMM_MFMA_PIPE4 || which == GEMM_MFMA_PIPE8) {
    if (!mfma_takes(g)) {
      return false;
    }
    which == GEMM_MFMA_PIPE4 ? launch_pipe_any<2, 2>(g, stream)
                             : launch_pipe_any<2, 4>(g, stream);
  } else if (which == GEMM_TILED) {
    if (!tiled_takes(g)) {
      return false;
    }
    switch (g.in_dtype) {
    case VX_DTYPE_F32:
      launch_tiled<VX_DTYPE_F32, VX_DTYPE_F32>(g, stream);
      break;
    case VX_DTYPE_F64:
      launch_tiled<VX_DTYPE_F64, VX_DTYPE_F64>(g, stream);
      break;
    case VX_DTYPE_BF16:
      g.out_dtype == VX_DTYPE_F32
          ? launch_tiled<VX_DTYPE_BF16, VX_DTYPE_F32>(g, stream)
          : launch_tiled<VX_DTYPE_BF16, VX_DTYPE_BF16>(g, stream);
      break;
    default:
      g.out_dtype == VX_DTYPE_F32
          ? launch_tiled<VX_DTYPE_F16, VX_DTYPE_F32>(g, stream)
          : launch_tiled<VX_DTYPE_F16, VX_DTYPE_F16>(g, stream);
      break;
    }
  } else {
    return false;
  }
  VX_HIP_CHECK(hipGetLastError());
  return true;
}

bool gemm_launch(const GemmArgs &g, hipStream_t stream) {
  return gemm_launch_kernel(gemm_pick(g), g, stream);
}

} // namespace vxk
