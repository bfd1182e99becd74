/*
 * vx_kernels.h -- host-side launchers of the gfx950 kernels.
 *
 * Each launcher checks the shape its kernel assumes before it launches, and
 * returns false for a shape that kernel does not take; the caller then picks
 * another kernel or refuses. Nothing here allocates device memory except
 * where a launcher's comment says so.
 */
#ifndef VX_AMD_KERNELS_H
#define VX_AMD_KERNELS_H

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vxk {

/* C[m,n] = A[m,k] * B[k,n], row-major with row strides in elements.
 * `in_dtype` / `out_dtype` are VX_DTYPE_* codes: (f32,f32), (f64,f64),
 * (bf16|f16, same) or (bf16|f16, f32). */
struct GemmArgs {
  int32_t in_dtype, out_dtype;
  int64_t m, n, k;
  const void *a;
  const void *b;
  void *c;
  int64_t lda, ldb, ldc;
};

/* Which kernel a GEMM of this shape takes. */
enum GemmKernel {
  GEMM_NONE = 0,
  GEMM_MFMA_256 = 1, /* bf16/f16 MFMA 32x32x16, 256x256x64 tiles */
  GEMM_TILED = 2,    /* any supported type, 64x64 tiles, exact k order */
  GEMM_MFMA_PIPE4 = 3, /* as 1, software-pipelined, 4 waves */
  GEMM_MFMA_PIPE8 = 4, /* as 1, software-pipelined, 8 waves */
  GEMM_MFMA_IL = 5,    /* as 1, every non-MFMA instruction in MFMA shadow */
  GEMM_MFMA_DMA = 6,   /* as 1, global -> LDS direct, 4-deep ring of K=32 */
  GEMM_MFMA_DMA8 = 7,  /* as 6, 8 waves (two per SIMD) */
  GEMM_MFMA_PP = 8,    /* as 7 on 16x16x32 MFMAs, SIMD-sharing waves alternate */
  GEMM_F32_MFMA = 9,   /* f32 on 32x32x2 f32 MFMAs, 128x128 tiles */
};

inline bool gemm_is_mfma(GemmKernel k) {
  return k == GEMM_MFMA_256 || k == GEMM_MFMA_PIPE4 || k == GEMM_MFMA_PIPE8 ||
         k == GEMM_MFMA_IL || k == GEMM_MFMA_DMA ||
         k == GEMM_MFMA_DMA8 || k == GEMM_MFMA_PP || k == GEMM_F32_MFMA;
}

GemmKernel gemm_pick(const GemmArgs &g);
/* Whether one specific kernel takes the arguments. */
bool gemm_kernel_takes(GemmKernel which, const GemmArgs &g);
/* Launch; false when no kernel takes the arguments. */
bool gemm_launch(const GemmArgs &g, hipStream_t stream);
/* Launch one specific kernel; false when it does not take the arguments. */
bool gemm_launch_kernel(GemmKernel which, const GemmArgs &g,
                        hipStream_t stream);

/* *p = v on `stream` (one thread; a kernel rather than hipMemsetAsync so a
 * launch sequence stays capturable in a graph). */
void fill_i32_launch(int *p, int v, hipStream_t stream);

} // namespace vxk

#endif /* VX_AMD_KERNELS_H */
