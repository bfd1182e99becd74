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
  /* Where the MFMA kernel records its clock counters (4 x u64: shader clock
   * and real-time counter at the start and end of workgroup 0), or null. */
  uint64_t *stamp = nullptr;
  /* Whether the launch may take a workspace of its own (false under graph
   * capture and for the no-alloc entry point): the stream-K launch needs
   * one. */
  bool may_split = false;
};

/* Which kernel a GEMM of this shape takes. */
enum GemmKernel {
  GEMM_NONE = 0,
  GEMM_TILED = 2,   /* any supported type, 64x64 tiles, exact k order */
  GEMM_MFMA_PP = 8, /* bf16/f16 on 16x16x32 MFMAs, 256x256 tiles, direct-to-LDS
                       4-slot ring, the two waves of a SIMD taking turns */
  GEMM_F32_MFMA = 9, /* f32 on 32x32x2 f32 MFMAs, 128x128 tiles */
  GEMM_MFMA_SK = 10, /* the ping-pong tiles on one workgroup per CU, the second
                        round's tiles cut at half of K between two workgroups
                        (grids of 1 to 1.5 rounds; needs a workspace) */
};

inline bool gemm_is_mfma(GemmKernel k) {
  return k == GEMM_MFMA_PP || k == GEMM_F32_MFMA || k == GEMM_MFMA_SK;
}

GemmKernel gemm_pick(const GemmArgs &g);
/* Whether one specific kernel takes the arguments. */
bool gemm_kernel_takes(GemmKernel which, const GemmArgs &g);
/* Launch; false when no kernel takes the arguments. */
bool gemm_launch(const GemmArgs &g, hipStream_t stream);
/* Launch one specific kernel; false when it does not take the arguments. */
bool gemm_launch_kernel(GemmKernel which, const GemmArgs &g,
                        hipStream_t stream);

/* Frees, in `stream`'s order, the stream-K workspace kept for `stream` on
 * every device (none while it is capturing); the number freed. */
int gemm_release_stream(hipStream_t stream);
/* Stream-K workspaces held, their bytes, and stream-K launches so far. */
void gemm_workspace_stats(int64_t *blocks, int64_t *bytes, int64_t *launches);

/* *p = v on `stream` (one thread; a kernel rather than hipMemsetAsync so a
 * launch sequence stays capturable in a graph). */
void fill_i32_launch(int *p, int v, hipStream_t stream);

} // namespace vxk

#endif /* VX_AMD_KERNELS_H */
