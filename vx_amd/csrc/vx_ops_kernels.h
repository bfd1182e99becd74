/*
 * vx_ops_kernels.h -- launchers of the library-op kernels (ops.cpp calls
 * them after validating arguments). Each returns false for a shape or
 * alignment its kernel does not take, and launches nothing then.
 */
#ifndef VX_AMD_OPS_KERNELS_H
#define VX_AMD_OPS_KERNELS_H

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vxk {

/* Widest rows the GEMV kernels take: their buffer ranges (64 rows of w, all
 * of x) are 31-bit byte counts. */
constexpr int64_t kGemvMaxCols = int64_t(1) << 24;

/* The GEMV kernels; GEMV_AUTO picks by shape. */
enum GemvKernel {
  GEMV_AUTO = 0,
  GEMV_ROWS = 1,    /* one-burst row groups on v_dot2 (batch 1 and 2) */
  GEMV_DOT2_B4 = 2, /* grid-stride v_dot2 (batch up to 4, cols <= 4096) */
  GEMV_LDS = 3,     /* MFMA through per-wave LDS tiles, x from L2 */
};

/* Force one kernel (GEMV_AUTO: the automatic choice again). */
void gemv_i8_force(GemvKernel which);

/* y[b, r] = scale[r] * sum_c w[r, c] * x[b, c]; cols % 16 == 0 and at most
 * kGemvMaxCols, batch 1..16, w and x 16-byte aligned. False (nothing
 * launched) for a shape or alignment the chosen kernel does not take. */
bool gemv_i8_launch(const int8_t *w, const float *scale, const uint16_t *x,
                    float *y, int64_t rows, int64_t cols, int64_t batch,
                    hipStream_t stream);

/* Flash-attention forward; layout as include/vx_hip_ops.h. head_dim 64 or
 * 128, seq lengths >= 1. With `allow_split`, a launch whose query blocks
 * fill less than one round of the GPU cuts the key range into splits (their
 * partials in HBM taken in the stream's order) and merges them. */
bool flash_attn_fwd_launch(const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, uint16_t *o, float *lse,
                           int64_t batch, int64_t heads, int64_t kv_heads,
                           int64_t seq_q, int64_t seq_k, int64_t head_dim,
                           float scale, bool causal, bool allow_split,
                           hipStream_t stream);

/* Force the key splits of flash_attn_fwd_launch (0: the automatic choice;
 * a forced count applies where splitting is allowed). */
void flash_attn_force_splits(int splits);

/* Frees, in `stream`'s order, the key-split workspace kept for `stream` on
 * any device (nothing for the default stream or a stream that is capturing);
 * returns the blocks freed. The stream must still exist. */
int flash_attn_release_stream(hipStream_t stream);

/* Split workspaces currently held, and their bytes. */
void flash_attn_workspace_stats(int64_t *blocks, int64_t *bytes);

} // namespace vxk

#endif /* VX_AMD_OPS_KERNELS_H */
