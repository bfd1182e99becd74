/*
 * vx_hip_ops.h -- library ops of the MI355X dispatch library that have no
 * `kind=` route, called from Vx through `extern "C"` blocks.
 *
 * The reference has no flash-attention op and no int8 GEMV
 * (packages/vx_nn/lib.vx:1 is a placeholder; packages/README.md:10-19), and
 * the compiler has no AMDGPU image pipeline, so these ops are exported by the
 * dispatch library and declared in Vx the way `std::collective` declares its
 * entry points (reference stdlib/std/collective.vx:14-29,
 * runtime/cuda_dispatch.cpp:2064-2123). A tensor cannot cross an `extern`
 * (E3022, reference docs/lang/abi.md section 2), so every op takes element
 * pointers plus extents. Pointers are HBM allocations from
 * vx_plugin_alloc_and_transfer on Topology::GPU[i]; the op runs on the device
 * that owns them, on the calling thread's stream (vx_cuda_set_stream), and
 * returns before the GPU finishes, like a routed GEMM.
 *
 * Each op returns 0 on success and a negative VX_OP_E* code (with a
 * `[Vx HIP]` line on stderr) for arguments it cannot take. A device fault is
 * fatal, as everywhere in the plugin ABI.
 *
 * bf16 and f16 elements travel as uint16_t bit patterns.
 */
#ifndef VX_HIP_OPS_H
#define VX_HIP_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  VX_OP_OK = 0,
  VX_OP_EINVAL = -1,   /* an extent, stride or argument is out of range */
  VX_OP_ENODEV = -2,   /* no GPU: this library has no host copy of the op */
  VX_OP_ENOTDEV = -3,  /* a pointer is not device memory */
  VX_OP_EUNSUPP = -4   /* a shape the kernels do not take */
};

/* Flash-attention forward (the op packages/vx_nn/lib.vx declares).
 *
 * q: [batch, heads, seq_q, head_dim] bf16; k, v: [batch, kv_heads, seq_k,
 * head_dim] bf16; o: like q; lse: [batch, heads, seq_q] f32 (may be NULL).
 * All dense row-major. Query head h reads kv head h / (heads / kv_heads).
 * o = softmax(scale * q k^T) v with f32 accumulation, o rounded to bf16 once;
 * lse = natural-log sum of exp of the scaled scores of each row. With
 * `causal`, query i sees key j iff j <= i + (seq_k - seq_q) (the queries are
 * the last seq_q positions). head_dim must be 64 or 128. */
int32_t vx_nn_flash_attention_fwd_bf16(const uint16_t *q, const uint16_t *k,
                                       const uint16_t *v, uint16_t *o,
                                       float *lse, int64_t batch, int64_t heads,
                                       int64_t kv_heads, int64_t seq_q,
                                       int64_t seq_k, int64_t head_dim,
                                       float scale, int32_t causal);

/* int8 weight-only GEMV / skinny GEMM.
 *
 * w: [rows, cols] int8 row-major; scale: [rows] f32; x: [batch, cols] bf16;
 * y: [batch, rows] f32. y[b, r] = scale[r] * sum_c w[r, c] * x[b, c], the sum
 * in f32. batch 1..16; cols a multiple of 16. */
int32_t vx_nn_gemv_i8_bf16(const int8_t *w, const float *scale,
                           const uint16_t *x, float *y, int64_t rows,
                           int64_t cols, int64_t batch);

#ifdef __cplusplus
}
#endif

#endif /* VX_HIP_OPS_H */
