/*
 * ops.cpp -- the library ops of include/vx_hip_ops.h: argument checks, then
 * a launch on the caller stream.
 *
 * Checks happen on the host before any launch, so a kernel never sees a
 * shape it does not assume. There is no host copy of these ops: without a
 * GPU they answer VX_OP_ENODEV.
 */
#include "../../include/vx_hip_ops.h"
#include "vx_hip_common.h"
#include "vx_ops_internal.h"
#include "vx_ops_kernels.h"

#include <cmath>

namespace {

int32_t refuse(int32_t code, const char *op, const char *why) {
  fprintf(stderr, "[Vx HIP] %s: %s\n", op, why);
  return code;
}

bool all_on_device(std::initializer_list<const void *> ptrs) {
  for (const void *p : ptrs) {
    if (p && !vxops::on_device(p)) {
      return false;
    }
  }
  return true;
}

} // namespace

extern "C" {

int32_t vx_nn_gemv_i8_bf16(const int8_t *w, const float *scale,
                           const uint16_t *x, float *y, int64_t rows,
                           int64_t cols, int64_t batch) {
  static const char op[] = "vx_nn_gemv_i8_bf16";
  if (!vxops::device_present()) {
    return refuse(VX_OP_ENODEV, op, "no GPU; this op has no host copy");
  }
  if (!w || !scale || !x || !y) {
    return refuse(VX_OP_EINVAL, op, "a pointer is NULL");
  }
  if (rows <= 0 || cols <= 0 || batch < 1 || batch > 16) {
    return refuse(VX_OP_EINVAL, op, "rows and cols must be positive and "
                                    "batch in 1..16");
  }
  if (cols % 16 != 0) {
    return refuse(VX_OP_EUNSUPP, op, "cols must be a multiple of 16");
  }
  if (cols > vxk::kGemvMaxCols) {
    return refuse(VX_OP_EUNSUPP, op, "cols must be at most 2^24");
  }
  if (!all_on_device({w, scale, x, y})) {
    return refuse(VX_OP_ENOTDEV, op, "every operand must be GPU memory");
  }
  if (!vxk::gemv_i8_launch(w, scale, x, y, rows, cols, batch,
                           vxops::stream())) {
    return refuse(VX_OP_EUNSUPP, op,
                  "w and x must be 16-byte aligned (or a forced kernel does "
                  "not take this shape)");
  }
  vxops::launched(op);
  return VX_OP_OK;
}

int32_t vx_nn_flash_attention_fwd_bf16(const uint16_t *q, const uint16_t *k,
                                       const uint16_t *v, uint16_t *o,
                                       float *lse, int64_t batch, int64_t heads,
                                       int64_t kv_heads, int64_t seq_q,
                                       int64_t seq_k, int64_t head_dim,
                                       float scale, int32_t causal) {
  static const char op[] = "vx_nn_flash_attention_fwd_bf16";
  if (!vxops::device_present()) {
    return refuse(VX_OP_ENODEV, op, "no GPU; this op has no host copy");
  }
  if (!q || !k || !v || !o) {
    return refuse(VX_OP_EINVAL, op, "q, k, v and o must not be NULL");
  }
  if (batch < 1 || heads < 1 || kv_heads < 1 || seq_q < 1 || seq_k < 1 ||
      heads % kv_heads != 0 || !std::isfinite(scale)) {
    return refuse(VX_OP_EINVAL, op,
                  "extents must be positive, heads a multiple of kv_heads, "
                  "and scale finite");
  }
  if (head_dim != 64 && head_dim != 128) {
    return refuse(VX_OP_EUNSUPP, op, "head_dim must be 64 or 128");
  }
  if (batch * heads > INT32_MAX || seq_q > INT32_MAX || seq_k > INT32_MAX) {
    return refuse(VX_OP_EUNSUPP, op, "extents past 2^31");
  }
  if (!all_on_device({q, k, v, o, lse})) {
    return refuse(VX_OP_ENOTDEV, op, "every operand must be GPU memory");
  }
  /* Splitting takes HBM for the partials in the stream's order; a graph
   * being captured gets the unsplit launch. */
  if (!vxk::flash_attn_fwd_launch(q, k, v, o, lse, batch, heads, kv_heads,
                                  seq_q, seq_k, head_dim, scale, causal != 0,
                                  !vxops::capturing(), vxops::stream())) {
    return refuse(VX_OP_EUNSUPP, op, "operands must be 16-byte aligned");
  }
  vxops::launched(op);
  return VX_OP_OK;
}

} // extern "C"
