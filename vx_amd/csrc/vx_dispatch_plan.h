/*
 * vx_dispatch_plan.h -- decode a vx_plugin_dispatch_async call into a GEMM.
 *
 * The compiler states everything a routed matmul needs: `kind=matmul` says the
 * region is fill(0) + matmul (reference src/dialect/VxLowering.cpp:347-402),
 * `roles=a:i,b:j,out:k` says which argument is which (:422-541), `outkind=`
 * says whether the result is a buffer to fill or a slot to publish through,
 * and each argument's tag gives its element type and rank. This header turns
 * those into a plan, or refuses; a refusal sends the dispatch to the outlined
 * kernel, so being strict costs speed and never correctness.
 *
 * Behaviour follows the reference decoder (runtime/vx_dispatch_plan.h:55-305)
 * refusal for refusal, with one widening the north star asks for: A and B in
 * bf16 (or f16) with an f32 result is accepted as a "mixed" plan. That is what
 * `matmul_into(&mut c_f32, &a_bf16, &b_bf16)` emits (reference
 * src/codegen/flat/emit/tensor.rs:1600-1647), and the reference decoder sends
 * it to the host loop nest instead.
 *
 * Vendor-free C so it is unit-tested on a machine with no GPU.
 */
#ifndef VX_AMD_DISPATCH_PLAN_H
#define VX_AMD_DISPATCH_PLAN_H

#include "../../include/vx_hardware_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { VX_GEMM_OUT_BUFFER = 0, VX_GEMM_OUT_SLOT = 1 };

/* Row-major C[m,n] = A[m,k] * B[k,n]; row strides in elements. */
typedef struct {
  int32_t dtype;     /* element type of A and B */
  int32_t out_dtype; /* element type of C: dtype, or f32 for a mixed plan */
  int64_t m, n, k;
  const void *a_data;
  const void *b_data;
  int64_t a_row_stride;
  int64_t b_row_stride;
  int32_t out_kind;
  void *out_data; /* NULL for a slot */
  int64_t out_row_stride;
  void *out_desc; /* descriptor storage to publish through; slot only */
} vx_gemm_plan;

/* Parse exactly `a:<i>,b:<j>,out:<k>` in any order, each role once, indices
 * non-negative decimal (reference runtime/vx_dispatch_plan.h:73-128). */
static inline int vx_parse_roles(const char *roles, int *a, int *b, int *out) {
  const char *p = roles;
  int seen = 0;
  if (!roles || !a || !b || !out) {
    return 0;
  }
  while (*p) {
    int *slot;
    int bit;
    long v;
    char *stop;
    if (strncmp(p, "a:", 2) == 0) {
      slot = a, bit = 1, p += 2;
    } else if (strncmp(p, "b:", 2) == 0) {
      slot = b, bit = 2, p += 2;
    } else if (strncmp(p, "out:", 4) == 0) {
      slot = out, bit = 4, p += 4;
    } else {
      return 0;
    }
    if (seen & bit) {
      return 0;
    }
    v = strtol(p, &stop, 10);
    if (stop == p || v < 0) {
      return 0;
    }
    *slot = (int)v;
    seen |= bit;
    p = stop;
    if (*p == ',') {
      ++p;
      if (*p == '\0') {
        return 0;
      }
    } else if (*p != '\0') {
      return 0;
    }
  }
  return seen == 7;
}

static inline int vx_gemm_dtype_supported(int32_t dtype) {
  return dtype == VX_DTYPE_F32 || dtype == VX_DTYPE_F64 ||
         dtype == VX_DTYPE_F16 || dtype == VX_DTYPE_BF16;
}

/* The pair (inputs, output) a routed GEMM may have: one supported type for all
 * three, or 16-bit inputs with an f32 result. */
static inline int vx_gemm_types_supported(int32_t in, int32_t b_in,
                                          int32_t out) {
  if (!vx_gemm_dtype_supported(in) || b_in != in) {
    return 0;
  }
  if (out == in) {
    return 1;
  }
  return (in == VX_DTYPE_BF16 || in == VX_DTYPE_F16) && out == VX_DTYPE_F32;
}

/* The descriptor an operand names: a slot argument holds one more level of
 * indirection (reference runtime/vx_dispatch_plan.h:138-149). */
static inline const void *vx_operand_desc(void **device_args,
                                          const int32_t *arg_tags, int idx) {
  const void *d = *(const void **)device_args[idx];
  if (d && VX_ABI_IS_SLOT(arg_tags[idx])) {
    d = vx_memref_aligned(d);
  }
  return d;
}

/* 1 and a filled plan when the dispatch is a GEMM this library can run, 0
 * otherwise (reference runtime/vx_dispatch_plan.h:157-295). */
static inline int vx_gemm_plan_decode(const void *payload, size_t payload_size,
                                      void **device_args,
                                      const int32_t *arg_tags, int64_t num_args,
                                      vx_gemm_plan *plan) {
  const char *kind, *roles, *outkind;
  int ai = -1, bi = -1, oi = -1;
  int32_t at, bt, ot, dt, odt;
  const void *ad, *bd, *od;
  const int64_t *asz, *bsz, *ast, *bst;

  if (!plan || !device_args || !arg_tags) {
    return 0;
  }
  kind = vx_payload_field(payload, payload_size, "kind=");
  if (!kind || strcmp(kind, "matmul") != 0) {
    return 0;
  }
  roles = vx_payload_field(payload, payload_size, "roles=");
  if (!vx_parse_roles(roles, &ai, &bi, &oi)) {
    return 0;
  }
  if (ai >= num_args || bi >= num_args || oi >= num_args || ai == bi ||
      ai == oi || bi == oi) {
    return 0;
  }
  outkind = vx_payload_field(payload, payload_size, "outkind=");
  if (!outkind) {
    return 0;
  }

  at = arg_tags[ai], bt = arg_tags[bi], ot = arg_tags[oi];
  if (VX_ABI_KIND(at) != VX_ABI_KIND_MEMREF ||
      VX_ABI_KIND(bt) != VX_ABI_KIND_MEMREF ||
      VX_ABI_KIND(ot) != VX_ABI_KIND_MEMREF) {
    return 0;
  }
  if (VX_ABI_RANK(at) != 2 || VX_ABI_RANK(bt) != 2 || VX_ABI_RANK(ot) != 2) {
    return 0;
  }
  dt = VX_ABI_ELEM(at);
  odt = VX_ABI_ELEM(ot);
  if (!vx_gemm_types_supported(dt, VX_ABI_ELEM(bt), odt)) {
    return 0;
  }

  ad = vx_operand_desc(device_args, arg_tags, ai);
  bd = vx_operand_desc(device_args, arg_tags, bi);
  od = vx_operand_desc(device_args, arg_tags, oi);
  if (!ad || !bd || !od) {
    return 0;
  }
  asz = vx_memref_sizes(ad), bsz = vx_memref_sizes(bd);
  ast = vx_memref_strides(ad, 2), bst = vx_memref_strides(bd, 2);
  if (ast[1] != 1 || bst[1] != 1) {
    return 0; /* rows must be contiguous */
  }
  if (asz[0] <= 0 || asz[1] <= 0 || bsz[1] <= 0 || bsz[0] != asz[1]) {
    return 0;
  }

  plan->dtype = dt;
  plan->out_dtype = odt;
  plan->m = asz[0];
  plan->k = asz[1];
  plan->n = bsz[1];
  plan->a_data = vx_memref_data(ad, dt);
  plan->b_data = vx_memref_data(bd, dt);
  plan->a_row_stride = ast[0];
  plan->b_row_stride = bst[0];
  plan->out_data = NULL;
  plan->out_desc = NULL;
  plan->out_row_stride = plan->n;

  if (strcmp(outkind, "slot") == 0) {
    if (!VX_ABI_IS_SLOT(ot)) {
      return 0; /* writing a descriptor needs storage for one */
    }
    plan->out_kind = VX_GEMM_OUT_SLOT;
    plan->out_desc = (void *)od;
  } else if (strcmp(outkind, "buffer") == 0) {
    const int64_t *osz = vx_memref_sizes(od);
    const int64_t *ost = vx_memref_strides(od, 2);
    if (ost[1] != 1 || osz[0] != plan->m || osz[1] != plan->n) {
      return 0;
    }
    plan->out_kind = VX_GEMM_OUT_BUFFER;
    plan->out_data = vx_memref_data(od, odt);
    plan->out_row_stride = ost[0];
    if (!plan->out_data) {
      return 0;
    }
  } else {
    return 0;
  }
  return plan->a_data && plan->b_data;
}

/* Publish a slot result: write a dense M x N descriptor naming `data` where
 * the kernel would have stored its own (reference :300-305). */
static inline void vx_gemm_publish_slot(const vx_gemm_plan *plan, void *data) {
  int64_t sizes[2];
  sizes[0] = plan->m;
  sizes[1] = plan->n;
  vx_memref_write_desc(plan->out_desc, data, 2, sizes);
}

#ifdef __cplusplus
}
#endif

#endif /* VX_AMD_DISPATCH_PLAN_H */
