/*
 * vx_hardware_runtime.h -- the Vx plugin C ABI, as the MI355X dispatch library
 * implements it.
 *
 * A compiled Vx program links exactly one dispatch library and calls the
 * `vx_plugin_*` entry points below directly. This header restates that
 * interface so that `libvx_hip_dispatch.so` is a drop-in for the CUDA or x86
 * library: every signature, constant, tag bit and payload rule here matches
 * the reference declaration it replaces (reference
 * include/vx_hardware_runtime.h; each block cites its lines). The inline
 * helpers are this project's own code implementing the same documented
 * behaviour, so a payload or descriptor the reference compiler wrote reads the
 * same way here.
 */
#ifndef VX_HARDWARE_RUNTIME_H
#define VX_HARDWARE_RUNTIME_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef __cplusplus
extern "C" {
#endif

/* What the program's machine model claimed about host access to the space a
 * transfer stages into (reference include/vx_hardware_runtime.h:23-34). */
typedef enum {
  VX_SPACE_ACCESS_UNKNOWN = 0,
  VX_SPACE_ACCESS_EXPLICIT = 1,
  VX_SPACE_ACCESS_HOST_READABLE = 2
} vx_space_access;

/* 1. Memory transfer (reference include/vx_hardware_runtime.h:43-51).
 * Allocates `bytes` in the memory of `topology_id` and copies `host_ptr` there
 * when it is not NULL. Topology 0, or no device, means host memory. */
void *vx_plugin_alloc_and_transfer(size_t bytes, void *host_ptr,
                                   uint32_t topology_id, uint32_t space_access);

/* As above for `transfer_async`: the copy may still run when this returns; each
 * later use of the result waits for it. */
void *vx_plugin_alloc_and_transfer_async(size_t bytes, void *host_ptr,
                                         uint32_t topology_id,
                                         uint32_t space_access);

/* Per-argument ABI tags (reference include/vx_hardware_runtime.h:53-88):
 *   bits  7..0   kind: 0 = memref descriptor, else the scalar's type code
 *   bits 15..8   element type code (memrefs)
 *   bits 23..16  rank (memrefs)
 *   bit  24      slot: the argument is storage holding a descriptor */
#define VX_ABI_KIND(tag) ((tag) & 0xFF)
#define VX_ABI_ELEM(tag) (((tag) >> 8) & 0xFF)
#define VX_ABI_RANK(tag) (((tag) >> 16) & 0xFF)
#define VX_ABI_IS_SLOT(tag) (((tag) >> 24) & 1)
#define VX_ABI_SLOT_BIT (1 << 24)
#define VX_ABI_MEMREF_TAG(elem, rank)                                          \
  (((int32_t)(rank) << 16) | ((int32_t)(elem) << 8))
#define VX_ABI_SLOT_TAG(elem, rank)                                            \
  (VX_ABI_SLOT_BIT | VX_ABI_MEMREF_TAG(elem, rank))

/* Largest rank a consumer must accept (reference :103). */
#define VX_ABI_MAX_RANK 8

/* Scalar kinds (reference :105-114). */
enum {
  VX_ABI_KIND_MEMREF = 0,
  VX_ABI_KIND_I1 = 1,
  VX_ABI_KIND_I8 = 2,
  VX_ABI_KIND_I16 = 3,
  VX_ABI_KIND_I32 = 4,
  VX_ABI_KIND_I64 = 5,
  VX_ABI_KIND_F32 = 6,
  VX_ABI_KIND_F64 = 7
};

/* Element type codes (reference :119-130). */
enum {
  VX_DTYPE_UNKNOWN = 0,
  VX_DTYPE_I1 = 1,
  VX_DTYPE_I8 = 2,
  VX_DTYPE_I16 = 3,
  VX_DTYPE_I32 = 4,
  VX_DTYPE_I64 = 5,
  VX_DTYPE_F32 = 6,
  VX_DTYPE_F64 = 7,
  VX_DTYPE_F16 = 8,
  VX_DTYPE_BF16 = 9
};

#define VX_DTYPE_MAX_BYTES 8

/* Bytes per element of a type code, 0 for a code with no size (reference
 * :137-155). */
static inline size_t vx_dtype_bytes(int32_t code) {
  static const unsigned char size_of[10] = {0, 1, 1, 2, 4, 8, 4, 8, 2, 2};
  return (code >= 0 && code < 10) ? (size_t)size_of[code] : 0;
}

/* Short name of a type code for diagnostics (reference :157-180). */
static inline const char *vx_dtype_name(int32_t code) {
  static const char *const names[10] = {"?",   "i1",  "i8",  "i16", "i32",
                                        "i64", "f32", "f64", "f16", "bf16"};
  return (code > 0 && code < 10) ? names[code] : "?";
}

/* A ranked memref descriptor is {allocated, aligned, offset, sizes[rank],
 * strides[rank]} (reference :182-212). */
static inline const int64_t *vx_memref_sizes(const void *desc) {
  return (const int64_t *)((const char *)desc + 2 * sizeof(void *) +
                           sizeof(int64_t));
}

static inline const int64_t *vx_memref_strides(const void *desc, int32_t rank) {
  return vx_memref_sizes(desc) + rank;
}

/* The aligned base pointer; for a slot, the descriptor the slot holds. */
static inline void *vx_memref_aligned(const void *desc) {
  return ((void *const *)desc)[1];
}

static inline int64_t vx_memref_offset(const void *desc) {
  return *(const int64_t *)((const char *)desc + 2 * sizeof(void *));
}

/* Address of element [0, ...] of the view: base + offset elements. */
static inline void *vx_memref_data(const void *desc, int32_t dtype) {
  return (char *)vx_memref_aligned(desc) +
         vx_memref_offset(desc) * (int64_t)vx_dtype_bytes(dtype);
}

/* Outcomes of vx_memref_view_span (reference :214-221). */
enum {
  VX_VIEW_OK = 0,
  VX_VIEW_UNKNOWN_ELEMENT,
  VX_VIEW_NEGATIVE,
  VX_VIEW_TOO_MANY_ELEMENTS,
  VX_VIEW_TOO_MANY_BYTES
};

/* Bytes from a view's first element to one past the last element it reaches,
 * (1 + sum((size[d]-1)*stride[d])) * element size, 0 when any size is 0
 * (reference :223-266). Prints nothing. */
static inline int vx_memref_view_span(const int64_t *sizes,
                                      const int64_t *strides, int32_t rank,
                                      int32_t elem, uint64_t *bytes,
                                      int32_t *dim) {
  uint64_t reach = 0, count = 0;
  int32_t d;
  size_t esz = vx_dtype_bytes(elem);
  if (esz == 0) {
    return VX_VIEW_UNKNOWN_ELEMENT;
  }
  for (d = 0; d < rank; ++d) {
    if (sizes[d] < 0 || strides[d] < 0) {
      *dim = d;
      return VX_VIEW_NEGATIVE;
    }
  }
  for (d = 0; d < rank; ++d) {
    if (sizes[d] == 0) {
      *bytes = 0;
      return VX_VIEW_OK;
    }
  }
  for (d = 0; d < rank; ++d) {
    uint64_t step;
    if (__builtin_mul_overflow((uint64_t)(sizes[d] - 1), (uint64_t)strides[d],
                               &step) ||
        __builtin_add_overflow(reach, step, &reach)) {
      return VX_VIEW_TOO_MANY_ELEMENTS;
    }
  }
  if (__builtin_add_overflow(reach, (uint64_t)1, &count)) {
    return VX_VIEW_TOO_MANY_ELEMENTS;
  }
  if (__builtin_mul_overflow(count, (uint64_t)esz, bytes)) {
    return VX_VIEW_TOO_MANY_BYTES;
  }
  return VX_VIEW_OK;
}

/* As vx_memref_view_span, stopping the program for a view with no byte size
 * (reference :268-312). */
static inline uint64_t vx_memref_view_bytes(const int64_t *sizes,
                                            const int64_t *strides,
                                            int32_t rank, int32_t elem) {
  uint64_t bytes = 0;
  int32_t d = 0;
  int why = vx_memref_view_span(sizes, strides, rank, elem, &bytes, &d);
  if (why == VX_VIEW_OK) {
    return bytes;
  }
  switch (why) {
  case VX_VIEW_UNKNOWN_ELEMENT:
    /* Code 0 is what the compiler writes for index and pointer elements. */
    fprintf(stderr,
            "[Vx] FATAL: no byte size is known for element type %d (index "
            "and pointer elements carry code 0), so a view of it cannot be "
            "copied\n",
            elem);
    break;
  case VX_VIEW_NEGATIVE:
    fprintf(stderr, "[Vx] FATAL: broken view descriptor: %s %lld in "
                    "dimension %d is below zero\n",
            sizes[d] < 0 ? "size" : "stride",
            (long long)(sizes[d] < 0 ? sizes[d] : strides[d]), d);
    break;
  case VX_VIEW_TOO_MANY_ELEMENTS:
    fprintf(stderr, "[Vx] FATAL: broken view descriptor: its element count "
                    "does not fit in 64 bits\n");
    break;
  default:
    fprintf(stderr, "[Vx] FATAL: broken view descriptor: its byte span does "
                    "not fit in 64 bits\n");
    break;
  }
  abort();
}

/* Write a dense row-major descriptor naming `data` (reference :314-341). */
static inline void vx_memref_write_desc(void *desc, void *data, int32_t rank,
                                        const int64_t *sizes) {
  void **base = (void **)desc;
  int64_t *fields = (int64_t *)((char *)desc + 2 * sizeof(void *));
  int64_t running = 1;
  int32_t d;
  base[0] = data;
  base[1] = data;
  fields[0] = 0;
  for (d = 0; d < rank; ++d) {
    fields[1 + d] = sizes[d];
  }
  for (d = rank - 1; d >= 0; --d) {
    fields[1 + rank + d] = running;
    running *= sizes[d];
  }
}

/* Payload layout (reference :343-475): the kernel name, then NUL-terminated
 * `key=value` entries; an empty entry ends the text part and a binary section
 * may follow it (u64 little-endian length, then the bytes).
 *
 * vx_payload_text_end: offset of the first byte after the text part. */
static inline size_t vx_payload_text_end(const void *payload,
                                         size_t payload_size) {
  const char *p = (const char *)payload;
  const char *nul;
  size_t at;
  if (!payload || payload_size == 0) {
    return 0;
  }
  nul = (const char *)memchr(p, '\0', payload_size);
  if (!nul) {
    return payload_size;
  }
  at = (size_t)(nul - p) + 1;
  while (at < payload_size) {
    nul = (const char *)memchr(p + at, '\0', payload_size - at);
    if (!nul) {
      return payload_size;
    }
    if (nul == p + at) {
      return at + 1; /* the empty entry */
    }
    at = (size_t)(nul - p) + 1;
  }
  return payload_size;
}

/* The value of entry `key` (which includes '='), or NULL when absent. An entry
 * equal to the key returns a pointer to its NUL, so present-but-empty differs
 * from absent. Size 0 means a producer predating entries: always absent. */
static inline const char *
vx_payload_field(const void *payload, size_t payload_size, const char *key) {
  const char *p = (const char *)payload;
  const char *nul;
  size_t klen, at;
  int terminated;
  if (!payload || payload_size == 0 || !key) {
    return NULL;
  }
  klen = strlen(key);
  terminated = p[payload_size - 1] == '\0';
  nul = (const char *)memchr(p, '\0', payload_size);
  if (!nul) {
    return NULL;
  }
  at = (size_t)(nul - p) + 1;
  while (at < payload_size) {
    const char *entry = p + at;
    size_t left = payload_size - at;
    size_t len;
    if (terminated && left > klen && memcmp(entry, key, klen) == 0) {
      return entry + klen;
    }
    nul = (const char *)memchr(entry, '\0', left);
    if (!nul) {
      return NULL;
    }
    len = (size_t)(nul - entry);
    if (len == 0) {
      return NULL; /* the section follows; its bytes are not keys */
    }
    if (len >= klen && memcmp(entry, key, klen) == 0) {
      return entry + klen;
    }
    at += len + 1;
  }
  return NULL;
}

/* Payload format version stamped as `abi=` (reference :477-484). */
#define VX_PAYLOAD_ABI 1

/* `abi=` as a number; -1 when absent, empty, not decimal, or out of range
 * (reference :486-509). */
static inline int32_t vx_payload_abi(const void *payload, size_t payload_size) {
  const char *v = vx_payload_field(payload, payload_size, "abi=");
  int64_t n = 0;
  if (!v || *v == '\0') {
    return -1;
  }
  for (; *v; ++v) {
    if (*v < '0' || *v > '9') {
      return -1;
    }
    n = n * 10 + (*v - '0');
    if (n > INT32_MAX) {
      return -1;
    }
  }
  return (int32_t)n;
}

/* The binary section: its length, with `*out` at its first byte; -1 no
 * section, -2 a length that does not account for the rest of the payload, -3
 * `out` NULL (reference :511-563). */
static inline int64_t
vx_payload_section(const void *payload, size_t payload_size, const void **out) {
  const unsigned char *sec;
  size_t start;
  uint64_t len = 0;
  int i;
  if (!out) {
    return -3;
  }
  if (!payload) {
    return -1;
  }
  start = vx_payload_text_end(payload, payload_size);
  if (start == payload_size) {
    return -1;
  }
  if (payload_size - start < 8) {
    return -2;
  }
  sec = (const unsigned char *)payload + start;
  for (i = 0; i < 8; ++i) {
    len |= (uint64_t)sec[i] << (8 * i);
  }
  if (len != payload_size - start - 8) {
    return -2;
  }
  *out = sec + 8;
  return (int64_t)len;
}

/* Topology id bands (reference :565-606). GPU[i] is 500 + i. */
#define VX_TOPO_CPU 0
#define VX_TOPO_NPU_BASE 100
#define VX_TOPO_ACCCORE_BASE 200
#define VX_TOPO_AMX 300
#define VX_TOPO_ANE 400
#define VX_TOPO_GPU_BASE 500
#define VX_TOPO_CPU_AVX512 600
#define VX_TOPO_CPU_NEON 700
#define VX_TOPO_NIC_BASE 800
#define VX_TOPO_REMOTE_BASE 900
#define VX_TOPO_SPIRV_BASE 1000
#define VX_TOPO_NUMA_BASE 1100
#define VX_TOPO_SLICE_BASE 2000
#define VX_TOPO_NAME_BASE 3000
#define VX_TOPO_BAND 100

/* Ordinal of `topology_id` within the band at `base`, -1 outside it
 * (reference :608-618). */
static inline int vx_topology_device_index(int32_t topology_id, int32_t base) {
  return (topology_id >= base && topology_id < base + VX_TOPO_BAND)
             ? (int)(topology_id - base)
             : -1;
}

/* NUMA node of an id, -1 when it names none (reference :620-629). */
static inline int vx_topology_numa_node(int32_t topology_id) {
  return (topology_id >= VX_TOPO_NUMA_BASE && topology_id < VX_TOPO_SLICE_BASE)
             ? (int)(topology_id - VX_TOPO_NUMA_BASE)
             : -1;
}

/* `topo=` as an integer, -1 when absent (reference :631-640). */
static inline int32_t vx_payload_topology(const void *payload,
                                          size_t payload_size) {
  const char *v = vx_payload_field(payload, payload_size, "topo=");
  if (!v || *v == '\0') {
    return -1;
  }
  return (int32_t)strtol(v, NULL, 10);
}

/* 2. Asynchronous execution (reference :642-650). `device_args[i]` points to
 * the i-th C-interface argument, `arg_tags[i]` is its tag. Returns a future id
 * at once. */
uint64_t vx_plugin_dispatch_async(const void *binary_payload,
                                  size_t payload_size, void **device_args,
                                  const int32_t *arg_tags, int64_t num_args);

/* 2.5 Flat f32 matvec xout[i] = sum_j w[i*n+j]*x[j], i < d (reference
 * :652-654). */
uint64_t vx_plugin_dispatch_async_flat(float *xout, float *x, float *w, int n,
                                       int d);

/* 3. Block until a dispatch has finished (reference :656-659). */
void vx_plugin_await_future(uint64_t future_id);

/* 4. Read-back, peer copy, free (reference :661-681). */
int32_t vx_plugin_transfer_device_to_host(void *device_ptr, void *host_ptr,
                                          size_t bytes, uint32_t topology_id);
void *vx_plugin_transfer_peer(void *src_device_ptr, uint32_t src_topology_id,
                              uint32_t dst_topology_id, size_t bytes);
void vx_plugin_free(void *device_ptr, uint32_t topology_id);

/* Arrival counts kept per launch site (reference :683-694). */
void *vx_plugin_arrivals_take(const void *site, size_t bytes, void *zeros,
                              uint32_t topology_id, uint32_t space_access);
void vx_plugin_arrivals_give(const void *site, void *count, size_t bytes,
                             uint32_t topology_id);

/* Release a future after its await (reference :696-697). */
void vx_plugin_release_future(uint64_t future_id);

/* 5. ioctl-style control (reference :699-741). */
int32_t vx_plugin_control(uint32_t opcode, void *payload);

#define VX_CTRL_INIT_DEVICE 0x01
#define VX_CTRL_SHUTDOWN 0x02
#define VX_CTRL_GET_DEVICE_COUNT 0x03
/* payload -> int32_t[2] {declared id, built-in id it stands for}. */
#define VX_CTRL_LOCAL_DEVICE 0x04
/* payload -> int32_t topology id. */
#define VX_CTRL_WAIT 0x05
/* payload -> vx_wait_for_tensors. */
#define VX_CTRL_WAIT_FOR_TENSORS 0x06
/* payload -> int32_t topology id. */
#define VX_CTRL_WAIT_FOR_THREAD 0x07
#define VX_CTRL_VENDOR_BASE 0x1000

typedef struct vx_wait_for_tensors {
  int32_t topology;
  int32_t count;
  void **args;
  const int32_t *tags;
} vx_wait_for_tensors;

/* Exported by every dispatch library so a host program links against any
 * build (reference runtime/host_dispatch_common.h:727-743). The tensor-map
 * entry answers 0: there is no TMA descriptor on AMD hardware. The stream
 * pair takes and gives a hipStream_t in the HIP library. */
int64_t vx_plugin_tensor_map(int64_t base, int64_t rank, int64_t elem_bytes,
                             int64_t d0, int64_t d1, int64_t d2, int64_t d3,
                             int64_t d4, int64_t s0, int64_t s1, int64_t s2,
                             int64_t s3, int64_t s4, int64_t b0, int64_t b1,
                             int64_t b2, int64_t b3, int64_t b4);
void vx_cuda_set_stream(void *stream);
void *vx_cuda_get_stream(void);

/* One-rank collectives (reference runtime/vx_collective_cpu.h,
 * runtime/cuda_dispatch.cpp:2064-2123; ABI in stdlib/std/collective.vx:14-29).
 * A job here has exactly one rank: each collective copies input to output. */
void vx_collective_init(int32_t rank, int32_t ranks);
void vx_collective_finish(void);
int32_t vx_collective_rank(void);
int32_t vx_collective_ranks(void);
void vx_collective_all_reduce_sum_f32(const float *input, float *output,
                                      int64_t count);
void vx_collective_all_reduce_sum_bf16(const uint16_t *input, uint16_t *output,
                                       int64_t count);
void vx_collective_all_gather_f32(const float *input, float *output,
                                  int64_t count);
void vx_collective_all_gather_bf16(const uint16_t *input, uint16_t *output,
                                   int64_t count);

/* Host worker identity inside an outlined host kernel (reference
 * runtime/vx_host_call.h:151-156). The HIP library runs a host fallback on
 * one worker, so these answer 0 of 1. */
int64_t vx_host_worker_id(void);
int64_t vx_host_worker_count(void);

#ifdef __cplusplus
}
#endif

#endif /* VX_HARDWARE_RUNTIME_H */
