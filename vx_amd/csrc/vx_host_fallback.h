/*
 * vx_host_fallback.h -- run a dispatch the GPU does not take on the host.
 *
 * A region the compiler did not classify as `kind=matmul`, and that carries no
 * device image this library can load (the compiler has no AMDGPU image
 * pipeline: reference src/dialect/VxLowering.cpp:6522-6534), runs as its
 * outlined host kernel `_vx_ciface_<name>`, called through libffi with the
 * calling convention rebuilt from the tags (reference
 * runtime/vx_host_call.h:60-130, :323-383).
 *
 * Operands in HBM are copied to host memory for the call and back afterwards
 * (reference runtime/cuda_dispatch.cpp:1733-1860, runtime/vx_view_copy.h).
 * Two arguments can be views of the same bytes -- one tensor passed as the
 * output and as an input, or two overlapping row ranges -- and the call must
 * see one copy of those bytes, or the copy back of the stale view would land
 * over the result in the other. So the views are planned into spans:
 *
 *  - views whose byte ranges overlap join one span, copied once each way,
 *    and keep their strides inside the span's copy;
 *  - a view alone in its span whose elements take fewer bytes than its span
 *    (a column of a matrix) is copied densely instead, and the call sees it
 *    with row-major strides;
 *  - an empty view is passed through untouched (nothing reads it).
 *
 * The caller's descriptors are never modified: the call sees private
 * descriptors that point into the copies. A result the region publishes
 * through a slot is handed back with its pointers translated from a copy to
 * the HBM it stands for.
 *
 * `launch=` and `host_blocks=` regions were proven by the compiler to have
 * disjoint iterations; they run on several host threads, each reading its
 * slice from vx_host_worker_id / vx_host_worker_count (reference
 * runtime/vx_host_call.h:132-238, `VX_HOST_THREADS`).
 *
 * Vendor-free: the copies go through the HostCopies hooks, so the planner and
 * the call run in a CPU-only unit test (tests/native/host_fallback_test.cpp).
 *
 * This is the reference ABI's behaviour for unroutable regions, not a second
 * path for the routed ops: a routed GEMM that the GPU cannot run is refused
 * loudly by the dispatch library instead of landing here.
 */
#ifndef VX_AMD_HOST_FALLBACK_H
#define VX_AMD_HOST_FALLBACK_H

#include "../../include/vx_hardware_runtime.h"
#include "vx_image_launch.h"

#include <dlfcn.h>
#include <ffi.h>
#include <pthread.h>
#include <sched.h>
#include <xmmintrin.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <functional>
#include <vector>

namespace vx {

inline ffi_type *ffi_type_for_tag(int32_t tag) {
  switch (VX_ABI_KIND(tag)) {
  case VX_ABI_KIND_I1:
    return &ffi_type_uint8;
  case VX_ABI_KIND_I8:
    return &ffi_type_sint8;
  case VX_ABI_KIND_I16:
    return &ffi_type_sint16;
  case VX_ABI_KIND_I32:
    return &ffi_type_sint32;
  case VX_ABI_KIND_I64:
    return &ffi_type_sint64;
  case VX_ABI_KIND_F32:
    return &ffi_type_float;
  case VX_ABI_KIND_F64:
    return &ffi_type_double;
  default:
    return &ffi_type_pointer;
  }
}

/* `_vx_ciface_<name>`, looked up first in the library holding the payload
 * (every library numbers its kernels from 0), then globally. */
inline void *host_kernel_symbol(const char *kernel_name) {
  char sym[256];
  snprintf(sym, sizeof(sym), "_vx_ciface_%s", kernel_name);
  Dl_info info;
  if (dladdr(kernel_name, &info) && info.dli_fname) {
    void *lib = dlopen(info.dli_fname, RTLD_LAZY | RTLD_NOLOAD);
    if (lib) {
      void *fn = dlsym(lib, sym);
      dlclose(lib);
      if (fn) {
        return fn;
      }
    }
  }
  return dlsym(RTLD_DEFAULT, sym);
}

/* ---- host workers ---- */

/* The slice of a split region the calling thread runs: worker `index` of
 * `total`. A thread that never ran a split region reads 0 of 1, the whole
 * range. */
inline thread_local int64_t host_worker_index = 0;
inline thread_local int64_t host_worker_total = 1;

/* How many host threads a region runs on. 1 unless the payload proves the
 * region splits: `launch=<trip>` (one level; the two-level `launch=B,T` is
 * not split) or `host_blocks=` with a `grid=`, whose x axis is the block
 * count. Then `VX_HOST_THREADS` if set (below 1: serial), else the CPUs this
 * thread may run on, never more than the trip count. */
inline int host_worker_count_for(const void *payload, size_t payload_size,
                                 void *const *args, const int32_t *tags,
                                 int64_t num_args) {
  long trip = 0;
  if (vx_payload_field(payload, payload_size, "launch=")) {
    long threads = 0;
    trip = image_launch_trip(payload, payload_size, args, tags, num_args,
                             &threads);
    if (threads != 0) {
      return 1;
    }
  } else if (vx_payload_field(payload, payload_size, "host_blocks=")) {
    unsigned grid[3] = {1, 1, 1}, block = 1;
    char why[160];
    if (image_launch_shape(payload, payload_size, args, tags, num_args, grid,
                           &block, why, sizeof why) != 1) {
      return 1;
    }
    trip = (long)grid[0];
  } else {
    return 1;
  }
  if (trip <= 1) {
    return 1;
  }
  long want;
  if (const char *env = getenv("VX_HOST_THREADS")) {
    want = strtol(env, nullptr, 10);
    if (want < 1) {
      return 1;
    }
  } else {
    cpu_set_t set;
    CPU_ZERO(&set);
    want = sched_getaffinity(0, sizeof set, &set) == 0 ? CPU_COUNT(&set) : 1;
    if (want < 1) {
      want = 1;
    }
  }
  return (int)(want < trip ? want : trip);
}

/* A payload built for the Apple GPU (`format=msl`) flushes subnormal f32 to
 * zero there, so its host copy must too (reference
 * runtime/vx_host_call.h:240-245). */
inline bool host_flushes_subnormals(const void *payload, size_t payload_size) {
  const char *format = vx_payload_field(payload, payload_size, "format=");
  return format && strcmp(format, "msl") == 0;
}

struct HostWorker {
  ffi_cif *cif;
  void *kernel;
  void **args;
  int64_t index, total;
  bool flush;
};

inline void host_worker_run(const HostWorker &w) {
  host_worker_index = w.index;
  host_worker_total = w.total;
  void (*fn)(void) = reinterpret_cast<void (*)(void)>(w.kernel);
  if (w.flush) {
    /* FTZ (bit 15) and DAZ (bit 6) of MXCSR, for this call only. */
    const unsigned csr = _mm_getcsr();
    _mm_setcsr(csr | 0x8040u);
    ffi_call(w.cif, fn, nullptr, w.args);
    _mm_setcsr(csr);
  } else {
    ffi_call(w.cif, fn, nullptr, w.args);
  }
  host_worker_index = 0;
  host_worker_total = 1;
}

inline void *host_worker_thread(void *p) {
  host_worker_run(*static_cast<HostWorker *>(p));
  return nullptr;
}

/* Run the prepared call on `workers` threads (the caller's thread is worker
 * 0). A thread that cannot be created has its slice run here instead: a
 * slice nobody runs would leave a hole in the result. */
inline void host_call_split(ffi_cif *cif, void *kernel, void **args,
                            int workers, bool flush) {
  if (workers <= 1) {
    host_worker_run(HostWorker{cif, kernel, args, 0, 1, flush});
    return;
  }
  std::vector<HostWorker> jobs((size_t)workers);
  std::vector<pthread_t> threads((size_t)workers);
  std::vector<char> started((size_t)workers, 0);
  for (int w = 0; w < workers; ++w) {
    jobs[(size_t)w] = HostWorker{cif, kernel, args, w, workers, flush};
  }
  for (int w = 1; w < workers; ++w) {
    if (pthread_create(&threads[(size_t)w], nullptr, host_worker_thread,
                       &jobs[(size_t)w]) == 0) {
      started[(size_t)w] = 1;
    } else {
      host_worker_run(jobs[(size_t)w]);
    }
  }
  host_worker_run(jobs[0]);
  for (int w = 1; w < workers; ++w) {
    if (started[(size_t)w]) {
      pthread_join(threads[(size_t)w], nullptr);
    }
  }
}

/* ---- copies of HBM views ---- */

/* Copy hooks. `is_device` says whether an address is HBM. `sync` runs once
 * before the first copy out of HBM (kernels still writing it must finish).
 * The 2-D copies move `height` runs of `width` bytes, `dpitch`/`spitch`
 * bytes apart at the destination/source. */
struct HostCopies {
  std::function<bool(const void *)> is_device;
  std::function<void()> sync;
  std::function<void(void *dst, size_t dpitch, const void *src, size_t spitch,
                     size_t width, size_t height)>
      to_host;
  std::function<void(void *dst, size_t dpitch, const void *src, size_t spitch,
                     size_t width, size_t height)>
      to_device;
};

/* One HBM view an argument hands the call. */
struct HbmView {
  const void *desc = nullptr; /* the caller's descriptor (read only) */
  int32_t rank = 0, elem = 0;
  int64_t arg = -1;
  /* planned */
  uintptr_t first = 0; /* address of the view's first element */
  uint64_t bytes = 0;  /* bytes from its first element to its last; 0 empty */
  int64_t span = -1;   /* its span, -1 for an empty view */
  uint64_t at = 0;     /* where the view starts in its span's copy */
  bool dense = false;  /* it has its span to itself, copied densely */
};

/* Bytes copied as one block: every byte of its views' ranges, or for a
 * dense span the elements of its one view in row-major order. */
struct HbmSpan {
  uintptr_t first = 0;
  uint64_t bytes = 0;
  int64_t dense_view = -1;
  std::vector<unsigned char> copy;
};

/* Whether view `v` reaches each of its elements once with positive strides
 * (so a dense copy can stand for it), and its dense byte count. */
inline bool view_packs(const HbmView &v, uint64_t *dense) {
  const int64_t *sizes = vx_memref_sizes(v.desc);
  const int64_t *strides = vx_memref_strides(v.desc, v.rank);
  struct Dim {
    int64_t size, stride;
  } dims[VX_ABI_MAX_RANK];
  int n = 0;
  uint64_t count = 1;
  for (int32_t d = 0; d < v.rank; ++d) {
    count *= (uint64_t)sizes[d];
    if (sizes[d] > 1) {
      if (strides[d] <= 0) {
        return false;
      }
      dims[n++] = Dim{sizes[d], strides[d]};
    }
  }
  std::sort(dims, dims + n,
            [](const Dim &a, const Dim &b) { return a.stride < b.stride; });
  /* Walking out from the smallest stride, each dimension's step must clear
   * the whole extent of the ones inside it. */
  for (int i = 1; i < n; ++i) {
    if (dims[i].stride < dims[i - 1].stride * dims[i - 1].size) {
      return false;
    }
  }
  *dense = count * vx_dtype_bytes(v.elem);
  return true;
}

/* Plan the spans of `views`. False, with the view's index in `*bad`, for a
 * view whose offset is negative or whose bytes leave the address space. */
inline bool plan_spans(std::vector<HbmView> &views, std::vector<HbmSpan> &spans,
                       size_t *bad) {
  spans.clear();
  std::vector<size_t> order;
  for (size_t i = 0; i < views.size(); ++i) {
    HbmView &v = views[i];
    v.span = -1;
    v.at = 0;
    v.dense = false;
    v.bytes = vx_memref_view_bytes(vx_memref_sizes(v.desc),
                                   vx_memref_strides(v.desc, v.rank), v.rank,
                                   v.elem);
    if (v.bytes == 0) {
      continue;
    }
    const int64_t offset = vx_memref_offset(v.desc);
    uint64_t first = 0, end = 0;
    if (offset < 0 ||
        __builtin_mul_overflow((uint64_t)offset,
                               (uint64_t)vx_dtype_bytes(v.elem), &first) ||
        __builtin_add_overflow(
            (uint64_t)(uintptr_t)vx_memref_aligned(v.desc), first, &first) ||
        __builtin_add_overflow(first, v.bytes, &end) ||
        end > (uint64_t)UINTPTR_MAX) {
      *bad = i;
      return false;
    }
    v.first = (uintptr_t)first;
    order.push_back(i);
  }
  /* By first byte; a view joins the open span when it starts before that
   * span's end (byte ranges that merely touch stay apart). */
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
    return views[a].first < views[b].first;
  });
  for (size_t i : order) {
    HbmView &v = views[i];
    const uint64_t end = (uint64_t)v.first + v.bytes;
    if (!spans.empty() &&
        (uint64_t)v.first < (uint64_t)spans.back().first + spans.back().bytes) {
      HbmSpan &s = spans.back();
      const uint64_t s_end = (uint64_t)s.first + s.bytes;
      s.bytes = (end > s_end ? end : s_end) - s.first;
    } else {
      HbmSpan s;
      s.first = v.first;
      s.bytes = v.bytes;
      spans.push_back(std::move(s));
    }
    v.span = (int64_t)spans.size() - 1;
  }
  std::vector<int64_t> members(spans.size(), 0);
  for (HbmView &v : views) {
    if (v.span >= 0) {
      v.at = v.first - spans[(size_t)v.span].first;
      ++members[(size_t)v.span];
    }
  }
  for (size_t i : order) {
    HbmView &v = views[i];
    uint64_t dense = 0;
    if (members[(size_t)v.span] == 1 && view_packs(v, &dense) &&
        dense < v.bytes) {
      v.dense = true;
      v.at = 0;
      spans[(size_t)v.span].bytes = dense;
      spans[(size_t)v.span].dense_view = (int64_t)i;
    }
  }
  return true;
}

/* The dense copy of a view in row-major order of its own dimensions, as
 * blocks: each block is `height` runs of `width` bytes, `pitch` bytes apart
 * in HBM, back to back from byte `dense` of the copy. */
template <typename Fn> void for_each_dense_block(const HbmView &v, Fn &&fn) {
  const int64_t *sizes = vx_memref_sizes(v.desc);
  const int64_t *strides = vx_memref_strides(v.desc, v.rank);
  const uint64_t esz = vx_dtype_bytes(v.elem);
  int32_t dims[VX_ABI_MAX_RANK];
  int32_t n = 0;
  for (int32_t d = 0; d < v.rank; ++d) {
    if (sizes[d] > 1) {
      dims[n++] = d;
    }
  }
  if (n == 0) {
    fn((uint64_t)0, v.first, esz, esz, (uint64_t)1);
    return;
  }
  /* The innermost dimension is one run when its stride is 1; the block's
   * rows step along the next one out. */
  uint64_t width = esz;
  int32_t row = n - 1;
  if (strides[dims[n - 1]] == 1) {
    width = (uint64_t)sizes[dims[n - 1]] * esz;
    row = n - 2;
  }
  uint64_t height = 1, pitch = width;
  if (row >= 0) {
    height = (uint64_t)sizes[dims[row]];
    pitch = (uint64_t)strides[dims[row]] * esz;
  }
  int64_t idx[VX_ABI_MAX_RANK] = {0};
  uint64_t dense = 0;
  for (;;) {
    uint64_t off = 0;
    for (int32_t k = 0; k < row; ++k) {
      off += (uint64_t)idx[k] * (uint64_t)strides[dims[k]] * esz;
    }
    fn(dense, v.first + (uintptr_t)off, width, height == 1 ? width : pitch,
       height);
    dense += width * height;
    int32_t k = row - 1;
    for (; k >= 0; --k) {
      if (++idx[k] < sizes[dims[k]]) {
        break;
      }
      idx[k] = 0;
    }
    if (k < 0) {
      return;
    }
  }
}

/* Row-major stride of dimension d of a view with `sizes`. */
inline int64_t dense_stride(const int64_t *sizes, int32_t rank, int32_t d) {
  int64_t s = 1;
  for (int32_t k = rank - 1; k > d; --k) {
    s *= sizes[k];
  }
  return s;
}

/* A private descriptor the call sees for view `v`: its span copy's address,
 * offset 0, and row-major strides for a dense copy. */
inline void point_into_copy(const HbmView &v, const HbmSpan &s,
                            std::vector<int64_t> &desc) {
  const size_t words = 3 + 2 * (size_t)v.rank;
  desc.assign(words, 0);
  memcpy(desc.data(), v.desc, words * sizeof(int64_t));
  void *at = const_cast<unsigned char *>(s.copy.data()) + v.at;
  void **ptrs = reinterpret_cast<void **>(desc.data());
  ptrs[0] = at;
  ptrs[1] = at;
  desc[2] = 0;
  if (v.dense) {
    const int64_t *sizes = vx_memref_sizes(v.desc);
    for (int32_t d = 0; d < v.rank; ++d) {
      desc[3 + (size_t)v.rank + (size_t)d] = dense_stride(sizes, v.rank, d);
    }
  }
}

/* Re-express a descriptor that points into the dense copy of `v` (element
 * offset `*offset` from the copy's start, `rank` dimensions of `sizes` and
 * `strides` in dense units) in the view's own layout. Exact or false: each
 * published dimension must step along one dimension of the view by a whole
 * multiple of its dense stride, and stay inside it. */
inline bool dense_to_view(const HbmView &v, int64_t *offset,
                          const int64_t *sizes, int64_t *strides,
                          int32_t rank) {
  const int64_t *vs = vx_memref_sizes(v.desc);
  const int64_t *vt = vx_memref_strides(v.desc, v.rank);
  if (*offset < 0 || rank > VX_ABI_MAX_RANK) {
    return false;
  }
  int64_t idx[VX_ABI_MAX_RANK] = {0}, reach[VX_ABI_MAX_RANK] = {0};
  int64_t rest = *offset;
  for (int32_t k = 0; k < v.rank; ++k) {
    const int64_t ds = dense_stride(vs, v.rank, k);
    idx[k] = rest / ds;
    rest -= idx[k] * ds;
  }
  if (rest != 0) {
    return false;
  }
  int64_t out[VX_ABI_MAX_RANK] = {0};
  for (int32_t j = 0; j < rank; ++j) {
    if (sizes[j] <= 1) {
      continue;
    }
    /* Dense strides of the view's dimensions of more than one element fall
     * from the outside in, so the first that divides is the coarsest. */
    int32_t into = -1;
    int64_t times = 0;
    for (int32_t k = 0; k < v.rank && into < 0; ++k) {
      const int64_t ds = dense_stride(vs, v.rank, k);
      if (vs[k] > 1 && strides[j] > 0 && strides[j] % ds == 0) {
        into = k;
        times = strides[j] / ds;
      }
    }
    if (into < 0) {
      return false;
    }
    reach[into] += (sizes[j] - 1) * times;
    out[j] = times * vt[into];
  }
  int64_t off = vx_memref_offset(v.desc);
  for (int32_t k = 0; k < v.rank; ++k) {
    if (idx[k] + reach[k] >= (vs[k] > 0 ? vs[k] : 1)) {
      return false;
    }
    off += idx[k] * vt[k];
  }
  for (int32_t j = 0; j < rank; ++j) {
    strides[j] = sizes[j] <= 1 ? 0 : out[j];
  }
  *offset = off;
  return true;
}

/* A descriptor the region published (rank `rank`) that may point into a
 * copy: give it the HBM the copy stands for. A descriptor whose data starts
 * where a view's copy starts becomes a view of that view's HBM (its own
 * offset added to the view's). False when it points into a copy in a way no
 * HBM layout expresses; the caller stops the program rather than hand back
 * a pointer into freed host memory. */
inline bool publish_from_copy(void *d, int32_t rank,
                              const std::vector<HbmView> &views,
                              const std::vector<HbmSpan> &spans) {
  void **ptrs = reinterpret_cast<void **>(d);
  const uintptr_t p = (uintptr_t)ptrs[1];
  for (const HbmView &v : views) {
    if (v.span < 0) {
      continue;
    }
    const HbmSpan &s = spans[(size_t)v.span];
    if (p != (uintptr_t)s.copy.data() + v.at) {
      continue;
    }
    int64_t *offset =
        reinterpret_cast<int64_t *>(reinterpret_cast<char *>(d) +
                                    2 * sizeof(void *));
    if (v.dense &&
        !dense_to_view(v, offset, vx_memref_sizes(d),
                       const_cast<int64_t *>(vx_memref_strides(d, rank)),
                       rank)) {
      return false;
    }
    if (!v.dense) {
      *offset += vx_memref_offset(v.desc);
    }
    ptrs[0] = reinterpret_cast<void *const *>(v.desc)[0];
    ptrs[1] = vx_memref_aligned(v.desc);
    return true;
  }
  for (const HbmSpan &s : spans) {
    const uintptr_t c = (uintptr_t)s.copy.data();
    if (p >= c && p < c + s.copy.size()) {
      return false;
    }
  }
  return true;
}

/* Call `kernel` with `args`/`tags` on `workers` host threads, HBM views
 * copied through the host as planned above. Returns 1; 0 when libffi
 * rejects the signature; -1 with the argument in `*bad_arg` for a view
 * whose bytes leave the address space; -2 with the argument in `*bad_arg`
 * when a published result points into a copy in a way no HBM layout
 * expresses. */
inline int call_on_host(void *kernel, void **device_args,
                        const int32_t *arg_tags, int64_t num_args, int workers,
                        bool flush_subnormals, const HostCopies &io,
                        int64_t *bad_arg) {
  const size_t n = (size_t)(num_args > 0 ? num_args : 0);
  std::vector<ffi_type *> types(n ? n : 1);
  std::vector<void *> args(n ? n : 1);

  /* The descriptor argument i names (a slot's: the one it holds), or null. */
  auto arg_desc = [&](size_t i) -> void * {
    const int32_t tag = arg_tags[i];
    if (VX_ABI_KIND(tag) != VX_ABI_KIND_MEMREF || !device_args[i] ||
        VX_ABI_RANK(tag) > VX_ABI_MAX_RANK) {
      return nullptr;
    }
    void *desc = *(void **)device_args[i];
    if (desc && VX_ABI_IS_SLOT(tag)) {
      desc = vx_memref_aligned(desc);
    }
    return desc;
  };

  std::vector<HbmView> views;
  std::vector<int64_t> view_of(n, -1);
  for (size_t i = 0; i < n; ++i) {
    types[i] = ffi_type_for_tag(arg_tags[i]);
    args[i] = device_args[i];
    void *desc = arg_desc(i);
    const int32_t elem = VX_ABI_ELEM(arg_tags[i]);
    if (!desc || (VX_ABI_RANK(arg_tags[i]) == 0 && elem == VX_DTYPE_UNKNOWN)) {
      continue;
    }
    void *aligned = vx_memref_aligned(desc);
    if (!aligned || !io.is_device(aligned)) {
      continue;
    }
    HbmView v;
    v.desc = desc;
    v.rank = VX_ABI_RANK(arg_tags[i]);
    v.elem = elem;
    v.arg = (int64_t)i;
    view_of[i] = (int64_t)views.size();
    views.push_back(v);
  }

  std::vector<HbmSpan> spans;
  size_t bad = 0;
  if (!plan_spans(views, spans, &bad)) {
    *bad_arg = views[bad].arg;
    return -1;
  }

  for (HbmSpan &s : spans) {
    s.copy.resize(s.bytes ? (size_t)s.bytes : 1);
  }
  if (!spans.empty() && io.sync) {
    io.sync();
  }
  for (HbmSpan &s : spans) {
    if (s.dense_view >= 0) {
      for_each_dense_block(
          views[(size_t)s.dense_view],
          [&](uint64_t dense, uintptr_t hbm, uint64_t width, uint64_t pitch,
              uint64_t height) {
            io.to_host(s.copy.data() + dense, (size_t)width,
                       reinterpret_cast<const void *>(hbm), (size_t)pitch,
                       (size_t)width, (size_t)height);
          });
    } else {
      io.to_host(s.copy.data(), (size_t)s.bytes,
                 reinterpret_cast<const void *>(s.first), (size_t)s.bytes,
                 (size_t)s.bytes, 1);
    }
  }

  /* Private descriptors (and, for slots, private slots holding them). */
  const size_t max_words = 3 + 2 * (size_t)VX_ABI_MAX_RANK;
  std::vector<std::vector<int64_t>> descs(n);
  std::vector<std::vector<int64_t>> before(n);
  std::vector<void *> desc_ptr(n, nullptr);
  std::vector<std::vector<int64_t>> slots(n);
  std::vector<void *> slot_ptr(n, nullptr);
  for (size_t i = 0; i < n; ++i) {
    if (view_of[i] < 0) {
      continue;
    }
    const HbmView &v = views[(size_t)view_of[i]];
    if (v.span < 0) {
      continue; /* empty: passed through */
    }
    point_into_copy(v, spans[(size_t)v.span], descs[i]);
    descs[i].resize(max_words, 0);
    before[i] = descs[i];
    if (VX_ABI_IS_SLOT(arg_tags[i])) {
      slots[i].assign(3, 0);
      void **sp = reinterpret_cast<void **>(slots[i].data());
      sp[0] = descs[i].data();
      sp[1] = descs[i].data();
      slot_ptr[i] = slots[i].data();
      args[i] = &slot_ptr[i];
    } else {
      desc_ptr[i] = descs[i].data();
      args[i] = &desc_ptr[i];
    }
  }

  ffi_cif cif;
  if (ffi_prep_cif(&cif, FFI_DEFAULT_ABI, (unsigned)n, &ffi_type_void,
                   types.data()) != FFI_OK) {
    return 0;
  }
  host_call_split(&cif, kernel, args.data(), workers, flush_subnormals);

  for (HbmSpan &s : spans) {
    if (s.dense_view >= 0) {
      for_each_dense_block(
          views[(size_t)s.dense_view],
          [&](uint64_t dense, uintptr_t hbm, uint64_t width, uint64_t pitch,
              uint64_t height) {
            io.to_device(reinterpret_cast<void *>(hbm), (size_t)pitch,
                         s.copy.data() + dense, (size_t)width, (size_t)width,
                         (size_t)height);
          });
    } else {
      io.to_device(reinterpret_cast<void *>(s.first), (size_t)s.bytes,
                   s.copy.data(), (size_t)s.bytes, (size_t)s.bytes, 1);
    }
  }

  /* Slots: a result the region published goes back to the caller with its
   * pointers in HBM. A private slot whose descriptor the region left alone
   * publishes nothing. */
  for (size_t i = 0; i < n; ++i) {
    if (VX_ABI_KIND(arg_tags[i]) != VX_ABI_KIND_MEMREF ||
        !VX_ABI_IS_SLOT(arg_tags[i])) {
      continue;
    }
    const int32_t rank = VX_ABI_RANK(arg_tags[i]);
    if (!slot_ptr[i]) {
      void *d = arg_desc(i);
      if (d && !publish_from_copy(d, rank, views, spans)) {
        *bad_arg = (int64_t)i;
        return -2;
      }
      continue;
    }
    if (descs[i] == before[i]) {
      continue;
    }
    if (!publish_from_copy(descs[i].data(), rank, views, spans)) {
      *bad_arg = (int64_t)i;
      return -2;
    }
    memcpy(arg_desc(i), descs[i].data(), (3 + 2 * (size_t)rank) * sizeof(int64_t));
  }
  return 1;
}

} // namespace vx

#endif /* VX_AMD_HOST_FALLBACK_H */
