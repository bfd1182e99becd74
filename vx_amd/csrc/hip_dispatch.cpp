/*
 * hip_dispatch.cpp -- libvx_hip_dispatch.so, the vx_plugin_* ABI on one or
 * more MI355X GPUs (gfx950).
 *
 * A drop-in for the CUDA dispatch library (reference
 * runtime/cuda_dispatch.cpp): a compiled Vx program links it through
 * VX_DISPATCH_LIB (reference src/jit.rs:235-265) and calls the entry points of
 * include/vx_hardware_runtime.h. What differs is below the ABI:
 *
 *  - a routed `a @ b` (kind=matmul) runs on hand-written gfx950 kernels
 *    (kernels/gemm.hip): no vendor BLAS;
 *  - the mixed plan (bf16/f16 inputs, f32 result) the reference sends to the
 *    host loop nest is routed to the GPU too;
 *  - operands already in HBM are used in place; host operands are staged
 *    through an exact-size pool (vx_device_pool_hip.h);
 *  - a region whose payload carries a gfx950 code object (`format=hsaco`,
 *    the image in the payload's binary section) runs from that image, with
 *    its parameters marshalled and counted against the image's metadata
 *    (vx_image_launch.h; reference runtime/cuda_dispatch.cpp:1364-1675 does
 *    the same for PTX);
 *  - everything else runs as the outlined host kernel, with HBM views copied
 *    out and back (vx_host_fallback.h);
 *  - flash attention and the int8 GEMV are library ops (include/vx_hip_ops.h).
 *
 * Streams: each thread launches on its caller stream (vx_cuda_set_stream;
 * default the null stream), as the reference does (:205-207). A launch
 * returns at once; waits happen at read-backs, awaits and VX_CTRL_WAIT*.
 *
 * Waits (vx_stream_policy.h): a wait covers the caller stream, or every
 * device this library used when none is set; while the caller stream is
 * capturing a hipGraph, anything that must block the host is refused with a
 * message. A wait that finds a fault names the last kernel launched there.
 * With a caller stream, HBM from vx_plugin_alloc_and_transfer is taken and
 * given back in that stream's order (hipMallocAsync / hipFreeAsync).
 *
 * Environment: VX_DISPATCH_VERBOSE (routing narrative on stderr),
 * VX_TIME_KERNEL (device time of each routed GEMM and image launch on
 * stderr), VX_HIP_SYNC=1 (wait after every launch, so a fault names its
 * launch), VX_HIP_POOL_MAX_MB, VX_HOST_THREADS (host workers of a split
 * region on the host).
 */
#include "../../include/vx_hardware_runtime.h"
#include "../../include/vx_hip_ops.h"
#include "vx_device_pool_hip.h"
#include "vx_dispatch_plan.h"
#include "vx_hip_common.h"
#include "vx_host_fallback.h"
#include "vx_image_launch.h"
#include "vx_kernels.h"
#include "vx_ops_internal.h"
#include "vx_ops_kernels.h"
#include "vx_stream_policy.h"

#include <dlfcn.h>

#include <atomic>
#include <cstring>
#include <map>
#include <string>
#include <mutex>
#include <tuple>

namespace {

bool verbose() {
  static const bool on = [] {
    const char *v = getenv("VX_DISPATCH_VERBOSE");
    return v && *v && strcmp(v, "0") != 0;
  }();
  return on;
}

bool sync_each_launch() {
  static const bool on = [] {
    const char *v = getenv("VX_HIP_SYNC");
    return v && *v && strcmp(v, "0") != 0;
  }();
  return on;
}

bool hip_available() {
  static const bool ok = [] {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
      (void)hipGetLastError();
      fprintf(stderr,
              "[Vx HIP] no HIP device (%s); kernels will run on the host\n",
              e == hipSuccess ? "none present" : hipGetErrorString(e));
      return false;
    }
    return true;
  }();
  return ok;
}

thread_local hipStream_t caller_stream = nullptr;

/* Declared ids the program said stand for a built-in device
 * (VX_CTRL_LOCAL_DEVICE). Entries are written before the count that
 * publishes them (reference runtime/cuda_dispatch.cpp:632-655). */
struct LocalDevice {
  int32_t declared;
  int32_t builtin;
};
LocalDevice local_devices[64];
std::atomic<size_t> local_device_count{0};
std::mutex local_devices_mutex;

int gpu_index(int32_t topology_id) {
  const size_t n = local_device_count.load(std::memory_order_acquire);
  for (size_t i = 0; i < n; ++i) {
    if (local_devices[i].declared == topology_id) {
      topology_id = local_devices[i].builtin;
      break;
    }
  }
  return vx_topology_device_index(topology_id, VX_TOPO_GPU_BASE);
}

/* Make the GPU `topology_id` names current. A non-GPU or absent id leaves the
 * current device alone; a GPU this machine lacks is fatal (reference
 * runtime/cuda_dispatch.cpp:707-729). */
void select_device(int32_t topology_id, const char *why) {
  const int index = gpu_index(topology_id);
  if (index < 0) {
    return;
  }
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || index >= count) {
    fprintf(stderr,
            "[Vx HIP] FATAL: launch targets GPU %d, but this machine has %d\n",
            index, count);
    abort();
  }
  VX_HIP_CHECK(hipSetDevice(index));
  if (verbose()) {
    fprintf(stderr, "[Vx HIP] device %d %s\n", index, why);
  }
}

/* True for memory the GPU owns (hipMalloc'd). Host memory, registered or not,
 * answers false. */
bool is_device_ptr(const void *p) {
  if (!p || !hip_available()) {
    return false;
  }
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return attr.type == hipMemoryTypeDevice;
}

void *device_malloc(size_t bytes) {
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return p;
}

void device_release(void *p, size_t) { (void)hipFree(p); }

using Pool = vx::HipDevicePool<void *(*)(size_t), void (*)(void *, size_t)>;
Pool &pool() {
  static Pool *p =
      new Pool(&device_malloc, &device_release, vx::hip_pool_cap_from_env());
  return *p;
}

/* The last kernel each device started that no wait has covered yet, so that
 * a wait that finds a fault can name a suspect (reference
 * runtime/cuda_dispatch.cpp:190-300). VX_HIP_SYNC=1 waits after every launch
 * instead, which names the faulting kernel itself. */
std::mutex unwaited_mutex;
std::map<int, std::string> &unwaited() {
  static auto *m = new std::map<int, std::string>();
  return *m;
}
/* The last kernel this thread started on its caller stream. */
thread_local std::string last_on_stream;

/* HBM this library took with hipMallocAsync on a caller's stream: freed in
 * that stream's order (hipFreeAsync), also once the caller has moved on to
 * another stream. */
std::mutex stream_allocs_mutex;
std::map<void *, hipStream_t> &stream_allocs() {
  static auto *m = new std::map<void *, hipStream_t>();
  return *m;
}

/* Whether the caller's stream is being captured into a hipGraph now. */
bool capturing() {
  if (!caller_stream) {
    return false;
  }
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(caller_stream, &status);
  if (e != hipSuccess) {
    fprintf(stderr,
            "[Vx HIP] FATAL: cannot tell whether the stream given to "
            "vx_hip_set_stream is capturing a graph: %s\n",
            hipGetErrorString(e));
    abort();
  }
  return status != hipStreamCaptureStatusNone;
}

/* `what` cannot be recorded into the graph the caller's stream is capturing;
 * `fix` says what the program can do instead. */
[[noreturn]] void refuse_in_capture(
    const char *what,
    const char *fix = "Pass only tensors already in GPU memory while the "
                      "capture runs, and read results after it ends.") {
  fprintf(stderr,
          "[Vx HIP] FATAL: %s while the stream given to vx_hip_set_stream is "
          "capturing a hipGraph, and a graph cannot record that. %s\n",
          what, fix);
  abort();
}

/* Waits for every device this library launched on (the current one always),
 * naming the last kernel started there when one faulted. */
void wait_for_devices() {
  std::map<int, std::string> started;
  {
    std::lock_guard<std::mutex> hold(unwaited_mutex);
    started.swap(unwaited());
  }
  int current = 0;
  VX_HIP_CHECK(hipGetDevice(&current));
  started.emplace(current, std::string());
  for (const auto &entry : started) {
    if (entry.first != current) {
      VX_HIP_CHECK(hipSetDevice(entry.first));
    }
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      fprintf(stderr,
              "[Vx HIP] FATAL: GPU %d reported a fault: %s. Last kernel "
              "launched there: %s (VX_HIP_SYNC=1 waits after each launch to "
              "name the one that faulted)\n",
              entry.first, hipGetErrorString(e),
              entry.second.empty() ? "none by this library"
                                   : entry.second.c_str());
      abort();
    }
  }
  VX_HIP_CHECK(hipSetDevice(current));
}

/* Waits for the work before `why`: the caller's stream if one is set, else
 * every device this library used. */
void wait_for_kernels(const char *why) {
  if (verbose()) {
    fprintf(stderr, "[Vx HIP] wait: %s\n", why);
  }
  switch (vx::wait_action(caller_stream != nullptr, capturing())) {
  case vx::WaitAction::kDevice:
    wait_for_devices();
    return;
  case vx::WaitAction::kRefuse: {
    char what[256];
    snprintf(what, sizeof what, "a wait for the GPU (%s) came", why);
    refuse_in_capture(what);
  }
  case vx::WaitAction::kStream:
    break;
  }
  const hipError_t e = hipStreamSynchronize(caller_stream);
  if (e != hipSuccess) {
    fprintf(stderr,
            "[Vx HIP] FATAL: the stream given to vx_hip_set_stream reported a "
            "fault (%s) before %s. Last kernel launched on it: %s "
            "(VX_HIP_SYNC=1 waits after each launch to name the one that "
            "faulted)\n",
            hipGetErrorString(e), why,
            last_on_stream.empty() ? "none by this library"
                                   : last_on_stream.c_str());
    abort();
  }
}

/* After a launch of `name` on the current device. */
void started_kernel(const char *name) {
  int device = 0;
  VX_HIP_CHECK(hipGetDevice(&device));
  if (sync_each_launch()) {
    if (capturing()) {
      refuse_in_capture("VX_HIP_SYNC=1 asked for a wait after a launch",
                        "Unset VX_HIP_SYNC while capturing.");
    }
    const hipError_t e = caller_stream ? hipStreamSynchronize(caller_stream)
                                       : hipDeviceSynchronize();
    if (e != hipSuccess) {
      fprintf(stderr, "[Vx HIP] FATAL: %s faulted on GPU %d: %s\n", name,
              device, hipGetErrorString(e));
      abort();
    }
    return;
  }
  if (caller_stream) {
    last_on_stream = name;
  }
  std::lock_guard<std::mutex> hold(unwaited_mutex);
  unwaited()[device] = name;
}

/* HBM of `bytes`, in stream order on the caller's stream when one is set. */
hipError_t device_alloc(void **ptr, size_t bytes) {
  if (!caller_stream) {
    return hipMalloc(ptr, bytes);
  }
  const hipError_t e = hipMallocAsync(ptr, bytes, caller_stream);
  if (e == hipSuccess) {
    std::lock_guard<std::mutex> hold(stream_allocs_mutex);
    stream_allocs()[*ptr] = caller_stream;
  }
  return e;
}

/* Frees HBM from vx_plugin_alloc_and_transfer / transfer_peer. */
void device_free(void *ptr) {
  hipStream_t from = nullptr;
  bool ordered = false;
  {
    std::lock_guard<std::mutex> hold(stream_allocs_mutex);
    auto found = stream_allocs().find(ptr);
    if (found != stream_allocs().end()) {
      from = found->second;
      ordered = true;
      stream_allocs().erase(found);
    }
  }
  switch (vx::free_action(caller_stream != nullptr, capturing(), ordered)) {
  case vx::FreeAction::kOnStream:
    VX_HIP_CHECK(hipFreeAsync(ptr, from));
    return;
  case vx::FreeAction::kRefuse:
    refuse_in_capture("GPU memory that a launch may still read was freed");
  case vx::FreeAction::kAfterDeviceWait:
  case vx::FreeAction::kAfterStreamWait:
    wait_for_kernels("a device buffer was freed");
    VX_HIP_CHECK(hipFree(ptr));
    return;
  }
}

/* Counters a test reads to prove which path ran (VX_HIP_CTRL_STATS). */
std::atomic<int64_t> stat_gemm_device{0};
std::atomic<int64_t> stat_gemm_mfma{0};
std::atomic<int64_t> stat_gemm_tiled{0};
std::atomic<int64_t> stat_host_fallback{0};
std::atomic<int64_t> stat_staged_bytes{0};
std::atomic<int64_t> stat_scratch_staged_bytes{0}; /* of them, via the scratch */
std::atomic<int64_t> stat_image_launches{0};
std::atomic<int64_t> stat_image_loads{0};
std::atomic<int> forced_gemm_kernel{0};

/* Clock stamps of routed MFMA GEMMs (VX_HIP_CTRL_CLOCK_STAMPS): a ring of
 * `slots` records of 4 u64 in HBM, one per launch in turn; off when null. */
std::mutex stamps_mutex;
uint64_t *stamps_base = nullptr;
int64_t stamps_slots = 0, stamps_next = 0;

uint64_t *next_stamp() {
  std::lock_guard<std::mutex> hold(stamps_mutex);
  if (!stamps_base || stamps_slots <= 0) {
    return nullptr;
  }
  uint64_t *p = stamps_base + 4 * (stamps_next % stamps_slots);
  ++stamps_next;
  return p;
}

/* Where host operands and host results are staged: the pool, or (for
 * vx_hip_dispatch_async_noalloc) a region handed out front to back. */
struct Arena {
  unsigned char *base = nullptr; /* null: the pool */
  size_t size = 0, used = 0;
  void *take(size_t bytes) {
    const size_t at = (used + 255) / 256 * 256;
    if (at > size || bytes > size - at) {
      return nullptr;
    }
    used = at + bytes;
    return base + at;
  }
};

/* An operand on the device: used in place, or a pooled packed copy. */
struct DeviceOperand {
  void *ptr = nullptr;
  int64_t row_stride = 0;
  size_t bytes = 0;
  bool pooled = false;
  ~DeviceOperand() {
    if (pooled && ptr) {
      /* The copy may still be read by a launch on the caller stream. */
      wait_for_kernels("a staging buffer went back to the pool");
      pool().release(ptr, bytes);
    }
  }
};

void stage(const void *data, int64_t rows, int64_t cols, int64_t row_stride,
           size_t esz, DeviceOperand &out, Arena *arena) {
  if (is_device_ptr(data)) {
    out.ptr = const_cast<void *>(data);
    out.row_stride = row_stride;
    return;
  }
  if (capturing()) {
    refuse_in_capture("a GEMM operand in host memory was copied to the GPU");
  }
  const size_t width = (size_t)cols * esz;
  out.bytes = (size_t)rows * width;
  out.ptr = arena ? arena->take(out.bytes) : pool().acquire(out.bytes);
  if (!out.ptr) {
    fprintf(stderr,
            "[Vx HIP] FATAL: out of device memory staging %zu bytes "
            "(%lld x %lld)\n",
            out.bytes, (long long)rows, (long long)cols);
    abort();
  }
  out.pooled = arena == nullptr;
  out.row_stride = cols;
  stat_staged_bytes += (int64_t)out.bytes;
  if (arena) {
    stat_scratch_staged_bytes += (int64_t)out.bytes;
  }
  VX_HIP_CHECK(hipMemcpy2DAsync(out.ptr, width, data, (size_t)row_stride * esz,
                                width, (size_t)rows, hipMemcpyHostToDevice,
                                caller_stream));
}

/* `no_alloc`: the no-alloc entry point's call, which takes no device memory
 * beyond its scratch (so no stream-K workspace either). */
bool run_gemm(const vx_gemm_plan &plan, Arena *arena = nullptr, bool no_alloc = false) {
  const size_t in_esz = vx_dtype_bytes(plan.dtype);
  const size_t out_esz = vx_dtype_bytes(plan.out_dtype);
  if (!in_esz || !out_esz) {
    return false;
  }
  if (verbose()) {
    fprintf(stderr, "[Vx HIP] GEMM %lldx%lldx%lld %s -> %s %s\n",
            (long long)plan.m, (long long)plan.n, (long long)plan.k,
            vx_dtype_name(plan.dtype), vx_dtype_name(plan.out_dtype),
            plan.out_kind == VX_GEMM_OUT_SLOT ? "slot" : "buffer");
  }

  DeviceOperand a, b, c;
  stage(plan.a_data, plan.m, plan.k, plan.a_row_stride, in_esz, a, arena);
  stage(plan.b_data, plan.k, plan.n, plan.b_row_stride, in_esz, b, arena);
  const bool out_is_device =
      plan.out_kind == VX_GEMM_OUT_BUFFER && is_device_ptr(plan.out_data);
  if (out_is_device) {
    c.ptr = plan.out_data;
    c.row_stride = plan.out_row_stride;
  } else {
    c.bytes = (size_t)plan.m * (size_t)plan.n * out_esz;
    c.ptr = arena ? arena->take(c.bytes) : pool().acquire(c.bytes);
    if (!c.ptr) {
      fprintf(stderr, "[Vx HIP] FATAL: out of device memory for a %lldx%lld "
                      "GEMM result\n",
              (long long)plan.m, (long long)plan.n);
      abort();
    }
    c.pooled = arena == nullptr;
    c.row_stride = plan.n;
    if (arena) {
      stat_scratch_staged_bytes += (int64_t)c.bytes;
    }
  }

  vxk::GemmArgs g;
  g.in_dtype = plan.dtype;
  g.out_dtype = plan.out_dtype;
  g.m = plan.m, g.n = plan.n, g.k = plan.k;
  g.a = a.ptr, g.b = b.ptr, g.c = c.ptr;
  g.lda = a.row_stride, g.ldb = b.row_stride, g.ldc = c.row_stride;
  g.stamp = next_stamp();
  /* The stream-K launch keeps a workspace per stream: not for the no-alloc
   * entry point, and not into a graph being captured. */
  g.may_split = !no_alloc && arena == nullptr && !capturing();

  vxk::GemmKernel which = vxk::gemm_pick(g);
  const int forced = forced_gemm_kernel.load();
  if (forced != 0 && vxk::gemm_kernel_takes((vxk::GemmKernel)forced, g)) {
    /* A forced kernel applies where it takes the shape; elsewhere the
     * automatic choice stands. */
    which = (vxk::GemmKernel)forced;
  }

  const bool time_kernel = getenv("VX_TIME_KERNEL") != nullptr;
  if (time_kernel && capturing()) {
    refuse_in_capture("VX_TIME_KERNEL waits for each kernel",
                      "Unset VX_TIME_KERNEL while capturing.");
  }
  hipEvent_t t0 = nullptr, t1 = nullptr;
  if (time_kernel) {
    VX_HIP_CHECK(hipEventCreate(&t0));
    VX_HIP_CHECK(hipEventCreate(&t1));
    VX_HIP_CHECK(hipEventRecord(t0, caller_stream));
  }
  if (!vxk::gemm_launch_kernel(which, g, caller_stream)) {
    fprintf(stderr,
            "[Vx HIP] FATAL: no GPU kernel takes the GEMM %lldx%lldx%lld %s -> "
            "%s (strides %lld/%lld/%lld)\n",
            (long long)g.m, (long long)g.n, (long long)g.k,
            vx_dtype_name(g.in_dtype), vx_dtype_name(g.out_dtype),
            (long long)g.lda, (long long)g.ldb, (long long)g.ldc);
    abort();
  }
  if (time_kernel) {
    VX_HIP_CHECK(hipEventRecord(t1, caller_stream));
    VX_HIP_CHECK(hipEventSynchronize(t1));
    float ms = 0.0f;
    VX_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
    fprintf(stderr, "[Vx HIP] GEMM device time %.3f ms (%lldx%lldx%lld)\n", ms,
            (long long)g.m, (long long)g.n, (long long)g.k);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
  }
  ++stat_gemm_device;
  (vxk::gemm_is_mfma(which) ? stat_gemm_mfma : stat_gemm_tiled)++;
  started_kernel("a GEMM");

  if (out_is_device) {
    return true;
  }
  wait_for_kernels("a GEMM result was copied to host memory");
  const size_t width = (size_t)plan.n * out_esz;
  if (plan.out_kind == VX_GEMM_OUT_SLOT) {
    /* The program frees a slot result with free(): it must be malloc memory
     * (reference docs/lang/abi.md section 3.1). */
    void *result = malloc((size_t)plan.m * width);
    if (!result) {
      fprintf(stderr, "[Vx HIP] FATAL: out of memory for a %lldx%lld result\n",
              (long long)plan.m, (long long)plan.n);
      abort();
    }
    VX_HIP_CHECK(hipMemcpy(result, c.ptr, (size_t)plan.m * width,
                           hipMemcpyDeviceToHost));
    vx_gemm_publish_slot(&plan, result);
    return true;
  }
  VX_HIP_CHECK(hipMemcpy2D(plan.out_data, (size_t)plan.out_row_stride * out_esz,
                           c.ptr, width, width, (size_t)plan.m,
                           hipMemcpyDeviceToHost));
  return true;
}

vx::HostCopies host_copies() {
  vx::HostCopies io;
  io.is_device = [](const void *p) { return is_device_ptr(p); };
  io.sync = [] { wait_for_kernels("a host kernel read GPU memory"); };
  io.to_host = [](void *dst, size_t dpitch, const void *src, size_t spitch,
                  size_t width, size_t height) {
    VX_HIP_CHECK(hipMemcpy2D(dst, dpitch, src, spitch, width, height,
                             hipMemcpyDeviceToHost));
  };
  io.to_device = [](void *dst, size_t dpitch, const void *src, size_t spitch,
                    size_t width, size_t height) {
    VX_HIP_CHECK(hipMemcpy2D(dst, dpitch, src, spitch, width, height,
                             hipMemcpyHostToDevice));
  };
  return io;
}

/* The gfx name of the current device ("gfx950"), without feature flags. */
std::string device_arch() {
  int device = 0;
  VX_HIP_CHECK(hipGetDevice(&device));
  hipDeviceProp_t prop;
  VX_HIP_CHECK(hipGetDeviceProperties(&prop, device));
  std::string arch = prop.gcnArchName;
  const size_t colon = arch.find(':');
  return colon == std::string::npos ? arch : arch.substr(0, colon);
}

/* A loaded image's kernel. Keyed by kernel name, device, the library that
 * holds the payload (two libraries may use one kernel name), the image's
 * address and size, and a hash of its first and last 256 bytes (a payload
 * built at run time may reuse an address for another image). */
struct LoadedImage {
  hipModule_t module = nullptr;
  hipFunction_t fn = nullptr;
  int declared = -1;
};
std::mutex images_mutex;
std::map<std::string, LoadedImage> &images() {
  static auto *m = new std::map<std::string, LoadedImage>();
  return *m;
}

uint64_t image_edges_hash(const unsigned char *b, size_t n) {
  uint64_t h = 1469598103934665603ull;
  const size_t head = n < 256 ? n : 256;
  for (size_t i = 0; i < head; ++i) {
    h = (h ^ b[i]) * 1099511628211ull;
  }
  for (size_t i = n - head; i < n; ++i) {
    h = (h ^ b[i]) * 1099511628211ull;
  }
  return h;
}

/* The flag an `assert_flag=1` kernel sets when an assert fails: one int per
 * device, cleared before each such launch. */
int *assert_flag(int device) {
  static std::mutex m;
  static std::map<int, int *> flags;
  std::lock_guard<std::mutex> hold(m);
  int *&f = flags[device];
  if (!f) {
    VX_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&f), sizeof(int)));
  }
  return f;
}

/* Run the code object the payload carries. False -- leaving the host
 * fallback to run the region -- when the payload has no gfx950 image, or an
 * argument cannot be marshalled or lives in host memory. A broken image, a
 * parameter count that disagrees with the image, or a shape no GPU launches
 * is fatal (reference runtime/cuda_dispatch.cpp:1364-1675,
 * runtime/xpu_dispatch.cpp:470-705). */
bool run_device_image(const void *payload, size_t payload_size,
                      void **device_args, const int32_t *arg_tags,
                      int64_t num_args) {
  const char *name = static_cast<const char *>(payload);
  const char *format = vx_payload_field(payload, payload_size, "format=");
  if (!format || strcmp(format, "hsaco") != 0) {
    if (format && verbose()) {
      fprintf(stderr,
              "[Vx HIP] %s has format=%s, which this library does not load\n",
              name, format);
    }
    return false;
  }
  const void *image = nullptr;
  const int64_t image_size = vx_payload_section(payload, payload_size, &image);
  if (image_size <= 0 || !image) {
    if (verbose()) {
      fprintf(stderr,
              "[Vx HIP] %s says format=hsaco but carries no usable image "
              "section (code %lld)\n",
              name, (long long)image_size);
    }
    return false;
  }
  select_device(vx_payload_topology(payload, payload_size), "image launch");
  int device = 0;
  VX_HIP_CHECK(hipGetDevice(&device));

  const char *flag_field = vx_payload_field(payload, payload_size, "assert_flag=");
  const bool takes_flag = flag_field && strcmp(flag_field, "1") == 0;
  vx::ImageParams params;
  if (!vx::image_build_params(device_args, arg_tags, num_args, params) ||
      (takes_flag && params.count >= vx::kImageMaxParams)) {
    if (verbose()) {
      fprintf(stderr,
              "[Vx HIP] %s has an argument this path cannot marshal (a "
              "publication slot, or more than %d parameters); not "
              "launching\n",
              name, vx::kImageMaxParams);
    }
    return false;
  }
  for (int64_t i = 0; i < num_args; ++i) {
    if (VX_ABI_KIND(arg_tags[i]) != VX_ABI_KIND_MEMREF) {
      continue;
    }
    const void *desc = *static_cast<void *const *>(device_args[i]);
    if (!is_device_ptr(vx_memref_aligned(desc))) {
      if (verbose()) {
        fprintf(stderr,
                "[Vx HIP] %s: argument %lld is not in GPU memory; the host "
                "runs it\n",
                name, (long long)i);
      }
      return false;
    }
  }
  Dl_info info;
  const void *library = dladdr(payload, &info) ? info.dli_fbase : nullptr;
  char key[512];
  snprintf(key, sizeof key, "%s@%d@%p@%p@%lld@%016llx", name, device, library,
           image, (long long)image_size,
           (unsigned long long)image_edges_hash(
               static_cast<const unsigned char *>(image), (size_t)image_size));
  LoadedImage loaded;
  {
    std::lock_guard<std::mutex> hold(images_mutex);
    auto found = images().find(key);
    if (found != images().end()) {
      loaded = found->second;
    } else {
      const std::string arch = device_arch();
      loaded.declared = vx::code_object_param_count(
          image, (size_t)image_size, arch.c_str(), name);
      if (loaded.declared < 0) {
        fprintf(stderr,
                "[Vx HIP] FATAL: the image of %s holds no %s code object with "
                "an entry %s whose parameters can be read\n",
                name, arch.c_str(), name);
        abort();
      }
      hipError_t e = hipModuleLoadData(&loaded.module, image);
      if (e != hipSuccess) {
        fprintf(stderr, "[Vx HIP] FATAL: the device image for %s did not load: %s\n",
                name, hipGetErrorString(e));
        abort();
      }
      e = hipModuleGetFunction(&loaded.fn, loaded.module, name);
      if (e != hipSuccess) {
        fprintf(stderr,
                "[Vx HIP] FATAL: the device image loaded but has no entry "
                "%s: %s\n",
                name, hipGetErrorString(e));
        abort();
      }
      images().emplace(key, loaded);
      ++stat_image_loads;
    }
  }

  const int given = params.count + (takes_flag ? 1 : 0);
  if (loaded.declared != given) {
    fprintf(stderr,
            "[Vx HIP] FATAL: %s declares %d parameters and its arguments "
            "produced %d.\n"
            "          Launching would read past what was supplied.\n",
            name, loaded.declared, given);
    abort();
  }
  unsigned grid[3], block;
  char why[160];
  if (!vx::image_launch_geometry(payload, payload_size, device_args, arg_tags,
                                 num_args, grid, &block, why, sizeof why)) {
    fprintf(stderr, "[Vx HIP] FATAL: %s: %s\n", name, why);
    abort();
  }
  int *flag = nullptr;
  if (takes_flag) {
    flag = assert_flag(device);
    vxk::fill_i32_launch(flag, 0, caller_stream);
    params.p[params.count] = &flag;
  }
  const char *shared_field = vx_payload_field(payload, payload_size, "shared=");
  const unsigned shared =
      shared_field ? (unsigned)strtoul(shared_field, nullptr, 10) : 0u;
  const char *coop = vx_payload_field(payload, payload_size, "coop=");
  /* Device time of the launch on request, stamped by hipEvents on the launch
   * stream (the same instrument as a routed GEMM's). */
  const bool time_kernel = getenv("VX_TIME_KERNEL") != nullptr;
  if (time_kernel && capturing()) {
    refuse_in_capture("VX_TIME_KERNEL waits for each kernel",
                      "Unset VX_TIME_KERNEL while capturing.");
  }
  hipEvent_t t0 = nullptr, t1 = nullptr;
  if (time_kernel) {
    int resident = 0;
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(
            &resident, loaded.fn, (int)block, shared) == hipSuccess) {
      fprintf(stderr, "[Vx HIP] %s occupancy: %d workgroup(s) of %u per CU\n",
              name, resident, block);
    }
    VX_HIP_CHECK(hipEventCreate(&t0));
    VX_HIP_CHECK(hipEventCreate(&t1));
    VX_HIP_CHECK(hipEventRecord(t0, caller_stream));
  }
  hipError_t e;
  if (coop && strcmp(coop, "0") != 0) {
    /* Grid-wide barriers: every block must be resident at once, which the
     * cooperative launch checks instead of letting the barrier wait forever. */
    e = hipModuleLaunchCooperativeKernel(loaded.fn, grid[0], grid[1], grid[2],
                                         block, 1, 1, shared, caller_stream,
                                         params.p);
  } else {
    e = hipModuleLaunchKernel(loaded.fn, grid[0], grid[1], grid[2], block, 1,
                              1, shared, caller_stream, params.p, nullptr);
  }
  if (e != hipSuccess) {
    fprintf(stderr, "[Vx HIP] FATAL: launching %s failed: %s\n", name,
            hipGetErrorString(e));
    abort();
  }
  started_kernel(name);
  if (time_kernel) {
    VX_HIP_CHECK(hipEventRecord(t1, caller_stream));
    VX_HIP_CHECK(hipEventSynchronize(t1));
    float ms = 0.0f;
    VX_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
    fprintf(stderr, "[Vx HIP] %s device time %.3f ms (%ux%ux%u x %u)\n", name,
            ms, grid[0], grid[1], grid[2], block);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
  }
  ++stat_image_launches;
  if (takes_flag) {
    int failed = 0;
    wait_for_kernels("an assert flag");
    VX_HIP_CHECK(hipMemcpy(&failed, flag, sizeof failed, hipMemcpyDeviceToHost));
    if (failed != 0) {
      fprintf(stderr, "[Vx HIP] FATAL: an assert failed in %s\n", name);
      abort();
    }
  }
  if (verbose()) {
    fprintf(stderr,
            "[Vx HIP] %s ran on GPU %d from its own image (%d params, "
            "%ux%ux%u blocks of %u)\n",
            name, device, params.count, grid[0], grid[1], grid[2], block);
  }
  return true;
}

void run_on_host(const void *payload, size_t payload_size, void **device_args,
                 const int32_t *arg_tags, int64_t num_args) {
  const char *name = static_cast<const char *>(payload);
  if (vx_payload_field(payload, payload_size, "coop=")) {
    fprintf(stderr,
            "[Vx HIP] FATAL: %s is a cooperative kernel -- its barriers are "
            "inside the thread loop, so no serial order of that loop computes "
            "it, and this library has no device image for it\n",
            name);
    abort();
  }
  void *kernel = vx::host_kernel_symbol(name);
  if (!kernel) {
    fprintf(stderr, "[Vx HIP] FATAL: outlined kernel %s not found\n", name);
    abort();
  }
  if (verbose()) {
    const char *kind = vx_payload_field(payload, payload_size, "kind=");
    fprintf(stderr, "[Vx HIP] %s (kind=%s) runs on the host\n", name,
            kind ? kind : "<unclassified>");
  }
  ++stat_host_fallback;
  const int workers = vx::host_worker_count_for(payload, payload_size,
                                                device_args, arg_tags, num_args);
  int64_t bad = -1;
  const int rc = vx::call_on_host(
      kernel, device_args, arg_tags, num_args, workers,
      vx::host_flushes_subnormals(payload, payload_size), host_copies(), &bad);
  if (rc == 0) {
    fprintf(stderr, "[Vx HIP] FATAL: could not build a call for %s\n", name);
    abort();
  }
  if (rc == -1) {
    fprintf(stderr,
            "[Vx HIP] FATAL: argument %lld of %s is a GPU view with a negative "
            "offset or one that runs past the end of the address space\n",
            (long long)bad, name);
    abort();
  }
  if (rc == -2) {
    fprintf(stderr,
            "[Vx HIP] FATAL: %s published through argument %lld a view into a "
            "host copy of GPU memory that has no layout in the GPU tensor it "
            "was copied from\n",
            name, (long long)bad);
    abort();
  }
}

/* Arrival counts kept per (site, topology, stream), reference
 * runtime/vx_arrival_counts.h semantics: take gives back a kept count of at
 * least `bytes`; give keeps the larger of two and hands back the other. */
class ArrivalCounts {
public:
  void *take(const void *site, uint32_t topo, const void *stream,
             size_t bytes) {
    std::lock_guard<std::mutex> hold(mu_);
    auto it = kept_.find(Key{site, topo, stream});
    if (it == kept_.end() || it->second.second < bytes) {
      return nullptr;
    }
    void *count = it->second.first;
    kept_.erase(it);
    return count;
  }
  void *give(const void *site, uint32_t topo, const void *stream, void *count,
             size_t bytes) {
    std::lock_guard<std::mutex> hold(mu_);
    Key key{site, topo, stream};
    auto it = kept_.find(key);
    if (it == kept_.end()) {
      kept_.emplace(key, std::make_pair(count, bytes));
      return nullptr;
    }
    if (it->second.second >= bytes) {
      return count;
    }
    void *smaller = it->second.first;
    it->second = std::make_pair(count, bytes);
    return smaller;
  }

private:
  using Key = std::tuple<const void *, uint32_t, const void *>;
  std::mutex mu_;
  std::map<Key, std::pair<void *, size_t>> kept_;
};

ArrivalCounts &arrival_counts() {
  static ArrivalCounts *c = new ArrivalCounts();
  return *c;
}

/* One-rank job state (reference runtime/vx_collective.h:288-330). */
int32_t one_rank_ranks = 0;

void collective_fatal(const char *why) {
  fprintf(stderr, "[Vx HIP] FATAL: %s\n", why);
  abort();
}

void one_rank_copy(const void *in, void *out, int64_t count, size_t esz,
                   const char *name) {
  char msg[256];
  if (!one_rank_ranks) {
    snprintf(msg, sizeof(msg), "%s ran before vx_collective_init.", name);
    collective_fatal(msg);
  }
  if (count < 0) {
    snprintf(msg, sizeof(msg), "%s got a count of %lld.", name,
             (long long)count);
    collective_fatal(msg);
  }
  if (in == out || count == 0) {
    return;
  }
  const size_t bytes = (size_t)count * esz;
  if (is_device_ptr(in) || is_device_ptr(out)) {
    VX_HIP_CHECK(hipMemcpyAsync(out, in, bytes, hipMemcpyDefault,
                                caller_stream));
    started_kernel(name);
  } else {
    memmove(out, in, bytes);
  }
}

/* Staging of vx_hip_dispatch_async_noalloc: a fixed array in each device's
 * copy of this library's code object, allocated when the code object loads
 * and held until the process ends. Host code reaches it only through the
 * address hipGetSymbolAddress gives for the current device (the array's
 * name is a host-side stand-in, not a device address). */
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

/* One device's scratch: its address and the event recorded after the last
 * call that staged through it (null until then). */
struct Scratch {
  unsigned char *ptr = nullptr;
  hipEvent_t done = nullptr;
  std::mutex use; /* held by a call from its first staging copy to its record */
};

std::mutex scratch_mutex;
std::map<int, Scratch> &scratch_table() {
  static auto *m = new std::map<int, Scratch>();
  return *m;
}

/* This device's scratch, looked up (and its event created) once per device
 * with that device current; null (message printed) when the lookup fails. */
Scratch *noalloc_scratch() {
  int device = 0;
  VX_HIP_CHECK(hipGetDevice(&device));
  std::lock_guard<std::mutex> hold(scratch_mutex);
  Scratch &sc = scratch_table()[device];
  if (sc.ptr) {
    return &sc;
  }
  void *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) {
    (void)hipGetLastError();
    fprintf(stderr,
            "[Vx HIP] vx_hip_dispatch_async_noalloc: no scratch address on "
            "GPU %d: %s\n",
            device, hipGetErrorString(e));
    return nullptr;
  }
  hipEvent_t ev = nullptr;
  const hipError_t ee = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (ee != hipSuccess) {
    (void)hipGetLastError();
    fprintf(stderr,
            "[Vx HIP] vx_hip_dispatch_async_noalloc: no event on GPU %d: %s\n",
            device, hipGetErrorString(ee));
    return nullptr;
  }
  sc.ptr = static_cast<unsigned char *>(ptr);
  sc.done = ev;
  return &sc;
}

} // namespace

/* Used by the library ops (ops.cpp). */
namespace vxops {
hipStream_t stream() { return caller_stream; }
bool device_present() { return hip_available(); }
bool on_device(const void *p) { return is_device_ptr(p); }
void launched(const char *what) { started_kernel(what); }
bool chatty() { return verbose(); }
bool capturing() { return ::capturing(); }
} // namespace vxops

extern "C" {

void *vx_plugin_alloc_and_transfer(size_t bytes, void *host_ptr,
                                   uint32_t topology_id,
                                   uint32_t space_access) {
  if (!hip_available() || gpu_index((int32_t)topology_id) < 0) {
    void *p = malloc(bytes ? bytes : 1);
    if (p && host_ptr && bytes) {
      memcpy(p, host_ptr, bytes);
    }
    return p;
  }
  select_device((int32_t)topology_id, "stage");
  if (space_access == VX_SPACE_ACCESS_HOST_READABLE) {
    /* The model says the host may read this space; HBM is not host memory
     * (reference runtime/cuda_dispatch.cpp:1172-1197). */
    const char *strict = getenv("VX_STRICT_SPACES");
    fprintf(stderr,
            "[Vx HIP] %s: topology %u is declared host-readable, but its %zu "
            "bytes are GPU memory the host cannot read\n",
            strict ? "FATAL" : "WARNING", topology_id, bytes);
    if (strict) {
      abort();
    }
  }
  void *p = nullptr;
  VX_HIP_CHECK(device_alloc(&p, bytes ? bytes : 1));
  if (host_ptr && bytes) {
    if (capturing()) {
      refuse_in_capture("a tensor in host memory was copied to the GPU");
    }
    if (caller_stream) {
      VX_HIP_CHECK(hipMemcpyAsync(p, host_ptr, bytes, hipMemcpyHostToDevice,
                                  caller_stream));
      VX_HIP_CHECK(hipStreamSynchronize(caller_stream));
    } else {
      VX_HIP_CHECK(hipMemcpy(p, host_ptr, bytes, hipMemcpyHostToDevice));
    }
  }
  return p;
}

/* The copy ends before this returns, which the asynchronous contract allows:
 * "a device may still copy". */
void *vx_plugin_alloc_and_transfer_async(size_t bytes, void *host_ptr,
                                         uint32_t topology_id,
                                         uint32_t space_access) {
  return vx_plugin_alloc_and_transfer(bytes, host_ptr, topology_id,
                                      space_access);
}

uint64_t vx_plugin_dispatch_async(const void *binary_payload,
                                  size_t payload_size, void **device_args,
                                  const int32_t *arg_tags, int64_t num_args) {
  const int32_t abi = vx_payload_abi(binary_payload, payload_size);
  if (abi > VX_PAYLOAD_ABI) {
    fprintf(stderr,
            "[Vx HIP] FATAL: %s carries payload format abi=%d; this library "
            "reads formats up to %d\n",
            static_cast<const char *>(binary_payload), abi, VX_PAYLOAD_ABI);
    abort();
  }
  vx_gemm_plan plan;
  if (hip_available() &&
      vx_gemm_plan_decode(binary_payload, payload_size, device_args, arg_tags,
                          num_args, &plan)) {
    select_device(vx_payload_topology(binary_payload, payload_size),
                  "dispatch");
    if (run_gemm(plan)) {
      return 1;
    }
  }
  if (hip_available() && run_device_image(binary_payload, payload_size,
                                          device_args, arg_tags, num_args)) {
    return 1;
  }
  run_on_host(binary_payload, payload_size, device_args, arg_tags, num_args);
  return 1;
}

/* The kind=matmul dispatch without allocating: host operands and a host
 * result buffer are staged through this device's fixed scratch instead of
 * the pool. Everything else the ABI entry point would do that allocates or
 * blocks is refused (returns 0 with the reason on stderr, nothing
 * launched): regions that are not a routed GEMM, results published through
 * a slot (the program frees those with free()), staging beyond the scratch,
 * and staging while the caller stream captures a graph. Calls on one GPU
 * share its scratch and are ordered on it: a call that stages holds the
 * scratch from its first copy to the launch of its GEMM, and its stream
 * first waits (hipStreamWaitEvent) for the event the previous such call
 * recorded after its GEMM, so a later call on another stream or thread never
 * overwrites operands a GEMM still reads. */
uint64_t vx_hip_dispatch_async_noalloc(const void *binary_payload,
                                       size_t payload_size, void **device_args,
                                       const int32_t *arg_tags,
                                       int64_t num_args) {
  static const char op[] = "vx_hip_dispatch_async_noalloc";
  const int32_t abi = vx_payload_abi(binary_payload, payload_size);
  if (abi > VX_PAYLOAD_ABI) {
    fprintf(stderr, "[Vx HIP] %s: payload format abi=%d is newer than %d\n",
            op, abi, VX_PAYLOAD_ABI);
    return 0;
  }
  vx_gemm_plan plan;
  if (!hip_available() ||
      !vx_gemm_plan_decode(binary_payload, payload_size, device_args, arg_tags,
                           num_args, &plan)) {
    fprintf(stderr, "[Vx HIP] %s: %s is not a routed GEMM on a GPU\n", op,
            static_cast<const char *>(binary_payload));
    return 0;
  }
  if (plan.out_kind != VX_GEMM_OUT_BUFFER) {
    fprintf(stderr,
            "[Vx HIP] %s: a result published through a slot is host memory "
            "this entry point would have to allocate\n",
            op);
    return 0;
  }
  select_device(vx_payload_topology(binary_payload, payload_size), "dispatch");
  const size_t in_esz = vx_dtype_bytes(plan.dtype);
  const size_t out_esz = vx_dtype_bytes(plan.out_dtype);
  auto rounded = [](uint64_t b) { return (b + 255) / 256 * 256; };
  uint64_t need = 0;
  if (!is_device_ptr(plan.a_data)) {
    need += rounded((uint64_t)plan.m * (uint64_t)plan.k * in_esz);
  }
  if (!is_device_ptr(plan.b_data)) {
    need += rounded((uint64_t)plan.k * (uint64_t)plan.n * in_esz);
  }
  if (!is_device_ptr(plan.out_data)) {
    need += rounded((uint64_t)plan.m * (uint64_t)plan.n * out_esz);
  }
  if (need > kNoAllocScratchBytes) {
    fprintf(stderr,
            "[Vx HIP] %s: staging this GEMM's host operands takes %llu bytes; "
            "the scratch holds %zu\n",
            op, (unsigned long long)need, kNoAllocScratchBytes);
    return 0;
  }
  if (!need) {
    if (!run_gemm(plan, nullptr, true)) {
      fprintf(stderr, "[Vx HIP] %s: no GPU kernel takes this GEMM's types\n",
              op);
      return 0;
    }
    return 1;
  }
  if (capturing()) {
    fprintf(stderr,
            "[Vx HIP] %s: the caller stream is capturing a graph, and this "
            "GEMM has host operands or a host result, which a graph cannot "
            "copy in this call's order\n",
            op);
    return 0;
  }
  Scratch *sc = noalloc_scratch();
  if (!sc) {
    return 0;
  }
  std::lock_guard<std::mutex> hold(sc->use);
  VX_HIP_CHECK(hipStreamWaitEvent(caller_stream, sc->done, 0));
  Arena arena;
  arena.base = sc->ptr;
  arena.size = kNoAllocScratchBytes;
  if (!run_gemm(plan, &arena, true)) {
    fprintf(stderr, "[Vx HIP] %s: no GPU kernel takes this GEMM's types\n", op);
    return 0;
  }
  VX_HIP_CHECK(hipEventRecord(sc->done, caller_stream));
  return 1;
}

uint64_t vx_plugin_dispatch_async_flat(float *xout, float *x, float *w, int n,
                                       int d) {
  if (n <= 0 || d <= 0) {
    return 1;
  }
  if (!hip_available()) {
    /* No device: the plain loop the ABI documents (reference
     * runtime/host_dispatch_common.h:648-660). */
    for (int i = 0; i < d; ++i) {
      float acc = 0.0f;
      for (int j = 0; j < n; ++j) {
        acc += w[(size_t)i * n + j] * x[j];
      }
      xout[i] = acc;
    }
    return 1;
  }
  /* xout[d] = W[d,n] x[n] is a GEMM with m = d, k = n, N = 1. */
  DeviceOperand dw, dx, dy;
  stage(w, d, n, n, sizeof(float), dw, nullptr);
  stage(x, n, 1, 1, sizeof(float), dx, nullptr);
  const bool out_is_device = is_device_ptr(xout);
  if (out_is_device) {
    dy.ptr = xout;
  } else {
    dy.bytes = (size_t)d * sizeof(float);
    dy.ptr = pool().acquire(dy.bytes);
    dy.pooled = true;
  }
  vxk::GemmArgs g;
  g.in_dtype = g.out_dtype = VX_DTYPE_F32;
  g.m = d, g.n = 1, g.k = n;
  g.a = dw.ptr, g.b = dx.ptr, g.c = dy.ptr;
  g.lda = dw.row_stride, g.ldb = 1, g.ldc = 1;
  if (!vxk::gemm_launch(g, caller_stream)) {
    fprintf(stderr, "[Vx HIP] FATAL: no GPU kernel takes a %dx%d matvec\n", d,
            n);
    abort();
  }
  started_kernel("a matrix-vector product");
  if (!out_is_device) {
    wait_for_kernels("a matrix-vector product was copied to host memory");
    VX_HIP_CHECK(hipMemcpy(xout, dy.ptr, (size_t)d * sizeof(float),
                           hipMemcpyDeviceToHost));
  }
  return 1;
}

void vx_plugin_await_future(uint64_t future_id) {
  (void)future_id;
  if (hip_available()) {
    wait_for_kernels("a future was awaited");
  }
}

int32_t vx_plugin_transfer_device_to_host(void *device_ptr, void *host_ptr,
                                          size_t bytes, uint32_t topology_id) {
  if (is_device_ptr(device_ptr)) {
    select_device((int32_t)topology_id, "fetch");
    wait_for_kernels("a tensor was copied to host memory");
    VX_HIP_CHECK(hipMemcpy(host_ptr, device_ptr, bytes, hipMemcpyDeviceToHost));
  } else if (bytes) {
    memcpy(host_ptr, device_ptr, bytes);
  }
  return 1;
}

void *vx_plugin_transfer_peer(void *src_device_ptr, uint32_t src_topology_id,
                              uint32_t dst_topology_id, size_t bytes) {
  if (!is_device_ptr(src_device_ptr)) {
    void *dst = malloc(bytes ? bytes : 1);
    if (dst && src_device_ptr && bytes) {
      memcpy(dst, src_device_ptr, bytes);
    }
    return dst;
  }
  const int src = gpu_index((int32_t)src_topology_id);
  const int dst = gpu_index((int32_t)dst_topology_id);
  if (src < 0 || dst < 0) {
    fprintf(stderr,
            "[Vx HIP] FATAL: peer transfer between topologies %u and %u, "
            "which are not both GPUs\n",
            src_topology_id, dst_topology_id);
    abort();
  }
  select_device((int32_t)dst_topology_id, "peer");
  void *p = nullptr;
  VX_HIP_CHECK(device_alloc(&p, bytes ? bytes : 1));
  if (bytes) {
    if (src == dst) {
      VX_HIP_CHECK(hipMemcpyAsync(p, src_device_ptr, bytes,
                                  hipMemcpyDeviceToDevice, caller_stream));
    } else {
      VX_HIP_CHECK(hipMemcpyPeerAsync(p, dst, src_device_ptr, src, bytes,
                                      caller_stream));
    }
    started_kernel("a peer copy");
  }
  if (verbose()) {
    fprintf(stderr, "[Vx HIP] peer %d -> %d, %zu bytes\n", src, dst, bytes);
  }
  return p;
}

void vx_plugin_free(void *device_ptr, uint32_t topology_id) {
  if (!device_ptr) {
    return;
  }
  if (is_device_ptr(device_ptr)) {
    select_device((int32_t)topology_id, "free");
    device_free(device_ptr);
  } else {
    free(device_ptr);
  }
}

void *vx_plugin_arrivals_take(const void *site, size_t bytes, void *zeros,
                              uint32_t topology_id, uint32_t space_access) {
  if (void *kept = arrival_counts().take(site, topology_id, caller_stream,
                                         bytes)) {
    return kept;
  }
  return vx_plugin_alloc_and_transfer(bytes, zeros, topology_id, space_access);
}

void vx_plugin_arrivals_give(const void *site, void *count, size_t bytes,
                             uint32_t topology_id) {
  void *spare =
      arrival_counts().give(site, topology_id, caller_stream, count, bytes);
  if (spare) {
    vx_plugin_free(spare, topology_id);
  }
}

void vx_plugin_release_future(uint64_t future_id) { (void)future_id; }

int32_t vx_hip_image_param_count(const void *image, size_t image_size,
                                 const char *kernel) {
  return vx::code_object_param_count(image, image_size, "gfx950", kernel);
}

/* Vendor opcodes of this library (VX_CTRL_VENDOR_BASE and up). */
#define VX_HIP_CTRL_GEMM_KERNEL (VX_CTRL_VENDOR_BASE + 1)
#define VX_HIP_CTRL_STATS (VX_CTRL_VENDOR_BASE + 2)
#define VX_HIP_CTRL_POOL_DRAIN (VX_CTRL_VENDOR_BASE + 3)
#define VX_HIP_CTRL_IMAGE_STATS (VX_CTRL_VENDOR_BASE + 4)
#define VX_HIP_CTRL_CLOCK_STAMPS (VX_CTRL_VENDOR_BASE + 5)
#define VX_HIP_CTRL_GEMV_KERNEL (VX_CTRL_VENDOR_BASE + 6)
#define VX_HIP_CTRL_FA_SPLITS (VX_CTRL_VENDOR_BASE + 7)
#define VX_HIP_CTRL_FA_WORKSPACES (VX_CTRL_VENDOR_BASE + 8)
#define VX_HIP_CTRL_STAGING_STATS (VX_CTRL_VENDOR_BASE + 9)
#define VX_HIP_CTRL_GEMM_WORKSPACES (VX_CTRL_VENDOR_BASE + 10)

int32_t vx_plugin_control(uint32_t opcode, void *payload) {
  switch (opcode) {
  case VX_CTRL_GET_DEVICE_COUNT: {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    return n;
  }
  case VX_CTRL_INIT_DEVICE:
    return hip_available() ? 1 : 0;
  case VX_CTRL_WAIT:
  case VX_CTRL_WAIT_FOR_TENSORS:
  case VX_CTRL_WAIT_FOR_THREAD:
    if (hip_available()) {
      wait_for_kernels("a read of GPU memory in place");
    }
    return 1;
  case VX_CTRL_SHUTDOWN:
    if (hip_available()) {
      wait_for_kernels("shutdown");
      pool().drain();
    }
    return 1;
  case VX_CTRL_LOCAL_DEVICE: {
    const int32_t *pair = static_cast<const int32_t *>(payload);
    if (!pair) {
      return 0;
    }
    std::lock_guard<std::mutex> hold(local_devices_mutex);
    const size_t n = local_device_count.load(std::memory_order_relaxed);
    for (size_t i = 0; i < n; ++i) {
      if (local_devices[i].declared != pair[0]) {
        continue;
      }
      if (local_devices[i].builtin != pair[1]) {
        fprintf(stderr,
                "[Vx HIP] FATAL: the topology %d is declared as two local "
                "devices, %d and %d\n",
                pair[0], local_devices[i].builtin, pair[1]);
        abort();
      }
      return 1;
    }
    if (n == sizeof(local_devices) / sizeof(local_devices[0])) {
      fprintf(stderr, "[Vx HIP] FATAL: more than %zu declared local devices\n",
              n);
      abort();
    }
    local_devices[n] = {pair[0], pair[1]};
    local_device_count.store(n + 1, std::memory_order_release);
    return 1;
  }
  case VX_HIP_CTRL_GEMM_KERNEL: {
    /* payload -> int32_t: 0 automatic, 2 tiled (exact k order), 8 MFMA
     * ping-pong (16-bit inputs), 9 f32 on f32 MFMAs, 10 the ping-pong tiles
     * as a stream-K launch. A forced kernel applies where it takes the
     * shape. */
    const int32_t *which = static_cast<const int32_t *>(payload);
    if (!which || !(*which == 0 || *which == vxk::GEMM_TILED ||
                    *which == vxk::GEMM_MFMA_PP || *which == vxk::GEMM_F32_MFMA ||
                    *which == vxk::GEMM_MFMA_SK)) {
      return 0;
    }
    forced_gemm_kernel.store(*which);
    return 1;
  }
  case VX_HIP_CTRL_STATS: {
    /* payload -> int64_t[5]: routed GEMMs, of them MFMA, of them tiled, host
     * fallbacks, bytes staged from host memory. */
    int64_t *out = static_cast<int64_t *>(payload);
    if (!out) {
      return 0;
    }
    out[0] = stat_gemm_device.load();
    out[1] = stat_gemm_mfma.load();
    out[2] = stat_gemm_tiled.load();
    out[3] = stat_host_fallback.load();
    out[4] = stat_staged_bytes.load();
    return 1;
  }
  case VX_HIP_CTRL_IMAGE_STATS: {
    /* payload -> int64_t[2]: kernels launched from payload images, images
     * loaded (one per kernel, device and image). */
    int64_t *out = static_cast<int64_t *>(payload);
    if (!out) {
      return 0;
    }
    out[0] = stat_image_launches.load();
    out[1] = stat_image_loads.load();
    return 1;
  }
  case VX_HIP_CTRL_CLOCK_STAMPS: {
    /* payload -> {uint64_t *base; int64_t slots}: routed MFMA GEMMs record
     * their clock counters into base[4 * (launch % slots) ...] from now on
     * (base null: stop). The ring restarts at slot 0. */
    const struct {
      uint64_t *base;
      int64_t slots;
    } *ring = static_cast<const decltype(ring)>(payload);
    if (!ring || ring->slots < 0 || (ring->base && !is_device_ptr(ring->base))) {
      return 0;
    }
    std::lock_guard<std::mutex> hold(stamps_mutex);
    stamps_base = ring->base;
    stamps_slots = ring->slots;
    stamps_next = 0;
    return 1;
  }
  case VX_HIP_CTRL_GEMV_KERNEL: {
    /* payload -> int32_t: 0 automatic, 1 one-burst dot2 rows (batch 1-2),
     * 2 grid-stride dot2 (batch <= 4, cols <= 4096), 3 MFMA through LDS
     * tiles. A forced kernel that does not take a shape makes the op answer
     * VX_OP_EUNSUPP. */
    const int32_t *which = static_cast<const int32_t *>(payload);
    if (!which || *which < 0 || *which > 3) {
      return 0;
    }
    vxk::gemv_i8_force(static_cast<vxk::GemvKernel>(*which));
    return 1;
  }
  case VX_HIP_CTRL_FA_SPLITS: {
    /* payload -> int32_t: 0 automatic, n in 1..64 cuts every flash-attention
     * launch's key range into n splits (fewer when there are fewer key
     * blocks) wherever splitting is allowed. */
    const int32_t *splits = static_cast<const int32_t *>(payload);
    if (!splits || *splits < 0 || *splits > 64) {
      return 0;
    }
    vxk::flash_attn_force_splits(*splits);
    return 1;
  }
  case VX_HIP_CTRL_STAGING_STATS: {
    /* payload -> int64_t[3]: staging-pool acquires (reuses plus new
     * allocations), of them new allocations, bytes staged through the
     * no-alloc scratch. */
    int64_t *out = static_cast<int64_t *>(payload);
    if (!out) {
      return 0;
    }
    out[0] = (int64_t)(pool().hits() + pool().misses());
    out[1] = (int64_t)pool().misses();
    out[2] = stat_scratch_staged_bytes.load();
    return 1;
  }
  case VX_HIP_CTRL_FA_WORKSPACES: {
    /* payload -> int64_t[2]: flash-attention split workspaces held (one per
     * device and stream that split a launch) and their bytes. */
    int64_t *out = static_cast<int64_t *>(payload);
    if (!out) {
      return 0;
    }
    vxk::flash_attn_workspace_stats(&out[0], &out[1]);
    return 1;
  }
  case VX_HIP_CTRL_GEMM_WORKSPACES: {
    /* payload -> int64_t[4]: stream-K GEMM workspaces held (one per device
     * and stream that ran such a launch), their bytes, stream-K launches so
     * far, and the workgroups such a launch runs on the current device (its
     * CU count). */
    int64_t *out = static_cast<int64_t *>(payload);
    if (!out || !hip_available()) {
      return 0;
    }
    vxk::gemm_workspace_stats(&out[0], &out[1], &out[2]);
    out[3] = vxk::device_cu_count();
    return 1;
  }
  case VX_HIP_CTRL_POOL_DRAIN:
    if (hip_available()) {
      wait_for_kernels("pool drain");
      pool().drain();
    }
    return 1;
  default:
    return 0;
  }
}

/* No TMA on AMD hardware: a kernel asking for a tensor map gets 0 and copies
 * its tile itself (reference runtime/host_dispatch_common.h:727-738). */
int64_t vx_plugin_tensor_map(int64_t base, int64_t rank, int64_t elem_bytes,
                             int64_t d0, int64_t d1, int64_t d2, int64_t d3,
                             int64_t d4, int64_t s0, int64_t s1, int64_t s2,
                             int64_t s3, int64_t s4, int64_t b0, int64_t b1,
                             int64_t b2, int64_t b3, int64_t b4) {
  (void)base, (void)rank, (void)elem_bytes, (void)d0, (void)d1, (void)d2;
  (void)d3, (void)d4, (void)s0, (void)s1, (void)s2, (void)s3, (void)s4;
  (void)b0, (void)b1, (void)b2, (void)b3, (void)b4;
  return 0;
}

/* The caller stream, as a hipStream_t. The CUDA-named pair is what compiled
 * programs and host code already call (reference
 * runtime/cuda_dispatch.cpp:2030-2035); the HIP-named pair is the same.
 * Moving off a stream frees, in that stream's order, the flash-attention
 * split workspace and the stream-K GEMM workspace the library kept for it,
 * so a stream the caller then
 * destroys leaves nothing behind and a later stream at the same address
 * starts with none. A stream must stay alive while it is set. */
void vx_hip_set_stream(void *stream) {
  const hipStream_t next = static_cast<hipStream_t>(stream);
  if (caller_stream && caller_stream != next) {
    vxk::flash_attn_release_stream(caller_stream);
    vxk::gemm_release_stream(caller_stream);
  }
  caller_stream = next;
}
void vx_cuda_set_stream(void *stream) { vx_hip_set_stream(stream); }
void *vx_cuda_get_stream(void) { return caller_stream; }
void *vx_hip_get_stream(void) { return caller_stream; }

void vx_collective_init(int32_t rank, int32_t ranks) {
  char msg[256];
  if (one_rank_ranks) {
    collective_fatal("vx_collective_init ran a second time. Call "
                     "vx_collective_finish first.");
  }
  if (ranks != 1 || rank != 0) {
    snprintf(msg, sizeof(msg),
             "vx_collective_init got rank %d of %d ranks, but this process "
             "runs a job of one rank only: this build joins no other GPUs.",
             rank, ranks);
    collective_fatal(msg);
  }
  one_rank_ranks = 1;
}

void vx_collective_finish(void) {
  if (!one_rank_ranks) {
    collective_fatal("vx_collective_finish ran before vx_collective_init.");
  }
  one_rank_ranks = 0;
}

int32_t vx_collective_rank(void) { return one_rank_ranks ? 0 : -1; }
int32_t vx_collective_ranks(void) { return one_rank_ranks; }

void vx_collective_all_reduce_sum_f32(const float *input, float *output,
                                      int64_t count) {
  one_rank_copy(input, output, count, 4, "vx_collective_all_reduce_sum_f32");
}
void vx_collective_all_reduce_sum_bf16(const uint16_t *input, uint16_t *output,
                                       int64_t count) {
  one_rank_copy(input, output, count, 2, "vx_collective_all_reduce_sum_bf16");
}
void vx_collective_all_gather_f32(const float *input, float *output,
                                  int64_t count) {
  one_rank_copy(input, output, count, 4, "vx_collective_all_gather_f32");
}
void vx_collective_all_gather_bf16(const uint16_t *input, uint16_t *output,
                                   int64_t count) {
  one_rank_copy(input, output, count, 2, "vx_collective_all_gather_bf16");
}

int64_t vx_host_worker_id(void) { return vx::host_worker_index; }
int64_t vx_host_worker_count(void) { return vx::host_worker_total; }

} // extern "C"
