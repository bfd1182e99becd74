/*
 * read_probe.hip -- the measured HBM read ceiling the benchmark sets the
 * int8 GEMV entries beside (bench.py builds nothing: __graft_entry__.build()
 * compiles this file to read_probe.hsaco next to it, and bench.py launches
 * it through HIP's module API). Not part of the dispatch library.
 *
 * vx_read_probe_<n>_<a>: workgroup g reads the contiguous 16-byte units
 * [g * 256 n, (g + 1) * 256 n) of `src` with cache-policy bits a (0, or 2:
 * non-temporal, as the GEMV's weight loads) -- n units per thread, every load
 * issued before any is used -- and folds them into one word that is stored
 * only if it equals a value the data never produces (so the loads cannot be
 * dropped and nothing is written). One burst per workgroup, the read shape
 * the one-burst GEMV kernels use.
 */
#include <hip/hip_runtime.h>

#include <cstdint>

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <int kUnits, int kAux>
__device__ __forceinline__ void read_burst(const u32x4 *__restrict__ src,
                                           unsigned *__restrict__ out) {
  constexpr int kBytes = 256 * kUnits * 16;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(src + (uint64_t)blockIdx.x * 256 * kUnits), (short)0, kBytes, 0x00020000);
  u32x4 v[kUnits];
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(threadIdx.x * 16), i * 4096, kAux);
  }
  __builtin_amdgcn_sched_barrier(0);
  unsigned acc = 0;
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  }
  if (acc == 0x9e3779b9u) {
    out[blockIdx.x * 256 + threadIdx.x] = acc;
  }
}

/* 16, 32 and 64 KiB per workgroup, with default and non-temporal (nt)
 * loads: vx_read_probe_<units per thread>_<cache-policy bits>. */
#define VX_READ_PROBE(U, A)                                                    \
  extern "C" __global__ __launch_bounds__(256) void vx_read_probe_##U##_##A(  \
      const u32x4 *__restrict__ src, unsigned *__restrict__ out) {             \
    read_burst<U, A>(src, out);                                                \
  }
VX_READ_PROBE(4, 0)
VX_READ_PROBE(8, 0)
VX_READ_PROBE(16, 0)
VX_READ_PROBE(4, 2)
VX_READ_PROBE(8, 2)
VX_READ_PROBE(16, 2)
