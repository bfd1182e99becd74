/*
 * vx_device_pool_hip.h -- reuse of per-dispatch staging buffers in HBM.
 *
 * A dispatch whose operands are in host memory stages them into device
 * buffers; allocating and freeing those per call costs more than a mid-sized
 * GEMM (the reference measured 51% of a 2048^2 dispatch in the allocator,
 * runtime/vx_device_pool.h:12-17). This keeps released buffers on a free list
 * keyed by exact byte count and hands them out again.
 *
 * Same contract as the reference pool (runtime/vx_device_pool.h:52-175),
 * written for HIP:
 *  - exact-size buckets: a staging buffer is always the operand's packed size,
 *    so sizes repeat call after call and no buffer is ever split;
 *  - a cap on bytes held idle (VX_HIP_POOL_MAX_MB, default 2048 MiB; 288 GB of
 *    HBM leaves room, but idle memory is still memory a program cannot use);
 *  - on allocation failure the idle buffers are released and the allocation
 *    is retried once;
 *  - the lock is never held across an allocator call.
 * The allocator pair is a template parameter so tests drive it with a fake.
 */
#ifndef VX_AMD_DEVICE_POOL_HIP_H
#define VX_AMD_DEVICE_POOL_HIP_H

#include <cstddef>
#include <cstdlib>
#include <map>
#include <mutex>
#include <vector>

namespace vx {

template <typename Alloc, typename Free> class HipDevicePool {
public:
  HipDevicePool(Alloc alloc, Free release, size_t cap_bytes)
      : alloc_(alloc), free_(release), cap_(cap_bytes) {}

  /* A buffer of exactly `bytes`, or nullptr when even a retry after
   * releasing every idle buffer fails. */
  void *acquire(size_t bytes) {
    if (bytes == 0) {
      return nullptr;
    }
    {
      std::lock_guard<std::mutex> hold(mu_);
      auto it = idle_.find(bytes);
      if (it != idle_.end() && !it->second.empty()) {
        void *p = it->second.back();
        it->second.pop_back();
        idle_bytes_ -= bytes;
        ++hits_;
        return p;
      }
      ++misses_;
    }
    void *p = alloc_(bytes);
    if (!p) {
      drain();
      p = alloc_(bytes);
    }
    return p;
  }

  /* Return a buffer from acquire(). Kept when it fits under the cap. */
  void release(void *p, size_t bytes) {
    if (!p) {
      return;
    }
    {
      std::lock_guard<std::mutex> hold(mu_);
      if (idle_bytes_ + bytes <= cap_) {
        idle_[bytes].push_back(p);
        idle_bytes_ += bytes;
        return;
      }
    }
    free_(p, bytes);
  }

  /* Free every idle buffer. */
  void drain() {
    std::map<size_t, std::vector<void *>> taken;
    {
      std::lock_guard<std::mutex> hold(mu_);
      taken.swap(idle_);
      idle_bytes_ = 0;
    }
    for (auto &bucket : taken) {
      for (void *p : bucket.second) {
        free_(p, bucket.first);
      }
    }
  }

  size_t idle_bytes() {
    std::lock_guard<std::mutex> hold(mu_);
    return idle_bytes_;
  }
  size_t hits() {
    std::lock_guard<std::mutex> hold(mu_);
    return hits_;
  }
  size_t misses() {
    std::lock_guard<std::mutex> hold(mu_);
    return misses_;
  }

private:
  Alloc alloc_;
  Free free_;
  size_t cap_;
  std::mutex mu_;
  std::map<size_t, std::vector<void *>> idle_;
  size_t idle_bytes_ = 0;
  size_t hits_ = 0;
  size_t misses_ = 0;
};

/* The cap from VX_HIP_POOL_MAX_MB, in bytes; 2048 MiB when unset or invalid. */
inline size_t hip_pool_cap_from_env() {
  const char *v = getenv("VX_HIP_POOL_MAX_MB");
  if (v && *v) {
    char *end = nullptr;
    long long mb = strtoll(v, &end, 10);
    if (end != v && *end == '\0' && mb >= 0) {
      return (size_t)mb << 20;
    }
  }
  return (size_t)2048 << 20;
}

} // namespace vx

#endif /* VX_AMD_DEVICE_POOL_HIP_H */
