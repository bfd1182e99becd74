// pool_threads_test.cpp -- the staging pool (vx_amd/csrc/vx_device_pool_hip.h)
// under concurrent dispatch: dispatches may come from several threads
// (reference runtime/cuda_dispatch.cpp:1387-1390 keeps its caches behind a
// mutex; runtime/vx_device_pool.h:46-51 never holds the pool lock across an
// allocator call). Eight threads acquire and release buffers of a few sizes
// against a fake allocator whose calls are slow enough to overlap; each
// thread stamps every buffer it holds and checks the stamp before release,
// so a buffer handed to two threads at once is caught. The allocator's
// books must balance at the end, and the idle bytes must respect the cap.
// Built by tests/test_native.py (also under ThreadSanitizer); prints "ok".

#include "../../vx_amd/csrc/vx_device_pool_hip.h"

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

namespace {

std::atomic<int64_t> live_allocs{0};
std::atomic<int64_t> total_allocs{0};
std::atomic<int64_t> total_frees{0};
std::atomic<int> failures{0};
std::atomic<int64_t> refused{0};
/* Every 50th allocation a thread asks for is refused (never two in a row on
 * one thread, so the pool's drain-and-retry always succeeds). */
thread_local int alloc_calls = 0;

void *fake_alloc(size_t bytes) {
  if (++alloc_calls % 50 == 0) {
    ++refused;
    return nullptr;
  }
  std::this_thread::yield();
  void *p = malloc(bytes);
  if (p) {
    ++live_allocs;
    ++total_allocs;
  }
  return p;
}

void fake_free(void *p, size_t bytes) {
  (void)bytes;
  std::this_thread::yield();
  free(p);
  --live_allocs;
  ++total_frees;
}

using Pool = vx::HipDevicePool<void *(*)(size_t), void (*)(void *, size_t)>;

void check(bool ok, const char *what) {
  if (!ok) {
    fprintf(stderr, "FAIL: %s\n", what);
    ++failures;
  }
}

void worker(Pool &pool, int id, int rounds) {
  static const size_t kSizes[] = {64, 256, 4096, 65536};
  uint32_t state = 0x9e3779b9u * (uint32_t)(id + 1);
  std::vector<std::pair<uint32_t *, size_t>> held;
  for (int r = 0; r < rounds; ++r) {
    state = state * 1664525u + 1013904223u;
    const size_t bytes = kSizes[(state >> 16) % 4];
    auto *p = static_cast<uint32_t *>(pool.acquire(bytes));
    if (!p) {
      check(false, "acquire returned null");
      continue;
    }
    for (size_t i = 0; i < bytes / 4; ++i) {
      p[i] = (uint32_t)id * 2654435761u + (uint32_t)i;
    }
    held.emplace_back(p, bytes);
    /* hold up to three buffers, releasing the oldest */
    if (held.size() > 3 || (state & 1)) {
      auto [q, qb] = held.front();
      held.erase(held.begin());
      bool intact = true;
      for (size_t i = 0; i < qb / 4; ++i) {
        intact &= q[i] == (uint32_t)id * 2654435761u + (uint32_t)i;
      }
      check(intact, "a held buffer was written by another thread");
      pool.release(q, qb);
    }
  }
  for (auto [q, qb] : held) {
    pool.release(q, qb);
  }
}

} // namespace

int main() {
  {
    const size_t cap = 256 * 1024;
    Pool pool(fake_alloc, fake_free, cap);
    std::vector<std::thread> threads;
    for (int id = 0; id < 8; ++id) {
      threads.emplace_back(worker, std::ref(pool), id, 4000);
    }
    for (auto &t : threads) {
      t.join();
    }
    check(refused.load() > 0, "some allocations were refused and retried");
    check(pool.idle_bytes() <= cap, "idle bytes over the cap");
    check(pool.hits() + pool.misses() == 8 * 4000, "every acquire counted once");
    check(pool.hits() > 0, "buffers were reused");
    /* everything not freed is idle in the pool */
    pool.drain();
    check(pool.idle_bytes() == 0, "drain leaves nothing idle");
    check(live_allocs.load() == 0, "every allocation freed after the drain");
    check(total_allocs.load() == total_frees.load(), "allocator books balance");
  }
  if (failures.load()) {
    return 1;
  }
  printf("ok\n");
  return 0;
}
