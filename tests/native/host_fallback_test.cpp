// host_fallback_test.cpp -- GPU-free tests of vx_amd/csrc/vx_host_fallback.h:
// the span planner for HBM views, the call through libffi, the copies back,
// results published through a slot, and the host-worker split.
//
// "HBM" here is an arena the is_device hook recognises; the copy hooks are
// memcpy loops. The cases follow what the reference's planner must get right
// (reference runtime/vx_view_copy.h:14-23, tests/runtime/view_copy_test.cpp):
// one tensor passed as output and input in either order, overlapping row
// ranges, a transposed view, a column copied densely, a view published
// through a slot, empty and touching views.

#include "../../vx_amd/csrc/vx_host_fallback.h"

#include <atomic>
#include <cstdio>
#include <string>
#include <vector>

namespace {

int failures = 0;

void check(bool ok, const char *what) {
  if (!ok) {
    fprintf(stderr, "FAIL: %s\n", what);
    ++failures;
  }
}

template <int R> struct Desc {
  void *allocated;
  void *aligned;
  int64_t offset;
  int64_t sizes[R];
  int64_t strides[R];
};
using D1 = Desc<1>;
using D2 = Desc<2>;

struct Slot {
  void *allocated;
  void *aligned;
  int64_t offset;
};

/* The fake HBM: one arena; copies counted so a test can see each span moved
 * once per direction. */
std::vector<float> hbm(4096);
int copies_out = 0, copies_in = 0;
size_t bytes_out = 0;

bool in_hbm(const void *p) {
  const char *c = static_cast<const char *>(p);
  const char *b = reinterpret_cast<const char *>(hbm.data());
  return c >= b && c < b + hbm.size() * sizeof(float);
}

vx::HostCopies hooks() {
  vx::HostCopies io;
  io.is_device = in_hbm;
  io.sync = [] {};
  io.to_host = [](void *dst, size_t dp, const void *src, size_t sp, size_t w,
                  size_t h) {
    ++copies_out;
    bytes_out += w * h;
    for (size_t r = 0; r < h; ++r) {
      memcpy((char *)dst + r * dp, (const char *)src + r * sp, w);
    }
  };
  io.to_device = [](void *dst, size_t dp, const void *src, size_t sp, size_t w,
                    size_t h) {
    ++copies_in;
    for (size_t r = 0; r < h; ++r) {
      memcpy((char *)dst + r * dp, (const char *)src + r * sp, w);
    }
  };
  return io;
}

constexpr int32_t tag(int slot, int rank, int dtype) {
  return (int32_t)(((uint32_t)slot << 24) | ((uint32_t)rank << 16) |
                   ((uint32_t)dtype << 8) | (uint32_t)VX_ABI_KIND_MEMREF);
}
constexpr int32_t kF32_1 = tag(0, 1, VX_DTYPE_F32);
constexpr int32_t kF32_2 = tag(0, 2, VX_DTYPE_F32);

int call(void *kernel, std::vector<void *> args, std::vector<int32_t> tags,
         int workers = 1) {
  int64_t bad = -1;
  copies_out = copies_in = 0;
  bytes_out = 0;
  return vx::call_on_host(kernel, args.data(), tags.data(),
                          (int64_t)args.size(), workers, false, hooks(), &bad);
}

D1 vec(float *p, int64_t n, int64_t off = 0, int64_t stride = 1) {
  D1 d{};
  d.allocated = d.aligned = p;
  d.offset = off;
  d.sizes[0] = n;
  d.strides[0] = stride;
  return d;
}

D2 mat(float *p, int64_t rows, int64_t cols, int64_t rs, int64_t cs,
       int64_t off = 0) {
  D2 d{};
  d.allocated = d.aligned = p;
  d.offset = off;
  d.sizes[0] = rows;
  d.sizes[1] = cols;
  d.strides[0] = rs;
  d.strides[1] = cs;
  return d;
}

float &at(D1 *d, int64_t i) {
  return static_cast<float *>(d->aligned)[d->offset + i * d->strides[0]];
}
float &at(D2 *d, int64_t i, int64_t j) {
  return static_cast<float *>(
      d->aligned)[d->offset + i * d->strides[0] + j * d->strides[1]];
}

/* Outlined kernels in the C-interface shape: descriptors by pointer. */
extern "C" void k_out_in(D1 *out, D1 *in) {
  for (int64_t i = 0; i < out->sizes[0]; ++i) {
    at(out, i) = at(in, i) + 1.0f;
  }
}
extern "C" void k_in_out(D1 *in, D1 *out) {
  for (int64_t i = 0; i < out->sizes[0]; ++i) {
    at(out, i) = at(in, i) * 3.0f;
  }
}
/* b += 10, then a *= 2, over two row views that may overlap. */
extern "C" void k_rows(D2 *a, D2 *b) {
  for (int64_t i = 0; i < b->sizes[0]; ++i) {
    for (int64_t j = 0; j < b->sizes[1]; ++j) {
      at(b, i, j) += 10.0f;
    }
  }
  for (int64_t i = 0; i < a->sizes[0]; ++i) {
    for (int64_t j = 0; j < a->sizes[1]; ++j) {
      at(a, i, j) *= 2.0f;
    }
  }
}
/* t[i][j] = 100 i + j through whatever strides the call gives. */
std::vector<int64_t> seen_strides;
extern "C" void k_fill2(D2 *t) {
  seen_strides = {t->strides[0], t->strides[1]};
  for (int64_t i = 0; i < t->sizes[0]; ++i) {
    for (int64_t j = 0; j < t->sizes[1]; ++j) {
      at(t, i, j) = (float)(100 * i + j);
    }
  }
}
extern "C" void k_fill1(D1 *t) {
  seen_strides = {t->strides[0]};
  for (int64_t i = 0; i < t->sizes[0]; ++i) {
    at(t, i) = (float)(7 * i + 1);
  }
}
/* Fills the view a slot holds, publishing nothing new. */
extern "C" void k_fill_slot(Slot *slot) {
  k_fill1(static_cast<D1 *>(slot->aligned));
}
/* Publishes `in` (from its second element on) through the slot, as a region
 * that ends in a view of an operand does. */
extern "C" void k_publish_tail(Slot *slot, D1 *in) {
  D1 *out = static_cast<D1 *>(slot->aligned);
  *out = *in;
  out->offset += out->strides[0];
  out->sizes[0] -= 1;
}
/* Publishes a fresh host buffer. */
float fresh[4] = {1, 2, 3, 4};
extern "C" void k_publish_fresh(Slot *slot, D1 *in) {
  (void)in;
  D1 *out = static_cast<D1 *>(slot->aligned);
  *out = vec(fresh, 4);
}
/* Each worker fills its slice of 0..n (the split a `launch=` region
 * compiles to). */
std::atomic<int> worker_calls{0};
std::atomic<int> max_total{0};
extern "C" void k_split(D1 *out) {
  const int64_t w = vx::host_worker_index, t = vx::host_worker_total;
  worker_calls++;
  if (t > max_total) {
    max_total = (int)t;
  }
  for (int64_t i = w; i < out->sizes[0]; i += t) {
    at(out, i) += 1.0f;
  }
}

void fill_hbm() {
  for (size_t i = 0; i < hbm.size(); ++i) {
    hbm[i] = (float)i;
  }
}

void test_same_buffer_out_then_in() {
  fill_hbm();
  D1 d = vec(hbm.data(), 16, 4);
  void *p = &d, *q = &d;
  check(call((void *)k_out_in, {&p, &q}, {kF32_1, kF32_1}) == 1, "call 1");
  bool ok = true;
  for (int i = 0; i < 16; ++i) {
    ok &= hbm[4 + i] == (float)(4 + i) + 1.0f;
  }
  check(ok, "one buffer as output then input: the result survives");
  check(copies_out == 1 && copies_in == 1, "one span copied once each way");
  check(hbm[3] == 3.0f && hbm[20] == 20.0f, "bytes outside the view untouched");
}

void test_same_buffer_in_then_out() {
  fill_hbm();
  /* Two descriptors of the same bytes (the compiler may pass two). */
  D1 a = vec(hbm.data(), 16, 4), b = vec(hbm.data(), 16, 4);
  void *p = &a, *q = &b;
  check(call((void *)k_in_out, {&p, &q}, {kF32_1, kF32_1}) == 1, "call 2");
  bool ok = true;
  for (int i = 0; i < 16; ++i) {
    ok &= hbm[4 + i] == (float)(4 + i) * 3.0f;
  }
  check(ok, "one buffer as input then output");
  check(copies_out == 1 && copies_in == 1, "one span for two descriptors");
}

void test_overlapping_rows() {
  fill_hbm();
  /* 6 x 8 matrix at hbm[0]; a = rows 0..3, b = rows 2..5. */
  std::vector<float> want(hbm.begin(), hbm.begin() + 48);
  for (int i = 2; i < 6; ++i)
    for (int j = 0; j < 8; ++j) want[i * 8 + j] += 10.0f;
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 8; ++j) want[i * 8 + j] *= 2.0f;
  D2 a = mat(hbm.data(), 4, 8, 8, 1, 0), b = mat(hbm.data(), 4, 8, 8, 1, 16);
  void *p = &a, *q = &b;
  check(call((void *)k_rows, {&p, &q}, {kF32_2, kF32_2}) == 1, "call 3");
  bool ok = true;
  for (int i = 0; i < 48; ++i) {
    ok &= hbm[i] == want[i];
  }
  check(ok, "overlapping row views see one copy");
  check(copies_out == 1 && copies_in == 1, "overlapping rows: one span");
  check(bytes_out == 48 * 4, "the span covers both views' rows");
}

void test_touching_views_stay_apart() {
  fill_hbm();
  D2 a = mat(hbm.data(), 2, 8, 8, 1, 0), b = mat(hbm.data(), 2, 8, 8, 1, 16);
  void *p = &a, *q = &b;
  check(call((void *)k_rows, {&p, &q}, {kF32_2, kF32_2}) == 1, "call 4");
  check(copies_out == 2 && copies_in == 2, "touching views: two spans");
  check(hbm[0] == 0.0f && hbm[9] == 18.0f && hbm[16] == 26.0f,
        "touching views: results");
}

void test_transposed_view() {
  fill_hbm();
  /* A 3 x 5 matrix at hbm[100] seen as its 5 x 3 transpose: the view covers
   * its whole span, so it is copied as bytes and keeps its strides. */
  D2 t = mat(hbm.data(), 5, 3, 1, 5, 100);
  void *p = &t;
  check(call((void *)k_fill2, {&p}, {kF32_2}) == 1, "call 5");
  bool ok = true;
  for (int i = 0; i < 5; ++i)
    for (int j = 0; j < 3; ++j) ok &= hbm[100 + j * 5 + i] == (float)(100 * i + j);
  check(ok, "transposed view written through");
  check(seen_strides == std::vector<int64_t>({1, 5}), "transposed keeps strides");
  check(hbm[99] == 99.0f && hbm[115] == 115.0f, "transposed: neighbours kept");
}

void test_dense_column_and_block() {
  fill_hbm();
  /* Column 3 of a 6 x 8 matrix: 6 elements spread over 41. */
  D1 col = vec(hbm.data(), 6, 3, 8);
  void *p = &col;
  check(call((void *)k_fill1, {&p}, {kF32_1}) == 1, "call 6");
  bool ok = true;
  for (int i = 0; i < 6; ++i) ok &= hbm[3 + 8 * i] == (float)(7 * i + 1);
  check(ok, "column written back");
  check(seen_strides == std::vector<int64_t>({1}), "column seen densely");
  check(bytes_out == 6 * 4, "column: only its elements copied");
  check(hbm[4] == 4.0f && hbm[12] == 12.0f, "column: other columns kept");

  /* A transposed 3 x 2 block of a 4 x 8 matrix at hbm[200]: view[i][j] =
   * m[j][i + 1]. */
  fill_hbm();
  D2 blk = mat(hbm.data(), 3, 2, 1, 8, 201);
  p = &blk;
  check(call((void *)k_fill2, {&p}, {kF32_2}) == 1, "call 7");
  ok = true;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 2; ++j) ok &= hbm[200 + j * 8 + i + 1] == (float)(100 * i + j);
  check(ok, "transposed block written back");
  check(seen_strides == std::vector<int64_t>({2, 1}), "block seen row-major");
  check(bytes_out == 6 * 4, "block: only its elements copied");
  check(hbm[200] == 200.0f && hbm[204] == 204.0f, "block: neighbours kept");
}

void test_publish_view_of_operand() {
  fill_hbm();
  /* The slot holds an HBM view (the region's output storage); the region
   * publishes a view of its input instead. */
  D1 held = vec(hbm.data(), 4, 500);
  Slot s{&held, &held, 0};
  void *sp = &s;
  D1 in = vec(hbm.data(), 8, 300);
  void *ip = &in;
  check(call((void *)k_publish_tail, {&sp, &ip},
             {tag(1, 1, VX_DTYPE_F32), kF32_1}) == 1,
        "call 8");
  check(held.aligned == hbm.data() && held.allocated == hbm.data(),
        "published view points at HBM again");
  check(held.offset == 301 && held.sizes[0] == 7 && held.strides[0] == 1,
        "published view keeps its own offset on top of the operand's");

  /* A dense operand (a column) published whole: back in its own layout. */
  D1 held2 = vec(hbm.data(), 4, 500);
  Slot s2{&held2, &held2, 0};
  sp = &s2;
  D1 col = vec(hbm.data(), 6, 3, 8);
  ip = &col;
  check(call((void *)k_publish_tail, {&sp, &ip},
             {tag(1, 1, VX_DTYPE_F32), kF32_1}) == 1,
        "call 9");
  check(held2.aligned == hbm.data() && held2.offset == 3 + 8 &&
            held2.strides[0] == 8 && held2.sizes[0] == 5,
        "published tail of a dense copy restored to the column's layout");

  /* A slot whose held view the region leaves alone publishes nothing. */
  D1 held3 = vec(hbm.data(), 4, 500);
  Slot s3{&held3, &held3, 0};
  sp = &s3;
  check(call((void *)k_fill_slot, {&sp}, {tag(1, 1, VX_DTYPE_F32)}) == 1,
        "call 10");
  check(held3.aligned == hbm.data() && held3.offset == 500,
        "untouched slot keeps its descriptor");
  check(hbm[500] == 1.0f && hbm[503] == 22.0f, "slot's view written back");

  /* A fresh host result passes through. */
  D1 held4 = vec(hbm.data(), 4, 500);
  Slot s4{&held4, &held4, 0};
  sp = &s4;
  ip = &in;
  check(call((void *)k_publish_fresh, {&sp, &ip},
             {tag(1, 1, VX_DTYPE_F32), kF32_1}) == 1,
        "call 11");
  check(held4.aligned == fresh, "fresh host result handed back as is");
}

void test_empty_and_host_views() {
  fill_hbm();
  D1 empty = vec(hbm.data(), 0, 7);
  void *p = &empty;
  check(call((void *)k_fill1, {&p}, {kF32_1}) == 1, "call 12");
  check(copies_out == 0 && copies_in == 0, "empty view: no copies");
  float host[5] = {0};
  D1 h = vec(host, 5);
  p = &h;
  check(call((void *)k_fill1, {&p}, {kF32_1}) == 1, "call 13");
  check(copies_out == 0 && host[4] == 29.0f, "host view passed through");
}

void test_plan_directly() {
  /* Three views: [0,40) and [32,72) join; [100,104) alone; an empty one. */
  fill_hbm();
  D1 a = vec(hbm.data(), 10, 0), b = vec(hbm.data(), 10, 8),
     c = vec(hbm.data(), 1, 25), e = vec(hbm.data(), 0, 3);
  std::vector<vx::HbmView> views(4);
  D1 *ds[] = {&b, &c, &a, &e};
  for (int i = 0; i < 4; ++i) {
    views[(size_t)i].desc = ds[i];
    views[(size_t)i].rank = 1;
    views[(size_t)i].elem = VX_DTYPE_F32;
  }
  std::vector<vx::HbmSpan> spans;
  size_t bad = 0;
  check(vx::plan_spans(views, spans, &bad), "plan ok");
  check(spans.size() == 2, "two spans");
  check(views[0].span == views[2].span && views[1].span != views[0].span,
        "overlapping views share a span");
  check(views[3].span == -1, "empty view has no span");
  const vx::HbmSpan &s = spans[(size_t)views[0].span];
  check(s.bytes == 18 * 4 && views[2].at == 0 && views[0].at == 8 * 4,
        "span bounds and offsets");
  D1 neg = vec(hbm.data(), 2, -1);
  std::vector<vx::HbmView> bad_views(1);
  bad_views[0].desc = &neg;
  bad_views[0].rank = 1;
  bad_views[0].elem = VX_DTYPE_F32;
  check(!vx::plan_spans(bad_views, spans, &bad) && bad == 0,
        "negative offset refused");
}

void test_workers() {
  fill_hbm();
  std::string payload("k");
  payload.push_back('\0');
  payload += "launch=64";
  payload.push_back('\0');
  D1 out = vec(hbm.data(), 64, 1000);
  void *p = &out;
  int32_t t = kF32_1;
  setenv("VX_HOST_THREADS", "4", 1);
  const int n = vx::host_worker_count_for(payload.data(), payload.size(), &p,
                                          &t, 1);
  check(n == 4, "VX_HOST_THREADS=4 gives 4 workers");
  setenv("VX_HOST_THREADS", "0", 1);
  check(vx::host_worker_count_for(payload.data(), payload.size(), &p, &t, 1) ==
            1,
        "VX_HOST_THREADS=0 is serial");
  setenv("VX_HOST_THREADS", "1000", 1);
  check(vx::host_worker_count_for(payload.data(), payload.size(), &p, &t, 1) ==
            64,
        "no more workers than iterations");
  unsetenv("VX_HOST_THREADS");
  std::string two("k");
  two.push_back('\0');
  two += "launch=4,32";
  two.push_back('\0');
  check(vx::host_worker_count_for(two.data(), two.size(), &p, &t, 1) == 1,
        "two-level launch stays serial");
  std::string none("k");
  none.push_back('\0');
  check(vx::host_worker_count_for(none.data(), none.size(), &p, &t, 1) == 1,
        "unsplit region stays serial");

  worker_calls = 0;
  max_total = 0;
  check(call((void *)k_split, {&p}, {kF32_1}, n) == 1, "split call");
  bool ok = true;
  for (int i = 0; i < 64; ++i) ok &= hbm[1000 + i] == (float)(1000 + i) + 1.0f;
  check(ok, "every iteration ran exactly once over 4 workers");
  check(worker_calls == 4 && max_total == 4, "4 workers ran");
  check(vx::host_worker_index == 0 && vx::host_worker_total == 1,
        "the calling thread is a single worker again");
}

} // namespace

int main() {
  test_same_buffer_out_then_in();
  test_same_buffer_in_then_out();
  test_overlapping_rows();
  test_touching_views_stay_apart();
  test_transposed_view();
  test_dense_column_and_block();
  test_publish_view_of_operand();
  test_empty_and_host_views();
  test_plan_directly();
  test_workers();
  if (failures) {
    fprintf(stderr, "%d failure(s)\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
