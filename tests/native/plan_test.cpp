// plan_test.cpp -- GPU-free unit tests of the vendor-free headers of the HIP
// dispatch library: the payload walkers of include/vx_hardware_runtime.h,
// the GEMM plan decoder (vx_amd/csrc/vx_dispatch_plan.h) and the staging
// pool (vx_amd/csrc/vx_device_pool_hip.h).
//
// The cases restate the reference's own runtime tests as this build's tests
// (reference tests/runtime/gemm_plan_test.cpp:92-357, payload_test.cpp,
// device_pool_test.cpp): payloads and descriptors are written by hand the
// way the compiler writes them, and each decode is checked field by field.
// Built with -Wall -Werror (and the sanitizers when asked) by
// tests/test_native.py; prints "ok" and exits 0 when every check passes.

#include "../../vx_amd/csrc/vx_device_pool_hip.h"
#include "../../vx_amd/csrc/vx_dispatch_plan.h"

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
using D2 = Desc<2>;

D2 dense(void *p, int64_t rows, int64_t cols, int64_t ld) {
  D2 d{};
  d.allocated = d.aligned = p;
  d.sizes[0] = rows;
  d.sizes[1] = cols;
  d.strides[0] = ld;
  d.strides[1] = 1;
  return d;
}

struct Slot {
  void *allocated;
  void *aligned;
  int64_t offset;
};

std::string entries(const char *name, std::vector<std::string> kv) {
  std::string p(name);
  p.push_back('\0');
  for (auto &e : kv) {
    p += e;
    p.push_back('\0');
  }
  return p;
}

// The operand shape the compiler emits for `c = a @ b`: a, i64, b, i64, f32
// fill, result slot; roles a:0,b:2,out:5.
struct Matmul {
  std::vector<float> a, b;
  D2 ad, bd, result;
  Slot slot{}, aslot{}, bslot{};
  int64_t i0 = 0, i1 = 1;
  float fill = 0.0f;
  void *ap, *bp, *sp, *asp, *bsp;
  std::vector<void *> args;
  std::vector<int32_t> tags;
  Matmul(int64_t m, int64_t k, int64_t n, int32_t dt = VX_DTYPE_F32,
         int32_t odt = VX_DTYPE_F32)
      : a((size_t)(m * k), 1.0f), b((size_t)(k * n), 1.0f) {
    ad = dense(a.data(), m, k, k);
    bd = dense(b.data(), k, n, n);
    result = dense(nullptr, 0, 0, 0);
    slot = {&result, &result, 0};
    ap = &ad, bp = &bd, sp = &slot;
    args = {&ap, &i0, &bp, &i1, &fill, &sp};
    tags = {VX_ABI_MEMREF_TAG(dt, 2), VX_ABI_KIND_I64, VX_ABI_MEMREF_TAG(dt, 2),
            VX_ABI_KIND_I64,          VX_ABI_KIND_F32, VX_ABI_SLOT_TAG(odt, 2)};
  }
  void locals() {
    aslot = {&ad, &ad, 0};
    bslot = {&bd, &bd, 0};
    asp = &aslot, bsp = &bslot;
    args[0] = &asp;
    args[2] = &bsp;
    tags[0] |= VX_ABI_SLOT_BIT;
    tags[2] |= VX_ABI_SLOT_BIT;
  }
  bool decode(const std::string &p, vx_gemm_plan *plan) {
    return vx_gemm_plan_decode(p.data(), p.size(), args.data(), tags.data(),
                               (int64_t)args.size(), plan) != 0;
  }
};

std::string mm(const char *roles = "a:0,b:2,out:5",
               const char *outkind = "slot") {
  return entries("vx_npu_kernel_0", {"abi=1", "kind=matmul",
                                     std::string("roles=") + roles,
                                     std::string("outkind=") + outkind,
                                     "topo=500"});
}

void test_payload() {
  // The bytes the compiler stamps (reference
  // tests/optimizations/pass/kernel_kind_matmul.vx:68).
  std::string p = entries("k", {"kind=matmul", "roles=a:0,b:1,out:2",
                                "outkind=buffer"});
  check(p.find(std::string("\0kind=matmul\0roles=a:0,b:1,out:2\0outkind=buffer"
                           "\0",
                           46)) != std::string::npos,
        "payload bytes");
  const char *kind = vx_payload_field(p.data(), p.size(), "kind=");
  check(kind && std::string(kind) == "matmul", "kind= read back");
  check(!vx_payload_field(p.data(), p.size(), "image="), "absent key is NULL");
  check(!vx_payload_field(p.data(), 0, "kind="), "size 0 is never walked");
  check(vx_payload_abi(p.data(), p.size()) == -1, "no abi= reads -1");
  std::string q = entries("k", {"abi=1"});
  check(vx_payload_abi(q.data(), q.size()) == 1, "abi=1");
  std::string e = entries("k", {"abi="});
  const char *ev = vx_payload_field(e.data(), e.size(), "abi=");
  check(ev && *ev == '\0', "present but empty is not absent");
  check(vx_payload_abi(e.data(), e.size()) == -1, "empty abi reads -1");
  std::string x = entries("k", {"abi=1x"});
  check(vx_payload_abi(x.data(), x.size()) == -1, "non-decimal abi reads -1");
  std::string big = entries("k", {"abi=99999999999"});
  check(vx_payload_abi(big.data(), big.size()) == -1, "overflowing abi");
  // A binary section: empty entry, u64 LE length, bytes.
  std::string s = entries("k", {"format=spirv"});
  s.push_back('\0');
  const char img[5] = {1, 0, 2, 0, 3};
  uint64_t len = 5;
  for (int i = 0; i < 8; ++i) {
    s.push_back((char)((len >> (8 * i)) & 0xff));
  }
  s.append(img, 5);
  const void *out = nullptr;
  check(vx_payload_section(s.data(), s.size(), &out) == 5, "section length");
  check(out && memcmp(out, img, 5) == 0, "section bytes");
  check(!vx_payload_field(s.data(), s.size(), "image="),
        "section bytes are not keys");
  check(vx_payload_section(p.data(), p.size(), &out) == -1, "no section");
  std::string t = s.substr(0, s.size() - 1);
  check(vx_payload_section(t.data(), t.size(), &out) == -2, "truncated");
  check(vx_payload_section(s.data(), s.size(), nullptr) == -3, "NULL out");
}

void test_roles() {
  int a = -1, b = -1, o = -1;
  check(vx_parse_roles("a:0,b:2,out:5", &a, &b, &o) && a == 0 && b == 2 &&
            o == 5,
        "emitted order");
  check(vx_parse_roles("out:1,a:7,b:3", &a, &b, &o) && a == 7 && b == 3 &&
            o == 1,
        "any order");
  const char *bad[] = {"a:0,b:2",       "a:0,b:2,out:5,c:6", "a:0,b:2,out:",
                       "a:0,b:2,out:-1", "a:0,b:2,out:5,",   "a:0,a:1,b:2,out:5",
                       ""};
  for (const char *r : bad) {
    check(!vx_parse_roles(r, &a, &b, &o), r);
  }
  check(!vx_parse_roles(nullptr, &a, &b, &o), "absent roles");
}

void test_topology() {
  std::string p0 = mm();
  check(vx_payload_topology(p0.data(), p0.size()) == 500, "topo=500");
  std::string none = entries("k", {"kind=matmul"});
  check(vx_payload_topology(none.data(), none.size()) == -1, "absent not 0");
  check(vx_topology_device_index(500, VX_TOPO_GPU_BASE) == 0, "GPU[0]");
  check(vx_topology_device_index(507, VX_TOPO_GPU_BASE) == 7, "GPU[7]");
  check(vx_topology_device_index(100, VX_TOPO_GPU_BASE) == -1, "NPU");
  check(vx_topology_device_index(0, VX_TOPO_GPU_BASE) == -1, "CPU");
  check(vx_topology_device_index(600, VX_TOPO_GPU_BASE) == -1, "past band");
  check(vx_topology_numa_node(1100) == 0 && vx_topology_numa_node(1999) == 899 &&
            vx_topology_numa_node(2000) == -1,
        "NUMA band");
}

void test_slot_and_locals() {
  Matmul c(2, 3, 4);
  vx_gemm_plan plan;
  check(c.decode(mm(), &plan), "slot decodes");
  check(plan.m == 2 && plan.k == 3 && plan.n == 4, "extents");
  check(plan.dtype == VX_DTYPE_F32 && plan.out_dtype == VX_DTYPE_F32, "types");
  check(plan.a_data == c.a.data() && plan.b_data == c.b.data(), "A is 0, B 2");
  check(plan.out_kind == VX_GEMM_OUT_SLOT && plan.out_desc == &c.result &&
            !plan.out_data,
        "slot resolves one indirection in");
  std::vector<float> r(8, 7.0f);
  vx_gemm_publish_slot(&plan, r.data());
  check(c.result.aligned == r.data() && c.result.allocated == r.data() &&
            c.result.offset == 0,
        "published pointers");
  check(c.result.sizes[0] == 2 && c.result.sizes[1] == 4 &&
            c.result.strides[0] == 4 && c.result.strides[1] == 1,
        "published extents and strides");

  Matmul l(2, 3, 4);
  l.locals();
  check(l.decode(mm(), &plan) && plan.a_data == l.a.data() &&
            plan.b_data == l.b.data() && plan.m == 2 && plan.n == 4,
        "operands through slots");
}

void test_buffers() {
  Matmul c(2, 3, 4);
  std::vector<float> out(8);
  D2 od = dense(out.data(), 2, 4, 4);
  void *op = &od;
  c.args[5] = &op;
  c.tags[5] = VX_ABI_MEMREF_TAG(VX_DTYPE_F32, 2);
  vx_gemm_plan plan;
  check(c.decode(mm("a:0,b:2,out:5", "buffer"), &plan) &&
            plan.out_kind == VX_GEMM_OUT_BUFFER && plan.out_data == out.data() &&
            plan.out_row_stride == 4 && !plan.out_desc,
        "captured buffer");
  D2 wrong = dense(out.data(), 2, 3, 3);
  void *wp = &wrong;
  c.args[5] = &wp;
  check(!c.decode(mm("a:0,b:2,out:5", "buffer"), &plan), "extent mismatch");

  Matmul s(2, 3, 4);
  s.locals();
  Slot os = {&od, &od, 0};
  void *osp = &os;
  s.args[5] = &osp;
  check(s.decode(mm("a:0,b:2,out:5", "buffer"), &plan) &&
            plan.out_kind == VX_GEMM_OUT_BUFFER && plan.out_data == out.data(),
        "buffer through a slot is filled, not published");
}

void test_roles_beat_order() {
  Matmul c(3, 3, 3);
  vx_gemm_plan plan;
  check(c.decode(mm("a:2,b:0,out:5"), &plan) && plan.a_data == c.b.data() &&
            plan.b_data == c.a.data(),
        "roles decide, not order");
}

void test_refusals() {
  vx_gemm_plan plan;
  {
    Matmul c(2, 3, 4);
    check(!c.decode(entries("k", {}), &plan), "unclassified");
    std::string p = mm();
    check(!vx_gemm_plan_decode(p.data(), 0, c.args.data(), c.tags.data(), 6,
                               &plan),
          "size 0");
    check(!c.decode(entries("k", {"kind=conv2d", "roles=a:0,b:2,out:5",
                                  "outkind=slot"}),
                    &plan),
          "only matmul");
    check(!c.decode(mm("a:0,b:2,out:9"), &plan), "role past args");
    check(!c.decode(mm("a:0,b:0,out:5"), &plan), "two roles one arg");
    check(!c.decode(mm("a:0,b:2,out:5", "neither"), &plan), "unknown outkind");
  }
  {
    Matmul c(2, 3, 4);
    c.tags[5] = VX_ABI_MEMREF_TAG(VX_DTYPE_F32, 2);
    check(!c.decode(mm(), &plan), "slot outkind needs the slot bit");
  }
  {
    Matmul c(2, 3, 4);
    c.bd.sizes[0] = 5;
    check(!c.decode(mm(), &plan), "inner dims");
  }
  {
    Matmul c(2, 3, 4);
    c.tags[2] = VX_ABI_MEMREF_TAG(VX_DTYPE_F16, 2);
    check(!c.decode(mm(), &plan), "A and B types differ");
  }
  {
    Matmul c(2, 3, 4, VX_DTYPE_I32, VX_DTYPE_I32);
    check(!c.decode(mm(), &plan), "integer matmul runs as written");
  }
  {
    Matmul c(2, 3, 4);
    c.tags[0] = VX_ABI_MEMREF_TAG(VX_DTYPE_F32, 3);
    check(!c.decode(mm(), &plan), "rank 2 only");
  }
  {
    Matmul c(2, 3, 4);
    c.ad.strides[1] = 2;
    check(!c.decode(mm(), &plan), "contiguous rows");
  }
  {
    Matmul c(2, 3, 4);
    c.ad.strides[0] = 8;
    check(c.decode(mm(), &plan) && plan.a_row_stride == 8, "padded rows ok");
  }
  {
    Matmul c(2, 3, 4);
    c.ad.offset = 6;
    check(c.decode(mm(), &plan) && plan.a_data == c.a.data() + 6,
          "offset moves the data pointer");
  }
  {
    // f32 result of f64 operands is not a mixed plan this library takes.
    Matmul c(2, 3, 4, VX_DTYPE_F64, VX_DTYPE_F32);
    check(!c.decode(mm(), &plan), "f64 -> f32 refused");
    Matmul d(2, 3, 4, VX_DTYPE_F32, VX_DTYPE_BF16);
    check(!d.decode(mm(), &plan), "f32 -> bf16 refused");
  }
}

void test_mixed_plan() {
  // matmul_into(&mut c_f32, &a_bf16, &b_bf16): the plan the reference
  // decoder refuses and this one routes.
  Matmul c(2, 3, 4, VX_DTYPE_BF16, VX_DTYPE_F32);
  vx_gemm_plan plan;
  check(c.decode(mm(), &plan) && plan.dtype == VX_DTYPE_BF16 &&
            plan.out_dtype == VX_DTYPE_F32,
        "bf16 -> f32");
  Matmul h(2, 3, 4, VX_DTYPE_F16, VX_DTYPE_F32);
  check(h.decode(mm(), &plan) && plan.dtype == VX_DTYPE_F16 &&
            plan.out_dtype == VX_DTYPE_F32,
        "f16 -> f32");
  Matmul s(2, 3, 4, VX_DTYPE_BF16, VX_DTYPE_BF16);
  check(s.decode(mm(), &plan) && plan.out_dtype == VX_DTYPE_BF16,
        "bf16 -> bf16");
  // An offset on a 16-bit operand moves by 2 bytes per element.
  Matmul o(2, 3, 4, VX_DTYPE_BF16, VX_DTYPE_F32);
  o.ad.offset = 3;
  check(o.decode(mm(), &plan) &&
            (const char *)plan.a_data == (const char *)o.a.data() + 6,
        "16-bit offsets");
}

void test_view_span() {
  int64_t sizes[2] = {3, 4}, strides[2] = {10, 1};
  uint64_t bytes = 0;
  int32_t dim = -1;
  check(vx_memref_view_span(sizes, strides, 2, VX_DTYPE_F32, &bytes, &dim) ==
                VX_VIEW_OK &&
            bytes == (1 + 2 * 10 + 3) * 4,
        "padded span");
  int64_t tsizes[2] = {4, 3}, tstrides[2] = {1, 4};
  check(vx_memref_view_span(tsizes, tstrides, 2, VX_DTYPE_BF16, &bytes, &dim) ==
                VX_VIEW_OK &&
            bytes == (1 + 3 + 8) * 2,
        "transposed span");
  int64_t zs[2] = {0, 4};
  check(vx_memref_view_span(zs, strides, 2, VX_DTYPE_F32, &bytes, &dim) ==
                VX_VIEW_OK &&
            bytes == 0,
        "empty view");
  int64_t ns[2] = {3, -1};
  check(vx_memref_view_span(ns, strides, 2, VX_DTYPE_F32, &bytes, &dim) ==
                VX_VIEW_NEGATIVE &&
            dim == 1,
        "negative size");
  check(vx_memref_view_span(sizes, strides, 2, 0, &bytes, &dim) ==
            VX_VIEW_UNKNOWN_ELEMENT,
        "unknown element");
  int64_t huge[2] = {INT64_MAX, 2}, hs[2] = {INT64_MAX, 1};
  check(vx_memref_view_span(huge, hs, 2, VX_DTYPE_F32, &bytes, &dim) ==
            VX_VIEW_TOO_MANY_ELEMENTS,
        "overflow");
  check(vx_dtype_bytes(VX_DTYPE_BF16) == 2 && vx_dtype_bytes(VX_DTYPE_F64) == 8 &&
            vx_dtype_bytes(0) == 0 && vx_dtype_bytes(42) == 0,
        "dtype sizes");
}

// The pool with a fake allocator that records what it was asked.
std::vector<std::pair<void *, size_t>> live;
int allocs = 0, frees = 0, fail_next = 0;
void *fake_alloc(size_t n) {
  if (fail_next > 0) {
    --fail_next;
    return nullptr;
  }
  ++allocs;
  void *p = malloc(n);
  live.push_back({p, n});
  return p;
}
void fake_free(void *p, size_t) {
  ++frees;
  for (size_t i = 0; i < live.size(); ++i) {
    if (live[i].first == p) {
      live.erase(live.begin() + (long)i);
      break;
    }
  }
  free(p);
}

void test_pool() {
  vx::HipDevicePool<void *(*)(size_t), void (*)(void *, size_t)> pool(
      fake_alloc, fake_free, 1000);
  void *a = pool.acquire(100);
  check(a && allocs == 1, "first acquire allocates");
  pool.release(a, 100);
  check(pool.idle_bytes() == 100 && frees == 0, "release keeps it");
  void *b = pool.acquire(100);
  check(b == a && allocs == 1 && pool.hits() == 1, "same size is reused");
  void *c = pool.acquire(200);
  check(c != a && allocs == 2, "another size allocates");
  pool.release(b, 100);
  pool.release(c, 200);
  void *big = pool.acquire(900);
  pool.release(big, 900);
  check(frees == 1 && pool.idle_bytes() == 300, "over the cap is freed");
  fail_next = 1;
  void *d = pool.acquire(50);
  check(d && pool.idle_bytes() == 0 && frees == 3,
        "a failed allocation drains and retries");
  pool.release(d, 50);
  check(pool.acquire(0) == nullptr, "zero bytes");
  pool.drain();
  check(live.empty(), "drain frees everything");
}

} // namespace

int main() {
  test_payload();
  test_roles();
  test_topology();
  test_slot_and_locals();
  test_buffers();
  test_roles_beat_order();
  test_refusals();
  test_mixed_plan();
  test_view_span();
  test_pool();
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
