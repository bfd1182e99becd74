"""The routed `a @ b` on the GPU, through vx_plugin_dispatch_async exactly as
a compiled program calls it, checked against the CPU oracle (itself pinned to
the reference's own CPU library in test_oracle.py)."""

import ctypes

import numpy as np
import pytest

import oracle
from tests.conftest import announce
from tests.parity import BF16_ABS, FP32_REL, assert_max_abs, assert_rel, sum_invariant
from tests.test_oracle import roles_case, small_int_case
from vx_amd import abi
from vx_amd.abi import bf16_to_f32, f32_to_bf16
from vx_amd.runtime import DeviceArray, matmul

pytestmark = pytest.mark.gpu

NP_OUT = {abi.DTYPE_F32: np.float32, abi.DTYPE_F64: np.float64, abi.DTYPE_BF16: np.uint16,
          abi.DTYPE_F16: np.uint16}


def gpu_gemm(lib, a, b, in_dt, out_dt, outkind="buffer", kernel=abi.GEMM_AUTO, host=False):
    """C = A B through the plugin ABI. Operands in HBM (transfer) unless
    `host`; result in an HBM buffer (outkind=buffer) or published through a
    slot. Returns (C, stats delta)."""
    lib.force_gemm_kernel(kernel)
    before = lib.stats()
    m, k = a.shape
    n = b.shape[1]
    keep = []
    if host:
        ah, bh = np.ascontiguousarray(a), np.ascontiguousarray(b)
        keep += [ah, bh]
        ad = abi.Descriptor(ah.ctypes.data, (m, k))
        bd = abi.Descriptor(bh.ctypes.data, (k, n))
    else:
        da, db = DeviceArray.of(lib, a, in_dt), DeviceArray.of(lib, b, in_dt)
        keep += [da, db]
        ad, bd = da.descriptor(), db.descriptor()
    if outkind == "slot":
        out = abi.SlotStorage(2)
        matmul(lib, ad, in_dt, bd, in_dt, out, out_dt, outkind="slot")
        ptr, off, sizes, strides = out.published()
        assert sizes == [m, n] and strides == [n, 1] and off == 0
        npt = NP_OUT[out_dt]
        buf = (ctypes.c_char * (m * n * np.dtype(npt).itemsize)).from_address(ptr)
        c = np.frombuffer(buf, dtype=npt).reshape(m, n).copy()
        ctypes.CDLL(None).free(ctypes.c_void_p(ptr))
    else:
        dc = DeviceArray(lib, (m, n), out_dt)
        matmul(lib, ad, in_dt, bd, in_dt, dc.descriptor(), out_dt, outkind="buffer")
        c = dc.numpy()
        dc.free()
    for x in keep:
        if isinstance(x, DeviceArray):
            x.free()
    after = lib.stats()
    lib.force_gemm_kernel(abi.GEMM_AUTO)
    return c, {key: after[key] - before[key] for key in after}


def test_known_answers_roles(hiplib):
    """reference tests/backend/pass/gpu_matmul_roles.vx:47"""
    announce("gemm known answers roles")
    a, b, p, q = roles_case()
    c, st = gpu_gemm(hiplib, a, b, abi.DTYPE_F32, abi.DTYPE_F32)
    r, _ = gpu_gemm(hiplib, p, q, abi.DTYPE_F32, abi.DTYPE_F32)
    assert [c[0, 0], c[0, 3], c[1, 0], c[1, 3], r[0, 2], r[2, 0], r[1, 1]] == [38, 56, 83, 128, 9, 7, 10]
    assert st["gemm_device"] == 1 and st["host_fallback"] == 0


def test_known_answers_dtypes(hiplib):
    """reference tests/backend/pass/gpu_matmul_dtypes.vx:45"""
    announce("gemm known answers dtypes")
    cd, _ = gpu_gemm(hiplib, np.array([[1, 2], [3, 4]], np.float64),
                     np.array([[5, 6], [7, 8]], np.float64), abi.DTYPE_F64, abi.DTYPE_F64)
    e = np.eye(64, dtype=np.float32)
    bb = np.arange(64 * 64, dtype=np.float32).reshape(64, 64)
    r, _ = gpu_gemm(hiplib, e, bb, abi.DTYPE_F32, abi.DTYPE_F32)
    assert [cd[0, 0], cd[1, 1], r[3, 5], r[63, 0]] == [19, 50, 197, 4032]
    assert np.array_equal(r, bb)


@pytest.mark.parametrize("outkind", ["slot", "buffer"])
@pytest.mark.parametrize("host", [False, True])
def test_out_kinds_and_staging(hiplib, outkind, host, rng):
    announce(f"gemm outkind={outkind} host={host}")
    a = rng.uniform(-1, 1, (70, 45)).astype(np.float32)
    b = rng.uniform(-1, 1, (45, 33)).astype(np.float32)
    if host and outkind == "buffer":
        # a host result buffer: filled through a device result and a copy
        c = np.full((70, 33), np.nan, np.float32)
        hiplib.force_gemm_kernel(abi.GEMM_AUTO)
        matmul(hiplib, abi.Descriptor(a.ctypes.data, a.shape), abi.DTYPE_F32,
               abi.Descriptor(b.ctypes.data, b.shape), abi.DTYPE_F32,
               abi.Descriptor(c.ctypes.data, c.shape), abi.DTYPE_F32)
    else:
        c, st = gpu_gemm(hiplib, a, b, abi.DTYPE_F32, abi.DTYPE_F32, outkind, host=host)
        assert st["gemm_device"] == 1
        assert (st["staged_bytes"] > 0) == host
    assert_rel(c, oracle.gemm_f32(a, b), FP32_REL, "f32 70x45x33")


def test_fp32_512_config(hiplib):
    """M=N=K=512, U[-1,1], seeds 1 and 2."""
    announce("gemm f32 512^3")
    a = np.random.default_rng(1).uniform(-1, 1, (512, 512)).astype(np.float32)
    b = np.random.default_rng(2).uniform(-1, 1, (512, 512)).astype(np.float32)
    c, st = gpu_gemm(hiplib, a, b, abi.DTYPE_F32, abi.DTYPE_F32)
    want = oracle.gemm_f32(a, b)
    assert_rel(c, want, FP32_REL, "f32 512^3")
    # The tiled kernel adds the same terms in the same order with one
    # rounding per operation, so it reproduces the reference loop bit for bit.
    assert st["gemm_tiled"] == 1
    assert np.array_equal(c, want)


@pytest.mark.parametrize("n", [256, 512, 1024])
def test_bf16_mfma_matches_oracle(hiplib, n, rng):
    announce(f"gemm bf16->f32 mfma {n}")
    a16 = f32_to_bf16(rng.normal(0, 1 / 64, (n, n)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 64, (n, n)).astype(np.float32))
    c, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32)
    assert st["gemm_mfma"] == 1
    assert_max_abs(c, oracle.gemm_bf16_f32(a16, b16), BF16_ABS, f"bf16 {n}")
    exact = bf16_to_f32(a16).astype(np.float64) @ bf16_to_f32(b16).astype(np.float64)
    assert np.abs(c - exact).max() < 1e-5


def test_bf16_4096_config(hiplib):
    """M=N=K=4096, N(0, 1/64), f32 out: sampled rows
    against the oracle, every entry against f64, and the sum invariant."""
    announce("gemm bf16->f32 4096^3")
    rng = np.random.default_rng(42)
    a16 = f32_to_bf16(rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32))
    c, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32)
    assert st["gemm_mfma"] == 1
    rows = np.array([0, 1, 255, 256, 1023, 2048, 3071, 4095])
    for r in rows:
        want = oracle.gemm_bf16_f32(a16, b16, rows=slice(int(r), int(r) + 1))[r]
        assert_max_abs(c[r], want, BF16_ABS, f"row {r}")
    af, bf = bf16_to_f32(a16), bf16_to_f32(b16)
    exact = af.astype(np.float64) @ bf.astype(np.float64)
    assert_max_abs(c, exact, 1e-4, "4096 vs f64")
    assert abs(float(c.astype(np.float64).sum()) - sum_invariant(af, bf)) < 1e-2


def test_bf16_8192_random(hiplib):
    """BASELINE config 2's roofline point on random N(0, 1/64) operands (the
    1024-workgroup grid): 16 sampled rows, spread over every XCD's share of
    the tiles, against the oracle and against f64; the sum invariant over all
    of C (reference scripts/tools/vx_xpu_conformance.cpp:995-1017)."""
    announce("gemm bf16->f32 8192^3 random")
    n = 8192
    rng = np.random.default_rng(8192)
    a16 = f32_to_bf16(rng.normal(0, 1 / 64, (n, n)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 64, (n, n)).astype(np.float32))
    c, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32)
    assert st["gemm_mfma"] == 1
    rows = np.array([0, 1, 255, 256, 1023, 1024, 2047, 3000, 4095, 4096, 5555, 6143, 6144,
                     7000, 8190, 8191])
    af, bf = bf16_to_f32(a16), bf16_to_f32(b16)
    exact = af[rows].astype(np.float64) @ bf.astype(np.float64)
    for i, r in enumerate(rows):
        want = oracle.gemm_bf16_f32(a16, b16, rows=slice(int(r), int(r) + 1))[r]
        assert_max_abs(c[r], want, BF16_ABS, f"row {r}")
        assert_max_abs(c[r], exact[i], 1e-4, f"row {r} vs f64")
    assert np.isfinite(c).all()
    assert abs(float(c.astype(np.float64).sum()) - sum_invariant(af, bf)) < 5e-2


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 4096), (8192, 8192, 8192), (8192, 3072, 768)])
def test_bf16_small_integers_bit_exact(hiplib, m, n, k):
    """benchmarks/gpu_gemm inputs at the reference benchmark's sizes
    (run.sh: 8192 x 3072 x 768 and 4096^3) and 8192^3: every sum exact in
    f32, so every entry is compared bit for bit (the reference checks 64
    samples, v8_tile_128x128_8_subgroups.vx:65-103)."""
    announce(f"gemm bf16 small ints {m}x{n}x{k}")
    a16, b16 = small_int_case(m, k, n)
    c, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32)
    assert st["gemm_mfma"] == 1
    # A's rows repeat with period 7 and B's columns with period 5, so C is a
    # 7x5 table tiled over the matrix: every entry is checked exactly.
    a = bf16_to_f32(a16[:7]).astype(np.int64)
    b = bf16_to_f32(b16[:, :5]).astype(np.int64)
    table = (a @ b).astype(np.float32)
    assert np.array_equal(c, table[np.arange(m)[:, None] % 7, np.arange(n)[None, :] % 5])
    for s in range(64):
        i, j = (s * 7919) % m, (s * 104729) % n
        assert c[i, j] == oracle.gemm_bf16_point_f64(a16, b16, i, j)


def test_bf16_reference_benchmark_shape_random(hiplib):
    """8192 x 3072 x 768 (reference benchmarks/gpu_gemm/run.sh) on N(0, 1/64)
    operands: sampled rows against the oracle (the reference's loop order)
    and f64, and the sum invariant."""
    announce("gemm bf16 8192x3072x768 random")
    rng = np.random.default_rng(31)
    m, n, k = 8192, 3072, 768
    a16 = f32_to_bf16(rng.normal(0, 1 / 64, (m, k)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 64, (k, n)).astype(np.float32))
    c, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32)
    assert st["gemm_mfma"] == 1
    rows = [0, 1, 255, 256, 4095, 4096, 8190, 8191]
    af, bf = bf16_to_f32(a16), bf16_to_f32(b16)
    want = oracle.gemm_bf16_f32(a16[rows], b16)
    exact = af[rows].astype(np.float64) @ bf.astype(np.float64)
    for i, r in enumerate(rows):
        assert_max_abs(c[r], want[i], 1e-4, f"row {r} vs oracle")
        assert_max_abs(c[r], exact[i], 1e-4, f"row {r} vs f64")
    assert np.isfinite(c).all()
    assert abs(float(c.astype(np.float64).sum()) - sum_invariant(af, bf)) < 5e-2


def test_bf16_out_and_f16(hiplib, rng):
    announce("gemm bf16->bf16 and f16->f32")
    a16 = f32_to_bf16(rng.normal(0, 1, (512, 256)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1, (256, 768)).astype(np.float32))
    c16, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_BF16)
    assert st["gemm_mfma"] == 1
    want = oracle.gemm_bf16_f32(a16, b16)
    # one rounding of an f32 result: within one bf16 ulp of the oracle's
    assert_max_abs(bf16_to_f32(c16), want, float(np.abs(want).max()) * 2 ** -8 + 1e-6, "bf16 out")
    # Beside the reference CPU path for bf16 -> bf16 (the outlined linalg
    # loop, which rounds the running sum to bf16 at every k): the GPU rounds
    # once after f32 accumulation, as cuBLAS GemmEx does on the reference's
    # CUDA path, so the two differ by the per-step roundings; at config 2's
    # depth and scale (K = 4096, N(0, 1/64)) that stays within the 2e-2 bar.
    a16 = f32_to_bf16(rng.normal(0, 1 / 64, (256, 4096)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 64, (4096, 1024)).astype(np.float32))
    c16, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_BF16)
    assert st["gemm_mfma"] == 1
    lin = bf16_to_f32(oracle.gemm_bf16_bf16_linalg(a16, b16))
    assert_max_abs(bf16_to_f32(c16), lin, 2e-2, "bf16 out vs the reference's per-step rounding")
    want = oracle.gemm_bf16_f32(a16, b16)
    assert_max_abs(bf16_to_f32(c16), want, float(np.abs(want).max()) * 2 ** -8 + 1e-6,
                   "bf16 out at K = 4096")
    a = rng.normal(0, 1, (256, 512)).astype(np.float16)
    b = rng.normal(0, 1, (512, 256)).astype(np.float16)
    c, st = gpu_gemm(hiplib, a.view(np.uint16), b.view(np.uint16), abi.DTYPE_F16, abi.DTYPE_F32)
    assert st["gemm_mfma"] == 1
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert_max_abs(c, exact, 1e-3, "f16 -> f32")


@pytest.mark.parametrize("shape", [(37, 29, 53), (1, 768, 64), (300, 64, 257), (2, 3, 4),
                                   (65, 100, 70)])
@pytest.mark.parametrize("dt", [abi.DTYPE_F32, abi.DTYPE_BF16, abi.DTYPE_F64])
def test_ragged_shapes(hiplib, shape, dt, rng):
    """Exact-order kernel, bit-equal to the oracle: K under one step, one or
    many whole steps, and whole steps followed by a partial one (K = 100:
    one 64-deep f32 step plus 36; three 32-deep f64 steps plus 4)."""
    announce(f"gemm ragged {shape} dtype {dt}")
    m, k, n = shape
    a = rng.uniform(-1, 1, (m, k))
    b = rng.uniform(-1, 1, (k, n))
    if dt == abi.DTYPE_BF16:
        a16, b16 = f32_to_bf16(a.astype(np.float32)), f32_to_bf16(b.astype(np.float32))
        c, st = gpu_gemm(hiplib, a16, b16, dt, abi.DTYPE_F32)
        assert np.array_equal(c, oracle.gemm_bf16_f32(a16, b16))
    elif dt == abi.DTYPE_F32:
        a, b = a.astype(np.float32), b.astype(np.float32)
        c, st = gpu_gemm(hiplib, a, b, dt, dt)
        assert np.array_equal(c, oracle.gemm_f32(a, b))
    else:
        c, st = gpu_gemm(hiplib, a, b, dt, dt)
        assert np.array_equal(c, oracle.gemm_f64(a, b))
    assert st["gemm_tiled"] == 1


def test_views_with_offsets_and_padded_rows(hiplib, rng):
    """A view into a larger buffer (offset, padded row stride) for A, B and
    the result: the kernel must honour all three."""
    announce("gemm strided views")
    big_a = rng.uniform(-1, 1, (80, 100)).astype(np.float32)
    big_b = rng.uniform(-1, 1, (60, 90)).astype(np.float32)
    da, db = DeviceArray.of(hiplib, big_a, abi.DTYPE_F32), DeviceArray.of(hiplib, big_b, abi.DTYPE_F32)
    dc = DeviceArray.of(hiplib, np.zeros((50, 70), np.float32), abi.DTYPE_F32)
    # A = big_a[3:43, 5:55] (40x50), B = big_b[2:52, 7:37] (50x30), C = c[4:44, 9:39]
    ad = da.descriptor(sizes=(40, 50), strides=(100, 1), offset=3 * 100 + 5)
    bd = db.descriptor(sizes=(50, 30), strides=(90, 1), offset=2 * 90 + 7)
    cd = dc.descriptor(sizes=(40, 30), strides=(70, 1), offset=4 * 70 + 9)
    matmul(hiplib, ad, abi.DTYPE_F32, bd, abi.DTYPE_F32, cd, abi.DTYPE_F32)
    c = dc.numpy()
    want = oracle.gemm_f32(big_a[3:43, 5:55], big_b[2:52, 7:37])
    assert np.array_equal(c[4:44, 9:39], want)
    untouched = c.copy()
    untouched[4:44, 9:39] = 0
    assert not untouched.any()
    for x in (da, db, dc):
        x.free()


def test_mfma_and_tiled_agree(hiplib, rng):
    announce("gemm mfma vs tiled")
    a16 = f32_to_bf16(rng.normal(0, 1, (512, 512)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1, (512, 512)).astype(np.float32))
    c1, s1 = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32, kernel=abi.GEMM_MFMA_PP)
    c2, s2 = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32, kernel=abi.GEMM_TILED)
    assert s1["gemm_mfma"] == 1 and s2["gemm_tiled"] == 1
    assert np.array_equal(c2, oracle.gemm_bf16_f32(a16, b16))
    assert_max_abs(c1, c2, 1e-3, "mfma vs tiled")


@pytest.mark.parametrize("k", [32, 64, 96, 128, 192, 768])
@pytest.mark.parametrize("out_dt", [abi.DTYPE_F32, abi.DTYPE_BF16])
def test_mfma_pp_against_oracle(hiplib, k, out_dt, rng):
    """The ping-pong kernel adds 32-term MFMA sums in k order: it is held to
    the oracle and to f64 at K of 1, 2, 3, 4 and 6 stages (the ring's
    prologue and tail cases) and 24, and it is deterministic across calls."""
    announce(f"gemm mfma ping-pong k={k} out={out_dt}")
    a16 = f32_to_bf16(rng.normal(0, 1, (512, k)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1, (k, 768)).astype(np.float32))
    c, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, out_dt, kernel=abi.GEMM_MFMA_PP)
    assert st["gemm_mfma"] == 1
    again, _ = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, out_dt, kernel=abi.GEMM_MFMA_PP)
    assert np.array_equal(c, again)
    want = oracle.gemm_bf16_f32(a16, b16)
    exact = bf16_to_f32(a16).astype(np.float64) @ bf16_to_f32(b16).astype(np.float64)
    if out_dt == abi.DTYPE_F32:
        assert_max_abs(c, want, 1e-3, "ping-pong vs oracle")
        assert np.abs(c - exact).max() <= 1e-5 * max(1.0, np.abs(exact).max())
    else:
        got = bf16_to_f32(c)
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-3)


@pytest.mark.parametrize("m,n,k,ldb", [(1000, 776, 512, 776), (300, 4104, 64, 4104),
                                       (257, 776, 96, 784), (1, 8, 32, 8), (4100, 296, 128, 304)])
@pytest.mark.parametrize("out_dt", [abi.DTYPE_F32, abi.DTYPE_BF16])
@pytest.mark.parametrize("pad,col0", [(3, 1), (8, 4)])
def test_mfma_pp_ragged_edges(hiplib, m, n, k, ldb, out_dt, pad, col0, rng):
    """M and N that are not multiples of the 256x256 tile, and a B whose rows
    are padded (ldb > n): edge tiles read zeros past the operands' ends and
    store only inside C, which is checked to be untouched around the result.
    C is a view with row stride n + pad starting at column col0 of row 1:
    pad 3 puts its rows off the 4-element grid (the epilogue's element
    stores), pad 8 with col0 4 keeps them on it (its 16-byte f32 and 8-byte
    bf16 stores of 4 columns)."""
    announce(f"gemm ping-pong ragged {m}x{n}x{k} ldb={ldb} out={out_dt} pad={pad}")
    a16 = f32_to_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
    bpad = f32_to_bf16(rng.normal(0, 1, (k, ldb)).astype(np.float32))
    b16 = np.ascontiguousarray(bpad[:, :n])
    da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, bpad, abi.DTYPE_BF16)
    npt = np.float32 if out_dt == abi.DTYPE_F32 else np.uint16
    ldc = n + pad
    sentinel = np.full((m + 2, ldc), 7, npt)  # C is rows 1..m, cols col0..col0+n-1
    dc = DeviceArray.of(hiplib, sentinel, out_dt)
    hiplib.force_gemm_kernel(abi.GEMM_MFMA_PP)
    before = hiplib.stats()
    matmul(hiplib, da.descriptor(), abi.DTYPE_BF16,
           db.descriptor(sizes=(k, n), strides=(ldb, 1)), abi.DTYPE_BF16,
           dc.descriptor(sizes=(m, n), strides=(ldc, 1), offset=ldc + col0), out_dt)
    full = dc.numpy()
    after = hiplib.stats()
    hiplib.force_gemm_kernel(abi.GEMM_AUTO)
    assert after["gemm_mfma"] == before["gemm_mfma"] + 1
    c = full[1:m + 1, col0:col0 + n]
    rest = full.copy()
    rest[1:m + 1, col0:col0 + n] = 7
    assert np.all(rest == 7)
    want = oracle.gemm_bf16_f32(a16, b16)
    if out_dt == abi.DTYPE_F32:
        assert_max_abs(c, want, 1e-3 * max(1.0, float(np.abs(want).max())), "ragged vs oracle")
    else:
        got = bf16_to_f32(c)
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-3 * np.abs(want).max())
    for x in (da, db, dc):
        x.free()


def test_mfma_pp_declines_n_off_the_16_byte_grid(hiplib, rng):
    """N = 777: B's last row would end inside a 16-byte load, which the
    buffer range check zeroes whole, so the ping-pong kernel declines and the
    exact-order kernel runs (bit-equal to the oracle)."""
    announce("gemm ping-pong declines n=777")
    m, n, k = 257, 777, 96
    a16 = f32_to_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1, (k, n)).astype(np.float32))
    c, st = gpu_gemm(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32, kernel=abi.GEMM_MFMA_PP)
    assert st["gemm_tiled"] == 1 and st["gemm_mfma"] == 0
    assert np.array_equal(c, oracle.gemm_bf16_f32(a16, b16))


def test_mfma_pp_f16(hiplib, rng):
    """f16 operands through the ping-pong kernel's f16 MFMA."""
    announce("gemm mfma ping-pong f16")
    a = rng.normal(0, 1, (256, 256)).astype(np.float16)
    b = rng.normal(0, 1, (256, 512)).astype(np.float16)
    c, st = gpu_gemm(hiplib, a.view(np.uint16), b.view(np.uint16), abi.DTYPE_F16, abi.DTYPE_F32,
                     kernel=abi.GEMM_MFMA_PP)
    assert st["gemm_mfma"] == 1
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(c - exact).max() <= 1e-5 * np.abs(exact).max()


def test_f32_mfma_routed_at_1024(hiplib, rng):
    """f32 products of 2^30 multiply-adds and more go to the f32 MFMA
    kernel, whose sums round once per two products instead of once per
    product: held to the reference's 1e-4 rule against the oracle, closer to
    the f64 product than 1e-5 of its largest entry, and deterministic."""
    announce("gemm f32 mfma 1024^3")
    a = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    b = rng.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    c, st = gpu_gemm(hiplib, a, b, abi.DTYPE_F32, abi.DTYPE_F32)
    assert st["gemm_mfma"] == 1 and st["gemm_tiled"] == 0
    again, _ = gpu_gemm(hiplib, a, b, abi.DTYPE_F32, abi.DTYPE_F32)
    assert np.array_equal(c, again)
    assert_rel(c, oracle.gemm_f32(a, b), FP32_REL, "f32 mfma 1024^3")
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(c - exact).max() <= 1e-5 * np.abs(exact).max()


@pytest.mark.parametrize("m,n,k,lda,ldb", [(1000, 777, 333, 333, 777), (129, 131, 17, 20, 132),
                                           (1, 1, 1, 1, 1), (300, 260, 64, 64, 264),
                                           (130, 4100, 48, 52, 4100)])
def test_f32_mfma_ragged(hiplib, m, n, k, lda, ldb, rng):
    """The f32 MFMA kernel forced onto shapes off its 128x128x16 grid, with
    padded rows and row strides that are not multiples of four floats (the
    scalar load path): zeros past the operands' ends, stores only inside C,
    which sits in a sentinel-filled buffer."""
    announce(f"gemm f32 mfma ragged {m}x{n}x{k} lda={lda} ldb={ldb}")
    apad = rng.uniform(-1, 1, (m, lda)).astype(np.float32)
    bpad = rng.uniform(-1, 1, (k, ldb)).astype(np.float32)
    da, db = DeviceArray.of(hiplib, apad, abi.DTYPE_F32), DeviceArray.of(hiplib, bpad, abi.DTYPE_F32)
    sentinel = np.full((m + 2, n + 3), 7, np.float32)  # C is rows 1..m, cols 1..n of this
    dc = DeviceArray.of(hiplib, sentinel, abi.DTYPE_F32)
    hiplib.force_gemm_kernel(abi.GEMM_F32_MFMA)
    before = hiplib.stats()
    matmul(hiplib, da.descriptor(sizes=(m, k), strides=(lda, 1)), abi.DTYPE_F32,
           db.descriptor(sizes=(k, n), strides=(ldb, 1)), abi.DTYPE_F32,
           dc.descriptor(sizes=(m, n), strides=(n + 3, 1), offset=n + 3 + 1), abi.DTYPE_F32)
    full = dc.numpy()
    after = hiplib.stats()
    hiplib.force_gemm_kernel(abi.GEMM_AUTO)
    assert after["gemm_mfma"] == before["gemm_mfma"] + 1
    c = full[1:m + 1, 1:n + 1]
    rest = full.copy()
    rest[1:m + 1, 1:n + 1] = 7
    assert np.all(rest == 7)
    a, b = np.ascontiguousarray(apad[:, :k]), np.ascontiguousarray(bpad[:, :n])
    assert_rel(c, oracle.gemm_f32(a, b), FP32_REL, "f32 mfma ragged")
    for x in (da, db, dc):
        x.free()


def test_flat_matvec(hiplib, rng):
    """vx_plugin_dispatch_async_flat: xout[i] = sum_j w[i*n+j] x[j]."""
    announce("flat matvec")
    n, d = 300, 77
    w = rng.uniform(-1, 1, d * n).astype(np.float32)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    want = oracle.gemm_f32(w.reshape(d, n), x.reshape(n, 1)).ravel()
    out = np.zeros(d, np.float32)
    hiplib.lib.vx_plugin_dispatch_async_flat(out.ctypes.data, x.ctypes.data, w.ctypes.data, n, d)
    assert np.array_equal(out, want)
    dw, dx = DeviceArray.of(hiplib, w, abi.DTYPE_F32), DeviceArray.of(hiplib, x, abi.DTYPE_F32)
    dy = DeviceArray(hiplib, (d,), abi.DTYPE_F32)
    hiplib.lib.vx_plugin_dispatch_async_flat(dy.ptr, dx.ptr, dw.ptr, n, d)
    assert np.array_equal(dy.numpy(), want)
    for a in (dw, dx, dy):
        a.free()


def test_transfers_peer_collectives(hiplib, rng):
    announce("transfers, peer, collectives")
    lib = hiplib.lib
    x = rng.standard_normal(1000).astype(np.float32)
    d0 = hiplib.transfer(x)
    d1 = lib.vx_plugin_transfer_peer(d0, 500, 500, x.nbytes)
    back = np.empty_like(x)
    hiplib.fetch(d1, back)
    assert np.array_equal(back, x)
    lib.vx_collective_init(0, 1)
    assert lib.vx_collective_rank() == 0 and lib.vx_collective_ranks() == 1
    d2 = hiplib.transfer(None, x.nbytes)
    lib.vx_collective_all_reduce_sum_f32(d0, d2, x.size)
    hiplib.fetch(d2, back)
    assert np.array_equal(back, x)
    lib.vx_collective_finish()
    for p in (d0, d1, d2):
        hiplib.free(p)
    # host topology: plain host memory
    h = hiplib.transfer(x, topo=0)
    assert np.array_equal(np.ctypeslib.as_array((ctypes.c_float * x.size).from_address(h)), x)
    hiplib.free(h, 0)
    assert lib.vx_plugin_control(abi.CTRL_INIT_DEVICE, None) == 1
    pair = (ctypes.c_int32 * 2)(123456, 500)
    assert lib.vx_plugin_control(abi.CTRL_LOCAL_DEVICE, pair) == 1
    y = hiplib.transfer(x, topo=123456)  # a declared id standing for GPU[0]
    hiplib.fetch(y, back, topo=123456)
    assert np.array_equal(back, x)
    hiplib.free(y, 123456)
