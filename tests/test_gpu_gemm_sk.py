"""The stream-K launch of the ping-pong GEMM, for grids whose tiles end in a
partial round of at most half the CUs (the reference's own GEMM benchmark
shape, 8192 x 3072 x 768, is 384 tiles on 256 CUs; grids of more rounds run
the rounds before in a one-tile launch first): every workgroup runs its own tile,
and the second round's tiles are cut at half of K between two workgroups,
the second adding the first's sums to its own at the end. Results are
checked for determinism (bit-equal from launch to launch), against the
one-tile launch (whose sums differ only in where one addition falls) and
against the f64 product on sampled rows, exactly on small integers, on the
automatic choice, launches in a row with other data, other streams, and the
paths that must not take a workspace (graph capture, the no-alloc entry
point)."""

import ctypes

import numpy as np
import pytest

from tests.conftest import announce
from tests.parity import BF16_ABS, FP32_REL, assert_max_abs, assert_rel
from vx_amd import abi
from vx_amd.abi import bf16_to_f32, f32_to_bf16
from vx_amd.runtime import DeviceArray, HipTimer, matmul

pytestmark = pytest.mark.gpu


def groups(lib) -> int:
    return lib.gemm_workspaces()["groups"]


def run(lib, da, db, dc, in_dt, out_dt, kernel):
    """C = A B on resident operands with `kernel` forced; C's bits."""
    lib.force_gemm_kernel(kernel)
    try:
        matmul(lib, da.descriptor(), in_dt, db.descriptor(), in_dt, dc.descriptor(), out_dt)
        c = dc.numpy().copy()
    finally:
        lib.force_gemm_kernel(abi.GEMM_AUTO)
    return c.view(np.uint32 if c.dtype == np.float32 else np.uint16)


def operands(rng, m, n, k, in_dt, small_int=False):
    """(A, B) as the GPU reads them, in f32, and their 16-bit bits."""
    if small_int:
        a = rng.integers(-3, 4, (m, k)).astype(np.float32)
        b = rng.integers(-3, 4, (k, n)).astype(np.float32)
    else:
        a = rng.normal(0, 1 / 8, (m, k)).astype(np.float32)
        b = rng.normal(0, 1 / 8, (k, n)).astype(np.float32)
    if in_dt == abi.DTYPE_BF16:
        a16, b16 = f32_to_bf16(a), f32_to_bf16(b)
        return bf16_to_f32(a16), bf16_to_f32(b16), a16, b16
    ah, bh = a.astype(np.float16), b.astype(np.float16)
    return ah.astype(np.float32), bh.astype(np.float32), ah.view(np.uint16), bh.view(np.uint16)


def values(bits, out_dt):
    """C as f32 from the bits `run` returns."""
    return bf16_to_f32(bits) if out_dt == abi.DTYPE_BF16 else bits.view(np.float32)


def close_to_one_tile(sk, pp, out_dt, what):
    """The stream-K sums differ from the one-tile launch's only in where one
    addition falls (A + (B + C) against (A + B) + C over the tail tiles'
    stages): a few f32 roundings, which a 16-bit result can carry into one
    unit of its last place."""
    got, want = values(sk, out_dt), values(pp, out_dt)
    rel = 2.0 ** -7 if out_dt == abi.DTYPE_BF16 else 1e-5
    assert_rel(got, want, rel, what)


def against_f64(bits, a, b, out_dt, what):
    """Sampled rows, spread over every tile row, against the f64 product of
    the operands as the GPU read them."""
    m = a.shape[0]
    rows = np.unique(np.linspace(0, m - 1, 24).astype(int))
    want = a[rows].astype(np.float64) @ b.astype(np.float64)
    got = values(bits, out_dt)[rows]
    if out_dt == abi.DTYPE_BF16:
        assert_max_abs(got, want, BF16_ABS, what)
    else:
        assert_rel(got, want, FP32_REL, what)


def shapes(g: int):
    """(m, n, k) of grids the stream-K launch takes on g CUs: one and a half
    rounds (at g = 256 the reference's benchmark shape), an eighth of a
    round past one (32 of 128 pairs), ragged edges with an odd stage count
    (9), and two and a quarter rounds (a one-tile round, then stream-K)."""
    full = [(8192, 3072, 768)] if g == 256 else [(256 * (3 * g // 16), 2048, 768)]
    return full + [
        (256 * (9 * g // 64), 2048, 768),
        (256 * (3 * g // 16) - 100, 2040, 288),
        (256 * (9 * g // 32), 2048, 768),
    ]


def takes_stream_k(tiles: int, g: int) -> bool:
    """The library's rule: tiles = q g + r with q >= 1, 0 < r <= g / 2 and
    g + r a multiple of 8 (K of at least 8 stages)."""
    q, r = divmod(tiles, g)
    return g % 8 == 0 and q >= 1 and 0 < r <= g // 2 and (g + r) % 8 == 0


@pytest.mark.parametrize("case", [0, 1, 2, 3])
@pytest.mark.parametrize("dts", [(abi.DTYPE_BF16, abi.DTYPE_F32), (abi.DTYPE_BF16, abi.DTYPE_BF16),
                                 (abi.DTYPE_F16, abi.DTYPE_F32)])
def test_stream_k_deterministic_and_close(hiplib, rng, case, dts):
    g = groups(hiplib)
    if g % 16:
        pytest.skip(f"{g} CUs: no stream-K shape of whole 16ths")
    m, n, k = shapes(g)[case]
    in_dt, out_dt = dts
    announce(f"stream-K {m}x{n}x{k} in {in_dt} out {out_dt} on {g} CUs")
    a, b, a16, b16 = operands(rng, m, n, k, in_dt)
    da, db = DeviceArray.of(hiplib, a16, in_dt), DeviceArray.of(hiplib, b16, in_dt)
    dc = DeviceArray(hiplib, (m, n), out_dt)
    try:
        before = hiplib.gemm_workspaces()["launches"]
        sk = run(hiplib, da, db, dc, in_dt, out_dt, abi.GEMM_MFMA_SK)
        again = run(hiplib, da, db, dc, in_dt, out_dt, abi.GEMM_MFMA_SK)
        assert hiplib.gemm_workspaces()["launches"] == before + 2, "no stream-K launch ran"
        assert np.array_equal(sk, again), "stream-K results differ from launch to launch"
        pp = run(hiplib, da, db, dc, in_dt, out_dt, abi.GEMM_MFMA_PP)
        assert hiplib.gemm_workspaces()["launches"] == before + 2
        close_to_one_tile(sk, pp, out_dt, f"{m}x{n}x{k} against the one-tile launch")
        against_f64(sk, a, b, out_dt, f"{m}x{n}x{k} against f64")
    finally:
        for x in (da, db, dc):
            x.free()


def test_stream_k_exact_on_small_integers_and_chosen_by_default(hiplib, rng):
    """Small-integer operands: every product and sum is exact in f32, so C
    equals the f64 product exactly; the automatic choice takes the stream-K
    launch for this grid."""
    g = groups(hiplib)
    if g % 16:
        pytest.skip(f"{g} CUs: no stream-K shape of whole 16ths")
    m, n, k = shapes(g)[0]
    announce(f"stream-K small integers {m}x{n}x{k}, automatic choice")
    a, b, a16, b16 = operands(rng, m, n, k, abi.DTYPE_BF16, small_int=True)
    da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
    dc = DeviceArray(hiplib, (m, n), abi.DTYPE_F32)
    try:
        before = hiplib.gemm_workspaces()["launches"]
        c = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_AUTO).view(np.float32)
        assert hiplib.gemm_workspaces()["launches"] == before + 1, "automatic choice not stream-K"
        want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
        assert np.array_equal(c, want)
    finally:
        for x in (da, db, dc):
            x.free()


def test_stream_k_launches_in_a_row_with_other_data(hiplib, rng):
    """Three launches in a row on one stream, each with new operands: each
    reader must take its own launch's partial sums (a stale slot or flag
    from the launch before would show)."""
    g = groups(hiplib)
    if g % 16:
        pytest.skip(f"{g} CUs: no stream-K shape of whole 16ths")
    m, n, k = shapes(g)[0]
    announce(f"stream-K three launches in a row {m}x{n}x{k}")
    arrays = []
    try:
        outs = []
        for rep in range(3):
            _, _, a16, b16 = operands(rng, m, n, k, abi.DTYPE_BF16)
            da = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16)
            db = DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
            dc = DeviceArray(hiplib, (m, n), abi.DTYPE_F32)
            arrays += [da, db, dc]
            hiplib.force_gemm_kernel(abi.GEMM_MFMA_SK)
            matmul(hiplib, da.descriptor(), abi.DTYPE_BF16, db.descriptor(), abi.DTYPE_BF16,
                   dc.descriptor(), abi.DTYPE_F32)
            outs.append((da, db, dc))
        hiplib.force_gemm_kernel(abi.GEMM_AUTO)
        got = [dc.numpy().copy().view(np.uint32) for (_, _, dc) in outs]
        for rep, (da, db, dc) in enumerate(outs):
            pp = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_MFMA_PP)
            close_to_one_tile(got[rep], pp, abi.DTYPE_F32, f"launch {rep}")
    finally:
        hiplib.force_gemm_kernel(abi.GEMM_AUTO)
        for x in arrays:
            x.free()


def test_stream_k_workspace_freed_with_stream(hiplib, rng):
    """Streams created and destroyed in a loop, each running a stream-K
    launch: moving the thread's caller stream off a stream frees that
    stream's workspace, and every loop's result is the same."""
    g = groups(hiplib)
    if g % 16:
        pytest.skip(f"{g} CUs: no stream-K shape of whole 16ths")
    m, n, k = shapes(g)[1]
    announce(f"stream-K workspace per stream lifetime {m}x{n}x{k}")
    _, _, a16, b16 = operands(rng, m, n, k, abi.DTYPE_BF16)
    da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
    dc = DeviceArray(hiplib, (m, n), abi.DTYPE_F32)
    t = HipTimer()
    first = None
    try:
        base = hiplib.gemm_workspaces()["blocks"]
        for it in range(4):
            s = t.stream_create()
            try:
                hiplib.lib.vx_hip_set_stream(s)
                before = hiplib.gemm_workspaces()["launches"]
                hiplib.force_gemm_kernel(abi.GEMM_MFMA_SK)
                matmul(hiplib, da.descriptor(), abi.DTYPE_BF16, db.descriptor(), abi.DTYPE_BF16,
                       dc.descriptor(), abi.DTYPE_F32)
                st = hiplib.gemm_workspaces()
                assert st["launches"] == before + 1 and st["blocks"] == base + 1, (it, st)
                got = dc.numpy().copy().view(np.uint32)
            finally:
                hiplib.force_gemm_kernel(abi.GEMM_AUTO)
                hiplib.lib.vx_hip_set_stream(None)
                t.sync()
                t.stream_destroy(s)
            assert hiplib.gemm_workspaces()["blocks"] == base, f"loop {it}: workspace kept"
            if first is None:
                first = got
            assert np.array_equal(got, first), it
        pp = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_MFMA_PP)
        close_to_one_tile(first, pp, abi.DTYPE_F32, "per-stream launches")
    finally:
        hiplib.force_gemm_kernel(abi.GEMM_AUTO)
        hiplib.lib.vx_hip_set_stream(None)
        for x in (da, db, dc):
            x.free()


def test_capture_takes_the_one_tile_launch(hiplib, rng):
    """A GEMM of a stream-K grid dispatched while the caller stream captures
    takes no workspace (the one-tile launch records); each replay, with
    eager stream-K launches of other operands between, matches the eager
    one-tile result bit for bit."""
    g = groups(hiplib)
    if g % 16:
        pytest.skip(f"{g} CUs: no stream-K shape of whole 16ths")
    m, n, k = shapes(g)[1]
    announce(f"stream-K grid under graph capture {m}x{n}x{k}")
    _, _, a16, b16 = operands(rng, m, n, k, abi.DTYPE_BF16)
    _, _, x16, y16 = operands(rng, m, n, k, abi.DTYPE_BF16)
    da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
    dx, dy = DeviceArray.of(hiplib, x16, abi.DTYPE_BF16), DeviceArray.of(hiplib, y16, abi.DTYPE_BF16)
    dc = DeviceArray(hiplib, (m, n), abi.DTYPE_F32)
    t = HipTimer()
    s = t.stream_create()
    ex = None
    try:
        want = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_MFMA_PP)
        before = hiplib.gemm_workspaces()["launches"]
        hiplib.lib.vx_hip_set_stream(s)
        ex = t.capture(s, lambda: matmul(hiplib, da.descriptor(), abi.DTYPE_BF16, db.descriptor(),
                                          abi.DTYPE_BF16, dc.descriptor(), abi.DTYPE_F32))
        hiplib.lib.vx_hip_set_stream(None)
        assert hiplib.gemm_workspaces()["launches"] == before, "a captured launch took stream-K"
        for rep in range(3):
            # an eager stream-K launch of other operands clobbers C
            other = run(hiplib, dx, dy, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_MFMA_SK)
            assert not np.array_equal(other, want)
            t.graph_launch(ex, s)
            t.sync()
            assert np.array_equal(dc.numpy().view(np.uint32), want), f"replay {rep}"
        assert hiplib.gemm_workspaces()["launches"] == before + 3
    finally:
        hiplib.force_gemm_kernel(abi.GEMM_AUTO)
        hiplib.lib.vx_hip_set_stream(None)
        if ex is not None:
            t.graph_destroy(ex)
        t.stream_destroy(s)
        for x in (da, db, dx, dy, dc):
            x.free()


def test_noalloc_entry_takes_the_one_tile_launch(hiplib, rng):
    """The no-alloc entry point on resident operands of a stream-K grid:
    no stream-K launch (it would need a workspace), the same bits."""
    g = groups(hiplib)
    if g % 16:
        pytest.skip(f"{g} CUs: no stream-K shape of whole 16ths")
    m, n, k = shapes(g)[1]
    announce(f"stream-K grid through the no-alloc entry point {m}x{n}x{k}")
    _, _, a16, b16 = operands(rng, m, n, k, abi.DTYPE_BF16)
    da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
    dc = DeviceArray(hiplib, (m, n), abi.DTYPE_F32)
    try:
        want = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_MFMA_PP)
        before = hiplib.gemm_workspaces()["launches"]
        args = abi.CallArgs()
        args.memref(da.descriptor(), abi.DTYPE_BF16).scalar(0, abi.KIND_I64)
        args.memref(db.descriptor(), abi.DTYPE_BF16).scalar(1, abi.KIND_I64)
        args.scalar(0.0, abi.KIND_F32).memref(dc.descriptor(), abi.DTYPE_F32)
        payload = abi.matmul_payload()
        buf = ctypes.create_string_buffer(payload, len(payload))
        argv, tags, cnt = args.arrays()
        assert hiplib.lib.vx_hip_dispatch_async_noalloc(buf, len(payload), argv, tags, cnt) == 1
        hiplib.wait()
        assert hiplib.gemm_workspaces()["launches"] == before
        assert np.array_equal(dc.numpy().view(np.uint32), want)
    finally:
        for x in (da, db, dc):
            x.free()


def test_ragged_grids_choose_and_match(hiplib):
    """Seeded ragged shapes around the stream-K range, on the automatic
    choice: grids with a stream-K tail (takes_stream_k) take it and the rest
    the one-tile launch; every result is deterministic and within the 1e-4
    rule of the f64 product on sampled rows."""
    g = groups(hiplib)
    rng = np.random.default_rng(4242)
    cases = []
    while len(cases) < 8:
        tn = int(rng.integers(2, 13))
        tm = int(rng.integers(g // tn, (3 * g) // (2 * tn) + 3))
        m = 256 * tm - int(rng.integers(0, 200))
        n = 256 * tn - 8 * int(rng.integers(0, 20))
        k = 32 * int(rng.integers(8, 40))
        cases.append((m, n, k))
    for m, n, k in cases:
        tiles = ((m + 255) // 256) * ((n + 255) // 256)
        expect_sk = takes_stream_k(tiles, g)
        announce(f"ragged {m}x{n}x{k}: {tiles} tiles on {g} CUs, stream-K {expect_sk}")
        a, b, a16, b16 = operands(rng, m, n, k, abi.DTYPE_BF16)
        da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
        dc = DeviceArray(hiplib, (m, n), abi.DTYPE_F32)
        try:
            before = hiplib.gemm_workspaces()["launches"]
            c1 = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_AUTO)
            c2 = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_AUTO)
            took = hiplib.gemm_workspaces()["launches"] - before
            assert took == (2 if expect_sk else 0), (m, n, k, took)
            assert np.array_equal(c1, c2), f"{m}x{n}x{k}: results differ from launch to launch"
            against_f64(c1, a, b, abi.DTYPE_F32, f"{m}x{n}x{k} against f64")
        finally:
            for x in (da, db, dc):
                x.free()


def test_stream_k_from_threads(hiplib):
    """Four host threads, each on its own stream (the caller stream is per
    thread), alternate a one-and-a-half-round grid and a two-and-a-quarter-
    round grid, so stream-K launches of several streams, each with its own
    workspace, run at once and a reader can wait while other launches hold
    CUs. The launch is deterministic, so every result must equal the one
    the same call gives alone."""
    import threading

    g = groups(hiplib)
    if g % 16:
        pytest.skip(f"{g} CUs: no stream-K shape of whole 16ths")
    announce("stream-K GEMMs from four threads on four streams")
    rng = np.random.default_rng(99)
    cases = []
    for m, n, k in (shapes(g)[0], shapes(g)[3]):
        _, _, a16, b16 = operands(rng, m, n, k, abi.DTYPE_BF16)
        da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
        dc = DeviceArray(hiplib, (m, n), abi.DTYPE_F32)
        try:
            want = run(hiplib, da, db, dc, abi.DTYPE_BF16, abi.DTYPE_F32, abi.GEMM_AUTO)
        finally:
            for x in (da, db, dc):
                x.free()
        cases.append((m, n, a16, b16, want))
    launches = hiplib.gemm_workspaces()["launches"]
    errors = []

    def work(tid):
        t = HipTimer()
        s = t.stream_create()
        arrays = []
        try:
            hiplib.lib.vx_hip_set_stream(s)
            dev = []
            for m, n, a16, b16, _ in cases:
                xs = (DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16),
                      DeviceArray(hiplib, (m, n), abi.DTYPE_F32))
                arrays += list(xs)
                dev.append(xs)
            for it in range(4):
                ci = (tid + it) % 2
                da, db, dc = dev[ci]
                matmul(hiplib, da.descriptor(), abi.DTYPE_BF16, db.descriptor(), abi.DTYPE_BF16,
                       dc.descriptor(), abi.DTYPE_F32)
                if not np.array_equal(dc.numpy().view(np.uint32), cases[ci][4]):
                    errors.append((tid, it, "C differs from the launch alone"))
        except Exception as e:  # reported below, with the thread that raised it
            errors.append((tid, -1, repr(e)))
        finally:
            for x in arrays:
                x.free()
            hiplib.lib.vx_hip_set_stream(None)
            t.sync()
            t.stream_destroy(s)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=90)
    assert not any(th.is_alive() for th in threads), "a launching thread did not finish"
    assert not errors, errors
    assert hiplib.gemm_workspaces()["launches"] == launches + 16
