"""The int8 weight-only GEMV op on the GPU against the CPU oracle."""

import numpy as np
import pytest

import oracle
from tests.conftest import announce
from tests.parity import GEMV_REL, assert_rel
from vx_amd import abi
from vx_amd.abi import f32_to_bf16
from vx_amd.runtime import DeviceArray, gemv_i8

pytestmark = pytest.mark.gpu


def run(lib, w, s, x16, guard=0):
    """y through the op; with `guard`, y sits in a buffer `guard` floats
    longer whose tail must come back untouched."""
    rows, cols = w.shape
    batch = x16.shape[0]
    dw = DeviceArray.of(lib, w, abi.DTYPE_I8)
    ds = DeviceArray.of(lib, s, abi.DTYPE_F32)
    dx = DeviceArray.of(lib, x16, abi.DTYPE_BF16)
    dy = DeviceArray.of(lib, np.full(batch * rows + guard, 7, np.float32), abi.DTYPE_F32)
    rc = gemv_i8(lib, dw.ptr, ds.ptr, dx.ptr, dy.ptr, rows, cols, batch)
    assert rc == 0
    full = dy.numpy()
    for a in (dw, ds, dx, dy):
        a.free()
    assert np.all(full[batch * rows:] == 7)
    return full[:batch * rows].reshape(batch, rows)


def inputs(rng, rows, cols, batch):
    w = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    s = rng.uniform(0.001, 0.01, rows).astype(np.float32)
    x16 = f32_to_bf16(rng.standard_normal((batch, cols)).astype(np.float32))
    return w, s, x16


@pytest.mark.parametrize("shape", [(4096, 4096), (11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("batch", [1, 4, 16])
def test_llama7b_shapes(hiplib, shape, batch):
    """Llama-2-7B linear shapes, batch 1/4/16."""
    announce(f"gemv {shape} batch {batch}")
    rng = np.random.default_rng(hash((shape, batch)) % 2**32)
    w, s, x16 = inputs(rng, *shape, batch)
    y = run(hiplib, w, s, x16)
    assert_rel(y, oracle.gemv_i8_f64(w, s, x16), GEMV_REL, f"gemv {shape} b{batch}")
    # the f32 oracle sums in another order; both sit near the f64 value
    assert_rel(y, oracle.gemv_i8(w, s, x16), 2 * GEMV_REL, "vs f32 oracle")


@pytest.mark.parametrize("shape,batch", [((7, 16), 1), ((33, 48), 3), ((1000, 2064), 5),
                                         ((64, 4096), 16), ((1, 32), 2), ((9, 3000 + 8), 7),
                                         ((8200, 1040), 12), ((17, 4112), 1), ((100, 48), 6),
                                         ((8195, 4096), 16), ((31, 4160), 4),
                                         ((4099, 4096), 2), ((6, 4096), 3), ((5, 8208), 1),
                                         ((13, 12304), 1), ((3, 20480), 1), ((7, 2064), 4),
                                         ((8197, 272), 3), ((8197, 4112), 6)])
def test_ragged(hiplib, shape, batch, rng):
    """Rows that leave the last 16- or 32-row block (or 4-row group) partial,
    columns that end inside a 256-column tile, a 64-column step or a
    4096-column pass, one, two, three and more passes per load group, every
    kernel and tile height; nothing is written past y."""
    announce(f"gemv ragged {shape} batch {batch}")
    rows, cols = shape
    if cols % 16:
        cols += 16 - cols % 16
    w, s, x16 = inputs(rng, rows, cols, batch)
    y = run(hiplib, w, s, x16, guard=64)
    assert_rel(y, oracle.gemv_i8_f64(w, s, x16), GEMV_REL, f"gemv {shape}")


KERNEL_CASES = [
    (abi.GEMV_ROWS, (4096, 4096), 1), (abi.GEMV_ROWS, (1000, 4112), 2),
    (abi.GEMV_ROWS, (11008, 4096), 1), (abi.GEMV_ROWS, (4099, 11008), 1),
    (abi.GEMV_DOT2_B4, (4096, 4096), 4), (abi.GEMV_DOT2_B4, (1001, 2064), 3),
    (abi.GEMV_LDS, (4096, 4096), 16), (abi.GEMV_LDS, (8200, 1040), 12),
    (abi.GEMV_LDS, (4096, 4096), 1), (abi.GEMV_LDS, (65, 272), 3),
    (abi.GEMV_LDS, (11008, 4096), 8), (abi.GEMV_LDS, (4096, 11008), 2),
    # 16-row tiles at batches of 8 and more: 256 workgroups (x through LDS,
    # one round on 256 CUs), 257 (x straight from L2), and x through LDS with
    # a partial last tile and batch rows past nb
    (abi.GEMV_LDS, (4096, 1040), 8), (abi.GEMV_LDS, (4099, 1040), 8),
    (abi.GEMV_LDS, (100, 2064), 9),
    # batches of 8 and more over 8192 rows: 48-row tiles (171 workgroups), and
    # 64-row tiles where 48-row ones would not fit one round (258 > 256 CUs)
    (abi.GEMV_LDS, (8200, 1040), 16), (abi.GEMV_LDS, (12340, 272), 8),
]


@pytest.mark.parametrize("kernel,shape,batch", KERNEL_CASES)
def test_each_kernel(hiplib, kernel, shape, batch, rng):
    """Each GEMV kernel forced on shapes of the config and ragged ones,
    including shapes the automatic choice sends elsewhere, against the f64
    oracle; nothing is written past y."""
    announce(f"gemv kernel {kernel} {shape} batch {batch}")
    w, s, x16 = inputs(rng, *shape, batch)
    hiplib.force_gemv_kernel(kernel)
    try:
        y = run(hiplib, w, s, x16, guard=64)
    finally:
        hiplib.force_gemv_kernel(abi.GEMV_AUTO)
    assert_rel(y, oracle.gemv_i8_f64(w, s, x16), GEMV_REL, f"kernel {kernel} {shape} b{batch}")


def test_calls_back_to_back_and_in_a_graph(hiplib, rng):
    """Calls of different shapes and kernels one after another without a host
    wait, then the same calls replayed from a captured graph three times
    (eager calls between replays): all match the oracle and are identical
    from run to run."""
    from vx_amd.runtime import HipTimer
    announce("gemv back to back and captured")
    shapes = [((4096, 4096), 16), ((1000, 2064), 5), ((11008, 4096), 1), ((300, 4096), 3)]
    cases = []
    for shape, batch in shapes:
        w, s, x16 = inputs(rng, *shape, batch)
        d = [DeviceArray.of(hiplib, w, abi.DTYPE_I8), DeviceArray.of(hiplib, s, abi.DTYPE_F32),
             DeviceArray.of(hiplib, x16, abi.DTYPE_BF16),
             DeviceArray(hiplib, (batch, shape[0]), abi.DTYPE_F32)]
        cases.append((shape, batch, d, oracle.gemv_i8_f64(w, s, x16)))
    t = HipTimer()
    stream = t.stream_create()
    hiplib.lib.vx_hip_set_stream(stream)
    graph = None
    try:
        def calls():
            for shape, batch, d, _ in cases:
                assert gemv_i8(hiplib, d[0].ptr, d[1].ptr, d[2].ptr, d[3].ptr, *shape, batch) == 0

        calls()
        t.sync()
        first = [d[3].numpy().copy() for _, _, d, _ in cases]
        for (shape, batch, d, want), got in zip(cases, first):
            assert_rel(got, want, GEMV_REL, f"eager {shape} b{batch}")
        graph = t.capture(stream, calls)
        for _ in range(3):
            calls()
            t.graph_launch(graph, stream)
            t.sync()
            for (shape, batch, d, want), ref in zip(cases, first):
                assert np.array_equal(d[3].numpy(), ref), f"replay {shape} b{batch}"
    finally:
        hiplib.lib.vx_hip_set_stream(None)
        if graph is not None:
            t.graph_destroy(graph)
        t.stream_destroy(stream)
        for _, _, d, _ in cases:
            for a in d:
                a.free()


def test_exact_integers(hiplib, rng):
    """Integer activations: every partial sum is exact in f32 whatever the
    order, so the GPU must equal scale * (exact dot) bit for bit."""
    announce("gemv exact integers")
    w = rng.integers(-127, 128, (4096, 11008), dtype=np.int8)
    x = rng.integers(-8, 9, (4, 11008)).astype(np.float32)
    s = rng.uniform(0.001, 0.01, 4096).astype(np.float32)
    y = run(hiplib, w, s, f32_to_bf16(x))
    exact = (w.astype(np.float64) @ x.astype(np.float64).T).T
    assert np.array_equal(y, s[None, :] * exact.astype(np.float32))
    assert np.array_equal(y, oracle.gemv_i8(w, s, f32_to_bf16(x)))


def test_refusals(hiplib, rng):
    announce("gemv refusals")
    w, s, x16 = inputs(rng, 16, 32, 1)
    dw = DeviceArray.of(hiplib, w, abi.DTYPE_I8)
    ds = DeviceArray.of(hiplib, s, abi.DTYPE_F32)
    dx = DeviceArray.of(hiplib, x16, abi.DTYPE_BF16)
    dy = DeviceArray(hiplib, (1, 16), abi.DTYPE_F32)
    assert gemv_i8(hiplib, dw.ptr, ds.ptr, dx.ptr, dy.ptr, 16, 24, 1) == -4  # cols % 16
    assert gemv_i8(hiplib, dw.ptr, ds.ptr, dx.ptr, dy.ptr, 16, 32, 17) == -1  # batch
    assert gemv_i8(hiplib, dw.ptr, ds.ptr, dx.ptr, dy.ptr, 0, 32, 1) == -1
    assert gemv_i8(hiplib, w.ctypes.data, ds.ptr, dx.ptr, dy.ptr, 16, 32, 1) == -3  # host w
    assert gemv_i8(hiplib, 0, ds.ptr, dx.ptr, dy.ptr, 16, 32, 1) == -1
    for a in (dw, ds, dx, dy):
        a.free()
