"""The runtime around the kernels on a GPU: the host fallback with HBM
operands that share bytes, dispatches captured into a hipGraph, memory taken
in a caller stream's order, and the refusals a capture forces.

Reference behaviour: runtime/vx_view_copy.h:14-23 (one copy per span of
overlapping views), runtime/vx_stream_policy.h:23-58 and
runtime/cuda_dispatch.cpp:234-293, 593 (waits and frees on a recording
stream)."""

import ctypes
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.conftest import announce
from vx_amd import abi
from vx_amd.abi import f32_to_bf16
from vx_amd.runtime import DeviceArray, HipTimer, matmul

ROOT = Path(__file__).resolve().parent.parent
pytestmark = pytest.mark.gpu

KERNEL_C = r"""
#include <stdint.h>
typedef struct { float *alloc, *aligned; int64_t offset, sizes[1], strides[1]; } D1;
typedef struct { float *alloc, *aligned; int64_t offset, sizes[2], strides[2]; } D2;
#define AT1(d, i) (d)->aligned[(d)->offset + (i) * (d)->strides[0]]
#define AT2(d, i, j) (d)->aligned[(d)->offset + (i) * (d)->strides[0] + (j) * (d)->strides[1]]
/* out[i] = in[i] + 1 */
void _vx_ciface_vx_rt_kernel_0(D1 *out, D1 *in) {
  for (int64_t i = 0; i < out->sizes[0]; ++i) AT1(out, i) = AT1(in, i) + 1.0f;
}
/* b += 10, then a *= 2 */
void _vx_ciface_vx_rt_kernel_1(D2 *a, D2 *b) {
  for (int64_t i = 0; i < b->sizes[0]; ++i)
    for (int64_t j = 0; j < b->sizes[1]; ++j) AT2(b, i, j) += 10.0f;
  for (int64_t i = 0; i < a->sizes[0]; ++i)
    for (int64_t j = 0; j < a->sizes[1]; ++j) AT2(a, i, j) *= 2.0f;
}
/* t[i][j] = 100 i + j */
void _vx_ciface_vx_rt_kernel_2(D2 *t) {
  for (int64_t i = 0; i < t->sizes[0]; ++i)
    for (int64_t j = 0; j < t->sizes[1]; ++j) AT2(t, i, j) = (float)(100 * i + j);
}
"""


@pytest.fixture(scope="module")
def outlined(tmp_path_factory):
    d = tmp_path_factory.mktemp("rt_outlined")
    src = d / "k.c"
    src.write_text(KERNEL_C)
    so = d / "libk.so"
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", "-ffp-contract=off", str(src), "-o",
                    str(so)], check=True)
    return ctypes.CDLL(str(so), mode=ctypes.RTLD_GLOBAL)


def run_region(lib, name, memrefs):
    args = abi.CallArgs()
    for desc in memrefs:
        args.memref(desc, abi.DTYPE_F32)
    before = lib.stats()["host_fallback"]
    lib.dispatch(abi.payload(name, abi="1", topo="500"), args)
    assert lib.stats()["host_fallback"] == before + 1


def test_fallback_same_hbm_buffer_as_output_and_input(hiplib, outlined):
    announce("fallback: one HBM buffer as output and input")
    host = np.arange(64, dtype=np.float32)
    d = DeviceArray.of(hiplib, host, abi.DTYPE_F32)
    try:
        view = d.descriptor(sizes=[48], offset=8)
        run_region(hiplib, "vx_rt_kernel_0", [view, abi.Descriptor(d.ptr, [48], offset=8)])
        want = host.copy()
        want[8:56] += 1
        assert np.array_equal(d.numpy(), want)
    finally:
        d.free()


def test_fallback_overlapping_row_views(hiplib, outlined):
    announce("fallback: overlapping HBM row views")
    m = np.arange(48, dtype=np.float32).reshape(6, 8)
    d = DeviceArray.of(hiplib, m, abi.DTYPE_F32)
    try:
        a = d.descriptor(sizes=[4, 8], strides=[8, 1], offset=0)
        b = d.descriptor(sizes=[4, 8], strides=[8, 1], offset=16)
        run_region(hiplib, "vx_rt_kernel_1", [a, b])
        want = m.copy()
        want[2:6] += 10
        want[0:4] *= 2
        assert np.array_equal(d.numpy(), want)
    finally:
        d.free()


def test_fallback_transposed_and_strided_views(hiplib, outlined):
    announce("fallback: transposed HBM views")
    m = np.arange(64, dtype=np.float32).reshape(8, 8)
    d = DeviceArray.of(hiplib, m, abi.DTYPE_F32)
    try:
        # the whole matrix seen transposed (copied as bytes)
        run_region(hiplib, "vx_rt_kernel_2", [d.descriptor(sizes=[8, 8], strides=[1, 8])])
        want = (100 * np.arange(8)[:, None] + np.arange(8)[None, :]).astype(np.float32).T
        assert np.array_equal(d.numpy(), want)
        # a transposed 3x2 block starting at [1][2] (copied densely)
        before = d.numpy()
        run_region(hiplib, "vx_rt_kernel_2", [d.descriptor(sizes=[3, 2], strides=[1, 8],
                                                           offset=10)])
        want = before.copy()
        for i in range(3):
            for j in range(2):
                want[1 + j, 2 + i] = 100 * i + j
        assert np.array_equal(d.numpy(), want)
    finally:
        d.free()


def test_gemm_captured_into_a_graph_replays(hiplib, rng):
    """A resident-operand bf16 GEMM dispatched while the caller stream
    captures: no wait, so it records; each replay (with eager work and a
    host read between) matches the oracle."""
    announce("graph capture of a resident bf16 GEMM")
    t = HipTimer()
    n = 512
    a16 = f32_to_bf16(rng.normal(0, 1 / 16, (n, n)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 16, (n, n)).astype(np.float32))
    want = oracle.gemm_bf16_f32(a16, b16)
    da, db = DeviceArray.of(hiplib, a16, abi.DTYPE_BF16), DeviceArray.of(hiplib, b16, abi.DTYPE_BF16)
    dc = DeviceArray(hiplib, (n, n), abi.DTYPE_F32)
    s = t.stream_create()
    ex = None
    try:
        hiplib.lib.vx_hip_set_stream(s)
        ex = t.capture(s, lambda: matmul(hiplib, da.descriptor(), abi.DTYPE_BF16, db.descriptor(),
                                          abi.DTYPE_BF16, dc.descriptor(), abi.DTYPE_F32))
        hiplib.lib.vx_hip_set_stream(None)
        for rep in range(3):
            # clobber C eagerly, then replay the graph
            matmul(hiplib, db.descriptor(), abi.DTYPE_BF16, da.descriptor(), abi.DTYPE_BF16,
                   dc.descriptor(), abi.DTYPE_F32)
            hiplib.wait()
            t.graph_launch(ex, s)
            t.sync()
            c = dc.numpy()
            assert float(np.abs(c - want).max()) <= 2e-2, f"replay {rep}"
    finally:
        hiplib.lib.vx_hip_set_stream(None)
        if ex is not None:
            t.graph_destroy(ex)
        t.stream_destroy(s)
        for x in (da, db, dc):
            x.free()


def test_stream_ordered_memory(hiplib, rng):
    """With a caller stream set, transfers take HBM in that stream's order
    and free it there; a GEMM on such memory still runs on the GPU in place."""
    announce("stream-ordered transfer, GEMM, free")
    t = HipTimer()
    s = t.stream_create()
    try:
        hiplib.lib.vx_hip_set_stream(s)
        n = 256
        a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
        b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
        da, db = DeviceArray.of(hiplib, a, abi.DTYPE_F32), DeviceArray.of(hiplib, b, abi.DTYPE_F32)
        dc = DeviceArray(hiplib, (n, n), abi.DTYPE_F32)
        before = hiplib.stats()
        matmul(hiplib, da.descriptor(), abi.DTYPE_F32, db.descriptor(), abi.DTYPE_F32,
               dc.descriptor(), abi.DTYPE_F32)
        st = hiplib.stats()
        assert st["gemm_device"] == before["gemm_device"] + 1
        assert st["staged_bytes"] == before["staged_bytes"], "operands were not seen as HBM"
        c = dc.numpy()
        assert np.array_equal(c, oracle.gemm_f32(a, b))
        for x in (da, db, dc):
            x.free()
        t.sync()
    finally:
        hiplib.lib.vx_hip_set_stream(None)
        t.stream_destroy(s)


def test_concurrent_dispatch_from_threads(hiplib):
    """Dispatch from several threads at once, as tasks do (reference
    runtime/cuda_dispatch.cpp:1387-1390 keeps the library's caches behind
    mutexes; the caller stream is per thread, :205-207): four threads each
    run f32 GEMMs with host operands and a host result (staged through the
    shared pool), and with HBM operands, allocating, reading back and freeing
    as they go. The exact-order kernel takes these sizes, so every result is
    bit-equal to the oracle's."""
    import threading

    announce("dispatch from four threads at once")
    errors = []

    def work(tid):
        rng = np.random.default_rng(100 + tid)
        try:
            for it in range(8):
                n = 96 + 32 * ((tid + it) % 4)
                a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
                b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
                want = oracle.gemm_f32(a, b)
                c = np.full((n, n), np.nan, np.float32)
                matmul(hiplib, abi.Descriptor(a.ctypes.data, a.shape), abi.DTYPE_F32,
                       abi.Descriptor(b.ctypes.data, b.shape), abi.DTYPE_F32,
                       abi.Descriptor(c.ctypes.data, c.shape), abi.DTYPE_F32)
                if not np.array_equal(c, want):
                    errors.append((tid, it, "host operands"))
                da = DeviceArray.of(hiplib, a, abi.DTYPE_F32)
                db = DeviceArray.of(hiplib, b, abi.DTYPE_F32)
                dc = DeviceArray(hiplib, (n, n), abi.DTYPE_F32)
                matmul(hiplib, da.descriptor(), abi.DTYPE_F32, db.descriptor(), abi.DTYPE_F32,
                       dc.descriptor(), abi.DTYPE_F32)
                if not np.array_equal(dc.numpy(), want):
                    errors.append((tid, it, "HBM operands"))
                for x in (da, db, dc):
                    x.free()
        except Exception as e:  # reported below, with the thread that raised it
            errors.append((tid, -1, repr(e)))

    threads = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
    assert not any(t.is_alive() for t in threads), "a dispatching thread did not finish"
    assert not errors, errors


REFUSE = r"""
import sys
sys.path.insert(0, {root!r})
import numpy as np
from vx_amd import abi
from vx_amd.runtime import DispatchLibrary, DeviceArray, HipTimer, matmul
lib = DispatchLibrary()
t = HipTimer()
s = t.stream_create()
a = np.ones((64, 64), np.float32)
dc = DeviceArray(lib, (64, 64), abi.DTYPE_F32)
lib.lib.vx_hip_set_stream(s)
print("capturing", flush=True)
def body():
    {body}
t.capture(s, body)
print("not refused", flush=True)
"""

BODIES = {
    "host operand": "matmul(lib, abi.Descriptor(a.ctypes.data, a.shape), abi.DTYPE_F32, "
                    "dc.descriptor(), abi.DTYPE_F32, dc.descriptor(), abi.DTYPE_F32)",
    "read-back": "lib.fetch(dc.ptr, np.empty((64, 64), np.float32))",
    "wait": "lib.wait()",
}


@pytest.mark.parametrize("what", sorted(BODIES))
def test_capture_refuses_what_it_cannot_record(hiplib, what):
    """A host copy, a read-back or a wait while the caller stream captures
    stops the program with a message that names the capture (in a child
    process: the refusal aborts)."""
    announce(f"capture refusal: {what}")
    code = REFUSE.format(root=str(ROOT), body=BODIES[what])
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=120, env={**os.environ, "PYTHONUNBUFFERED": "1"})
    assert "capturing" in res.stdout
    assert res.returncode != 0 and "not refused" not in res.stdout
    assert "capturing a hipGraph" in res.stderr, res.stderr[-2000:]
