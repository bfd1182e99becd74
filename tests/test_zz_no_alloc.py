"""vx_hip_dispatch_async_noalloc on the GPU: the same results as
vx_plugin_dispatch_async for routed GEMMs, with host operands staged through
the library's fixed per-GPU scratch instead of its pool; two calls in a row
(the second smaller) on that shared scratch; the refusals."""

import ctypes

import numpy as np
import pytest

from tests.conftest import announce
from vx_amd import abi
from vx_amd.abi import f32_to_bf16
from vx_amd.runtime import DeviceArray

pytestmark = pytest.mark.gpu


def gemm_args(a, a_dt, b, b_dt, c, c_dt):
    """The compiler's six launch operands for `c = a @ b` (A at 0, B at 2,
    the result at 5); each of a, b, c is a host array or a DeviceArray."""
    def desc(x):
        if isinstance(x, DeviceArray):
            return x.descriptor()
        return abi.Descriptor(x.ctypes.data, x.shape)
    args = abi.CallArgs()
    args.memref(desc(a), a_dt).scalar(0, abi.KIND_I64).memref(desc(b), b_dt)
    args.scalar(1, abi.KIND_I64).scalar(0.0, abi.KIND_F32).memref(desc(c), c_dt)
    return args


def noalloc(lib, payload, args) -> int:
    buf = ctypes.create_string_buffer(payload, len(payload))
    argv, tags, n = args.arrays()
    return lib.lib.vx_hip_dispatch_async_noalloc(buf, len(payload), argv, tags, n)


def staging(lib):
    """(staging-pool acquires, of them new allocations, bytes staged through
    the no-alloc scratch)."""
    out = (ctypes.c_int64 * 3)()
    assert lib.control(abi.HIP_CTRL_STAGING_STATS, out) == 1
    return tuple(out)


def via_both(lib, a, b, a_dt, out_dt, host_out=True):
    """C through the ABI entry point and through the no-alloc one, from
    host operands (and a host or device result). The ABI entry point stages
    through its pool; the no-alloc one takes nothing from the pool and
    stages every host byte through its scratch."""
    m, n = a.shape[0], b.shape[1]
    np_out = np.float32 if out_dt == abi.DTYPE_F32 else np.uint16
    staged = a.nbytes + b.nbytes + (m * n * np.dtype(np_out).itemsize if host_out else 0)
    results = []
    for entry in ("abi", "noalloc"):
        if host_out:
            c = np.full((m, n), 7, np_out)
        else:
            c = DeviceArray(lib, (m, n), out_dt)
        args = gemm_args(a, a_dt, b, a_dt, c, out_dt)
        before = lib.stats()
        pool0 = staging(lib)
        if entry == "abi":
            lib.dispatch(abi.matmul_payload(), args)
            pool1 = staging(lib)
            assert pool1[0] == pool0[0] + (3 if host_out else 2) and pool1[2] == pool0[2]
        else:
            assert noalloc(lib, abi.matmul_payload(), args) == 1
            pool1 = staging(lib)
            assert pool1[:2] == pool0[:2], "the no-alloc entry point used the pool"
            assert pool1[2] == pool0[2] + staged
        st = lib.stats()
        assert st["gemm_device"] == before["gemm_device"] + 1
        if host_out:
            lib.wait()
            results.append(c.copy())
        else:
            results.append(c.numpy())
            c.free()
    return results


def test_noalloc_matches_the_abi_entry_point_twice_in_a_row(hiplib, rng):
    """Host bf16 operands (A 384x512, B 512x640: staged through the scratch)
    and a host f32 result, then a smaller f32 GEMM on the same scratch: each
    bit-equal to vx_plugin_dispatch_async's result (the same kernels run on
    the same staged values)."""
    announce("noalloc GEMM: bf16 384x512x640 host operands, then f32 96x64x80")
    a16 = f32_to_bf16(rng.normal(0, 1 / 16, (384, 512)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 16, (512, 640)).astype(np.float32))
    ref, got = via_both(hiplib, a16, b16, abi.DTYPE_BF16, abi.DTYPE_F32)
    assert np.array_equal(ref, got)
    assert np.isfinite(got).all() and not np.all(got == 7)
    a = rng.uniform(-1, 1, (96, 80)).astype(np.float32)
    b = rng.uniform(-1, 1, (80, 64)).astype(np.float32)
    ref, got = via_both(hiplib, a, b, abi.DTYPE_F32, abi.DTYPE_F32)
    assert np.array_equal(ref, got)
    # a device result with host operands
    ref, got = via_both(hiplib, a, b, abi.DTYPE_F32, abi.DTYPE_F32, host_out=False)
    assert np.array_equal(ref, got)


def test_noalloc_resident_operands_and_refusals(hiplib, rng):
    announce("noalloc GEMM: resident operands and refusals")
    a = rng.uniform(-1, 1, (128, 96)).astype(np.float32)
    b = rng.uniform(-1, 1, (96, 112)).astype(np.float32)
    da, db = DeviceArray.of(hiplib, a, abi.DTYPE_F32), DeviceArray.of(hiplib, b, abi.DTYPE_F32)
    dc1 = DeviceArray(hiplib, (128, 112), abi.DTYPE_F32)
    dc2 = DeviceArray(hiplib, (128, 112), abi.DTYPE_F32)
    hiplib.dispatch(abi.matmul_payload(), gemm_args(da, abi.DTYPE_F32, db, abi.DTYPE_F32, dc1,
                                                    abi.DTYPE_F32))
    assert noalloc(hiplib, abi.matmul_payload(),
                   gemm_args(da, abi.DTYPE_F32, db, abi.DTYPE_F32, dc2, abi.DTYPE_F32)) == 1
    assert np.array_equal(dc1.numpy(), dc2.numpy())
    # a region that is not a routed GEMM
    assert noalloc(hiplib, abi.payload("vx_not_a_gemm", abi="1"), abi.CallArgs()) == 0
    # a result published through a slot
    slot = abi.SlotStorage(2)
    args = abi.CallArgs()
    args.memref(da.descriptor(), abi.DTYPE_F32).scalar(0, abi.KIND_I64)
    args.memref(db.descriptor(), abi.DTYPE_F32).scalar(1, abi.KIND_I64).scalar(0.0, abi.KIND_F32)
    args.slot(slot, abi.DTYPE_F32, 2)
    assert noalloc(hiplib, abi.matmul_payload(outkind="slot"), args) == 0
    # staging past the 16 MiB scratch: host A and B of 8 MiB each plus C
    big_a = np.zeros((2048, 1024), np.float32)
    big_b = np.zeros((1024, 2048), np.float32)
    big_c = np.full((2048, 2048), 7, np.float32)
    assert noalloc(hiplib, abi.matmul_payload(),
                   gemm_args(big_a, abi.DTYPE_F32, big_b, abi.DTYPE_F32, big_c,
                             abi.DTYPE_F32)) == 0
    assert np.all(big_c == 7)
    for x in (da, db, dc1, dc2):
        x.free()


def test_noalloc_calls_on_two_streams_take_turns(hiplib, rng):
    """Two calls with host operands on two streams, the second issued while
    the first one's GEMM may still read the scratch: the second call's
    stream waits for it, so both results match the oracle."""
    import oracle
    from vx_amd.runtime import HipTimer

    announce("noalloc GEMM: two streams, host bf16 operands 512x2048x1024 each")
    t = HipTimer()
    cases = [(f32_to_bf16(rng.normal(0, 1 / 32, (512, 2048)).astype(np.float32)),
              f32_to_bf16(rng.normal(0, 1 / 32, (2048, 1024)).astype(np.float32)))
             for _ in range(2)]
    # results allocated with no stream set (memory taken while a stream is
    # set is freed in that stream's order, so it must go before the stream)
    outs = [DeviceArray(hiplib, (512, 1024), abi.DTYPE_F32) for _ in cases]
    streams = [t.stream_create(), t.stream_create()]
    try:
        for (a16, b16), c, s in zip(cases, outs, streams):
            hiplib.lib.vx_hip_set_stream(s)
            assert noalloc(hiplib, abi.matmul_payload(),
                           gemm_args(a16, abi.DTYPE_BF16, b16, abi.DTYPE_BF16, c,
                                     abi.DTYPE_F32)) == 1
        hiplib.lib.vx_hip_set_stream(None)
        t.sync()
        for (a16, b16), c in zip(cases, outs):
            want = oracle.gemm_bf16_f32(a16, b16)
            got = c.numpy()
            assert np.abs(got - want).max() <= 1e-4 * max(1.0, float(np.abs(want).max()))
    finally:
        hiplib.lib.vx_hip_set_stream(None)
        t.sync()
        for c in outs:
            c.free()
        for s in streams:
            t.stream_destroy(s)
