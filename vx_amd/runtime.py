"""Host-side mirror of the Vx plugin ABI over libvx_hip_dispatch.so.

This is what a compiled Vx program does at run time, spelled in Python so
tests and the benchmark drive the library through the same C entry points:
``transfer()`` is vx_plugin_alloc_and_transfer on Topology::GPU[0] (id 500),
``c = a @ b`` is vx_plugin_dispatch_async with a kind=matmul payload, a host
read is vx_plugin_transfer_device_to_host, and the vx_nn ops are the
``extern "C"`` entry points of include/vx_hip_ops.h.

The library is loaded from this package directory; nothing falls back to
another implementation when it is missing.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

from . import abi

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libvx_hip_dispatch.so"

_c_size = ctypes.c_size_t
_vp = ctypes.c_void_p
_i32, _i64, _u32, _u64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64

# Every symbol include/vx_hardware_runtime.h and include/vx_hip_ops.h declare,
# with (restype, argtypes).
SIGNATURES = {
    "vx_plugin_alloc_and_transfer": (_vp, [_c_size, _vp, _u32, _u32]),
    "vx_plugin_alloc_and_transfer_async": (_vp, [_c_size, _vp, _u32, _u32]),
    "vx_plugin_dispatch_async": (_u64, [_vp, _c_size, _vp, _vp, _i64]),
    "vx_plugin_dispatch_async_flat": (_u64, [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int]),
    "vx_plugin_await_future": (None, [_u64]),
    "vx_plugin_transfer_device_to_host": (_i32, [_vp, _vp, _c_size, _u32]),
    "vx_plugin_transfer_peer": (_vp, [_vp, _u32, _u32, _c_size]),
    "vx_plugin_free": (None, [_vp, _u32]),
    "vx_plugin_arrivals_take": (_vp, [_vp, _c_size, _vp, _u32, _u32]),
    "vx_plugin_arrivals_give": (None, [_vp, _vp, _c_size, _u32]),
    "vx_plugin_release_future": (None, [_u64]),
    "vx_plugin_control": (_i32, [_u32, _vp]),
    "vx_plugin_tensor_map": (_i64, [_i64] * 18),
    "vx_cuda_set_stream": (None, [_vp]),
    "vx_cuda_get_stream": (_vp, []),
    "vx_collective_init": (None, [_i32, _i32]),
    "vx_collective_finish": (None, []),
    "vx_collective_rank": (_i32, []),
    "vx_collective_ranks": (_i32, []),
    "vx_collective_all_reduce_sum_f32": (None, [_vp, _vp, _i64]),
    "vx_collective_all_reduce_sum_bf16": (None, [_vp, _vp, _i64]),
    "vx_collective_all_gather_f32": (None, [_vp, _vp, _i64]),
    "vx_collective_all_gather_bf16": (None, [_vp, _vp, _i64]),
    "vx_host_worker_id": (_i64, []),
    "vx_host_worker_count": (_i64, []),
}

HIP_SIGNATURES = {
    "vx_hip_set_stream": (None, [_vp]),
    "vx_hip_get_stream": (_vp, []),
    "vx_nn_flash_attention_fwd_bf16": (
        _i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _i32]),
    "vx_nn_gemv_i8_bf16": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64]),
    "vx_llama_i8_create": (_vp, [_vp, _vp, _u32]),
    "vx_llama_i8_generate": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp, _i32]),
    "vx_llama_i8_logits": (_i32, [_vp, _vp, _i32, _vp]),
    "vx_llama_i8_destroy": (None, [_vp]),
    "vx_llama_i8_read": (_i32, [ctypes.c_char_p, _vp, ctypes.POINTER(_vp)]),
    "vx_llama_i8_host_weights": (_vp, [_vp]),
    "vx_llama_i8_host_free": (None, [_vp]),
    "vx_llama_i8_save": (_i32, [ctypes.c_char_p, _vp, _vp]),
    "vx_hip_image_param_count": (_i32, [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p]),
    "vx_hip_dispatch_async_noalloc": (_u64, [_vp, _c_size, _vp, _vp, _i64]),
}


def bind(lib: ctypes.CDLL, table: dict) -> None:
    for name, (res, args) in table.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


class DispatchLibrary:
    """A loaded dispatch library and the ABI calls on it."""

    def __init__(self, path: os.PathLike | str = LIB_PATH, hip: bool = True,
                 global_scope: bool = True):
        """global_scope: load the library into the process's global symbol
        scope, as a program's one dispatch library is, so outlined host
        kernels resolve vx_host_worker_id / _count to it. A second dispatch
        library in the same process (the reference's, as a checker) loads
        with global_scope=False, so it never supplies those symbols."""
        path = Path(path)
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is not built; run `python -m vx_amd.build` (or __graft_entry__.build())")
        self.path = path
        self.lib = ctypes.CDLL(str(path),
                               mode=ctypes.RTLD_GLOBAL if global_scope else ctypes.RTLD_LOCAL)
        bind(self.lib, SIGNATURES)
        self.hip = hip
        if hip:
            bind(self.lib, HIP_SIGNATURES)

    # -- lifecycle ---------------------------------------------------------
    def device_count(self) -> int:
        return self.lib.vx_plugin_control(abi.CTRL_GET_DEVICE_COUNT, None)

    def control(self, opcode: int, payload=None) -> int:
        return self.lib.vx_plugin_control(opcode, payload)

    def wait(self, topo: int = abi.TOPO_GPU_BASE) -> None:
        t = ctypes.c_int32(topo)
        self.lib.vx_plugin_control(abi.CTRL_WAIT, ctypes.byref(t))

    def stats(self) -> dict:
        out = (ctypes.c_int64 * 5)()
        if not self.lib.vx_plugin_control(abi.HIP_CTRL_STATS, out):
            raise RuntimeError("the library answered no statistics")
        return dict(gemm_device=out[0], gemm_mfma=out[1], gemm_tiled=out[2],
                    host_fallback=out[3], staged_bytes=out[4])

    def image_stats(self) -> dict:
        out = (ctypes.c_int64 * 2)()
        if not self.lib.vx_plugin_control(abi.HIP_CTRL_IMAGE_STATS, out):
            raise RuntimeError("the library answered no image statistics")
        return dict(launches=out[0], loads=out[1])

    def image_param_count(self, image: bytes, kernel: str) -> int:
        return self.lib.vx_hip_image_param_count(image, len(image), kernel.encode())

    def force_gemm_kernel(self, which: int) -> None:
        v = ctypes.c_int32(which)
        if not self.lib.vx_plugin_control(abi.HIP_CTRL_GEMM_KERNEL, ctypes.byref(v)):
            raise ValueError(f"no GEMM kernel {which}")

    def gemm_workspaces(self) -> dict:
        """Stream-K GEMM workspaces held (one per device and stream that ran
        such a launch), their bytes, stream-K launches so far, and the
        workgroups (CUs) such a launch runs."""
        out = (ctypes.c_int64 * 4)()
        if not self.lib.vx_plugin_control(abi.HIP_CTRL_GEMM_WORKSPACES, out):
            raise RuntimeError("the library answered no stream-K statistics")
        return dict(blocks=out[0], bytes=out[1], launches=out[2], groups=out[3])

    def force_gemv_kernel(self, which: int) -> None:
        v = ctypes.c_int32(which)
        if not self.lib.vx_plugin_control(abi.HIP_CTRL_GEMV_KERNEL, ctypes.byref(v)):
            raise ValueError(f"no GEMV kernel {which}")

    def force_fa_splits(self, splits: int) -> None:
        """Cut every flash-attention launch's key range into `splits` parts
        (0: the automatic choice; graph capture always runs unsplit)."""
        v = ctypes.c_int32(splits)
        if not self.lib.vx_plugin_control(abi.HIP_CTRL_FA_SPLITS, ctypes.byref(v)):
            raise ValueError(f"no flash-attention split count {splits}")

    def clock_stamps(self, base: int | None, slots: int) -> None:
        """Have routed MFMA GEMMs record their clock counters (4 x u64 per
        launch: shader clock and 100 MHz real-time counter at the start and
        end of workgroup 0) into a ring of `slots` records at the HBM address
        `base`; base None stops it."""
        class _Ring(ctypes.Structure):
            _fields_ = [("base", ctypes.c_void_p), ("slots", ctypes.c_int64)]

        ring = _Ring(base, slots)
        if not self.lib.vx_plugin_control(abi.HIP_CTRL_CLOCK_STAMPS, ctypes.byref(ring)):
            raise ValueError("the library refused the clock-stamp ring")

    # -- memory ------------------------------------------------------------
    def transfer(self, array: np.ndarray | None, nbytes: int | None = None,
                 topo: int = abi.TOPO_GPU_BASE, space_access: int = 0) -> int:
        """vx_plugin_alloc_and_transfer: a new allocation in `topo`'s memory
        holding `array` (or `nbytes` uninitialised)."""
        if array is not None:
            array = np.ascontiguousarray(array)
            nbytes = array.nbytes
            src = array.ctypes.data
        else:
            src = None
        ptr = self.lib.vx_plugin_alloc_and_transfer(nbytes, src, topo, space_access)
        if not ptr:
            raise MemoryError(f"vx_plugin_alloc_and_transfer({nbytes}) returned NULL")
        return ptr

    def fetch(self, ptr: int, out: np.ndarray, topo: int = abi.TOPO_GPU_BASE) -> np.ndarray:
        assert out.flags.c_contiguous
        self.lib.vx_plugin_transfer_device_to_host(ptr, out.ctypes.data, out.nbytes, topo)
        return out

    def free(self, ptr: int, topo: int = abi.TOPO_GPU_BASE) -> None:
        self.lib.vx_plugin_free(ptr, topo)

    # -- dispatch ------------------------------------------------------------
    def dispatch(self, payload: bytes, args: abi.CallArgs) -> int:
        buf = ctypes.create_string_buffer(payload, len(payload))
        argv, tags, n = args.arrays()
        return self.lib.vx_plugin_dispatch_async(buf, len(payload), argv, tags, n)


class DeviceArray:
    """An allocation from vx_plugin_alloc_and_transfer with its shape and
    element type. `dtype` is an abi.DTYPE_* code; bf16/f16 travel as uint16."""

    NP = {abi.DTYPE_F32: np.float32, abi.DTYPE_F64: np.float64, abi.DTYPE_BF16: np.uint16,
          abi.DTYPE_F16: np.uint16, abi.DTYPE_I8: np.int8, abi.DTYPE_I32: np.int32,
          abi.DTYPE_I64: np.int64}

    def __init__(self, lib: DispatchLibrary, shape, dtype: int, host: np.ndarray | None = None,
                 topo: int = abi.TOPO_GPU_BASE):
        self.lib, self.shape, self.dtype, self.topo = lib, tuple(shape), dtype, topo
        self.nbytes = int(np.prod(self.shape)) * abi.DTYPE_BYTES[dtype]
        if host is not None:
            host = np.ascontiguousarray(host, dtype=self.NP[dtype])
            assert host.shape == self.shape, (host.shape, self.shape)
        self.ptr = lib.transfer(host, self.nbytes, topo)

    @classmethod
    def of(cls, lib, host: np.ndarray, dtype: int, topo: int = abi.TOPO_GPU_BASE) -> "DeviceArray":
        return cls(lib, host.shape, dtype, host, topo)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.NP[self.dtype])
        return self.lib.fetch(self.ptr, out, self.topo)

    def descriptor(self, strides=None, offset: int = 0, sizes=None) -> abi.Descriptor:
        return abi.Descriptor(self.ptr, sizes if sizes is not None else self.shape, strides, offset)

    def free(self) -> None:
        if self.ptr:
            self.lib.free(self.ptr, self.topo)
            self.ptr = 0


def matmul(lib: DispatchLibrary, a: abi.Descriptor, a_dtype: int, b: abi.Descriptor,
           b_dtype: int, out, out_dtype: int, outkind: str = "buffer",
           topo: int = abi.TOPO_GPU_BASE) -> int:
    """Dispatch ``out = a @ b`` in the argument shape the compiler emits for
    `c = a @ b`: six launch operands, A at 0, B at 2, the result at 5, loop
    bounds and the fill constant between (reference
    tests/runtime/gemm_plan_test.cpp:130-175). `out` is a Descriptor (buffer
    filled in place) or a SlotStorage (result published through the slot)."""
    args = abi.CallArgs()
    args.memref(a, a_dtype).scalar(0, abi.KIND_I64).memref(b, b_dtype)
    args.scalar(1, abi.KIND_I64).scalar(0.0, abi.KIND_F32)
    if isinstance(out, abi.SlotStorage):
        args.slot(out, out_dtype, 2)
    else:
        args.memref(out, out_dtype)
    return lib.dispatch(abi.matmul_payload(outkind=outkind, topo=topo), args)


def flash_attention_fwd(lib: DispatchLibrary, q: int, k: int, v: int, o: int, lse: int | None,
                        batch: int, heads: int, kv_heads: int, seq_q: int, seq_k: int,
                        head_dim: int, scale: float, causal: bool) -> int:
    return lib.lib.vx_nn_flash_attention_fwd_bf16(q, k, v, o, lse, batch, heads, kv_heads, seq_q,
                                                  seq_k, head_dim, scale, 1 if causal else 0)


def gemv_i8(lib: DispatchLibrary, w: int, scale: int, x: int, y: int, rows: int, cols: int,
            batch: int) -> int:
    return lib.lib.vx_nn_gemv_i8_bf16(w, scale, x, y, rows, cols, batch)


class HipTimer:
    """hipEvent timing on the stream the library launches on (the calling
    thread's caller stream; the null stream by default)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so", mode=ctypes.RTLD_GLOBAL)
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(_vp)]
        self.hip.hipEventRecord.argtypes = [_vp, _vp]
        self.hip.hipEventSynchronize.argtypes = [_vp]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _vp, _vp]
        self.hip.hipEventDestroy.argtypes = [_vp]
        self.hip.hipDeviceSynchronize.argtypes = []

    def event(self):
        e = _vp()
        self._check(self.hip.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e

    def record(self, e, stream=None) -> None:
        self._check(self.hip.hipEventRecord(e, stream), "hipEventRecord")

    def elapsed_ms(self, start, stop) -> float:
        self._check(self.hip.hipEventSynchronize(stop), "hipEventSynchronize")
        ms = ctypes.c_float()
        self._check(self.hip.hipEventElapsedTime(ctypes.byref(ms), start, stop),
                    "hipEventElapsedTime")
        return ms.value

    def sync(self) -> None:
        self._check(self.hip.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream_create(self):
        """A new stream at the default priority."""
        self.hip.hipStreamCreate.argtypes = [ctypes.POINTER(_vp)]
        s = _vp()
        self._check(self.hip.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s

    def stream_destroy(self, s) -> None:
        self.hip.hipStreamDestroy.argtypes = [_vp]
        self._check(self.hip.hipStreamDestroy(s), "hipStreamDestroy")

    def capture(self, stream, body):
        """Run body() with `stream` capturing (relaxed mode), and return the
        instantiated graph of what it launched there."""
        h = self.hip
        h.hipStreamBeginCapture.argtypes = [_vp, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [_vp, ctypes.POINTER(_vp)]
        h.hipGraphInstantiate.argtypes = [ctypes.POINTER(_vp), _vp, _vp, _vp, ctypes.c_size_t]
        h.hipGraphDestroy.argtypes = [_vp]
        self._check(h.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")
        try:
            body()
        finally:
            g = _vp()
            self._check(h.hipStreamEndCapture(stream, ctypes.byref(g)), "hipStreamEndCapture")
        ex = _vp()
        self._check(h.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0),
                    "hipGraphInstantiate")
        self._check(h.hipGraphDestroy(g), "hipGraphDestroy")
        return ex

    def graph_launch(self, ex, stream) -> None:
        self.hip.hipGraphLaunch.argtypes = [_vp, _vp]
        self._check(self.hip.hipGraphLaunch(ex, stream), "hipGraphLaunch")

    def graph_destroy(self, ex) -> None:
        self.hip.hipGraphExecDestroy.argtypes = [_vp]
        self._check(self.hip.hipGraphExecDestroy(ex), "hipGraphExecDestroy")

    @staticmethod
    def _check(rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")
