"""The Vx plugin ABI from the caller's side, for driving a dispatch library
exactly as compiled Vx code does.

Without vxc in this image, payloads, tags and descriptors are built by hand
from what the compiler emits (reference src/dialect/VxLowering.cpp:9609-9939
builds them; tests/runtime/gemm_plan_test.cpp:43-90 builds them by hand the
same way):

- a payload is the kernel name, then NUL-terminated ``key=value`` entries in
  the order abi=, kind=, roles=, outkind=, topo=, ...;
- an argument tag is ``slot << 24 | rank << 16 | dtype << 8 | kind``;
- ``device_args[i]`` points at the argument: for a memref, at a pointer to
  its descriptor ``{allocated, aligned, offset, sizes[r], strides[r]}``; for a
  scalar, at the value.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

# Tag layout and codes (reference include/vx_hardware_runtime.h:80-130).
KIND_MEMREF, KIND_I1, KIND_I8, KIND_I16, KIND_I32, KIND_I64, KIND_F32, KIND_F64 = range(8)
DTYPE_I1, DTYPE_I8, DTYPE_I16, DTYPE_I32, DTYPE_I64 = 1, 2, 3, 4, 5
DTYPE_F32, DTYPE_F64, DTYPE_F16, DTYPE_BF16 = 6, 7, 8, 9
SLOT_BIT = 1 << 24
PAYLOAD_ABI = 1
TOPO_CPU = 0
TOPO_GPU_BASE = 500

DTYPE_BYTES = {DTYPE_I1: 1, DTYPE_I8: 1, DTYPE_I16: 2, DTYPE_I32: 4, DTYPE_I64: 8,
               DTYPE_F32: 4, DTYPE_F64: 8, DTYPE_F16: 2, DTYPE_BF16: 2}

# Control opcodes (reference include/vx_hardware_runtime.h:705-732) and this
# library's vendor opcodes.
CTRL_INIT_DEVICE, CTRL_SHUTDOWN, CTRL_GET_DEVICE_COUNT = 0x01, 0x02, 0x03
CTRL_LOCAL_DEVICE, CTRL_WAIT, CTRL_WAIT_FOR_TENSORS, CTRL_WAIT_FOR_THREAD = 0x04, 0x05, 0x06, 0x07
CTRL_VENDOR_BASE = 0x1000
HIP_CTRL_GEMM_KERNEL = CTRL_VENDOR_BASE + 1
HIP_CTRL_STATS = CTRL_VENDOR_BASE + 2
HIP_CTRL_POOL_DRAIN = CTRL_VENDOR_BASE + 3
HIP_CTRL_IMAGE_STATS = CTRL_VENDOR_BASE + 4
HIP_CTRL_CLOCK_STAMPS = CTRL_VENDOR_BASE + 5
HIP_CTRL_GEMV_KERNEL = CTRL_VENDOR_BASE + 6
HIP_CTRL_FA_SPLITS = CTRL_VENDOR_BASE + 7
HIP_CTRL_FA_WORKSPACES = CTRL_VENDOR_BASE + 8
HIP_CTRL_STAGING_STATS = CTRL_VENDOR_BASE + 9
HIP_CTRL_GEMM_WORKSPACES = CTRL_VENDOR_BASE + 10
# Kernels the GEMV control opcode can force (0 = automatic choice).
GEMV_AUTO, GEMV_ROWS, GEMV_DOT2_B4, GEMV_LDS = 0, 1, 2, 3
# Kernels the GEMM control opcode can force (0 = automatic choice).
GEMM_AUTO, GEMM_TILED, GEMM_MFMA_PP, GEMM_F32_MFMA, GEMM_MFMA_SK = 0, 2, 8, 9, 10


def memref_tag(dtype: int, rank: int) -> int:
    return (rank << 16) | (dtype << 8)


def slot_tag(dtype: int, rank: int) -> int:
    return SLOT_BIT | memref_tag(dtype, rank)


def payload(name: str, **entries: str) -> bytes:
    """``name\\0k=v\\0...`` with the entries in the order given."""
    out = name.encode() + b"\0"
    for key, value in entries.items():
        out += f"{key}={value}".encode() + b"\0"
    return out


def matmul_payload(name: str = "vx_npu_kernel_0", roles: str = "a:0,b:2,out:5",
                   outkind: str = "buffer", topo: int | None = TOPO_GPU_BASE,
                   abi: int | None = PAYLOAD_ABI) -> bytes:
    """The payload LaunchOpLowering writes for a region classified
    ``kind=matmul`` (pinned bytes: reference
    tests/optimizations/pass/kernel_kind_matmul.vx:48-68)."""
    entries: dict[str, str] = {}
    if abi is not None:
        entries["abi"] = str(abi)
    entries["kind"] = "matmul"
    entries["roles"] = roles
    entries["outkind"] = outkind
    if topo is not None:
        entries["topo"] = str(topo)
    return payload(name, **entries)


def image_payload(name: str, image: bytes, fmt: str = "hsaco", **entries: str) -> bytes:
    """A payload whose device image rides in the binary section: the text
    entries (``abi=1``, the given ones, ``format=``), the empty entry, the
    image's length as a little-endian u64, then its bytes (the section
    grammar of reference include/vx_hardware_runtime.h:414-563)."""
    fields = {"abi": str(PAYLOAD_ABI), **entries, "format": fmt}
    return payload(name, **fields) + b"\0" + len(image).to_bytes(8, "little") + image


class Descriptor:
    """A ranked memref descriptor in its own storage (int64 words)."""

    def __init__(self, data_ptr: int, sizes, strides=None, offset: int = 0):
        sizes = list(sizes)
        rank = len(sizes)
        if strides is None:
            strides, run = [0] * rank, 1
            for d in range(rank - 1, -1, -1):
                strides[d] = run
                run *= sizes[d]
        self.rank = rank
        self.words = (ctypes.c_int64 * (3 + 2 * rank))()
        self.words[0] = data_ptr
        self.words[1] = data_ptr
        self.words[2] = offset
        for d in range(rank):
            self.words[3 + d] = sizes[d]
            self.words[3 + rank + d] = strides[d]

    @property
    def address(self) -> int:
        return ctypes.addressof(self.words)

    @property
    def aligned(self) -> int:
        return self.words[1]

    @property
    def offset(self) -> int:
        return self.words[2]

    @property
    def sizes(self) -> list[int]:
        return [self.words[3 + d] for d in range(self.rank)]

    @property
    def strides(self) -> list[int]:
        return [self.words[3 + self.rank + d] for d in range(self.rank)]


class SlotStorage:
    """Storage a kernel publishes a rank-r descriptor into, and the rank-0
    memref (the slot) that names it."""

    def __init__(self, rank: int):
        self.rank = rank
        self.inner = (ctypes.c_int64 * (3 + 2 * rank))()
        self.slot = (ctypes.c_int64 * 3)()
        self.slot[0] = ctypes.addressof(self.inner)
        self.slot[1] = ctypes.addressof(self.inner)
        self.slot[2] = 0

    @property
    def address(self) -> int:
        return ctypes.addressof(self.slot)

    def published(self) -> tuple[int, int, list[int], list[int]]:
        """(data pointer, offset, sizes, strides) the kernel wrote."""
        r = self.rank
        return (self.inner[1], self.inner[2], [self.inner[3 + d] for d in range(r)],
                [self.inner[3 + r + d] for d in range(r)])


@dataclass
class CallArgs:
    """``device_args`` and ``arg_tags`` for vx_plugin_dispatch_async, with
    everything they point at kept alive."""

    tags: list[int] = field(default_factory=list)
    _cells: list = field(default_factory=list)
    _ptrs: list[int] = field(default_factory=list)
    _launch_values: int = 0

    def memref(self, desc: Descriptor, dtype: int) -> "CallArgs":
        if self._launch_values:
            raise ValueError("launch values come after every kernel argument")
        cell = ctypes.c_void_p(desc.address)
        self._cells.append((cell, desc))
        self._ptrs.append(ctypes.addressof(cell))
        self.tags.append(memref_tag(dtype, desc.rank))
        return self

    def slot(self, storage, dtype: int, rank: int) -> "CallArgs":
        """A slot argument: `storage` is a SlotStorage, or a rank-0 slot
        memref naming an existing descriptor (a local tensor captured through
        its slot)."""
        if self._launch_values:
            raise ValueError("launch values come after every kernel argument")
        cell = ctypes.c_void_p(storage.address)
        self._cells.append((cell, storage))
        self._ptrs.append(ctypes.addressof(cell))
        self.tags.append(slot_tag(dtype, rank))
        return self

    def launch_value(self, value: int) -> "CallArgs":
        """An i32 launch value (`$j` of a payload's shape entries): placed after
        the kernel's arguments and not counted in num_args."""
        self._scalar(value, KIND_I32)
        self._launch_values += 1
        return self

    def scalar(self, value, kind: int) -> "CallArgs":
        if self._launch_values:
            raise ValueError("launch values come after every kernel argument")
        return self._scalar(value, kind)

    def _scalar(self, value, kind: int) -> "CallArgs":
        ctype = {KIND_I1: ctypes.c_uint8, KIND_I8: ctypes.c_int8, KIND_I16: ctypes.c_int16,
                 KIND_I32: ctypes.c_int32, KIND_I64: ctypes.c_int64, KIND_F32: ctypes.c_float,
                 KIND_F64: ctypes.c_double}[kind]
        cell = ctype(value)
        self._cells.append(cell)
        self._ptrs.append(ctypes.addressof(cell))
        self.tags.append(kind)
        return self

    def arrays(self):
        """(device_args, arg_tags, num_args); launch values follow the
        num_args kernel arguments in both arrays."""
        n = len(self._ptrs)
        args = (ctypes.c_void_p * max(n, 1))(*self._ptrs)
        tags = (ctypes.c_int32 * max(n, 1))(*[t if t < 2**31 else t - 2**32 for t in self.tags])
        self._cells.append((args, tags))
        return args, tags, n - self._launch_values


class SlotRef:
    """A rank-0 slot memref naming an existing descriptor."""

    def __init__(self, desc: Descriptor):
        self.desc = desc
        self.slot = (ctypes.c_int64 * 3)()
        self.slot[0] = desc.address
        self.slot[1] = desc.address
        self.slot[2] = 0

    @property
    def address(self) -> int:
        return ctypes.addressof(self.slot)


# bf16 helpers (numpy has no bf16): bit patterns travel as uint16.
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + (0x7FFF + ((u >> 16) & 1))) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
