"""Regions that carry their own gfx950 code object (`format=hsaco`) run from
it on the GPU: parameters marshalled from the ABI's descriptors, the launch
shape from `launch=` or `grid=`/`block=` with launch values, dynamic LDS from
`shared=`, the assert flag, the bundle form, and the module cache. Results
are checked against numpy on the same inputs (exact: every kernel here does
one rounding per element, in f32)."""

import ctypes

import numpy as np
import pytest

from tests.conftest import announce
from vx_amd import abi
from vx_amd.build import TEST_IMAGES
from vx_amd.runtime import DeviceArray

pytestmark = pytest.mark.gpu

ELF = TEST_IMAGES / "vx_image_kernels.hsaco"
BUNDLE = TEST_IMAGES / "vx_image_kernels.bundle.hsaco"


def counters(lib):
    return lib.image_stats(), lib.stats()["host_fallback"]


@pytest.mark.parametrize("image", [ELF, BUNDLE], ids=["elf", "bundle"])
def test_axpy_sized_by_launch_trip(hiplib, image, rng):
    announce(f"image axpy {image.name}")
    n = 100_003
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(n).astype(np.float32)
    dx, dy = DeviceArray.of(hiplib, x, abi.DTYPE_F32), DeviceArray.of(hiplib, y, abi.DTYPE_F32)
    args = abi.CallArgs()
    args.memref(dx.descriptor(), abi.DTYPE_F32).memref(dy.descriptor(), abi.DTYPE_F32)
    args.scalar(2.5, abi.KIND_F32)
    (st0, fb0) = counters(hiplib)
    hiplib.dispatch(abi.image_payload("vx_img_axpy", image.read_bytes(), topo="500",
                                      launch=str(n)), args)
    got = dy.numpy()
    (st1, fb1) = counters(hiplib)
    assert np.array_equal(got, np.float32(2.5) * x + y)
    assert st1["launches"] == st0["launches"] + 1 and fb1 == fb0
    dx.free()
    dy.free()


def test_strided_views_with_offsets(hiplib, rng):
    """x and y are views into larger buffers: offset 3, stride 2 and offset 5,
    stride 3 (the descriptor fields reach the kernel unchanged)."""
    announce("image axpy views")
    n = 5000
    xb = rng.standard_normal(3 + 2 * n).astype(np.float32)
    yb = rng.standard_normal(5 + 3 * n).astype(np.float32)
    dxb, dyb = DeviceArray.of(hiplib, xb, abi.DTYPE_F32), DeviceArray.of(hiplib, yb, abi.DTYPE_F32)
    xv = abi.Descriptor(dxb.ptr, (n,), strides=(2,), offset=3)
    yv = abi.Descriptor(dyb.ptr, (n,), strides=(3,), offset=5)
    args = abi.CallArgs()
    args.memref(xv, abi.DTYPE_F32).memref(yv, abi.DTYPE_F32).scalar(-0.75, abi.KIND_F32)
    hiplib.dispatch(abi.image_payload("vx_img_axpy", ELF.read_bytes(), topo="500",
                                      launch=f"{n // 7},64"), args)
    got = dyb.numpy()
    want = yb.copy()
    want[5::3][:n] = np.float32(-0.75) * xb[3::2][:n] + yb[5::3][:n]
    assert np.array_equal(got, want)
    dxb.free()
    dyb.free()


def test_grid_and_block_from_launch_values(hiplib, rng):
    """grid=$0,$1 (blocks over rows, split across two axes), block=$2: the
    i32 launch values after the kernel's arguments set the shape."""
    announce("image rows grid")
    rows, cols = 300, 777
    m = rng.standard_normal((rows, cols)).astype(np.float32)
    dm = DeviceArray.of(hiplib, m, abi.DTYPE_F32)
    args = abi.CallArgs()
    args.memref(dm.descriptor(), abi.DTYPE_F32).scalar(3, abi.KIND_I32)
    args.launch_value(150).launch_value(2).launch_value(96)
    hiplib.dispatch(abi.image_payload("vx_img_rows", ELF.read_bytes(), topo="500",
                                      grid="$0,$1", block="$2"), args)
    assert np.array_equal(dm.numpy(), 2 * m + 3)
    dm.free()


def test_dynamic_lds_from_shared(hiplib, rng):
    announce("image reverse shared")
    n, block = 1000, 256
    x = rng.standard_normal(n).astype(np.float32)
    dx = DeviceArray.of(hiplib, x, abi.DTYPE_F32)
    args = abi.CallArgs()
    args.memref(dx.descriptor(), abi.DTYPE_F32)
    args.launch_value((n + block - 1) // block)
    hiplib.dispatch(abi.image_payload("vx_img_reverse", ELF.read_bytes(), topo="500",
                                      grid="$0", block=str(block), shared=str(4 * block)), args)
    want = np.concatenate([x[i:i + block][::-1] for i in range(0, n, block)])
    assert np.array_equal(dx.numpy(), want)
    dx.free()


def test_assert_flag_that_holds(hiplib, rng):
    """assert_flag=1: the library appends a cleared device int; a kernel whose
    asserts hold leaves it 0 and the program goes on."""
    announce("image assert flag")
    x = np.abs(rng.standard_normal(4096).astype(np.float32))
    dx = DeviceArray.of(hiplib, x, abi.DTYPE_F32)
    args = abi.CallArgs()
    args.memref(dx.descriptor(), abi.DTYPE_F32)
    for _ in range(2):
        hiplib.dispatch(abi.image_payload("vx_img_check", ELF.read_bytes(), topo="500",
                                          launch="4096", assert_flag="1"), args)
    assert np.array_equal(dx.numpy(), x)
    dx.free()


def test_module_cache_loads_once(hiplib, rng):
    announce("image cache")
    x = rng.standard_normal(64).astype(np.float32)
    y = np.zeros(64, np.float32)
    dx, dy = DeviceArray.of(hiplib, x, abi.DTYPE_F32), DeviceArray.of(hiplib, y, abi.DTYPE_F32)
    args = abi.CallArgs()
    args.memref(dx.descriptor(), abi.DTYPE_F32).memref(dy.descriptor(), abi.DTYPE_F32)
    args.scalar(1.0, abi.KIND_F32)
    payload = abi.image_payload("vx_img_axpy", ELF.read_bytes(), topo="500", launch="64")
    buf = ctypes.create_string_buffer(payload, len(payload))
    argv, tags, na = args.arrays()
    st0 = hiplib.image_stats()
    for _ in range(5):
        hiplib.lib.vx_plugin_dispatch_async(buf, len(payload), argv, tags, na)
    got = dy.numpy()
    st1 = hiplib.image_stats()
    assert st1["launches"] - st0["launches"] == 5
    assert st1["loads"] - st0["loads"] <= 1
    assert np.array_equal(got, 5 * x)
    dx.free()
    dy.free()


HOST_AXPY_C = r"""
#include <stdint.h>
typedef struct { float *alloc, *aligned; int64_t offset, size, stride; } D1;
int64_t vx_host_worker_id(void);
int64_t vx_host_worker_count(void);
/* the outlined host form of vx_img_axpy: a `launch=` region, so (as the
 * compiler emits it) each host worker takes its slice of the range */
void _vx_ciface_vx_img_axpy(D1 *x, D1 *y, float a) {
  for (int64_t i = vx_host_worker_id(); i < x->size; i += vx_host_worker_count())
    y->aligned[y->offset + i * y->stride] =
        a * x->aligned[x->offset + i * x->stride] + y->aligned[y->offset + i * y->stride];
}
"""


@pytest.fixture(scope="module")
def host_axpy(tmp_path_factory):
    import subprocess
    d = tmp_path_factory.mktemp("host_axpy")
    (d / "k.c").write_text(HOST_AXPY_C)
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", "-ffp-contract=off", str(d / "k.c"), "-o",
                    str(d / "libk.so")], check=True)
    return ctypes.CDLL(str(d / "libk.so"), mode=ctypes.RTLD_GLOBAL)


def test_host_operands_take_the_host_path(hiplib, host_axpy, rng):
    """Views of host memory cannot be handed to the image: the region runs as
    its outlined host kernel instead, and no image launch is counted."""
    announce("image host operands")
    x = rng.standard_normal(100).astype(np.float32)
    y = rng.standard_normal(100).astype(np.float32)
    want = np.float32(1.5) * x + y
    args = abi.CallArgs()
    args.memref(abi.Descriptor(x.ctypes.data, x.shape), abi.DTYPE_F32)
    args.memref(abi.Descriptor(y.ctypes.data, y.shape), abi.DTYPE_F32).scalar(1.5, abi.KIND_F32)
    (st0, fb0) = counters(hiplib)
    hiplib.dispatch(abi.image_payload("vx_img_axpy", ELF.read_bytes(), topo="500", launch="100"),
                    args)
    (st1, fb1) = counters(hiplib)
    assert np.array_equal(y, want)
    assert st1["launches"] == st0["launches"] and fb1 == fb0 + 1


TIMED = r"""
import sys
sys.path.insert(0, {root!r})
import numpy as np
from vx_amd import abi
from vx_amd.build import TEST_IMAGES
from vx_amd.runtime import DispatchLibrary, DeviceArray
lib = DispatchLibrary()
n = 4096
x = np.arange(n, dtype=np.float32)
dx, dy = DeviceArray.of(lib, x, abi.DTYPE_F32), DeviceArray.of(lib, x, abi.DTYPE_F32)
args = abi.CallArgs()
args.memref(dx.descriptor(), abi.DTYPE_F32).memref(dy.descriptor(), abi.DTYPE_F32)
args.scalar(2.0, abi.KIND_F32)
img = (TEST_IMAGES / "vx_image_kernels.hsaco").read_bytes()
lib.dispatch(abi.image_payload("vx_img_axpy", img, topo="500", launch=str(n)), args)
assert np.array_equal(dy.numpy(), 3 * x)
print("ok", flush=True)
"""


def test_time_kernel_brackets_image_launches():
    """VX_TIME_KERNEL prints the device time of an image launch, not only of
    a routed GEMM (reference runtime/cuda_dispatch.cpp:1613-1665); run in a
    child process so the variable is read fresh."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    announce("VX_TIME_KERNEL on an image launch")
    root = Path(__file__).resolve().parent.parent
    res = subprocess.run([sys.executable, "-c", TIMED.format(root=str(root))],
                         capture_output=True, text=True, timeout=120,
                         env={**os.environ, "VX_TIME_KERNEL": "1"})
    assert res.returncode == 0 and "ok" in res.stdout, res.stderr[-2000:]
    assert "vx_img_axpy device time" in res.stderr, res.stderr[-2000:]
    assert "vx_img_axpy occupancy" in res.stderr, res.stderr[-2000:]
