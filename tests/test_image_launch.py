"""The device-image path on the CPU: the parameter count the library reads
from a gfx950 code object's metadata (the check it makes before any launch),
on the bare ELF and on the clang offload bundle the build makes from
tests/images/vx_image_kernels.hip, and an image payload on a machine without
a GPU running the outlined host kernel instead."""

import ctypes
import subprocess

import numpy as np
import pytest

from tests.test_library import KERNEL_C, gpu_present
from vx_amd import abi
from vx_amd.runtime import LIB_PATH, DispatchLibrary
from vx_amd.build import TEST_IMAGES

IMAGES = [TEST_IMAGES / "vx_image_kernels.hsaco", TEST_IMAGES / "vx_image_kernels.bundle.hsaco"]

# Memref arguments explode into 3 + 2·rank parameters (allocated, aligned,
# offset, sizes, strides), scalars into one (reference
# tests/runtime/kernel_launch_test.cpp: 28 for four rank-2 memrefs).
WANT = {"vx_img_axpy": 5 + 5 + 1, "vx_img_rows": 7 + 1, "vx_img_check": 5 + 1,
        "vx_img_reverse": 5}


@pytest.fixture(scope="module")
def cpulib():
    if not LIB_PATH.exists() or not all(p.exists() for p in IMAGES):
        from vx_amd.build import build, build_test_images
        build()
        build_test_images()
    return DispatchLibrary()


@pytest.mark.parametrize("image", IMAGES, ids=["elf", "bundle"])
def test_declared_parameter_counts(cpulib, image):
    data = image.read_bytes()
    for kernel, n in WANT.items():
        assert cpulib.image_param_count(data, kernel) == n, kernel


@pytest.mark.parametrize("image", IMAGES, ids=["elf", "bundle"])
def test_absent_entries_and_broken_images(cpulib, image):
    data = image.read_bytes()
    # a prefix of a name is not the name, and an absent kernel is -1, not 0
    assert cpulib.image_param_count(data, "vx_img_ax") == -1
    assert cpulib.image_param_count(data, "vx_img_axpy2") == -1
    assert cpulib.image_param_count(data, "nothing") == -1
    # truncations anywhere fail closed
    for cut in (3, 16, 64, len(data) // 3, len(data) // 2, len(data) - 1):
        assert cpulib.image_param_count(data[:cut], "vx_img_axpy") in (-1, WANT["vx_img_axpy"])
    assert cpulib.image_param_count(b"\x7fELF" + bytes(60), "vx_img_axpy") == -1
    assert cpulib.image_param_count(b"not an image at all", "vx_img_axpy") == -1


def test_bundle_for_another_target_is_not_read(cpulib):
    """The bundle's entries are chosen by target: renaming gfx950 in every
    entry's triple leaves nothing this library runs."""
    data = bytearray(IMAGES[1].read_bytes())
    head = bytes(data[:4096])
    at = head.find(b"gfx950")
    assert at > 0
    while at > 0:
        data[at:at + 6] = b"gfx942"
        at = bytes(data[:4096]).find(b"gfx950")
    assert cpulib.image_param_count(bytes(data), "vx_img_axpy") == -1


def test_payload_section_framing():
    """text entries, the empty entry, a little-endian u64 length, the bytes"""
    p = abi.image_payload("vx_img_axpy", b"\x01\x02\x03", launch="7")
    assert p.startswith(b"vx_img_axpy\0abi=1\0launch=7\0format=hsaco\0\0")
    assert p.endswith((3).to_bytes(8, "little") + b"\x01\x02\x03")


@pytest.fixture(scope="module")
def outlined(tmp_path_factory):
    d = tmp_path_factory.mktemp("outlined_img")
    src = d / "k.c"
    src.write_text(KERNEL_C)
    so = d / "libk.so"
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", "-ffp-contract=off", str(src), "-o", str(so)],
                   check=True)
    return ctypes.CDLL(str(so), mode=ctypes.RTLD_GLOBAL)


def test_image_payload_with_host_operands_runs_on_the_host(cpulib, outlined):
    """Host memory cannot be handed to a device image: the region runs as its
    outlined host kernel, as any region with no usable image does."""
    if gpu_present(cpulib):
        pytest.skip("checked on the GPU by test_gpu_image.py")
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    out = np.zeros((3, 4), np.float32)
    args = abi.CallArgs()
    args.memref(abi.Descriptor(a.ctypes.data, a.shape), abi.DTYPE_F32)
    args.scalar(2.5, abi.KIND_F32)
    args.memref(abi.Descriptor(out.ctypes.data, out.shape), abi.DTYPE_F32)
    cpulib.dispatch(abi.image_payload("vx_test_kernel_0", IMAGES[0].read_bytes(), topo="500"), args)
    assert np.array_equal(out, a * 2.5 + 1)
