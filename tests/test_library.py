"""CPU-side checks of libvx_hip_dispatch.so: it loads, exports every symbol
include/*.h declares, and (on a machine without a GPU) answers the ABI the
way the reference libraries do without a device: host memory for
transfers, the outlined host kernel for a dispatch, errors for the ops."""

import ctypes
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from vx_amd import abi
from vx_amd.runtime import HIP_SIGNATURES, LIB_PATH, SIGNATURES, DispatchLibrary

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^[A-Za-z_][\w \*]*?\b(vx_\w+)\s*\(", re.M)


def declared(header: Path) -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    text = re.sub(r"#define[^\n]*(\\\n[^\n]*)*", "", text)
    names = set()
    for m in DECL.finditer(text):
        line = text[m.start():text.index("\n", m.start())]
        if "static inline" in line or line.lstrip().startswith("return"):
            continue
        names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def cpulib():
    if not LIB_PATH.exists():
        from vx_amd.build import build
        build()
    return DispatchLibrary()


def test_every_declared_symbol_is_exported(cpulib):
    want = set()
    for h in (ROOT / "include").glob("*.h"):
        want |= declared(h)
    assert "vx_plugin_dispatch_async" in want and "vx_nn_gemv_i8_bf16" in want
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = want - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    # and every one of them is bound with a signature on the Python side
    assert want <= set(SIGNATURES) | set(HIP_SIGNATURES)


def test_same_plugin_symbols_as_reference_library():
    import oracle
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built")
    def syms(p):
        out = subprocess.run(["nm", "-D", "--defined-only", str(p)], capture_output=True,
                             text=True, check=True).stdout
        return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    ref = {s for s in syms(oracle.REF_LIB) if s.startswith("vx_")}
    ours = syms(LIB_PATH)
    assert ref <= ours, f"reference exports we lack: {sorted(ref - ours)}"


def test_exports_only_the_c_abi():
    """Every dynamic symbol the library defines is part of the C ABI (vx_*):
    its C++ internals stay local, so two libraries loaded into one process
    (two builds of this one, or another with the same C++ names) never bind
    to each other's internals."""
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    names = [ln.split()[-1] for ln in out.splitlines() if ln.strip()]
    assert names and all(n.startswith("vx_") for n in names), \
        sorted(n for n in names if not n.startswith("vx_"))[:10]


def gpu_present(lib) -> bool:
    return lib.device_count() > 0


def test_without_a_gpu_transfers_are_host_memory(cpulib):
    if gpu_present(cpulib):
        pytest.skip("a GPU is present")
    x = np.arange(10, dtype=np.float32)
    p = cpulib.transfer(x, topo=500)
    assert np.array_equal(np.ctypeslib.as_array((ctypes.c_float * 10).from_address(p)), x)
    back = np.zeros_like(x)
    cpulib.fetch(p, back)
    assert np.array_equal(back, x)
    q = cpulib.lib.vx_plugin_transfer_peer(p, 500, 500, 40)
    cpulib.free(q)
    cpulib.free(p)
    assert cpulib.lib.vx_plugin_control(abi.CTRL_INIT_DEVICE, None) == 0
    assert cpulib.lib.vx_plugin_tensor_map(*([0] * 18)) == 0
    assert cpulib.lib.vx_host_worker_id() == 0 and cpulib.lib.vx_host_worker_count() == 1


def test_without_a_gpu_ops_refuse(cpulib):
    if gpu_present(cpulib):
        pytest.skip("a GPU is present")
    assert cpulib.lib.vx_nn_gemv_i8_bf16(1, 1, 1, 1, 16, 16, 1) == -2
    assert cpulib.lib.vx_nn_flash_attention_fwd_bf16(1, 1, 1, 1, None, 1, 1, 1, 1, 1, 64,
                                                     0.1, 1) == -2


KERNEL_C = r"""
#include <stdint.h>
typedef struct { float *alloc, *aligned; int64_t offset, sizes[2], strides[2]; } D2;
/* an outlined region: out[i][j] = a[i][j] * s + 1 */
void _vx_ciface_vx_test_kernel_0(D2 *a, float s, D2 *out) {
  for (int64_t i = 0; i < a->sizes[0]; ++i)
    for (int64_t j = 0; j < a->sizes[1]; ++j)
      out->aligned[out->offset + i * out->strides[0] + j * out->strides[1]] =
          a->aligned[a->offset + i * a->strides[0] + j * a->strides[1]] * s + 1.0f;
}
/* a `launch=` region split over host workers: each worker takes every
 * count-th row from its id, and records its id and the worker count */
int64_t vx_host_worker_id(void);
int64_t vx_host_worker_count(void);
void _vx_ciface_vx_test_kernel_2(D2 *out) {
  for (int64_t i = vx_host_worker_id(); i < out->sizes[0]; i += vx_host_worker_count()) {
    out->aligned[out->offset + i * out->strides[0]] = (float)vx_host_worker_id();
    out->aligned[out->offset + i * out->strides[0] + 1] = (float)vx_host_worker_count();
  }
}
/* the outlined loop nest of a classified matmul (used when no GPU runs it) */
void _vx_ciface_vx_test_kernel_1(D2 *a, int64_t i0, D2 *b, int64_t i1, float fill, D2 *c) {
  for (int64_t i = 0; i < a->sizes[0]; ++i)
    for (int64_t j = 0; j < b->sizes[1]; ++j) {
      float acc = fill;
      for (int64_t k = 0; k < a->sizes[1]; ++k)
        acc += a->aligned[a->offset + i * a->strides[0] + k] *
               b->aligned[b->offset + k * b->strides[0] + j];
      c->aligned[c->offset + i * c->strides[0] + j] = acc;
    }
}
"""


@pytest.fixture(scope="module")
def outlined(tmp_path_factory):
    d = tmp_path_factory.mktemp("outlined")
    src = d / "k.c"
    src.write_text(KERNEL_C)
    so = d / "libk.so"
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", "-ffp-contract=off", str(src), "-o", str(so)],
                   check=True)
    return ctypes.CDLL(str(so), mode=ctypes.RTLD_GLOBAL)


def test_unrouted_dispatch_runs_the_outlined_host_kernel(cpulib, outlined):
    """A region with no kind= goes to _vx_ciface_<name> through libffi, with
    the calling convention rebuilt from the tags (memref, f32, memref)."""
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    out = np.zeros((3, 4), np.float32)
    args = abi.CallArgs()
    args.memref(abi.Descriptor(a.ctypes.data, a.shape), abi.DTYPE_F32)
    args.scalar(2.5, abi.KIND_F32)
    args.memref(abi.Descriptor(out.ctypes.data, out.shape), abi.DTYPE_F32)
    cpulib.dispatch(abi.payload("vx_test_kernel_0", abi="1", topo="500"), args)
    assert np.array_equal(out, a * 2.5 + 1)


@pytest.mark.parametrize("threads,payload_entries,want", [
    ("3", {"launch": "12"}, 3),           # VX_HOST_THREADS wins
    ("100", {"launch": "12"}, 12),        # never more workers than iterations
    ("0", {"launch": "12"}, 1),           # 0 (or nonsense) is serial
    ("4", {"launch": "12,64"}, 1),        # the two-level form is not split
    ("4", {}, 1),                         # an unproven region is not split
    ("4", {"host_blocks": "1", "grid": "6", "block": "32"}, 4),
])
def test_split_regions_run_on_host_workers(cpulib, outlined, monkeypatch, threads,
                                           payload_entries, want):
    """`launch=`/`host_blocks=` regions run on VX_HOST_THREADS workers, each
    reading its slice from vx_host_worker_id/count (reference
    runtime/vx_host_call.h:132-238)."""
    monkeypatch.setenv("VX_HOST_THREADS", threads)
    out = np.full((12, 2), -1, np.float32)
    args = abi.CallArgs()
    args.memref(abi.Descriptor(out.ctypes.data, out.shape), abi.DTYPE_F32)
    cpulib.dispatch(abi.payload("vx_test_kernel_2", abi="1", **payload_entries), args)
    assert np.all(out[:, 1] == want), out
    assert np.array_equal(out[:, 0], np.arange(12) % want), out
    assert cpulib.lib.vx_host_worker_id() == 0 and cpulib.lib.vx_host_worker_count() == 1


def test_reference_library_loaded_first_supplies_no_symbols(cpulib, outlined):
    """The reference library loaded into the same process before this one (as
    the oracle's checker or the bench's CPU baseline may load it) stays out of
    the global symbol scope: an outlined kernel's vx_host_worker_id / _count
    still resolve to this library and see its worker split. A fresh process,
    so that the load order is the one under test."""
    import oracle
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built")
    script = f"""
import ctypes, sys
import numpy as np
sys.path.insert(0, {str(ROOT)!r})
import oracle
from vx_amd import abi
from vx_amd.runtime import DispatchLibrary
ref = oracle.ref_lib()
lib = DispatchLibrary()
ctypes.CDLL({outlined._name!r}, mode=ctypes.RTLD_GLOBAL)
out = np.full((12, 2), -1, np.float32)
args = abi.CallArgs()
args.memref(abi.Descriptor(out.ctypes.data, out.shape), abi.DTYPE_F32)
lib.dispatch(abi.payload("vx_test_kernel_2", abi="1", launch="12"), args)
print(" ".join(str(int(v)) for v in out[:, 1]))
"""
    res = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                         timeout=120, env={**os.environ, "VX_HOST_THREADS": "3"})
    assert res.returncode == 0, res.stderr
    assert res.stdout.split() == ["3"] * 12, res.stdout


def test_matmul_without_a_gpu_runs_the_outlined_loop(cpulib, outlined):
    if gpu_present(cpulib):
        pytest.skip("a GPU is present: the GEMM would run there")
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.arange(12, dtype=np.float32).reshape(3, 4)
    c = np.zeros((2, 4), np.float32)
    args = abi.CallArgs()
    args.memref(abi.Descriptor(a.ctypes.data, a.shape), abi.DTYPE_F32).scalar(0, abi.KIND_I64)
    args.memref(abi.Descriptor(b.ctypes.data, b.shape), abi.DTYPE_F32).scalar(1, abi.KIND_I64)
    args.scalar(0.0, abi.KIND_F32).memref(abi.Descriptor(c.ctypes.data, c.shape), abi.DTYPE_F32)
    cpulib.dispatch(abi.matmul_payload(name="vx_test_kernel_1"), args)
    assert np.array_equal(c, a @ b)


def test_a_newer_payload_format_is_refused(cpulib, outlined):
    """abi= above what the library reads stops the program (a value it
    misreads is worse than a key it ignores)."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "from vx_amd.runtime import DispatchLibrary\nfrom vx_amd import abi\n"
        "lib = DispatchLibrary()\n"
        "lib.dispatch(abi.payload('vx_test_kernel_0', abi='2'), abi.CallArgs())\n" % str(ROOT))
    res = subprocess.run(["python", "-c", code], capture_output=True, text=True)
    assert res.returncode != 0 and "abi=2" in res.stderr
