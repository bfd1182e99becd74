"""Build libvx_hip_dispatch.so for gfx950, in-tree.

Every source under vx_amd/csrc is compiled with hipcc for gfx950 and linked
into vx_amd/libvx_hip_dispatch.so, next to this file, so the library travels
with the tree. libffi (the host fallback's call mechanism, as in the
reference's dispatch libraries) comes from the image.

    python -m vx_amd.build            # build (always recompiles)
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libvx_hip_dispatch.so"

ARCH = "gfx950"
FFI_INC = Path("/opt/conda/include")
FFI_LIB = Path("/usr/lib/x86_64-linux-gnu/libffi.so.8")

# -packed-fp32-ops off: hipcc would otherwise form v_pk_{add,mul,fma}_f32 from
# ordinary float code.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.cpp")) + sorted((CSRC / "kernels").glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / f"{src.parent.name}_{src.stem}.o"
    cmd = [hipcc(), *HIP_FLAGS, f"-I{FFI_INC}", "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in res.stderr.splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile and link the dispatch library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-shared",
        "-fPIC",
        "-o",
        str(tmp),
        *map(str, objs),
        str(FFI_LIB),
        "-ldl",
        "-lpthread",
        f"-Wl,--version-script={CSRC / 'exports.map'}",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking {LIB.name} failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


TEST_IMAGES = ROOT / "tests" / "images"


def build_test_images(verbose: bool = False) -> list[Path]:
    """Code objects for the payload-image tests: each tests/images/*.hip as a
    bare gfx950 ELF (<name>.hsaco) and as a clang offload bundle
    (<name>.bundle.hsaco). Contraction off, so each kernel's f32 arithmetic
    rounds once per operation, as numpy does."""
    out = []
    for src in sorted(TEST_IMAGES.glob("*.hip")):
        for bundle in (False, True):
            dst = src.with_suffix(".bundle.hsaco" if bundle else ".hsaco")
            cmd = [hipcc(), "--genco", f"--offload-arch={ARCH}", "-O3", "-std=c++17",
                   "-ffp-contract=off",
                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                   *([] if bundle else ["--no-gpu-bundle-output"]), str(src), "-o", str(dst)]
            if verbose:
                print(" ".join(cmd), flush=True)
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"compiling {src.name} failed:\n{res.stderr}")
            out.append(dst)
    return out


PROBES = PKG / "probes"


def build_probes(verbose: bool = False) -> list[Path]:
    """Measurement kernels that are not part of the library (the HBM read
    ceiling bench.py reports): each vx_amd/probes/*.hip as a bare gfx950 code
    object next to its source."""
    out = []
    for src in sorted(PROBES.glob("*.hip")):
        dst = src.with_suffix(".hsaco")
        cmd = [hipcc(), "--genco", f"--offload-arch={ARCH}", "-O3", "-std=c++17",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "--no-gpu-bundle-output", str(src), "-o", str(dst)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"compiling {src.name} failed:\n{res.stderr}")
        out.append(dst)
    return out


def build_oracle(verbose: bool = False) -> None:
    """The CPU checker (oracle/liboracle.so) and, where the reference checkout
    exists, oracle/_ref/libvx_x86_dispatch.so built from its sources."""
    res = subprocess.run(["make", "-C", str(ROOT / "oracle"), "-B"], capture_output=True, text=True)
    if verbose:
        print(res.stdout)
    if res.returncode != 0:
        raise RuntimeError(f"building oracle/ failed:\n{res.stdout}\n{res.stderr}")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    build_test_images(verbose="-v" in sys.argv)
    build_probes(verbose="-v" in sys.argv)
    build_oracle(verbose="-v" in sys.argv)
