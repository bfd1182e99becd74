"""Builds and runs the GPU-free C++ unit tests of the vendor-free headers
(tests/native/*.cpp), as the reference's runtime tests are built and run
(reference tests/integration_test/runtime_test_build.rs: -Wall -Werror, and
ASan/UBSan on request), and also under ThreadSanitizer: the host fallback's
worker split and the staging pool run on several threads. The host-fallback
test calls through libffi, so every test is linked with the image's libffi,
as the dispatch library is."""

import os
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
NATIVE = HERE / "native"
FFI_INC = Path("/opt/conda/include")
FFI_LIB = Path("/usr/lib/x86_64-linux-gnu/libffi.so.8")


@pytest.mark.parametrize("src", sorted(p.name for p in NATIVE.glob("*_test.cpp")))
@pytest.mark.parametrize("sanitize", [None, "address,undefined", "thread"])
def test_native(src, sanitize, tmp_path):
    exe = tmp_path / src.replace(".cpp", "")
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{FFI_INC}", str(NATIVE / src),
           "-o", str(exe), str(FFI_LIB), "-ldl", "-lpthread"]
    if sanitize:
        cmd[1:1] = [f"-fsanitize={sanitize}", "-fno-omit-frame-pointer"]
    subprocess.run(cmd, check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    assert res.stdout.strip() == "ok"
