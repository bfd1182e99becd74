"""CPU-side checks of bench.py's contract: one GPU only (--gpus N > 1 exits
with a message), the measured traffic it reads from profiles/, the spread
of timed regions it reports, and both CPU-baseline legs (the reference
library built from its sources, and the oracle restatement) on a small
matrix."""

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import bench
import oracle
from vx_amd.abi import f32_to_bf16

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""


def test_traffic_figures_come_from_the_committed_profiles():
    gemm = bench.traffic_from_profiles("gemm_bf16_4096")
    fa = bench.traffic_from_profiles("fa_causal_4x32x2048x128")
    dec = bench.traffic_from_profiles("decode_i8", "bytes_per_position")
    # HBM bytes per launch at least the algorithmic bytes (GEMM: A + B read,
    # C written; attention: Q, K, V read, O and LSE written)
    assert isinstance(gemm, int) and gemm >= 2 * 4096 * 4096 * 2 + 4096 * 4096 * 4
    assert isinstance(fa, int) and fa >= 269_000_000
    assert isinstance(dec, int) and dec >= 110_000_000
    assert bench.traffic_from_profiles("no_such_kernel") is None
    gemv = bench.gemv_traffic_from_profiles()
    assert sorted(gemv) == sorted(f"{r}x{c}_b{b}" for r, c in
                                  ((4096, 4096), (11008, 4096), (4096, 11008))
                                  for b in (1, 4, 16))
    for key, v in gemv.items():
        rows, cols = map(int, key.split("_")[0].split("x"))
        assert v >= rows * cols  # every weight byte is read


def test_spread_keeps_every_region():
    s = bench.spread([3.0, 1.0, 2.0, 10.0])
    assert s == dict(median=2.5, min=1.0, max=10.0, n=4)


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
def test_reference_cpu_baseline_leg():
    rng = np.random.default_rng(0)
    a16 = f32_to_bf16(rng.normal(0, 1 / 8, (64, 64)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 8, (64, 64)).astype(np.float32))
    want = oracle.gemm_bf16_f32(a16, b16)
    r = bench.cpu_baseline_ref_gemm(a16, b16, budget_s=0.05, gpu_rows=want[:8])
    assert r["kind"] == "reference" and r["cores"] == 1 and r["unit"] == "TFLOP/s"
    assert r["value"] > 0 and "oracle/_ref" in r["sample"]
    assert r["rows_vs_gpu"]["rows"] == 8 and r["rows_vs_gpu"]["within"]
    off = want[:8].copy()
    off[7, 63] += 2e-4  # a wrong element in the last compared row is seen
    r = bench.cpu_baseline_ref_gemm(a16, b16, budget_s=0.05, gpu_rows=off)
    assert not r["rows_vs_gpu"]["within"] and r["rows_vs_gpu"]["max_abs_diff"] >= 1.9e-4


def test_port_cpu_baseline_leg():
    rng = np.random.default_rng(0)
    a16 = f32_to_bf16(rng.normal(0, 1 / 8, (64, 64)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 8, (64, 64)).astype(np.float32))
    want = oracle.gemm_bf16_f32(a16, b16)
    r = bench.cpu_baseline_gemm(a16[:, :32], b16[:32], budget_s=0.05, gpu_rows=None)
    assert r["kind"] == "port" and r["cores"] == 1 and r["value"] > 0
    assert "64x64x32" in r["sample"] and "rows_vs_gpu" not in r
    r = bench.cpu_baseline_gemm(a16, b16, budget_s=0.05, gpu_rows=want[:64])
    assert r["rows_vs_gpu"]["within"] and r["rows_vs_gpu"]["max_abs_diff"] == 0.0
