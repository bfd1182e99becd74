#!/usr/bin/env python3
"""Benchmark of the MI355X dispatch library on BASELINE.json's metric.

One step = one `c = a @ b` dispatch of BASELINE config 2 (bf16 x bf16 -> f32,
M = N = K = 4096, N(0, 1/64) inputs resident in HBM, result into an HBM
buffer) through vx_plugin_dispatch_async, exactly as a compiled Vx program
issues it. `value` is whole-job TFLOP/s over the K timed steps.

The same JSON line carries:
  - roofline: the GEMM kernel's algorithmic FLOPs over its average duration
    (hipEvents on the launch stream over the timed region) against the
    MI355X dense bf16 MFMA peak, and its HBM traffic per launch from the
    committed rocprofv3 PMC summary when one exists;
  - cpu_baseline: the reference's CPU path for the same GEMM, one thread,
    timed on a bounded block of rows: its x86 dispatch library built here
    from its sources (oracle/_ref, kind "reference"), or where that was not
    built the CPU oracle's restatement of it (kind "port");
  - extra: flash-attention forward (config 3), int8 GEMV (config 5, weights
    rotated through more than the 256 MB MALL), int8 greedy decode
    (config 4), the 8192^3 GEMM roofline point and the f32 512^3 plumbing
    GEMM (config 1, with its parity against the oracle); with the CPU leg,
    the oracle's own rate beside each of them on a bounded sample.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--only gemm,fa,gemv,decode]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_CLOCK_MHZ = 2400.0    # the clock the bf16 peak is quoted at


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_from_profiles(name: str, key: str = "bytes_per_launch"):
    """HBM bytes per launch (or per decode position) measured with rocprofv3
    PMC counters, committed as profiles/<name>_traffic.json; None when not
    measured."""
    p = ROOT / "profiles" / f"{name}_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get(key)
        except (ValueError, OSError):
            return None
    return None


def gemv_traffic_from_profiles() -> dict:
    """HBM bytes per GEMV launch keyed "<rows>x<cols>_b<batch>", from
    profiles/gemv_i8_traffic.json (rocprofv3 PMC counters); empty when not
    measured."""
    p = ROOT / "profiles" / "gemv_i8_traffic.json"
    try:
        cases = json.loads(p.read_text())["cases"]
        return {k: v["bytes_per_launch"] for k, v in cases.items()}
    except (ValueError, OSError, KeyError, TypeError):
        return {}


SETTLE_MS = 200.0  # untimed GPU work before each kernel's warmup steps


def spread(xs) -> dict:
    """Median, fastest and slowest of a list of timings (every run kept in
    the summary, as the reference's benchmarking policy asks)."""
    xs = sorted(xs)
    return dict(median=round(float(np.median(xs)), 3), min=round(xs[0], 3),
                max=round(xs[-1], 3), n=len(xs))


def timed_runs(call, timer, steps: int, runs: int = 3, stream=None) -> list:
    """`runs` timed regions of `steps` calls each; the per-call milliseconds
    of each region (hipEvents on the launch stream)."""
    out = []
    for _ in range(runs):
        e0, e1 = timer.event(), timer.event()
        timer.record(e0, stream)
        for _ in range(steps):
            call()
        timer.record(e1, stream)
        out.append(timer.elapsed_ms(e0, e1) / steps)
    return out


def settle(call, timer, min_ms: float = SETTLE_MS) -> float:
    """Run `call` untimed until at least `min_ms` of GPU time has passed, so
    the timed steps see the clocks a sustained workload runs at (a cold GPU
    measures up to a quarter slower on the first milliseconds). Returns the
    GPU milliseconds spent."""
    spent = 0.0
    while spent < min_ms:
        e0, e1 = timer.event(), timer.event()
        timer.record(e0)
        for _ in range(10):
            call()
        timer.record(e1)
        spent += timer.elapsed_ms(e0, e1)
    return spent


def bench_gemm(lib, timer, steps: int, warmup: int, n: int = 4096, m: int | None = None,
               k: int | None = None, runs: int = 3):
    """C[m, n] = A[m, k] B[k, n] (m = k = n unless given), bf16 in, f32
    out, through vx_plugin_dispatch_async. `runs` timed regions of `steps`
    dispatches each (hipEvents around each region); the rate is the median
    region's, and every region is kept in `runs_us` (per-step median, fastest
    and slowest region)."""
    from vx_amd import abi
    from vx_amd.abi import f32_to_bf16
    from vx_amd.runtime import DeviceArray, matmul

    m = n if m is None else m
    k = n if k is None else k
    rng = np.random.default_rng(2024)
    a16 = f32_to_bf16(rng.normal(0, 1 / 64, (m, k)).astype(np.float32))
    b16 = f32_to_bf16(rng.normal(0, 1 / 64, (k, n)).astype(np.float32))
    da, db = DeviceArray.of(lib, a16, abi.DTYPE_BF16), DeviceArray.of(lib, b16, abi.DTYPE_BF16)
    dc = DeviceArray(lib, (m, n), abi.DTYPE_F32)
    ad, bd, cd = da.descriptor(), db.descriptor(), dc.descriptor()
    args = abi.CallArgs()
    args.memref(ad, abi.DTYPE_BF16).scalar(0, abi.KIND_I64).memref(bd, abi.DTYPE_BF16)
    args.scalar(1, abi.KIND_I64).scalar(0.0, abi.KIND_F32).memref(cd, abi.DTYPE_F32)
    import ctypes
    pl = abi.matmul_payload(outkind="buffer")
    buf = ctypes.create_string_buffer(pl, len(pl))
    argv, tags, nargs = args.arrays()
    dispatch = lib.lib.vx_plugin_dispatch_async

    before = lib.stats()
    sk_before = lib.gemm_workspaces()["launches"]
    settled = [0]

    def one():
        dispatch(buf, len(pl), argv, tags, nargs)
        settled[0] += 1

    settle(one, timer)
    for _ in range(warmup):
        dispatch(buf, len(pl), argv, tags, nargs)
    timer.sync()
    # Clock stamps of the timed launches (workgroup 0's shader-clock and
    # 100 MHz real-time counters at its start and end), one slot per step.
    stamps = lib.transfer(None, 32 * steps * runs)
    lib.clock_stamps(stamps, steps * runs)
    region_ms = []
    t0 = time.perf_counter()
    for _ in range(runs):
        e0, e1 = timer.event(), timer.event()
        timer.record(e0)
        for i in range(steps):
            dispatch(buf, len(pl), argv, tags, nargs)
        timer.record(e1)
        region_ms.append(timer.elapsed_ms(e0, e1))
    timer.sync()
    wall = time.perf_counter() - t0
    ms_events = float(np.median(region_ms))
    lib.clock_stamps(None, 0)
    # The spread: the same steps again, each bracketed by its own events (an
    # event between two launches can delay the second, so these do not
    # enter `ms_per_step`).
    events = [timer.event() for _ in range(steps + 1)]
    timer.record(events[0])
    for i in range(steps):
        dispatch(buf, len(pl), argv, tags, nargs)
        timer.record(events[i + 1])
    timer.sync()
    step_ms = [timer.elapsed_ms(events[i], events[i + 1]) for i in range(steps)]
    st = np.empty((steps * runs, 4), np.uint64)
    lib.fetch(stamps, st)
    lib.free(stamps)
    clk = (st[:, 2] - st[:, 0]).astype(np.float64)
    rt = (st[:, 3] - st[:, 1]).astype(np.float64)
    clock_mhz = float(clk.sum() / rt.sum() * 100.0) if rt.sum() > 0 else None
    after = lib.stats()
    total = (runs + 1) * steps + warmup + settled[0]
    assert after["gemm_mfma"] - before["gemm_mfma"] == total, "GEMM did not take the MFMA path"
    # Which launch ran: the stream-K one (one workgroup per CU, second-round
    # tiles cut along K) for grids ending in a partial round of at most half,
    # else one 256x256 tile per workgroup.
    sk = lib.gemm_workspaces()["launches"] - sk_before
    assert sk in (0, total), "the launch kind changed between dispatches"
    launch = "stream-K" if sk else "one tile per workgroup"
    c = dc.numpy()
    assert np.isfinite(c).all()
    for x in (da, db, dc):
        x.free()
    flops = 2.0 * m * n * k
    ms_step = ms_events / steps
    return dict(n=n, m=m, k=k, ms_per_step=ms_step, wall_ms_per_step=wall * 1e3 / (steps * runs),
                tflops=flops / (ms_step * 1e-3) / 1e12, flops=flops, a16=a16, b16=b16,
                c_head=np.ascontiguousarray(c[:64]),
                runs_us=spread([x * 1e3 / steps for x in region_ms]),
                tflops_runs=spread([flops / (x / steps * 1e-3) / 1e12 for x in region_ms]),
                steps_us=spread([x * 1e3 for x in step_ms]), clock_mhz=clock_mhz,
                launch=launch)


def bench_gemm_f32(lib, timer, steps: int = 50, n: int = 512):
    """BASELINE config 1 (the plumbing GEMM): f32 512^3, U[-1,1] operands,
    through the ABI onto the exact-order tiled kernel. Reports the device
    time per dispatch (hipEvents), the host wall time per dispatch, and the
    largest relative error against the CPU oracle (the reference's loop)."""
    import ctypes

    import oracle
    from vx_amd import abi
    from vx_amd.runtime import DeviceArray

    a = np.random.default_rng(1).uniform(-1, 1, (n, n)).astype(np.float32)
    b = np.random.default_rng(2).uniform(-1, 1, (n, n)).astype(np.float32)
    da, db = DeviceArray.of(lib, a, abi.DTYPE_F32), DeviceArray.of(lib, b, abi.DTYPE_F32)
    dc = DeviceArray(lib, (n, n), abi.DTYPE_F32)
    args = abi.CallArgs()
    args.memref(da.descriptor(), abi.DTYPE_F32).scalar(0, abi.KIND_I64)
    args.memref(db.descriptor(), abi.DTYPE_F32).scalar(1, abi.KIND_I64)
    args.scalar(0.0, abi.KIND_F32).memref(dc.descriptor(), abi.DTYPE_F32)
    pl = abi.matmul_payload(outkind="buffer")
    buf = ctypes.create_string_buffer(pl, len(pl))
    argv, tags, nargs = args.arrays()
    dispatch = lib.lib.vx_plugin_dispatch_async

    def one():
        dispatch(buf, len(pl), argv, tags, nargs)

    settle(one, timer, 50.0)
    timer.sync()
    e0, e1 = timer.event(), timer.event()
    t0 = time.perf_counter()
    timer.record(e0)
    for _ in range(steps):
        one()
    timer.record(e1)
    ms = timer.elapsed_ms(e0, e1) / steps
    timer.sync()
    wall_us = (time.perf_counter() - t0) / steps * 1e6
    c = dc.numpy()
    for x in (da, db, dc):
        x.free()
    t0 = time.perf_counter()
    want = oracle.gemm_f32(a, b)
    cpu_s = time.perf_counter() - t0
    rel = float(np.max(np.abs(c - want) / np.maximum(1.0, np.abs(want))))
    flops = 2.0 * n ** 3
    return dict(config=f"f32 {n}^3, U[-1,1] seeds 1/2 (BASELINE config 1)", us=ms * 1e3,
                wall_us_per_dispatch=wall_us, tflops=flops / (ms * 1e-3) / 1e12,
                max_rel_err_vs_oracle=rel, parity_bound=1e-4,
                cpu=dict(value=flops / cpu_s / 1e12, unit="TFLOP/s", cores=1, kind="port",
                         sample=f"the whole {n}^3 GEMM, oracle/vx_oracle.c loop nest"))


def cpu_fa(rows: int = 96):
    """The CPU oracle's attention on `rows` query rows spread over config 3
    (one thread); TFLOP/s over the exact causal work of those rows."""
    import oracle
    from vx_amd.abi import f32_to_bf16

    b, h, s, d = 4, 32, 2048, 128
    rng = np.random.default_rng(7)
    q, k, v = (f32_to_bf16(rng.standard_normal((b, h, s, d)).astype(np.float32)) for _ in range(3))
    pick = np.random.default_rng(3)
    sel = np.stack([pick.integers(0, b, rows), pick.integers(0, h, rows), pick.integers(0, s, rows)],
                   axis=1).astype(np.int64)
    t0 = time.perf_counter()
    oracle.attention_rows(q, k, v, h, h, 1.0 / np.sqrt(d), True, sel)
    dt = time.perf_counter() - t0
    flops = float(np.sum(4.0 * d * (sel[:, 2] + 1)))
    return dict(value=flops / dt / 1e12, unit="TFLOP/s", cores=1, kind="port",
                sample=f"{rows} random query rows of causal [4,32,2048,128] ({flops / 1e9:.2f} GFLOP "
                       f"in {dt:.2f} s), oracle/vx_oracle.c")


def cpu_gemv(rows: int = 11008, cols: int = 4096):
    import oracle
    from vx_amd.abi import f32_to_bf16

    rng = np.random.default_rng(11)
    w = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    sc = rng.uniform(0.001, 0.01, rows).astype(np.float32)
    x = f32_to_bf16(rng.standard_normal((1, cols)).astype(np.float32))
    t0 = time.perf_counter()
    oracle.gemv_i8(w, sc, x)
    dt = time.perf_counter() - t0
    return dict(value=rows * cols / dt / 1e9, unit="GB/s (weight bytes)", cores=1, kind="port",
                sample=f"{rows}x{cols} batch 1, oracle/vx_oracle.c")


def cpu_decode(n_steps: int = 8):
    import oracle
    from vx_amd.llama import CONFIG_DECODE, make_model, make_prompt

    cfg = CONFIG_DECODE
    model = make_model(cfg, seed=0)
    prompt = make_prompt(cfg, n=16, seed=1)
    t0 = time.perf_counter()
    oracle.llama_generate(cfg.as_dict(), model, prompt, n_steps)
    dt = time.perf_counter() - t0
    positions = len(prompt) + n_steps - 1
    return dict(value=positions / dt, unit="positions/s (= tok/s once past the prompt)", cores=1,
                kind="port", sample=f"16-token prompt + {n_steps} greedy tokens of config 4 "
                                    f"({positions} positions in {dt:.1f} s), oracle/vx_oracle.c")


def bench_fa(lib, timer, steps: int, warmup: int):
    from vx_amd import abi
    from vx_amd.abi import f32_to_bf16
    from vx_amd.runtime import DeviceArray, flash_attention_fwd

    b, h, s, d = 4, 32, 2048, 128
    rng = np.random.default_rng(7)
    arrs = [DeviceArray.of(lib, f32_to_bf16(rng.standard_normal((b, h, s, d)).astype(np.float32)),
                           abi.DTYPE_BF16) for _ in range(3)]
    do = DeviceArray(lib, (b, h, s, d), abi.DTYPE_BF16)
    dl = DeviceArray(lib, (b, h, s), abi.DTYPE_F32)
    q, k, v = (x.ptr for x in arrs)

    def call():
        rc = flash_attention_fwd(lib, q, k, v, do.ptr, dl.ptr, b, h, h, s, s, d, 1.0 / np.sqrt(d), True)
        assert rc == 0

    settle(call, timer)
    for _ in range(warmup):
        call()
    timer.sync()
    runs = timed_runs(call, timer, steps)
    ms = float(np.median(runs))
    for x in arrs + [do, dl]:
        x.free()
    flops = 2.0 * b * h * s * s * d  # causal: half of 4*B*H*S^2*D
    tflops = flops / (ms * 1e-3) / 1e12
    return dict(config="causal [4,32,2048,128] bf16", ms=ms, tflops=tflops,
                frac_of_peak=tflops / PEAK_BF16_TFLOPS,
                runs_us=spread([x * 1e3 for x in runs]), steps_per_run=steps,
                roofline={"bound": "mfma", "achieved": round(tflops, 2),
                          "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                          "traffic": traffic_from_profiles("fa_causal_4x32x2048x128")})


def bench_fa_chunks(lib, timer, steps: int = 20):
    """The reference's own flash-attention benchmark shape (reference
    benchmarks/apple_gpu_mlir_kernels/README.md:30-37): a 512-token causal
    prefill chunk at position 0, 1536 and 7680, 32 query heads over 4 KV
    heads, head_dim 128, bf16 (the reference's kernel reads f16 K/V on an
    Apple M4, 1.26 / 7.6 / 33.6 ms: context, not a target). Microseconds per
    call and TFLOP/s over the causal work."""
    from vx_amd import abi
    from vx_amd.abi import f32_to_bf16
    from vx_amd.runtime import DeviceArray, flash_attention_fwd

    out = {}
    rng = np.random.default_rng(9)
    b, h, hk, sq, d = 1, 32, 4, 512, 128
    for start in (0, 1536, 7680):
        sk = start + sq
        q = DeviceArray.of(lib, f32_to_bf16(rng.standard_normal((b, h, sq, d)).astype(np.float32)),
                           abi.DTYPE_BF16)
        k = DeviceArray.of(lib, f32_to_bf16(rng.standard_normal((b, hk, sk, d)).astype(np.float32)),
                           abi.DTYPE_BF16)
        v = DeviceArray.of(lib, f32_to_bf16(rng.standard_normal((b, hk, sk, d)).astype(np.float32)),
                           abi.DTYPE_BF16)
        o = DeviceArray(lib, (b, h, sq, d), abi.DTYPE_BF16)
        lse = DeviceArray(lib, (b, h, sq), abi.DTYPE_F32)

        def call():
            assert flash_attention_fwd(lib, q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, b, h, hk, sq, sk,
                                       d, 1.0 / np.sqrt(d), True) == 0

        # query i sees start + i + 1 keys
        flops = 4.0 * b * h * d * float(np.sum(start + np.arange(sq) + 1))
        row = {}
        # the library's own choice (these 128 query blocks get a key split),
        # then the same call forced unsplit
        for key, splits in (("", 0), ("unsplit_", 1)):
            lib.force_fa_splits(splits)
            try:
                for _ in range(3):
                    call()
                timer.sync()
                runs = timed_runs(call, timer, steps)
            finally:
                lib.force_fa_splits(0)
            us = float(np.median(runs)) * 1e3
            row[key + "us"] = round(us, 2)
            row[key + "tflops"] = round(flops / (us * 1e-6) / 1e12, 1)
            row[key + "runs_us"] = spread([x * 1e3 for x in runs])
        out[str(start)] = row
        for x in (q, k, v, o, lse):
            x.free()
    return out


def bench_gemv(lib, timer, steps: int, warmup: int):
    """BASELINE config 5 through vx_nn_gemv_i8_bf16. Each shape rotates
    through enough weight copies to exceed twice the 256 MB MALL, so every
    call streams its weights from HBM. `us` is the per-call time of a
    hipGraph replay of the calls (the kernels back to back, as in a captured
    decode step); `us_eager` the per-call time of the same calls made one by
    one from Python, which adds the host's launch cost where that is the
    longer of the two."""
    from vx_amd import abi
    from vx_amd.abi import f32_to_bf16
    from vx_amd.runtime import DeviceArray, gemv_i8

    out = []
    gemv_traffic = gemv_traffic_from_profiles()
    rng = np.random.default_rng(11)
    stream = timer.stream_create()
    lib.lib.vx_hip_set_stream(stream)
    try:
        for rows, cols in ((4096, 4096), (11008, 4096), (4096, 11008)):
            wbytes = rows * cols
            copies = max(6, -(-512 * 2**20 // wbytes))  # > 2x the 256 MB MALL
            w = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
            ws = [DeviceArray.of(lib, w, abi.DTYPE_I8) for _ in range(copies)]
            sc = DeviceArray.of(lib, rng.uniform(0.001, 0.01, rows).astype(np.float32),
                                abi.DTYPE_F32)
            for batch in (1, 4, 16):
                x = DeviceArray.of(lib, f32_to_bf16(rng.standard_normal((batch, cols))
                                                    .astype(np.float32)), abi.DTYPE_BF16)
                y = DeviceArray(lib, (batch, rows), abi.DTYPE_F32)
                n_calls = max(steps, copies)

                def calls():
                    for i in range(n_calls):
                        rc = gemv_i8(lib, ws[i % copies].ptr, sc.ptr, x.ptr, y.ptr, rows,
                                     cols, batch)
                        assert rc == 0

                for i in range(warmup):
                    gemv_i8(lib, ws[i % copies].ptr, sc.ptr, x.ptr, y.ptr, rows, cols, batch)
                timer.sync()
                e0, e1 = timer.event(), timer.event()
                timer.record(e0, stream)
                calls()
                timer.record(e1, stream)
                us_eager = timer.elapsed_ms(e0, e1) / n_calls * 1e3
                graph = timer.capture(stream, calls)
                timer.graph_launch(graph, stream)  # warm
                reps = 4
                ev = [timer.event() for _ in range(reps + 1)]
                timer.record(ev[0], stream)
                for r in range(reps):
                    timer.graph_launch(graph, stream)
                    timer.record(ev[r + 1], stream)
                us = timer.elapsed_ms(ev[0], ev[-1]) / (reps * n_calls) * 1e3
                per_rep = [timer.elapsed_ms(ev[r], ev[r + 1]) / n_calls * 1e3 for r in range(reps)]
                timer.graph_destroy(graph)
                nbytes = rows * cols + 4 * rows + 2 * batch * cols + 4 * batch * rows
                gbs = nbytes / (us * 1e-6) / 1e9
                out.append(dict(shape=[rows, cols], batch=batch, us=us, gbs=gbs,
                                frac_of_hbm=gbs / PEAK_HBM_GBS, us_eager=us_eager,
                                runs_us=spread(per_rep), rotated_copies=copies,
                                roofline={"bound": "hbm", "achieved": round(gbs, 1),
                                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                          "frac": round(gbs / PEAK_HBM_GBS, 4),
                                          "traffic": gemv_traffic.get(f"{rows}x{cols}_b{batch}")}))
                x.free()
                y.free()
            for a in ws + [sc]:
                a.free()
    finally:
        timer.sync()
        lib.lib.vx_hip_set_stream(None)
        timer.stream_destroy(stream)
    return out


def cpu_baseline_ref_gemm(a16, b16, budget_s: float = 10.0, gpu_rows=None):
    """The reference's own CPU path on a block of rows of the same GEMM
    (the headline 4096^3 one, and the 8192^3 one in extra): its x86 dispatch library (reference runtime/x86_dispatch.cpp, built
    from its sources into oracle/_ref by oracle/Makefile) driven through the
    plugin ABI as a compiled `c = a @ b` drives it, on the bf16 operands
    extended to f32 (the arithmetic of its bf16 -> f32 route: extend, f32
    multiply-add in k order; tests/test_oracle.py pins the two bit-equal).
    One thread: the reference's matmul route runs on the dispatching thread
    (reference runtime/host_dispatch_common.h:616-623). With `gpu_rows`
    (the first rows of the GPU's C), the rows both computed are compared."""
    import oracle
    from vx_amd import abi
    from vx_amd.abi import bf16_to_f32
    from vx_amd.runtime import matmul

    lib = oracle.ref_lib()
    a = np.ascontiguousarray(bf16_to_f32(a16), np.float32)
    b = np.ascontiguousarray(bf16_to_f32(b16), np.float32)
    n, k = a.shape
    bd = abi.Descriptor(b.ctypes.data, b.shape)

    def run(rows: int):
        c = np.empty((rows, b.shape[1]), np.float32)
        t0 = time.perf_counter()
        matmul(lib, abi.Descriptor(a.ctypes.data, (rows, k)), abi.DTYPE_F32, bd, abi.DTYPE_F32,
               abi.Descriptor(c.ctypes.data, c.shape), abi.DTYPE_F32, outkind="buffer",
               topo=abi.TOPO_CPU)
        dt = time.perf_counter() - t0
        assert np.isfinite(c).all()
        return dt, c

    per_row = run(2)[0] / 2
    rows = int(max(2, min(n, budget_s / max(per_row, 1e-6))))
    dt, c = run(rows)
    flops = 2.0 * rows * k * b.shape[1]
    out = dict(value=flops / dt / 1e12, unit="TFLOP/s", cores=1, kind="reference",
               sample=f"rows 0..{rows} of the {n}x{b.shape[1]}x{k} GEMM ({flops / 1e9:.1f} GFLOP "
                      f"in {dt:.1f} s) through the reference x86 dispatch library (oracle/_ref), "
                      f"f32 on the bf16 operands extended, 1 thread")
    return _rows_vs_gpu(out, c, gpu_rows)


def _rows_vs_gpu(out: dict, cpu_rows, gpu_rows) -> dict:
    """Adds the comparison of the CPU leg's rows with the GPU's first rows
    of the same C (the largest absolute difference, against the 1e-4 the
    GEMM parity tests hold)."""
    if gpu_rows is not None:
        r = min(len(cpu_rows), len(gpu_rows))
        d = float(np.abs(cpu_rows[:r].astype(np.float64) - gpu_rows[:r]).max())
        out["rows_vs_gpu"] = dict(rows=r, max_abs_diff=d, bound=1e-4, within=d <= 1e-4)
    return out


def cpu_baseline_gemm(a16, b16, budget_s: float = 10.0, gpu_rows=None):
    """The CPU oracle's bf16 -> f32 GEMM (one thread) on a block of rows of
    the same GEMM, sized to about `budget_s` of work; with `gpu_rows`, its
    rows compared with the GPU's."""
    import oracle

    m, k = a16.shape
    n = b16.shape[1]
    t0 = time.perf_counter()
    oracle.gemm_bf16_f32(a16, b16, rows=slice(0, 2))
    per_row = (time.perf_counter() - t0) / 2
    rows = int(max(2, min(m, budget_s / max(per_row, 1e-6))))
    t0 = time.perf_counter()
    c = oracle.gemm_bf16_f32(a16, b16, rows=slice(0, rows))
    dt = time.perf_counter() - t0
    flops = 2.0 * rows * k * n
    out = dict(value=flops / dt / 1e12, unit="TFLOP/s", cores=1, kind="port",
               sample=f"rows 0..{rows} of the {m}x{n}x{k} bf16->f32 GEMM ({flops / 1e9:.1f} GFLOP "
                      f"in {dt:.1f} s), oracle/vx_oracle.c loop nest, 1 thread")
    return _rows_vs_gpu(out, c[:rows], gpu_rows)


def read_ceiling(lib, timer, sizes) -> dict:
    """The measured HBM read ceiling beside the 8 TB/s nameplate: one
    dispatch of vx_amd/probes/read_probe.hip (each workgroup reads one
    contiguous burst, every load issued before any is used) over n bytes,
    for each size, at bursts of 16, 32 and 64 KiB per workgroup with plain
    and non-temporal loads; the fastest is the ceiling. Like the GEMV entries, each size rotates through
    enough buffers (over 1 GiB) that every dispatch streams from HBM rather
    than the 256 MB MALL, and is timed as hipGraph replays (four, per-call
    median) so the host's launch rate does not enter. GB/s counts the bytes
    read. `sizes` maps a name to a byte count (a multiple of 64 KiB)."""
    import ctypes

    hip = timer.hip
    vp = ctypes.c_void_p
    path = ROOT / "vx_amd" / "probes" / "read_probe.hsaco"
    if not path.exists():
        raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
    mod = vp()
    hip.hipModuleLoad.argtypes = [ctypes.POINTER(vp), ctypes.c_char_p]
    assert hip.hipModuleLoad(ctypes.byref(mod), str(path).encode()) == 0, "hipModuleLoad"
    hip.hipModuleGetFunction.argtypes = [ctypes.POINTER(vp), vp, ctypes.c_char_p]
    hip.hipModuleLaunchKernel.argtypes = [vp] + [ctypes.c_uint] * 7 + [vp, ctypes.POINTER(vp), vp]
    funcs = {}
    for units in (4, 8, 16):
        for aux in (0, 2):
            f = vp()
            assert hip.hipModuleGetFunction(ctypes.byref(f), mod,
                                            f"vx_read_probe_{units}_{aux}".encode()) == 0
            funcs[(units, aux)] = f
    stream = timer.stream_create()
    out = {}
    try:
        for name, nbytes in sizes.items():
            assert nbytes % (64 * 1024) == 0, name
            copies = max(4, -(-2**30 // nbytes))
            bufs = [lib.transfer(None, nbytes) for _ in range(copies)]
            sink = lib.transfer(None, nbytes // 4)  # the store a probe never makes
            best = None
            for (units, aux), f in funcs.items():
                grid = nbytes // (256 * units * 16)
                params = [(vp(b), vp(sink)) for b in bufs]
                arrays = [(ctypes.c_void_p * 2)(ctypes.addressof(a), ctypes.addressof(o))
                          for a, o in params]

                def calls():
                    for arr in arrays:
                        rc = hip.hipModuleLaunchKernel(f, grid, 1, 1, 256, 1, 1, 0, stream,
                                                       ctypes.cast(arr, ctypes.POINTER(vp)), None)
                        assert rc == 0, f"hipModuleLaunchKernel failed with {rc}"

                graph = timer.capture(stream, calls)
                timer.graph_launch(graph, stream)  # warm
                reps = 4
                ev = [timer.event() for _ in range(reps + 1)]
                timer.record(ev[0], stream)
                for r in range(reps):
                    timer.graph_launch(graph, stream)
                    timer.record(ev[r + 1], stream)
                per_rep = [timer.elapsed_ms(ev[r], ev[r + 1]) / copies * 1e3 for r in range(reps)]
                timer.graph_destroy(graph)
                us = float(np.median(per_rep))
                row = dict(bytes=nbytes, burst_kib=units * 4, nontemporal=aux == 2, us=round(us, 3),
                           gbs=round(nbytes / (us * 1e-6) / 1e9, 1), runs_us=spread(per_rep),
                           rotated_copies=copies)
                if best is None or row["us"] < best["us"]:
                    best = row
            out[name] = best
            for b in bufs + [sink]:
                lib.free(b)
    finally:
        timer.sync()
        timer.stream_destroy(stream)
        hip.hipModuleUnload.argtypes = [vp]
        hip.hipModuleUnload(mod)
    return out


def copy_probe() -> int:
    """A plain copy of known size: 256 MiB read and 256 MiB written per
    launch, three launches."""
    from vx_amd.runtime import DispatchLibrary, HipTimer

    lib = DispatchLibrary()
    timer = HipTimer()
    nbytes = 256 * 2**20
    src = lib.transfer(np.ones(nbytes // 4, np.float32))
    for _ in range(3):
        dst = lib.lib.vx_plugin_transfer_peer(src, 500, 500, nbytes)
        timer.sync()
        lib.free(dst)
    lib.free(src)
    log(f"copied {nbytes} bytes device to device 3 times")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", default="gemm,fa,gemv,decode")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 256 MiB device to device through vx_plugin_transfer_peer, "
                         "three times: the reference launch for scaling rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE readings to bytes")
    ns = ap.parse_args()
    if ns.copy_probe:
        return copy_probe()
    if ns.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (how it would "
              "shard is a design only). Run with --gpus 1.", file=sys.stderr)
        return 2
    only = set(ns.only.split(","))

    from vx_amd.runtime import DispatchLibrary, HipTimer

    lib = DispatchLibrary()
    if lib.device_count() < 1:
        print("no GPU visible", file=sys.stderr)
        return 1
    timer = HipTimer()

    log(f"gemm bf16->f32 4096^3: warmup {ns.warmup}, steps {ns.steps}")
    g = bench_gemm(lib, timer, ns.steps, ns.warmup)
    log(f"gemm {g['tflops']:.1f} TFLOP/s ({g['ms_per_step'] * 1e3:.1f} us/step, clock "
        f"{g['clock_mhz'] or 0:.0f} MHz)")

    extra = {}
    if "fa" in only:
        log("flash attention config 3")
        extra["flash_attn_fwd"] = bench_fa(lib, timer, max(10, ns.steps // 2), 3)
        extra["flash_attn_prefill_chunks"] = bench_fa_chunks(lib, timer)
        log(f"fa {extra['flash_attn_fwd']['tflops']:.1f} TFLOP/s")
    if "gemv" in only:
        log("int8 gemv config 5")
        extra["gemv_i8"] = bench_gemv(lib, timer, max(20, ns.steps), 3)
        # what one dispatch reading each shape's weight bytes reaches on this
        # box (the single-dispatch burst read), beside the nameplate
        ceil = read_ceiling(lib, timer, {"4096x4096": 4096 * 4096, "11008x4096": 11008 * 4096,
                                         "256MiB": 256 * 2**20})
        extra["hbm_read_ceiling"] = ceil
        for r in extra["gemv_i8"]:
            # 11008x4096 and 4096x11008 stream the same 45.1 MB of weights;
            # the ceiling reads the weight bytes alone
            c = ceil["4096x4096" if r["shape"] == [4096, 4096] else "11008x4096"]
            r["roofline"]["read_ceiling_us"] = c["us"]
            r["roofline"]["read_ceiling_gbs"] = c["gbs"]
            r["roofline"]["frac_of_read_ceiling"] = round(c["us"] / r["us"], 4)
        b1 = {tuple(r["shape"]): r["us"] for r in extra["gemv_i8"] if r["batch"] == 1}
        for r in extra["gemv_i8"]:
            # the cost of the batch: this call's time over the batch-1 call's
            r["vs_batch1"] = round(r["us"] / b1[tuple(r["shape"])], 3)
        log("gemv " + ", ".join(f"{r['shape'][0]}x{r['shape'][1]}b{r['batch']}:{r['gbs']:.0f}GB/s"
                                for r in extra["gemv_i8"]))
    if "decode" in only:
        from vx_amd import decode as _decode

        log("int8 decode config 4")
        dec = _decode.bench(lib, timer)
        # the step's algorithmic bytes (int8 weights, scales, norms, the KV
        # rows it reads and writes) over the whole generate call's time
        dec["roofline"] = {"bound": "hbm", "achieved": round(dec["bytes_gbs"], 1),
                           "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(dec["bytes_gbs"] / PEAK_HBM_GBS, 4),
                           "traffic": traffic_from_profiles("decode_i8", "bytes_per_position")}
        extra["decode_i8"] = dec

    if "gemm" in only:
        log("gemm bf16->f32 8192^3 (roofline point)")
        g8 = bench_gemm(lib, timer, 10, 2, n=8192)
        extra["gemm_bf16_8192"] = dict(config="bf16 x bf16 -> f32 GEMM, M=N=K=8192", ms=g8["ms_per_step"],
                                       tflops=g8["tflops"], frac_of_peak=g8["tflops"] / PEAK_BF16_TFLOPS,
                                       steps_us=g8["steps_us"], clock_mhz=g8["clock_mhz"],
                                       launch=g8["launch"])
        log(f"gemm 8192 {g8['tflops']:.1f} TFLOP/s")
        # the reference's own GEMM benchmark shape (benchmarks/gpu_gemm/run.sh:
        # 8192 x 3072 x 768 beside 4096^3; cuBLAS on an A100 214.2 TFLOP/s,
        # context only)
        log("gemm bf16->f32 8192x3072x768 (reference benchmark shape)")
        gr = bench_gemm(lib, timer, 50, 5, n=3072, m=8192, k=768)
        extra["gemm_bf16_8192x3072x768"] = dict(
            config="bf16 x bf16 -> f32 GEMM, M=8192 N=3072 K=768", ms=gr["ms_per_step"],
            tflops=gr["tflops"], frac_of_peak=gr["tflops"] / PEAK_BF16_TFLOPS,
            steps_us=gr["steps_us"], clock_mhz=gr["clock_mhz"], launch=gr["launch"],
            # HBM-side bytes per launch from the committed counter profile of
            # the stream-K launch (when that is the launch that ran)
            traffic=(traffic_from_profiles("gemm_bf16_8192x3072x768_sk")
                     if gr["launch"] == "stream-K" else None))
        log(f"gemm 8192x3072x768 {gr['tflops']:.1f} TFLOP/s ({gr['launch']})")
        log("gemm f32 512^3 (config 1)")
        extra["gemm_f32_512"] = bench_gemm_f32(lib, timer)
        log(f"gemm f32 512: {extra['gemm_f32_512']['us']:.1f} us device, "
            f"{extra['gemm_f32_512']['wall_us_per_dispatch']:.1f} us per dispatch, "
            f"max rel err {extra['gemm_f32_512']['max_rel_err_vs_oracle']:.2e}")

    cpu = None
    if not ns.skip_cpu:
        log("cpu baseline")
        import oracle

        # the reference's own CPU path where its library was built here
        # (oracle/_ref), else the restatement (oracle/vx_oracle.c)
        if oracle.ref_available():
            cpu = cpu_baseline_ref_gemm(g["a16"], g["b16"], gpu_rows=g["c_head"])
        else:
            cpu = cpu_baseline_gemm(g["a16"], g["b16"], gpu_rows=g["c_head"])
        cpu["nproc"] = os.cpu_count()
        if "gemm_bf16_8192" in extra:
            # the same CPU path on a timed block of rows of the 8192^3 GEMM
            cpu8 = cpu_baseline_ref_gemm if oracle.ref_available() else cpu_baseline_gemm
            extra["gemm_bf16_8192"]["cpu"] = cpu8(g8["a16"], g8["b16"], budget_s=3.0,
                                                  gpu_rows=g8["c_head"])
        if "flash_attn_fwd" in extra:
            extra["flash_attn_fwd"]["cpu"] = cpu_fa()
        if "gemv_i8" in extra:
            extra["gemv_i8_cpu"] = cpu_gemv()
        if "decode_i8" in extra:
            extra["decode_i8"]["cpu"] = cpu_decode()

    achieved = g["tflops"]
    line = {
        "metric": "GEMM & flash-attn fwd TFLOP/s (% MI355X bf16 peak); int8 decode tok/s bs=1",
        "value": round(g["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": ns.steps,
        "warmup": ns.warmup,
        "settle_ms": SETTLE_MS,
        "ms_per_step": round(g["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "bf16 x bf16 -> f32 GEMM, M=N=K=4096 (BASELINE config 2), "
                               "operands resident in HBM, one vx_plugin_dispatch_async per step",
                   "m": 4096, "n": 4096, "k": 4096},
        "runs_us": g["runs_us"],
        "tflops_runs": g["tflops_runs"],
        "steps_us": g["steps_us"],
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profiles("gemm_bf16_4096"),
                     # the shader clock the timed launches ran at, and the
                     # fraction of the dense peak at that clock (the nameplate
                     # figure assumes 2.4 GHz)
                     "clock_mhz": None if g["clock_mhz"] is None else round(g["clock_mhz"], 1),
                     "frac_at_clock": None if not g["clock_mhz"] else
                     round(achieved / (PEAK_BF16_TFLOPS * g["clock_mhz"] / PEAK_CLOCK_MHZ), 4)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
