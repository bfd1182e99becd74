"""The flash-attention forward op on the GPU against the CPU oracle (f64
two-pass softmax), including the full BASELINE config on sampled rows."""

import ctypes

import numpy as np
import pytest

import oracle
from tests.conftest import announce
from tests.parity import BF16_ABS, assert_max_abs
from vx_amd import abi
from vx_amd.abi import bf16_to_f32, f32_to_bf16
from vx_amd.runtime import DeviceArray, HipTimer, flash_attention_fwd

pytestmark = pytest.mark.gpu


BF16_NAN = 0x7FC0


def run(lib, q16, k16, v16, heads, kv_heads, scale, causal, with_lse=True, poison=False):
    """One launch. With `poison` the output and lse buffers start as NaN, so
    an element the kernel never writes stays NaN."""
    b, _, sq, d = q16.shape
    sk = k16.shape[2]
    dq = DeviceArray.of(lib, q16, abi.DTYPE_BF16)
    dk = DeviceArray.of(lib, k16, abi.DTYPE_BF16)
    dv = DeviceArray.of(lib, v16, abi.DTYPE_BF16)
    if poison:
        do = DeviceArray.of(lib, np.full(q16.shape, BF16_NAN, np.uint16), abi.DTYPE_BF16)
        dl = DeviceArray.of(lib, np.full((b, heads, sq), np.nan, np.float32), abi.DTYPE_F32)
    else:
        do = DeviceArray(lib, q16.shape, abi.DTYPE_BF16)
        dl = DeviceArray(lib, (b, heads, sq), abi.DTYPE_F32) if with_lse else None
    rc = flash_attention_fwd(lib, dq.ptr, dk.ptr, dv.ptr, do.ptr, dl.ptr if dl else None, b, heads,
                             kv_heads, sq, sk, d, scale, causal)
    assert rc == 0
    o = bf16_to_f32(do.numpy())
    lse = dl.numpy() if dl else None
    for a in (dq, dk, dv, do) + ((dl,) if dl else ()):
        a.free()
    return o, lse


def randn16(rng, shape):
    return f32_to_bf16(rng.standard_normal(shape).astype(np.float32))


CASES = [
    # batch, heads, kv_heads, seq_q, seq_k, head_dim
    (1, 2, 2, 128, 128, 128),
    (2, 4, 2, 200, 200, 64),
    (1, 2, 1, 64, 300, 128),
    (1, 1, 1, 1, 1, 128),
    (1, 3, 3, 129, 129, 64),
    (2, 2, 2, 300, 70, 128),
]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("case", CASES)
def test_matches_oracle(hiplib, case, causal, rng):
    announce(f"flash attn {case} causal={causal}")
    b, h, hk, sq, sk, d = case
    q16, k16, v16 = randn16(rng, (b, h, sq, d)), randn16(rng, (b, hk, sk, d)), randn16(rng, (b, hk, sk, d))
    scale = 1.0 / np.sqrt(d)
    o, lse = run(hiplib, q16, k16, v16, h, hk, scale, causal)
    rows = oracle.attention_all_rows(b, h, sq)
    wo, wl = oracle.attention_rows(q16, k16, v16, h, hk, scale, causal, rows)
    assert_max_abs(o.reshape(-1, d), wo, BF16_ABS, f"o {case}")
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(lse.ravel()), fin)
    assert_max_abs(lse.ravel()[fin], wl[fin], 1e-3, f"lse {case}")
    assert np.all(o.reshape(-1, d)[~fin] == 0)


def test_closed_forms(hiplib, rng):
    announce("flash attn closed forms")
    b, h, s, d = 1, 4, 256, 128
    k16, v16 = randn16(rng, (b, h, s, d)), randn16(rng, (b, h, s, d))
    q16 = randn16(rng, (b, h, s, d))
    o, lse = run(hiplib, q16, k16, v16, h, h, 0.125, True)
    v = bf16_to_f32(v16)
    # causal row 0 is V[0] (rounded once to bf16)
    assert np.array_equal(o[:, :, 0], bf16_to_f32(f32_to_bf16(v[:, :, 0])))
    # zero queries: prefix mean of V, lse = ln(count)
    o0, l0 = run(hiplib, np.zeros_like(q16), k16, v16, h, h, 0.125, True)
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, s + 1)[None, None, :, None]
    assert_max_abs(o0, prefix, 1e-2, "prefix mean")
    assert_max_abs(l0, np.broadcast_to(np.log(np.arange(1, s + 1)), l0.shape), 1e-4, "ln count")


def numpy_head_f64(q16, k16, v16, bi, hi, scale):
    """Causal softmax(q k^T * scale) v of one whole head in f64, vectorised
    (written independently of the C oracle)."""
    q = bf16_to_f32(q16[bi, hi]).astype(np.float64)
    k = bf16_to_f32(k16[bi, hi]).astype(np.float64)
    v = bf16_to_f32(v16[bi, hi]).astype(np.float64)
    s = (q @ k.T) * scale
    s[np.triu_indices(s.shape[0], 1)] = -np.inf
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(axis=1, keepdims=True)
    return (p @ v) / l, (m + np.log(l))[:, 0]


def test_baseline_config_sampled(hiplib):
    """[4, 32, 2048, 128] causal, N(0,1), scale 1/sqrt(128).

    The output and lse start as NaN, so every element being finite proves the
    launch wrote all of them. Against the f64 oracle: the first and last row
    of every (batch, head), one row in every 128-query block of every head
    (the unit the launch order maps workgroups to, at a different offset per
    block), and extra rows at block boundaries; one whole head per batch is
    compared row by row against a numpy f64 softmax. A launch order that ran
    one (head, block) twice and skipped another fails here."""
    announce("flash attn config 3")
    rng = np.random.default_rng(7)
    b, h, s, d = 4, 32, 2048, 128
    q16, k16, v16 = (randn16(rng, (b, h, s, d)) for _ in range(3))
    scale = 1.0 / np.sqrt(d)
    o, lse = run(hiplib, q16, k16, v16, h, h, scale, True, poison=True)
    assert np.isfinite(o).all() and np.isfinite(lse).all(), "unwritten output or lse"
    rows = set()
    for bi in range(b):
        for hi in range(h):
            rows.update({(bi, hi, 0), (bi, hi, s - 1)})
            for qb in range(s // 128):
                rows.add((bi, hi, qb * 128 + ((bi * h + hi) * 37 + qb * 11) % 128))
    picks = [1, 31, 32, 63, 64, 127, 128, 129, 1000, 1023, 1024, 2046]
    rows.update((bi, hi, qi) for bi in range(b) for hi in (0, 13, 31) for qi in picks)
    rows = np.array(sorted(rows), np.int64)
    wo, wl = oracle.attention_rows(q16, k16, v16, h, h, scale, True, rows)
    got = o[rows[:, 0], rows[:, 1], rows[:, 2]]
    assert_max_abs(got, wo, BF16_ABS, "config 3 rows")
    assert_max_abs(lse[rows[:, 0], rows[:, 1], rows[:, 2]], wl, 1e-3, "config 3 lse")
    for bi in range(b):
        hi = (11 * bi + 5) % h
        wo_head, wl_head = numpy_head_f64(q16, k16, v16, bi, hi, scale)
        assert_max_abs(o[bi, hi], wo_head, BF16_ABS, f"config 3 whole head ({bi}, {hi})")
        assert_max_abs(lse[bi, hi], wl_head, 1e-3, f"config 3 whole head lse ({bi}, {hi})")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("rise", [320.0, 1024.0, -1024.0])
def test_scores_rising_after_the_first_block(hiplib, causal, rise, rng):
    """Keys 64 and up score `rise` above keys 0-63 for every query (q and k
    share a large first component), so the running max a row takes from its
    first key block is far below its true max. At 320 the rise is 40.8 in
    base-2 exponent units (scale 1/sqrt(128) times log2(e)); at 1024 it is
    130.6, past f32's exponent range were p not taken against the moved
    max: the reference max moves, O and l are rescaled, and the first
    block's terms vanish. At -1024 the later keys all but vanish. Every row
    against the f64 oracle."""
    announce(f"flash attn score rise {rise} causal={causal}")
    b, h, s, d = 1, 2, 320, 128
    q = rng.standard_normal((b, h, s, d)).astype(np.float32) * 0.1
    k = rng.standard_normal((b, h, s, d)).astype(np.float32) * 0.1
    v = rng.standard_normal((b, h, s, d)).astype(np.float32)
    q[..., 0] = 32.0
    k[..., :64, 0] = 0.0
    k[..., 64:, 0] = rise / 32.0
    q16, k16, v16 = f32_to_bf16(q), f32_to_bf16(k), f32_to_bf16(v)
    scale = 1.0 / np.sqrt(d)
    o, lse = run(hiplib, q16, k16, v16, h, h, scale, causal, poison=True)
    rows = oracle.attention_all_rows(b, h, s)
    wo, wl = oracle.attention_rows(q16, k16, v16, h, h, scale, causal, rows)
    assert_max_abs(o.reshape(-1, d), wo, BF16_ABS, f"rise {rise}")
    assert_max_abs(lse.ravel(), wl, 1e-3, f"rise {rise} lse")


@pytest.mark.parametrize("start", [0, 1536, 7680])
def test_reference_prefill_chunks(hiplib, start):
    """The reference's own flash-attention benchmark shape (reference
    benchmarks/apple_gpu_mlir_kernels/README.md:30-37): a 512-token causal
    prefill chunk at position 0, 1536 and 7680 of the cache, 32 query heads
    over 4 KV heads, head_dim 128. Queries sit at the end of the keys
    (seq_k = start + 512), so query i sees keys up to start + i. Sampled rows
    against the f64 oracle."""
    announce(f"flash attn prefill chunk at {start}")
    rng = np.random.default_rng(start + 5)
    b, h, hk, sq, d = 1, 32, 4, 512, 128
    sk = start + sq
    q16, k16, v16 = randn16(rng, (b, h, sq, d)), randn16(rng, (b, hk, sk, d)), randn16(rng, (b, hk, sk, d))
    scale = 1.0 / np.sqrt(d)
    o, lse = run(hiplib, q16, k16, v16, h, hk, scale, True)
    picks = [0, 1, 63, 64, 255, 256, 510, 511]
    rows = np.array([(0, hi, qi) for hi in (0, 7, 8, 31) for qi in picks], np.int64)
    wo, wl = oracle.attention_rows(q16, k16, v16, h, hk, scale, True, rows)
    assert_max_abs(o[rows[:, 0], rows[:, 1], rows[:, 2]], wo, BF16_ABS, f"chunk at {start}")
    assert_max_abs(lse[rows[:, 0], rows[:, 1], rows[:, 2]], wl, 1e-3, f"chunk lse at {start}")
    assert np.isfinite(o).all()


SPLIT_CASES = [
    # batch, heads, kv_heads, seq_q, seq_k, head_dim, causal, splits
    (1, 4, 2, 1, 1000, 128, True, 4),      # one query row over a long cache
    (1, 2, 1, 64, 700, 128, True, 3),      # queries at the end of the keys, GQA
    (2, 2, 2, 200, 200, 64, True, 4),      # causal square: late splits empty for early rows
    (1, 3, 3, 129, 577, 64, False, 5),     # ragged key tail, non-causal
    (1, 2, 2, 300, 70, 128, True, 8),      # more splits than key blocks (clamped)
    (1, 2, 2, 64, 4100, 128, False, 64),   # the largest forced count
]


@pytest.mark.parametrize("case", SPLIT_CASES)
def test_key_splits_match_oracle(hiplib, case, rng):
    """Key-split launches (each split's partial in f32, then the merge) on
    shapes the automatic choice would not split: every row against the
    oracle, and the split output against the unsplit launch of the same
    inputs. Rows no split saw (causal rows with no key) must merge to o = 0
    and lse = -inf."""
    announce(f"flash attn split {case}")
    b, h, hk, sq, sk, d, causal, splits = case
    q16, k16, v16 = randn16(rng, (b, h, sq, d)), randn16(rng, (b, hk, sk, d)), randn16(rng, (b, hk, sk, d))
    scale = 1.0 / np.sqrt(d)
    hiplib.force_fa_splits(splits)
    try:
        o, lse = run(hiplib, q16, k16, v16, h, hk, scale, causal)
        o_nolse, _ = run(hiplib, q16, k16, v16, h, hk, scale, causal, with_lse=False)
    finally:
        hiplib.force_fa_splits(0)
    hiplib.force_fa_splits(1)
    try:
        o1, lse1 = run(hiplib, q16, k16, v16, h, hk, scale, causal)
    finally:
        hiplib.force_fa_splits(0)
    rows = oracle.attention_all_rows(b, h, sq)
    wo, wl = oracle.attention_rows(q16, k16, v16, h, hk, scale, causal, rows)
    assert_max_abs(o.reshape(-1, d), wo, BF16_ABS, f"split o {case}")
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(lse.ravel()), fin)
    assert_max_abs(lse.ravel()[fin], wl[fin], 1e-3, f"split lse {case}")
    assert np.all(o.reshape(-1, d)[~fin] == 0)
    assert np.array_equal(o, o_nolse)
    # the split and unsplit launches differ only by f32 rounding in the merge
    assert_max_abs(o.reshape(-1, d), o1.reshape(-1, d), BF16_ABS, f"split vs unsplit {case}")
    assert_max_abs(lse.ravel()[fin], lse1.ravel()[fin], 1e-4, f"split vs unsplit lse {case}")


def test_capture_runs_unsplit(hiplib, rng):
    """A launch recorded into a hipGraph takes no stream-ordered workspace,
    so it runs unsplit even with splits forced: every replay (with eager
    launches that overwrite O in between) equals the eager unsplit launch
    bit for bit, and the eager split launch matches it to rounding."""
    announce("flash attn captured with splits forced")
    b, h, hk, sq, sk, d = 1, 32, 4, 512, 2048, 128
    q16, k16, v16 = randn16(rng, (b, h, sq, d)), randn16(rng, (b, hk, sk, d)), randn16(rng, (b, hk, sk, d))
    q2 = randn16(rng, (b, h, sq, d))
    scale = 1.0 / np.sqrt(d)
    dq, dq2 = DeviceArray.of(hiplib, q16, abi.DTYPE_BF16), DeviceArray.of(hiplib, q2, abi.DTYPE_BF16)
    dk, dv = DeviceArray.of(hiplib, k16, abi.DTYPE_BF16), DeviceArray.of(hiplib, v16, abi.DTYPE_BF16)
    do = DeviceArray(hiplib, (b, h, sq, d), abi.DTYPE_BF16)
    dl = DeviceArray(hiplib, (b, h, sq), abi.DTYPE_F32)

    def call(qp):
        assert flash_attention_fwd(hiplib, qp, dk.ptr, dv.ptr, do.ptr, dl.ptr, b, h, hk, sq, sk, d,
                                   scale, True) == 0

    t = HipTimer()
    s = t.stream_create()
    ex = None
    try:
        hiplib.force_fa_splits(1)
        call(dq.ptr)
        o1, l1 = do.numpy().copy(), dl.numpy().copy()
        hiplib.force_fa_splits(4)
        call(dq.ptr)
        o4, l4 = do.numpy().copy(), dl.numpy().copy()
        assert_max_abs(bf16_to_f32(o4), bf16_to_f32(o1), BF16_ABS, "split vs unsplit")
        assert_max_abs(l4, l1, 1e-4, "split vs unsplit lse")
        hiplib.lib.vx_hip_set_stream(s)
        ex = t.capture(s, lambda: call(dq.ptr))
        hiplib.lib.vx_hip_set_stream(None)
        for rep in range(3):
            call(dq2.ptr)  # eager, split: overwrites O and LSE
            hiplib.wait()
            t.graph_launch(ex, s)
            t.sync()
            assert np.array_equal(do.numpy(), o1), f"replay {rep}"
            assert np.array_equal(dl.numpy(), l1), f"replay {rep} lse"
    finally:
        hiplib.force_fa_splits(0)
        hiplib.lib.vx_hip_set_stream(None)
        if ex is not None:
            t.graph_destroy(ex)
        t.stream_destroy(s)
        for x in (dq, dq2, dk, dv, do, dl):
            x.free()


def test_split_workspaces_from_threads(hiplib):
    """Four host threads, each on its own stream (the caller stream is per
    thread), launch the automatically split prefill-chunk shape at two
    cache lengths in turn, so each stream's partials block grows while the
    others are in use. The split path is deterministic, so every result must
    equal the one the same call gives alone."""
    import threading

    announce("flash attn split workspaces from four threads")
    b, h, hk, sq, d = 1, 32, 4, 512, 128
    scale = 1.0 / np.sqrt(d)
    rng = np.random.default_rng(77)
    cases = []
    for sk in (2048, 8192):
        q16, k16, v16 = (randn16(rng, (b, h, sq, d)), randn16(rng, (b, hk, sk, d)),
                         randn16(rng, (b, hk, sk, d)))
        o, lse = run(hiplib, q16, k16, v16, h, hk, scale, True)
        cases.append((q16, k16, v16, sk, f32_to_bf16(o), lse))
    errors = []

    def work(tid):
        t = HipTimer()
        s = t.stream_create()
        arrays = []
        try:
            hiplib.lib.vx_hip_set_stream(s)
            dev = []
            for q16, k16, v16, sk, _, _ in cases:
                xs = (DeviceArray.of(hiplib, q16, abi.DTYPE_BF16), DeviceArray.of(hiplib, k16, abi.DTYPE_BF16),
                      DeviceArray.of(hiplib, v16, abi.DTYPE_BF16),
                      DeviceArray(hiplib, (b, h, sq, d), abi.DTYPE_BF16),
                      DeviceArray(hiplib, (b, h, sq), abi.DTYPE_F32))
                arrays += list(xs)
                dev.append(xs)
            for it in range(6):
                ci = (tid + it) % 2
                dq, dk, dv, do, dl = dev[ci]
                sk = cases[ci][3]
                rc = flash_attention_fwd(hiplib, dq.ptr, dk.ptr, dv.ptr, do.ptr, dl.ptr, b, h, hk, sq,
                                         sk, d, scale, True)
                if rc != 0:
                    errors.append((tid, it, f"rc {rc}"))
                    continue
                if not np.array_equal(do.numpy(), cases[ci][4]):
                    errors.append((tid, it, "o"))
                if not np.array_equal(dl.numpy(), cases[ci][5]):
                    errors.append((tid, it, "lse"))
        except Exception as e:  # reported below, with the thread that raised it
            errors.append((tid, -1, repr(e)))
        finally:
            for x in arrays:
                x.free()
            hiplib.lib.vx_hip_set_stream(None)
            t.sync()
            t.stream_destroy(s)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=90)
    assert not any(th.is_alive() for th in threads), "a launching thread did not finish"
    assert not errors, errors


def fa_workspaces(lib):
    out = (ctypes.c_int64 * 2)()
    assert lib.control(abi.HIP_CTRL_FA_WORKSPACES, out) == 1
    return out[0], out[1]


def test_split_workspace_freed_with_stream(hiplib, rng):
    """Streams created and destroyed in a loop, each splitting a launch:
    setting the thread's stream back to NULL frees that stream's workspace
    (so none is left for a destroyed stream, and a new stream at a reused
    address starts with none), and every loop's result is the same."""
    announce("flash attn split workspace per stream lifetime")
    b, h, hk, sq, sk, d = 1, 4, 2, 64, 1024, 128
    q16, k16, v16 = randn16(rng, (b, h, sq, d)), randn16(rng, (b, hk, sk, d)), randn16(rng, (b, hk, sk, d))
    scale = 1.0 / np.sqrt(d)
    dq, dk, dv = (DeviceArray.of(hiplib, x, abi.DTYPE_BF16) for x in (q16, k16, v16))
    do = DeviceArray(hiplib, (b, h, sq, d), abi.DTYPE_BF16)
    dl = DeviceArray(hiplib, (b, h, sq), abi.DTYPE_F32)
    t = HipTimer()
    first = None
    try:
        hiplib.force_fa_splits(4)
        base_blocks, _ = fa_workspaces(hiplib)
        for it in range(6):
            s = t.stream_create()
            try:
                hiplib.lib.vx_hip_set_stream(s)
                assert flash_attention_fwd(hiplib, dq.ptr, dk.ptr, dv.ptr, do.ptr, dl.ptr, b, h, hk,
                                           sq, sk, d, scale, True) == 0
                blocks, nbytes = fa_workspaces(hiplib)
                assert blocks == base_blocks + 1 and nbytes >= 4 * b * h * sq * (d + 1) * 4, it
                got = (do.numpy().copy(), dl.numpy().copy())
            finally:
                hiplib.lib.vx_hip_set_stream(None)
                t.sync()
                t.stream_destroy(s)
            assert fa_workspaces(hiplib)[0] == base_blocks, f"loop {it}: workspace kept"
            if first is None:
                first = got
            assert np.array_equal(got[0], first[0]) and np.array_equal(got[1], first[1]), it
        wo, wl = oracle.attention_rows(q16, k16, v16, h, hk, scale, True,
                                       oracle.attention_all_rows(b, h, sq))
        assert_max_abs(bf16_to_f32(first[0]).reshape(-1, d), wo, BF16_ABS, "split per stream")
    finally:
        hiplib.force_fa_splits(0)
        hiplib.lib.vx_hip_set_stream(None)
        for x in (dq, dk, dv, do, dl):
            x.free()


def test_split_control_refusals(hiplib):
    with pytest.raises(ValueError):
        hiplib.force_fa_splits(-1)
    with pytest.raises(ValueError):
        hiplib.force_fa_splits(65)
    hiplib.force_fa_splits(0)


def test_no_lse_and_refusals(hiplib, rng):
    announce("flash attn refusals")
    q16 = randn16(rng, (1, 2, 64, 64))
    o, lse = run(hiplib, q16, q16, q16, 2, 2, 0.125, False, with_lse=False)
    assert lse is None and np.isfinite(o).all()
    dq = DeviceArray.of(hiplib, q16, abi.DTYPE_BF16)
    p = dq.ptr
    # head_dim 96 is not a kernel shape
    assert flash_attention_fwd(hiplib, p, p, p, p, None, 1, 2, 2, 64, 64, 96, 0.125, False) == -4
    # 3 heads cannot share 2 kv heads
    assert flash_attention_fwd(hiplib, p, p, p, p, None, 1, 3, 2, 64, 64, 64, 0.125, False) == -1
    # host memory is refused
    assert flash_attention_fwd(hiplib, q16.ctypes.data, p, p, p, None, 1, 2, 2, 64, 64, 64, 0.125,
                               False) == -3
    dq.free()
