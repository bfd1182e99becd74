"""Pins the CPU oracle (oracle/liboracle.so) before anything is checked
against it: against the reference's own x86 dispatch library built from its
sources, the reference's known answers, closed forms, and independent numpy
restatements on small inputs."""

import numpy as np
import pytest

import oracle
from tests import np_reference as npr
from vx_amd import abi
from vx_amd.abi import bf16_to_f32, f32_to_bf16
from vx_amd.llama import CONFIG_TINY, make_model, make_prompt, quantize_rows
from vx_amd.runtime import matmul

needs_ref = pytest.mark.skipif(not oracle.ref_available(),
                               reason="oracle/_ref not built (reference sources absent)")


def ref_matmul(a: np.ndarray, b: np.ndarray, dtype: int, outkind: str = "slot") -> np.ndarray:
    """C = A B through the reference x86 dispatch library, driven through the
    plugin ABI exactly as a compiled `c = a @ b` drives it (host memory,
    topology 0)."""
    lib = oracle.ref_lib()
    npt = np.float32 if dtype == abi.DTYPE_F32 else np.float64
    a = np.ascontiguousarray(a, npt)
    b = np.ascontiguousarray(b, npt)
    m, k = a.shape
    n = b.shape[1]
    ad = abi.Descriptor(a.ctypes.data, (m, k))
    bd = abi.Descriptor(b.ctypes.data, (k, n))
    if outkind == "slot":
        out = abi.SlotStorage(2)
        matmul(lib, ad, dtype, bd, dtype, out, dtype, outkind="slot", topo=abi.TOPO_CPU)
        ptr, off, sizes, strides = out.published()
        assert sizes == [m, n] and strides == [n, 1] and off == 0
        import ctypes
        buf = (ctypes.c_char * (m * n * np.dtype(npt).itemsize)).from_address(ptr)
        res = np.frombuffer(buf, dtype=npt).reshape(m, n).copy()
        ctypes.CDLL(None).free(ctypes.c_void_p(ptr))
        return res
    c = np.full((m, n), np.nan, npt)
    cd = abi.Descriptor(c.ctypes.data, (m, n))
    matmul(lib, ad, dtype, bd, dtype, cd, dtype, outkind="buffer", topo=abi.TOPO_CPU)
    return c


# -- GEMM f32 / f64 -----------------------------------------------------------

def roles_case():
    a = np.array([[i * 3 + j + 1 for j in range(3)] for i in range(2)], np.float32)
    b = np.array([[i * 4 + j + 1 for j in range(4)] for i in range(3)], np.float32)
    p = np.array([[i * 3 + j + 1 for j in range(3)] for i in range(3)], np.float32)
    q = np.diag([1.0, 2.0, 3.0]).astype(np.float32)
    return a, b, p, q


def test_known_answers_roles_oracle():
    """reference tests/backend/pass/gpu_matmul_roles.vx:47: 38 56 83 128 9 7 10"""
    a, b, p, q = roles_case()
    c = oracle.gemm_f32(a, b)
    r = oracle.gemm_f32(p, q)
    assert [c[0, 0], c[0, 3], c[1, 0], c[1, 3], r[0, 2], r[2, 0], r[1, 1]] == [38, 56, 83, 128, 9, 7, 10]


def test_known_answers_dtypes_oracle():
    """reference tests/backend/pass/gpu_matmul_dtypes.vx:45: 19 50 197 4032"""
    ad = np.array([[1, 2], [3, 4]], np.float64)
    bd = np.array([[5, 6], [7, 8]], np.float64)
    cd = oracle.gemm_f64(ad, bd)
    e = np.eye(64, dtype=np.float32)
    b = np.arange(64 * 64, dtype=np.float32).reshape(64, 64)
    r = oracle.gemm_f32(e, b)
    assert [cd[0, 0], cd[1, 1], r[3, 5], r[63, 0]] == [19, 50, 197, 4032]
    assert np.array_equal(r, b)


@needs_ref
@pytest.mark.parametrize("outkind", ["slot", "buffer"])
def test_reference_library_known_answers(outkind):
    a, b, p, q = roles_case()
    c = ref_matmul(a, b, abi.DTYPE_F32, outkind)
    r = ref_matmul(p, q, abi.DTYPE_F32, outkind)
    assert [c[0, 0], c[0, 3], c[1, 0], c[1, 3], r[0, 2], r[2, 0], r[1, 1]] == [38, 56, 83, 128, 9, 7, 10]
    cd = ref_matmul(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]]), abi.DTYPE_F64, outkind)
    assert [cd[0, 0], cd[1, 1]] == [19, 50]


@needs_ref
@pytest.mark.parametrize("shape", [(37, 29, 53), (128, 128, 128), (1, 768, 64)])
def test_oracle_f32_bit_equal_to_reference(shape, rng):
    m, k, n = shape
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    assert np.array_equal(oracle.gemm_f32(a, b), ref_matmul(a, b, abi.DTYPE_F32))


@needs_ref
def test_oracle_f64_bit_equal_to_reference(rng):
    a = rng.standard_normal((33, 47))
    b = rng.standard_normal((47, 21))
    assert np.array_equal(oracle.gemm_f64(a, b), ref_matmul(a, b, abi.DTYPE_F64))


def test_oracle_f32_close_to_f64(rng):
    a = rng.uniform(-1, 1, (64, 512)).astype(np.float32)
    b = rng.uniform(-1, 1, (512, 48)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    got = oracle.gemm_f32(a, b)
    assert np.all(np.abs(got - exact) <= 1e-4 * np.maximum(1.0, np.abs(exact)))


# -- bf16 ---------------------------------------------------------------------

def small_int_case(m, k, n):
    """benchmarks/gpu_gemm/*.vx inputs: A[i][k] = ((3i+5k)%7)-3,
    B[k][j] = ((2k+j)%5)-2; every f32 sum is exact."""
    i = np.arange(m)[:, None]
    kk = np.arange(k)[None, :]
    a = ((i * 3 + kk * 5) % 7 - 3).astype(np.float32)
    k2 = np.arange(k)[:, None]
    j = np.arange(n)[None, :]
    b = ((k2 * 2 + j) % 5 - 2).astype(np.float32)
    return f32_to_bf16(a), f32_to_bf16(b)


@needs_ref
def test_oracle_bf16_f32_equals_reference_f32_of_extended(rng):
    """The mixed plan's semantics (extend, f32 multiply, f32 add, k in order)
    are the reference's f32 loop on the extended values: bit-equal."""
    a16 = f32_to_bf16(rng.standard_normal((48, 96)).astype(np.float32))
    b16 = f32_to_bf16(rng.standard_normal((96, 80)).astype(np.float32))
    got = oracle.gemm_bf16_f32(a16, b16)
    want = ref_matmul(bf16_to_f32(a16), bf16_to_f32(b16), abi.DTYPE_F32)
    assert np.array_equal(got, want)


def test_oracle_bf16_small_ints_exact():
    a16, b16 = small_int_case(64, 256, 96)
    exact = bf16_to_f32(a16).astype(np.int64) @ bf16_to_f32(b16).astype(np.int64)
    assert np.array_equal(oracle.gemm_bf16_f32(a16, b16), exact.astype(np.float32))


def test_oracle_bf16_rows_and_points(rng):
    a16 = f32_to_bf16(rng.standard_normal((20, 64)).astype(np.float32))
    b16 = f32_to_bf16(rng.standard_normal((64, 30)).astype(np.float32))
    full = oracle.gemm_bf16_f32(a16, b16)
    part = oracle.gemm_bf16_f32(a16, b16, rows=slice(5, 9))
    assert np.array_equal(part[5:9], full[5:9]) and not part[:5].any() and not part[9:].any()
    exact = bf16_to_f32(a16).astype(np.float64) @ bf16_to_f32(b16).astype(np.float64)
    assert oracle.gemm_bf16_point_f64(a16, b16, 7, 11) == pytest.approx(exact[7, 11], abs=1e-12)


def test_oracle_bf16_linalg_matches_bruteforce(rng):
    a16 = f32_to_bf16(rng.standard_normal((7, 19)).astype(np.float32))
    b16 = f32_to_bf16(rng.standard_normal((19, 5)).astype(np.float32))
    assert np.array_equal(oracle.gemm_bf16_bf16_linalg(a16, b16), npr.gemm_bf16_linalg(a16, b16))
    # Small integers: every partial sum exact in bf16, so per-step rounding is
    # the same as one rounding of the exact result.
    s16, t16 = small_int_case(8, 8, 8)
    once = f32_to_bf16(oracle.gemm_bf16_f32(s16, t16))
    assert np.array_equal(oracle.gemm_bf16_bf16_linalg(s16, t16), once)


def test_bf16_rounding_matches_python_side():
    lib = oracle.lib()
    vals = np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.1415926, -2.5e-38, 1e38,
                     np.inf, -np.inf, np.nan, 65504.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9],
                    np.float32)
    py = f32_to_bf16(vals)
    c = np.array([lib.vx_oracle_f32_to_bf16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(py, c)
    # ties go to even: 1 + 2^-8 lies halfway between 1 and 1 + 2^-7
    assert py[12] == 0x3F80


# -- attention ----------------------------------------------------------------

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 4, 2, 33, 33, 16), (1, 2, 1, 5, 40, 8), (1, 2, 2, 48, 17, 8)])
def test_oracle_attention_matches_numpy(shape, causal, rng):
    b, h, hk, sq, sk, d = shape
    q16 = f32_to_bf16(rng.standard_normal((b, h, sq, d)).astype(np.float32))
    k16 = f32_to_bf16(rng.standard_normal((b, hk, sk, d)).astype(np.float32))
    v16 = f32_to_bf16(rng.standard_normal((b, hk, sk, d)).astype(np.float32))
    scale = 1.0 / np.sqrt(d)
    rows = oracle.attention_all_rows(b, h, sq)
    o, lse = oracle.attention_rows(q16, k16, v16, h, hk, scale, causal, rows)
    wo, wl = npr.attention_f64(q16, k16, v16, h, hk, scale, causal)
    np.testing.assert_allclose(o, wo.reshape(-1, d), atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(lse, wl.reshape(-1), atol=1e-5, rtol=1e-6)


def test_oracle_attention_closed_forms(rng):
    b, h, s, d = 1, 2, 24, 8
    v16 = f32_to_bf16(rng.standard_normal((b, h, s, d)).astype(np.float32))
    k16 = f32_to_bf16(rng.standard_normal((b, h, s, d)).astype(np.float32))
    q16 = f32_to_bf16(rng.standard_normal((b, h, s, d)).astype(np.float32))
    rows = oracle.attention_all_rows(b, h, s)
    # causal row 0 sees only key 0: o = V[0], lse = scale * q0 . k0
    o, lse = oracle.attention_rows(q16, k16, v16, h, h, 0.5, True, rows)
    o = o.reshape(b, h, s, d)
    lse = lse.reshape(b, h, s)
    v = bf16_to_f32(v16)
    np.testing.assert_allclose(o[:, :, 0], v[:, :, 0], rtol=1e-6)
    qk0 = (bf16_to_f32(q16)[:, :, 0].astype(np.float64) * bf16_to_f32(k16)[:, :, 0]).sum(-1) * 0.5
    np.testing.assert_allclose(lse[:, :, 0], qk0, rtol=1e-5, atol=1e-6)
    # zero queries: every score 0, o = prefix mean of V, lse = ln(count)
    zq = np.zeros_like(q16)
    o0, l0 = oracle.attention_rows(zq, k16, v16, h, h, 0.5, True, rows)
    o0 = o0.reshape(b, h, s, d)
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, s + 1)[None, None, :, None]
    np.testing.assert_allclose(o0, prefix, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(l0.reshape(b, h, s),
                               np.broadcast_to(np.log(np.arange(1, s + 1)), (b, h, s)), rtol=1e-6)


def test_oracle_attention_row_without_keys():
    q16 = f32_to_bf16(np.ones((1, 1, 4, 8), np.float32))
    k16 = f32_to_bf16(np.ones((1, 1, 2, 8), np.float32))
    rows = oracle.attention_all_rows(1, 1, 4)
    o, lse = oracle.attention_rows(q16, k16, k16, 1, 1, 1.0, True, rows)
    # queries are the last 4 of 2 keys: rows 0 and 1 see none
    assert np.all(o[:2] == 0) and np.all(np.isneginf(lse[:2])) and np.isfinite(lse[2:]).all()


# -- int8 GEMV ----------------------------------------------------------------

def test_oracle_gemv_exact_integers(rng):
    w = rng.integers(-127, 128, (96, 512), dtype=np.int8)
    x = rng.integers(-8, 9, (4, 512)).astype(np.float32)
    s = rng.uniform(0.001, 0.01, 96).astype(np.float32)
    y = oracle.gemv_i8(w, s, f32_to_bf16(x))
    exact = (w.astype(np.int64) @ x.astype(np.int64).T).T.astype(np.float32)
    assert np.array_equal(y, s[None, :] * exact)


def test_oracle_gemv_close_to_f64(rng):
    w = rng.integers(-127, 128, (64, 1024), dtype=np.int8)
    x16 = f32_to_bf16(rng.standard_normal((3, 1024)).astype(np.float32))
    s = rng.uniform(0.001, 0.01, 64).astype(np.float32)
    y = oracle.gemv_i8(w, s, x16)
    y64 = oracle.gemv_i8_f64(w, s, x16)
    want = (w.astype(np.float64) @ bf16_to_f32(x16).astype(np.float64).T).T * s[None, :]
    np.testing.assert_allclose(y64, want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(y, want, rtol=1e-4, atol=1e-4)


def test_oracle_gemv_f32_input(rng):
    w = rng.integers(-127, 128, (80, 768), dtype=np.int8)
    x = rng.standard_normal(768).astype(np.float32)
    s = rng.uniform(0.001, 0.01, 80).astype(np.float32)
    y = oracle.gemv_i8_f32in(w, s, x)
    want = s.astype(np.float64) * (w.astype(np.float64) @ x.astype(np.float64))
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-6)
    xi = rng.integers(-8, 9, 768).astype(np.float32)  # exact sums
    assert np.array_equal(oracle.gemv_i8_f32in(w, s, xi),
                          s * (w.astype(np.int64) @ xi.astype(np.int64)).astype(np.float32))


def test_quantize_matches_package(rng):
    w = rng.standard_normal((33, 77)).astype(np.float32) * 0.02
    w[3] = 0.0
    q, s = oracle.quantize_rows(w)
    pq, ps = quantize_rows(w)
    assert np.array_equal(q, pq) and np.array_equal(s, ps)
    assert s[3] == 1.0 and not q[3].any()
    assert np.all(np.abs(q).max(axis=1)[np.arange(33) != 3] == 127)
    np.testing.assert_allclose(q * s[:, None], w, atol=float(s.max()) / 2 + 1e-9)


# -- decode -------------------------------------------------------------------

def test_oracle_llama_matches_numpy_tiny():
    cfg = CONFIG_TINY
    model = make_model(cfg, seed=3)
    prompt = make_prompt(cfg, n=4, seed=5)
    kv = np.zeros(2 * cfg.n_layers * cfg.seq_len * cfg.kv_dim, np.float32)
    tokens = list(prompt) + [7, 11, 13]
    want = npr.llama_logits(cfg, model, tokens)
    for pos, tok in enumerate(tokens):
        got = oracle.llama_forward(cfg.as_dict(), model, kv, int(tok), pos)
        np.testing.assert_allclose(got, want[pos], rtol=1e-4, atol=1e-5)


def test_oracle_llama_generate_greedy_is_argmax_chain():
    cfg = CONFIG_TINY
    model = make_model(cfg, seed=3)
    prompt = make_prompt(cfg, n=4, seed=5)
    toks, margin = oracle.llama_generate(cfg.as_dict(), model, prompt, 6)
    kv = np.zeros(2 * cfg.n_layers * cfg.seq_len * cfg.kv_dim, np.float32)
    feed = list(prompt)
    got = []
    for pos in range(len(prompt) + 6 - 1 + 1):
        tok = feed[pos] if pos < len(feed) else got[-1]
        logits = oracle.llama_forward(cfg.as_dict(), model, kv, int(tok), pos)
        if pos >= len(prompt) - 1:
            got.append(int(np.argmax(logits)))
        if len(got) == 6:
            break
    assert list(toks) == got
    assert np.all(margin >= 0)


def test_decode_golden_fixture_prefix():
    """The committed config-4 fixture is the oracle's: its first tokens are
    recomputed here (the whole stream takes the oracle ~85 s)."""
    import json
    from pathlib import Path
    from vx_amd.llama import CONFIG_DECODE

    g = json.loads((Path(__file__).parent / "golden" / "decode_config4.json").read_text())
    cfg = CONFIG_DECODE
    assert g["config"] == cfg.as_dict()
    model = make_model(cfg, seed=g["model_seed"])
    prompt = make_prompt(cfg, n=16, seed=g["prompt_seed"])
    assert list(map(int, prompt)) == g["prompt"]
    toks, margin = oracle.llama_generate(cfg.as_dict(), model, prompt, 3)
    assert list(map(int, toks)) == g["tokens"][:3]
    np.testing.assert_allclose(margin, g["margins"][:3], rtol=1e-6)


def test_checker_catches_planted_error(rng):
    """The comparison the GPU tests use fails when one value of the oracle's
    answer is moved by more than the tolerance (the conformance harness's
    perturbation switch, reference scripts/tools/vx_xpu_conformance.cpp:916-927)."""
    from tests.parity import assert_max_abs

    a16 = f32_to_bf16(rng.standard_normal((16, 32)).astype(np.float32))
    b16 = f32_to_bf16(rng.standard_normal((32, 16)).astype(np.float32))
    want = oracle.gemm_bf16_f32(a16, b16)
    planted = want.copy()
    planted[3, 4] += 0.03
    assert_max_abs(want.copy(), want, 2e-2)
    with pytest.raises(AssertionError):
        assert_max_abs(planted, want, 2e-2)
