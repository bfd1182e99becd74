"""ctypes bindings to the CPU oracle (liboracle.so) and to the reference's own
x86 dispatch library built from its sources (_ref/libvx_x86_dispatch.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline. The
product path never imports it.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libvx_x86_dispatch.so"

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


class LlamaConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")]


LLAMA_WEIGHT_FIELDS = ("tok_q", "tok_s", "rms_att", "wq_q", "wq_s", "wk_q", "wk_s", "wv_q", "wv_s",
                       "wo_q", "wo_s", "rms_ffn", "w1_q", "w1_s", "w2_q", "w2_s", "w3_q", "w3_s",
                       "rms_final", "rope")


class LlamaWeights(ctypes.Structure):
    _fields_ = [(n, _p) for n in LLAMA_WEIGHT_FIELDS]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise FileNotFoundError(f"{LIB} is not built; run `make -C oracle`")
        L = ctypes.CDLL(str(LIB))
        sig = {
            "vx_oracle_gemm_f32": (None, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64]),
            "vx_oracle_gemm_f64": (None, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64]),
            "vx_oracle_gemm_bf16_f32_rows": (None, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64]),
            "vx_oracle_gemm_bf16_bf16_linalg": (None, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64]),
            "vx_oracle_gemm_bf16_point_f64": (ctypes.c_double, [_p, _i64, _p, _i64, _i64, _i64, _i64]),
            "vx_oracle_attention_rows": (None, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                                ctypes.c_double, _i32, _p, _i64, _p, _p]),
            "vx_oracle_gemv_i8": (None, [_p, _p, _p, _p, _i64, _i64, _i64]),
            "vx_oracle_gemv_i8_f64": (None, [_p, _p, _p, _p, _i64, _i64, _i64]),
            "vx_oracle_gemv_i8_f32in": (None, [_p, _p, _p, _p, _i64, _i64]),
            "vx_oracle_quantize_rows": (None, [_p, _i64, _i64, _p, _p]),
            "vx_oracle_llama_generate": (_i32, [ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaWeights),
                                                _p, _i32, _i32, _p, _p]),
            "vx_oracle_llama_forward": (None, [ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaWeights),
                                               _p, _i32, _i32, _p]),
            "vx_oracle_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "vx_oracle_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


def gemm_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _c(a, np.float32), _c(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().vx_oracle_gemm_f32(a.ctypes.data, k, b.ctypes.data, n, c.ctypes.data, n, m, n, k)
    return c


def gemm_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _c(a, np.float64), _c(b, np.float64)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float64)
    lib().vx_oracle_gemm_f64(a.ctypes.data, k, b.ctypes.data, n, c.ctypes.data, n, m, n, k)
    return c


def gemm_bf16_f32(a16: np.ndarray, b16: np.ndarray, rows: slice | None = None) -> np.ndarray:
    """bf16 bit patterns in, f32 out; `rows` limits the computed rows (others
    are left 0)."""
    a16, b16 = _c(a16, np.uint16), _c(b16, np.uint16)
    m, k = a16.shape
    n = b16.shape[1]
    c = np.zeros((m, n), np.float32)
    r0, r1 = (0, m) if rows is None else (rows.start or 0, rows.stop)
    lib().vx_oracle_gemm_bf16_f32_rows(a16.ctypes.data, k, b16.ctypes.data, n, c.ctypes.data, n,
                                       r0, r1 - r0, n, k)
    return c


def gemm_bf16_bf16_linalg(a16: np.ndarray, b16: np.ndarray) -> np.ndarray:
    a16, b16 = _c(a16, np.uint16), _c(b16, np.uint16)
    m, k = a16.shape
    n = b16.shape[1]
    c = np.empty((m, n), np.uint16)
    lib().vx_oracle_gemm_bf16_bf16_linalg(a16.ctypes.data, k, b16.ctypes.data, n, c.ctypes.data, n,
                                          m, n, k)
    return c


def gemm_bf16_point_f64(a16, b16, i: int, j: int) -> float:
    a16, b16 = _c(a16, np.uint16), _c(b16, np.uint16)
    k = a16.shape[1]
    return lib().vx_oracle_gemm_bf16_point_f64(a16.ctypes.data, k, b16.ctypes.data, b16.shape[1],
                                               i, j, k)


def attention_rows(q16, k16, v16, heads: int, kv_heads: int, scale: float, causal: bool,
                   rows: np.ndarray):
    """rows: int64 [n, 3] of (batch, head, query). Returns (o [n, d] f32, lse [n] f32)."""
    q16, k16, v16 = _c(q16, np.uint16), _c(k16, np.uint16), _c(v16, np.uint16)
    batch, _, seq_q, d = q16.shape
    seq_k = k16.shape[2]
    rows = _c(rows, np.int64).reshape(-1, 3)
    o = np.empty((len(rows), d), np.float32)
    lse = np.empty(len(rows), np.float32)
    lib().vx_oracle_attention_rows(q16.ctypes.data, k16.ctypes.data, v16.ctypes.data, batch, heads,
                                   kv_heads, seq_q, seq_k, d, scale, 1 if causal else 0,
                                   rows.ctypes.data, len(rows), o.ctypes.data, lse.ctypes.data)
    return o, lse


def attention_all_rows(batch: int, heads: int, seq_q: int) -> np.ndarray:
    b, h, i = np.meshgrid(np.arange(batch), np.arange(heads), np.arange(seq_q), indexing="ij")
    return np.stack([b.ravel(), h.ravel(), i.ravel()], axis=1).astype(np.int64)


def gemv_i8(w: np.ndarray, scale: np.ndarray, x16: np.ndarray) -> np.ndarray:
    w, scale, x16 = _c(w, np.int8), _c(scale, np.float32), _c(x16, np.uint16)
    rows, cols = w.shape
    batch = x16.shape[0]
    y = np.empty((batch, rows), np.float32)
    lib().vx_oracle_gemv_i8(w.ctypes.data, scale.ctypes.data, x16.ctypes.data, y.ctypes.data, rows,
                            cols, batch)
    return y


def gemv_i8_f64(w, scale, x16) -> np.ndarray:
    w, scale, x16 = _c(w, np.int8), _c(scale, np.float32), _c(x16, np.uint16)
    rows, cols = w.shape
    batch = x16.shape[0]
    y = np.empty((batch, rows), np.float64)
    lib().vx_oracle_gemv_i8_f64(w.ctypes.data, scale.ctypes.data, x16.ctypes.data, y.ctypes.data,
                                rows, cols, batch)
    return y


def gemv_i8_f32in(w, scale, x) -> np.ndarray:
    w, scale, x = _c(w, np.int8), _c(scale, np.float32), _c(x, np.float32)
    rows, cols = w.shape
    y = np.empty(rows, np.float32)
    lib().vx_oracle_gemv_i8_f32in(w.ctypes.data, scale.ctypes.data, x.ctypes.data, y.ctypes.data,
                                  rows, cols)
    return y


def quantize_rows(w: np.ndarray):
    w = _c(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().vx_oracle_quantize_rows(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data)
    return q, s


def _weights_struct(model: dict) -> tuple[LlamaWeights, list]:
    keep = []
    ws = LlamaWeights()
    for name in LLAMA_WEIGHT_FIELDS:
        arr = model[name]
        keep.append(arr)
        setattr(ws, name, arr.ctypes.data)
    return ws, keep


def llama_generate(cfg: dict, model: dict, prompt, n_steps: int):
    c = LlamaConfig(**cfg)
    ws, keep = _weights_struct(model)
    prompt = _c(prompt, np.int32)
    toks = np.empty(n_steps, np.int32)
    margin = np.empty(n_steps, np.float32)
    rc = lib().vx_oracle_llama_generate(ctypes.byref(c), ctypes.byref(ws), prompt.ctypes.data,
                                        len(prompt), n_steps, toks.ctypes.data, margin.ctypes.data)
    if rc != 0:
        raise ValueError("vx_oracle_llama_generate refused the arguments")
    return toks, margin


def llama_forward(cfg: dict, model: dict, kv: np.ndarray, token: int, pos: int) -> np.ndarray:
    c = LlamaConfig(**cfg)
    ws, keep = _weights_struct(model)
    logits = np.empty(cfg["vocab_size"], np.float32)
    lib().vx_oracle_llama_forward(ctypes.byref(c), ctypes.byref(ws), kv.ctypes.data, token, pos,
                                  logits.ctypes.data)
    return logits


def ref_available() -> bool:
    return REF_LIB.exists()


def ref_lib():
    """The reference x86 dispatch library (built from the reference sources)
    bound with the plugin ABI signatures."""
    from vx_amd.runtime import DispatchLibrary
    # local scope: loaded beside this build's library, it must not supply the
    # vx_* symbols that outlined host kernels resolve in the global scope
    return DispatchLibrary(REF_LIB, hip=False, global_scope=False)
