"""Synthetic Llama-2-style decoder weights for the int8 decode path.

The model is the one reference examples/llama.vx runs (llama2.c layout:
matrices stored [out][in], the classifier shares the token embedding table,
RMSNorm eps 1e-5, RoPE base 10000), with random-init weights since there is
no checkpoint here: every matrix N(0, 0.02) in f32 from a seed, RMSNorm
weights 1, then each matrix quantized per output row to int8 with an f32
scale (scale = max|w| / 127, q = round-half-even(w / scale)).

The RoPE angle table is computed once on the host from the reference's
formula (pos * 10000^(-i / head_size) in f32, tests/modules/llama_rt.vx:82-85)
and handed to both the GPU path and the CPU checker, so neither side's libm
decides a token.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass

import math

import numpy as np


@dataclass(frozen=True)
class LlamaConfig:
    dim: int = 768
    hidden_dim: int = 2048
    n_layers: int = 12
    n_heads: int = 12
    n_kv_heads: int = 12
    vocab_size: int = 32000
    seq_len: int = 1024

    @property
    def head_size(self) -> int:
        return self.dim // self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.dim * self.n_kv_heads // self.n_heads

    def as_dict(self) -> dict:
        return asdict(self)

    def int8_weight_bytes(self) -> int:
        """Weight bytes one token reads: every int8 matrix plus its scales."""
        d, h, kv, L = self.dim, self.hidden_dim, self.kv_dim, self.n_layers
        per_layer = d * d * 2 + kv * d * 2 + h * d * 3
        scales = 4 * (L * (d * 2 + kv * 2 + h * 2 + d) + self.vocab_size)
        norms = 4 * (L * 2 * d + d)
        return L * per_layer + self.vocab_size * d + scales + norms

    def kv_bytes(self, pos: int) -> int:
        """KV-cache bytes the step at position `pos` moves: every layer reads
        the f32 key and value rows 0..pos and writes row pos of each."""
        return self.n_layers * 2 * self.kv_dim * 4 * (pos + 2)


# dim 768, 12 layers, 12 heads, SwiGLU 2048, vocab 32000.
CONFIG_DECODE = LlamaConfig()
# A small model with grouped-query attention for CPU-sized checks.
CONFIG_TINY = LlamaConfig(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                          vocab_size=256, seq_len=64)


def quantize_rows(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int8: scale = max|w| / 127 (1 for a zero row),
    q = round-half-even(w / scale) in [-127, 127]."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.abs(w).max(axis=-1)
    scale = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.rint(w / scale[..., None]).clip(-127, 127).astype(np.int8)
    return q, scale


def rope_inv_freq(head_size: int) -> np.ndarray:
    """10000^(-i/hs) for even i as the reference's f32 `powf` gives it
    (reference tests/modules/llama_rt.vx:82-85; stdlib/core/num.vx:2476-2479
    documents powf as correctly rounded): the exponent -(i as f32) / (hs as
    f32) in f32, the power in double (glibc's pow, under 1 ulp of double),
    rounded to f32 once."""
    e = [float(-np.float32(i) / np.float32(head_size)) for i in range(0, head_size, 2)]
    return np.array([math.pow(10000.0, x) for x in e], np.float64).astype(np.float32)


def rope_table(cfg: LlamaConfig, positions: int | None = None) -> np.ndarray:
    """[positions, head_size / 2, 2] of (cos, sin) of the f32 angle
    (pos as f32) * rope_inv_freq, as reference examples/llama.vx:244-246
    computes them: f32 `cos`/`sin`, which reference stdlib/core/num.vx:2434-2442
    documents as correctly rounded. Each is the double cos/sin of the f32
    angle (glibc, under 1 ulp of double) rounded to f32 once; a CPU test
    checks every entry against a 60-digit evaluation where the rounding is
    close."""
    positions = cfg.seq_len if positions is None else positions
    hs = cfg.head_size
    inv = rope_inv_freq(hs)
    pos = np.arange(positions, dtype=np.float32)[:, None]
    ang = (pos * inv[None, :]).astype(np.float32).astype(np.float64)
    cos = np.vectorize(math.cos, otypes=[np.float64])(ang)
    sin = np.vectorize(math.sin, otypes=[np.float64])(ang)
    return np.stack([cos, sin], axis=-1).astype(np.float32)


def make_model(cfg: LlamaConfig, seed: int = 0) -> dict[str, np.ndarray]:
    """Random-init int8 model, keyed as the CPU checker's weight struct."""
    rng = np.random.default_rng(seed)
    d, h, kv, L = cfg.dim, cfg.hidden_dim, cfg.kv_dim, cfg.n_layers

    def mat(*shape):
        return rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)

    m: dict[str, np.ndarray] = {}
    m["tok_q"], m["tok_s"] = quantize_rows(mat(cfg.vocab_size, d))
    for name, (rows, cols) in (("wq", (d, d)), ("wk", (kv, d)), ("wv", (kv, d)), ("wo", (d, d)),
                               ("w1", (h, d)), ("w2", (d, h)), ("w3", (h, d))):
        q, s = quantize_rows(mat(L, rows, cols))
        m[f"{name}_q"], m[f"{name}_s"] = q, s
    m["rms_att"] = np.ones((L, d), np.float32)
    m["rms_ffn"] = np.ones((L, d), np.float32)
    m["rms_final"] = np.ones(d, np.float32)
    m["rope"] = rope_table(cfg)
    return {k: np.ascontiguousarray(v) for k, v in m.items()}


def make_prompt(cfg: LlamaConfig, n: int = 16, seed: int = 1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, cfg.vocab_size, size=n, dtype=np.int32)
