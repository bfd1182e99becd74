"""Greedy int8 decode on the GPU through vx_llama_i8_* (include/vx_hip_ops.h).

    model = LlamaI8(lib, cfg, weights)     # upload (weights from vx_amd.llama)
    tokens, margin = model.generate(prompt, n_steps)
    logits = model.logits(tokens)          # per position, for parity checks
"""

from __future__ import annotations

import ctypes
import time

import numpy as np

from .llama import CONFIG_DECODE, LlamaConfig, make_model, make_prompt

WEIGHT_FIELDS = ("tok_q", "tok_s", "rms_att", "wq_q", "wq_s", "wk_q", "wk_s", "wv_q", "wv_s",
                 "wo_q", "wo_s", "rms_ffn", "w1_q", "w1_s", "w2_q", "w2_s", "w3_q", "w3_s",
                 "rms_final", "rope")
GRAPH = 1


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")]


class _Weights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in WEIGHT_FIELDS]


class LlamaI8:
    def __init__(self, lib, cfg: LlamaConfig, weights: dict, topo: int = 500):
        self.lib, self.cfg = lib, cfg
        c = _Config(**cfg.as_dict())
        w = _Weights()
        keep = []
        for name in WEIGHT_FIELDS:
            arr = np.ascontiguousarray(weights[name])
            keep.append(arr)
            setattr(w, name, arr.ctypes.data)
        self.handle = lib.lib.vx_llama_i8_create(ctypes.byref(c), ctypes.byref(w), topo)
        if not self.handle:
            raise RuntimeError("vx_llama_i8_create refused the model")

    def generate(self, prompt, n_steps: int, graph: bool = True):
        prompt = np.ascontiguousarray(prompt, np.int32)
        toks = np.empty(n_steps, np.int32)
        margin = np.empty(n_steps, np.float32)
        rc = self.lib.lib.vx_llama_i8_generate(self.handle, prompt.ctypes.data, len(prompt), n_steps,
                                               toks.ctypes.data, margin.ctypes.data,
                                               GRAPH if graph else 0)
        if rc != 0:
            raise RuntimeError(f"vx_llama_i8_generate returned {rc}")
        return toks, margin

    def logits(self, tokens) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((len(tokens), self.cfg.vocab_size), np.float32)
        rc = self.lib.lib.vx_llama_i8_logits(self.handle, tokens.ctypes.data, len(tokens),
                                             out.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"vx_llama_i8_logits returned {rc}")
        return out

    def close(self) -> None:
        if self.handle:
            self.lib.lib.vx_llama_i8_destroy(self.handle)
            self.handle = None


def bench(lib, timer, n_prompt: int = 16, n_steps: int = 256, reps: int = 3) -> dict:
    """dim 768 / 12 layers, int8, bs=1, 16-token prompt
    then 256 greedy tokens. Reports tokens per second of the whole generate
    call (prompt positions included in the time) and the weight bytes each
    position streams."""
    cfg = CONFIG_DECODE
    model = LlamaI8(lib, cfg, make_model(cfg, seed=0))
    prompt = make_prompt(cfg, n=n_prompt, seed=1)
    model.generate(prompt, 8)  # warm: graph instantiation, first-touch
    times = []
    toks = None
    for _ in range(reps):
        t0 = time.perf_counter()
        toks, margin = model.generate(prompt, n_steps)
        times.append(time.perf_counter() - t0)
    model.close()
    best = min(times)
    positions = n_prompt + n_steps - 1
    wbytes = cfg.int8_weight_bytes()
    return dict(config="dim 768, 12 layers, int8 weights, bs=1, 16-token prompt + 256 greedy tokens",
                tok_per_s=n_steps / best, positions_per_s=positions / best,
                ms_per_position=best / positions * 1e3, runs_s=times,
                weight_bytes_per_position=wbytes,
                weight_gbs=wbytes * positions / best / 1e9,
                first_tokens=[int(t) for t in toks[:8]])
