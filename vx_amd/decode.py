"""Greedy int8 decode on the GPU through vx_llama_i8_* (include/vx_hip_ops.h).

    model = LlamaI8(lib, cfg, weights)     # upload (weights from vx_amd.llama)
    tokens, margin = model.generate(prompt, n_steps)
    logits = model.logits(tokens)          # per position, for parity checks
    cfg, weights = read_model(lib, path)   # a llama2.c checkpoint or VXQ8 file
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


def _shapes(cfg: LlamaConfig) -> dict[str, tuple[tuple[int, ...], type]]:
    d, h, kv, L, hs = cfg.dim, cfg.hidden_dim, cfg.kv_dim, cfg.n_layers, cfg.head_size
    i8, f32 = np.int8, np.float32
    return {
        "tok_q": ((cfg.vocab_size, d), i8), "tok_s": ((cfg.vocab_size,), f32),
        "rms_att": ((L, d), f32),
        "wq_q": ((L, d, d), i8), "wq_s": ((L, d), f32),
        "wk_q": ((L, kv, d), i8), "wk_s": ((L, kv), f32),
        "wv_q": ((L, kv, d), i8), "wv_s": ((L, kv), f32),
        "wo_q": ((L, d, d), i8), "wo_s": ((L, d), f32),
        "rms_ffn": ((L, d), f32),
        "w1_q": ((L, h, d), i8), "w1_s": ((L, h), f32),
        "w2_q": ((L, d, h), i8), "w2_s": ((L, d), f32),
        "w3_q": ((L, h, d), i8), "w3_s": ((L, h), f32),
        "rms_final": ((d,), f32), "rope": ((cfg.seq_len, hs // 2, 2), f32),
    }


def read_model(lib, path) -> tuple[LlamaConfig, dict[str, np.ndarray]]:
    """Read a llama2.c checkpoint (quantized on the way in) or a VXQ8 file
    through vx_llama_i8_read; returns the config and numpy copies of the
    weights, keyed as make_model's."""
    c = _Config()
    h = ctypes.c_void_p()
    rc = lib.lib.vx_llama_i8_read(str(path).encode(), ctypes.byref(c), ctypes.byref(h))
    if rc != 0:
        raise OSError(rc, f"vx_llama_i8_read refused {path}")
    try:
        cfg = LlamaConfig(**{n: getattr(c, n) for n, _ in _Config._fields_})
        w = _Weights.from_address(lib.lib.vx_llama_i8_host_weights(h))
        out = {}
        for name, (shape, dtype) in _shapes(cfg).items():
            n = int(np.prod(shape))
            buf = (ctypes.c_char * (n * np.dtype(dtype).itemsize)).from_address(getattr(w, name))
            out[name] = np.frombuffer(bytes(buf), dtype=dtype).reshape(shape)
    finally:
        lib.lib.vx_llama_i8_host_free(h)
    return cfg, out


def save_model(lib, path, cfg: LlamaConfig, weights: dict) -> None:
    """Write weights (keyed as make_model's) as a VXQ8 file."""
    c = _Config(**cfg.as_dict())
    w = _Weights()
    keep = []
    for name in WEIGHT_FIELDS:
        arr = np.ascontiguousarray(weights[name])
        keep.append(arr)
        setattr(w, name, arr.ctypes.data)
    rc = lib.lib.vx_llama_i8_save(str(path).encode(), ctypes.byref(c), ctypes.byref(w))
    if rc != 0:
        raise OSError(rc, f"vx_llama_i8_save refused {path}")


def write_checkpoint(path, cfg: LlamaConfig, f32: dict[str, np.ndarray], rope_arrays: bool = True) -> None:
    """A llama2.c checkpoint of f32 weights (keys tok, rms_att, wq, wk, wv,
    wo, rms_ffn, w1, w2, w3, rms_final): the seven-int header, the arrays in
    the reference's order, and (as llama2.c writes them) the RoPE cos/sin
    arrays it leaves unread."""
    hdr = np.array([cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
                    cfg.vocab_size, cfg.seq_len], np.int32)
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        for name in ("tok", "rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3",
                     "rms_final"):
            f.write(np.ascontiguousarray(f32[name], np.float32).tobytes())
        if rope_arrays:
            half = cfg.seq_len * cfg.head_size // 2
            f.write(np.zeros(2 * half, np.float32).tobytes())


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
    call (prompt positions included in the time) with the step replayed as
    a hipGraph (`tok_per_s_graph`) and launched kernel by kernel
    (`tok_per_s_eager`); `tok_per_s` is the faster of the two (`mode`
    names it; both produce the same tokens, which the run asserts). Also
    the weight bytes each position streams."""
    cfg = CONFIG_DECODE
    model = LlamaI8(lib, cfg, make_model(cfg, seed=0))
    prompt = make_prompt(cfg, n=n_prompt, seed=1)
    model.generate(prompt, n_steps)  # warm: graph instantiation, first-touch
    model.generate(prompt, n_steps, graph=False)
    times, eager = [], []
    toks = None
    for _ in range(reps):
        t0 = time.perf_counter()
        toks, margin = model.generate(prompt, n_steps)
        times.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        toks_e, _ = model.generate(prompt, n_steps, graph=False)
        eager.append(time.perf_counter() - t0)
        assert np.array_equal(toks, toks_e), "graph and eager steps disagree"
    model.close()
    graph_best, eager_best = min(times), min(eager)
    best = min(graph_best, eager_best)
    positions = n_prompt + n_steps - 1
    wbytes = cfg.int8_weight_bytes()
    kv_total = sum(cfg.kv_bytes(p) for p in range(positions))
    step_bytes = wbytes * positions + kv_total
    return dict(config="dim 768, 12 layers, int8 weights, bs=1, 16-token prompt + 256 greedy tokens",
                tok_per_s=n_steps / best, positions_per_s=positions / best,
                ms_per_position=best / positions * 1e3,
                mode="graph" if graph_best <= eager_best else "eager",
                tok_per_s_graph=n_steps / graph_best, runs_graph_s=times,
                tok_per_s_eager=n_steps / eager_best, runs_eager_s=eager,
                weight_bytes_per_position=wbytes,
                weight_gbs=wbytes * positions / best / 1e9,
                kv_bytes_per_position=kv_total / positions,
                bytes_gbs=step_bytes / best / 1e9,
                first_tokens=[int(t) for t in toks[:8]])


def main(argv=None) -> int:
    """Generate from the BASELINE config-4 model (random N(0, 0.02) weights,
    seed 0; 16-token prompt, seed 1) and print tokens per second: the
    program a kernel trace of the decode step profiles.

        python -m vx_amd.decode [--steps N] [--eager] [--lib PATH]
    """
    import argparse

    from .runtime import DispatchLibrary, LIB_PATH

    ap = argparse.ArgumentParser(description=main.__doc__.splitlines()[0])
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--eager", action="store_true",
                    help="launch the step's kernels one by one instead of replaying a hipGraph")
    ap.add_argument("--lib", default=str(LIB_PATH))
    ns = ap.parse_args(argv)
    lib = DispatchLibrary(ns.lib)
    cfg = CONFIG_DECODE
    model = LlamaI8(lib, cfg, make_model(cfg, seed=0))
    try:
        prompt = make_prompt(cfg, n=16, seed=1)
        model.generate(prompt, 4, graph=not ns.eager)  # warm
        t0 = time.perf_counter()
        toks, _ = model.generate(prompt, ns.steps, graph=not ns.eager)
        dt = time.perf_counter() - t0
    finally:
        model.close()
    mode = "eager" if ns.eager else "graph"
    print(f"{ns.steps} tokens ({mode}) in {dt * 1e3:.2f} ms: {ns.steps / dt:.0f} tok/s; "
          f"first tokens {[int(t) for t in toks[:8]]}", flush=True)
    return 0


if __name__ == "__main__":
    import sys

    sys.exit(main())
