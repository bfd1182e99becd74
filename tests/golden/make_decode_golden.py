"""Writes tests/golden/decode_config4.json: the CPU oracle's greedy tokens
for BASELINE config 4 (dim 768, 12 layers, 12 heads, hidden 2048, vocab
32000, seq 1024; int8 weights from vx_amd.llama.make_model(seed=0); prompt
vx_amd.llama.make_prompt(n=16, seed=1); 256 generated tokens), with each
token's logit lead over the runner-up. The oracle is oracle/vx_oracle.c
(test infrastructure); nothing of the reference is imported.

    python tests/golden/make_decode_golden.py
"""

import json
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402
from vx_amd.llama import CONFIG_DECODE, make_model, make_prompt  # noqa: E402


# Positions whose top-16 logits are kept: every 16th of the 271, the last
# prompt position and the last position.
PROBES = tuple(sorted(set(range(0, 271, 16)) | {15, 143, 270}))


def main(n_steps: int = 256) -> None:
    cfg = CONFIG_DECODE
    model = make_model(cfg, seed=0)
    prompt = make_prompt(cfg, n=16, seed=1)
    t0 = time.perf_counter()
    toks, margin = oracle.llama_generate(cfg.as_dict(), model, prompt, n_steps)
    dt = time.perf_counter() - t0
    # Logits at the probed positions of the same sequence: the top 16
    # (index, value) pairs, for a check stronger than the argmax alone; and
    # at every position the mean and standard deviation of all the logits,
    # which a wrong term anywhere in the vocabulary would move.
    import numpy as np
    seq = [int(t) for t in prompt] + [int(t) for t in toks[:-1]]
    kv = np.zeros(2 * cfg.n_layers * cfg.seq_len * cfg.kv_dim, np.float32)
    probes = {}
    moments = []
    for pos, tok in enumerate(seq):
        logits = oracle.llama_forward(cfg.as_dict(), model, kv, tok, pos)
        l64 = logits.astype(np.float64)
        moments.append([float(l64.mean()), float(l64.std())])
        if pos in PROBES:
            top = np.argsort(-logits, kind="stable")[:16]
            probes[str(pos)] = {"index": [int(i) for i in top],
                                "value": [float(logits[i]) for i in top]}
    out = {"config": cfg.as_dict(), "model_seed": 0, "prompt_seed": 1,
           "prompt": [int(t) for t in prompt], "n_steps": n_steps,
           "tokens": [int(t) for t in toks], "margins": [float(m) for m in margin],
           "logit_probes": probes, "logit_moments": moments,
           "oracle_seconds": round(dt, 1)}
    (HERE / "decode_config4.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"{n_steps} tokens in {dt:.1f} s; min margin {float(margin.min()):.3g}")


if __name__ == "__main__":
    main()
