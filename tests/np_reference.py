"""Independent numpy restatements used to pin the C oracle: matrix forms of
the same definitions, written differently from the oracle's loops so that a
dropped term, a wrong index or a transposed operand in either disagrees."""

from __future__ import annotations

import numpy as np

from vx_amd.abi import bf16_to_f32, f32_to_bf16


def bf16_round(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(np.asarray(x, np.float32)))


def attention_f64(q16, k16, v16, heads: int, kv_heads: int, scale: float, causal: bool):
    """softmax(scale q k^T) v per (batch, head), full matrices in f64.
    Returns (o [b, h, sq, d], lse [b, h, sq])."""
    q = bf16_to_f32(q16).astype(np.float64)
    k = bf16_to_f32(k16).astype(np.float64)
    v = bf16_to_f32(v16).astype(np.float64)
    group = heads // kv_heads
    k = np.repeat(k, group, axis=1)
    v = np.repeat(v, group, axis=1)
    sq, sk = q.shape[2], k.shape[2]
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    if causal:
        mask = np.arange(sk)[None, :] > (np.arange(sq)[:, None] + (sk - sq))
        s = np.where(mask[None, None], -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    empty = ~np.isfinite(m)
    m = np.where(empty, 0.0, m)
    p = np.exp(s - m)
    tot = p.sum(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore"):
        o = np.where(tot > 0, (p @ v) / np.where(tot > 0, tot, 1.0), 0.0)
        lse = np.where(tot[..., 0] > 0, (m + np.log(np.where(tot > 0, tot, 1.0)))[..., 0], -np.inf)
    return o, lse


def gemm_bf16_linalg(a16, b16) -> np.ndarray:
    """Per-step bf16 rounding of product and partial sum, vectorised over the
    output, k in order."""
    a = bf16_to_f32(a16)
    b = bf16_to_f32(b16)
    m, kk = a.shape
    n = b.shape[1]
    acc = np.zeros((m, n), np.float32)
    for p in range(kk):
        prod = bf16_round(np.outer(a[:, p], b[p, :]).astype(np.float32))
        acc = bf16_round(acc + prod)
    return f32_to_bf16(acc)


def llama_logits(cfg, model: dict, tokens) -> list[np.ndarray]:
    """Logits after each of `tokens` fed at positions 0.., restating
    reference examples/llama.vx:173-420 with the int8 weights (f32
    activations) and the shared RoPE table."""
    d, hd, L = cfg.dim, cfg.hidden_dim, cfg.n_layers
    hs, kvd = cfg.head_size, cfg.kv_dim
    kv_mul = cfg.n_heads // cfg.n_kv_heads
    kc = np.zeros((L, cfg.seq_len, kvd), np.float32)
    vc = np.zeros((L, cfg.seq_len, kvd), np.float32)

    def gemv(q, s, x):
        xb = np.asarray(x, np.float32).astype(np.float64)
        return (s.astype(np.float64) * (q.astype(np.float64) @ xb)).astype(np.float32)

    def rms(x, w):
        ss = np.float32(np.dot(x.astype(np.float64), x.astype(np.float64)))
        inv = np.float32(1.0) / np.sqrt(ss / np.float32(x.size) + np.float32(1e-5))
        return (w * (inv * x)).astype(np.float32)

    out = []
    for pos, tok in enumerate(tokens):
        x = model["tok_q"][tok].astype(np.float32) * model["tok_s"][tok]
        cos = model["rope"][pos, :, 0]
        sin = model["rope"][pos, :, 1]
        for l in range(L):
            xb = rms(x, model["rms_att"][l])
            q = gemv(model["wq_q"][l], model["wq_s"][l], xb)
            k = gemv(model["wk_q"][l], model["wk_s"][l], xb)
            v = gemv(model["wv_q"][l], model["wv_s"][l], xb)
            qh = q.reshape(cfg.n_heads, hs // 2, 2)
            kh = k.reshape(cfg.n_kv_heads, hs // 2, 2)
            q = np.stack([qh[..., 0] * cos - qh[..., 1] * sin,
                          qh[..., 0] * sin + qh[..., 1] * cos], -1).reshape(d)
            k = np.stack([kh[..., 0] * cos - kh[..., 1] * sin,
                          kh[..., 0] * sin + kh[..., 1] * cos], -1).reshape(kvd)
            kc[l, pos], vc[l, pos] = k, v
            att = np.empty(d, np.float32)
            for h in range(cfg.n_heads):
                hk = h // kv_mul
                qv = q[h * hs:(h + 1) * hs].astype(np.float64)
                keys = kc[l, :pos + 1, hk * hs:(hk + 1) * hs].astype(np.float64)
                vals = vc[l, :pos + 1, hk * hs:(hk + 1) * hs].astype(np.float64)
                sc = keys @ qv / np.sqrt(hs)
                p = np.exp(sc - sc.max())
                att[h * hs:(h + 1) * hs] = (p @ vals) / p.sum()
            x = x + gemv(model["wo_q"][l], model["wo_s"][l], att)
            xb = rms(x, model["rms_ffn"][l])
            h1 = gemv(model["w1_q"][l], model["w1_s"][l], xb)
            h3 = gemv(model["w3_q"][l], model["w3_s"][l], xb)
            hb = (h1 / (1.0 + np.exp(-h1.astype(np.float64)))).astype(np.float32) * h3
            x = x + gemv(model["w2_q"][l], model["w2_s"][l], hb)
        x = rms(x, model["rms_final"])
        out.append(gemv(model["tok_q"], model["tok_s"], x))
    return out
