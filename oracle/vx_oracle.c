/*
 * vx_oracle.c -- CPU restatement of the Vx CPU path (see vx_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the timed
 * CPU baseline, never the thing measured or shipped.
 *
 * Built with `gcc -O2 -ffp-contract=off` (oracle/Makefile): no fused
 * multiply-add and no reassociation, so each f32 operation rounds exactly
 * where the reference loop nest rounds.
 *
 * How each function is pinned (tests/test_oracle.py):
 *  - gemm_f32: bit-equal to the reference's own x86 dispatch library
 *    (oracle/_ref, built from runtime/x86_dispatch.cpp) on the same payload;
 *    the reference known answers 38 56 83 128 9 7 10
 *    (tests/backend/pass/gpu_matmul_roles.vx:47) and 19 50 197 4032
 *    (tests/backend/pass/gpu_matmul_dtypes.vx:45); identity times B.
 *  - gemm_f64: the same reference library (f64 route) and known answers.
 *  - gemm_bf16_f32_rows: bit-equal to the reference library's f32 GEMM of the
 *    bf16 values extended to f32 (the two are the same arithmetic); the exact
 *    small-integer case of benchmarks/gpu_gemm/*.vx; f64 point values.
 *  - gemm_bf16_bf16_linalg: brute force with explicit per-step rounding in
 *    numpy on tiny shapes; equals gemm_bf16_f32 rounded once where every
 *    partial sum is exact (small integers).
 *  - attention_rows: numpy matrix softmax in f64 on small shapes; closed
 *    forms: causal row 0 is V[0]; zero queries give the prefix mean of V and
 *    lse = ln(count); one key gives lse = scale * q.k.
 *  - gemv_i8 / gemv_i8_f64: numpy int64 exact dot for integer x; f64 matrix
 *    product otherwise.
 *  - quantize_rows: numpy round-half-even; the extremes map to +-127.
 *  - gemv_i8_f32in: numpy f64 matrix product (f32-activation form the
 *    decode uses).
 *  - llama_forward / llama_generate: a vectorised numpy restatement of
 *    examples/llama.vx on a tiny config, position by position (logits within
 *    f32 tolerance, identical tokens).
 */
#include "vx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

uint16_t vx_oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    return (uint16_t)((u >> 16) | 0x40);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float vx_oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float bf(uint16_t h) { return vx_oracle_bf16_to_f32(h); }

void vx_oracle_gemm_f32(const float *a, int64_t lda, const float *b,
                        int64_t ldb, float *c, int64_t ldc, int64_t m,
                        int64_t n, int64_t k) {
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (int64_t p = 0; p < k; ++p) {
        acc += a[i * lda + p] * b[p * ldb + j];
      }
      c[i * ldc + j] = acc;
    }
  }
}

void vx_oracle_gemm_f64(const double *a, int64_t lda, const double *b,
                        int64_t ldb, double *c, int64_t ldc, int64_t m,
                        int64_t n, int64_t k) {
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int64_t p = 0; p < k; ++p) {
        acc += a[i * lda + p] * b[p * ldb + j];
      }
      c[i * ldc + j] = acc;
    }
  }
}

void vx_oracle_gemm_bf16_f32_rows(const uint16_t *a, int64_t lda,
                                  const uint16_t *b, int64_t ldb, float *c,
                                  int64_t ldc, int64_t row0, int64_t rows,
                                  int64_t n, int64_t k) {
  /* Row-wise with the k loop outside j: per element the terms are still
   * added in k order, one rounding per multiply and per add, so the result
   * is the i, j, k loop's; this order streams B instead of striding it. */
  float *bf_row = (float *)malloc((size_t)n * sizeof(float));
  for (int64_t i = row0; i < row0 + rows; ++i) {
    float *out = c + i * ldc;
    for (int64_t j = 0; j < n; ++j) {
      out[j] = 0.0f;
    }
    for (int64_t p = 0; p < k; ++p) {
      const float av = bf(a[i * lda + p]);
      const uint16_t *brow = b + p * ldb;
      for (int64_t j = 0; j < n; ++j) {
        bf_row[j] = bf(brow[j]);
      }
      for (int64_t j = 0; j < n; ++j) {
        float prod = av * bf_row[j];
        out[j] = out[j] + prod;
      }
    }
  }
  free(bf_row);
}

void vx_oracle_gemm_bf16_bf16_linalg(const uint16_t *a, int64_t lda,
                                     const uint16_t *b, int64_t ldb,
                                     uint16_t *c, int64_t ldc, int64_t m,
                                     int64_t n, int64_t k) {
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      uint16_t acc = 0; /* +0.0 in bf16 */
      for (int64_t p = 0; p < k; ++p) {
        uint16_t prod =
            vx_oracle_f32_to_bf16(bf(a[i * lda + p]) * bf(b[p * ldb + j]));
        acc = vx_oracle_f32_to_bf16(bf(acc) + bf(prod));
      }
      c[i * ldc + j] = acc;
    }
  }
}

double vx_oracle_gemm_bf16_point_f64(const uint16_t *a, int64_t lda,
                                     const uint16_t *b, int64_t ldb, int64_t i,
                                     int64_t j, int64_t k) {
  double acc = 0.0;
  for (int64_t p = 0; p < k; ++p) {
    acc += (double)bf(a[i * lda + p]) * (double)bf(b[p * ldb + j]);
  }
  return acc;
}

void vx_oracle_attention_rows(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, int64_t batch, int64_t heads,
                              int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                              int64_t head_dim, double scale, int32_t causal,
                              const int64_t *rows, int64_t nrows, float *o_rows,
                              float *lse_rows) {
  double *s = (double *)malloc((size_t)(seq_k > 0 ? seq_k : 1) * sizeof(double));
  double *acc = (double *)malloc((size_t)head_dim * sizeof(double));
  const int64_t group = heads / kv_heads;
  for (int64_t r = 0; r < nrows; ++r) {
    const int64_t bi = rows[3 * r], hi = rows[3 * r + 1], qi = rows[3 * r + 2];
    const int64_t hk = hi / group;
    const uint16_t *qrow = q + ((bi * heads + hi) * seq_q + qi) * head_dim;
    const uint16_t *kbase = k + (bi * kv_heads + hk) * seq_k * head_dim;
    const uint16_t *vbase = v + (bi * kv_heads + hk) * seq_k * head_dim;
    int64_t last = seq_k - 1;
    if (causal) {
      last = qi + (seq_k - seq_q);
      if (last > seq_k - 1) {
        last = seq_k - 1;
      }
    }
    float *orow = o_rows + r * head_dim;
    if (last < 0) {
      for (int64_t d = 0; d < head_dim; ++d) {
        orow[d] = 0.0f;
      }
      lse_rows[r] = -INFINITY;
      continue;
    }
    double mx = -INFINITY;
    for (int64_t j = 0; j <= last; ++j) {
      double dot = 0.0;
      for (int64_t d = 0; d < head_dim; ++d) {
        dot += (double)bf(qrow[d]) * (double)bf(kbase[j * head_dim + d]);
      }
      s[j] = dot * scale;
      if (s[j] > mx) {
        mx = s[j];
      }
    }
    double sum = 0.0;
    for (int64_t d = 0; d < head_dim; ++d) {
      acc[d] = 0.0;
    }
    for (int64_t j = 0; j <= last; ++j) {
      const double p = exp(s[j] - mx);
      sum += p;
      for (int64_t d = 0; d < head_dim; ++d) {
        acc[d] += p * (double)bf(vbase[j * head_dim + d]);
      }
    }
    for (int64_t d = 0; d < head_dim; ++d) {
      orow[d] = (float)(acc[d] / sum);
    }
    lse_rows[r] = (float)(mx + log(sum));
  }
  free(s);
  free(acc);
}

void vx_oracle_gemv_i8(const int8_t *w, const float *scale, const uint16_t *x,
                       float *y, int64_t rows, int64_t cols, int64_t batch) {
  for (int64_t b = 0; b < batch; ++b) {
    const uint16_t *xb = x + b * cols;
    for (int64_t r = 0; r < rows; ++r) {
      const int8_t *wr = w + r * cols;
      float acc = 0.0f;
      for (int64_t c = 0; c < cols; ++c) {
        float prod = (float)wr[c] * bf(xb[c]);
        acc = acc + prod;
      }
      y[b * rows + r] = scale[r] * acc;
    }
  }
}

void vx_oracle_gemv_i8_f64(const int8_t *w, const float *scale,
                           const uint16_t *x, double *y, int64_t rows,
                           int64_t cols, int64_t batch) {
  for (int64_t b = 0; b < batch; ++b) {
    const uint16_t *xb = x + b * cols;
    for (int64_t r = 0; r < rows; ++r) {
      const int8_t *wr = w + r * cols;
      double acc = 0.0;
      for (int64_t c = 0; c < cols; ++c) {
        acc += (double)wr[c] * (double)bf(xb[c]);
      }
      y[b * rows + r] = (double)scale[r] * acc;
    }
  }
}

void vx_oracle_gemv_i8_f32in(const int8_t *w, const float *scale,
                             const float *x, float *y, int64_t rows,
                             int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const int8_t *wr = w + r * cols;
    float acc = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      float prod = (float)wr[c] * x[c];
      acc = acc + prod;
    }
    y[r] = scale[r] * acc;
  }
}

void vx_oracle_quantize_rows(const float *w, int64_t rows, int64_t cols,
                             int8_t *q, float *scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *wr = w + r * cols;
    float amax = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      float a = fabsf(wr[c]);
      if (a > amax) {
        amax = a;
      }
    }
    float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    scale[r] = s;
    for (int64_t c = 0; c < cols; ++c) {
      float t = nearbyintf(wr[c] / s); /* default rounding: half to even */
      if (t > 127.0f) {
        t = 127.0f;
      }
      if (t < -127.0f) {
        t = -127.0f;
      }
      q[r * cols + c] = (int8_t)t;
    }
  }
}

/* RMSNorm as reference examples/llama.vx:145-158: ss = sum x^2 in order,
 * ss/size + 1e-5, 1/sqrt, o = w * (ss * x). `o` may alias `x`. */
static void rmsnorm(float *o, const float *x, const float *weight, int size) {
  float ss = 0.0f;
  for (int j = 0; j < size; ++j) {
    ss = ss + x[j] * x[j];
  }
  float div = ss / (float)size;
  float add = div + 0.00001f;
  ss = 1.0f / sqrtf(add);
  for (int j = 0; j < size; ++j) {
    o[j] = weight[j] * (ss * x[j]);
  }
}

void vx_oracle_llama_forward(const vx_llama_config *cfg,
                             const vx_llama_weights *w, float *kv,
                             int32_t token, int32_t pos, float *logits) {
  const int dim = cfg->dim, hidden = cfg->hidden_dim;
  const int kv_dim = (cfg->dim * cfg->n_kv_heads) / cfg->n_heads;
  const int hs = dim / cfg->n_heads;
  const int kv_mul = cfg->n_heads / cfg->n_kv_heads;
  const int64_t layer_kv = (int64_t)cfg->seq_len * kv_dim;
  float *key_cache = kv;
  float *value_cache = kv + (int64_t)cfg->n_layers * layer_kv;

  float *x = (float *)malloc(sizeof(float) * dim);
  float *xb = (float *)malloc(sizeof(float) * dim);
  float *xb2 = (float *)malloc(sizeof(float) * dim);
  float *q = (float *)malloc(sizeof(float) * dim);
  float *kk = (float *)malloc(sizeof(float) * kv_dim);
  float *vv = (float *)malloc(sizeof(float) * kv_dim);
  float *h1 = (float *)malloc(sizeof(float) * hidden);
  float *h3 = (float *)malloc(sizeof(float) * hidden);

  /* 1. Embedding: the int8 row times its scale (reference
   * examples/llama.vx:182-185 reads the f32 table). */
  for (int i = 0; i < dim; ++i) {
    x[i] = (float)w->tok_q[(int64_t)token * dim + i] * w->tok_s[token];
  }

  for (int l = 0; l < cfg->n_layers; ++l) {
    /* 2.1 attention RMSNorm */
    rmsnorm(xb, x, w->rms_att + (int64_t)l * dim, dim);
    /* 2.2 Q, K, V: int8 weights, f32 activations (reference :191-233 is the
     * f32 `@` with M = 1). */
    vx_oracle_gemv_i8_f32in(w->wq_q + (int64_t)l * dim * dim,
                            w->wq_s + (int64_t)l * dim, xb, q, dim, dim);
    vx_oracle_gemv_i8_f32in(w->wk_q + (int64_t)l * kv_dim * dim,
                            w->wk_s + (int64_t)l * kv_dim, xb, kk, kv_dim, dim);
    vx_oracle_gemv_i8_f32in(w->wv_q + (int64_t)l * kv_dim * dim,
                            w->wv_s + (int64_t)l * kv_dim, xb, vv, kv_dim, dim);
    /* 2.3 RoPE on (even, odd) pairs (reference :235-264); the angle's cos and
     * sin come from the shared table. */
    for (int i = 0; i < dim; i += 2) {
      const int hd = i % hs;
      const float fcr = w->rope[((int64_t)pos * (hs / 2) + hd / 2) * 2];
      const float fci = w->rope[((int64_t)pos * (hs / 2) + hd / 2) * 2 + 1];
      float q0 = q[i], q1 = q[i + 1];
      q[i] = q0 * fcr - q1 * fci;
      q[i + 1] = q0 * fci + q1 * fcr;
      if (i < kv_dim) {
        float k0 = kk[i], k1 = kk[i + 1];
        kk[i] = k0 * fcr - k1 * fci;
        kk[i + 1] = k0 * fci + k1 * fcr;
      }
    }
    /* 2.4 KV cache (reference :266-273) */
    float *kc = key_cache + (int64_t)l * layer_kv;
    float *vc = value_cache + (int64_t)l * layer_kv;
    memcpy(kc + (int64_t)pos * kv_dim, kk, sizeof(float) * kv_dim);
    memcpy(vc + (int64_t)pos * kv_dim, vv, sizeof(float) * kv_dim);
    /* 2.5 attention with online softmax (reference :275-325) */
    for (int h = 0; h < cfg->n_heads; ++h) {
      const int qo = h * hs;
      const int ko = (h / kv_mul) * hs;
      float m = -999999.0f;
      float lsum = 0.0f;
      for (int i = 0; i < hs; ++i) {
        xb[qo + i] = 0.0f;
      }
      for (int t = 0; t <= pos; ++t) {
        float score = 0.0f;
        const float *krow = kc + (int64_t)t * kv_dim + ko;
        for (int i = 0; i < hs; ++i) {
          score = score + q[qo + i] * krow[i];
        }
        score = score / sqrtf((float)hs);
        float m_new = m;
        if (score > m) {
          m_new = score;
        }
        const float corr = expf(m - m_new);
        const float e = expf(score - m_new);
        lsum = lsum * corr + e;
        const float *vrow = vc + (int64_t)t * kv_dim + ko;
        for (int i = 0; i < hs; ++i) {
          xb[qo + i] = xb[qo + i] * corr + e * vrow[i];
        }
        m = m_new;
      }
      const float inv = 1.0f / lsum;
      for (int i = 0; i < hs; ++i) {
        xb[qo + i] = xb[qo + i] * inv;
      }
    }
    /* 2.6 output projection and residual (reference :327-344) */
    vx_oracle_gemv_i8_f32in(w->wo_q + (int64_t)l * dim * dim,
                            w->wo_s + (int64_t)l * dim, xb, xb2, dim, dim);
    for (int i = 0; i < dim; ++i) {
      x[i] = x[i] + xb2[i];
    }
    /* 2.7-2.8 FFN RMSNorm, W1/W3, SwiGLU, W2, residual (reference :346-395) */
    rmsnorm(xb, x, w->rms_ffn + (int64_t)l * dim, dim);
    vx_oracle_gemv_i8_f32in(w->w1_q + (int64_t)l * hidden * dim,
                            w->w1_s + (int64_t)l * hidden, xb, h1, hidden, dim);
    vx_oracle_gemv_i8_f32in(w->w3_q + (int64_t)l * hidden * dim,
                            w->w3_s + (int64_t)l * hidden, xb, h3, hidden, dim);
    for (int i = 0; i < hidden; ++i) {
      float val = h1[i];
      float neg = 0.0f - val;
      val = val * (1.0f / (1.0f + expf(neg)));
      val = val * h3[i];
      h1[i] = val;
    }
    vx_oracle_gemv_i8_f32in(w->w2_q + (int64_t)l * dim * hidden,
                            w->w2_s + (int64_t)l * dim, h1, xb, dim, hidden);
    for (int i = 0; i < dim; ++i) {
      x[i] = x[i] + xb[i];
    }
  }
  /* 3-4. final RMSNorm in place, classifier (reference :397-417) */
  rmsnorm(x, x, w->rms_final, dim);
  vx_oracle_gemv_i8_f32in(w->tok_q, w->tok_s, x, logits, cfg->vocab_size, dim);

  free(x);
  free(xb);
  free(xb2);
  free(q);
  free(kk);
  free(vv);
  free(h1);
  free(h3);
}

int32_t vx_oracle_llama_generate(const vx_llama_config *cfg,
                                 const vx_llama_weights *w,
                                 const int32_t *prompt, int32_t n_prompt,
                                 int32_t n_steps, int32_t *out_tokens,
                                 float *out_margin) {
  if (n_prompt < 1 || n_steps < 0 || n_prompt + n_steps > cfg->seq_len + 1 ||
      cfg->dim % cfg->n_heads != 0 || cfg->n_heads % cfg->n_kv_heads != 0) {
    return -1;
  }
  const int kv_dim = (cfg->dim * cfg->n_kv_heads) / cfg->n_heads;
  float *kv = (float *)calloc((size_t)2 * cfg->n_layers * cfg->seq_len * kv_dim,
                              sizeof(float));
  float *logits = (float *)malloc(sizeof(float) * cfg->vocab_size);
  int32_t token = prompt[0];
  int32_t made = 0;
  for (int32_t pos = 0; made < n_steps; ++pos) {
    vx_oracle_llama_forward(cfg, w, kv, token, pos, logits);
    /* argmax, strict '>' so the lowest index wins a tie (reference
     * examples/llama.vx:160-171) */
    int32_t best = 0;
    float best_v = logits[0];
    for (int32_t i = 1; i < cfg->vocab_size; ++i) {
      if (logits[i] > best_v) {
        best = i;
        best_v = logits[i];
      }
    }
    if (pos + 1 < n_prompt) {
      token = prompt[pos + 1];
      continue;
    }
    float second = -INFINITY;
    for (int32_t i = 0; i < cfg->vocab_size; ++i) {
      if (i != best && logits[i] > second) {
        second = logits[i];
      }
    }
    out_tokens[made] = best;
    if (out_margin) {
      out_margin[made] = best_v - second;
    }
    ++made;
    token = best;
  }
  free(kv);
  free(logits);
  return 0;
}
