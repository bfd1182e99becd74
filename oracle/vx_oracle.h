/*
 * vx_oracle.h -- CPU restatement of the Vx CPU path for the tensor hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load this library, and only as the checker or
 * the timed CPU baseline. The product path (libvx_hip_dispatch.so) never
 * links, loads or calls it.
 *
 * Each function names the reference code it restates. Pinning (what checks
 * each function against something other than itself) is listed per function
 * in vx_oracle.c's header.
 */
#ifndef VX_ORACLE_H
#define VX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* C = A B, f32, loop order i, j, k, f32 accumulator from 0, one multiply and
 * one add per term (reference runtime/host_dispatch_common.h:65-79). */
void vx_oracle_gemm_f32(const float *a, int64_t lda, const float *b,
                        int64_t ldb, float *c, int64_t ldc, int64_t m,
                        int64_t n, int64_t k);
/* The same loop in f64. */
void vx_oracle_gemm_f64(const double *a, int64_t lda, const double *b,
                        int64_t ldb, double *c, int64_t ldc, int64_t m,
                        int64_t n, int64_t k);
/* bf16 x bf16 -> f32 as the outlined linalg.fill + linalg.matmul computes it
 * (reference src/codegen/flat/emit/tensor.rs:1600-1647): out starts at 0;
 * each term extends both operands to f32, multiplies in f32, adds into out in
 * f32; k in order. Rows [row0, row0 + rows) of C only (C points at row 0). */
void vx_oracle_gemm_bf16_f32_rows(const uint16_t *a, int64_t lda,
                                  const uint16_t *b, int64_t ldb, float *c,
                                  int64_t ldc, int64_t row0, int64_t rows,
                                  int64_t n, int64_t k);
/* bf16 x bf16 -> bf16 with linalg.matmul's element type semantics: the
 * product and each partial sum are rounded to bf16 (round to nearest even). */
void vx_oracle_gemm_bf16_bf16_linalg(const uint16_t *a, int64_t lda,
                                     const uint16_t *b, int64_t ldb,
                                     uint16_t *c, int64_t ldc, int64_t m,
                                     int64_t n, int64_t k);
/* f64 dot of row i of A (bf16) with column j of B (bf16): the exact value
 * the f32 results are compared against at sampled points. */
double vx_oracle_gemm_bf16_point_f64(const uint16_t *a, int64_t lda,
                                     const uint16_t *b, int64_t ldb, int64_t i,
                                     int64_t j, int64_t k);

/* Softmax attention forward, f64 accumulation, two passes (max, then sums),
 * as the reference's CPU checks of its attention kernels compute it
 * (tests/optimizations/pass/std_nn_kernels_match_loops_on_the_cpu.vx:347-390;
 * benchmarks/apple_gpu_mlir_kernels/flash_attention.vx:309-336). Layout and
 * masking as include/vx_hip_ops.h vx_nn_flash_attention_fwd_bf16. Computes
 * only the `nrows` rows listed as (b, h, i) triples in `rows`; o_rows gets
 * head_dim f32 values per listed row, lse_rows one f32 each. A row that sees
 * no key gets o = 0 and lse = -inf. */
void vx_oracle_attention_rows(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, int64_t batch, int64_t heads,
                              int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                              int64_t head_dim, double scale, int32_t causal,
                              const int64_t *rows, int64_t nrows, float *o_rows,
                              float *lse_rows);

/* y[b, r] = scale[r] * sum_c w[r, c] * x[b, c]; sum in f32, c in order, then
 * one multiply by the scale (the scale-after-dot structure of reference
 * stdlib/std/nn.vx:1338-1344). x is bf16. */
void vx_oracle_gemv_i8(const int8_t *w, const float *scale, const uint16_t *x,
                       float *y, int64_t rows, int64_t cols, int64_t batch);
/* The same in f64 (the exact value up to the final rounding). */
void vx_oracle_gemv_i8_f64(const int8_t *w, const float *scale,
                           const uint16_t *x, double *y, int64_t rows,
                           int64_t cols, int64_t batch);

/* y[r] = scale[r] * sum_c w[r, c] * x[c] with an f32 activation vector:
 * the weight-only int8 linear of the decode step (activations stay f32, as
 * in reference examples/llama.vx). */
void vx_oracle_gemv_i8_f32in(const int8_t *w, const float *scale,
                             const float *x, float *y, int64_t rows,
                             int64_t cols);

/* Per-output-row symmetric int8 quantization: scale = max|w| / 127 (1 for an
 * all-zero row), q = round-half-even(w / scale) clamped to [-127, 127]. */
void vx_oracle_quantize_rows(const float *w, int64_t rows, int64_t cols,
                             int8_t *q, float *scale);

/* llama2.c-layout model in int8 with per-row f32 scales (matrices stored
 * [out][in]; the classifier is the token embedding table). */
typedef struct {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} vx_llama_config;

typedef struct {
  const int8_t *tok_q;      /* [vocab, dim] */
  const float *tok_s;       /* [vocab] */
  const float *rms_att;     /* [layers, dim] */
  const int8_t *wq_q;       /* [layers, dim, dim] */
  const float *wq_s;        /* [layers, dim] */
  const int8_t *wk_q;       /* [layers, kv_dim, dim] */
  const float *wk_s;        /* [layers, kv_dim] */
  const int8_t *wv_q;       /* [layers, kv_dim, dim] */
  const float *wv_s;        /* [layers, kv_dim] */
  const int8_t *wo_q;       /* [layers, dim, dim] */
  const float *wo_s;        /* [layers, dim] */
  const float *rms_ffn;     /* [layers, dim] */
  const int8_t *w1_q;       /* [layers, hidden, dim] */
  const float *w1_s;        /* [layers, hidden] */
  const int8_t *w2_q;       /* [layers, dim, hidden] */
  const float *w2_s;        /* [layers, dim] */
  const int8_t *w3_q;       /* [layers, hidden, dim] */
  const float *w3_s;        /* [layers, hidden] */
  const float *rms_final;   /* [dim] */
  const float *rope;        /* [seq_len, head_size/2, 2] = (cos, sin) */
} vx_llama_weights;

/* Greedy decode: feed prompt[0..n_prompt), then generate n_steps tokens,
 * each the argmax of the previous position's logits. Writes the generated
 * tokens to out_tokens[n_steps] and, per generated token, the gap between
 * the best and the second-best logit to out_margin (may be NULL). Returns 0,
 * or -1 when the arguments do not fit the config. Follows reference
 * examples/llama.vx:145-420 with int8 weights (per-row scales) and f32
 * activations; the embedding is the int8 row times its scale and the
 * RoPE angles come from the `rope` table. */
int32_t vx_oracle_llama_generate(const vx_llama_config *cfg,
                                 const vx_llama_weights *w,
                                 const int32_t *prompt, int32_t n_prompt,
                                 int32_t n_steps, int32_t *out_tokens,
                                 float *out_margin);

/* One position of the forward pass; logits[vocab] out. `kv` holds
 * 2 * layers * seq_len * kv_dim floats (keys, then values) and persists
 * between positions. */
void vx_oracle_llama_forward(const vx_llama_config *cfg,
                             const vx_llama_weights *w, float *kv,
                             int32_t token, int32_t pos, float *logits);

/* f32 -> bf16 round to nearest even (NaN stays quiet NaN), and back. */
uint16_t vx_oracle_f32_to_bf16(float f);
float vx_oracle_bf16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif

#endif /* VX_ORACLE_H */
