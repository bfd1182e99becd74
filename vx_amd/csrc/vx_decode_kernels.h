/*
 * vx_decode_kernels.h -- launchers of the decode-step kernels
 * (kernels/decode.hip), driven by decode.cpp. Every pointer is device
 * memory; `pos` is the device-resident position of the step.
 */
#ifndef VX_AMD_DECODE_KERNELS_H
#define VX_AMD_DECODE_KERNELS_H

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vxk {

/* Best and runner-up logit of a workgroup's rows (classifier epilogue). */
struct StepBest {
  float v1;
  int i1;
  float v2;
};

/* The token of a position: the prompt's while it lasts, else the argmax
 * over the previous step's classifier candidates (lowest index on a tie),
 * recorded in out_tokens / out_margin from position n_prompt on. */
struct StepTokenArgs {
  const StepBest *cand; /* ncand entries left by the previous classifier */
  int ncand;
  const int *prompt;
  int n_prompt;
  int *out_tokens;
  float *out_margin;
  int out_cap;
  const int8_t *tok_q; /* embedding table [vocab, dim], int8 rows */
  const float *tok_s;  /* and their scales */
  int vocab;
};

/* Position 0 (step_start) and the token after the last step (step_record). */
struct StepArgmaxArgs {
  StepTokenArgs tok;
  int *pos;
};

struct StepGemvArgs {
  const int8_t *w;     /* [rows, cols] */
  const float *scale;  /* [rows] */
  int rows, cols;
  const float *x;      /* residual stream, normalised on the way in */
  const float *norm;   /* RMSNorm weight */
  const float *in;     /* input vector (residual modes; the Wo GEMV reads
                          the attention partials and merges them) */
  float *out;          /* q, x (accumulated) or logits */
  float *hout;         /* SwiGLU output */
  float *kcache, *vcache; /* this layer's [seq, kv_dim] */
  const float *rope;   /* this step's row of the rotary table: [hs/2, 2] */
  int *pos;            /* the classifier advances it; the rest only read it */
  int dim, kv_dim, hs;
  /* Classifier only: one StepBest per workgroup. */
  StepBest *part;
};

/* Layer 0's QKV GEMV (step_gemv_embed) also takes: the token of this
 * position, whose embedding row is its input (also stored to xout), and the
 * rotary table [seq_len, hs/2, 2], read at pos directly and whose row it
 * stores to rope_out for the other layers. (A second argument of that one
 * kernel, so that the other GEMVs' arguments stay small.) */
struct StepEmbedArgs {
  StepTokenArgs tok;
  float *xout;
  const float *rope_table;
  float *rope_out;
  int seq_len;
};

/* Workgroups per head in step_attention: split s takes positions s,
 * s + kAttnSplit, s + 2 kAttnSplit, ... and the Wo GEMV merges the splits.
 * (2, 4 and 8 decode config 4 within run-to-run noise of one another.) */
#ifndef VX_ATTN_SPLIT
#define VX_ATTN_SPLIT 4
#endif
constexpr int kAttnSplit = VX_ATTN_SPLIT;
static_assert(kAttnSplit % 2 == 0, "the merge reads (max, sum) pairs two splits at a time");

/* Floats of the attention partials for a model of `dim` = heads * hs:
 * [kAttnSplit][dim] unnormalised weighted value sums, then
 * [heads][kAttnSplit] (running max, sum of exponentials) pairs. */
inline int64_t attn_part_floats(int dim, int heads) {
  return (int64_t)kAttnSplit * dim + (int64_t)heads * kAttnSplit * 2;
}

struct StepAttnArgs {
  const float *q;
  const float *kcache, *vcache;
  float *part; /* attn_part_floats(heads * hs, heads) */
  const int *pos;
  int kv_dim, hs, kv_mul;
  int seq_len; /* rows of the cache (bounds loads issued before pos is known) */
};


/* rows even, cols a multiple of 16 and at most 4096. */
bool step_gemv_ok(int rows, int cols);
void step_gemv_qkv(const StepGemvArgs &a, hipStream_t s);
/* Layer 0's QKV GEMV: picks the position's token (e.tok) and reads its
 * embedding row instead of a.x. */
void step_gemv_embed(const StepGemvArgs &a, const StepEmbedArgs &e, hipStream_t s);
void step_gemv_resid(const StepGemvArgs &a, hipStream_t s);
/* x += Wo merge(attention partials); cols = heads * hs, hs dividing cols. */
void step_gemv_attn_resid(const StepGemvArgs &a, hipStream_t s);
void step_gemv_swiglu(const StepGemvArgs &a, hipStream_t s);
/* The classifier; leaves step_logits_groups(rows) StepBest entries in
 * `part` for the next step's token (step_gemv_embed, or step_record after
 * the last step), and moves pos on by one. */
void step_gemv_logits(const StepGemvArgs &a, hipStream_t s);
int step_logits_groups(int rows);
/* Records the token of position *pos (after the last step). */
void step_record_launch(const StepArgmaxArgs &a, hipStream_t s);
/* hs divides 256 and is at most 256; seq_len * 4 bytes of LDS. `near`:
 * every position this launch may run at is below step_attention_near(hs),
 * which takes a variant with smaller rounds of rows (any position gives
 * the same result either way; only the speed differs). */
void step_attention_launch(const StepAttnArgs &a, int heads, int seq_len,
                           hipStream_t s, bool near = false);
int step_attention_near(int hs);
/* pos = 0. */
void step_start_launch(const StepArgmaxArgs &a, hipStream_t s);

} // namespace vxk

#endif /* VX_AMD_DECODE_KERNELS_H */
