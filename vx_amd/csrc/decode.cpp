/*
 * decode.cpp -- vx_llama_i8_*: an int8 Llama-2-style decoder resident in HBM
 * and its greedy generation loop (include/vx_hip_ops.h).
 *
 * Weights are re-laid out once at upload so each fused kernel streams one
 * matrix: per layer [Wq; Wk; Wv] stacked (one GEMV feeds RoPE and the KV
 * cache) and W1/W3 interleaved row by row (one GEMV feeds SwiGLU). The
 * position and the next token live in device memory; a step is a fixed
 * sequence of 5 * layers + 1 launches that, with VX_LLAMA_GRAPH, is captured
 * into hipGraphs of kGraphSteps steps and of one step (kept with the model
 * while the prompt length and I/O buffers stay the same) and replayed with
 * no host synchronisation until the tokens are read back.
 */
#include "../../include/vx_hardware_runtime.h"
#include "../../include/vx_hip_ops.h"
#include "vx_decode_kernels.h"
#include "vx_hip_common.h"
#include "vx_ops_internal.h"

#include <cstring>
#include <vector>

namespace {

/* Steps per replay of the long graph (the positions left over go through
 * the one-step graph). */
#ifndef VX_DEC_GRAPH_STEPS
#define VX_DEC_GRAPH_STEPS 8
#endif
constexpr int kGraphSteps = VX_DEC_GRAPH_STEPS;

struct LlamaI8 {
  vx_llama_i8_config cfg;
  int hs = 0, kv_dim = 0, device = 0;
  int8_t *tok_q = nullptr, *wqkv = nullptr, *wo = nullptr, *w13 = nullptr,
         *w2 = nullptr;
  float *tok_s = nullptr, *sqkv = nullptr, *so = nullptr, *s13 = nullptr,
        *s2 = nullptr;
  float *rms_att = nullptr, *rms_ffn = nullptr, *rms_final = nullptr,
        *rope = nullptr, *rope_now = nullptr;
  float *kcache = nullptr, *vcache = nullptr;
  float *x = nullptr, *q = nullptr, *logits = nullptr;
  float *att = nullptr, *hb = nullptr;
  int *pos = nullptr, *prompt = nullptr, *out_tokens = nullptr;
  float *out_margin = nullptr;
  vxk::StepBest *best = nullptr; /* one per classifier workgroup */
  int prompt_cap = 0, out_cap = 0;
  hipStream_t stream = nullptr;
  /* The instantiated step graphs (one step, kGraphSteps steps; [1]: for
   * steps whose positions are all below step_attention_near, whose
   * attention takes smaller rounds of rows), kept across generate calls:
   * they bake in the prompt length and the I/O buffers, so they are dropped
   * when either changes. */
  hipGraphExec_t step_exec[2] = {nullptr, nullptr};
  hipGraphExec_t steps_exec[2] = {nullptr, nullptr};
  int step_exec_prompt = -1;
  std::vector<void *> owned;
};

template <typename T> T *upload(LlamaI8 &m, const T *host, size_t count) {
  void *p = nullptr;
  VX_HIP_CHECK(hipMalloc(&p, count * sizeof(T) + 16));
  if (host) {
    VX_HIP_CHECK(hipMemcpy(p, host, count * sizeof(T), hipMemcpyHostToDevice));
  }
  m.owned.push_back(p);
  return static_cast<T *>(p);
}

template <typename T> T *alloc(LlamaI8 &m, size_t count) {
  return upload<T>(m, nullptr, count);
}

void drop_step_graph(LlamaI8 &m) {
  for (hipGraphExec_t *g : {&m.step_exec[0], &m.step_exec[1], &m.steps_exec[0],
                            &m.steps_exec[1]}) {
    if (*g) {
      (void)hipGraphExecDestroy(*g);
      *g = nullptr;
    }
  }
  m.step_exec_prompt = -1;
}

void release(LlamaI8 &m) {
  drop_step_graph(m);
  if (m.stream) {
    (void)hipStreamSynchronize(m.stream);
    (void)hipStreamDestroy(m.stream);
  }
  for (void *p : m.owned) {
    (void)hipFree(p);
  }
  m.owned.clear();
}

int32_t refuse(int32_t code, const char *why) {
  fprintf(stderr, "[Vx HIP] vx_llama_i8: %s\n", why);
  return code;
}

bool ensure_io(LlamaI8 &m, int n_prompt, int n_out) {
  if (n_prompt > m.prompt_cap) {
    m.prompt = alloc<int>(m, (size_t)n_prompt);
    m.prompt_cap = n_prompt;
    drop_step_graph(m);
  }
  if (n_out > m.out_cap) {
    m.out_tokens = alloc<int>(m, (size_t)n_out);
    m.out_margin = alloc<float>(m, (size_t)n_out);
    m.out_cap = n_out;
    drop_step_graph(m);
  }
  return true;
}

vxk::StepTokenArgs token_args(LlamaI8 &m, int n_prompt) {
  vxk::StepTokenArgs a;
  a.cand = m.best;
  a.ncand = vxk::step_logits_groups(m.cfg.vocab_size);
  a.prompt = m.prompt;
  a.n_prompt = n_prompt;
  a.out_tokens = m.out_tokens;
  a.out_margin = m.out_margin;
  a.out_cap = m.out_cap;
  a.tok_q = m.tok_q;
  a.tok_s = m.tok_s;
  a.vocab = m.cfg.vocab_size;
  return a;
}

vxk::StepArgmaxArgs argmax_args(LlamaI8 &m, int n_prompt) {
  vxk::StepArgmaxArgs a;
  a.tok = token_args(m, n_prompt);
  a.pos = m.pos;
  return a;
}

/* One token step on the model's stream; `near`: its position is below
 * step_attention_near (the attention launches take smaller rounds). */
void enqueue_step(LlamaI8 &m, int n_prompt, bool near) {
  const vx_llama_i8_config &c = m.cfg;
  const int qkv_rows = c.dim + 2 * m.kv_dim;
  const int64_t layer_kv = (int64_t)c.seq_len * m.kv_dim;
  for (int l = 0; l < c.n_layers; ++l) {
    vxk::StepGemvArgs g{};
    g.pos = m.pos;
    g.dim = c.dim;
    g.kv_dim = m.kv_dim;
    g.hs = m.hs;
    g.rope = m.rope_now;
    g.kcache = m.kcache + l * layer_kv;
    g.vcache = m.vcache + l * layer_kv;

    vxk::StepGemvArgs qkv = g;
    qkv.w = m.wqkv + (int64_t)l * qkv_rows * c.dim;
    qkv.scale = m.sqkv + (int64_t)l * qkv_rows;
    qkv.rows = qkv_rows;
    qkv.cols = c.dim;
    qkv.x = m.x;
    qkv.norm = m.rms_att + (int64_t)l * c.dim;
    qkv.out = m.q;
    if (l == 0) {
      /* the position's token and its embedding as x; the rotary row */
      vxk::StepEmbedArgs e;
      e.tok = token_args(m, n_prompt);
      e.xout = m.x;
      e.rope_table = m.rope;
      e.rope_out = m.rope_now;
      e.seq_len = c.seq_len;
      vxk::step_gemv_embed(qkv, e, m.stream);
    } else {
      vxk::step_gemv_qkv(qkv, m.stream);
    }

    vxk::StepAttnArgs at;
    at.q = m.q;
    at.kcache = g.kcache;
    at.vcache = g.vcache;
    at.part = m.att;
    at.pos = m.pos;
    at.kv_dim = m.kv_dim;
    at.hs = m.hs;
    at.kv_mul = c.n_heads / c.n_kv_heads;
    at.seq_len = c.seq_len;
    vxk::step_attention_launch(at, c.n_heads, c.seq_len, m.stream, near);

    vxk::StepGemvArgs wo = g;
    wo.w = m.wo + (int64_t)l * c.dim * c.dim;
    wo.scale = m.so + (int64_t)l * c.dim;
    wo.rows = c.dim;
    wo.cols = c.dim;
    wo.in = m.att;
    wo.out = m.x;
    vxk::step_gemv_attn_resid(wo, m.stream);

    vxk::StepGemvArgs ffn = g;
    ffn.w = m.w13 + (int64_t)l * 2 * c.hidden_dim * c.dim;
    ffn.scale = m.s13 + (int64_t)l * 2 * c.hidden_dim;
    ffn.rows = 2 * c.hidden_dim;
    ffn.cols = c.dim;
    ffn.x = m.x;
    ffn.norm = m.rms_ffn + (int64_t)l * c.dim;
    ffn.hout = m.hb;
    vxk::step_gemv_swiglu(ffn, m.stream);

    vxk::StepGemvArgs w2 = g;
    w2.w = m.w2 + (int64_t)l * c.dim * c.hidden_dim;
    w2.scale = m.s2 + (int64_t)l * c.dim;
    w2.rows = c.dim;
    w2.cols = c.hidden_dim;
    w2.in = m.hb;
    w2.out = m.x;
    vxk::step_gemv_resid(w2, m.stream);
  }
  vxk::StepGemvArgs lg{};
  lg.w = m.tok_q;
  lg.scale = m.tok_s;
  lg.rows = c.vocab_size;
  lg.cols = c.dim;
  lg.x = m.x;
  lg.norm = m.rms_final;
  lg.out = m.logits;
  lg.pos = m.pos;
  lg.part = m.best;
  vxk::step_gemv_logits(lg, m.stream);
}

} // namespace

extern "C" {

void *vx_llama_i8_create(const vx_llama_i8_config *cfg,
                         const vx_llama_i8_weights *w, uint32_t topology_id) {
  if (!vxops::device_present()) {
    refuse(VX_OP_ENODEV, "no GPU; this op has no host copy");
    return nullptr;
  }
  if (!cfg || !w) {
    refuse(VX_OP_EINVAL, "config and weights must not be NULL");
    return nullptr;
  }
  const vx_llama_i8_config c = *cfg;
  if (c.dim <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_layers <= 0 ||
      c.hidden_dim <= 0 || c.vocab_size <= 0 || c.seq_len <= 0 ||
      c.dim % c.n_heads || c.n_heads % c.n_kv_heads) {
    refuse(VX_OP_EINVAL, "config extents must be positive, dim a multiple "
                         "of n_heads and n_heads of n_kv_heads");
    return nullptr;
  }
  const int hs = c.dim / c.n_heads;
  const int kv_dim = c.dim * c.n_kv_heads / c.n_heads;
  if (hs % 2 || hs > 256 || 256 % hs || !vxk::step_gemv_ok(c.dim, c.dim) ||
      !vxk::step_gemv_ok(2 * c.hidden_dim, c.dim) ||
      !vxk::step_gemv_ok(c.dim, c.hidden_dim) ||
      !vxk::step_gemv_ok(c.vocab_size, c.dim) || kv_dim % 2 ||
      c.seq_len > 16384) {
    refuse(VX_OP_EUNSUPP, "shape not taken by the decode kernels (head size "
                          "must divide 256; dim and hidden_dim multiples of "
                          "16 and at most 4096; vocab even; seq_len <= 16384)");
    return nullptr;
  }
  const int device =
      vx_topology_device_index((int32_t)topology_id, VX_TOPO_GPU_BASE);
  if (device < 0) {
    refuse(VX_OP_EINVAL, "topology_id must name a GPU (500 + index)");
    return nullptr;
  }
  VX_HIP_CHECK(hipSetDevice(device));

  LlamaI8 *m = new LlamaI8();
  m->cfg = c;
  m->hs = hs;
  m->kv_dim = kv_dim;
  m->device = device;
  const size_t L = (size_t)c.n_layers, D = (size_t)c.dim,
               H = (size_t)c.hidden_dim, KV = (size_t)kv_dim;
  const size_t qkv_rows = D + 2 * KV;

  /* [Wq; Wk; Wv] per layer, with their scales. */
  std::vector<int8_t> qkv(L * qkv_rows * D);
  std::vector<float> sqkv(L * qkv_rows);
  for (size_t l = 0; l < L; ++l) {
    int8_t *dst = qkv.data() + l * qkv_rows * D;
    memcpy(dst, w->wq_q + l * D * D, D * D);
    memcpy(dst + D * D, w->wk_q + l * KV * D, KV * D);
    memcpy(dst + (D + KV) * D, w->wv_q + l * KV * D, KV * D);
    float *sd = sqkv.data() + l * qkv_rows;
    memcpy(sd, w->wq_s + l * D, D * 4);
    memcpy(sd + D, w->wk_s + l * KV, KV * 4);
    memcpy(sd + D + KV, w->wv_s + l * KV, KV * 4);
  }
  /* W1 and W3 rows interleaved per layer. */
  std::vector<int8_t> w13(L * 2 * H * D);
  std::vector<float> s13(L * 2 * H);
  for (size_t l = 0; l < L; ++l) {
    for (size_t r = 0; r < H; ++r) {
      memcpy(&w13[(l * 2 * H + 2 * r) * D], w->w1_q + (l * H + r) * D, D);
      memcpy(&w13[(l * 2 * H + 2 * r + 1) * D], w->w3_q + (l * H + r) * D, D);
      s13[l * 2 * H + 2 * r] = w->w1_s[l * H + r];
      s13[l * 2 * H + 2 * r + 1] = w->w3_s[l * H + r];
    }
  }
  m->wqkv = upload(*m, qkv.data(), qkv.size());
  m->sqkv = upload(*m, sqkv.data(), sqkv.size());
  m->w13 = upload(*m, w13.data(), w13.size());
  m->s13 = upload(*m, s13.data(), s13.size());
  m->wo = upload(*m, w->wo_q, L * D * D);
  m->so = upload(*m, w->wo_s, L * D);
  m->w2 = upload(*m, w->w2_q, L * D * H);
  m->s2 = upload(*m, w->w2_s, L * D);
  m->tok_q = upload(*m, w->tok_q, (size_t)c.vocab_size * D);
  m->tok_s = upload(*m, w->tok_s, (size_t)c.vocab_size);
  m->rms_att = upload(*m, w->rms_att, L * D);
  m->rms_ffn = upload(*m, w->rms_ffn, L * D);
  m->rms_final = upload(*m, w->rms_final, D);
  m->rope = upload(*m, w->rope, (size_t)c.seq_len * hs);
  m->rope_now = alloc<float>(*m, (size_t)hs);
  m->kcache = alloc<float>(*m, L * (size_t)c.seq_len * KV);
  m->vcache = alloc<float>(*m, L * (size_t)c.seq_len * KV);
  /* Rows past the position are read (and discarded) by the attention
   * kernels' early loads: start them at zero rather than at whatever the
   * allocation held. */
  VX_HIP_CHECK(hipMemset(m->kcache, 0, L * (size_t)c.seq_len * KV * sizeof(float)));
  VX_HIP_CHECK(hipMemset(m->vcache, 0, L * (size_t)c.seq_len * KV * sizeof(float)));
  m->x = alloc<float>(*m, D);
  m->q = alloc<float>(*m, D);
  m->logits = alloc<float>(*m, (size_t)c.vocab_size);
  m->att = alloc<float>(*m, (size_t)vxk::attn_part_floats(c.dim, c.n_heads));
  m->hb = alloc<float>(*m, H);
  m->pos = alloc<int>(*m, 1);
  m->best = alloc<vxk::StepBest>(*m, (size_t)vxk::step_logits_groups(c.vocab_size));
  VX_HIP_CHECK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
  return m;
}

int32_t vx_llama_i8_generate(void *model, const int32_t *prompt,
                             int32_t n_prompt, int32_t n_steps,
                             int32_t *out_tokens, float *out_margin,
                             int32_t flags) {
  LlamaI8 *m = static_cast<LlamaI8 *>(model);
  if (!m || !prompt || !out_tokens || n_prompt < 1 || n_steps < 1) {
    return refuse(VX_OP_EINVAL, "need a model, a prompt of at least one "
                                "token and at least one step");
  }
  if (n_prompt + n_steps - 1 > m->cfg.seq_len) {
    return refuse(VX_OP_EINVAL, "prompt + steps exceed the model's seq_len");
  }
  for (int i = 0; i < n_prompt; ++i) {
    if (prompt[i] < 0 || prompt[i] >= m->cfg.vocab_size) {
      return refuse(VX_OP_EINVAL, "a prompt token is outside the vocabulary");
    }
  }
  VX_HIP_CHECK(hipSetDevice(m->device));
  ensure_io(*m, n_prompt, n_steps);
  VX_HIP_CHECK(hipMemcpyAsync(m->prompt, prompt, sizeof(int) * n_prompt,
                              hipMemcpyHostToDevice, m->stream));
  vxk::StepArgmaxArgs start = argmax_args(*m, n_prompt);
  vxk::step_start_launch(start, m->stream);
  const int positions = n_prompt + n_steps - 1;
  const int near_pos = vxk::step_attention_near(m->hs);
  if (flags & VX_LLAMA_GRAPH) {
    if (m->step_exec_prompt != n_prompt) {
      drop_step_graph(*m);
      m->step_exec_prompt = n_prompt;
    }
    /* the graph of `steps` steps for positions p .. p + steps - 1,
     * captured when first needed */
    auto graph_for = [&](int p, int steps) {
      const int near = p + steps - 1 < near_pos ? 1 : 0;
      hipGraphExec_t &exec = steps == 1 ? m->step_exec[near] : m->steps_exec[near];
      if (!exec) {
        hipGraph_t graph = nullptr;
        VX_HIP_CHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < steps; ++i) {
          enqueue_step(*m, n_prompt, near != 0);
        }
        VX_HIP_CHECK(hipStreamEndCapture(m->stream, &graph));
        VX_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        VX_HIP_CHECK(hipGraphDestroy(graph));
      }
      return exec;
    };
    int p = 0;
    for (; kGraphSteps > 1 && p + kGraphSteps <= positions; p += kGraphSteps) {
      VX_HIP_CHECK(hipGraphLaunch(graph_for(p, kGraphSteps), m->stream));
    }
    for (; p < positions; ++p) {
      VX_HIP_CHECK(hipGraphLaunch(graph_for(p, 1), m->stream));
    }
  } else {
    for (int p = 0; p < positions; ++p) {
      enqueue_step(*m, n_prompt, p < near_pos);
    }
  }
  /* the token after the last step */
  vxk::step_record_launch(start, m->stream);
  VX_HIP_CHECK(hipGetLastError());
  VX_HIP_CHECK(hipMemcpyAsync(out_tokens, m->out_tokens,
                              sizeof(int) * n_steps, hipMemcpyDeviceToHost,
                              m->stream));
  if (out_margin) {
    VX_HIP_CHECK(hipMemcpyAsync(out_margin, m->out_margin,
                                sizeof(float) * n_steps,
                                hipMemcpyDeviceToHost, m->stream));
  }
  VX_HIP_CHECK(hipStreamSynchronize(m->stream));
  return VX_OP_OK;
}

int32_t vx_llama_i8_logits(void *model, const int32_t *tokens, int32_t n,
                           float *logits) {
  LlamaI8 *m = static_cast<LlamaI8 *>(model);
  if (!m || !tokens || !logits || n < 1 || n > m->cfg.seq_len) {
    return refuse(VX_OP_EINVAL, "need a model, 1..seq_len tokens and an "
                                "output buffer");
  }
  for (int i = 0; i < n; ++i) {
    if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size) {
      return refuse(VX_OP_EINVAL, "a token is outside the vocabulary");
    }
  }
  VX_HIP_CHECK(hipSetDevice(m->device));
  ensure_io(*m, n, 1);
  VX_HIP_CHECK(hipMemcpyAsync(m->prompt, tokens, sizeof(int) * n,
                              hipMemcpyHostToDevice, m->stream));
  vxk::step_start_launch(argmax_args(*m, n), m->stream);
  const size_t vocab = (size_t)m->cfg.vocab_size;
  const int near_pos = vxk::step_attention_near(m->hs);
  for (int p = 0; p < n; ++p) {
    enqueue_step(*m, n, p < near_pos);
    VX_HIP_CHECK(hipMemcpyAsync(logits + p * vocab, m->logits,
                                sizeof(float) * vocab, hipMemcpyDeviceToHost,
                                m->stream));
  }
  VX_HIP_CHECK(hipStreamSynchronize(m->stream));
  return VX_OP_OK;
}

void vx_llama_i8_destroy(void *model) {
  LlamaI8 *m = static_cast<LlamaI8 *>(model);
  if (!m) {
    return;
  }
  (void)hipSetDevice(m->device);
  release(*m);
  delete m;
}

} // extern "C"
