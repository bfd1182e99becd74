/*
 * vx_hip_ops.h -- library ops of the MI355X dispatch library that have no
 * `kind=` route, called from Vx through `extern "C"` blocks.
 *
 * The reference has no flash-attention op and no int8 GEMV
 * (packages/vx_nn/lib.vx:1 is a placeholder; packages/README.md:10-19), and
 * the compiler has no AMDGPU image pipeline, so these ops are exported by the
 * dispatch library and declared in Vx the way `std::collective` declares its
 * entry points (reference stdlib/std/collective.vx:14-29,
 * runtime/cuda_dispatch.cpp:2064-2123). A tensor cannot cross an `extern`
 * (E3022, reference docs/lang/abi.md section 2), so every op takes element
 * pointers plus extents. Pointers are HBM allocations from
 * vx_plugin_alloc_and_transfer on Topology::GPU[i]; the op runs on the device
 * that owns them, on the calling thread's stream (vx_cuda_set_stream), and
 * returns before the GPU finishes, like a routed GEMM.
 *
 * Each op returns 0 on success and a negative VX_OP_E* code (with a
 * `[Vx HIP]` line on stderr) for arguments it cannot take. A device fault is
 * fatal, as everywhere in the plugin ABI.
 *
 * bf16 and f16 elements travel as uint16_t bit patterns.
 */
#ifndef VX_HIP_OPS_H
#define VX_HIP_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  VX_OP_OK = 0,
  VX_OP_EINVAL = -1,   /* an extent, stride or argument is out of range */
  VX_OP_ENODEV = -2,   /* no GPU: this library has no host copy of the op */
  VX_OP_ENOTDEV = -3,  /* a pointer is not device memory */
  VX_OP_EUNSUPP = -4,  /* a shape the kernels do not take */
  VX_OP_ENOMEM = -5    /* host or device memory ran out */
};

/* Flash-attention forward (the op packages/vx_nn/lib.vx declares).
 *
 * q: [batch, heads, seq_q, head_dim] bf16; k, v: [batch, kv_heads, seq_k,
 * head_dim] bf16; o: like q; lse: [batch, heads, seq_q] f32 (may be NULL).
 * All dense row-major. Query head h reads kv head h / (heads / kv_heads).
 * o = softmax(scale * q k^T) v with f32 accumulation, o rounded to bf16 once;
 * lse = natural-log sum of exp of the scaled scores of each row. With
 * `causal`, query i sees key j iff j <= i + (seq_k - seq_q) (the queries are
 * the last seq_q positions). head_dim must be 64 or 128.
 *
 * A launch whose query blocks fill less than one round of the GPU (for
 * example 512 queries of 32 heads over a long cache) may cut the key range
 * into splits and merge them in f32 (same result to within f32 rounding
 * before the one bf16 rounding). The split partials live in HBM the
 * library keeps per (device, stream): at most 8 x batch x heads x seq_q x
 * (head_dim + 1) x 4 bytes, taken in the stream's order. A stream's block
 * is freed, in its order, when the calling thread's stream is set to
 * another one (so set another stream, or NULL, before destroying one); the
 * default stream's block stays until the process ends. A stream that is
 * capturing a graph gets the unsplit launch. */
int32_t vx_nn_flash_attention_fwd_bf16(const uint16_t *q, const uint16_t *k,
                                       const uint16_t *v, uint16_t *o,
                                       float *lse, int64_t batch, int64_t heads,
                                       int64_t kv_heads, int64_t seq_q,
                                       int64_t seq_k, int64_t head_dim,
                                       float scale, int32_t causal);

/* int8 weight-only GEMV / skinny GEMM.
 *
 * w: [rows, cols] int8 row-major; scale: [rows] f32; x: [batch, cols] bf16;
 * y: [batch, rows] f32. y[b, r] = scale[r] * sum_c w[r, c] * x[b, c], the sum
 * in f32. batch 1..16; cols a multiple of 16 and at most 2^24. */
int32_t vx_nn_gemv_i8_bf16(const int8_t *w, const float *scale,
                           const uint16_t *x, float *y, int64_t rows,
                           int64_t cols, int64_t batch);

/* Greedy int8 decode of a Llama-2-style model, resident in HBM.
 *
 * The token step of reference examples/llama.vx:173-420 (RMSNorm eps 1e-5,
 * Q/K/V, RoPE, KV cache, causal attention, Wo, SwiGLU FFN, residuals, final
 * RMSNorm, classifier sharing the embedding table, argmax with the lowest
 * index winning a tie) as GPU library ops: every linear is an int8
 * weight-only GEMV with per-row f32 scales; activations and everything else
 * are f32, as in the reference. The position and the next token stay on the GPU,
 * so a whole step is replayable as one hipGraph with no host round trip.
 *
 * Weights are host pointers in llama2.c order, matrices [out][in]:
 * tok [vocab, dim] (embedding and classifier); per layer wq [dim, dim],
 * wk/wv [kv_dim, dim], wo [dim, dim], w1/w3 [hidden, dim], w2 [dim, hidden],
 * each with one f32 scale per row; RMSNorm weights f32; `rope` the
 * [seq_len, head_size / 2] table of (cos, sin) of the rotary angles. */
typedef struct vx_llama_i8_config {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} vx_llama_i8_config;

typedef struct vx_llama_i8_weights {
  const int8_t *tok_q;
  const float *tok_s;
  const float *rms_att; /* [layers, dim] */
  const int8_t *wq_q;
  const float *wq_s;
  const int8_t *wk_q;
  const float *wk_s;
  const int8_t *wv_q;
  const float *wv_s;
  const int8_t *wo_q;
  const float *wo_s;
  const float *rms_ffn; /* [layers, dim] */
  const int8_t *w1_q;
  const float *w1_s;
  const int8_t *w2_q;
  const float *w2_s;
  const int8_t *w3_q;
  const float *w3_s;
  const float *rms_final; /* [dim] */
  const float *rope;      /* [seq_len, head_size / 2, 2] */
} vx_llama_i8_weights;

/* Capture the token step as hipGraphs (8 steps, and 1 for the remainder;
 * one pair for positions whose attention takes the small rounds, one for
 * the rest) and replay them (else: stream launches, one by one). */
#define VX_LLAMA_GRAPH 1

/* Upload a model to GPU[topology_id - 500]; NULL (and a [Vx HIP] line) when
 * the config is not one the kernels take or there is no GPU. */
void *vx_llama_i8_create(const vx_llama_i8_config *cfg,
                         const vx_llama_i8_weights *w, uint32_t topology_id);

/* Feed prompt[0..n_prompt), then generate n_steps tokens greedily into
 * out_tokens; out_margin (may be NULL) gets each generated token's logit
 * lead over the runner-up. Returns 0, or a VX_OP_E* code. */
int32_t vx_llama_i8_generate(void *model, const int32_t *prompt,
                             int32_t n_prompt, int32_t n_steps,
                             int32_t *out_tokens, float *out_margin,
                             int32_t flags);

/* Feed tokens[0..n) at positions 0..n-1 and copy the logits after each
 * position to logits[n, vocab]. Returns 0 or a VX_OP_E* code. */
int32_t vx_llama_i8_logits(void *model, const int32_t *tokens, int32_t n,
                           float *logits);

void vx_llama_i8_destroy(void *model);

/* ---- Model files (host side; no GPU needed) ----
 *
 * Two formats are read:
 *  - a llama2.c checkpoint, the file reference examples/llama.vx loads
 *    (stdlib/rust_core/src/ffi/llama.rs:10-45 reads it: seven int32 --
 *    dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len --
 *    then the f32 arrays in the order of examples/llama.vx:80-120; the
 *    RoPE arrays llama2.c appends after rms_final may be present or not).
 *    Every matrix is quantized per output row on the way in (scale =
 *    max|w| / 127, q = round-half-even(w / scale));
 *  - the int8 file vx_llama_i8_save writes ("VXQ8" version 1: the config,
 *    then every array of vx_llama_i8_weights in field order, then a 64-bit
 *    FNV-1a of everything before it), so the quantization is done once.
 * Either way the RoPE table is computed from the config (base 10000), the
 * classifier is the token table (a negative vocab_size -- an unshared
 * classifier -- is refused), and the result feeds vx_llama_i8_create. */
typedef struct vx_llama_i8_host vx_llama_i8_host;

/* Read `path`; on VX_OP_OK, *cfg holds the config and *out the weights
 * (free with vx_llama_i8_host_free). VX_OP_EINVAL for an unreadable,
 * truncated or corrupt file, VX_OP_EUNSUPP for a layout this build does
 * not take. */
int32_t vx_llama_i8_read(const char *path, vx_llama_i8_config *cfg,
                         vx_llama_i8_host **out);
/* The weights of a read model, valid until vx_llama_i8_host_free. */
const vx_llama_i8_weights *vx_llama_i8_host_weights(const vx_llama_i8_host *h);
void vx_llama_i8_host_free(vx_llama_i8_host *h);
/* Write cfg and w as a "VXQ8" file. */
int32_t vx_llama_i8_save(const char *path, const vx_llama_i8_config *cfg,
                         const vx_llama_i8_weights *w);

/* ---- device images in the payload ------------------------------------
 *
 * vx_plugin_dispatch_async runs a region whose payload says `format=hsaco`
 * from the gfx950 code object in the payload's binary section (a bare ELF or
 * a clang offload bundle): one parameter per memref field (allocated,
 * aligned, offset, sizes, strides) and per scalar, as the reference's PTX
 * path marshals them (runtime/vx_kernel_launch.h:57-140); the launch shape
 * from `grid=`/`block=`/`grid_loops=` or `launch=`; `assert_flag=1` appends
 * a pointer to a cleared device int that a failed assert sets; `shared=`
 * bytes of dynamic LDS; `coop=1` launches cooperatively. Before the first
 * launch the count below is compared with what the arguments produce.
 *
 * How many of its own parameters (not the hidden ones the runtime appends)
 * `kernel` declares in the gfx950 code object `image`, read from the code
 * object's metadata; -1 when the image, its metadata or the kernel is
 * absent. Replaces, for AMDGPU images, the reference's
 * vx_launch_entry_param_count (runtime/vx_kernel_launch.h:206-222, PTX) and
 * vx_launch_entry_param_count_spirv (:248-315). */
int32_t vx_hip_image_param_count(const void *image, size_t image_size,
                                 const char *kernel);

/* ---- a routed GEMM that allocates nothing -----------------------------
 *
 * No counterpart in the reference. For callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc): the
 * kind=matmul dispatch of vx_plugin_dispatch_async, with the same payload,
 * arguments and result, except that host operands and a host result buffer
 * are staged through a fixed 16 MiB array per GPU (in this library's code
 * object) instead of the staging pool. Grids of 256x256 tiles that end in
 * a partial round of at most half the CUs run here one tile per workgroup,
 * where vx_plugin_dispatch_async ends them with a stream-K launch that needs
 * a workspace: the results then agree to 1e-5 relative (one bf16 unit for
 * bf16 output), not bit for bit. Returns 1 when the GEMM was issued,
 * 0 (reason on stderr, nothing launched) for a region that is not a routed
 * GEMM, a result published through a slot (host memory the program frees),
 * staging beyond 16 MiB, or staging while the caller stream is capturing a
 * graph. Operands already in GPU memory need no staging. Calls on one GPU
 * share its array and take turns on it: a call that stages waits, in its
 * stream's order, for the GEMM of the previous such call (on any stream or
 * thread) before it overwrites the array. */
uint64_t vx_hip_dispatch_async_noalloc(const void *binary_payload,
                                       size_t payload_size, void **device_args,
                                       const int32_t *arg_tags,
                                       int64_t num_args);

#ifdef __cplusplus
}
#endif

#endif /* VX_HIP_OPS_H */
