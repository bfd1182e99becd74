/*
 * decode.hip -- the GPU-resident token step of a Llama-2-style int8 decoder
 * (the semantics of reference examples/llama.vx:145-420).
 *
 * A step is 5 launches per layer plus 2, each reading the position from
 * device memory so that a captured step replays unchanged:
 *
 *   step_gemv<kQkv>    RMSNorm(x), [Wq; Wk; Wv] int8 GEMV, RoPE on
 *                      q and k, k and v into the KV cache at `pos`
 *   step_attention     one workgroup per head: softmax(q k^T / sqrt(hs)) v
 *                      over positions 0..pos
 *   step_gemv<kResid>  x += Wo att
 *   step_gemv<kSwiglu> RMSNorm(x), [W1; W3] GEMV with rows interleaved,
 *                      silu(h1) * h3
 *   step_gemv<kResid>  x += W2 h
 *   step_gemv<kLogits> final RMSNorm, classifier (the embedding table)
 *   step_argmax        argmax (lowest index wins a tie) or the next prompt
 *                      token; x = embedding of that token; pos += 1
 *
 * Every GEMV is weight-only int8 with one f32 scale per row over f32
 * activations (as in the reference, which is f32 throughout), f32 sums;
 * each wave owns two adjacent rows, so the even/odd RoPE
 * pair and the (h1, h3) SwiGLU pair finish in one lane. Contraction is off
 * so the elementwise arithmetic rounds where the reference's f32 loop nest
 * rounds; only the summation order differs.
 */
#include "../vx_hip_common.h"
#include "../vx_decode_kernels.h"

#include <cmath>

namespace vxk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxCols = 4096;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v += __shfl_xor(v, off, 64);
  }
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v = fmaxf(v, __shfl_xor(v, off, 64));
  }
  return v;
}

/* Sum over the workgroup, the same order on every thread. */
__device__ float block_sum(float v, float *scratch) {
  const int nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    scratch[threadIdx.x >> 6] = v;
  }
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < nw; ++i) {
    t += scratch[i];
  }
  return t;
}

__device__ float block_max(float v, float *scratch) {
  const int nw = blockDim.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    scratch[threadIdx.x >> 6] = v;
  }
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; ++i) {
    t = fmaxf(t, scratch[i]);
  }
  return t;
}

enum Mode { kQkv = 0, kResid = 1, kSwiglu = 2, kLogits = 3 };

template <int kMode>
__global__ __launch_bounds__(kThreads) void step_gemv(StepGemvArgs a) {
#pragma clang fp contract(off)
  __shared__ float xin[kMaxCols];
  __shared__ float scratch[kThreads / 64];
  const int t = threadIdx.x;
  const int cols = a.cols;
  if constexpr (kMode == kResid) {
    for (int i = t; i < cols; i += kThreads) {
      xin[i] = a.in[i];
    }
  } else {
    /* RMSNorm as reference examples/llama.vx:145-158. */
    float ss = 0.0f;
    for (int i = t; i < cols; i += kThreads) {
      const float v = a.x[i];
      ss += v * v;
    }
    ss = block_sum(ss, scratch);
    const float inv = 1.0f / sqrtf(ss / (float)cols + 0.00001f);
    for (int i = t; i < cols; i += kThreads) {
      xin[i] = a.norm[i] * (inv * a.x[i]);
    }
  }
  __syncthreads();

  const int wave = t >> 6;
  const int lane = t & 63;
  const int r0 = (blockIdx.x * (kThreads / 64) + wave) * 2;
  if (r0 >= a.rows) {
    return;
  }
  const int8_t *w0 = a.w + (int64_t)r0 * cols;
  const int8_t *w1 = w0 + cols;
  float acc0 = 0.0f, acc1 = 0.0f;
  for (int c = lane * 16; c < cols; c += 64 * 16) {
    const u32x4 p = *reinterpret_cast<const u32x4 *>(w0 + c);
    const u32x4 q = *reinterpret_cast<const u32x4 *>(w1 + c);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float xv = xin[c + k];
      acc0 += (float)(int8_t)(p[k >> 2] >> (8 * (k & 3))) * xv;
      acc1 += (float)(int8_t)(q[k >> 2] >> (8 * (k & 3))) * xv;
    }
  }
  acc0 = wave_sum(acc0);
  acc1 = wave_sum(acc1);
  if (lane != 0) {
    return;
  }
  const float y0 = a.scale[r0] * acc0;
  const float y1 = a.scale[r0 + 1] * acc1;

  if constexpr (kMode == kQkv) {
    const int pos = *a.pos;
    const int dim = a.dim, kv_dim = a.kv_dim, hs = a.hs;
    if (r0 < dim + kv_dim) {
      /* RoPE on the (even, odd) pair (reference :235-264). */
      const int i = r0 < dim ? r0 : r0 - dim;
      const int hd = i % hs;
      const float *cs = a.rope + ((int64_t)pos * (hs / 2) + hd / 2) * 2;
      const float fcr = cs[0], fci = cs[1];
      const float e0 = y0 * fcr - y1 * fci;
      const float e1 = y0 * fci + y1 * fcr;
      if (r0 < dim) {
        a.out[r0] = e0;
        a.out[r0 + 1] = e1;
      } else {
        a.kcache[(int64_t)pos * kv_dim + i] = e0;
        a.kcache[(int64_t)pos * kv_dim + i + 1] = e1;
      }
    } else {
      const int i = r0 - dim - kv_dim;
      a.vcache[(int64_t)pos * kv_dim + i] = y0;
      a.vcache[(int64_t)pos * kv_dim + i + 1] = y1;
    }
  } else if constexpr (kMode == kResid) {
    a.out[r0] = a.out[r0] + y0;
    a.out[r0 + 1] = a.out[r0 + 1] + y1;
  } else if constexpr (kMode == kSwiglu) {
    /* rows interleaved: 2i is W1 row i, 2i + 1 is W3 row i (reference
     * :377-384: val * (1 / (1 + exp(-val))) * h3). */
    float val = y0;
    const float neg = 0.0f - val;
    val = val * (1.0f / (1.0f + expf(neg)));
    val = val * y1;
    a.hout[r0 >> 1] = val;
  } else {
    a.out[r0] = y0;
    a.out[r0 + 1] = y1;
  }
}

/* One workgroup per query head over positions 0..pos (reference
 * :275-325); scores in dynamic LDS. */
__global__ __launch_bounds__(kThreads) void step_attention(StepAttnArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float score[];
  __shared__ float qs[256];
  __shared__ float part[kThreads];
  __shared__ float scratch[kThreads / 64];
  const int t = threadIdx.x;
  const int h = blockIdx.x;
  const int hs = a.hs;
  const int hk = h / a.kv_mul;
  const int pos = *a.pos;
  const int n = pos + 1;
  if (t < hs) {
    qs[t] = a.q[h * hs + t];
  }
  __syncthreads();
  const float *kb = a.kcache + hk * hs;
  const float *vb = a.vcache + hk * hs;
  const float root = sqrtf((float)hs);
  float mx = -INFINITY;
  for (int j = t; j < n; j += kThreads) {
    const float *kr = kb + (int64_t)j * a.kv_dim;
    float dot = 0.0f;
    for (int i = 0; i < hs; ++i) {
      dot = dot + qs[i] * kr[i];
    }
    const float s = dot / root;
    score[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max(mx, scratch);
  float sum = 0.0f;
  for (int j = t; j < n; j += kThreads) {
    const float p = expf(score[j] - mx);
    score[j] = p;
    sum += p;
  }
  sum = block_sum(sum, scratch); /* also orders the score writes */
  const int groups = kThreads / hs;
  const int g = t / hs;
  const int i = t - g * hs;
  float acc = 0.0f;
  for (int j = g; j < n; j += groups) {
    acc = acc + score[j] * vb[(int64_t)j * a.kv_dim + i];
  }
  part[t] = acc;
  __syncthreads();
  if (t < hs) {
    float o = 0.0f;
    for (int gg = 0; gg < groups; ++gg) {
      o += part[gg * hs + t];
    }
    const float inv = 1.0f / sum;
    a.att[h * hs + t] = o * inv;
  }
}

struct Best {
  float v1;  /* best value */
  int i1;    /* its index (lowest among equals) */
  float v2;  /* runner-up value */
};

__device__ __forceinline__ Best merge(Best a, Best b) {
  Best r;
  if (b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1)) {
    r.v1 = b.v1;
    r.i1 = b.i1;
    r.v2 = fmaxf(a.v1, b.v2);
  } else {
    r.v1 = a.v1;
    r.i1 = a.i1;
    r.v2 = fmaxf(a.v2, b.v1);
  }
  return r;
}

constexpr int kArgThreads = 1024;

/* Argmax with strict '>' in index order (reference :160-171), or the next
 * prompt token while the prompt lasts; then the embedding of the chosen
 * token into x, and pos + 1. */
__global__ __launch_bounds__(kArgThreads) void step_argmax(StepArgmaxArgs a) {
  __shared__ Best part[kArgThreads / 64];
  __shared__ int chosen;
  const int t = threadIdx.x;
  const int pos = *a.pos;
  Best b{-INFINITY, 0x7fffffff, -INFINITY};
  for (int i = t; i < a.vocab; i += kArgThreads) {
    const float v = a.logits[i];
    if (v > b.v1) {
      b.v2 = b.v1;
      b.v1 = v;
      b.i1 = i;
    } else if (v > b.v2) {
      b.v2 = v;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    Best o;
    o.v1 = __shfl_xor(b.v1, off, 64);
    o.i1 = __shfl_xor(b.i1, off, 64);
    o.v2 = __shfl_xor(b.v2, off, 64);
    b = merge(b, o);
  }
  if ((t & 63) == 0) {
    part[t >> 6] = b;
  }
  __syncthreads();
  if (t == 0) {
    Best r = part[0];
    for (int w = 1; w < kArgThreads / 64; ++w) {
      r = merge(r, part[w]);
    }
    int tok;
    if (pos + 1 < a.n_prompt) {
      tok = a.prompt[pos + 1];
    } else {
      tok = r.i1;
      const int at = pos + 1 - a.n_prompt;
      if (at < a.out_cap) {
        a.out_tokens[at] = tok;
        a.out_margin[at] = r.v1 - r.v2;
      }
    }
    chosen = tok;
  }
  __syncthreads();
  const int tok = chosen;
  const float s = a.tok_s[tok];
  for (int i = t; i < a.dim; i += kArgThreads) {
    a.x[i] = (float)a.tok_q[(int64_t)tok * a.dim + i] * s;
  }
  if (t == 0) {
    *a.pos = pos + 1;
  }
}

/* Position 0: the first prompt token's embedding. */
__global__ void step_start(StepArgmaxArgs a) {
  const int tok = a.prompt[0];
  const float s = a.tok_s[tok];
  for (int i = threadIdx.x; i < a.dim; i += blockDim.x) {
    a.x[i] = (float)a.tok_q[(int64_t)tok * a.dim + i] * s;
  }
  if (threadIdx.x == 0) {
    *a.pos = 0;
  }
}

template <int kMode>
void launch_gemv(const StepGemvArgs &a, hipStream_t s) {
  const int groups = (a.rows / 2 + (kThreads / 64) - 1) / (kThreads / 64);
  hipLaunchKernelGGL((step_gemv<kMode>), dim3(groups), dim3(kThreads), 0, s, a);
}

} // namespace

bool step_gemv_ok(int rows, int cols) {
  return rows > 0 && rows % 2 == 0 && cols > 0 && cols % 16 == 0 &&
         cols <= kMaxCols;
}

void step_gemv_qkv(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kQkv>(a, s); }
void step_gemv_resid(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kResid>(a, s); }
void step_gemv_swiglu(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kSwiglu>(a, s); }
void step_gemv_logits(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kLogits>(a, s); }

void step_attention_launch(const StepAttnArgs &a, int heads, int seq_len,
                           hipStream_t s) {
  hipLaunchKernelGGL(step_attention, dim3(heads), dim3(kThreads),
                     (size_t)seq_len * sizeof(float), s, a);
}

void step_argmax_launch(const StepArgmaxArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(step_argmax, dim3(1), dim3(kArgThreads), 0, s, a);
}

void step_start_launch(const StepArgmaxArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(step_start, dim3(1), dim3(256), 0, s, a);
}

} // namespace vxk
