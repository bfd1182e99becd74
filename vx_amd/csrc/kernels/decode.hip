/*
 * decode.hip -- the GPU-resident token step of a Llama-2-style int8 decoder
 * (the semantics of reference examples/llama.vx:145-420).
 *
 * A step is 5 launches per layer plus 1, each reading the position from
 * device memory so that a captured step replays unchanged:
 *
 *   step_gemv<kEmbed>  (layer 0) the position's token: the prompt's, or the
 *                      argmax of the previous step's classifier candidates
 *                      (lowest index wins a tie), recorded from the end of
 *                      the prompt on; x = that token's embedding row, and
 *                      the rotary row read at pos (and stored for the other
 *                      layers); then as kQkv
 *   step_gemv<kQkv>    RMSNorm(x), [Wq; Wk; Wv] int8 GEMV, RoPE on
 *                      q and k, k and v into the KV cache at `pos`
 *   step_attention     kAttnSplit workgroups per head, each over every
 *                      kAttnSplit-th position of 0..pos: its running max,
 *                      sum of exponentials and unnormalised weighted sum of
 *                      values (flash-decoding partials)
 *   step_gemv<kAttnResid>  merges the partials into softmax(q k^T /
 *                      sqrt(hs)) v on the way in, x += Wo att
 *   step_gemv<kSwiglu> RMSNorm(x), [W1; W3] GEMV with rows interleaved,
 *                      silu(h1) * h3
 *   step_gemv<kResid>  x += W2 h
 *   step_gemv<kLogits> final RMSNorm, classifier (the embedding table);
 *                      each workgroup also leaves the best and runner-up of
 *                      its rows; pos += 1
 *
 * step_start sets up position 0 and step_record records the token that
 * follows the last step.
 *
 * Every GEMV is weight-only int8 with one f32 scale per row over f32
 * activations (as in the reference, which is f32 throughout), f32 sums;
 * each wave owns pairs of adjacent rows (one pair, two for [W1; W3], four
 * for the classifier), so the even/odd RoPE pair and the (h1, h3) SwiGLU
 * pair finish in one lane. Contraction is off
 * so the elementwise arithmetic rounds where the reference's f32 loop nest
 * rounds; the GEMV dot products, whose summation order differs from the
 * reference's anyway, use fused multiply-adds.
 */
#include "../vx_hip_common.h"
#include "../vx_decode_kernels.h"

#include <cmath>

namespace vxk {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxCols = 4096;

/* Wave-wide all-reduce with VALU data movement (DPP within 16-lane rows,
 * v_permlane16/32_swap across them) instead of LDS-crossbar shuffles. */
template <int kO> __device__ __forceinline__ float partner(float v) {
  static_assert(kO == 1 || kO == 2 || kO == 4 || kO == 8, "within a row");
  /* Lane i of a 16-lane row reads the lane differing in bit 3 (rotate by
   * 8), bit 2 (mirror within 8), bit 1 or bit 0 (quad permutes). */
  constexpr int ctrl = kO == 8 ? 0x128 : kO == 4 ? 0x141 : kO == 2 ? 0x4e : 0xb1;
  return __uint_as_float(
      __builtin_amdgcn_update_dpp(0u, __float_as_uint(v), ctrl, 0xf, 0xf, false));
}

/* Sum over groups of kN consecutive lanes (kN a power of two, <= 64); every
 * lane of a group ends with its group's sum. */
template <int kN> __device__ __forceinline__ float group_sum(float v) {
  if constexpr (kN >= 2) v += partner<1>(v);
  if constexpr (kN >= 4) v += partner<2>(v);
  if constexpr (kN >= 8) v += partner<4>(v);
  if constexpr (kN >= 16) v += partner<8>(v);
  if constexpr (kN >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                    __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (kN >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                    __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, partner<1>(v));
  v = fmaxf(v, partner<2>(v));
  v = fmaxf(v, partner<4>(v));
  v = fmaxf(v, partner<8>(v));
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                    __float_as_uint(v), false,
                                                    false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                    __float_as_uint(v), false,
                                                    false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
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

/* Best and runner-up of a set of logits; i1 is the lowest index holding
 * the best value. */
using Best = StepBest;

__device__ __forceinline__ Best merge(Best a, Best b) {
  /* selects, not branches: a merge needs no wait on loads it does not use */
  const bool bw = (b.v1 > a.v1) | ((b.v1 == a.v1) & (b.i1 < a.i1));
  Best r;
  r.v1 = bw ? b.v1 : a.v1;
  r.i1 = bw ? b.i1 : a.i1;
  r.v2 = bw ? fmaxf(a.v1, b.v2) : fmaxf(a.v2, b.v1);
  return r;
}


/* The better of a and its partner lane's Best (kO = 1, 2, 4, 8: within a
 * 16-lane row by DPP; 16, 32: across rows by v_permlane16/32_swap, which
 * hands each lane both halves' values, so merging the two gives the pair's
 * result in either order). */
template <int kO> __device__ __forceinline__ Best best_xchg(Best b) {
  if constexpr (kO <= 8) {
    Best o;
    o.v1 = partner<kO>(b.v1);
    o.i1 = __float_as_int(partner<kO>(__int_as_float(b.i1)));
    o.v2 = partner<kO>(b.v2);
    return merge(b, o);
  } else {
    auto sw = [](uint32_t x) {
      return kO == 16 ? __builtin_amdgcn_permlane16_swap(x, x, false, false)
                      : __builtin_amdgcn_permlane32_swap(x, x, false, false);
    };
    const auto v1 = sw(__float_as_uint(b.v1));
    const auto i1 = sw((uint32_t)b.i1);
    const auto v2 = sw(__float_as_uint(b.v2));
    return merge(Best{__uint_as_float(v1[0]), (int)i1[0], __uint_as_float(v2[0])},
                 Best{__uint_as_float(v1[1]), (int)i1[1], __uint_as_float(v2[1])});
  }
}


/* Classifier epilogue: the best and runner-up of this workgroup's rows
 * (each wave's lane 0 holds its own in `b`) into part[blockIdx.x], for the
 * next step's token choice (step_gemv_embed, or step_record) to merge. */
template <int kWaves>
__device__ void logits_best(const StepGemvArgs &a, Best b) {
  __shared__ Best wbest[kWaves];
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  if (lane == 0) {
    wbest[wave] = b;
  }
  __syncthreads();
  if (t == 0) {
    Best m = wbest[0];
    for (int w = 1; w < kWaves; ++w) {
      m = merge(m, wbest[w]);
    }
    a.part[blockIdx.x] = m;
  }
}

enum Mode { kQkv = 0, kResid = 1, kSwiglu = 2, kLogits = 3, kAttnResid = 4, kEmbed = 5 };

/* Classifier candidates each thread of the kEmbed GEMV requests before the
 * weights (4 x 256 threads: vocabularies up to 32768 with 16 rows per
 * candidate); any further ones are read after them. */
constexpr int kEmbedCand = 4;

/* Cache policy of the weight loads (0: default; 2: non-temporal). */
#ifndef VX_DEC_W_CPOL
#define VX_DEC_W_CPOL 0
#endif
/* Row pairs per wave: the classifier's waves take several, so its
 * thousands of rows need fewer workgroups (one round over the CUs); the
 * [W1; W3] GEMV's take two, so half as many waves each load and normalise
 * the input row for the same weights (config 4, graph mode, two rounds:
 * 1 pair 4867-4871 tok/s, 2 pairs 4946-4951, 4 pairs 4773-4774). Two
 * pairs for the QKV GEMVs measured 4927-4932 against 4939-4953, for W2
 * (48 workgroups instead of 96) 4825-4828: those keep one. */
#ifndef VX_DEC_LOGIT_PAIRS
#define VX_DEC_LOGIT_PAIRS 4
#endif
#ifndef VX_DEC_SWIGLU_PAIRS
#define VX_DEC_SWIGLU_PAIRS 2
#endif
/* Key and value rows each lane of step_attention_rows requests per round
 * (two rounds in flight): 4, and 2 for launches whose positions the first
 * two rounds of 2 cover (kNearChunk; the host picks, see
 * step_attention_near). Smaller rounds make the first round, requested
 * before the position is known, and each round's arithmetic cheaper; larger
 * ones need fewer round trips at long caches. Config 4, graph mode: 4 and
 * 2 about 3% faster than 8 (whose first round fetches 64 KiB per workgroup
 * before the position is known); 2 at every position 5013-5015 tok/s
 * against 4949-4952 for 4, and 1 at every position 4964-4968. */
#ifndef VX_ATTN_CHUNK
#define VX_ATTN_CHUNK 4
#endif
constexpr int kNearChunk = 2;
/* The GEMVs' dot products with fused multiply-adds (1) or a multiply and an
 * add per term (0). Their summation order differs from the reference's loop
 * in either case; the elementwise arithmetic stays unfused. Fused: one VALU
 * instruction per weight fewer after the weights land; config-4 decode 2%
 * faster in paired runs (graph 4534 -> 4638 tok/s), tokens identical over
 * 900 steps. */
#ifndef VX_DEC_DOT_FMA
#define VX_DEC_DOT_FMA 1
#endif
#ifndef VX_DEC_QKV_PAIRS
#define VX_DEC_QKV_PAIRS 1
#endif
#ifndef VX_DEC_RESID_PAIRS
#define VX_DEC_RESID_PAIRS 1
#endif
/* Waves per workgroup of each GEMV: 4 (256 threads), but 2 for the QKV
 * GEMVs of layers 1-11 (576 workgroups of one row pair per wave) and for
 * W2 (192 workgroups). Config 4, graph mode, variants interleaved on one
 * box (tok/s):
 *   QKV 4 / 2 / 1 waves: 4928-4932 / 4961 / 4965-4971, and on another box
 *     4 / 2: 4994-5001 / 5019-5025;
 *   [W1; W3] 2 / 8 waves: 4887-4894 / 4773-4776 against 4994-5001 at 4;
 *   W2 1 / 2 / 8 waves: 5094-5098 / 5111-5115 / 4894-4900 against
 *     5050-5057 at 4;
 *   Wo 2 / 8 waves: 4734-4745 / 5055-5057 against 5055-5056 at 4 (each Wo
 *     workgroup merges every column's attention partials, so more
 *     workgroups repeat that work);
 *   the classifier 2 / 8 waves: 5021-5022 / 5055-5057, layer 0's QKV 2
 *     waves: 5031-5035, against 5055-5056 at 4. */
#ifndef VX_DEC_QKV_WAVES
#define VX_DEC_QKV_WAVES 2
#endif
#ifndef VX_DEC_SWIGLU_WAVES
#define VX_DEC_SWIGLU_WAVES 4
#endif
#ifndef VX_DEC_RESID_WAVES
#define VX_DEC_RESID_WAVES 2
#endif
#ifndef VX_DEC_WO_WAVES
#define VX_DEC_WO_WAVES 4
#endif
#ifndef VX_DEC_LOGIT_WAVES
#define VX_DEC_LOGIT_WAVES 4
#endif
#ifndef VX_DEC_EMBED_WAVES
#define VX_DEC_EMBED_WAVES 4
#endif
template <int kMode> constexpr int group_threads() {
  return 64 * (kMode == kQkv          ? VX_DEC_QKV_WAVES
               : kMode == kSwiglu     ? VX_DEC_SWIGLU_WAVES
               : kMode == kResid      ? VX_DEC_RESID_WAVES
               : kMode == kAttnResid  ? VX_DEC_WO_WAVES
               : kMode == kLogits     ? VX_DEC_LOGIT_WAVES
                                      : VX_DEC_EMBED_WAVES);
}
template <int kMode> constexpr int pairs_per_wave() {
  return kMode == kLogits   ? VX_DEC_LOGIT_PAIRS
         : kMode == kSwiglu ? VX_DEC_SWIGLU_PAIRS
         : kMode == kQkv    ? VX_DEC_QKV_PAIRS
         : kMode == kResid  ? VX_DEC_RESID_PAIRS
                            : 1;
}

/* The results of the row pair r, r + 1 (lane 0 of the wave that owns it;
 * y0, y1 its scaled sums): q, k (with RoPE) and v at the cache position pos;
 * the residual adds x += y (res the residual's old values); or SwiGLU. */
template <int kMode>
__device__ __forceinline__ void pair_out(const StepGemvArgs &a, int r, int pos, float y0,
                                         float y1, float fcr, float fci, float res0,
                                         float res1) {
#pragma clang fp contract(off)
  if constexpr (kMode == kQkv || kMode == kEmbed) {
    const int dim = a.dim, kv_dim = a.kv_dim;
    if (r < dim + kv_dim) {
      /* RoPE on the (even, odd) pair (reference :235-264). */
      const int i = r < dim ? r : r - dim;
      const float e0 = y0 * fcr - y1 * fci;
      const float e1 = y0 * fci + y1 * fcr;
      if (r < dim) {
        a.out[r] = e0;
        a.out[r + 1] = e1;
      } else {
        a.kcache[(int64_t)pos * kv_dim + i] = e0;
        a.kcache[(int64_t)pos * kv_dim + i + 1] = e1;
      }
    } else {
      const int i = r - dim - kv_dim;
      a.vcache[(int64_t)pos * kv_dim + i] = y0;
      a.vcache[(int64_t)pos * kv_dim + i + 1] = y1;
    }
  } else if constexpr (kMode == kResid || kMode == kAttnResid) {
    a.out[r] = res0 + y0;
    a.out[r + 1] = res1 + y1;
  } else if constexpr (kMode == kSwiglu) {
    /* rows interleaved: 2i is W1 row i, 2i + 1 is W3 row i (reference
     * :377-384: val * (1 / (1 + exp(-val))) * h3). */
    float val = y0;
    const float neg = 0.0f - val;
    val = val * (1.0f / (1.0f + expf(neg)));
    val = val * y1;
    a.hout[r >> 1] = val;
  }
}

/* kSegs: 1024-column segments the kernel is built for (cols <= 1024 kSegs),
 * so registers and LDS are sized to the matrix rather than to kMaxCols. */
template <int kMode, int kSegs>
__device__ __forceinline__ void gemv_body(const StepGemvArgs &a, const StepEmbedArgs &e) {
#pragma clang fp contract(off)
  constexpr int kT = group_threads<kMode>(); /* threads per workgroup */
  constexpr int kCols = kSegs * 1024;
  __shared__ float xin[kCols];
  __shared__ float scratch[kT / 64];
  constexpr int kPairs = pairs_per_wave<kMode>();
  const int t = threadIdx.x;
  const int cols = a.cols;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int pair0 = (blockIdx.x * (kT / 64) + wave) * kPairs;
  const int r0 = pair0 * 2; /* the first (for kPairs == 1, the only) pair */
  constexpr bool kRes = kMode == kResid || kMode == kAttnResid;
  constexpr bool kQkvLike = kMode == kQkv || kMode == kEmbed;
  /* The modes whose input is a row vector read as it is (normalised or
   * not): each lane loads the 16 columns per segment that its weights
   * multiply, and a wave, whose lanes hold every column, reduces the norm's
   * sum of squares by itself. No wave waits at a workgroup barrier for
   * another wave's loads, and the input makes no LDS round trip. */
  constexpr bool kWaveIn =
      kMode == kQkv || kMode == kSwiglu || kMode == kLogits || kMode == kResid;

  /* Every load is a buffer load whose offset points past its range where
   * the element does not exist (zeros come back), so no branch surrounds a
   * load and the compiler can wait for exactly the loads it needs. Order
   * of issue = order of arrival: first this thread's inputs (x and the norm
   * weights, or the residual kernels' input vector), so the normalisation
   * runs while the weights stream; then the weights; then the epilogue's
   * operands (row scales; for the residual kernels the residual itself). */
  constexpr uint32_t kOut = 0x80000000u; /* past every range */
  constexpr int kPer = kCols / kT;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)a.w, (short)0, a.rows * cols, 0x00020000);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)a.scale, (short)0, a.rows * 4, 0x00020000);
  const int heads = kMode == kAttnResid ? cols / a.hs : 0;
  const int in_bytes =
      kMode == kAttnResid ? (kAttnSplit * cols + heads * kAttnSplit * 2) * 4 : cols * 4;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(kRes ? a.in : a.x), (short)0, in_bytes, 0x00020000);
  float xv[kPer], nv[kPer];
  /* Attention partials of this thread's columns: each split's sum, and the
   * (max, sum) pairs of the column's head, two splits per load. */
  float ov[kMode == kAttnResid ? kAttnSplit : 1][kPer];
  u32x4 ml[kMode == kAttnResid ? kPer : 1][kAttnSplit / 2];
  /* kEmbed: the previous classifier's candidates first (kEmbedCand per
   * thread; a slot past ncand loads zeros and is replaced by an empty
   * Best); the position and the prompt's token at it once the weights are
   * requested (the prompt index waits for the position); the embedding row,
   * which waits for the choice, last. */
  constexpr int kCand = kMode == kEmbed ? kEmbedCand : 1;
  float cv1[kCand], cv2[kCand];
  int ci1[kCand];
  int pos = 0;
  int ptok = 0;
  if constexpr (kMode == kEmbed) {
    const int ncand = e.tok.ncand;
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)e.tok.cand, (short)0, ncand * (int)sizeof(Best), 0x00020000);
#pragma unroll
    for (int c = 0; c < kCand; ++c) {
      const int j = t + c * kT;
      const bool ok = j < ncand;
      const uint32_t off = (uint32_t)(j * (int)sizeof(Best));
      cv1[c] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(cr, (int)(ok ? off : kOut), 0, 0));
      ci1[c] = (int)__builtin_amdgcn_raw_buffer_load_b32(cr, (int)(ok ? off + 4 : kOut), 0, 0);
      cv2[c] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(cr, (int)(ok ? off + 8 : kOut), 0, 0));
    }
  }
  /* kWaveIn: this lane's input columns s * 1024 + 16 lane .. + 15 (all
   * inside or all past cols, a multiple of 16), four floats per load. */
  u32x4 xw[kWaveIn ? kSegs : 1][4], nw[kWaveIn && !kRes ? kSegs : 1][4];
  if constexpr (kWaveIn) {
#pragma unroll
    for (int s = 0; s < kSegs; ++s) {
      const int c = s * 1024 + lane * 16;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xw[s][q] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (int)(c < cols ? (uint32_t)((c + 4 * q) * 4) : kOut), 0, 0);
      }
    }
    if constexpr (!kRes) {
      const __amdgpu_buffer_rsrc_t nr = __builtin_amdgcn_make_buffer_rsrc(
          (void *)a.norm, (short)0, cols * 4, 0x00020000);
#pragma unroll
      for (int s = 0; s < kSegs; ++s) {
        const int c = s * 1024 + lane * 16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          nw[s][q] = __builtin_amdgcn_raw_buffer_load_b128(
              nr, (int)(c < cols ? (uint32_t)((c + 4 * q) * 4) : kOut), 0, 0);
        }
      }
    }
  } else if constexpr (kMode == kAttnResid) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = t + k * kT;
      const bool ok = i < cols;
#pragma unroll
      for (int p = 0; p < kAttnSplit; ++p) {
        ov[p][k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            xr, (int)(ok ? (uint32_t)((p * cols + i) * 4) : kOut), 0, 0));
      }
      const uint32_t mo = (uint32_t)((kAttnSplit * cols + (i / a.hs) * kAttnSplit * 2) * 4);
#pragma unroll
      for (int q = 0; q < kAttnSplit / 2; ++q) {
        ml[k][q] = __builtin_amdgcn_raw_buffer_load_b128(
            xr, (int)(ok ? mo + 16 * q : kOut), 0, 0);
      }
    }
  }
  if constexpr (kMode == kEmbed) {
    const __amdgpu_buffer_rsrc_t nr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.norm, (short)0, cols * 4, 0x00020000);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = t + k * kT;
      nv[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          nr, (int)(i < cols ? (uint32_t)(i * 4) : kOut), 0, 0));
    }
  }

  u32x4 wp[kPairs][kSegs], wq[kPairs][kSegs];
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    const int r = r0 + 2 * p;
    const bool ok_r = r < a.rows;
#pragma unroll
    for (int s = 0; s < kSegs; ++s) {
      const int c = s * 1024 + lane * 16;
      const bool ok = ok_r && c < cols;
      const uint32_t off = ok ? (uint32_t)(r * cols + c) : kOut;
      wp[p][s] = __builtin_amdgcn_raw_buffer_load_b128(wr, (int)off, 0, VX_DEC_W_CPOL);
      wq[p][s] = __builtin_amdgcn_raw_buffer_load_b128(
          wr, (int)(ok ? off + (uint32_t)cols : kOut), 0, VX_DEC_W_CPOL);
    }
  }

  float sc0[kPairs], sc1[kPairs];
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    const int r = r0 + 2 * p;
    const bool ok_r = r < a.rows;
    sc0[p] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        sr, (int)(ok_r ? (uint32_t)(r * 4) : kOut), 0, 0));
    sc1[p] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        sr, (int)(ok_r ? (uint32_t)(r * 4 + 4) : kOut), 0, 0));
  }
  if constexpr (kMode == kEmbed) {
    /* keep the position's round trip behind every weight request */
    __builtin_amdgcn_sched_barrier(0);
    pos = *a.pos;
    ptok = e.tok.prompt[min(pos, e.tok.n_prompt - 1)]; /* clamped: no branch */
  }
  float res0[kPairs], res1[kPairs];
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    res0[p] = 0.0f;
    res1[p] = 0.0f;
  }
  if constexpr (kRes) {
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.out, (short)0, a.rows * 4, 0x00020000);
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      const int r = r0 + 2 * p;
      const bool ok = r < a.rows;
      res0[p] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rr, (int)(ok ? (uint32_t)(r * 4) : kOut), 0, 0));
      res1[p] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rr, (int)(ok ? (uint32_t)(r * 4 + 4) : kOut), 0, 0));
    }
  }
  if constexpr (kMode == kAttnResid) {
    /* Keep the merge's arithmetic behind every load: scheduled earlier, it
     * would wait for the partials before the weights are requested. */
    __builtin_amdgcn_sched_barrier(0);
  }

  /* The rotary factors of this wave's (even, odd) pair at this step's
   * position. Layer 0 (kEmbed) reads them from the table at pos, which it
   * loaded first, and workgroup 0 also takes the whole row (ropev) to store
   * it for the other layers, whose a.rope then holds it: those request
   * theirs behind the weights without waiting for the position. */
  float fcr[kPairs], fci[kPairs], ropev = 0.0f;
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    fcr[p] = 0.0f;
    fci[p] = 0.0f;
  }
  if constexpr (kQkvLike) {
    const bool embed = kMode == kEmbed;
    const int row0 = embed ? pos * a.hs : 0; /* first float of the row */
    const __amdgpu_buffer_rsrc_t ropr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(embed ? e.rope_table : a.rope), (short)0,
        (embed ? e.seq_len : 1) * a.hs * 4, 0x00020000);
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      const int r = r0 + 2 * p;
      const int i = r < a.dim ? r : r - a.dim;
      const bool rot = r < a.rows && r < a.dim + a.kv_dim;
      const uint32_t roff = rot ? (uint32_t)((row0 + i % a.hs) * 4) : kOut;
      fcr[p] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ropr, (int)roff, 0, 0));
      fci[p] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(ropr, (int)(rot ? roff + 4 : kOut), 0, 0));
    }
    if constexpr (embed) {
      const bool mine = blockIdx.x == 0 && t < a.hs;
      ropev = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          ropr, (int)(mine ? (uint32_t)((row0 + t) * 4) : kOut), 0, 0));
    }
  }
  /* kWaveIn: the input of this lane's columns, normalised for the norm
   * modes. */
  float xn[kWaveIn ? kSegs : 1][16];
  if constexpr (kWaveIn) {
    if constexpr (kMode == kQkv) {
      pos = *a.pos; /* where k and v go in the cache */
    }
    if constexpr (kRes) {
#pragma unroll
      for (int s = 0; s < kSegs; ++s) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          xn[s][k] = __uint_as_float(xw[s][k >> 2][k & 3]);
        }
      }
    } else {
      /* RMSNorm as reference examples/llama.vx:145-158. */
      float ss = 0.0f;
#pragma unroll
      for (int s = 0; s < kSegs; ++s) {
        if (s * 1024 + lane * 16 < cols) {
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const float v = __uint_as_float(xw[s][k >> 2][k & 3]);
            ss += v * v;
          }
        }
      }
      ss = wave_sum(ss);
      const float inv = 1.0f / sqrtf(ss / (float)cols + 0.00001f);
#pragma unroll
      for (int s = 0; s < kSegs; ++s) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          xn[s][k] = __uint_as_float(nw[s][k >> 2][k & 3]) *
                     (inv * __uint_as_float(xw[s][k >> 2][k & 3]));
        }
      }
    }
  } else if constexpr (kMode == kAttnResid) {
    /* softmax(scores) v = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M),
     * M the largest split max (an empty split has m = -inf, l = o = 0). */
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = t + k * kT;
      float mv[kAttnSplit], lv[kAttnSplit];
#pragma unroll
      for (int p = 0; p < kAttnSplit; ++p) {
        mv[p] = __uint_as_float(ml[k][p >> 1][2 * (p & 1)]);
        lv[p] = __uint_as_float(ml[k][p >> 1][2 * (p & 1) + 1]);
      }
      float mx = mv[0];
#pragma unroll
      for (int p = 1; p < kAttnSplit; ++p) {
        mx = fmaxf(mx, mv[p]);
      }
      float num = 0.0f, den = 0.0f;
#pragma unroll
      for (int p = 0; p < kAttnSplit; ++p) {
        const float w = expf(mv[p] - mx);
        num = num + ov[p][k] * w;
        den = den + lv[p] * w;
      }
      /* Stored whatever i (xin holds kCols >= cols floats; columns from
       * cols on are never read): a branch here would let the compiler sink
       * this column's loads behind the weights. */
      xin[i] = num / den;
    }
  } else {
    static_assert(kMode == kEmbed, "the other modes take kWaveIn");
    {
      /* This position's token: the merge of the candidates (every thread
       * ends with the same Best: the waves exchange theirs through LDS and
       * each thread merges them in the same order). */
      __shared__ Best wb[kT / 64];
      Best b{-INFINITY, 0x7fffffff, -INFINITY};
#pragma unroll
      for (int c = 0; c < kCand; ++c) {
        const bool ok = t + c * kT < e.tok.ncand;
        b = merge(b, Best{ok ? cv1[c] : -INFINITY, ok ? ci1[c] : 0x7fffffff,
                          ok ? cv2[c] : -INFINITY});
      }
      for (int j = t + kCand * kT; j < e.tok.ncand; j += kT) {
        b = merge(b, e.tok.cand[j]);
      }
      b = best_xchg<1>(b);
      b = best_xchg<2>(b);
      b = best_xchg<4>(b);
      b = best_xchg<8>(b);
      b = best_xchg<16>(b);
      b = best_xchg<32>(b);
      if (lane == 0) {
        wb[wave] = b;
      }
      __syncthreads();
      Best r = wb[0];
#pragma unroll
      for (int w = 1; w < kT / 64; ++w) {
        r = merge(r, wb[w]);
      }
      const bool prompt = pos < e.tok.n_prompt;
      if (blockIdx.x == 0 && t == 0 && !prompt) {
        const int at = pos - e.tok.n_prompt;
        if (at < e.tok.out_cap) {
          e.tok.out_tokens[at] = r.i1;
          e.tok.out_margin[at] = r.v1 - r.v2;
        }
      }
      /* Every logit NaN leaves no winner (index 0x7fffffff): read row 0
       * rather than past the table; the NaN margin reports it. */
      int tok = prompt ? ptok : r.i1;
      tok = tok >= 0 && tok < e.tok.vocab ? tok : 0;
      tok = __builtin_amdgcn_readfirstlane(tok);
      const __amdgpu_buffer_rsrc_t er = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(e.tok.tok_q + (int64_t)tok * cols), (short)0, cols, 0x00020000);
      const float es = e.tok.tok_s[tok];
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int i = t + k * kT;
        const int8_t e = (int8_t)__builtin_amdgcn_raw_buffer_load_b8(
            er, (int)(i < cols ? (uint32_t)i : kOut), 0, 0);
        xv[k] = (float)e * es;
      }
      if (blockIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int i = t + k * kT;
          if (i < cols) {
            e.xout[i] = xv[k];
          }
        }
      }
    }
    /* RMSNorm as reference examples/llama.vx:145-158. */
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (t + k * kT < cols) {
        ss += xv[k] * xv[k];
      }
    }
    ss = block_sum(ss, scratch);
    const float inv = 1.0f / sqrtf(ss / (float)cols + 0.00001f);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = t + k * kT;
      if (i < cols) {
        xin[i] = nv[k] * (inv * xv[k]);
      }
    }
  }
  if constexpr (!kWaveIn) {
    __syncthreads();
  }

  float acc0 = 0.0f, acc1 = 0.0f;
  Best best{-INFINITY, 0x7fffffff, -INFINITY};
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    acc0 = 0.0f;
    acc1 = 0.0f;
#pragma unroll
    for (int s = 0; s < kSegs; ++s) {
      const int c = s * 1024 + lane * 16;
      if (c < cols) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const float xv = kWaveIn ? xn[s][k] : xin[c + k];
          const float w0 = (float)(int8_t)(wp[p][s][k >> 2] >> (8 * (k & 3)));
          const float w1 = (float)(int8_t)(wq[p][s][k >> 2] >> (8 * (k & 3)));
#if VX_DEC_DOT_FMA
          acc0 = __builtin_fmaf(w0, xv, acc0);
          acc1 = __builtin_fmaf(w1, xv, acc1);
#else
          acc0 += w0 * xv;
          acc1 += w1 * xv;
#endif
        }
      }
    }
    acc0 = wave_sum(acc0);
    acc1 = wave_sum(acc1);
    if constexpr (kMode == kLogits) {
      const int r = r0 + 2 * p;
      if (lane == 0 && r < a.rows) {
        const float y0 = sc0[p] * acc0;
        const float y1 = sc1[p] * acc1;
        a.out[r] = y0;
        a.out[r + 1] = y1;
        best = merge(best, Best{y0, r, -INFINITY});
        best = merge(best, Best{y1, r + 1, -INFINITY});
      }
    }
    if constexpr (kMode != kLogits) {
      /* this pair's results out as its sums land */
      const int r = r0 + 2 * p;
      if (lane == 0 && r < a.rows) {
        pair_out<kMode>(a, r, pos, sc0[p] * acc0, sc1[p] * acc1, fcr[p], fci[p], res0[p],
                        res1[p]);
      }
    }
  }
  if constexpr (kMode == kLogits) {
    /* The next step's position: a vector atomic, nothing waits for it (no
     * other workgroup of this launch reads pos). */
    if (blockIdx.x == 0 && t == 0) {
      atomicAdd(a.pos, 1);
    }
    logits_best<kT / 64>(a, best);
    return;
  }
  if constexpr (kMode == kEmbed) {
    if (blockIdx.x == 0 && t < a.hs) {
      e.rope_out[t] = ropev;
    }
  }
}

template <int kMode, int kSegs>
__global__ __launch_bounds__(group_threads<kMode>()) void step_gemv(StepGemvArgs a) {
  gemv_body<kMode, kSegs>(a, StepEmbedArgs{});
}

template <int kSegs>
__global__ __launch_bounds__(group_threads<kEmbed>()) void step_gemv_embed(StepGemvArgs a,
                                                                           StepEmbedArgs e) {
  gemv_body<kEmbed, kSegs>(a, e);
}

/* Workgroup (h, sp) of query head h over positions sp, sp + kAttnSplit,
 * ... up to pos (reference :275-325, split flash-decoding style so that
 * kAttnSplit CUs share a head's key and value rows); scores in dynamic LDS,
 * indexed by m for position sp + kAttnSplit m. It leaves its max M, its
 * sum of e^(score - M) and its unnormalised weighted sum of values; the Wo
 * GEMV merges the splits.
 *
 * Scores: kL lanes share a position, each taking kE consecutive elements of
 * the head (hs = kE * kL), so a wave reads 64 / kL whole key rows with one
 * coalesced load; a lane sums its kE products in order and the kL lanes add
 * theirs by DPP, eight key rows per lane in flight. Values: a lane owns
 * four consecutive elements of the head (one float4; one element for heads
 * under 16), the lane groups take positions round-robin, each adds its
 * positions in increasing order with eight rows in flight, and the groups'
 * partial sums meet in LDS. */
template <int kE, int kL>
__global__ __launch_bounds__(kThreads) void step_attention(StepAttnArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float score[];
  __shared__ float qs[256];
  __shared__ float part[kThreads * 4];
  __shared__ float scratch[kThreads / 64];
  constexpr int kPerWave = 64 / kL; /* positions one wave scores at a time */
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int h = blockIdx.x;
  const int sp = blockIdx.y;
  const int hs = kE * kL;
  const int hk = h / a.kv_mul;
  const int sub = lane % kL;  /* this lane's slice of the head */
  const int slot = lane / kL; /* which of the wave's positions */
  /* kChunk rows of keys per lane in flight at once (a wave covers
   * kChunk * kPerWave positions per round trip to memory). */
  constexpr int kChunk = 8;
  constexpr int kStride = 4 * kPerWave; /* positions between a wave's rows */
  /* The layer's caches as buffer ranges: a load past `bound` gets an
   * offset past the range and returns zeros, so no branch surrounds a load
   * (a branch would make the compiler wait for each load at the join). */
  const int cache_bytes = a.seq_len * a.kv_dim * 4;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)a.kcache, (short)0, cache_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)a.vcache, (short)0, cache_bytes, 0x00020000);
  constexpr uint32_t kOut = 0x80000000u; /* past every range */
  auto key_rows = [&](int m0, int bound, float (&kv)[kChunk][kE]) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int m = m0 + c * kStride + slot;
      const int j = sp + kAttnSplit * m;
      const uint32_t off =
          m < bound ? (uint32_t)((j * a.kv_dim + hk * hs + sub * kE) * 4) : kOut;
      if constexpr (kE == 4) {
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)off, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kv[c][e] = __uint_as_float(w[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < kE; ++e) {
          kv[c][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
              krs, (int)(off == kOut ? kOut : off + 4 * e), 0, 0));
        }
      }
    }
  };
  /* Values: a lane owns kVec consecutive elements of a position's row
   * (float4 where the head allows), so a wave reads whole rows; the lane
   * groups take positions round-robin. */
  constexpr int kHs = kE * kL;
  constexpr int kVec = (kHs % 4 == 0 && kHs >= 16) ? 4 : 1;
  constexpr int kRowLanes = kHs / kVec;
  constexpr int kGroups = kThreads / kRowLanes;
  constexpr int kRows = 8; /* value rows per lane in flight */
  const int g = t / kRowLanes;
  const int i = (t - g * kRowLanes) * kVec;
  /* Value row of local index mm (position sp + kAttnSplit mm), zeros from
   * mm >= bound. */
  auto row = [&](int mm, int bound, float (&v)[kVec]) {
    const int jj = sp + kAttnSplit * mm;
    const uint32_t off =
        mm < bound ? (uint32_t)((jj * a.kv_dim + hk * hs + i) * 4) : kOut;
    if constexpr (kVec == 4) {
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)off, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = __uint_as_float(w[e]);
      }
    } else {
      v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(vrs, (int)off, 0, 0));
    }
  };

  /* q, the first chunk of key rows and the first value rows do not depend
   * on the position: they are requested together with it, bounded by the
   * cache's length rather than by pos (rows past pos are never used). */
  const float qt = t < hs ? a.q[h * hs + t] : 0.0f;
  const int ms = (a.seq_len - sp + kAttnSplit - 1) / kAttnSplit; /* split's rows < seq_len */
  float kv0[kChunk][kE];
  key_rows(wave * kPerWave, ms, kv0);
  float v0[kRows][kVec];
#pragma unroll
  for (int u = 0; u < kRows; ++u) {
    row(g + u * kGroups, ms, v0[u]);
  }
  const int pos = *a.pos;
  /* This split's positions: sp + kAttnSplit m for m < n (none if sp > pos). */
  const int n = pos >= sp ? (pos - sp) / kAttnSplit + 1 : 0;
  if (t < hs) {
    qs[t] = qt;
  }
  __syncthreads();
  const float root = sqrtf((float)hs);
  float qv[kE];
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    qv[e] = qs[sub * kE + e];
  }
  float mx = -INFINITY;
  auto score_chunk = [&](int j0, const float (&kv)[kChunk][kE]) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int j = j0 + c * kStride + slot; /* local index */
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < kE; ++e) {
        dot = dot + qv[e] * kv[c][e];
      }
      dot = group_sum<kL>(dot);
      if (j < n) {
        const float sc = dot / root;
        if (sub == 0) {
          score[j] = sc;
        }
        mx = fmaxf(mx, sc);
      }
    }
  };
  score_chunk(wave * kPerWave, kv0);
  for (int j0 = wave * kPerWave + kStride * kChunk; j0 < n; j0 += kStride * kChunk) {
    float kv[kChunk][kE];
    key_rows(j0, n, kv);
    score_chunk(j0, kv);
  }
  mx = block_max(mx, scratch); /* also orders the score writes */
  float sum = 0.0f;
  for (int j = t; j < n; j += kThreads) {
    const float p = expf(score[j] - mx);
    score[j] = p;
    sum += p;
  }
  sum = block_sum(sum, scratch); /* also orders the probability writes */
  float acc[kVec];
#pragma unroll
  for (int e = 0; e < kVec; ++e) {
    acc[e] = 0.0f;
  }
  /* Each group adds its positions in increasing order: the preloaded rows
   * first, then eight rows in flight at a time, then the tail. */
#pragma unroll
  for (int u = 0; u < kRows; ++u) {
    const int jj = g + u * kGroups;
    if (jj < n) {
      const float p = score[jj];
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        acc[e] = acc[e] + p * v0[u][e];
      }
    }
  }
  int j = g + kRows * kGroups;
  for (; j + (kRows - 1) * kGroups < n; j += kRows * kGroups) {
    float v[kRows][kVec];
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      row(j + u * kGroups, n, v[u]);
    }
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      const float p = score[j + u * kGroups];
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        acc[e] = acc[e] + p * v[u][e];
      }
    }
  }
  for (; j < n; j += kGroups) {
    float v[kVec];
    row(j, n, v);
    const float p = score[j];
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      acc[e] = acc[e] + p * v[e];
    }
  }
#pragma unroll
  for (int e = 0; e < kVec; ++e) {
    part[g * kHs + i + e] = acc[e];
  }
  __syncthreads();
  const int dim = gridDim.x * hs;
  if (t < hs) {
    float o = 0.0f;
    for (int gg = 0; gg < kGroups; ++gg) {
      o += part[gg * kHs + t];
    }
    a.part[sp * dim + h * hs + t] = o;
  }
  if (t == 0) {
    a.part[kAttnSplit * dim + (h * kAttnSplit + sp) * 2] = mx;
    a.part[kAttnSplit * dim + (h * kAttnSplit + sp) * 2 + 1] = sum;
  }
}

/* Sum over the lanes that share lane % kL (partners at xor kL, 2 kL, ...,
 * 32), each an exact xor pairing for kL >= 8. */
template <int kL> __device__ __forceinline__ float slot_sum(float v) {
  static_assert(kL >= 8 && kL <= 64, "xor partners from 8 up");
  if constexpr (kL <= 8) v += partner<8>(v);
  if constexpr (kL <= 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                    __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (kL <= 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                    __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return v;
}

/* The same partials as step_attention for heads of 32 to 256 (kL = hs / 4
 * lanes per position, 4 elements each), with each wave's softmax kept in
 * registers: the kL lanes that score a position also hold that position's
 * value row (the same float4 slice of it), so the probability never leaves
 * them. Wave w takes the split's local rows w * 64/kL + slot + c * 256/kL
 * (c < kChunk) of each round, keys and values requested together; rounds
 * repeat with the usual online rescale while positions remain, the next
 * round's rows in flight while one is scored. The four waves' (max, sum,
 * weighted values) then meet once in LDS. */
template <int kL, int kChunk> /* kChunk: rows per lane in flight */
__global__ __launch_bounds__(kThreads) void step_attention_rows(StepAttnArgs a) {
#pragma clang fp contract(off)
  constexpr int kE = 4;
  constexpr int hs = kE * kL;
  constexpr int kPerWave = 64 / kL;       /* positions a wave scores at once */
  constexpr int kStride = 4 * kPerWave;   /* local rows between a wave's rows */
  constexpr int kRound = kStride * kChunk; /* local rows per round */
  __shared__ float wo[4][hs];
  __shared__ float wm[4], wl[4];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int h = blockIdx.x;
  const int sp = blockIdx.y;
  const int hk = h / a.kv_mul;
  const int sub = lane % kL;
  const int slot = lane / kL;
  constexpr uint32_t kOut = 0x80000000u; /* past every range */
  const int cache_bytes = a.seq_len * a.kv_dim * 4;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)a.kcache, (short)0, cache_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)a.vcache, (short)0, cache_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)a.q, (short)0, (int)gridDim.x * hs * 4, 0x00020000);
  const uint32_t col = (uint32_t)((hk * hs + sub * kE) * 4);
  /* Key and value slices of this lane's rows of round r0; zeros from local
   * row `bound` on. */
  auto load_rows = [&](int r0, int bound, u32x4 (&kw)[kChunk], u32x4 (&vw)[kChunk]) {
    const int m0 = r0 + wave * kPerWave + slot;
    const uint32_t row_bytes = (uint32_t)a.kv_dim * 4;
    const uint32_t base = (uint32_t)(sp + kAttnSplit * m0) * row_bytes + col;
    const uint32_t step = (uint32_t)(kStride * kAttnSplit) * row_bytes;
    uint32_t off[kChunk];
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      off[c] = m0 + c * kStride < bound ? base + (uint32_t)c * step : kOut;
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      kw[c] = __builtin_amdgcn_raw_buffer_load_b128(krs, (int)off[c], 0, 0);
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      vw[c] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)off[c], 0, 0);
    }
  };

  /* q and the first round's rows do not depend on the position: requested
   * with it, bounded by the cache's length (rows past pos are never used). */
  const u32x4 qw = __builtin_amdgcn_raw_buffer_load_b128(
      qrs, (int)((h * hs + sub * kE) * 4), 0, 0);
  const int ms = (a.seq_len - sp + kAttnSplit - 1) / kAttnSplit;
  /* Two rounds of rows in flight: round r + 1 is requested before round r
   * is scored, so a long cache costs one memory round trip per two rounds
   * rather than one per round. The first round does not depend on the
   * position; the second is requested as soon as the position is known
   * (all of it past n, so no memory traffic, when one round covers n). */
  u32x4 kw0[kChunk], vw0[kChunk], kw1[kChunk], vw1[kChunk];
  load_rows(0, ms, kw0, vw0);
  const int pos = *a.pos;
  const int n = pos >= sp ? (pos - sp) / kAttnSplit + 1 : 0;
  load_rows(kRound, n, kw1, vw1);
  const float root = sqrtf((float)hs);
  float q[kE];
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    q[e] = __uint_as_float(qw[e]);
  }
  float m_run = -INFINITY, l_run = 0.0f, acc[kE];
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    acc[e] = 0.0f;
  }
  /* Scores of round r0's rows, then the online-softmax update of this
   * wave's max, sum and weighted values. */
  auto score_round = [&](int r0, const u32x4 (&kw)[kChunk], const u32x4 (&vw)[kChunk]) {
    float sc[kChunk];
    float mr = -INFINITY;
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int m = r0 + wave * kPerWave + c * kStride + slot;
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < kE; ++e) {
        dot = dot + q[e] * __uint_as_float(kw[c][e]);
      }
      dot = group_sum<kL>(dot);
      sc[c] = dot / root;
      mr = m < n ? fmaxf(mr, sc[c]) : mr;
    }
    mr = wave_max(mr);
    const float mnew = fmaxf(m_run, mr);
    if (mnew != -INFINITY) { /* wave-uniform: some row of this wave is live */
      const float alpha = expf(m_run - mnew); /* 0 while m_run is -inf */
      float ps = 0.0f;
#pragma unroll
      for (int e = 0; e < kE; ++e) {
        acc[e] = acc[e] * alpha;
      }
#pragma unroll
      for (int c = 0; c < kChunk; ++c) {
        const int m = r0 + wave * kPerWave + c * kStride + slot;
        const bool live = m < n;
        const float p = live ? expf(sc[c] - mnew) : 0.0f;
        ps = ps + p;
        /* Rows from n on were loaded (bounded by the cache's length) but
         * never written: their bits may be Inf or NaN, and 0 * Inf is NaN,
         * so they are selected away rather than multiplied by zero. */
#pragma unroll
        for (int e = 0; e < kE; ++e) {
          const float pv = p * __uint_as_float(vw[c][e]);
          acc[e] = acc[e] + (live ? pv : 0.0f);
        }
      }
      l_run = l_run * alpha + ps;
      m_run = mnew;
    }
  };
  for (int r0 = 0;; r0 += 2 * kRound) {
    score_round(r0, kw0, vw0);
    if (r0 + kRound >= n) {
      break;
    }
    load_rows(r0 + 2 * kRound, n, kw0, vw0);
    score_round(r0 + kRound, kw1, vw1);
    if (r0 + 2 * kRound >= n) {
      break;
    }
    load_rows(r0 + 3 * kRound, n, kw1, vw1);
  }
  /* Every lane of a slot holds that slot's sums: add the slots. */
  l_run = slot_sum<kL>(l_run);
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    acc[e] = slot_sum<kL>(acc[e]);
  }
  if (slot == 0) {
#pragma unroll
    for (int e = 0; e < kE; ++e) {
      wo[wave][sub * kE + e] = acc[e];
    }
  }
  if (lane == 0) {
    wm[wave] = m_run;
    wl[wave] = l_run;
  }
  __syncthreads();
  const int dim = gridDim.x * hs;
  if (t < hs) {
    float mx = wm[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      mx = fmaxf(mx, wm[w]);
    }
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = wm[w] == -INFINITY ? 0.0f : expf(wm[w] - mx);
      o = o + wo[w][t] * f;
      l = l + wl[w] * f;
    }
    a.part[sp * dim + h * hs + t] = o;
    if (t == 0) {
      a.part[kAttnSplit * dim + (h * kAttnSplit + sp) * 2] = mx;
      a.part[kAttnSplit * dim + (h * kAttnSplit + sp) * 2 + 1] = l;
    }
  }
}

constexpr int kChooseThreads = 1024;

/* The token after the last step: the argmax of the last classifier's
 * candidates (lowest index wins a tie, reference examples/llama.vx:160-171),
 * recorded for position *pos, which the last classifier moved past the
 * prompt; the steps themselves record the tokens before it. */
__global__ __launch_bounds__(kChooseThreads) void step_record(StepArgmaxArgs a) {
  __shared__ Best merged[kChooseThreads / 64];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int nparts = a.tok.ncand;
  Best b{-INFINITY, 0x7fffffff, -INFINITY};
  for (int i = t; i < nparts; i += kChooseThreads) {
    b = merge(b, a.tok.cand[i]);
  }
  b = best_xchg<1>(b);
  b = best_xchg<2>(b);
  b = best_xchg<4>(b);
  b = best_xchg<8>(b);
  b = best_xchg<16>(b);
  b = best_xchg<32>(b);
  if (lane == 0) {
    merged[t >> 6] = b;
  }
  __syncthreads();
  if (t == 0) {
    Best r = merged[0];
    for (int w = 1; w < kChooseThreads / 64; ++w) {
      r = merge(r, merged[w]);
    }
    const int pos = *a.pos;
    const int at = pos - a.tok.n_prompt;
    if (at >= 0 && at < a.tok.out_cap) {
      a.tok.out_tokens[at] = r.i1;
      a.tok.out_margin[at] = r.v1 - r.v2;
    }
  }
}

/* Position 0; layer 0 of the first step reads its token and rotary row. */
__global__ void step_start(StepArgmaxArgs a) {
  if (threadIdx.x == 0) {
    *a.pos = 0;
  }
}

template <int kMode> int gemv_groups(int rows) {
  constexpr int kPerGroup = (group_threads<kMode>() / 64) * pairs_per_wave<kMode>();
  return (rows / 2 + kPerGroup - 1) / kPerGroup;
}

template <int kMode>
void launch_gemv(const StepGemvArgs &a, hipStream_t s) {
  const dim3 grid(gemv_groups<kMode>(a.rows));
  const dim3 block(group_threads<kMode>());
  if (a.cols <= 1024) {
    hipLaunchKernelGGL((step_gemv<kMode, 1>), grid, block, 0, s, a);
  } else if (a.cols <= 2048) {
    hipLaunchKernelGGL((step_gemv<kMode, 2>), grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL((step_gemv<kMode, kMaxCols / 1024>), grid, block, 0, s, a);
  }
}

void launch_embed(const StepGemvArgs &a, const StepEmbedArgs &e, hipStream_t s) {
  const dim3 grid(gemv_groups<kEmbed>(a.rows));
  const dim3 block(group_threads<kEmbed>());
  if (a.cols <= 1024) {
    hipLaunchKernelGGL((step_gemv_embed<1>), grid, block, 0, s, a, e);
  } else if (a.cols <= 2048) {
    hipLaunchKernelGGL((step_gemv_embed<2>), grid, block, 0, s, a, e);
  } else {
    hipLaunchKernelGGL((step_gemv_embed<kMaxCols / 1024>), grid, block, 0, s, a, e);
  }
}

} // namespace

bool step_gemv_ok(int rows, int cols) {
  /* The weights are one buffer range: rows * cols bytes in 31 bits. */
  return rows > 0 && rows % 2 == 0 && cols > 0 && cols % 16 == 0 &&
         cols <= kMaxCols && (int64_t)rows * cols <= INT32_MAX;
}

void step_gemv_qkv(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kQkv>(a, s); }
void step_gemv_embed(const StepGemvArgs &a, const StepEmbedArgs &e, hipStream_t s) {
  launch_embed(a, e, s);
}
void step_gemv_resid(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kResid>(a, s); }
void step_gemv_attn_resid(const StepGemvArgs &a, hipStream_t s) {
  launch_gemv<kAttnResid>(a, s);
}
void step_gemv_swiglu(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kSwiglu>(a, s); }
void step_gemv_logits(const StepGemvArgs &a, hipStream_t s) { launch_gemv<kLogits>(a, s); }

int step_logits_groups(int rows) { return gemv_groups<kLogits>(rows); }

void step_record_launch(const StepArgmaxArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(step_record, dim3(1), dim3(kChooseThreads), 0, s, a);
}

template <int kL>
void launch_rows(const StepAttnArgs &a, dim3 grid, bool near, hipStream_t s) {
  if (near) {
    hipLaunchKernelGGL((step_attention_rows<kL, kNearChunk>), grid, dim3(kThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((step_attention_rows<kL, VX_ATTN_CHUNK>), grid, dim3(kThreads), 0, s, a);
  }
}

void step_attention_launch(const StepAttnArgs &a, int heads, int seq_len,
                           hipStream_t s, bool near) {
  const size_t lds = (size_t)((seq_len + kAttnSplit - 1) / kAttnSplit) * sizeof(float);
  const dim3 grid(heads, kAttnSplit);
  switch (a.hs) {
  case 2: hipLaunchKernelGGL((step_attention<2, 1>), grid, dim3(kThreads), lds, s, a); break;
  case 4: hipLaunchKernelGGL((step_attention<4, 1>), grid, dim3(kThreads), lds, s, a); break;
  case 8: hipLaunchKernelGGL((step_attention<4, 2>), grid, dim3(kThreads), lds, s, a); break;
  case 16: hipLaunchKernelGGL((step_attention<4, 4>), grid, dim3(kThreads), lds, s, a); break;
  case 32: launch_rows<8>(a, grid, near, s); break;
  case 64: launch_rows<16>(a, grid, near, s); break;
  case 128: launch_rows<32>(a, grid, near, s); break;
  default: launch_rows<64>(a, grid, near, s); break;
  }
}

int step_attention_near(int hs) {
  if (hs < 32) {
    return 0; /* the per-thread kernel has one shape */
  }
  /* positions the first two small rounds cover: 2 rounds x (4 waves x
   * 64 / (hs / 4) positions per wave x kNearChunk) local rows x kAttnSplit */
  return 2 * 4 * (64 / (hs / 4)) * kNearChunk * kAttnSplit;
}

void step_start_launch(const StepArgmaxArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(step_start, dim3(1), dim3(64), 0, s, a);
}

} // namespace vxk
