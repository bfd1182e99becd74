/*
 * flash_attn.hip -- flash-attention forward on gfx950 MFMA (bf16 in, f32
 * accumulate, bf16 out, f32 log-sum-exp).
 *
 * Workgroup = 4 waves = 128 query rows of one (batch, head); each wave owns
 * 32 rows. K and V walk in blocks of 64 keys through a double-buffered LDS
 * ring, one barrier per block.
 *
 * The wave computes the transposed products so the softmax needs no
 * cross-lane data movement:
 *   S^T[key][q] = K Q^T   (v_mfma_f32_32x32x16_bf16; A = K rows from LDS,
 *                          B = Q^T, the wave's Q held in registers)
 *   O^T[d][q]  += V^T P^T (A = V^T from LDS, B = P^T straight from the S^T
 *                          accumulators)
 * In the 32x32 accumulator layout lane l holds column l % 32 -- one query --
 * so a query's running max and sum live in lane l and its partner l ^ 32:
 * the row reduction is 16 in-lane steps and one cross-lane exchange. The
 * MFMA's k-slots of lane group g = l / 32 are keys {4g..4g+3, 8+4g..8+4g+3}
 * of each 16-key step, which is exactly the key set the S^T accumulator
 * elements 8h..8h+7 of that lane hold, so P^T is S^T rounded to bf16 in
 * place. V is stored in LDS transposed ([d][key]) with the keys of each
 * 16-key step in that same order, built by an 8x4 register transpose on the
 * way in; its rows are XOR-swizzled in 16-byte chunks for conflict-free
 * ds_read_b128.
 *
 * Softmax runs in base 2 with scale * log2(e) folded into one multiply;
 * lse = (m + log2(l)) * ln 2. A row that sees no key writes o = 0 and
 * lse = -inf. Causal blocks past a wave's last visible key are skipped; the
 * diagonal and the sequence tail are masked. Workgroups start with the
 * heaviest query blocks (causal work grows with the block index) and keep a
 * head's blocks on one XCD when the head count allows.
 */
#include "../vx_hip_common.h"
#include "../vx_ops_kernels.h"

#include <cmath>

namespace vxk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kBlockQ = 128;
constexpr int kBlockK = 64;

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

/* Physical 16-byte chunk of logical chunk c in row `row` of a plane whose
 * rows have kChunks chunks. */
template <int kChunks>
__device__ __forceinline__ int swz(int row, int c) {
  if constexpr (kChunks == 16) {
    return c ^ (row & 15);
  } else {
    return c ^ (row & 7) ^ ((row >> 3) & 1);
  }
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

template <int kD>
__global__ __launch_bounds__(kThreads, 2) void flash_fwd(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
    const uint16_t *__restrict__ V, uint16_t *__restrict__ O,
    float *__restrict__ LSE, int heads, int group, int seq_q, int seq_k,
    int bh_total, int q_blocks, float scale_log2, bool causal) {
  constexpr int kKChunks = kD / 8;      /* 16-byte chunks per K row */
  constexpr int kVChunks = kBlockK / 8; /* 16-byte chunks per V^T row */
  constexpr int kDSteps = kD / 16;      /* MFMA k-steps over d */
  constexpr int kDTiles = kD / 32;      /* 32-wide d tiles of O^T */
  __shared__ u32x4 k_lds[2][kBlockK * kKChunks];
  __shared__ u32x4 v_lds[2][kD * kVChunks];

  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int lq = lane & 31;
  const int g = lane >> 5;

  /* Launch order -> (head, query block): heaviest blocks first, and one
   * head's blocks on one XCD (workgroup i runs on XCD i % 8). */
  int id = blockIdx.x;
  int bh, qb;
  if ((bh_total & 7) == 0) {
    const int xcd = id & 7;
    const int local = id >> 3;
    const int per = bh_total >> 3;
    bh = xcd + 8 * (local % per);
    qb = q_blocks - 1 - local / per;
  } else {
    bh = id % bh_total;
    qb = q_blocks - 1 - id / bh_total;
  }
  const int b = bh / heads;
  const int h = bh - b * heads;
  const int hk = h / group;
  const int kv_heads = heads / group;

  const int64_t q_base = ((int64_t)bh * seq_q) * kD;
  const int64_t kv_base = ((int64_t)(b * kv_heads + hk) * seq_k) * kD;
  const int shift = seq_k - seq_q; /* query i sees keys <= i + shift */

  const int q0 = qb * kBlockQ;
  const int qw0 = q0 + wave * 32;
  const int my_q = qw0 + lq;

  /* Keys any row of this workgroup may see, and this wave's last key. */
  int kv_end = seq_k;
  int wave_last = seq_k - 1;
  if (causal) {
    kv_end = min(seq_k, q0 + kBlockQ + shift);
    wave_last = min(seq_k - 1, qw0 + 31 + shift);
  }
  const int nblocks = kv_end > 0 ? (kv_end + kBlockK - 1) / kBlockK : 0;

  /* The wave's Q^T as MFMA B operands: lane (q = lq, group g) holds
   * d = 16s + 8g .. +8 for each d-step s. */
  u32x4 qf[kDSteps];
  {
    const bool ok = my_q < seq_q;
    const uint16_t *src = Q + q_base + (int64_t)(ok ? my_q : 0) * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < kDSteps; ++s) {
      qf[s] = ok ? *reinterpret_cast<const u32x4 *>(src + 16 * s)
                 : u32x4{0, 0, 0, 0};
    }
  }

  /* K stage: kBlockK rows x kKChunks chunks, thread-strided. */
  constexpr int kKLoads = kBlockK * kKChunks / kThreads;
  /* V stage: thread owns 8 keys (one physical group kg) x 4 d. */
  const int kg = t & 7;
  const int dg = t >> 3; /* 0..31: d = 4*dg .. +3; D = 64 uses dg < 16 */
  constexpr int kVOwners = kD / 4 * 8; /* threads with a V block */
  int vkey[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    vkey[e] = 16 * (kg >> 1) + 8 * (e >> 2) + 4 * (kg & 1) + (e & 3);
  }

  u32x4 kreg[kKLoads];
  u32x2 vreg[8];

  auto fetch = [&](int blk) {
    const int key0 = blk * kBlockK;
#pragma unroll
    for (int i = 0; i < kKLoads; ++i) {
      const int idx = t + i * kThreads;
      const int row = idx / kKChunks;
      const int c = idx - row * kKChunks;
      const int key = key0 + row;
      kreg[i] = key < seq_k ? *reinterpret_cast<const u32x4 *>(
                                  K + kv_base + (int64_t)key * kD + c * 8)
                            : u32x4{0, 0, 0, 0};
    }
    if (t < kVOwners) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = key0 + vkey[e];
        vreg[e] = key < seq_k ? *reinterpret_cast<const u32x2 *>(
                                    V + kv_base + (int64_t)key * kD + 4 * dg)
                              : u32x2{0, 0};
      }
    }
  };

  auto stash = [&](int s) {
    u32x4 *kl = k_lds[s];
#pragma unroll
    for (int i = 0; i < kKLoads; ++i) {
      const int idx = t + i * kThreads;
      const int row = idx / kKChunks;
      const int c = idx - row * kKChunks;
      kl[row * kKChunks + swz<kKChunks>(row, c)] = kreg[i];
    }
    if (t < kVOwners) {
      /* 8 keys x 4 d -> 4 rows of V^T, each one 16-byte chunk of 8 keys. */
      u32x4 *vl = v_lds[s];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int w = j >> 1;
        const bool hi = j & 1;
        u32x4 col;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const uint32_t x = vreg[2 * qd][w];
          const uint32_t y = vreg[2 * qd + 1][w];
          col[qd] = hi ? ((x >> 16) | (y & 0xffff0000u))
                       : ((x & 0xffffu) | (y << 16));
        }
        const int row = 4 * dg + j;
        vl[row * kVChunks + swz<kVChunks>(row, kg)] = col;
      }
    }
  };

  f32x16 o_acc[kDTiles];
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o_acc[i][r] = 0.0f;
    }
  }
  float m_run = -INFINITY; /* base-2 running max of this lane's query */
  float l_run = 0.0f;

  if (nblocks > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  for (int blk = 0; blk < nblocks; ++blk) {
    const int s = blk & 1;
    if (blk + 1 < nblocks) {
      fetch(blk + 1);
    }
    const int key0 = blk * kBlockK;
    if (key0 <= wave_last) {
      const u32x4 *kl = k_lds[s];
      const u32x4 *vl = v_lds[s];
      /* S^T for keys key0 + 32*kt + (row), queries qw0 + lq. */
      f32x16 st[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          st[kt][r] = 0.0f;
        }
        const int row = kt * 32 + lq;
#pragma unroll
        for (int ds = 0; ds < kDSteps; ++ds) {
          const u32x4 a = kl[row * kKChunks + swz<kKChunks>(row, 2 * ds + g)];
          st[kt] = mfma(a, qf[ds], st[kt]);
        }
      }
      /* Scale into base 2 and mask keys past the diagonal or the sequence. */
      const bool need_mask =
          key0 + kBlockK > seq_k || (causal && key0 + kBlockK - 1 > qw0 + shift);
      const int limit = causal ? min(seq_k - 1, my_q + shift) : seq_k - 1;
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = st[kt][r] * scale_log2;
          if (need_mask) {
            const int key = key0 + 32 * kt + 8 * (r >> 2) + 4 * g + (r & 3);
            x = key <= limit ? x : -INFINITY;
          }
          st[kt][r] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      /* All keys so far masked: keep exponents finite (everything is 0). */
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = exp2f(m_run - m_use);
      float psum = 0.0f;
      u32x4 pt[4]; /* P^T operands for the 4 key steps of 16 */
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float p[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            p[e] = exp2f(st[kt][8 * hh + e] - m_use);
            psum += p[e];
          }
          u32x4 v;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            v[w] = pack_bf16(p[2 * w], p[2 * w + 1]);
          }
          pt[2 * kt + hh] = v;
        }
      }
      psum += __shfl_xor(psum, 32, 64);
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          o_acc[i][r] *= alpha;
        }
      }
      /* O^T += V^T P^T over the 4 key steps. */
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int i = 0; i < kDTiles; ++i) {
          const int row = i * 32 + lq;
          const u32x4 a = vl[row * kVChunks + swz<kVChunks>(row, 2 * ks + g)];
          o_acc[i] = mfma(a, pt[ks], o_acc[i]);
        }
      }
    }
    if (blk + 1 < nblocks) {
      stash(s ^ 1);
    }
    __syncthreads();
  }

  if (my_q >= seq_q) {
    return;
  }
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  uint16_t *orow = O + q_base + (int64_t)my_q * kD;
#pragma unroll
  for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d = i * 32 + 8 * r4 + 4 * g;
      u32x2 out;
      out[0] = pack_bf16(o_acc[i][4 * r4] * inv, o_acc[i][4 * r4 + 1] * inv);
      out[1] = pack_bf16(o_acc[i][4 * r4 + 2] * inv, o_acc[i][4 * r4 + 3] * inv);
      *reinterpret_cast<u32x2 *>(orow + d) = out;
    }
  }
  if (LSE && g == 0) {
    LSE[(int64_t)bh * seq_q + my_q] =
        l_run > 0.0f ? (m_run + log2f(l_run)) * 0.69314718055994531f
                     : -INFINITY;
  }
}

} // namespace

bool flash_attn_fwd_launch(const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, uint16_t *o, float *lse,
                           int64_t batch, int64_t heads, int64_t kv_heads,
                           int64_t seq_q, int64_t seq_k, int64_t head_dim,
                           float scale, bool causal, hipStream_t stream) {
  for (const void *p : {(const void *)q, (const void *)k, (const void *)v,
                        (const void *)o}) {
    if (reinterpret_cast<uintptr_t>(p) & 15) {
      return false;
    }
  }
  if ((head_dim != 64 && head_dim != 128) || batch < 1 || heads < 1 ||
      kv_heads < 1 || heads % kv_heads || seq_q < 1 || seq_k < 1) {
    return false;
  }
  const int64_t bh = batch * heads;
  const int64_t qblocks = (seq_q + kBlockQ - 1) / kBlockQ;
  if (bh * qblocks > INT32_MAX || bh > INT32_MAX) {
    return false;
  }
  const float scale_log2 = scale * 1.4426950408889634f;
  const int group = (int)(heads / kv_heads);
  dim3 grid((unsigned)(bh * qblocks));
  if (head_dim == 128) {
    hipLaunchKernelGGL((flash_fwd<128>), grid, dim3(kThreads), 0, stream, q, k,
                       v, o, lse, (int)heads, group, (int)seq_q, (int)seq_k,
                       (int)bh, (int)qblocks, scale_log2, causal);
  } else {
    hipLaunchKernelGGL((flash_fwd<64>), grid, dim3(kThreads), 0, stream, q, k,
                       v, o, lse, (int)heads, group, (int)seq_q, (int)seq_k,
                       (int)bh, (int)qblocks, scale_log2, causal);
  }
  VX_HIP_CHECK(hipGetLastError());
  return true;
}

} // namespace vxk
