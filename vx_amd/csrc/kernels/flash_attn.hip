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
#include <type_traits>

namespace vxk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#define VX_LDS __attribute__((address_space(3)))

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

/* K/V planes in LDS keep global order, [key][d] in 16-byte chunks.
 * K: chunk XORed with the key's low bits so a ds_read_b128 of 16
 * consecutive keys at one chunk hits distinct banks. V: chunk XORed with a
 * function of key mod 4, so the transposing read (4 consecutive keys x 32
 * bytes per 16-lane group) hits distinct banks. */
template <int kChunks>
__device__ __forceinline__ int swz_v(int key, int c) {
  const int q = key & 3;
  if constexpr (kChunks >= 16) {
    return c ^ ((q << 1) ^ (q << 2));
  } else {
    return c ^ (q << 1);
  }
}

/* Buffer descriptor for raw 32-bit-dword loads of `bytes` bytes at `base`;
 * loads past the end return zeros. */
__device__ __forceinline__ i32x4 buffer_rsrc(const void *base, int bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xffffu);
  r[2] = bytes;
  r[3] = 0x00020000;
  return r;
}

/* One 16-byte-per-lane load straight into LDS (lane i writes lds + 16*i).
 * Assembly, so the compiler neither waits for it at every LDS read nor
 * orders it with a fenced barrier; the kernel waits with vmcnt itself. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm" /* m0 is reserved: declared */
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ void wait_all_loads() {
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); /* vmcnt(0) */
}

/* Barrier without the release fence (which would wait for the prefetch);
 * LDS reads are drained first so a slot is never refilled under a reader. */
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f); /* lgkmcnt(0) */
  asm volatile("s_barrier" ::: "memory");
}

/* x of lanes l and l ^ 32 side by side: returns the partner's value. */
__device__ __forceinline__ float other_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false,
                                                  false);
  /* Lane l < 32 finds lane l + 32's x in r[1]; lane l >= 32 finds lane
   * l - 32's in r[0]. */
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

template <int kD>
__global__ __launch_bounds__(kThreads, 2) void flash_fwd(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
    const uint16_t *__restrict__ V, uint16_t *__restrict__ O,
    float *__restrict__ LSE, int heads, int group, int seq_q, int seq_k,
    int bh_total, int q_blocks, float scale_log2, bool causal) {
  constexpr int kChunks = kD / 8;                 /* 16-byte chunks per row */
  constexpr int kUnits = kBlockK * kChunks;       /* 16-byte units per plane */
  constexpr int kLoads = kUnits / kThreads;       /* per thread per plane */
  constexpr int kDSteps = kD / 16;                /* MFMA k-steps over d */
  constexpr int kDTiles = kD / 32;                /* 32-wide d tiles of O^T */
  constexpr int kRowBytes = kD * 2;
  /* [stage][K|V][unit] */
  __shared__ u32x4 ring[2][2][kUnits];

  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
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

  /* Load offsets: unit u = (p * kThreads + t) of a plane is key u / kChunks,
   * physical chunk u % kChunks, filled from the logical chunk the swizzle
   * puts there. */
  uint32_t k_off[kLoads], v_off[kLoads];
#pragma unroll
  for (int p = 0; p < kLoads; ++p) {
    const int u = p * kThreads + t;
    const int key = u / kChunks;
    const int pc = u % kChunks;
    k_off[p] = (uint32_t)(key * kRowBytes + swz<kChunks>(key, pc) * 16);
    v_off[p] = (uint32_t)(key * kRowBytes + swz_v<kChunks>(key, pc) * 16);
  }
  const uint32_t ring_base =
      (uint32_t)(uintptr_t)(VX_LDS void *)&ring[0][0][0];
  auto issue = [&](int blk) {
    const int key0 = blk * kBlockK;
    const int bytes = min(kBlockK, seq_k - key0) * kRowBytes;
    const i32x4 rk = buffer_rsrc(K + kv_base + (int64_t)key0 * kD, bytes);
    const i32x4 rv = buffer_rsrc(V + kv_base + (int64_t)key0 * kD, bytes);
    const uint32_t base = ring_base + (uint32_t)((blk & 1) * 2 * kUnits * 16);
#pragma unroll
    for (int p = 0; p < kLoads; ++p) {
      dma16(rk, k_off[p], base + (uint32_t)(p * kThreads + wave * 64) * 16);
    }
#pragma unroll
    for (int p = 0; p < kLoads; ++p) {
      dma16(rv, v_off[p],
            base + (uint32_t)(kUnits + p * kThreads + wave * 64) * 16);
    }
  };

  /* Transposed V read: lane (g, row group j = (lane >> 4) & 1, i = lane &
   * 15) reads key 4g + 8h + i/4 of a 16-key step at d 16j + 4(i%4) of a
   * 32-wide d tile, which hands each lane the 8 keys its MFMA k-slots need
   * (the P^T order below) at d = lane % 32. */
  const int tr_key = 4 * g + ((lane & 15) >> 2);
  const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

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
  const bool scale_pos = scale_log2 >= 0.0f;

  if (nblocks > 0) {
    issue(0);
  }
  for (int blk = 0; blk < nblocks; ++blk) {
    wait_all_loads();
    lds_barrier();
    if (blk + 1 < nblocks) {
      issue(blk + 1);
    }
    const int key0 = blk * kBlockK;
    if (key0 > wave_last) {
      continue;
    }
    const u32x4 *kl = ring[blk & 1][0];
    const VX_LDS char *vl = (const VX_LDS char *)&ring[blk & 1][1][0];

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
        const u32x4 a = kl[row * kChunks + swz<kChunks>(row, 2 * ds + g)];
        st[kt] = mfma(a, qf[ds], st[kt]);
      }
    }

    /* Row max in raw scores (the scale's sign picks max or min), masked
     * keys excluded. */
    const bool need_mask =
        key0 + kBlockK > seq_k || (causal && key0 + kBlockK - 1 > qw0 + shift);
    const int limit = causal ? min(seq_k - 1, my_q + shift) : seq_k - 1;
    const float hide = scale_pos ? -INFINITY : INFINITY;
    if (need_mask) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + 32 * kt + 8 * (r >> 2) + 4 * g + (r & 3);
          st[kt][r] = key <= limit ? st[kt][r] : hide;
        }
      }
    }
    float ext = hide;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        ext = scale_pos ? fmaxf(ext, st[kt][r]) : fminf(ext, st[kt][r]);
      }
    }
    {
      const float o = other_half(ext);
      ext = scale_pos ? fmaxf(ext, o) : fminf(ext, o);
    }
    const float mx = ext == hide ? -INFINITY : ext * scale_log2;
    const float m_new = fmaxf(m_run, mx);
    /* All keys so far masked: keep exponents finite (everything is 0). */
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);

    /* P = 2^(s * scale - m); masked scores (+-inf in raw form) are set to
     * exactly 0. */
    float psum = 0.0f;
    u32x4 pt[4]; /* P^T operands for the 4 key steps of 16 */
    auto probs = [&](auto masked) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float p[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = st[kt][8 * hh + e];
            p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x, scale_log2, -m_use));
            if constexpr (decltype(masked)::value) {
              p[e] = x == hide ? 0.0f : p[e];
            }
            psum += p[e];
          }
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            pt[2 * kt + hh][w] = pack2(p[2 * w], p[2 * w + 1]);
          }
        }
      }
    };
    if (need_mask) {
      probs(std::true_type{});
    } else {
      probs(std::false_type{});
    }
    psum += other_half(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    /* Rescale O only when some lane's max moved (alpha < 1). */
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          o_acc[i][r] *= alpha;
        }
      }
    }

    /* O^T += V^T P^T over the 4 key steps. */
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int i = 0; i < kDTiles; ++i) {
        const int d = 32 * i + tr_d;
        u32x4 a;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int key = 16 * ks + tr_key + 8 * hh;
          const int at = key * kRowBytes + swz_v<kChunks>(key, d >> 3) * 16 +
                         (d & 7) * 2;
          const u32x2 w = __builtin_bit_cast(
              u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                         (VX_LDS i16x4 *)(vl + at)));
          a[2 * hh] = w[0];
          a[2 * hh + 1] = w[1];
        }
        o_acc[i] = mfma(a, pt[ks], o_acc[i]);
      }
    }
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
      out[0] = pack2(o_acc[i][4 * r4] * inv, o_acc[i][4 * r4 + 1] * inv);
      out[1] = pack2(o_acc[i][4 * r4 + 2] * inv, o_acc[i][4 * r4 + 3] * inv);
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
