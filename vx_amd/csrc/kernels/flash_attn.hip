/*
 * flash_attn.hip -- flash-attention forward on gfx950 MFMA (bf16 in, f32
 * accumulate, bf16 out, f32 log-sum-exp).
 *
 * Workgroup = 4 waves; each wave owns 32 * kQT query rows of one
 * (batch, head) (kQT = 1 by default: two workgroups share a CU, so one
 * wave's softmax runs beside the other's MFMAs). K and V walk in blocks of
 * kBK keys through a two-slot LDS ring filled by buffer-to-LDS loads, in
 * their global [key][d] order; one barrier per block.
 *
 * The wave computes the transposed products so the softmax needs almost no
 * cross-lane data movement:
 *   S^T[key][q] = K Q^T   (v_mfma_f32_32x32x16_bf16; A = K rows read with
 *                          ds_read_b128, B = Q^T held in registers)
 *   O^T[d][q]  += V^T P^T (A = V^T read with ds_read_b64_tr_b16 from the
 *                          [key][d] plane, B = P^T from the S^T accumulators)
 * In the 32x32 accumulator layout lane l holds column l % 32 -- one query --
 * so a query's running max and sum live in lane l and its partner l ^ 32:
 * the row reduction is in-lane plus one v_permlane32_swap. The MFMA's
 * k-slots of lane group g = l / 32 are keys {4g..4g+3, 8+4g..8+4g+3} of each
 * 16-key step, exactly the key set the S^T accumulator elements 8h..8h+7 of
 * that lane hold, so P^T is S^T converted to bf16 in place; the transposing
 * V read is addressed to hand each lane those same keys.
 *
 * Softmax runs in base 2: p = 2^(s * scale * log2(e) - m) with the scale
 * folded into one fma; lse = (m + log2(l)) * ln 2. The reference max m only
 * moves when a block's max passes it by more than 2^8, so most blocks skip
 * rescaling O. A row that sees no key writes o = 0 and lse = -inf. Causal
 * blocks past a wave's last visible key are skipped; the diagonal and the
 * sequence tail are masked. K is requested two blocks ahead and V one, so
 * the next block's score MFMAs are issued while this block's softmax runs.
 * Workgroups start with the heaviest query blocks (causal work grows with
 * the block index); each XCD keeps a few heads' K/V in its L2 at a time.
 *
 * Key splits: when the query blocks alone give fewer workgroups than one
 * round of two per CU (a 512-query prefill chunk over a long cache gives
 * 128), the key range is cut into splits, each workgroup writes its rows'
 * normalised output and log-sum-exp in f32, and a second kernel merges
 * them (the flash-decoding merge). Merging inside the split kernel (the
 * last workgroup of a block combining) measured slower: the device-scope
 * release and acquire it needs write back and invalidate the whole L2 of
 * the XCD, so the other workgroups lose their K/V lines.
 */
#include "../vx_hip_common.h"
#include "../vx_ops_kernels.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <map>
#include <mutex>
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
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#define VX_LDS __attribute__((address_space(3)))

constexpr int kThreads = 256;
/* Query tiles of 32 per wave (a workgroup of 4 waves covers 128 * kQT
 * queries) and keys per K/V block (a multiple of 32). Two tiles halve the
 * LDS operand reads per MFMA but need one wave per SIMD, which loses more
 * to exposed latency than it saves (measured: 508 vs 820 TFLOP/s for the
 * causal [4,32,2048,128] case). */
#ifndef VX_FA_QT
#define VX_FA_QT 1
#endif
#ifndef VX_FA_BK
#define VX_FA_BK 64
#endif
/* VALU instructions the scheduler places after each score MFMA in the
 * straight-line softmax region (measured best at 3 for head_dim 128). */
#ifndef VX_FA_SGB
#define VX_FA_SGB 3
#endif
/* V^T reads issued ahead of the first PV MFMA (0: the compiler's order).
 * 8 measured 1-2% faster than the compiler's order on config 3 (paired runs;
 * 4 and 12 within noise of 8). */
#ifndef VX_FA_PV_LEAD
#define VX_FA_PV_LEAD 8
#endif
constexpr float kSlack = 8.0f; /* base-2 headroom of the stale row max */
/* Heads an XCD works through together (0: all of its heads at once). */
#ifndef VX_FA_HG
#define VX_FA_HG 4
#endif
constexpr int kHeadGroup = VX_FA_HG;

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

/* x of lanes l and l ^ 32: each lane gets both values (its own and its
 * partner's, in some order), for a max or a sum across the two halves. */
__device__ __forceinline__ f32x2 halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false,
                                                  false);
  return f32x2{__uint_as_float(r[0]), __uint_as_float(r[1])};
}

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

/* kQT query tiles of 32 per wave: a wave owns 32 * kQT queries, so each K
 * and V operand read from LDS feeds kQT MFMAs. */
template <int kD, int kQT, int kBK, bool kSplit>
__global__ __launch_bounds__(kThreads, kQT == 1 ? 2 : 1) void flash_fwd(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K,
    const uint16_t *__restrict__ V, uint16_t *__restrict__ O,
    float *__restrict__ LSE, int heads, int group, int seq_q, int seq_k,
    int bh_total, int q_blocks, float scale_log2, bool causal, int splits,
    float *__restrict__ Opart, float *__restrict__ Lpart) {
  constexpr int kBlockK = kBK;                    /* keys per block */
  constexpr int kKT = kBlockK / 32;               /* 32-key tiles per block */
  constexpr int kKS = kBlockK / 16;               /* 16-key MFMA steps */
  constexpr int kChunks = kD / 8;                 /* 16-byte chunks per row */
  constexpr int kUnits = kBlockK * kChunks;       /* 16-byte units per plane */
  constexpr int kLoads = kUnits / kThreads;       /* per thread per plane */
  constexpr int kDSteps = kD / 16;                /* MFMA k-steps over d */
  constexpr int kDTiles = kD / 32;                /* 32-wide d tiles of O^T */
  constexpr int kRowBytes = kD * 2;
  constexpr int kWaveQ = 32 * kQT;                /* queries per wave */
  constexpr int kBlockQ = 4 * kWaveQ;             /* queries per workgroup */
  /* [stage][K|V][unit] */
  __shared__ u32x4 ring[2][2][kUnits];

  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63;
  const int lq = lane & 31;
  const int g = lane >> 5;

  /* Launch order -> (head, query block). Workgroup i runs on XCD i % 8, so
   * each XCD gets every 8th head; it walks them kHeadGroup heads at a time
   * (all query blocks of the group, heaviest first), which keeps the K/V of
   * only a few heads live in its L2 at once. */
  int id = blockIdx.x;
  /* Split mode: workgroup (item, sp) takes key blocks sp * per .. of its
   * item, per = ceil(key blocks of the whole sequence / splits). */
  int sp = 0;
  if constexpr (kSplit) {
    sp = id % splits;
    id /= splits;
  }
  int bh, qb;
  if ((bh_total & 7) == 0) {
    const int xcd = id & 7;
    const int local = id >> 3;
    const int per = bh_total >> 3;
    if (kHeadGroup > 0 && per % kHeadGroup == 0) {
      const int span = kHeadGroup * q_blocks;
      const int grp = local / span;
      const int in = local - grp * span;
      bh = xcd + 8 * (grp * kHeadGroup + in % kHeadGroup);
      qb = q_blocks - 1 - in / kHeadGroup;
    } else {
      bh = xcd + 8 * (local % per);
      qb = q_blocks - 1 - local / per;
    }
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
  const int qw0 = q0 + wave * kWaveQ;

  /* Keys any row of this workgroup may see, and this wave's last key. */
  int kv_end = seq_k;
  int wave_last = seq_k - 1;
  if (causal) {
    kv_end = min(seq_k, q0 + kBlockQ + shift);
    wave_last = min(seq_k - 1, qw0 + kWaveQ - 1 + shift);
  }
  int nblocks = kv_end > 0 ? (kv_end + kBlockK - 1) / kBlockK : 0;
  int first = 0; /* first key block of this workgroup */
  if constexpr (kSplit) {
    const int per = ((seq_k + kBlockK - 1) / kBlockK + splits - 1) / splits;
    first = sp * per;
    nblocks = min(nblocks, first + per);
  }

  /* The wave's Q^T as MFMA B operands: lane (q = lq, group g) of tile qt
   * holds d = 16s + 8g .. +8 of query qw0 + 32 qt + lq for each d-step s. */
  u32x4 qf[kQT][kDSteps];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const int q = qw0 + 32 * qt + lq;
    const bool ok = q < seq_q;
    const uint16_t *src = Q + q_base + (int64_t)(ok ? q : 0) * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < kDSteps; ++s) {
      qf[qt][s] = ok ? *reinterpret_cast<const u32x4 *>(src + 16 * s)
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
  /* Block b of K and of V lives in slot (b - first) % 2 of its plane
   * (counted from the workgroup's first block, so the loop below, which
   * steps two blocks at a time from there, sees constant slots). */
  auto issue = [&](int blk, int plane) {
    const int key0 = blk * kBlockK;
    const int bytes = min(kBlockK, seq_k - key0) * kRowBytes;
    const uint16_t *src = plane == 0 ? K : V;
    const i32x4 rs = buffer_rsrc(src + kv_base + (int64_t)key0 * kD, bytes);
    const uint32_t *off = plane == 0 ? k_off : v_off;
    const uint32_t base =
        ring_base + (uint32_t)(((((blk - first) & 1) * 2 + plane) * kUnits + wave * 64) * 16);
#pragma unroll
    for (int p = 0; p < kLoads; ++p) {
      dma16(rs, off[p], base + (uint32_t)(p * kThreads * 16));
    }
  };

  /* Transposed V read: lane (g, row group j = (lane >> 4) & 1, i = lane &
   * 15) reads key 4g + 8h + i/4 of a 16-key step at d 16j + 4(i%4) of a
   * 32-wide d tile, which hands each lane the 8 keys its MFMA k-slots need
   * (the P^T order below) at d = lane % 32. */
  const int tr_key = 4 * g + ((lane & 15) >> 2);
  const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  f32x16 o_acc[kQT][kDTiles];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
#pragma unroll
    for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        o_acc[qt][i][r] = 0.0f;
      }
    }
  }
  /* Base-2 running reference max and sum of this lane's query per tile. */
  float m_run[kQT], l_run[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.0f;
  }

  typedef f32x16 Scores[kKT][kQT]; /* [key tile][query tile] */

  /* S^T of block `blk` for this wave: keys 32*kt + (row), queries of tile
   * qt; one K operand read feeds all query tiles. */
  auto scores = [&](int blk, Scores &st) {
    const u32x4 *kl = ring[(blk - first) & 1][0];
#pragma unroll
    for (int ds = 0; ds < kDSteps; ++ds) {
#pragma unroll
      for (int kt = 0; kt < kKT; ++kt) {
        const int row = kt * 32 + lq;
        const u32x4 a = kl[row * kChunks + swz<kChunks>(row, 2 * ds + g)];
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          st[kt][qt] = mfma(a, qf[qt][ds], ds == 0 ? f32x16{} : st[kt][qt]);
        }
      }
    }
  };

  const float hide = scale_log2 >= 0.0f ? -INFINITY : INFINITY;

  /* Softmax of one query tile's raw scores against its running reference
   * max: the P^T operands in `pt`, the factor O and l take, and whether the
   * reference moved. Masked scores are +-inf (the scale's sign) in raw form
   * and come out as exactly 0. */
  auto softmax = [&](Scores &st, int qt, u32x4 (&pt)[kKS], float &alpha,
                     auto masked, auto pos) -> bool {
    constexpr bool kMasked = decltype(masked)::value;
    constexpr bool kPos = decltype(pos)::value;
    float ext = kPos ? -INFINITY : INFINITY;
#pragma unroll
    for (int kt = 0; kt < kKT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        ext = kPos ? fmaxf(ext, st[kt][qt][r]) : fminf(ext, st[kt][qt][r]);
      }
    }
    {
      const auto r = halves(ext);
      ext = kPos ? fmaxf(r[0], r[1]) : fminf(r[0], r[1]);
    }
    const float mx = ext == hide ? -INFINITY : ext * scale_log2;
    /* The reference max m moves only when a block's max passes it by more
     * than kSlack (and always from -inf): p = 2^(s - m) then stays below
     * 2^kSlack, and O and l share the stale m, so the result is the same up
     * to rounding while most blocks skip the O rescale. */
    const bool bump = mx > m_run[qt] + kSlack;
    const float m_next = bump ? mx : m_run[qt];
    /* All keys so far masked: keep exponents finite (everything is 0). */
    const float m_use = m_next == -INFINITY ? 0.0f : m_next;
    alpha = bump ? __builtin_amdgcn_exp2f(m_run[qt] - m_use) : 1.0f;
    float psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < kKT; ++kt) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = st[kt][qt][8 * hh + e];
          p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x, scale_log2, -m_use));
          if constexpr (kMasked) {
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
    {
      const auto r = halves(psum);
      psum = r[0] + r[1];
    }
    l_run[qt] = l_run[qt] * alpha + psum;
    m_run[qt] = m_next;
    return bump;
  };

  /* O^T = alpha O^T + V^T P^T over the 4 key steps of block `blk`; one V
   * operand read feeds all query tiles. */
  auto accumulate = [&](int blk, const u32x4 (&pt)[kQT][kKS],
                        const float (&alpha)[kQT], const bool (&bump)[kQT]) {
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      if (__builtin_amdgcn_ballot_w64(bump[qt]) != 0) {
#pragma unroll
        for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            o_acc[qt][i][r] *= alpha[qt];
          }
        }
      }
    }
    const VX_LDS char *vl = (const VX_LDS char *)&ring[(blk - first) & 1][1][0];
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
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
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          o_acc[qt][i] = mfma(a, pt[qt][ks], o_acc[qt][i]);
        }
      }
    }
#if VX_FA_PV_LEAD > 0
    /* The transposing reads run VX_FA_PV_LEAD reads (a few MFMAs) ahead of
     * the MFMAs that consume them, then two per MFMA. */
    __builtin_amdgcn_sched_group_barrier(0x100, VX_FA_PV_LEAD, 0); /* DS read */
#pragma unroll
    for (int g = 0; g < (2 * kKS * kDTiles - VX_FA_PV_LEAD) / 2; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); /* MFMA */
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(
        0x008, kKS * kDTiles - (2 * kKS * kDTiles - VX_FA_PV_LEAD) / 2, 0);
#endif
  };

  /* One key block. Entering it, K of this block and the next and V of this
   * block have been requested, and this block's scores are in `st`. After
   * the barrier the slots of the previous block are free: K two blocks
   * ahead and V one block ahead go into them. The next block's score MFMAs
   * are issued alongside this block's softmax; on a block that needs no
   * mask (the common case) they form one straight-line region whose MFMAs
   * are spread between the softmax's VALU instructions. */
  auto step = [&](int blk, Scores &st, Scores &sn) {
    wait_all_loads();
    lds_barrier();
    if (blk + 2 < nblocks) {
      issue(blk + 2, 0);
    }
    if (blk + 1 < nblocks) {
      issue(blk + 1, 1);
    }
    const int key0 = blk * kBlockK;
    if (key0 > wave_last) {
      return;
    }
    const bool need_mask =
        key0 + kBlockK > seq_k || (causal && key0 + kBlockK - 1 > qw0 + shift);
    const bool next = blk + 1 < nblocks && key0 + kBlockK <= wave_last;
    u32x4 pt[kQT][kKS];
    float alpha[kQT];
    bool bump[kQT];
    if (!need_mask && next && scale_log2 >= 0.0f) {
      scores(blk + 1, sn);
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        bump[qt] = softmax(st, qt, pt[qt], alpha[qt], std::false_type{},
                           std::true_type{});
      }
#if VX_FA_SGB > 0
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0); /* DS read */
#pragma unroll
      for (int i = 0; i < 8 * kKT * kQT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); /* MFMA */
        __builtin_amdgcn_sched_group_barrier(0x002, VX_FA_SGB, 0); /* VALU */
        if (i < 12) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
#endif
    } else {
      if (next) {
        scores(blk + 1, sn);
      }
      if (need_mask || scale_log2 < 0.0f) {
        /* The lane's group g, read again from the lane id: the mask is its
         * only use inside the key loop, and a value kept live across the
         * loop for it was spilled (its reload waited for every load in
         * flight). The asm keeps the compiler from hoisting it. */
        int gm;
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\t"
                     "v_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
                     "v_lshrrev_b32 %0, 5, %0"
                     : "=v"(gm));
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          const int my_q = qw0 + 32 * qt + lq;
          const int limit =
              causal ? min(seq_k - 1, my_q + shift) : seq_k - 1;
#pragma unroll
          for (int kt = 0; kt < kKT; ++kt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = key0 + 32 * kt + 8 * (r >> 2) + 4 * gm + (r & 3);
              st[kt][qt][r] = key <= limit ? st[kt][qt][r] : hide;
            }
          }
          bump[qt] = scale_log2 >= 0.0f
                         ? softmax(st, qt, pt[qt], alpha[qt], std::true_type{},
                                   std::true_type{})
                         : softmax(st, qt, pt[qt], alpha[qt], std::true_type{},
                                   std::false_type{});
        }
      } else {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          bump[qt] = softmax(st, qt, pt[qt], alpha[qt], std::false_type{},
                             std::true_type{});
        }
      }
    }
    accumulate(blk, pt, alpha, bump);
  };

  Scores sa, sb;
  if (first < nblocks) {
    issue(first, 0);
    issue(first, 1);
    if (first + 1 < nblocks) {
      issue(first + 1, 0);
    }
    wait_all_loads();
    lds_barrier();
    if (first * kBlockK <= wave_last) {
      scores(first, sa);
    }
  }
  for (int blk = first; blk < nblocks; blk += 2) {
    step(blk, sa, sb);
    if (blk + 1 < nblocks) {
      step(blk + 1, sb, sa);
    }
  }

#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const int my_q = qw0 + 32 * qt + lq;
    if (my_q >= seq_q) {
      continue;
    }
    const float inv = l_run[qt] > 0.0f ? 1.0f / l_run[qt] : 0.0f;
    if constexpr (kSplit) {
      /* This split's normalised output and log-sum-exp, in f32, for the
       * merge: part sp of [splits][bh_total][seq_q]. A row the split never
       * saw writes only its lse (-inf); the merge reads no output for it. */
      const int64_t row = ((int64_t)sp * bh_total + bh) * seq_q + my_q;
      if (l_run[qt] > 0.0f) {
        float *prow = Opart + row * kD;
#pragma unroll
        for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int d = i * 32 + 8 * r4 + 4 * g;
            *reinterpret_cast<f32x4v *>(prow + d) = f32x4v{
                o_acc[qt][i][4 * r4] * inv, o_acc[qt][i][4 * r4 + 1] * inv,
                o_acc[qt][i][4 * r4 + 2] * inv, o_acc[qt][i][4 * r4 + 3] * inv};
          }
        }
      }
      if (g == 0) {
        Lpart[row] = l_run[qt] > 0.0f
                         ? (m_run[qt] + log2f(l_run[qt])) * 0.69314718055994531f
                         : -INFINITY;
      }
      continue;
    }
    uint16_t *orow = O + q_base + (int64_t)my_q * kD;
#pragma unroll
    for (int i = 0; i < kDTiles; ++i) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = i * 32 + 8 * r4 + 4 * g;
        u32x2 out;
        out[0] = pack2(o_acc[qt][i][4 * r4] * inv, o_acc[qt][i][4 * r4 + 1] * inv);
        out[1] = pack2(o_acc[qt][i][4 * r4 + 2] * inv,
                       o_acc[qt][i][4 * r4 + 3] * inv);
        *reinterpret_cast<u32x2 *>(orow + d) = out;
      }
    }
    if (LSE && g == 0) {
      LSE[(int64_t)bh * seq_q + my_q] =
          l_run[qt] > 0.0f
              ? (m_run[qt] + log2f(l_run[qt])) * 0.69314718055994531f
              : -INFINITY;
    }
  }
}

/* Merge of the key splits' partials (the flash-decoding merge, as
 * reference stdlib/std/nn.vx's attention parts and merge). Per row: M the
 * largest split lse, w_s = e^(lse_s - M) (0 for a split that saw no key),
 * o = sum_s w_s o_s / sum_s w_s rounded to bf16 once, lse = M + ln sum_s
 * w_s; a row no split saw gets o = 0 and lse = -inf. kD / 4 threads per
 * row, four columns each. Every split's lse is read first and every output
 * load issued before any is used (an unseen split's output is not written
 * by the split kernel and is dropped by a select, never multiplied). */
template <int kD>
__global__ __launch_bounds__(256) void flash_merge(
    const float *__restrict__ Opart, const float *__restrict__ Lpart,
    uint16_t *__restrict__ O, float *__restrict__ LSE, int64_t rows,
    int splits) {
  constexpr int kVec = kD / 4;
  constexpr int kBatch = 4; /* splits combined per round of loads */
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = t / kVec;
  const int c = (int)(t % kVec);
  if (row >= rows) {
    return;
  }
  float mx = -INFINITY;
  for (int s = 0; s < splits; ++s) {
    mx = fmaxf(mx, Lpart[s * rows + row]);
  }
  float sum = 0.0f;
  f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
  if (mx != -INFINITY) {
    for (int s0 = 0; s0 < splits; s0 += kBatch) {
      float l[kBatch];
      f32x4v ov[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int s = min(s0 + j, splits - 1);
        l[j] = s0 + j < splits ? Lpart[s * rows + row] : -INFINITY;
        ov[j] = *reinterpret_cast<const f32x4v *>(Opart + (s * rows + row) * kD +
                                                  4 * c);
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const bool seen = l[j] != -INFINITY;
        const float w = seen ? expf(l[j] - mx) : 0.0f;
        sum += w;
        acc[0] += seen ? w * ov[j][0] : 0.0f;
        acc[1] += seen ? w * ov[j][1] : 0.0f;
        acc[2] += seen ? w * ov[j][2] : 0.0f;
        acc[3] += seen ? w * ov[j][3] : 0.0f;
      }
    }
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  u32x2 out;
  out[0] = pack2(acc[0] * inv, acc[1] * inv);
  out[1] = pack2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<u32x2 *>(O + row * kD + 4 * c) = out;
  if (LSE && c == 0) {
    LSE[row] = sum > 0.0f ? mx + logf(sum) : -INFINITY;
  }
}

template <int kD, int kQT, int kBK>
void launch(const uint16_t *q, const uint16_t *k, const uint16_t *v,
            uint16_t *o, float *lse, int heads, int group, int seq_q, int seq_k,
            int bh, float scale_log2, bool causal, int splits, float *opart,
            float *lpart, hipStream_t stream) {
  constexpr int kBlockQ = 4 * 32 * kQT;
  const int qblocks = (seq_q + kBlockQ - 1) / kBlockQ;
  if (splits <= 1) {
    hipLaunchKernelGGL((flash_fwd<kD, kQT, kBK, false>),
                       dim3((unsigned)(bh * qblocks)), dim3(kThreads), 0, stream,
                       q, k, v, o, lse, heads, group, seq_q, seq_k, bh, qblocks,
                       scale_log2, causal, 1, nullptr, nullptr);
    return;
  }
  hipLaunchKernelGGL((flash_fwd<kD, kQT, kBK, true>),
                     dim3((unsigned)(bh * qblocks * splits)), dim3(kThreads), 0,
                     stream, q, k, v, o, lse, heads, group, seq_q, seq_k, bh,
                     qblocks, scale_log2, causal, splits, opart, lpart);
  const int64_t rows = (int64_t)bh * seq_q;
  const int64_t threads = rows * (kD / 4);
  hipLaunchKernelGGL((flash_merge<kD>), dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, stream, opart, lpart, o, lse, rows, splits);
}

std::atomic<int> forced_splits{0};

/* Key splits for a launch: the query blocks alone give `items` workgroups.
 * Below one round of two per CU, the key range is cut so that about one such
 * round runs, with at least 16 key blocks per split and at most 8 splits
 * (measured on the 512-query prefill chunks, 128 items: over 2048 keys 2
 * splits 35.5 us against 37.6 for 4; over 8192 keys 4 splits 88.8 us against
 * 100.7 for 2 and 98-101 for 6 and 8; over 512 keys no split pays). */
int pick_splits(int64_t items, int64_t key_blocks, int cus) {
  const int forced = forced_splits.load();
  if (forced > 0) {
    return (int)std::min<int64_t>(forced, std::max<int64_t>(key_blocks, 1));
  }
  const int64_t slots = 2 * (int64_t)cus;
  if (items >= slots) {
    return 1;
  }
  const int64_t want = (slots + items - 1) / items;
  return (int)std::max<int64_t>(1, std::min<int64_t>({want, 8, key_blocks / 16}));
}

/* Split partials of one (device, stream). Launches on one stream run in
 * order, so they share the block; it grows (the old block freed in the
 * stream's order). A stream's block is freed, in that stream's order, when
 * the caller stream of a thread moves off it (flash_attn_release_stream);
 * the default stream's block lives until the process ends. */
struct SplitSpace {
  float *base = nullptr;
  size_t bytes = 0;
};
std::mutex spaces_mutex;
std::map<std::pair<int, hipStream_t>, SplitSpace> &spaces() {
  static auto *m = new std::map<std::pair<int, hipStream_t>, SplitSpace>();
  return *m;
}

/* Makes `sp` hold `bytes` on `stream` (caller holds spaces_mutex); false
 * when the memory cannot be had. */
bool reserve(SplitSpace &sp, size_t bytes, hipStream_t stream) {
  if (sp.base && bytes <= sp.bytes) {
    return true;
  }
  void *fresh = nullptr;
  if (hipMallocAsync(&fresh, bytes, stream) != hipSuccess || !fresh) {
    (void)hipGetLastError();
    return false;
  }
  if (sp.base) {
    VX_HIP_CHECK(hipFreeAsync(sp.base, stream));
  }
  sp.base = static_cast<float *>(fresh);
  sp.bytes = bytes;
  return true;
}

} // namespace

void flash_attn_force_splits(int splits) { forced_splits.store(splits > 0 ? splits : 0); }

int flash_attn_release_stream(hipStream_t stream) {
  if (!stream) {
    return 0;
  }
  /* A stream that is capturing would record the free into its graph: its
   * block stays until a later release finds it idle. */
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &status) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (status != hipStreamCaptureStatusNone) {
    return 0;
  }
  std::lock_guard<std::mutex> hold(spaces_mutex);
  int freed = 0;
  auto &m = spaces();
  for (auto it = m.begin(); it != m.end();) {
    if (it->first.second != stream) {
      ++it;
      continue;
    }
    if (it->second.base) {
      VX_HIP_CHECK(hipFreeAsync(it->second.base, stream));
      ++freed;
    }
    it = m.erase(it);
  }
  return freed;
}

void flash_attn_workspace_stats(int64_t *blocks, int64_t *bytes) {
  std::lock_guard<std::mutex> hold(spaces_mutex);
  int64_t n = 0, total = 0;
  for (const auto &e : spaces()) {
    if (e.second.base) {
      ++n;
      total += (int64_t)e.second.bytes;
    }
  }
  *blocks = n;
  *bytes = total;
}

bool flash_attn_fwd_launch(const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, uint16_t *o, float *lse,
                           int64_t batch, int64_t heads, int64_t kv_heads,
                           int64_t seq_q, int64_t seq_k, int64_t head_dim,
                           float scale, bool causal, bool allow_split,
                           hipStream_t stream) {
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
  /* One workgroup per 128 * kQT queries of a head; the grid stays within
   * int32 for any accepted shape when it does for 128-query blocks. */
  if (bh * ((seq_q + 127) / 128) > INT32_MAX || seq_k > INT32_MAX / 256) {
    return false;
  }
  const float scale_log2 = scale * 1.4426950408889634f;
  const int group = (int)(heads / kv_heads);
  constexpr int kBlockQ = 4 * 32 * VX_FA_QT;
  const int64_t items = bh * ((seq_q + kBlockQ - 1) / kBlockQ);
  const int64_t key_blocks = (seq_k + VX_FA_BK - 1) / VX_FA_BK;
  int splits = allow_split ? pick_splits(items, key_blocks, device_cu_count()) : 1;
  /* Both grids stay within 32-bit workgroup and thread counts. */
  if (items * splits > INT32_MAX || bh * seq_q * (head_dim / 4) > INT32_MAX) {
    splits = 1;
  }
  if (splits > 1) {
    /* Held from the workspace lookup through the launch, so a growth on one
     * thread cannot free a block another thread's launch is about to use. */
    std::lock_guard<std::mutex> hold(spaces_mutex);
    int dev = 0;
    VX_HIP_CHECK(hipGetDevice(&dev));
    SplitSpace &sp = spaces()[{dev, stream}];
    const size_t rows = (size_t)bh * (size_t)seq_q;
    const size_t bytes =
        (size_t)splits * rows * ((size_t)head_dim + 1) * sizeof(float);
    if (reserve(sp, bytes, stream)) {
      float *opart = sp.base;
      float *lpart = opart + (size_t)splits * rows * (size_t)head_dim;
      if (head_dim == 128) {
        launch<128, VX_FA_QT, VX_FA_BK>(q, k, v, o, lse, (int)heads, group,
                                        (int)seq_q, (int)seq_k, (int)bh,
                                        scale_log2, causal, splits, opart, lpart,
                                        stream);
      } else {
        launch<64, VX_FA_QT, VX_FA_BK>(q, k, v, o, lse, (int)heads, group,
                                       (int)seq_q, (int)seq_k, (int)bh,
                                       scale_log2, causal, splits, opart, lpart,
                                       stream);
      }
      VX_HIP_CHECK(hipGetLastError());
      return true;
    }
    splits = 1; /* no workspace: run unsplit */
  }
  if (head_dim == 128) {
    launch<128, VX_FA_QT, VX_FA_BK>(q, k, v, o, lse, (int)heads, group, (int)seq_q,
                          (int)seq_k, (int)bh, scale_log2, causal, 1, nullptr,
                          nullptr, stream);
  } else {
    launch<64, VX_FA_QT, VX_FA_BK>(q, k, v, o, lse, (int)heads, group, (int)seq_q,
                         (int)seq_k, (int)bh, scale_log2, causal, 1, nullptr,
                         nullptr, stream);
  }
  VX_HIP_CHECK(hipGetLastError());
  return true;
}

} // namespace vxk
