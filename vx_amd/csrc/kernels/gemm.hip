/*
 * gemm.hip -- the routed `a @ b` on gfx950.
 *
 * 16-bit inputs (bf16 or f16), f32 accumulate, f32 or 16-bit output, on
 * MFMA tiles: one workgroup owns a 256x256 tile of C. The default kernel is
 * gemm_mfma_pp (8 waves, two per SIMD, on v_mfma_f32_16x16x32): K is walked
 * in stages of 32 through a 4-slot LDS ring filled by buffer-to-LDS loads
 * three stages ahead; B keeps its global k-major order in LDS and reaches the
 * MFMA through the transposing ds_read_b64_tr_b16; the two waves that share
 * a SIMD alternate between loading operands and computing, so the MFMA pipe,
 * the LDS and the load path work at the same time. Workgroups are renumbered
 * so the 32 consecutive tiles each XCD receives form a patch of C (4 tile
 * rows deep; 2 for a grid of at most one round), which keeps each XCD's A
 * and B panels in its own L2. Grids of q rounds of the CUs plus a partial
 * round of at most half take gemm_mfma_sk for their last full round and the
 * partial one (after a one-tile launch of the q - 1 rounds before): the same
 * tiles on one workgroup per CU, the partial round's tiles cut along K
 * between two workgroups (stream-K).
 *
 * gemm_tiled takes every supported type pair, any shape and row stride:
 * 64x64 tiles, 16-deep K stages through LDS, one multiply and one add per
 * term with contraction off, k in order: for f32 this is the same
 * arithmetic, term for term, as the reference CPU loop nest
 * (runtime/host_dispatch_common.h:65-79), and for bf16 -> f32 the same as
 * the outlined linalg.matmul (extend, f32 multiply, f32 add, k sequential;
 * src/codegen/flat/emit/tensor.rs:1600-1647).
 *
 * f32 products of 2^30 multiply-adds and more go to gemm_f32_mfma
 * (v_mfma_f32_32x32x2_f32, 128x128 tiles), which is within the reference's
 * 1e-4 rule of that loop but not bit-equal to it; smaller f32 products,
 * BASELINE's 512^3 plumbing case among them, stay exact-order.
 */
#include "../../../include/vx_hardware_runtime.h"
#include "../vx_hip_common.h"
#include "../vx_kernels.h"
#include "gemm_pp_layout.h"

#include <atomic>
#include <map>
#include <mutex>
#include <type_traits>

namespace vxk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileM = pp::kTileM;
constexpr int kTileN = pp::kTileN;
/* Launch order (pp::tile_of): tile rows per group 4, and 2 for grids of at
 * most one round (256 tiles). Measured on the ping-pong kernel (bf16 -> f32,
 * paired runs on one box): 4096^3 with groups of 1, 2, 4 and 16 rows
 * 1231-1235, 1231-1235, 1196-1201 and 1220-1230 TFLOP/s; 8192^3 with 2, 4, 8
 * and 16 rows 1240-1254, 1282-1290, 1269-1280 and 1248-1255. */

template <int kOut>
__device__ __forceinline__ void put(void *c, int64_t at, float v) {
  if constexpr (kOut == VX_DTYPE_F32) {
    static_cast<float *>(c)[at] = v;
  } else if constexpr (kOut == VX_DTYPE_BF16) {
    static_cast<uint16_t *>(c)[at] = f32_to_bf16(v);
  } else {
    static_cast<uint16_t *>(c)[at] = f32_to_f16(v);
  }
}

/* Direct-to-LDS staging for gfx950: K is walked in stages of 32 through a
 * ring of LDS slots (32 KiB each: a 256 x 32 plane of A and a 32 x 256 plane
 * of B).
 *
 * Global data goes straight into LDS (buffer_load_dwordx4 ... lds): lane i of
 * a load writes the 16 bytes at LDS base + 16*i, so each lane fetches the
 * global 16 bytes that belong at its LDS slot. No staging registers, no LDS
 * write instructions, and a stage's loads are issued three stages before the
 * stage is consumed.
 *
 * A's plane is row-major [256 rows][4 chunks of 8 k], chunk index XORed with
 * bits 1-2 of the row so a ds_read_b128 of 16 rows at one chunk covers all
 * (row mod 4, chunk) bank slots. B's plane keeps global order, [32 k][256 n]
 * in 16-byte chunks with the chunk index XORed by a function of k mod 4; its
 * MFMA operand (8 consecutive k per lane) comes from two ds_read_b64_tr_b16,
 * which, within each group of 16 lanes, hands lane j element j%4 of the
 * 8 bytes read by lane 4e + j/4 as its element e: lanes 4e..4e+3 read row
 * k+e, 4 columns each, and lane j receives column j of rows k..k+3.
 *
 * The buffer descriptors bound each load to the operand's extent, so an
 * offset past it reads zeros instead of faulting. */
constexpr int kDStageK = pp::kStageK;
constexpr int kDUnits = pp::kUnits; /* 16-byte units per plane */
constexpr int kBufferFlags = 0x00020000;       /* raw 32-bit dwords */

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
#define VX_LDS __attribute__((address_space(3)))

/* Wait until at most `n` of this wave's vector memory operations are
 * outstanding (vmcnt n; lgkmcnt and expcnt untouched). */
template <int n>
__device__ __forceinline__ void wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

/* Wait until at most `newer` (0..kMax) whole stages of this wave's loads are
 * outstanding; each stage is kPer loads. */
template <int kMax, int kPer>
__device__ __forceinline__ void wait_stages(int newer) {
  if constexpr (kMax >= 3) {
    if (newer >= 3) {
      wait_vm<3 * kPer>();
      return;
    }
  }
  if constexpr (kMax >= 2) {
    if (newer >= 2) {
      wait_vm<2 * kPer>();
      return;
    }
  }
  if constexpr (kMax >= 1) {
    if (newer >= 1) {
      wait_vm<kPer>();
      return;
    }
  }
  wait_vm<0>();
}

/* One 16-byte-per-lane load from the buffer `rsrc` at byte offset `voff`
 * into LDS at `lds` + 16*lane. Written as assembly so the compiler neither
 * waits for it at every LDS read (it cannot tell which ring slot the load
 * fills) nor drops the barrier-time vmcnt(0) it adds for a fenced barrier:
 * the kernel orders these loads itself with wait_vm and lds_barrier. The
 * nop covers the one wait state between the M0 write and its use. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm" /* m0 is reserved: declared */
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

/* Workgroup barrier without the release fence __syncthreads carries (that
 * fence waits for every outstanding global load, the prefetches included).
 * LDS reads are drained first so a slot is never refilled under a reader. */
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f); /* lgkmcnt(0) */
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ i32x4 buffer_rsrc(const void *base, int bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xffffu); /* stride 0 */
  r[2] = bytes;
  r[3] = kBufferFlags;
  return r;
}

/* Ping-pong variant on v_mfma_f32_16x16x32: the same 256x256 tile, the same
 * 4-slot ring of K=32 stages filled by buffer-to-LDS loads, 8 waves (2x4,
 * 128x64 of C each), and the two waves that share a SIMD take turns.
 *
 * The waves with wm = 0 (one per SIMD) form group 0, those with wm = 1
 * group 1. Each wave alternates a load phase (issue its share of the DMA
 * three stages ahead, read all operands of its next stage from LDS, wait for
 * them) and a compute phase (the stage's 32 MFMAs, from registers). Group 1
 * starts one phase late, so on every SIMD one wave computes while the other
 * loads, and the MFMA pipe, the LDS and the load path are busy at the same
 * time instead of in turns. A workgroup barrier separates the phases; group
 * 1's extra barrier at the start is matched by group 0's at the end, after
 * its epilogue, so every wave executes the same number of barriers.
 *
 * Ring invariants (phase p of the barrier sequence: group 0 loads stage j in
 * phase 2j and computes it in 2j+1; group 1 loads it in 2j+1 and computes it
 * in 2j+2): stage j+3 is issued by group 0 in phase 2j and by group 1 in
 * phase 2j+1 into slot (j+3) % 4, whose previous stage j-1 was last read in
 * phase 2j-1 (every wave drains its LDS reads before each barrier); each wave
 * waits for its share of stage j+1 before the barrier that opens phase 2j+2,
 * the first phase that reads it.
 *
 * The 16x16x32 MFMA takes a whole stage's k in one instruction and draws
 * less power per flop than 32x32x16 on random operands (about 2.09 against
 * 1.85 PFLOP/s sustained when MFMA-bound on this part), which is what bounds
 * this kernel. A operands are one ds_read_b128 per 16x32 block (lane l: row
 * l%16, k chunk l/16); B operands two ds_read_b64_tr_b16 per 32x16 block.
 * B's LDS chunk swizzle also folds in bit 3 of k, so the four k chunks one
 * transposing read touches land in distinct banks. Each accumulator adds its
 * 32-term stage sums in k order, so results are deterministic (not
 * bit-identical to the 32x32x16 kernels, which add 16-term sums). */

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool kBf16>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
        0);
  }
}

/* Four consecutive elements of C from `at` (one 16-byte store of f32, or
 * 8 bytes of bf16 / f16, where `vec` says the address allows it). */
template <int kOut>
__device__ __forceinline__ void put4(void *c, int64_t at, f32x4 v, bool vec) {
  if (vec) {
    if constexpr (kOut == VX_DTYPE_F32) {
      *reinterpret_cast<f32x4 *>(static_cast<float *>(c) + at) = v;
    } else {
      uint32_t h[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        h[r] = kOut == VX_DTYPE_BF16 ? f32_to_bf16(v[r]) : f32_to_f16(v[r]);
      }
      *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(c) + at) =
          uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      put<kOut>(c, at + r, v[r]);
    }
  }
}

/* A wave's 8 x 4 accumulator blocks of the C tile at (m0, n0): each lane
 * stores 4 consecutive columns of a row per block, 32 stores per wave. N is
 * a multiple of 8 and the first column a multiple of 4, so the 4 are all
 * inside C or all past N. With `through` (the host sets it only when C is
 * aligned for the vector stores and 256 of its rows stay within 31 bits of
 * byte offset), the stores go through a buffer descriptor based at the tile
 * with the agent-coherent policy (sc1): written through to memory rather
 * than left dirty in the XCD's L2 for the end of the kernel to write back.
 * On grids of short K, where C's write-out is a large part of the launch,
 * that measured 3% faster (8192 x 3072 x 768 and 4096 x 4096 x 768, f32
 * out); at K = 4096 and 8192 it was within noise or 1% slower. */
template <int kOut>
__device__ __forceinline__ void store_c(void *C, int64_t M, int64_t N, int64_t ldc,
                                        int64_t m0, int64_t n0, int wm, int wn, int l16,
                                        int kc, const f32x4 (&acc)[pp::kTM][pp::kTN],
                                        bool vec, bool through) {
  constexpr int kEsz = kOut == VX_DTYPE_F32 ? 4 : 2;
  if (through) {
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<char *>(C) + (m0 * ldc + n0) * kEsz, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int i = 0; i < pp::kTM; ++i) {
#pragma unroll
      for (int jj = 0; jj < pp::kTN; ++jj) {
        const int r = pp::c_row(wm, i, l16), c = pp::c_col(wn, jj, kc);
        if (m0 + r < M && n0 + c < N) {
          const int at = (int)(((int64_t)r * ldc + c) * kEsz);
          if constexpr (kOut == VX_DTYPE_F32) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][jj]), cr,
                                                   at, 0, 16 /* sc1 */);
          } else {
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              h[e] = kOut == VX_DTYPE_BF16 ? f32_to_bf16(acc[i][jj][e])
                                           : f32_to_f16(acc[i][jj][e]);
            }
            __builtin_amdgcn_raw_buffer_store_b64(
                u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)}, cr, at, 0, 16 /* sc1 */);
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < pp::kTM; ++i) {
#pragma unroll
    for (int jj = 0; jj < pp::kTN; ++jj) {
      const int64_t row = m0 + pp::c_row(wm, i, l16);
      const int64_t col = n0 + pp::c_col(wn, jj, kc);
      if (row < M && col < N) {
        put4<kOut>(C, row * ldc + col, acc[i][jj], vec);
      }
    }
  }
}

template <bool kBf16, int kOut>
__global__ __launch_bounds__(512, 1) void gemm_mfma_pp(
    const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
    void *__restrict__ C, int64_t M, int64_t N, int K, int64_t lda,
    int64_t ldb, int64_t ldc, int tiles_m, int tiles_n, int through,
    uint64_t *__restrict__ stamp) {
  constexpr int kNS = 4;
  /* Optional clock stamp (null in ordinary launches; the branch is uniform):
   * workgroup 0 records the shader-clock counter and the constant 100 MHz
   * real-time counter at its start and end, so a caller can read the clock
   * the kernel actually ran at. */
  uint64_t clk0 = 0, rt0 = 0;
  if (stamp && blockIdx.x == 0) {
    clk0 = __builtin_amdgcn_s_memtime();
    rt0 = __builtin_amdgcn_s_memrealtime();
  }
  constexpr int kLoads = pp::kLoads; /* per wave per plane */
  constexpr int kTM = pp::kTM;       /* 16-row blocks per wave */
  constexpr int kTN = pp::kTN;       /* 16-column blocks per wave */
  static_assert(kNS == pp::kSlots, "ring depth");
  __shared__ u32x4 ring[kNS][2][kDUnits];

  const int t = threadIdx.x;
  const pp::Tile tile = pp::tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n);
  const int64_t m0 = (int64_t)tile.tm * kTileM;
  const int64_t n0 = (int64_t)tile.tn * kTileN;

  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63;

  uint32_t a_off[kLoads], b_off[kLoads];
#pragma unroll
  for (int p = 0; p < kLoads; ++p) {
    a_off[p] = pp::a_load_off(wave, p, lane, lda);
    b_off[p] = pp::b_load_off(wave, p, lane, ldb);
  }
  /* A stage's loads cover a 256 x 32 block of A and a 32 x 256 block of B;
   * each buffer ends at the last element of its matrix, so rows of A past M
   * and the tail of B's last row read zeros. Columns of B past N within
   * earlier rows read whatever follows them, which only reaches outputs past
   * N, and those are not stored. */
  const uint32_t ring_base =
      (uint32_t)(uintptr_t)(VX_LDS void *)&ring[0][0][0];
  auto issue = [&](int step, int slot) {
    const int64_t a0 = pp::a_stage_base(m0, lda, step);
    const int64_t b0 = pp::b_stage_base(n0, ldb, step);
    const i32x4 ra = buffer_rsrc(A + a0, pp::a_stage_bytes(M, K, lda, a0));
    const i32x4 rb = buffer_rsrc(B + b0, pp::b_stage_bytes(N, K, ldb, b0));
#pragma unroll
    for (int p = 0; p < kLoads; ++p) {
      dma16(ra, a_off[p], ring_base + pp::lds_a_dst(slot, wave, p));
    }
#pragma unroll
    for (int p = 0; p < kLoads; ++p) {
      dma16(rb, b_off[p], ring_base + pp::lds_b_dst(slot, wave, p));
    }
  };

  f32x4 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }

  const int wm = wave >> 2; /* also the group */
  const int wn = wave & 3;
  const int l16 = lane & 15;
  const int kc = lane >> 4; /* k chunk of this lane's operands */

  auto frags = [&](int slot, u32x4 (&af)[kTM], u32x4 (&bfr)[kTN]) {
    const u32x4 *la = ring[slot][0];
    const VX_LDS char *lb = (const VX_LDS char *)&ring[slot][1][0];
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      af[i] = la[pp::lds_a_read(wm, i, l16, kc)];
    }
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int at = pp::lds_b_read(wn, j, h, l16, kc);
        const u32x2 w = __builtin_bit_cast(
            u32x2,
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS i16x4 *)(lb + at)));
        bfr[j][2 * h] = w[0];
        bfr[j][2 * h + 1] = w[1];
      }
    }
  };

  const int steps = K / kDStageK;
#pragma unroll
  for (int s = 0; s < kNS - 1; ++s) {
    if (s < steps) {
      issue(s, s);
    }
  }
  wait_stages<kNS - 2, 2 * kLoads>(min(steps - 1, kNS - 2));
  lds_barrier();
  if (wm == 1) {
    lds_barrier();
  }
  u32x4 af[kTM], bfr[kTN];
  for (int j = 0; j < steps; ++j) {
    /* load phase */
    if (j + kNS - 1 < steps) {
      issue(j + kNS - 1, (j + kNS - 1) % kNS);
    }
    frags(j % kNS, af, bfr);
    if (j + 1 < steps) {
      wait_stages<kNS - 2, 2 * kLoads>(min(steps - 2 - j, kNS - 2));
    }
    lds_barrier();
    /* compute phase: column blocks outer, row blocks snaking, so the B
     * operand stays put for 8 MFMAs and consecutive MFMAs always share one
     * operand (fewer operand toggles; about 3% faster at the power limit).
     * B's fragment goes first: the block accumulates C^T, whose lane layout
     * puts 4 consecutive columns of one C row in each lane (the operands'
     * lane layouts are the same, so the sums are the same bits). */
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int jj = 0; jj < kTN; ++jj) {
#pragma unroll
      for (int i0 = 0; i0 < kTM; ++i0) {
        const int i = (jj & 1) ? kTM - 1 - i0 : i0;
        acc[i][jj] = mfma16<kBf16>(bfr[jj], af[i], acc[i][jj]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  }

  const bool vec = (ldc & 3) == 0 &&
                   ((uintptr_t)C & (kOut == VX_DTYPE_F32 ? 15 : 7)) == 0;
  store_c<kOut>(C, M, N, ldc, m0, n0, wm, wn, l16, kc, acc, vec, through != 0);
  if (wm == 0) {
    lds_barrier(); /* matches group 1's extra barrier before the loop */
  }
  if (stamp && blockIdx.x == 0 && t == 0) {
    const uint64_t clk1 = __builtin_amdgcn_s_memtime();
    const uint64_t rt1 = __builtin_amdgcn_s_memrealtime();
    stamp[0] = clk0;
    stamp[1] = rt0;
    stamp[2] = clk1;
    stamp[3] = rt1;
  }
}

/* Stream-K variant of gemm_mfma_pp for G < T <= 1.5 G tiles on G
 * workgroups, one per CU (pp::sk_fits): a whole grid of one to one and a half
 * rounds, or the last G + r tiles of a grid of q G + r (pp::sk_base, after a
 * one-tile launch of the rest). The same ring, phases and MFMA
 * order, with each workgroup walking one or two units of stages in one
 * stream (the issue side runs into the second unit while the compute side
 * finishes the first). A CU thus runs its own tile plus part of a second-
 * round tile instead of two whole tiles in turn, while the one-tile launch
 * leaves half the CUs idle in its second round. Unit assignment, the split
 * point and the workspace layout are in gemm_pp_layout.h (sk_*).
 *
 * A second-round tile is cut at stage h of K between a writer and a reader
 * workgroup on one XCD. The writer runs stages [0, h) first and leaves the
 * sums in a workspace slot (agent-coherent stores, sc1), waits until they
 * are written and sets one flag per wave to `seq`; then it runs its own
 * tile. The reader runs its own tile, stores it without waiting, runs stages
 * [h, steps) from zero, and at the end waits for the flag of the writer wave
 * with its index (polled by lane 0, bounded), adds the writer's sums to its
 * own and clears the flag for the next launch. No L2 write-back is needed:
 * the sums never sit dirty in a non-coherent cache level. Each element of
 * such a tile is (its stages [0, h) in order) + (its stages [h, steps) in
 * order): deterministic, though not the one-tile launch's bits. (Continuing
 * the writer's sums instead would keep those bits, but the reader must then
 * load them into the accumulators that still hold its own tile, so it waits
 * out its own tile's stores first: 5-9 us of stall that made it no faster.)
 *
 * The writer was dispatched before the reader, so it is resident or done
 * and normally long finished; a poll that runs out (2^21 polls of an
 * agent-scope load and a 128-clock sleep: seconds at most) makes the reader
 * store NaN over its tile instead of hanging. C goes out written through
 * (store_c), since every tile of this launch ends in its last stretch. */
constexpr int kSkPolls = 1 << 21;

template <bool kBf16, int kOut>
__global__ __launch_bounds__(512, 1) void gemm_mfma_sk(
    const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
    void *__restrict__ C, int64_t M, int64_t N, int K, int64_t lda,
    int64_t ldb, int64_t ldc, int tiles_m, int tiles_n, int id_base, char *__restrict__ ws,
    int seq, int through, uint64_t *__restrict__ stamp) {
  constexpr int kNS = 4;
  uint64_t clk0 = 0, rt0 = 0;
  if (stamp && blockIdx.x == 0) {
    clk0 = __builtin_amdgcn_s_memtime();
    rt0 = __builtin_amdgcn_s_memrealtime();
  }
  constexpr int kLoads = pp::kLoads;
  constexpr int kTM = pp::kTM;
  constexpr int kTN = pp::kTN;
  static_assert(kNS == pp::kSlots, "ring depth");
  __shared__ u32x4 ring[kNS][2][kDUnits];

  const int t = threadIdx.x;
  const int steps = K / kDStageK;
  const pp::SkUnits un = pp::sk_units((int)blockIdx.x, tiles_m, tiles_n, id_base,
                                      tiles_m * tiles_n - id_base, (int)gridDim.x, steps);
  const int slot = un.slot;
  const bool writer = un.writer, reader = un.reader;
  const int len0 = un.len0, len1 = un.len1, begin1 = un.begin1;
  const int total = len0 + len1;
  /* the units' tiles as plain integers (the reader's own tile is its unit
   * 0; the tile stored last is unit 1's where there is one) */
  const int tm0 = un.u0.tm, tn0 = un.u0.tn, tm1 = un.u1.tm, tn1 = un.u1.tn;
  const int last_tm = len1 > 0 ? tm1 : tm0, last_tn = len1 > 0 ? tn1 : tn0;

  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63;

  uint32_t a_off[kLoads], b_off[kLoads];
#pragma unroll
  for (int p = 0; p < kLoads; ++p) {
    a_off[p] = pp::a_load_off(wave, p, lane, lda);
    b_off[p] = pp::b_load_off(wave, p, lane, ldb);
  }
  const uint32_t ring_base =
      (uint32_t)(uintptr_t)(VX_LDS void *)&ring[0][0][0];
  /* Stage s of the workgroup's stream: stage s of unit 0, or stage
   * begin1 + s - len0 of unit 1. */
  auto issue = [&](int s, int slot_) {
    int tm, tn, step;
    pp::sk_stage(len0, begin1, tm0, tn0, tm1, tn1, s, tm, tn, step);
    const int64_t a0 = pp::a_stage_base((int64_t)tm * kTileM, lda, step);
    const int64_t b0 = pp::b_stage_base((int64_t)tn * kTileN, ldb, step);
    const i32x4 ra = buffer_rsrc(A + a0, pp::a_stage_bytes(M, K, lda, a0));
    const i32x4 rb = buffer_rsrc(B + b0, pp::b_stage_bytes(N, K, ldb, b0));
#pragma unroll
    for (int p = 0; p < kLoads; ++p) {
      dma16(ra, a_off[p], ring_base + pp::lds_a_dst(slot_, wave, p));
    }
#pragma unroll
    for (int p = 0; p < kLoads; ++p) {
      dma16(rb, b_off[p], ring_base + pp::lds_b_dst(slot_, wave, p));
    }
  };

  f32x4 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }

  const int wm = wave >> 2;
  const int wn = wave & 3;
  const int l16 = lane & 15;
  const int kc = lane >> 4;

  auto frags = [&](int slot_, u32x4 (&af)[kTM], u32x4 (&bfr)[kTN]) {
    const u32x4 *la = ring[slot_][0];
    const VX_LDS char *lb = (const VX_LDS char *)&ring[slot_][1][0];
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      af[i] = la[pp::lds_a_read(wm, i, l16, kc)];
    }
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int at = pp::lds_b_read(wn, j, hh, l16, kc);
        const u32x2 v = __builtin_bit_cast(
            u32x2,
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((VX_LDS i16x4 *)(lb + at)));
        bfr[j][2 * hh] = v[0];
        bfr[j][2 * hh + 1] = v[1];
      }
    }
  };

  const bool vec = (ldc & 3) == 0 &&
                   ((uintptr_t)C & (kOut == VX_DTYPE_F32 ? 15 : 7)) == 0;
  auto store_tile = [&](int tm, int tn) {
    store_c<kOut>(C, M, N, ldc, (int64_t)tm * kTileM, (int64_t)tn * kTileN, wm, wn, l16, kc,
                  acc, vec, through != 0);
  };

  /* Between the units, per wave: the writer leaves the sums of its tail
   * stages in its slice of the slot and sets its flag once they are written;
   * the reader stores its own tile, without waiting for the stores. Both
   * restart their accumulators from zero. The writer's partial-sum stores
   * and the reader's tile stores take the same path through the code (the
   * side that does not make them points its stores past the slot's range,
   * where they are dropped, or skips the tile), so the accumulators take
   * one path. */
  constexpr uint32_t kPast = 0x80000000u; /* past every range */
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(ws + pp::sk_slot_off(slot < 0 ? 0 : slot)), (short)0, pp::kSkSlotFloats * 4,
      0x00020000);
  int *flag = reinterpret_cast<int *>(ws) + pp::sk_flag(slot < 0 ? 0 : slot, wave);
  auto hand_over = [&]() {
    if (reader) {
      store_tile(tm0, tn0);
    }
    const int put_at = (int)(writer ? (uint32_t)lane * 16u : kPast);
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int jj = 0; jj < kTN; ++jj) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][jj]), pr,
                                               put_at, (int)pp::sk_part_off(wave, i, jj, 0),
                                               16 /* sc1 */);
        acc[i][jj] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
    if (writer) {
      wait_vm<0>(); /* the slice is written before the flag says so */
      if (lane == 0) {
        __hip_atomic_store(flag, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  };
  /* The reader, after its tail stages: waits for the writer wave's flag
   * (polled by lane 0, bounded), adds the writer's sums to its own, a
   * quarter of the blocks at a time with the next quarter's loads in flight,
   * and clears the flag for the next launch. Each C element of a tail tile
   * is thus (sum of stages [0, h)) + (sum of stages [h, steps)), each adding
   * its stages in order. False when the wait ran out. */
  auto take_partial = [&]() -> bool {
    int got = seq;
    if (lane == 0) {
      for (int n = 0; n < kSkPolls; ++n) {
        got = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (got == seq) {
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    const bool ok = __builtin_amdgcn_readfirstlane(got) == seq;
    const int get_at = (int)(ok ? (uint32_t)lane * 16u : kPast);
    constexpr int kQ = kTM / 4; /* rows of blocks per quarter */
    f32x4 part[2][kQ][kTN];
    auto fetch = [&](int q, f32x4 (&dst)[kQ][kTN]) {
#pragma unroll
      for (int i = 0; i < kQ; ++i) {
#pragma unroll
        for (int jj = 0; jj < kTN; ++jj) {
          dst[i][jj] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         pr, get_at, (int)pp::sk_part_off(wave, q * kQ + i, jj, 0),
                         16 /* sc1 */));
        }
      }
    };
    auto add = [&](int q, const f32x4 (&src)[kQ][kTN]) {
#pragma unroll
      for (int i = 0; i < kQ; ++i) {
#pragma unroll
        for (int jj = 0; jj < kTN; ++jj) {
          acc[q * kQ + i][jj] = src[i][jj] + acc[q * kQ + i][jj];
        }
      }
    };
    fetch(0, part[0]);
    fetch(1, part[1]);
    wait_vm<kQ * kTN>();
    add(0, part[0]);
    fetch(2, part[0]);
    wait_vm<kQ * kTN>();
    add(1, part[1]);
    fetch(3, part[1]);
    wait_vm<kQ * kTN>();
    add(2, part[0]);
    wait_vm<0>();
    add(3, part[1]);
    if (lane == 0) {
      __hip_atomic_store(flag, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return ok;
  };

#pragma unroll
  for (int s = 0; s < kNS - 1; ++s) {
    if (s < total) {
      issue(s, s);
    }
  }
  wait_stages<kNS - 2, 2 * kLoads>(min(total - 1, kNS - 2));
  lds_barrier();
  if (wm == 1) {
    lds_barrier();
  }
  /* One load phase and one compute phase; the issue side runs three stages
   * ahead, across the boundary between the units. */
  auto stage = [&](int j) {
    u32x4 af[kTM], bfr[kTN];
    if (j + kNS - 1 < total) {
      issue(j + kNS - 1, (j + kNS - 1) % kNS);
    }
    frags(j % kNS, af, bfr);
    if (j + 1 < total) {
      wait_stages<kNS - 2, 2 * kLoads>(min(total - 2 - j, kNS - 2));
    }
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int jj = 0; jj < kTN; ++jj) {
#pragma unroll
      for (int i0 = 0; i0 < kTM; ++i0) {
        const int i = (jj & 1) ? kTM - 1 - i0 : i0;
        acc[i][jj] = mfma16<kBf16>(bfr[jj], af[i], acc[i][jj]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  };
  for (int j = 0; j < len0; ++j) {
    stage(j);
  }
  bool ok = true;
  if (len1 > 0) {
    hand_over();
    for (int j = len0; j < total; ++j) {
      stage(j);
    }
    if (reader) {
      ok = take_partial();
    }
  }
  store_tile(last_tm, last_tn);
  if (!ok) {
    /* the writer's sums never came: the tile is marked as wrong */
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int jj = 0; jj < kTN; ++jj) {
        acc[i][jj] = f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                           __builtin_nanf("")};
      }
    }
    store_tile(last_tm, last_tn);
  }
  if (wm == 0) {
    lds_barrier(); /* matches group 1's extra barrier before the loop */
  }
  if (stamp && blockIdx.x == 0 && t == 0) {
    const uint64_t clk1 = __builtin_amdgcn_s_memtime();
    const uint64_t rt1 = __builtin_amdgcn_s_memrealtime();
    stamp[0] = clk0;
    stamp[1] = rt0;
    stamp[2] = clk1;
    stamp[3] = rt1;
  }
}

/* f32 GEMM on v_mfma_f32_32x32x2_f32, for products large enough that the
 * exact-order kernel's rate matters: 128x128 tiles, 4 waves of 64x64 (2x2
 * accumulators of 32x32), K in stages of 16 through a double-buffered LDS
 * ring, the next stage's loads in registers while the current one computes.
 * A is stored transposed ([k][m]) so that both operands reach the MFMA as 32
 * consecutive floats per half-wave; rows are padded by 32 floats so the two
 * half-waves hit different banks. Edge tiles load zeros outside the
 * operands and store only inside C. Products are exact in f32 and each MFMA
 * step rounds its sums, so results agree with the exact-order loop to about
 * 1e-6 relative, not bit for bit. */
constexpr int kF32Tile = 128;
constexpr int kF32Ks = 16;
constexpr int kF32Pad = kF32Tile + 32;

typedef float f32x4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256, 2) void gemm_f32_mfma(
    const float *__restrict__ A, const float *__restrict__ B,
    float *__restrict__ C, int64_t M, int64_t N, int64_t K, int64_t lda,
    int64_t ldb, int64_t ldc) {
  __shared__ float As[2][kF32Ks][kF32Pad]; /* [k][m] */
  __shared__ float Bs[2][kF32Ks][kF32Pad]; /* [k][n] */
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * kF32Tile;
  const int64_t n0 = (int64_t)blockIdx.x * kF32Tile;
  const bool vec_a = (lda & 3) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  const bool vec_b = (ldb & 3) == 0 && (reinterpret_cast<uintptr_t>(B) & 15) == 0;

  /* Thread t loads A rows (t + 256e) / 4, k columns 4 ((t + 256e) % 4) ..+3,
   * and B k-row (t + 256e) / 32, columns 4 ((t + 256e) % 32) ..+3. */
  f32x4v ra[2], rb[2];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int idx = t + 256 * e;
      const int64_t gm = m0 + (idx >> 2), gk = k0 + 4 * (idx & 3);
      if (vec_a && gm < M && gk + 3 < K) {
        ra[e] = *reinterpret_cast<const f32x4v *>(A + gm * lda + gk);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          ra[e][q] = (gm < M && gk + q < K) ? A[gm * lda + gk + q] : 0.0f;
        }
      }
      const int64_t hk = k0 + (idx >> 5), hn = n0 + 4 * (idx & 31);
      if (vec_b && hk < K && hn + 3 < N) {
        rb[e] = *reinterpret_cast<const f32x4v *>(B + hk * ldb + hn);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          rb[e][q] = (hk < K && hn + q < N) ? B[hk * ldb + hn + q] : 0.0f;
        }
      }
    }
  };
  auto stash = [&](int s) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int idx = t + 256 * e;
      const int am = idx >> 2, ak = 4 * (idx & 3);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        As[s][ak + q][am] = ra[e][q];
      }
      *reinterpret_cast<f32x4v *>(&Bs[s][idx >> 5][4 * (idx & 31)]) = rb[e];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.0f;
      }
    }
  }
  const int lr = lane & 31;
  const int lk = lane >> 5;
  const int64_t stages = (K + kF32Ks - 1) / kF32Ks;
  load(0);
  stash(0);
  __syncthreads();
  for (int64_t st = 0; st < stages; ++st) {
    const int s = (int)(st & 1);
    if (st + 1 < stages) {
      load((st + 1) * kF32Ks);
    }
#pragma unroll
    for (int kk = 0; kk < kF32Ks; kk += 2) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = As[s][kk + lk][wm * 64 + i * 32 + lr];
        b[i] = Bs[s][kk + lk][wn * 64 + i * 32 + lr];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
      }
    }
    if (st + 1 < stages) {
      stash(s ^ 1);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (row < M && col < N) {
          C[row * ldc + col] = acc[i][j][r];
        }
      }
    }
  }
}

template <int kIn>
__device__ __forceinline__ auto load_in(const void *p, int64_t at) {
  if constexpr (kIn == VX_DTYPE_F64) {
    return static_cast<const double *>(p)[at];
  } else if constexpr (kIn == VX_DTYPE_F32) {
    return static_cast<const float *>(p)[at];
  } else if constexpr (kIn == VX_DTYPE_BF16) {
    return bf16_to_f32(static_cast<const uint16_t *>(p)[at]);
  } else {
    return f16_to_f32(static_cast<const uint16_t *>(p)[at]);
  }
}

template <int kOut, typename Acc>
__device__ __forceinline__ void put_any(void *c, int64_t at, Acc v) {
  if constexpr (kOut == VX_DTYPE_F64) {
    static_cast<double *>(c)[at] = v;
  } else {
    put<kOut>(c, at, (float)v);
  }
}

/* kT x kT output tile per workgroup (256 threads as 16 x 16, each with
 * (kT/16)^2 outputs); kT shrinks for small grids so every CU gets work. */
template <int kIn, int kOut, int kT>
__global__ __launch_bounds__(256) void gemm_tiled(const void *__restrict__ A,
                                                  const void *__restrict__ B,
                                                  void *__restrict__ C,
                                                  int64_t M, int64_t N,
                                                  int64_t K, int64_t lda,
                                                  int64_t ldb, int64_t ldc) {
#pragma clang fp contract(off)
  using Acc = decltype(load_in<kIn>(nullptr, 0));
  constexpr int kR = kT / 16;        /* outputs per thread per dimension */
  /* k per step: deep enough that a step's arithmetic covers the next
   * step's loads (64 for f32, 32 for f64 to keep the tiles in 33 KiB) */
  constexpr int kKs = sizeof(Acc) == 8 ? 32 : 64;
  constexpr int kLoads = kT * kKs / 256;
  __shared__ Acc As[kKs][kT + 1]; /* [k][m] */
  __shared__ Acc Bs[kKs][kT + 1]; /* [k][n] */
  const int t = threadIdx.x;
  const int tx = t & 15;
  const int ty = t >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * kT;
  const int64_t n0 = (int64_t)blockIdx.x * kT;
  Acc acc[kR][kR];
#pragma unroll
  for (int i = 0; i < kR; ++i) {
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      acc[i][j] = Acc(0);
    }
  }
  /* One kKs-deep step of A and B in registers: the next step's loads are in
   * flight while this step computes from LDS. */
  Acc ra[kLoads], rb[kLoads];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int e = 0; e < kLoads; ++e) {
      const int idx = t + e * 256;
      const int am = idx / kKs, ak = idx % kKs;
      const int64_t gm = m0 + am, gk = k0 + ak;
      ra[e] = (gm < M && gk < K) ? load_in<kIn>(A, gm * lda + gk) : Acc(0);
      const int bk = idx / kT, bn = idx % kT;
      const int64_t hk = k0 + bk, hn = n0 + bn;
      rb[e] = (hk < K && hn < N) ? load_in<kIn>(B, hk * ldb + hn) : Acc(0);
    }
  };
  auto term = [&](int kk) {
    Acc a[kR], b[kR];
#pragma unroll
    for (int i = 0; i < kR; ++i) {
      a[i] = As[kk][ty * kR + i];
      b[i] = Bs[kk][tx * kR + i];
    }
#pragma unroll
    for (int i = 0; i < kR; ++i) {
#pragma unroll
      for (int j = 0; j < kR; ++j) {
        Acc prod = a[i] * b[j];
        acc[i][j] = acc[i][j] + prod;
      }
    }
  };
  fetch(0);
  for (int64_t k0 = 0; k0 < K; k0 += kKs) {
#pragma unroll
    for (int e = 0; e < kLoads; ++e) {
      const int idx = t + e * 256;
      As[idx % kKs][idx / kKs] = ra[e];
      Bs[idx / kT][idx % kT] = rb[e];
    }
    __syncthreads();
    if (k0 + kKs < K) {
      fetch(k0 + kKs);
    }
    /* k in order for every output, as before; a full step unrolled */
    if (K - k0 >= kKs) {
#pragma unroll
      for (int kk = 0; kk < kKs; ++kk) {
        term(kk);
      }
    } else {
      for (int kk = 0; kk < (int)(K - k0); ++kk) {
        term(kk);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    const int64_t gm = m0 + ty * kR + i;
    if (gm >= M) {
      continue;
    }
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      const int64_t gn = n0 + tx * kR + j;
      if (gn < N) {
        put_any<kOut>(C, gm * ldc + gn, acc[i][j]);
      }
    }
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

/* The ping-pong kernel takes any M and any N that is a multiple of 8: edge
 * tiles read zeros past the operands' ends and store only inside C. K must
 * be whole stages of 32, and rows must start on 16-byte boundaries for the
 * buffer-to-LDS loads. (The buffer range check zeroes a whole 16-byte load
 * that straddles the end of B, so B's last row must end on a 16-byte
 * boundary: N a multiple of 8.) */
bool pp_takes(const GemmArgs &g) {
  const bool sixteen = g.in_dtype == VX_DTYPE_BF16 || g.in_dtype == VX_DTYPE_F16;
  const bool out_ok = g.out_dtype == VX_DTYPE_F32 || g.out_dtype == g.in_dtype;
  return sixteen && out_ok && aligned16(g.a) && aligned16(g.b) &&
         pp::shape_ok(g.m, g.n, g.k, g.lda, g.ldb, g.ldc);
}

bool f32_mfma_takes(const GemmArgs &g) {
  return g.in_dtype == VX_DTYPE_F32 && g.out_dtype == VX_DTYPE_F32 && g.m > 0 &&
         g.n > 0 && g.k > 0 && g.lda >= g.k && g.ldb >= g.n && g.ldc >= g.n &&
         (g.m + kF32Tile - 1) / kF32Tile <= 65535 &&
         (g.n + kF32Tile - 1) / kF32Tile <= INT32_MAX;
}

void launch_f32_mfma(const GemmArgs &g, hipStream_t s) {
  dim3 grid((unsigned)((g.n + kF32Tile - 1) / kF32Tile),
            (unsigned)((g.m + kF32Tile - 1) / kF32Tile));
  hipLaunchKernelGGL(gemm_f32_mfma, grid, dim3(256), 0, s,
                     static_cast<const float *>(g.a),
                     static_cast<const float *>(g.b), static_cast<float *>(g.c),
                     g.m, g.n, g.k, g.lda, g.ldb, g.ldc);
}

bool tiled_takes(const GemmArgs &g) {
  if (g.m <= 0 || g.n <= 0 || g.k <= 0 || g.lda < g.k || g.ldb < g.n ||
      g.ldc < g.n) {
    return false;
  }
  if ((g.m + 63) / 64 > 65535) {
    return false; /* grid.y limit */
  }
  switch (g.in_dtype) {
  case VX_DTYPE_F32:
  case VX_DTYPE_F64:
    return g.out_dtype == g.in_dtype;
  case VX_DTYPE_BF16:
  case VX_DTYPE_F16:
    return g.out_dtype == g.in_dtype || g.out_dtype == VX_DTYPE_F32;
  default:
    return false;
  }
}

/* Whether store_c may write C through a tile-based buffer descriptor: C
 * aligned for the vector stores and 256 rows of it within 31 bits of byte
 * offset. */
bool c_through_ok(const GemmArgs &g, int out) {
  const int64_t esz = out == VX_DTYPE_F32 ? 4 : 2;
  return (g.ldc & 3) == 0 && ((uintptr_t)g.c & (esz == 4 ? 15 : 7)) == 0 &&
         (int64_t)kTileM * g.ldc * esz < (int64_t)INT32_MAX;
}
/* The one-tile launch writes C through for K up to this (measured faster at
 * K = 768, the same or slower at 4096 and 8192); the stream-K launch, whose
 * tiles all end in its last stretch, always does. */
constexpr int64_t kThroughMaxK = 1536;

template <bool kBf16, int kOut>
void launch_pp(const GemmArgs &g, hipStream_t s) {
  const int tiles_m = (int)((g.m + kTileM - 1) / kTileM);
  const int tiles_n = (int)((g.n + kTileN - 1) / kTileN);
  const int through = c_through_ok(g, kOut) && g.k <= kThroughMaxK;
  hipLaunchKernelGGL((gemm_mfma_pp<kBf16, kOut>), dim3(tiles_m * tiles_n),
                     dim3(512), 0, s, static_cast<const uint16_t *>(g.a),
                     static_cast<const uint16_t *>(g.b), g.c, g.m, g.n,
                     (int)g.k, g.lda, g.ldb, g.ldc, tiles_m, tiles_n, through, g.stamp);
}

void launch_pp_any(const GemmArgs &g, hipStream_t s) {
  const bool bf = g.in_dtype == VX_DTYPE_BF16;
  if (g.out_dtype == VX_DTYPE_F32) {
    bf ? launch_pp<true, VX_DTYPE_F32>(g, s) : launch_pp<false, VX_DTYPE_F32>(g, s);
  } else if (bf) {
    launch_pp<true, VX_DTYPE_BF16>(g, s);
  } else {
    launch_pp<false, VX_DTYPE_F16>(g, s);
  }
}

/* The stream-K launch takes what the ping-pong kernel takes when a workspace
 * may be had (not under graph capture, not for the no-alloc entry point)
 * and the grid ends in a partial round of at most half the CUs
 * (pp::sk_base). */
bool sk_takes(const GemmArgs &g) {
  if (!g.may_split || !pp_takes(g)) {
    return false;
  }
  const int64_t tiles = ((g.m + kTileM - 1) / kTileM) * ((g.n + kTileN - 1) / kTileN);
  const int cus = device_cu_count();
  return cus / 2 <= pp::kSkMaxSlots &&
         pp::sk_base((int)tiles, cus, (int)(g.k / kDStageK)) >= 0;
}

/* Stream-K workspaces, one per (device, stream) like the flash-attention
 * split workspace: launches on one stream run in order and share it; it
 * grows (the old block freed in the stream's order) and is freed when the
 * caller stream of a thread moves off it (gemm_release_stream). A fresh block
 * has its flags zeroed; every reader clears the flag it consumed, and each
 * launch marks its hand-overs with a new sequence number, so a flag left by
 * an earlier launch never passes for this one's. */
struct SkSpace {
  char *base = nullptr;
  size_t bytes = 0;
  int seq = 0;
};
std::mutex sk_mutex;
std::atomic<int64_t> sk_launches{0};
std::map<std::pair<int, hipStream_t>, SkSpace> &sk_spaces() {
  static auto *m = new std::map<std::pair<int, hipStream_t>, SkSpace>();
  return *m;
}

bool sk_reserve(SkSpace &sp, size_t bytes, hipStream_t stream) {
  if (sp.base && bytes <= sp.bytes) {
    return true;
  }
  void *fresh = nullptr;
  if (hipMallocAsync(&fresh, bytes, stream) != hipSuccess || !fresh) {
    (void)hipGetLastError();
    return false;
  }
  VX_HIP_CHECK(hipMemsetAsync(fresh, 0, (size_t)pp::kSkFlagBytes, stream));
  if (sp.base) {
    VX_HIP_CHECK(hipFreeAsync(sp.base, stream));
  }
  sp.base = static_cast<char *>(fresh);
  sp.bytes = bytes;
  return true;
}

/* A grid of q G + r tiles, q >= 2: the one-tile launch runs the first
 * id_base = (q - 1) G launch-order ids (its workgroup renumbering is a
 * bijection on them), then the stream-K launch the last G + r. */
template <bool kBf16, int kOut>
void launch_sk(const GemmArgs &g, char *ws, int seq, hipStream_t s) {
  const int tiles_m = (int)((g.m + kTileM - 1) / kTileM);
  const int tiles_n = (int)((g.n + kTileN - 1) / kTileN);
  const int cus = device_cu_count();
  const int id_base = pp::sk_base(tiles_m * tiles_n, cus, (int)(g.k / kDStageK));
  if (id_base > 0) {
    const int through = c_through_ok(g, kOut) && g.k <= kThroughMaxK;
    hipLaunchKernelGGL((gemm_mfma_pp<kBf16, kOut>), dim3(id_base), dim3(512), 0, s,
                       static_cast<const uint16_t *>(g.a),
                       static_cast<const uint16_t *>(g.b), g.c, g.m, g.n, (int)g.k, g.lda,
                       g.ldb, g.ldc, tiles_m, tiles_n, through, (uint64_t *)nullptr);
  }
  hipLaunchKernelGGL((gemm_mfma_sk<kBf16, kOut>), dim3(cus), dim3(512), 0, s,
                     static_cast<const uint16_t *>(g.a),
                     static_cast<const uint16_t *>(g.b), g.c, g.m, g.n, (int)g.k, g.lda,
                     g.ldb, g.ldc, tiles_m, tiles_n, id_base, ws, seq,
                     (int)c_through_ok(g, kOut), g.stamp);
}

/* False when no workspace could be had (the caller runs the ping-pong
 * launch instead). */
bool launch_sk_any(const GemmArgs &g, hipStream_t s) {
  std::lock_guard<std::mutex> hold(sk_mutex);
  int dev = 0;
  VX_HIP_CHECK(hipGetDevice(&dev));
  SkSpace &sp = sk_spaces()[{dev, s}];
  const int64_t tiles = ((g.m + kTileM - 1) / kTileM) * ((g.n + kTileN - 1) / kTileN);
  const int cus = device_cu_count();
  const int id_base = pp::sk_base((int)tiles, cus, (int)(g.k / kDStageK));
  if (!sk_reserve(sp, (size_t)pp::sk_bytes((int)(tiles - id_base - cus)), s)) {
    return false;
  }
  sp.seq = sp.seq == INT32_MAX ? 1 : sp.seq + 1;
  const bool bf = g.in_dtype == VX_DTYPE_BF16;
  if (g.out_dtype == VX_DTYPE_F32) {
    bf ? launch_sk<true, VX_DTYPE_F32>(g, sp.base, sp.seq, s)
       : launch_sk<false, VX_DTYPE_F32>(g, sp.base, sp.seq, s);
  } else if (bf) {
    launch_sk<true, VX_DTYPE_BF16>(g, sp.base, sp.seq, s);
  } else {
    launch_sk<false, VX_DTYPE_F16>(g, sp.base, sp.seq, s);
  }
  ++sk_launches;
  return true;
}

template <int kIn, int kOut>
void launch_tiled(const GemmArgs &g, hipStream_t s) {
  /* The largest tile that still gives every CU (256 on gfx950) a workgroup;
   * the arithmetic per output is the same at every tile size. */
  const int64_t tiles64 = ((g.n + 63) / 64) * ((g.m + 63) / 64);
  const int64_t tiles32 = ((g.n + 31) / 32) * ((g.m + 31) / 32);
  if (tiles64 >= 256) {
    dim3 grid((unsigned)((g.n + 63) / 64), (unsigned)((g.m + 63) / 64));
    hipLaunchKernelGGL((gemm_tiled<kIn, kOut, 64>), grid, dim3(256), 0, s, g.a,
                       g.b, g.c, g.m, g.n, g.k, g.lda, g.ldb, g.ldc);
  } else if (tiles32 >= 256 || (g.m + 15) / 16 > 65535) {
    dim3 grid((unsigned)((g.n + 31) / 32), (unsigned)((g.m + 31) / 32));
    hipLaunchKernelGGL((gemm_tiled<kIn, kOut, 32>), grid, dim3(256), 0, s, g.a,
                       g.b, g.c, g.m, g.n, g.k, g.lda, g.ldb, g.ldc);
  } else {
    dim3 grid((unsigned)((g.n + 15) / 16), (unsigned)((g.m + 15) / 16));
    hipLaunchKernelGGL((gemm_tiled<kIn, kOut, 16>), grid, dim3(256), 0, s, g.a,
                       g.b, g.c, g.m, g.n, g.k, g.lda, g.ldb, g.ldc);
  }
}

} // namespace

bool gemm_kernel_takes(GemmKernel which, const GemmArgs &g) {
  switch (which) {
  case GEMM_MFMA_PP:
    return pp_takes(g);
  case GEMM_MFMA_SK:
    return sk_takes(g);
  case GEMM_F32_MFMA:
    return f32_mfma_takes(g);
  case GEMM_TILED:
    return tiled_takes(g);
  default:
    return false;
  }
}

GemmKernel gemm_pick(const GemmArgs &g) {
  /* Small products stay on the exact-order kernel: a 256x256 tile of mostly
   * padding costs more than it saves there. */
  const bool big = g.m >= 64 && g.n >= 64 && (double)g.m * g.n * g.k >= 16777216.0;
  if (big && pp_takes(g)) {
    return sk_takes(g) ? GEMM_MFMA_SK : GEMM_MFMA_PP;
  }
  /* f32: the exact-order kernel (bit-equal to the reference's host loop)
   * below 2^30 multiply-adds, the MFMA kernel above. */
  if (g.m >= 128 && g.n >= 128 && (double)g.m * g.n * g.k >= 1073741824.0 &&
      f32_mfma_takes(g)) {
    return GEMM_F32_MFMA;
  }
  if (tiled_takes(g)) {
    return GEMM_TILED;
  }
  return GEMM_NONE;
}

bool gemm_launch_kernel(GemmKernel which, const GemmArgs &g,
                        hipStream_t stream) {
  if (which == GEMM_MFMA_PP) {
    if (!pp_takes(g)) {
      return false;
    }
    launch_pp_any(g, stream);
  } else if (which == GEMM_MFMA_SK) {
    if (!sk_takes(g)) {
      return false;
    }
    if (!launch_sk_any(g, stream)) {
      launch_pp_any(g, stream);
    }
  } else if (which == GEMM_F32_MFMA) {
    if (!f32_mfma_takes(g)) {
      return false;
    }
    launch_f32_mfma(g, stream);
  } else if (which == GEMM_TILED) {
    if (!tiled_takes(g)) {
      return false;
    }
    switch (g.in_dtype) {
    case VX_DTYPE_F32:
      launch_tiled<VX_DTYPE_F32, VX_DTYPE_F32>(g, stream);
      break;
    case VX_DTYPE_F64:
      launch_tiled<VX_DTYPE_F64, VX_DTYPE_F64>(g, stream);
      break;
    case VX_DTYPE_BF16:
      g.out_dtype == VX_DTYPE_F32
          ? launch_tiled<VX_DTYPE_BF16, VX_DTYPE_F32>(g, stream)
          : launch_tiled<VX_DTYPE_BF16, VX_DTYPE_BF16>(g, stream);
      break;
    default:
      g.out_dtype == VX_DTYPE_F32
          ? launch_tiled<VX_DTYPE_F16, VX_DTYPE_F32>(g, stream)
          : launch_tiled<VX_DTYPE_F16, VX_DTYPE_F16>(g, stream);
      break;
    }
  } else {
    return false;
  }
  VX_HIP_CHECK(hipGetLastError());
  return true;
}

bool gemm_launch(const GemmArgs &g, hipStream_t stream) {
  return gemm_launch_kernel(gemm_pick(g), g, stream);
}

int gemm_release_stream(hipStream_t stream) {
  if (!stream) {
    return 0;
  }
  /* A capturing stream would record the free into its graph: its block
   * stays until a later release finds it idle. */
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &status) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (status != hipStreamCaptureStatusNone) {
    return 0;
  }
  std::lock_guard<std::mutex> hold(sk_mutex);
  int freed = 0;
  auto &m = sk_spaces();
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

void gemm_workspace_stats(int64_t *blocks, int64_t *bytes, int64_t *launches) {
  std::lock_guard<std::mutex> hold(sk_mutex);
  int64_t n = 0, total = 0;
  for (const auto &e : sk_spaces()) {
    if (e.second.base) {
      ++n;
      total += (int64_t)e.second.bytes;
    }
  }
  *blocks = n;
  *bytes = total;
  *launches = sk_launches.load();
}

namespace {
__global__ void fill_i32(int *p, int v) { *p = v; }
} // namespace

void fill_i32_launch(int *p, int v, hipStream_t stream) {
  hipLaunchKernelGGL(fill_i32, dim3(1), dim3(1), 0, stream, p, v);
  VX_HIP_CHECK(hipGetLastError());
}

} // namespace vxk
