/*
 * gemm_pp_layout.h -- the address arithmetic of gemm_mfma_pp and its
 * stream-K launch gemm_mfma_sk (gemm.hip), written once for the kernels and
 * for the CPU check that walks it (tests/native/gemm_pp_addr_test.cpp): the
 * launch order, the buffer-to-LDS load offsets and buffer ranges of each K
 * stage, the LDS slots those loads fill, the LDS reads of the MFMA operands,
 * the epilogue's C indices, and the stream-K units and workspace.
 * Plain C++ apart from the host/device qualifier, so g++ builds the check.
 */
#ifndef VX_AMD_GEMM_PP_LAYOUT_H
#define VX_AMD_GEMM_PP_LAYOUT_H

#include <cstdint>
#include <climits>

#if defined(__HIPCC__)
#define VX_PP_FN __host__ __device__ __forceinline__
#else
#define VX_PP_FN inline
#endif

namespace vxk {
namespace pp {

constexpr int kTileM = 256;                   /* C tile rows per workgroup */
constexpr int kTileN = 256;                   /* C tile columns */
constexpr int kStageK = 32;                   /* K per stage (one MFMA) */
constexpr int kUnits = kTileM * kStageK / 8;  /* 16-byte units per plane */
constexpr int kWaves = 8;
constexpr int kLoads = kUnits / 64 / kWaves;  /* loads per wave per plane */
constexpr int kSlots = 4;                     /* ring depth */
constexpr int kPlaneBytes = kUnits * 16;      /* 16 KiB: A or B of a stage */
constexpr int kRingBytes = kSlots * 2 * kPlaneBytes; /* 128 KiB */
constexpr int kTM = 8;                        /* 16-row blocks per wave */
constexpr int kTN = 4;                        /* 16-column blocks per wave */
/* Tile rows per launch-order group: 4, and 2 for grids of at most one
 * round (256 tiles). */
constexpr int kGroupM = 4;
constexpr int kSmallGrid = 256;
constexpr int kSmallGroupM = 2;

/* The shapes the kernel takes (besides 16-bit inputs and 16-byte aligned
 * A and B): any M, N a multiple of 8, K whole stages, rows on 16-byte
 * boundaries, and every buffer range and load offset within 31 bits. (The
 * buffer range check zeroes a whole 16-byte load that straddles the end of
 * B, so B's last row must end on a 16-byte boundary: N a multiple of 8.) */
VX_PP_FN bool shape_ok(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                       int64_t ldc) {
  if (m <= 0 || n <= 0 || k <= 0 || k % kStageK != 0 || k > INT32_MAX ||
      n % 8 != 0 || lda % 8 != 0 || ldb % 8 != 0 || lda < k || ldb < n ||
      ldc < n) {
    return false;
  }
  const int64_t tiles = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN);
  return tiles <= INT32_MAX && (kTileM - 1) * lda * 2 + kStageK * 2 <= INT32_MAX &&
         (kStageK - 1) * ldb * 2 + kTileN * 2 <= INT32_MAX;
}

struct Tile {
  int tm, tn;
};

/* The C tile at launch-order id `id`: ids walk C in groups of group_m tile
 * rows, column by column. */
VX_PP_FN Tile tile_at(int id, int tiles_m, int tiles_n) {
  const int group_m = tiles_m * tiles_n <= kSmallGrid ? kSmallGroupM : kGroupM;
  const int group_size = group_m * tiles_n;
  const int first_m = (id / group_size) * group_m;
  const int rows_in_group =
      tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  const int in_group = id % group_size;
  return Tile{first_m + in_group % rows_in_group, in_group / rows_in_group};
}

/* The C tile workgroup `block` of `nwg` computes. Workgroup i runs on XCD
 * i % 8; the renumbering gives each XCD consecutive ids. */
VX_PP_FN Tile tile_of(int block, int nwg, int tiles_m, int tiles_n) {
  int id = block;
  if ((nwg & 7) == 0) {
    id = (id & 7) * (nwg >> 3) + (id >> 3);
  }
  return tile_at(id, tiles_m, tiles_n);
}

/* Stream-K launch (gemm_mfma_sk), for grids of more tiles than the G
 * workgroups that fit the GPU at once (one per CU) but at most half again as
 * many. Its G workgroups take the T tiles of the one-tile-per-workgroup
 * launch: workgroup w computes the tile the first round's workgroup w would
 * (sk_full_id), and the T - G tiles of the second round are each cut at half
 * of K between two workgroups of one XCD, w and w + 8 with w / 8 even
 * (dispatch puts workgroup i on XCD i % 8). The lower id, the writer, runs
 * stages [0, h) of its tail tile first and leaves the sums in a workspace
 * slot, then its own tile; the higher id, the reader, runs its own tile,
 * then stages [h, steps) of the tail tile, and adds the writer's sums at the
 * end. The reader waits only for a workgroup dispatched before it. */
VX_PP_FN bool sk_fits(int tiles, int groups, int steps) {
  return groups >= 16 && groups % 8 == 0 && tiles % 8 == 0 && tiles > groups &&
         2 * (tiles - groups) <= groups && steps >= 8;
}
/* For a grid of `all` tiles: the first launch-order id the stream-K launch
 * takes (the one-tile launch runs the ids before it), or -1 when the grid
 * has no such tail: `all` = q G + r with q >= 1 and 0 < r <= G / 2, and
 * G + r taken by sk_fits. */
VX_PP_FN int sk_base(int all, int groups, int steps) {
  if (groups <= 0 || all <= groups) {
    return -1;
  }
  const int q = all / groups, r = all - q * groups;
  if (r == 0 || !sk_fits(groups + r, groups, steps)) {
    return -1;
  }
  return (q - 1) * groups;
}
VX_PP_FN int sk_full_id(int w, int tiles) { return (w & 7) * (tiles >> 3) + (w >> 3); }
/* The tail slot (0 .. T - G - 1) workgroup w shares, or -1. */
VX_PP_FN int sk_slot(int w, int tiles, int groups) {
  const int per_xcd = (tiles - groups) >> 3;
  const int pair = w >> 4;
  return pair < per_xcd ? (w & 7) * per_xcd + pair : -1;
}
VX_PP_FN int sk_tail_id(int slot, int tiles, int groups) {
  const int per_xcd = (tiles - groups) >> 3;
  return (slot / per_xcd) * (tiles >> 3) + (groups >> 3) + slot % per_xcd;
}
VX_PP_FN bool sk_reader(int w) { return ((w >> 3) & 1) != 0; }
/* The split: the writer takes 5 stages past half, since the reader's part
 * carries the hand-over and the final sum (about 10 us more fixed time per
 * tile than the writer's, in a per-workgroup timeline of 8192 x 3072 x 768;
 * splits at 1/2 and 2/3 left the reader or, at K = 4096, the writer last). */
VX_PP_FN int sk_split(int steps) {
  return steps / 2 + 5 < steps - 1 ? steps / 2 + 5 : steps - 1;
}

/* The stages workgroup w runs: unit 0 (len0 stages from stage 0 of tile
 * u0), then unit 1 (len1 stages from stage begin1 of tile u1; none for a
 * workgroup without a tail slot). */
struct SkUnits {
  Tile u0, u1;
  int len0, begin1, len1;
  int slot;
  bool writer, reader;
};
/* The stream-K launch takes the `tiles` launch-order ids from `id_base` on:
 * all of a grid of one to one and a half rounds (id_base 0), or the last
 * G + r ids of a grid of q G + r tiles, q >= 2, whose first (q - 1) G ids
 * the one-tile launch runs before it (sk_base). */
VX_PP_FN SkUnits sk_units(int w, int tiles_m, int tiles_n, int id_base, int tiles, int groups,
                          int steps) {
  SkUnits u;
  u.slot = sk_slot(w, tiles, groups);
  u.reader = u.slot >= 0 && sk_reader(w);
  u.writer = u.slot >= 0 && !sk_reader(w);
  const Tile own = tile_at(id_base + sk_full_id(w, tiles), tiles_m, tiles_n);
  const Tile tail =
      u.slot >= 0 ? tile_at(id_base + sk_tail_id(u.slot, tiles, groups), tiles_m, tiles_n) : own;
  const int h = sk_split(steps);
  /* field by field: a select between whole structs can become an indexed
   * load from a private copy, which the GPU compiler treats as per-lane */
  u.u0.tm = u.writer ? tail.tm : own.tm;
  u.u0.tn = u.writer ? tail.tn : own.tn;
  u.u1.tm = u.writer ? own.tm : tail.tm;
  u.u1.tn = u.writer ? own.tn : tail.tn;
  u.len0 = u.writer ? h : steps;
  u.begin1 = u.reader ? h : 0;
  u.len1 = u.slot < 0 ? 0 : (u.reader ? steps - h : steps);
  return u;
}
/* Tile and K stage of the workgroup's stage s (0 .. len0 + len1 - 1), from
 * its units' fields (plain integers, so the GPU keeps them scalar). */
VX_PP_FN void sk_stage(int len0, int begin1, int tm0, int tn0, int tm1, int tn1, int s,
                       int &tm, int &tn, int &step) {
  const bool second = s >= len0;
  tm = second ? tm1 : tm0;
  tn = second ? tn1 : tn0;
  step = second ? begin1 + (s - len0) : s;
}
VX_PP_FN void sk_stage(const SkUnits &u, int s, int &tm, int &tn, int &step) {
  sk_stage(u.len0, u.begin1, u.u0.tm, u.u0.tn, u.u1.tm, u.u1.tn, s, tm, tn, step);
}

/* The stream-K workspace: kSkMaxSlots x kWaves flags (ints) at its start,
 * then each slot's partial sums, 256 x 256 floats laid out as [wave][i][jj]
 * [lane] f32x4, so writer and reader waves of the same index move whole
 * 1 KiB rows of their accumulators. */
constexpr int kSkMaxSlots = 1024;
constexpr int kSkSlotFloats = kTileM * kTileN;
constexpr int64_t kSkFlagBytes = (int64_t)kSkMaxSlots * kWaves * 4;
VX_PP_FN int64_t sk_bytes(int slots) {
  return kSkFlagBytes + (int64_t)slots * kSkSlotFloats * 4;
}
VX_PP_FN int sk_flag(int slot, int wave) { return slot * kWaves + wave; }
/* Byte offset, within slot `slot`'s partial sums, of the f32x4 that block
 * (i, jj) of `wave` holds in `lane`. */
VX_PP_FN uint32_t sk_part_off(int wave, int i, int jj, int lane) {
  return (uint32_t)((((wave * kTM + i) * kTN + jj) * 64 + lane) * 16);
}
VX_PP_FN int64_t sk_slot_off(int slot) {
  return kSkFlagBytes + (int64_t)slot * kSkSlotFloats * 4;
}

/* A's LDS plane is [256 rows][4 chunks of 8 k], chunk XORed with bits 1-2
 * of the row; B's keeps global order [32 k][256 n] in 16-byte chunks, chunk
 * XORed by a function of k (bits 0, 1 and 3). */
VX_PP_FN int dswz_a(int row, int c) { return c ^ (((row >> 1) ^ (row >> 2)) & 3); }
VX_PP_FN int pswz_b(int k, int c) {
  return c ^ (((k & 3) | (((k >> 3) & 1) << 2)) << 1);
}

/* Byte offset, from the stage's A base, of load p of `wave` for `lane`: the
 * global 16 bytes that belong at the LDS unit that load writes. */
VX_PP_FN uint32_t a_load_off(int wave, int p, int lane, int64_t lda) {
  const int u = (wave * kLoads + p) * 64 + lane;
  const int arow = u >> 2;
  return (uint32_t)(arow * lda * 2 + dswz_a(arow, u & 3) * 16);
}
VX_PP_FN uint32_t b_load_off(int wave, int p, int lane, int64_t ldb) {
  const int u = (wave * kLoads + p) * 64 + lane;
  const int bk = u >> 5;
  return (uint32_t)(bk * ldb * 2 + pswz_b(bk, u & 31) * 16);
}

/* LDS byte address (from the ring's start) where load p of `wave` writes;
 * lane i's 16 bytes land at this + 16 i. */
VX_PP_FN uint32_t lds_a_dst(int slot, int wave, int p) {
  return (uint32_t)(slot * 2 * kPlaneBytes) + (uint32_t)(wave * kLoads * 64 * 16) +
         (uint32_t)(p * 64 * 16);
}
VX_PP_FN uint32_t lds_b_dst(int slot, int wave, int p) {
  return lds_a_dst(slot, wave, p) + (uint32_t)kPlaneBytes;
}

/* Element offsets of K stage `step`'s A and B blocks for the tile at
 * (m0, n0). */
VX_PP_FN int64_t a_stage_base(int64_t m0, int64_t lda, int step) {
  return m0 * lda + (int64_t)step * kStageK;
}
VX_PP_FN int64_t b_stage_base(int64_t n0, int64_t ldb, int step) {
  return (int64_t)step * kStageK * ldb + n0;
}

/* The buffer range (bytes) of a stage whose A block starts at element a0:
 * the whole 256 x 32 block, cut at the last element of A, so rows past M
 * read zeros. Likewise for B (32 x 256 from b0, cut at B's last element). */
VX_PP_FN int a_stage_bytes(int64_t M, int K, int64_t lda, int64_t a0) {
  const int64_t full = (kTileM - 1) * lda * 2 + kStageK * 2;
  const int64_t end = ((M - 1) * lda + K) * 2;
  const int64_t left = end - a0 * 2;
  return (int)(full < left ? full : left);
}
VX_PP_FN int b_stage_bytes(int64_t N, int K, int64_t ldb, int64_t b0) {
  const int64_t full = (kStageK - 1) * ldb * 2 + kTileN * 2;
  const int64_t end = ((int64_t)(K - 1) * ldb + N) * 2;
  const int64_t left = end - b0 * 2;
  return (int)(full < left ? full : left);
}

/* A lane's operand fields: l16 = lane % 16, kc = lane / 16. */

/* The A operand of row block i of wave (wm, .) for the lane (l16, kc): the
 * index of its 16-byte unit in the stage's A plane (row l16, k chunk kc). */
VX_PP_FN int lds_a_read(int wm, int i, int l16, int kc) {
  const int row = wm * 128 + i * 16 + l16;
  return row * 4 + dswz_a(row, kc);
}

/* Byte offset in the stage's B plane of half h of the B operand of column
 * block j of wave (., wn) for the lane (l16, kc) (one ds_read_b64_tr_b16:
 * lanes 4e..4e+3 of each group of 16 read 4 columns of row k + e). */
VX_PP_FN int lds_b_read(int wn, int j, int h, int l16, int kc) {
  const int n = wn * 64 + j * 16 + 4 * (l16 & 3);
  const int k = 8 * kc + 4 * h + (l16 >> 2);
  return k * (kTileN * 2) + pswz_b(k, n >> 3) * 16 + (n & 7) * 2;
}

/* Row and first column within the tile of the C elements that block
 * (i, jj) of wave (wm, wn) holds for the lane (l16, kc). The MFMA takes B's
 * fragment as its first operand and A's as its second, so it accumulates
 * C^T: the lane's accumulator elements r = 0..3 are columns c_col + r of
 * row c_row (one 16-byte store of f32). */
VX_PP_FN int c_row(int wm, int i, int l16) { return wm * 128 + i * 16 + l16; }
VX_PP_FN int c_col(int wn, int jj, int kc) { return wn * 64 + jj * 16 + 4 * kc; }

} // namespace pp
} // namespace vxk

#endif /* VX_AMD_GEMM_PP_LAYOUT_H */
