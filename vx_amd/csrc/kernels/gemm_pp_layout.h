/*
 * gemm_pp_layout.h -- the address arithmetic of gemm_mfma_pp (gemm.hip),
 * written once for the kernel and for the CPU check that walks it
 * (tests/native/gemm_pp_addr_test.cpp): the launch order, the buffer-to-LDS
 * load offsets and buffer ranges of each K stage, the LDS slots those loads
 * fill, the LDS reads of the MFMA operands and the epilogue's C indices.
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

/* The C tile workgroup `block` of `nwg` computes. Workgroup i runs on XCD
 * i % 8; the renumbering gives each XCD consecutive ids, which walk C in
 * groups of group_m tile rows, column by column. */
VX_PP_FN Tile tile_of(int block, int nwg, int tiles_m, int tiles_n) {
  int id = block;
  if ((nwg & 7) == 0) {
    id = (id & 7) * (nwg >> 3) + (id >> 3);
  }
  const int group_m = tiles_m * tiles_n <= kSmallGrid ? kSmallGroupM : kGroupM;
  const int group_size = group_m * tiles_n;
  const int first_m = (id / group_size) * group_m;
  const int rows_in_group =
      tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  const int in_group = id % group_size;
  return Tile{first_m + in_group % rows_in_group, in_group / rows_in_group};
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
