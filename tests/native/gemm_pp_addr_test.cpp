// Walks the addressing of the ping-pong MFMA GEMM (gemm_mfma_pp) on the CPU,
// through the same functions the kernel calls (vx_amd/csrc/kernels/
// gemm_pp_layout.h), for every shape class the GPU tests and the bench run:
// the 4096^3 and 8192^3 configs, the reference benchmark's 8192x3072x768,
// ragged and padded edges, and views with padded rows.
//
// For each shape it checks, against the smallest allocations a caller may
// pass (A: (M-1)*lda + K elements, B: (K-1)*ldb + N, C: (M-1)*ldc + N):
//  - the launch order is a bijection from workgroups onto C tiles;
//  - every stage's buffer base and range stay inside A and B (a load whose
//    16 bytes pass the range reads zeros and touches no memory), with every
//    range and load offset inside 31 bits;
//  - every buffer-to-LDS load of a stage writes its own 16 bytes of that
//    stage's 32 KiB slot, inside the 128 KiB ring;
//  - every A operand read finds, in LDS, the global row and k chunk the
//    MFMA expects (the swizzles of the load and of the read undo each
//    other), and every B operand read stays inside its plane;
//  - the epilogue stores every C element once, inside C.
// Prints "ok" when every check holds.

#include "../../vx_amd/csrc/kernels/gemm_pp_layout.h"

#include <cstdio>
#include <cstdlib>
#include <map>
#include <vector>

namespace pp = vxk::pp;

static int failures = 0;
#define CHECK(cond, ...)                                                   \
  do {                                                                     \
    if (!(cond)) {                                                         \
      if (failures++ < 20) {                                               \
        fprintf(stderr, "%s:%d: %s: ", __FILE__, __LINE__, #cond);         \
        fprintf(stderr, __VA_ARGS__);                                      \
        fprintf(stderr, "\n");                                             \
      }                                                                    \
    }                                                                      \
  } while (0)

struct Shape {
  int64_t m, n, k, lda, ldb, ldc;
};

static void walk(const Shape &s) {
  CHECK(pp::shape_ok(s.m, s.n, s.k, s.lda, s.ldb, s.ldc), "shape %lldx%lldx%lld",
        (long long)s.m, (long long)s.n, (long long)s.k);
  const int tiles_m = (int)((s.m + pp::kTileM - 1) / pp::kTileM);
  const int tiles_n = (int)((s.n + pp::kTileN - 1) / pp::kTileN);
  const int nwg = tiles_m * tiles_n;
  const int steps = (int)(s.k / pp::kStageK);
  const int64_t a_bytes = ((s.m - 1) * s.lda + s.k) * 2;
  const int64_t b_bytes = ((s.k - 1) * s.ldb + s.n) * 2;
  const int64_t c_elems = (s.m - 1) * s.ldc + s.n;

  // Load offsets of one stage, the same for every workgroup and stage.
  std::vector<int64_t> a_off, b_off;
  std::vector<uint32_t> a_dst_unit, b_dst_unit;
  for (int wave = 0; wave < pp::kWaves; ++wave) {
    for (int p = 0; p < pp::kLoads; ++p) {
      for (int lane = 0; lane < 64; ++lane) {
        const int u = (wave * pp::kLoads + p) * 64 + lane;
        const int arow = u >> 2, bk = u >> 5;
        const int64_t ao = arow * s.lda * 2 + pp::dswz_a(arow, u & 3) * 16;
        const int64_t bo = bk * s.ldb * 2 + pp::pswz_b(bk, u & 31) * 16;
        CHECK(ao == (int64_t)pp::a_load_off(wave, p, lane, s.lda) && ao < INT32_MAX,
              "A load offset %lld", (long long)ao);
        CHECK(bo == (int64_t)pp::b_load_off(wave, p, lane, s.ldb) && bo < INT32_MAX,
              "B load offset %lld", (long long)bo);
        a_off.push_back(ao);
        b_off.push_back(bo);
      }
    }
  }

  // LDS destinations: each slot's 2048 units written once, inside the ring.
  for (int slot = 0; slot < pp::kSlots; ++slot) {
    std::vector<int> hits(2 * pp::kUnits, 0);
    for (int wave = 0; wave < pp::kWaves; ++wave) {
      for (int p = 0; p < pp::kLoads; ++p) {
        for (int lane = 0; lane < 64; ++lane) {
          const uint32_t ad = pp::lds_a_dst(slot, wave, p) + 16u * lane;
          const uint32_t bd = pp::lds_b_dst(slot, wave, p) + 16u * lane;
          CHECK(ad + 16 <= (uint32_t)pp::kRingBytes && bd + 16 <= (uint32_t)pp::kRingBytes,
                "LDS destination %u / %u", ad, bd);
          const uint32_t base = (uint32_t)(slot * 2 * pp::kPlaneBytes);
          CHECK(ad >= base && bd >= base, "LDS destination below slot %d", slot);
          if (ad >= base && ad < base + 2 * pp::kPlaneBytes) {
            hits[(ad - base) / 16]++;
          }
          if (bd >= base && bd < base + 2 * pp::kPlaneBytes) {
            hits[(bd - base) / 16]++;
          }
          if (slot == 0) {
            a_dst_unit.push_back(ad / 16);
            b_dst_unit.push_back((bd - pp::kPlaneBytes) / 16);
          }
        }
      }
    }
    for (int u = 0; u < 2 * pp::kUnits; ++u) {
      CHECK(hits[u] == 1, "slot %d unit %d written %d times", slot, u, hits[u]);
    }
  }

  // A operand reads: the unit read holds the row and k chunk the MFMA needs.
  std::map<uint32_t, int64_t> a_unit_src;  // A-plane unit -> global byte offset
  for (size_t i = 0; i < a_off.size(); ++i) {
    a_unit_src[a_dst_unit[i]] = a_off[i];
  }
  for (int wm = 0; wm < 2; ++wm) {
    for (int i = 0; i < pp::kTM; ++i) {
      for (int lane = 0; lane < 64; ++lane) {
        const int l16 = lane & 15, kc = lane >> 4;
        const int u = pp::lds_a_read(wm, i, l16, kc);
        CHECK(u >= 0 && u < pp::kUnits, "A read unit %d", u);
        const auto found = a_unit_src.find((uint32_t)u);
        CHECK(found != a_unit_src.end(), "A unit %d never loaded", u);
        if (found != a_unit_src.end()) {
          const int64_t row = found->second / (s.lda * 2);
          const int64_t chunk = (found->second % (s.lda * 2)) / 16;
          CHECK(row == wm * 128 + i * 16 + l16 && chunk == kc,
                "A read (wm %d, i %d, lane %d) finds row %lld chunk %lld", wm, i, lane,
                (long long)row, (long long)chunk);
        }
      }
    }
  }
  // B operand reads stay inside the B plane (the transposing read takes 8
  // bytes at each lane's address).
  for (int wn = 0; wn < 4; ++wn) {
    for (int j = 0; j < pp::kTN; ++j) {
      for (int h = 0; h < 2; ++h) {
        for (int lane = 0; lane < 64; ++lane) {
          const int at = pp::lds_b_read(wn, j, h, lane & 15, lane >> 4);
          CHECK(at >= 0 && at + 8 <= pp::kPlaneBytes && at % 8 == 0, "B read at %d", at);
        }
      }
    }
  }

  // Per workgroup: the tile, every stage's ranges, the epilogue stores.
  std::vector<uint8_t> tile_seen((size_t)nwg, 0);
  std::vector<uint8_t> c_seen((size_t)c_elems, 0);
  int64_t a_max_off = 0, b_max_off = 0;
  for (size_t i = 0; i < a_off.size(); ++i) {
    a_max_off = a_off[i] > a_max_off ? a_off[i] : a_max_off;
    b_max_off = b_off[i] > b_max_off ? b_off[i] : b_max_off;
  }
  for (int block = 0; block < nwg; ++block) {
    const pp::Tile t = pp::tile_of(block, nwg, tiles_m, tiles_n);
    CHECK(t.tm >= 0 && t.tm < tiles_m && t.tn >= 0 && t.tn < tiles_n, "block %d -> (%d, %d)",
          block, t.tm, t.tn);
    if (t.tm < 0 || t.tm >= tiles_m || t.tn < 0 || t.tn >= tiles_n) {
      continue;
    }
    CHECK(tile_seen[(size_t)t.tm * tiles_n + t.tn]++ == 0, "tile (%d, %d) twice", t.tm, t.tn);
    const int64_t m0 = (int64_t)t.tm * pp::kTileM, n0 = (int64_t)t.tn * pp::kTileN;
    for (int step = 0; step < steps; ++step) {
      const int64_t a0 = pp::a_stage_base(m0, s.lda, step);
      const int64_t b0 = pp::b_stage_base(n0, s.ldb, step);
      const int ra = pp::a_stage_bytes(s.m, (int)s.k, s.lda, a0);
      const int rb = pp::b_stage_bytes(s.n, (int)s.k, s.ldb, b0);
      CHECK(a0 >= 0 && ra > 0 && a0 * 2 + ra <= a_bytes, "A stage %d of block %d: base %lld range %d",
            step, block, (long long)a0, ra);
      CHECK(b0 >= 0 && rb > 0 && b0 * 2 + rb <= b_bytes, "B stage %d of block %d: base %lld range %d",
            step, block, (long long)b0, rb);
      // A load is made only when its 16 bytes fit the range; the largest
      // offset that does must then lie inside the allocation.
      if (a_max_off + 16 <= ra) {
        CHECK(a0 * 2 + a_max_off + 16 <= a_bytes, "A load past the allocation");
      }
      if (b_max_off + 16 <= rb) {
        CHECK(b0 * 2 + b_max_off + 16 <= b_bytes, "B load past the allocation");
      }
    }
    for (int wave = 0; wave < pp::kWaves; ++wave) {
      const int wm = wave >> 2, wn = wave & 3;
      for (int lane = 0; lane < 64; ++lane) {
        for (int i = 0; i < pp::kTM; ++i) {
          for (int jj = 0; jj < pp::kTN; ++jj) {
            // the kernel's guard: the row and the first of the lane's 4
            // columns; the 4 must then all lie in the row
            const int64_t row = m0 + pp::c_row(wm, i, lane & 15);
            const int64_t col0 = n0 + pp::c_col(wn, jj, lane >> 4);
            if (!(row < s.m && col0 < s.n)) {
              continue;
            }
            CHECK(col0 + 3 < s.n, "C columns %lld..+3 pass N", (long long)col0);
            if (s.ldc % 4 == 0) {
              CHECK((row * s.ldc + col0) % 4 == 0, "16-byte C store misaligned");
            }
            for (int r = 0; r < 4; ++r) {
              const int64_t col = col0 + r;
              const int64_t at = row * s.ldc + col;
              CHECK(at >= 0 && at < c_elems, "C store at %lld", (long long)at);
              if (at >= 0 && at < c_elems) {
                CHECK(c_seen[(size_t)at]++ == 0, "C (%lld, %lld) stored twice", (long long)row,
                      (long long)col);
              }
            }
          }
        }
      }
    }
  }
  for (int64_t row = 0; row < s.m; ++row) {
    for (int64_t col = 0; col < s.n; ++col) {
      CHECK(c_seen[(size_t)(row * s.ldc + col)] == 1, "C (%lld, %lld) never stored",
            (long long)row, (long long)col);
      if (failures > 20) {
        return;
      }
    }
  }
}

int main() {
  const Shape shapes[] = {
      {4096, 4096, 4096, 4096, 4096, 4096},
      {8192, 8192, 8192, 8192, 8192, 8192},    // its roofline point
      {8192, 3072, 768, 768, 3072, 3072},      // the reference's own GEMM benchmark
      {1000, 776, 512, 512, 776, 779},         // ragged, C inside a sentinel frame
      {300, 4104, 64, 64, 4104, 4107},
      {257, 776, 96, 96, 784, 779},            // B rows padded
      {1, 8, 32, 32, 8, 11},
      {4100, 296, 128, 128, 304, 299},
      {512, 512, 512, 520, 520, 530},          // views with padded rows
      {256, 256, 32, 32, 256, 256},            // one tile, one stage
      {2048, 2048, 96, 104, 2056, 2048},       // ragged-free, deep padding
  };
  for (const Shape &s : shapes) {
    walk(s);
    if (failures) {
      fprintf(stderr, "failed on %lldx%lldx%lld\n", (long long)s.m, (long long)s.n,
              (long long)s.k);
      return 1;
    }
  }
  // The predicate refuses what the kernel cannot take.
  CHECK(!pp::shape_ok(257, 777, 96, 96, 777, 777), "N = 777 taken");
  CHECK(!pp::shape_ok(256, 256, 100, 104, 256, 256), "K = 100 taken");
  CHECK(!pp::shape_ok(256, 256, 96, 100, 256, 256), "lda = 100 taken");
  CHECK(!pp::shape_ok(256, 256, 96, 96, 252, 256), "ldb < N taken");
  CHECK(!pp::shape_ok(1 << 20, 256, 96, 1 << 23, 256, 256), "lda past 31 bits taken");
  if (failures) {
    return 1;
  }
  printf("ok\n");
  return 0;
}
