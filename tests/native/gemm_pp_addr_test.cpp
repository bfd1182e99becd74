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
// For the stream-K launch (the last G + r tiles of grids of q G + r tiles,
// 0 < r <= G / 2, after a one-tile launch of the first (q - 1) G; G = 16 ..
// 304) it checks that every (tile, K stage) is run by
// exactly one workgroup, each tail tile's two halves by a writer and a reader
// on one XCD (reader = writer + 8) whose stage ranges meet at the split, the
// reader continuing the writer's order; that each workgroup's own tile is
// the one the one-tile launch gives its first-round workgroup and the tail
// tiles of an XCD are that launch's second-round tiles on it; that every
// tile is stored once; and that slots, flags and partial-sum offsets stay in
// the workspace.
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

static void walk_sk(const Shape &s, int groups) {
  const int tiles_m = (int)((s.m + pp::kTileM - 1) / pp::kTileM);
  const int tiles_n = (int)((s.n + pp::kTileN - 1) / pp::kTileN);
  const int all = tiles_m * tiles_n;
  const int steps = (int)(s.k / pp::kStageK);
  // The one-tile launch runs launch-order ids [0, base), the stream-K launch
  // the last `tiles`.
  const int base = pp::sk_base(all, groups, steps);
  CHECK(base >= 0 && base % groups == 0, "%d tiles on %d groups refused", all, groups);
  if (base < 0 || base % groups != 0) {
    return;
  }
  const int tiles = all - base;
  CHECK(pp::sk_fits(tiles, groups, steps), "%d stream-K tiles on %d groups", tiles, groups);
  const int slots = tiles - groups;
  CHECK(slots > 0 && slots <= pp::kSkMaxSlots, "%d slots", slots);
  if (!pp::sk_fits(tiles, groups, steps) || slots <= 0 || slots > pp::kSkMaxSlots) {
    return;
  }
  // The tile the one-tile launch of the stream-K share's ids gives its
  // workgroup p (p in [0, tiles)).
  auto launch_tile = [&](int p) {
    return pp::tile_at(base + ((p & 7) * (tiles >> 3) + (p >> 3)), tiles_m, tiles_n);
  };
  std::vector<int> cover((size_t)all * steps, 0), stored((size_t)all, 0);
  std::vector<int> writer_of((size_t)slots, -1), reader_of((size_t)slots, -1);
  for (int b = 0; b < base; ++b) {
    const pp::Tile t = pp::tile_of(b, base, tiles_m, tiles_n);
    for (int st = 0; st < steps; ++st) {
      cover[((size_t)t.tm * tiles_n + t.tn) * steps + st]++;
    }
    stored[(size_t)t.tm * tiles_n + t.tn]++;
  }
  for (int w = 0; w < groups; ++w) {
    const pp::SkUnits u = pp::sk_units(w, tiles_m, tiles_n, base, tiles, groups, steps);
    // its own tile is the one-tile launch's first-round tile of w
    const pp::Tile first = launch_tile(w);
    const pp::Tile own = u.writer ? u.u1 : u.u0;
    CHECK(own.tm == first.tm && own.tn == first.tn, "workgroup %d own tile", w);
    CHECK(u.writer + u.reader == (u.slot >= 0 ? 1 : 0), "workgroup %d role", w);
    CHECK(u.len0 >= 1 && u.len1 >= 0 && u.len0 + u.len1 < 2 * steps,
          "workgroup %d lengths %d %d", w, u.len0, u.len1);
    for (int st = 0; st < u.len0 + u.len1; ++st) {
      int tm, tn, step;
      pp::sk_stage(u, st, tm, tn, step);
      CHECK(tm >= 0 && tm < tiles_m && tn >= 0 && tn < tiles_n && step >= 0 && step < steps,
            "workgroup %d stage %d -> (%d, %d) step %d", w, st, tm, tn, step);
      if (tm >= 0 && tm < tiles_m && tn >= 0 && tn < tiles_n && step >= 0 && step < steps) {
        cover[((size_t)tm * tiles_n + tn) * steps + step]++;
      }
    }
    // the tiles it stores: a reader both units, others its last unit
    if (u.reader) {
      stored[(size_t)u.u0.tm * tiles_n + u.u0.tn]++;
    }
    const pp::Tile last = u.len1 > 0 ? u.u1 : u.u0;
    stored[(size_t)last.tm * tiles_n + last.tn]++;
    if (u.slot >= 0) {
      CHECK(u.slot < slots, "workgroup %d slot %d", w, u.slot);
      if (u.slot < slots) {
        (u.writer ? writer_of : reader_of)[(size_t)u.slot] = w;
      }
    }
  }
  for (int t = 0; t < all; ++t) {
    CHECK(stored[(size_t)t] == 1, "tile %d stored %d times", t, stored[(size_t)t]);
    for (int st = 0; st < steps; ++st) {
      CHECK(cover[(size_t)t * steps + st] == 1, "tile %d stage %d run %d times", t, st,
            cover[(size_t)t * steps + st]);
    }
    if (failures > 20) {
      return;
    }
  }
  std::vector<int> second_round((size_t)all, 0);
  for (int p = groups; p < tiles; ++p) {
    const pp::Tile t = launch_tile(p);
    second_round[(size_t)t.tm * tiles_n + t.tn] = 1 + (p & 7);
  }
  for (int sl = 0; sl < slots; ++sl) {
    const int wr = writer_of[(size_t)sl], rd = reader_of[(size_t)sl];
    CHECK(wr >= 0 && rd == wr + 8 && (wr & 7) == (rd & 7), "slot %d: writer %d reader %d", sl,
          wr, rd);
    if (wr < 0 || rd < 0) {
      continue;
    }
    const pp::SkUnits a = pp::sk_units(wr, tiles_m, tiles_n, base, tiles, groups, steps);
    const pp::SkUnits b = pp::sk_units(rd, tiles_m, tiles_n, base, tiles, groups, steps);
    CHECK(a.u0.tm == b.u1.tm && a.u0.tn == b.u1.tn, "slot %d: halves of two tiles", sl);
    CHECK(a.len0 == b.begin1 && b.begin1 + b.len1 == steps, "slot %d: split %d / %d + %d", sl,
          a.len0, b.begin1, b.len1);
    CHECK(second_round[(size_t)a.u0.tm * tiles_n + a.u0.tn] == 1 + (wr & 7),
          "slot %d: tail tile not the one-tile launch's second-round tile on XCD %d", sl,
          wr & 7);
    for (int wave = 0; wave < pp::kWaves; ++wave) {
      CHECK(pp::sk_flag(sl, wave) < pp::kSkMaxSlots * pp::kWaves, "flag of slot %d", sl);
    }
    CHECK(pp::sk_slot_off(sl) + (int64_t)pp::kSkSlotFloats * 4 <= pp::sk_bytes(slots) &&
              pp::sk_slot_off(sl) >= pp::kSkFlagBytes && pp::sk_slot_off(sl) % 256 == 0,
          "slot %d at %lld", sl, (long long)pp::sk_slot_off(sl));
  }
}

static void walk_sk_slot_layout() {
  std::vector<int> seen((size_t)pp::kSkSlotFloats / 4, 0);
  for (int wave = 0; wave < pp::kWaves; ++wave) {
    for (int i = 0; i < pp::kTM; ++i) {
      for (int jj = 0; jj < pp::kTN; ++jj) {
        for (int lane = 0; lane < 64; ++lane) {
          const uint32_t off = pp::sk_part_off(wave, i, jj, lane);
          CHECK(off == pp::sk_part_off(wave, i, jj, 0) + 16u * lane, "lane stride");
          CHECK(off % 16 == 0 && off + 16 <= (uint32_t)pp::kSkSlotFloats * 4, "part at %u", off);
          if (off % 16 == 0 && off + 16 <= (uint32_t)pp::kSkSlotFloats * 4) {
            seen[off / 16]++;
          }
        }
      }
    }
  }
  for (size_t u = 0; u < seen.size(); ++u) {
    CHECK(seen[u] == 1, "partial unit %zu written %d times", u, seen[u]);
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
  walk_sk_slot_layout();
  const struct {
    Shape s;
    int groups;
  } sk_cases[] = {
      {{8192, 3072, 768, 768, 3072, 3072}, 256},   // the reference's benchmark: 384 tiles
      {{8192, 2304, 768, 768, 2304, 2304}, 256},   // 288 tiles: 32 of 128 pairs
      {{8000, 3000, 288, 288, 3000, 3001}, 256},   // ragged, odd stage count (9)
      {{4864, 6144, 512, 512, 6144, 6144}, 304},   // 456 tiles on 304 CUs
      {{2048, 2560, 4096, 4096, 2560, 2560}, 64},  // 80 tiles on 64
      {{1024, 1536, 256, 264, 1544, 1540}, 16},    // 24 tiles on 16, padded rows
      {{12288, 3072, 768, 768, 3072, 3072}, 256},  // 576 tiles: one-tile round, then 320
      {{7936, 8192, 512, 512, 8192, 8192}, 304},   // 992 tiles: two one-tile rounds, then 384
      {{12100, 2800, 320, 320, 2800, 2803}, 256},  // ragged, 2 rounds + 40 (11 x 48 = 528)
  };
  for (const auto &c : sk_cases) {
    walk_sk(c.s, c.groups);
    if (failures) {
      fprintf(stderr, "stream-K failed on %lldx%lldx%lld at %d groups\n", (long long)c.s.m,
              (long long)c.s.n, (long long)c.s.k, c.groups);
      return 1;
    }
  }
  CHECK(!pp::sk_fits(256, 256, 24), "one round taken");
  CHECK(!pp::sk_fits(392, 256, 24), "more than one and a half rounds taken");
  CHECK(!pp::sk_fits(300, 256, 24), "tiles not a multiple of 8 taken");
  CHECK(!pp::sk_fits(384, 256, 4), "too few stages taken");
  CHECK(pp::sk_base(384, 256, 24) == 0 && pp::sk_base(640, 256, 24) == 256 &&
            pp::sk_base(1152, 256, 24) == 768,
        "stream-K share of multi-round grids");
  CHECK(pp::sk_base(256, 256, 24) < 0 && pp::sk_base(512, 256, 24) < 0 &&
            pp::sk_base(448, 256, 24) < 0 && pp::sk_base(300, 256, 24) < 0,
        "grids without a stream-K tail taken");

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
