/*
 * vx_image_launch.h -- the host side of running a device image that a
 * dispatch payload carries (`format=hsaco`): turning the plugin ABI's
 * arguments into kernel parameters, reading the launch shape the payload
 * asks for, and reading how many parameters the image's kernel declares.
 * No HIP calls here, so all of it can be checked on a machine without a GPU.
 *
 * Parameters. A compiled kernel takes one parameter per *field* of each
 * memref argument -- allocated pointer, aligned pointer, offset, then one
 * size and one stride per dimension, every one 8 bytes -- and one per scalar.
 * A descriptor in memory is already those fields in that order, so the
 * parameter list is addresses into the descriptors the caller passed, the
 * form hipModuleLaunchKernel takes (reference runtime/vx_kernel_launch.h:
 * 57-140 for the same layout on the CUDA side).
 *
 * Shape. `grid=` and `block=` (each size a number or `$j`, the i32 launch
 * value j after the kernel's arguments; `grid_loops=` clamps instead of
 * refusing), else `launch=` (the trip count of a grid-strided loop, or `B,T`),
 * else one thread (reference runtime/vx_kernel_launch.h:366-473 and
 * runtime/cuda_dispatch.cpp:1560-1606).
 *
 * Declared parameters. An AMDGPU code object records each kernel's
 * arguments in its metadata note (NT_AMDGPU_METADATA, a MessagePack map:
 * amdhsa.kernels -> [{.name, .args: [{.value_kind, ...}]}]). The arguments
 * whose kind starts with "hidden_" are the ones the runtime appends (block
 * counts, group sizes, offsets); the rest are the kernel's own and must equal
 * what the ABI produces, or the launch would read parameters never written.
 * The image is a bare ELF or a clang offload bundle holding one per target.
 */
#pragma once

#include "../../include/vx_hardware_runtime.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace vx {

constexpr int kImageMaxParams = 128;

struct ImageParams {
  void *p[kImageMaxParams];
  int count = 0;
};

/* Parameters one argument expands into; 0 for one that cannot be marshalled
 * (a publication slot, whose descriptor does not exist before the kernel
 * writes it, or an unknown scalar type). */
inline int image_param_width(int32_t tag) {
  if (VX_ABI_IS_SLOT(tag)) {
    return 0;
  }
  if (VX_ABI_KIND(tag) == VX_ABI_KIND_MEMREF) {
    const int32_t rank = (int32_t)VX_ABI_RANK(tag);
    return rank < 0 || rank > VX_ABI_MAX_RANK ? 0 : 3 + 2 * rank;
  }
  return vx_dtype_bytes(VX_ABI_KIND(tag)) ? 1 : 0;
}

/* The parameter list of a dispatch: false (and nothing partial) when an
 * argument cannot be marshalled or the list would not fit. */
inline bool image_build_params(void *const *args, const int32_t *tags,
                               int64_t n, ImageParams &out) {
  out.count = 0;
  if (!args || !tags || n < 0) {
    return false;
  }
  int count = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int width = image_param_width(tags[i]);
    if (width == 0 || count + width > kImageMaxParams || !args[i]) {
      return false;
    }
    if (VX_ABI_KIND(tags[i]) != VX_ABI_KIND_MEMREF) {
      out.p[count++] = args[i];
      continue;
    }
    char *desc = static_cast<char *>(*static_cast<void *const *>(args[i]));
    if (!desc) {
      return false;
    }
    const int32_t rank = (int32_t)VX_ABI_RANK(tags[i]);
    for (int f = 0; f < 3 + 2 * rank; ++f) {
      out.p[count++] = desc + 8 * f;
    }
  }
  out.count = count;
  return true;
}

/* One size of a shape entry at `*text`: a number, or `$j` for launch value j
 * (an i32 after the n arguments). Moves past the size and its comma; -1 when
 * launch value j is missing or not an i32. */
inline long image_launch_size(const char **text, void *const *args,
                              const int32_t *tags, int64_t n) {
  char *end = nullptr;
  long value;
  if (**text == '$') {
    const long j = strtol(*text + 1, &end, 10);
    if (j < 0 || j > 3 || tags[n + j] != VX_ABI_KIND_I32) {
      return -1;
    }
    value = *static_cast<const int32_t *>(args[n + j]);
  } else {
    value = strtol(*text, &end, 10);
  }
  *text = end;
  if (**text == ',') {
    ++*text;
  }
  return value;
}

/* `launch=`: the trip count (0 when absent, -1 when malformed); a `B,T`
 * entry also gives the block size in `*threads` (else 0). */
inline long image_launch_trip(const void *payload, size_t size,
                              void *const *args, const int32_t *tags,
                              int64_t n, long *threads) {
  const char *at = vx_payload_field(payload, size, "launch=");
  *threads = 0;
  if (!at) {
    return 0;
  }
  const long trip = image_launch_size(&at, args, tags, n);
  if (trip >= 0 && *at) {
    *threads = image_launch_size(&at, args, tags, n);
  }
  return trip;
}

/* `grid=` + `block=`: 1 with the shape filled in, 0 when the payload names
 * none, -1 (reason in `why`) for a size no GPU launches; with `grid_loops=`
 * the blocks loop over the grid, so out-of-range grid sizes are clamped. */
inline int image_launch_shape(const void *payload, size_t size,
                              void *const *args, const int32_t *tags,
                              int64_t n, unsigned grid[3], unsigned *block,
                              char *why, size_t why_size) {
  static const long kLimits[3] = {2147483647L, 65535L, 65535L};
  const char *at = vx_payload_field(payload, size, "grid=");
  const char *block_text = vx_payload_field(payload, size, "block=");
  if (!at || !block_text) {
    return 0;
  }
  const bool loops = vx_payload_field(payload, size, "grid_loops=") != nullptr;
  for (int axis = 0; axis < 3; ++axis) {
    long v = *at ? image_launch_size(&at, args, tags, n) : 1;
    if (loops) {
      v = v < 1 ? 1 : v > kLimits[axis] ? kLimits[axis] : v;
    } else if (v < 1 || v > kLimits[axis]) {
      snprintf(why, why_size,
               "grid axis %d has %ld blocks, and a GPU launches 1 to %ld on "
               "that axis",
               axis, v, kLimits[axis]);
      return -1;
    }
    grid[axis] = (unsigned)v;
  }
  const long threads = image_launch_size(&block_text, args, tags, n);
  if (threads < 1 || threads > 1024) {
    snprintf(why, why_size,
             "a block of %ld threads, and a block holds 1 to 1024 threads",
             threads);
    return -1;
  }
  *block = (unsigned)threads;
  return 1;
}

/* The launch of a dispatch: the payload's shape, else its trip count (one
 * iteration per thread up to blocks of 128, at most 4096 blocks, which a
 * grid-strided loop absorbs), else one thread. False with `why` set for a
 * shape no GPU launches. */
inline bool image_launch_geometry(const void *payload, size_t size,
                                  void *const *args, const int32_t *tags,
                                  int64_t n, unsigned grid[3],
                                  unsigned *block, char *why,
                                  size_t why_size) {
  grid[0] = grid[1] = grid[2] = 1;
  *block = 1;
  const int set = image_launch_shape(payload, size, args, tags, n, grid, block,
                                     why, why_size);
  if (set < 0) {
    return false;
  }
  if (set > 0) {
    return true;
  }
  long threads = 0;
  const long trip = image_launch_trip(payload, size, args, tags, n, &threads);
  if (trip < 0 || threads < 0) {
    snprintf(why, why_size, "`launch=` names a launch value that is not an i32");
    return false;
  }
  if (threads != 0) {
    if (trip > 0 && threads > 0) {
      grid[0] = trip > 4096 ? 4096u : (unsigned)trip;
      *block = threads > 1024 ? 1024u : (unsigned)threads;
    }
  } else if (trip > 1) {
    *block = trip < 128 ? (unsigned)trip : 128u;
    const unsigned long need = ((unsigned long)trip + *block - 1) / *block;
    grid[0] = need > 4096 ? 4096u : (unsigned)need;
  }
  return true;
}

/* ---- code object metadata ---- */

/* A bounds-checked MessagePack reader over [p, e). Any read past the end
 * clears `ok`, and every later read fails. */
struct MsgPack {
  const uint8_t *p;
  const uint8_t *e;
  bool ok = true;

  bool has(size_t k) {
    if (!ok || (size_t)(e - p) < k) {
      ok = false;
    }
    return ok;
  }
  uint64_t big_endian(int k) {
    uint64_t v = 0;
    if (!has((size_t)k)) {
      return 0;
    }
    for (int i = 0; i < k; ++i) {
      v = (v << 8) | p[i];
    }
    p += k;
    return v;
  }
  bool container(uint8_t fix_hi, uint8_t c16, uint8_t c32, uint32_t &n) {
    if (!has(1)) {
      return false;
    }
    const uint8_t c = *p;
    if ((c & 0xf0) == fix_hi) {
      n = c & 15;
      ++p;
      return true;
    }
    if (c == c16 || c == c32) {
      ++p;
      n = (uint32_t)big_endian(c == c16 ? 2 : 4);
      return ok;
    }
    return false;
  }
  bool map(uint32_t &n) { return container(0x80, 0xde, 0xdf, n); }
  bool array(uint32_t &n) { return container(0x90, 0xdc, 0xdd, n); }
  bool str(const char *&s, uint32_t &n) {
    if (!has(1)) {
      return false;
    }
    const uint8_t c = *p;
    if ((c & 0xe0) == 0xa0) {
      n = c & 31;
      ++p;
    } else if (c >= 0xd9 && c <= 0xdb) {
      ++p;
      n = (uint32_t)big_endian(c == 0xd9 ? 1 : c == 0xda ? 2 : 4);
    } else {
      return false;
    }
    if (!has(n)) {
      return false;
    }
    s = reinterpret_cast<const char *>(p);
    p += n;
    return true;
  }
  bool skip_bytes(uint64_t n) {
    if (!has((size_t)n)) {
      return false;
    }
    p += n;
    return true;
  }
  /* Step over one value of any type. */
  bool skip(int depth = 0) {
    if (depth > 32 || !has(1)) {
      return ok = false;
    }
    const uint8_t c = *p;
    uint32_t n = 0;
    if (c <= 0x7f || c >= 0xe0 || c == 0xc0 || c == 0xc2 || c == 0xc3) {
      ++p;
      return true;
    }
    if (map(n)) {
      for (uint64_t i = 0; i < 2ull * n; ++i) {
        if (!skip(depth + 1)) {
          return false;
        }
      }
      return true;
    }
    if (array(n)) {
      for (uint32_t i = 0; i < n; ++i) {
        if (!skip(depth + 1)) {
          return false;
        }
      }
      return true;
    }
    const char *s;
    if (str(s, n)) {
      return true;
    }
    ++p;
    switch (c) {
    case 0xc4: case 0xc5: case 0xc6: /* bin 8/16/32 */
      return skip_bytes(big_endian(c == 0xc4 ? 1 : c == 0xc5 ? 2 : 4));
    case 0xc7: case 0xc8: case 0xc9: { /* ext 8/16/32: length, type, data */
      const uint64_t len = big_endian(c == 0xc7 ? 1 : c == 0xc8 ? 2 : 4);
      return skip_bytes(len + 1);
    }
    case 0xca: return skip_bytes(4);
    case 0xcb: return skip_bytes(8);
    case 0xcc: case 0xd0: return skip_bytes(1);
    case 0xcd: case 0xd1: return skip_bytes(2);
    case 0xce: case 0xd2: return skip_bytes(4);
    case 0xcf: case 0xd3: return skip_bytes(8);
    case 0xd4: return skip_bytes(2); /* fixext 1: type + 1 */
    case 0xd5: return skip_bytes(3);
    case 0xd6: return skip_bytes(5);
    case 0xd7: return skip_bytes(9);
    case 0xd8: return skip_bytes(17);
    default: return ok = false;
    }
  }
};

inline bool key_is(const char *s, uint32_t n, const char *want) {
  return strlen(want) == n && memcmp(s, want, n) == 0;
}

/* The code object for `arch` inside `image`: the image itself when it is an
 * ELF, or the matching entry of an (uncompressed) clang offload bundle. */
inline bool code_object_elf(const void *image, size_t size, const char *arch,
                            const uint8_t **elf, size_t *elf_size) {
  const uint8_t *b = static_cast<const uint8_t *>(image);
  if (size >= 4 && memcmp(b, "\x7f" "ELF", 4) == 0) {
    *elf = b;
    *elf_size = size;
    return true;
  }
  static const char kMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
  if (size < 32 || memcmp(b, kMagic, 24) != 0) {
    return false;
  }
  auto u64 = [&](size_t at) {
    uint64_t v;
    memcpy(&v, b + at, 8);
    return v;
  };
  const uint64_t entries = u64(24);
  size_t at = 32;
  for (uint64_t i = 0; i < entries; ++i) {
    if (at + 24 > size) {
      return false;
    }
    const uint64_t off = u64(at), len = u64(at + 8), tlen = u64(at + 16);
    at += 24;
    if (tlen > size - at) {
      return false;
    }
    const char *triple = reinterpret_cast<const char *>(b + at);
    at += tlen;
    const size_t alen = strlen(arch);
    bool match = false;
    for (uint64_t k = 0; k + alen <= tlen; ++k) {
      if (memcmp(triple + k, arch, alen) == 0 &&
          (k + alen == tlen || triple[k + alen] == ':')) {
        match = true;
        break;
      }
    }
    if (match && off <= size && len <= size - off && len >= 4 &&
        memcmp(b + off, "\x7f" "ELF", 4) == 0) {
      *elf = b + off;
      *elf_size = len;
      return true;
    }
  }
  return false;
}

/* The AMDGPU metadata note (owner "AMDGPU", type 32) of an ELF64 code
 * object. */
inline bool code_object_metadata(const uint8_t *elf, size_t size,
                                 const uint8_t **meta, size_t *meta_size) {
  if (size < 64 || elf[4] != 2 /* ELFCLASS64 */ || elf[5] != 1 /* LE */) {
    return false;
  }
  uint64_t shoff;
  uint16_t shentsize, shnum;
  memcpy(&shoff, elf + 0x28, 8);
  memcpy(&shentsize, elf + 0x3a, 2);
  memcpy(&shnum, elf + 0x3c, 2);
  if (shentsize < 64 || shoff > size || (uint64_t)shnum * shentsize > size - shoff) {
    return false;
  }
  for (uint16_t s = 0; s < shnum; ++s) {
    const uint8_t *sh = elf + shoff + (size_t)s * shentsize;
    uint32_t type;
    uint64_t off, len;
    memcpy(&type, sh + 4, 4);
    memcpy(&off, sh + 0x18, 8);
    memcpy(&len, sh + 0x20, 8);
    if (type != 7 /* SHT_NOTE */ || off > size || len > size - off) {
      continue;
    }
    size_t at = 0;
    while (at + 12 <= len) {
      uint32_t namesz, descsz, ntype;
      memcpy(&namesz, elf + off + at, 4);
      memcpy(&descsz, elf + off + at + 4, 4);
      memcpy(&ntype, elf + off + at + 8, 4);
      const size_t name_at = at + 12;
      const size_t desc_at = name_at + ((namesz + 3u) & ~3u);
      if (desc_at > len || descsz > len - desc_at) {
        break;
      }
      if (ntype == 32 && namesz == 7 &&
          memcmp(elf + off + name_at, "AMDGPU", 7) == 0) {
        *meta = elf + off + desc_at;
        *meta_size = descsz;
        return true;
      }
      at = desc_at + ((descsz + 3u) & ~3u);
    }
  }
  return false;
}

/* How many of its own (non-hidden) parameters kernel `name` declares in the
 * code object for `arch`; -1 when the image, its metadata or the kernel is
 * not there, so "absent" and "takes none" stay distinct. */
inline int code_object_param_count(const void *image, size_t size,
                                   const char *arch, const char *name) {
  const uint8_t *elf, *meta;
  size_t elf_size, meta_size;
  if (!image || !name || !code_object_elf(image, size, arch, &elf, &elf_size) ||
      !code_object_metadata(elf, elf_size, &meta, &meta_size)) {
    return -1;
  }
  MsgPack m{meta, meta + meta_size};
  uint32_t root = 0;
  if (!m.map(root)) {
    return -1;
  }
  for (uint32_t r = 0; r < root; ++r) {
    const char *k;
    uint32_t kn, kernels;
    if (!m.str(k, kn)) {
      return -1;
    }
    if (!key_is(k, kn, "amdhsa.kernels")) {
      if (!m.skip()) {
        return -1;
      }
      continue;
    }
    if (!m.array(kernels)) {
      return -1;
    }
    for (uint32_t i = 0; i < kernels; ++i) {
      uint32_t fields;
      if (!m.map(fields)) {
        return -1;
      }
      bool named = false;
      int own = -1;
      for (uint32_t f = 0; f < fields; ++f) {
        const char *fk;
        uint32_t fkn;
        if (!m.str(fk, fkn)) {
          return -1;
        }
        if (key_is(fk, fkn, ".name")) {
          const char *v;
          uint32_t vn;
          if (!m.str(v, vn)) {
            return -1;
          }
          named = key_is(v, vn, name);
        } else if (key_is(fk, fkn, ".args")) {
          uint32_t args;
          if (!m.array(args)) {
            return -1;
          }
          own = 0;
          for (uint32_t a = 0; a < args; ++a) {
            uint32_t afields;
            if (!m.map(afields)) {
              return -1;
            }
            bool hidden = false;
            for (uint32_t q = 0; q < afields; ++q) {
              const char *ak;
              uint32_t akn;
              if (!m.str(ak, akn)) {
                return -1;
              }
              if (key_is(ak, akn, ".value_kind")) {
                const char *v;
                uint32_t vn;
                if (!m.str(v, vn)) {
                  return -1;
                }
                hidden = vn >= 7 && memcmp(v, "hidden_", 7) == 0;
              } else if (!m.skip()) {
                return -1;
              }
            }
            own += hidden ? 0 : 1;
          }
        } else if (!m.skip()) {
          return -1;
        }
      }
      if (named) {
        return own < 0 ? 0 : own;
      }
    }
    return -1;
  }
  return -1;
}

} // namespace vx
