/*
 * llama_io.cpp -- model files for the int8 decode path (host side).
 *
 * Reads the llama2.c checkpoint the reference's examples/llama.vx loads
 * (header of reference stdlib/rust_core/src/ffi/llama.rs:10-45, array order
 * of examples/llama.vx:80-120), quantizing each matrix per output row, and
 * reads and writes this build's own int8 file so that quantization happens
 * once. Nothing here touches the GPU.
 */
#include "../../include/vx_hip_ops.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

struct vx_llama_i8_host {
  vx_llama_i8_config cfg{};
  std::vector<int8_t> tok_q, wq_q, wk_q, wv_q, wo_q, w1_q, w2_q, w3_q;
  std::vector<float> tok_s, wq_s, wk_s, wv_s, wo_s, w1_s, w2_s, w3_s;
  std::vector<float> rms_att, rms_ffn, rms_final, rope;
  vx_llama_i8_weights w{};
};

namespace {

constexpr char kMagic[4] = {'V', 'X', 'Q', '8'};
constexpr uint32_t kVersion = 1;

int32_t fail(int32_t code, const std::string &why) {
  fprintf(stderr, "[Vx HIP] vx_llama_i8 file: %s\n", why.c_str());
  return code;
}

bool read_file(const char *path, std::vector<unsigned char> &bytes) {
  FILE *f = fopen(path, "rb");
  if (!f) {
    return false;
  }
  bool ok = fseek(f, 0, SEEK_END) == 0;
  const long n = ok ? ftell(f) : -1;
  ok = ok && n >= 0 && fseek(f, 0, SEEK_SET) == 0;
  if (ok) {
    bytes.resize((size_t)n);
    ok = n == 0 || fread(bytes.data(), 1, (size_t)n, f) == (size_t)n;
  }
  fclose(f);
  return ok;
}

uint64_t fnv1a(const unsigned char *p, size_t n) {
  uint64_t h = 1469598103934665603ull;
  for (size_t i = 0; i < n; ++i) {
    h = (h ^ p[i]) * 1099511628211ull;
  }
  return h;
}

/* Extents the kernels and the file layouts assume; false for nonsense. */
bool config_ok(const vx_llama_i8_config &c) {
  return c.dim > 0 && c.hidden_dim > 0 && c.n_layers > 0 && c.n_heads > 0 &&
         c.n_kv_heads > 0 && c.vocab_size > 0 && c.seq_len > 0 &&
         c.dim % c.n_heads == 0 && c.n_heads % c.n_kv_heads == 0 &&
         (c.dim / c.n_heads) % 2 == 0 && c.dim <= (1 << 16) &&
         c.hidden_dim <= (1 << 18) && c.n_layers <= 4096 &&
         c.vocab_size <= (1 << 22) && c.seq_len <= (1 << 20);
}

/* Per-row symmetric int8 (the same arithmetic as the CPU checker's
 * quantizer): scale = max|w| / 127 (1 for a zero row), q = nearest, ties to
 * even, clamped to [-127, 127]. */
void quantize_rows(const float *w, int64_t rows, int64_t cols, int8_t *q,
                   float *scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *wr = w + r * cols;
    float amax = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      const float a = fabsf(wr[c]);
      if (a > amax) {
        amax = a;
      }
    }
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    scale[r] = s;
    for (int64_t c = 0; c < cols; ++c) {
      float t = nearbyintf(wr[c] / s);
      t = t > 127.0f ? 127.0f : t < -127.0f ? -127.0f : t;
      q[r * cols + c] = (int8_t)t;
    }
  }
}

/* [seq_len, hs / 2, 2] of (cos, sin) of the f32 angle (pos as f32) *
 * 10000^(-(i as f32) / (hs as f32)), even i, as reference
 * tests/modules/llama_rt.vx:82-85 and examples/llama.vx:244-246 compute it
 * with f32 powf, cos and sin, which reference stdlib/core/num.vx:2434-2479
 * documents as correctly rounded. Each is evaluated in double (glibc, under
 * 1 ulp of double) and rounded to f32 once. */
void rope_table(const vx_llama_i8_config &c, std::vector<float> &out) {
  const int hs = c.dim / c.n_heads;
  out.resize((size_t)c.seq_len * (hs / 2) * 2);
  std::vector<float> inv(hs / 2);
  for (int i = 0; i < hs; i += 2) {
    const float e = -(float)i / (float)hs;
    inv[i / 2] = (float)pow(10000.0, (double)e);
  }
  for (int p = 0; p < c.seq_len; ++p) {
    for (int j = 0; j < hs / 2; ++j) {
      const float ang = (float)p * inv[j];
      out[((size_t)p * (hs / 2) + j) * 2] = (float)cos((double)ang);
      out[((size_t)p * (hs / 2) + j) * 2 + 1] = (float)sin((double)ang);
    }
  }
}

void bind(vx_llama_i8_host &h) {
  vx_llama_i8_weights &w = h.w;
  w.tok_q = h.tok_q.data();
  w.tok_s = h.tok_s.data();
  w.rms_att = h.rms_att.data();
  w.wq_q = h.wq_q.data();
  w.wq_s = h.wq_s.data();
  w.wk_q = h.wk_q.data();
  w.wk_s = h.wk_s.data();
  w.wv_q = h.wv_q.data();
  w.wv_s = h.wv_s.data();
  w.wo_q = h.wo_q.data();
  w.wo_s = h.wo_s.data();
  w.rms_ffn = h.rms_ffn.data();
  w.w1_q = h.w1_q.data();
  w.w1_s = h.w1_s.data();
  w.w2_q = h.w2_q.data();
  w.w2_s = h.w2_s.data();
  w.w3_q = h.w3_q.data();
  w.w3_s = h.w3_s.data();
  w.rms_final = h.rms_final.data();
  w.rope = h.rope.data();
}

/* One matrix family per layer: rows x cols per layer. */
struct Mat {
  int8_t *q;
  float *s;
  int64_t rows, cols;
};

/* The stored arrays in vx_llama_i8_weights field order (the RoPE table is
 * not stored: it is recomputed from the config), each with its byte count,
 * for the VXQ8 payload (both directions). */
struct Field {
  void *data;
  size_t bytes;
};

std::vector<Field> fields(vx_llama_i8_host &h) {
  auto f = [](auto &v) {
    return Field{v.data(), v.size() * sizeof(v[0])};
  };
  return {f(h.tok_q),   f(h.tok_s), f(h.rms_att), f(h.wq_q),   f(h.wq_s),
          f(h.wk_q),    f(h.wk_s),  f(h.wv_q),    f(h.wv_s),   f(h.wo_q),
          f(h.wo_s),    f(h.rms_ffn), f(h.w1_q),  f(h.w1_s),   f(h.w2_q),
          f(h.w2_s),    f(h.w3_q),  f(h.w3_s),    f(h.rms_final)};
}

void size_all(vx_llama_i8_host &h) {
  const vx_llama_i8_config &c = h.cfg;
  const int64_t d = c.dim, hd = c.hidden_dim, L = c.n_layers;
  const int64_t kv = d * c.n_kv_heads / c.n_heads;
  h.tok_q.resize(c.vocab_size * d);
  h.tok_s.resize(c.vocab_size);
  h.rms_att.resize(L * d);
  h.wq_q.resize(L * d * d);
  h.wq_s.resize(L * d);
  h.wk_q.resize(L * kv * d);
  h.wk_s.resize(L * kv);
  h.wv_q.resize(L * kv * d);
  h.wv_s.resize(L * kv);
  h.wo_q.resize(L * d * d);
  h.wo_s.resize(L * d);
  h.rms_ffn.resize(L * d);
  h.w1_q.resize(L * hd * d);
  h.w1_s.resize(L * hd);
  h.w2_q.resize(L * d * hd);
  h.w2_s.resize(L * d);
  h.w3_q.resize(L * hd * d);
  h.w3_s.resize(L * hd);
  h.rms_final.resize(d);
}

int32_t read_checkpoint(const std::vector<unsigned char> &b,
                        vx_llama_i8_host &h) {
  int32_t hdr[7];
  memcpy(hdr, b.data(), sizeof hdr);
  vx_llama_i8_config c{hdr[0], hdr[1], hdr[2], hdr[3], hdr[4], hdr[5], hdr[6]};
  if (c.vocab_size < 0) {
    return fail(VX_OP_EUNSUPP,
                "checkpoint has an unshared classifier (negative vocab_size); "
                "the decode path uses the token table as the classifier");
  }
  if (!config_ok(c)) {
    return fail(VX_OP_EINVAL, "checkpoint header is not a usable config");
  }
  h.cfg = c;
  const int64_t d = c.dim, hd = c.hidden_dim, L = c.n_layers;
  const int64_t kv = d * c.n_kv_heads / c.n_heads, hs = d / c.n_heads;
  /* f32 counts in file order (examples/llama.vx:80-120). */
  const int64_t counts[] = {c.vocab_size * d, L * d,      L * d * d,
                            L * kv * d,       L * kv * d, L * d * d,
                            L * d,            L * hd * d, L * d * hd,
                            L * hd * d,       d};
  int64_t floats = 0;
  for (int64_t n : counts) {
    floats += n;
  }
  const int64_t rope_floats = (int64_t)c.seq_len * hs; /* real + imag */
  const size_t base = 28 + (size_t)floats * 4;
  if (b.size() != base && b.size() != base + (size_t)rope_floats * 4) {
    return fail(VX_OP_EINVAL,
                "checkpoint size " + std::to_string(b.size()) +
                    " does not match its header (expected " +
                    std::to_string(base) + " or " +
                    std::to_string(base + (size_t)rope_floats * 4) + " bytes)");
  }
  size_all(h);
  /* The f32 payload may sit unaligned; copy each array out. */
  size_t at = 28;
  std::vector<float> tmp;
  auto next = [&](int64_t n) -> const float * {
    tmp.resize((size_t)n);
    memcpy(tmp.data(), b.data() + at, (size_t)n * 4);
    at += (size_t)n * 4;
    return tmp.data();
  };
  quantize_rows(next(counts[0]), c.vocab_size, d, h.tok_q.data(),
                h.tok_s.data());
  memcpy(h.rms_att.data(), next(counts[1]), (size_t)counts[1] * 4);
  const Mat mats[] = {{h.wq_q.data(), h.wq_s.data(), d, d},
                      {h.wk_q.data(), h.wk_s.data(), kv, d},
                      {h.wv_q.data(), h.wv_s.data(), kv, d},
                      {h.wo_q.data(), h.wo_s.data(), d, d}};
  for (const Mat &m : mats) {
    quantize_rows(next(L * m.rows * m.cols), L * m.rows, m.cols, m.q, m.s);
  }
  memcpy(h.rms_ffn.data(), next(counts[6]), (size_t)counts[6] * 4);
  const Mat ffn[] = {{h.w1_q.data(), h.w1_s.data(), hd, d},
                     {h.w2_q.data(), h.w2_s.data(), d, hd},
                     {h.w3_q.data(), h.w3_s.data(), hd, d}};
  for (const Mat &m : ffn) {
    quantize_rows(next(L * m.rows * m.cols), L * m.rows, m.cols, m.q, m.s);
  }
  memcpy(h.rms_final.data(), next(counts[10]), (size_t)counts[10] * 4);
  rope_table(c, h.rope);
  return VX_OP_OK;
}

int32_t read_q8(const std::vector<unsigned char> &b, vx_llama_i8_host &h) {
  uint32_t version;
  memcpy(&version, b.data() + 4, 4);
  if (version != kVersion) {
    return fail(VX_OP_EUNSUPP,
                "VXQ8 file version " + std::to_string(version) + " (this build reads 1)");
  }
  if (b.size() < 8 + 28 + 8) {
    return fail(VX_OP_EINVAL, "VXQ8 file is truncated");
  }
  int32_t hdr[7];
  memcpy(hdr, b.data() + 8, sizeof hdr);
  vx_llama_i8_config c{hdr[0], hdr[1], hdr[2], hdr[3], hdr[4], hdr[5], hdr[6]};
  if (!config_ok(c)) {
    return fail(VX_OP_EINVAL, "VXQ8 header is not a usable config");
  }
  /* The payload's size follows from the header alone; it is compared with
   * the file before anything is allocated, so a corrupt header cannot ask
   * for more memory than the file holds. Every count fits in int64 within
   * config_ok's limits. */
  const int64_t d = c.dim, hd = c.hidden_dim, L = c.n_layers;
  const int64_t kv = d * c.n_kv_heads / c.n_heads;
  const int64_t rows = (int64_t)c.vocab_size + L * (3 * d + 2 * kv + 2 * hd);
  const int64_t int8s = (int64_t)c.vocab_size * d + L * (2 * d * d + 2 * kv * d + 3 * hd * d);
  const int64_t norms = L * 2 * d + d;
  const uint64_t payload = (uint64_t)int8s + 4 * (uint64_t)(rows + norms);
  const uint64_t body = 8 + 28 + payload;
  if ((uint64_t)b.size() != body + 8) {
    return fail(VX_OP_EINVAL, "VXQ8 file size " + std::to_string(b.size()) +
                                  " does not match its header (expected " +
                                  std::to_string(body + 8) + ")");
  }
  h.cfg = c;
  size_all(h);
  rope_table(c, h.rope);
  uint64_t want;
  memcpy(&want, b.data() + body, 8);
  if (fnv1a(b.data(), body) != want) {
    return fail(VX_OP_EINVAL, "VXQ8 checksum mismatch (corrupt file)");
  }
  size_t at = 8 + 28;
  for (const Field &f : fields(h)) {
    memcpy(f.data, b.data() + at, f.bytes);
    at += f.bytes;
  }
  return VX_OP_OK;
}

} // namespace

extern "C" {

int32_t vx_llama_i8_read(const char *path, vx_llama_i8_config *cfg,
                         vx_llama_i8_host **out) {
  if (!path || !cfg || !out) {
    return fail(VX_OP_EINVAL, "path, cfg and out must not be NULL");
  }
  *out = nullptr;
  std::vector<unsigned char> bytes;
  if (!read_file(path, bytes)) {
    return fail(VX_OP_EINVAL, std::string("cannot read ") + path);
  }
  if (bytes.size() < 28) {
    return fail(VX_OP_EINVAL, std::string(path) + " is too short for a model");
  }
  vx_llama_i8_host *h = new (std::nothrow) vx_llama_i8_host();
  if (!h) {
    return fail(VX_OP_ENOMEM, "out of host memory for a model");
  }
  int32_t rc;
  try {
    rc = memcmp(bytes.data(), kMagic, 4) == 0 ? read_q8(bytes, *h)
                                              : read_checkpoint(bytes, *h);
  } catch (const std::bad_alloc &) {
    /* No exception may cross the C boundary. */
    rc = fail(VX_OP_ENOMEM, std::string("out of host memory reading ") + path);
  }
  if (rc != VX_OP_OK) {
    delete h;
    return rc;
  }
  bind(*h);
  *cfg = h->cfg;
  *out = h;
  return VX_OP_OK;
}

const vx_llama_i8_weights *vx_llama_i8_host_weights(const vx_llama_i8_host *h) {
  return h ? &h->w : nullptr;
}

void vx_llama_i8_host_free(vx_llama_i8_host *h) { delete h; }

int32_t vx_llama_i8_save(const char *path, const vx_llama_i8_config *cfg,
                         const vx_llama_i8_weights *w) {
  if (!path || !cfg || !w) {
    return fail(VX_OP_EINVAL, "path, cfg and weights must not be NULL");
  }
  if (!config_ok(*cfg)) {
    return fail(VX_OP_EINVAL, "config is not one a model file can hold");
  }
  /* Copy into a host image so the field list (and its sizes) is the one the
   * reader uses. */
  vx_llama_i8_host h;
  h.cfg = *cfg;
  size_all(h);
  const void *src[] = {w->tok_q, w->tok_s, w->rms_att, w->wq_q,    w->wq_s,
                       w->wk_q,  w->wk_s,  w->wv_q,    w->wv_s,    w->wo_q,
                       w->wo_s,  w->rms_ffn, w->w1_q,  w->w1_s,    w->w2_q,
                       w->w2_s,  w->w3_q,  w->w3_s,    w->rms_final};
  const std::vector<Field> fs = fields(h);
  std::vector<unsigned char> out(8 + 28);
  memcpy(out.data(), kMagic, 4);
  memcpy(out.data() + 4, &kVersion, 4);
  const int32_t hdr[7] = {cfg->dim,        cfg->hidden_dim, cfg->n_layers,
                          cfg->n_heads,    cfg->n_kv_heads, cfg->vocab_size,
                          cfg->seq_len};
  memcpy(out.data() + 8, hdr, sizeof hdr);
  for (size_t i = 0; i < fs.size(); ++i) {
    if (!src[i]) {
      return fail(VX_OP_EINVAL, "a weight array is NULL");
    }
    const unsigned char *p = static_cast<const unsigned char *>(src[i]);
    out.insert(out.end(), p, p + fs[i].bytes);
  }
  const uint64_t sum = fnv1a(out.data(), out.size());
  const unsigned char *sp = reinterpret_cast<const unsigned char *>(&sum);
  out.insert(out.end(), sp, sp + 8);
  FILE *f = fopen(path, "wb");
  if (!f) {
    return fail(VX_OP_EINVAL, std::string("cannot write ") + path);
  }
  const bool ok = fwrite(out.data(), 1, out.size(), f) == out.size();
  const bool closed = fclose(f) == 0;
  if (!ok || !closed) {
    return fail(VX_OP_EINVAL, std::string("short write to ") + path);
  }
  return VX_OP_OK;
}

} // extern "C"
