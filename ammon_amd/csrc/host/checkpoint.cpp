// checkpoint.cpp -- llama2.c checkpoints (legacy run.c layout and the
// version-1 "ak42" export) streamed into device memory.  The layouts are
// described in include/ammon/ammon_checkpoint.h.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>

#include "../runtime/internal.h"
#include "ammon/ammon.hpp"
#include "ammon/ammon_checkpoint.h"

namespace {

constexpr uint32_t kMagic = 0x616b3432u;  // "ak42"
constexpr size_t kStage = 8u << 20;        // floats per staging half (32 MiB)

struct Header {
  ammon_llama_config cfg{};
  uint32_t format = AMMON_CHECKPOINT_LEGACY;
  bool shared = true;
  uint64_t data_offset = 0;  // bytes before the first weight
  uint64_t expected = 0;     // file size the shape implies
};

struct File {
  FILE *f = nullptr;
  explicit File(const char *path) : f(std::fopen(path, "rb")) {}
  ~File() {
    if (f) std::fclose(f);
  }
};

uint16_t f32_to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

Header read_header(const char *path) {
  File file(path);
  if (!file.f) throw ammon::Error(AMMON_E_VALIDATION, std::string("checkpoint: cannot open ") + path);
  int32_t h[9];
  Header hd;
  if (std::fread(h, 4, 2, file.f) != 2)
    throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: file too short for a header");
  int32_t p[7];
  if ((uint32_t)h[0] == kMagic) {
    if (h[1] != 1)
      throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: unsupported export version " +
                                                 std::to_string(h[1]) + " (fp32 version 1 only)");
    uint8_t shared = 0;
    if (std::fread(p, 4, 7, file.f) != 7 || std::fread(&shared, 1, 1, file.f) != 1)
      throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: truncated version-1 header");
    hd.format = AMMON_CHECKPOINT_V1;
    hd.shared = shared != 0;
    hd.data_offset = 256;
  } else {
    p[0] = h[0];
    p[1] = h[1];
    if (std::fread(p + 2, 4, 5, file.f) != 5)
      throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: truncated header");
    hd.format = AMMON_CHECKPOINT_LEGACY;
    hd.shared = p[5] > 0;
    if (p[5] < 0) p[5] = -p[5];
    hd.data_offset = 28;
  }
  for (int i = 0; i < 7; ++i)
    if (p[i] <= 0)
      throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: header field " + std::to_string(i) +
                                                 " is " + std::to_string(p[i]) + ", not positive");
  const uint32_t dim = (uint32_t)p[0], hidden = (uint32_t)p[1], L = (uint32_t)p[2];
  const uint32_t heads = (uint32_t)p[3], kv = (uint32_t)p[4];
  if (dim % heads || heads % kv)
    throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: dim " + std::to_string(dim) +
                                               ", heads " + std::to_string(heads) + ", kv heads " +
                                               std::to_string(kv) + " do not divide");
  ammon_llama_config &c = hd.cfg;
  c.dim = dim;
  c.hidden = hidden;
  c.n_layers = L;
  c.n_heads = heads;
  c.n_kv_heads = kv;
  c.vocab = (uint32_t)p[5];
  c.max_seq = (uint32_t)p[6];
  c.theta = 10000.0f;
  c.eps = 1e-5f;
  c.w_dtype = AMMON_F32;
  c.kv_dtype = AMMON_F32;
  c.use_graph = 1;
  // all size arithmetic in 64 bits: dim * dim alone overflows 32 bits for
  // dim >= 65536
  const uint64_t D = dim, head = D / heads, kvd = head * kv;
  uint64_t floats = (uint64_t)c.vocab * D + 2ull * L * D + D +
                    (uint64_t)L * (D * D + 2 * kvd * D + D * D + 3ull * hidden * D);
  if (hd.format == AMMON_CHECKPOINT_LEGACY) floats += (uint64_t)c.max_seq * head;  // RoPE tables
  if (!hd.shared) floats += (uint64_t)c.vocab * dim;
  hd.expected = hd.data_offset + floats * 4;
  return hd;
}

}  // namespace

struct ammon_checkpoint {
  ammon::Runtime rt;
  Header hd;
  ammon_dtype w_dtype = AMMON_F32;
  std::vector<ammon::Tensor> bufs;
  ammon_llama_weights w{};
};

namespace {

// Two pinned staging halves: the file is read into one while the other's
// asynchronous upload runs; a half is refilled only after its event says
// its previous upload finished.
struct Stager {
  ammon_runtime *rt = nullptr;
  float *half[2] = {nullptr, nullptr};
  ammon_event done[2] = {nullptr, nullptr};
  bool pending[2] = {false, false};
  int next = 0;

  explicit Stager(ammon_runtime *r) : rt(r) {
    for (int i = 0; i < 2; ++i) {
      ammon::check(ammon_alloc_host(rt, kStage * 4, (void **)&half[i]), "checkpoint staging");
      ammon::check(ammon_event_create(rt, &done[i]), "checkpoint staging");
    }
  }
  ~Stager() {
    for (int i = 0; i < 2; ++i) {
      if (pending[i]) ammon_event_synchronize(rt, done[i]);
      if (done[i]) ammon_event_destroy(rt, done[i]);
      if (half[i]) ammon_free_host(rt, half[i]);
    }
  }

  // Reads `n` floats at the file's position into device buffer `dst`,
  // converted to bf16 when `bf16`.
  void stream(FILE *f, void *dst, uint64_t n, bool bf16, const char *what) {
    uint64_t at = 0;
    while (at < n) {
      const int h = next;
      next ^= 1;
      if (pending[h]) ammon::check(ammon_event_synchronize(rt, done[h]), "checkpoint upload");
      float *stage = half[h];
      const size_t k = (size_t)std::min<uint64_t>(kStage, n - at);
      if (std::fread(stage, 4, k, f) != k)
        throw ammon::Error(AMMON_E_VALIDATION, std::string("checkpoint: file ends inside ") + what);
      size_t bytes = k * 4;
      if (bf16) {
        uint16_t *o = (uint16_t *)stage;  // in place: output i never passes input i
        for (size_t i = 0; i < k; ++i) o[i] = f32_to_bf16(stage[i]);
        bytes = k * 2;
      }
      char *d = (char *)dst + at * (bf16 ? 2 : 4);
      ammon::check(ammon_memcpy(rt, d, stage, bytes, AMMON_COPY_H2D, nullptr), "checkpoint upload");
      ammon::check(ammon_event_record(rt, done[h], nullptr), "checkpoint upload");
      pending[h] = true;
      at += k;
    }
  }
};

void skip(FILE *f, uint64_t bytes) {
  if (std::fseek(f, (long)bytes, SEEK_CUR) != 0)
    throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: file ends inside the RoPE tables");
}

}  // namespace

extern "C" {

ammon_status ammon_checkpoint_probe(const char *path, ammon_llama_config *cfg, uint32_t *format,
                                    uint32_t *shared_classifier, uint64_t *expected_bytes) {
  AMMON_CHECK(path && cfg, "checkpoint_probe: NULL argument");
  try {
    const Header hd = read_header(path);
    *cfg = hd.cfg;
    if (format) *format = hd.format;
    if (shared_classifier) *shared_classifier = hd.shared ? 1u : 0u;
    if (expected_bytes) *expected_bytes = hd.expected;
    return AMMON_OK;
  } catch (const ammon::Error &e) {
    return ammon_rt::set_error(e.status(), "%s", e.what());
  }
}

ammon_status ammon_checkpoint_load(ammon_runtime *rt, const char *path, ammon_dtype w_dtype,
                                   ammon_checkpoint **out) {
  AMMON_CHECK(rt && path && out, "checkpoint_load: NULL argument");
  AMMON_CHECK(w_dtype == AMMON_F32 || w_dtype == AMMON_BF16, "checkpoint_load: unknown dtype %d",
              (int)w_dtype);
  ammon_checkpoint *c = new ammon_checkpoint();
  try {
    c->rt = ammon::Runtime::create(rt->device);
    c->hd = read_header(path);
    c->w_dtype = w_dtype;
    File file(path);
    if (!file.f) throw ammon::Error(AMMON_E_VALIDATION, std::string("checkpoint: cannot open ") + path);
    std::fseek(file.f, 0, SEEK_END);
    const long size = std::ftell(file.f);
    if (size < 0 || (uint64_t)size != c->hd.expected)
      throw ammon::Error(AMMON_E_VALIDATION,
                         "checkpoint: file is " + std::to_string(size) + " bytes, the header's shape needs " +
                             std::to_string(c->hd.expected));
    std::fseek(file.f, (long)c->hd.data_offset, SEEK_SET);
    const ammon_llama_config &g = c->hd.cfg;
    const uint32_t L = g.n_layers, D = g.dim, H = g.hidden, V = g.vocab;
    const uint32_t head = D / g.n_heads, kvd = head * g.n_kv_heads;
    const bool bf = w_dtype == AMMON_BF16;
    const ammon::DType wt = bf ? ammon::DType::BF16 : ammon::DType::F32;
    // every tensor is checked against the 32-bit element count of a Shape
    // before anything is allocated or streamed into it
    const uint64_t counts[] = {(uint64_t)V * D, (uint64_t)L * D, (uint64_t)L * D * D,
                               (uint64_t)L * kvd * D, (uint64_t)L * H * D};
    for (uint64_t n : counts)
      if (n >= (1ull << 32))
        throw ammon::Error(AMMON_E_VALIDATION, "checkpoint: a tensor of " + std::to_string(n) +
                                                   " elements exceeds 2^32 - 1");
    auto make = [&](uint64_t n, ammon::DType dt) -> void * {
      c->bufs.push_back(ammon::Tensor::zeros(c->rt, ammon::Shape::vector((uint32_t)n), dt));
      return c->bufs.back().data();
    };
    ammon_llama_weights &w = c->w;
    w.tok_emb = make((uint64_t)V * D, wt);
    w.rms_att = (const float *)make((uint64_t)L * D, ammon::DType::F32);
    w.rms_ffn = (const float *)make((uint64_t)L * D, ammon::DType::F32);
    w.rms_final = (const float *)make(D, ammon::DType::F32);
    w.wq = make((uint64_t)L * D * D, wt);
    w.wk = make((uint64_t)L * kvd * D, wt);
    w.wv = make((uint64_t)L * kvd * D, wt);
    w.wo = make((uint64_t)L * D * D, wt);
    w.w1 = make((uint64_t)L * H * D, wt);
    w.w2 = make((uint64_t)L * D * H, wt);
    w.w3 = make((uint64_t)L * H * D, wt);
    w.wcls = c->hd.shared ? w.tok_emb : make((uint64_t)V * D, wt);
    FILE *f = file.f;
    ammon_runtime *r = c->rt.raw();
    Stager stager(r);
    auto mat = [&](const void *dst, uint64_t n, const char *what) {
      stager.stream(f, (void *)dst, n, bf, what);
    };
    auto vec = [&](const void *dst, uint64_t n, const char *what) {
      stager.stream(f, (void *)dst, n, false, what);
    };
    if (c->hd.format == AMMON_CHECKPOINT_LEGACY) {
      mat(w.tok_emb, (uint64_t)V * D, "token_embedding");
      vec(w.rms_att, (uint64_t)L * D, "rms_att");
      mat(w.wq, (uint64_t)L * D * D, "wq");
      mat(w.wk, (uint64_t)L * kvd * D, "wk");
      mat(w.wv, (uint64_t)L * kvd * D, "wv");
      mat(w.wo, (uint64_t)L * D * D, "wo");
      vec(w.rms_ffn, (uint64_t)L * D, "rms_ffn");
      mat(w.w1, (uint64_t)L * H * D, "w1");
      mat(w.w2, (uint64_t)L * D * H, "w2");
      mat(w.w3, (uint64_t)L * H * D, "w3");
      vec(w.rms_final, D, "rms_final");
      skip(f, (uint64_t)g.max_seq * head * 4);  // freq_cis_real + freq_cis_imag
      if (!c->hd.shared) mat(w.wcls, (uint64_t)V * D, "classifier");
    } else {
      vec(w.rms_att, (uint64_t)L * D, "rms_att");
      vec(w.rms_ffn, (uint64_t)L * D, "rms_ffn");
      vec(w.rms_final, D, "rms_final");
      mat(w.tok_emb, (uint64_t)V * D, "token_embedding");
      mat(w.wq, (uint64_t)L * D * D, "wq");
      mat(w.wk, (uint64_t)L * kvd * D, "wk");
      mat(w.wv, (uint64_t)L * kvd * D, "wv");
      mat(w.wo, (uint64_t)L * D * D, "wo");
      mat(w.w1, (uint64_t)L * H * D, "w1");
      mat(w.w2, (uint64_t)L * D * H, "w2");
      mat(w.w3, (uint64_t)L * H * D, "w3");
      if (!c->hd.shared) mat(w.wcls, (uint64_t)V * D, "classifier");
    }
    ammon::check(ammon_stream_synchronize(r, nullptr), "checkpoint upload");
    *out = c;
    return AMMON_OK;
  } catch (const ammon::Error &e) {
    delete c;
    return ammon_rt::set_error(e.status(), "%s", e.what());
  } catch (const std::bad_alloc &) {
    delete c;
    return ammon_rt::set_error(AMMON_E_OOM, "checkpoint: out of host memory");
  }
}

ammon_status ammon_checkpoint_config(const ammon_checkpoint *c, ammon_llama_config *cfg) {
  AMMON_CHECK(c && cfg, "checkpoint_config: NULL argument");
  *cfg = c->hd.cfg;
  cfg->w_dtype = c->w_dtype;
  return AMMON_OK;
}

ammon_status ammon_checkpoint_weights(const ammon_checkpoint *c, ammon_llama_weights *w) {
  AMMON_CHECK(c && w, "checkpoint_weights: NULL argument");
  *w = c->w;
  return AMMON_OK;
}

ammon_status ammon_checkpoint_free(ammon_checkpoint *c) {
  delete c;
  return AMMON_OK;
}

}  // extern "C"
