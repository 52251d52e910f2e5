// tokenizer.cpp -- llama2.c-compatible BPE tokenizer and text generation
// (reference src/tokenizer.rs:18-177, src/generate.rs:93-118).
//
// Host-only byte work.  Behaviour kept identical to the reference where it
// is observable: pieces go through a lossy UTF-8 decode on load (invalid
// sequences become U+FFFD, one per maximal invalid subpart, as Rust's
// String::from_utf8_lossy), the sorted piece table is searched with the
// Rust slice binary search (among equal pieces it settles on the last, i.e.
// the highest id), and a byte piece "<0xNN>" decodes to the character
// U+00NN (Rust's `byte as char`), so bytes >= 0x80 come out as two UTF-8
// bytes.  Where the reference would panic (a byte-fallback id past the
// vocabulary, an empty prompt) this throws a validation error instead.
#include <algorithm>
#include <cstdio>
#include <cstring>

#include "ammon/ammon.hpp"

namespace ammon {

namespace {

const char kReplacement[] = "\xEF\xBF\xBD";  // U+FFFD

// Length of the valid UTF-8 sequence starting at s[i], or 0 with `bad` set
// to the length of the maximal invalid subpart to replace (>= 1).
size_t utf8_step(const unsigned char *s, size_t n, size_t i, size_t *bad) {
  const unsigned char b = s[i];
  if (b < 0x80) return 1;
  size_t need;
  unsigned char lo = 0x80, hi = 0xBF;  // range of the second byte
  if (b >= 0xC2 && b <= 0xDF) {
    need = 1;
  } else if (b == 0xE0) {
    need = 2, lo = 0xA0;
  } else if ((b >= 0xE1 && b <= 0xEC) || b == 0xEE || b == 0xEF) {
    need = 2;
  } else if (b == 0xED) {
    need = 2, hi = 0x9F;
  } else if (b == 0xF0) {
    need = 3, lo = 0x90;
  } else if (b >= 0xF1 && b <= 0xF3) {
    need = 3;
  } else if (b == 0xF4) {
    need = 3, hi = 0x8F;
  } else {
    *bad = 1;
    return 0;
  }
  for (size_t k = 1; k <= need; ++k) {
    const size_t j = i + k;
    const unsigned char l = k == 1 ? lo : 0x80, h = k == 1 ? hi : 0xBF;
    if (j >= n || s[j] < l || s[j] > h) {
      *bad = k;  // the lead byte and the continuation bytes that fit
      return 0;
    }
  }
  return need + 1;
}

std::string utf8_lossy(const std::string &in) {
  const unsigned char *s = (const unsigned char *)in.data();
  const size_t n = in.size();
  std::string out;
  out.reserve(n);
  for (size_t i = 0; i < n;) {
    size_t bad = 0;
    const size_t len = utf8_step(s, n, i, &bad);
    if (len) {
      out.append(in, i, len);
      i += len;
    } else {
      out += kReplacement;
      i += bad;
    }
  }
  return out;
}

bool utf8_valid(const std::string &in) {
  const unsigned char *s = (const unsigned char *)in.data();
  for (size_t i = 0; i < in.size();) {
    size_t bad = 0;
    const size_t len = utf8_step(s, in.size(), i, &bad);
    if (!len) return false;
    i += len;
  }
  return true;
}

// u8::from_str_radix(s, 16): an optional '+', then one or more hex digits,
// value at most 255.
bool parse_hex_u8(const std::string &s, unsigned *out) {
  size_t i = 0;
  if (!s.empty() && s[0] == '+') i = 1;
  if (i >= s.size()) return false;
  unsigned v = 0;
  for (; i < s.size(); ++i) {
    const char c = s[i];
    unsigned d;
    if (c >= '0' && c <= '9')
      d = (unsigned)(c - '0');
    else if (c >= 'a' && c <= 'f')
      d = (unsigned)(c - 'a' + 10);
    else if (c >= 'A' && c <= 'F')
      d = (unsigned)(c - 'A' + 10);
    else
      return false;
    v = v * 16 + d;
    if (v > 255) return false;
  }
  *out = v;
  return true;
}

// "<0xNN>" -> NN (src/tokenizer.rs:173-176)
bool parse_byte_token(const std::string &piece, unsigned *byte) {
  if (piece.size() < 4 || piece.compare(0, 3, "<0x") != 0 || piece.back() != '>') return false;
  return parse_hex_u8(piece.substr(3, piece.size() - 4), byte);
}

// UTF-8 of the code point U+00NN
std::string latin1_char(unsigned b) {
  std::string s;
  if (b < 0x80) {
    s += (char)b;
  } else {
    s += (char)(0xC0 | (b >> 6));
    s += (char)(0x80 | (b & 0x3F));
  }
  return s;
}

bool read_exact(FILE *f, void *dst, size_t n) { return std::fread(dst, 1, n, f) == n; }

}  // namespace

BpeTokenizer BpeTokenizer::from_parts(std::vector<std::string> vocab, std::vector<float> scores,
                                      uint32_t max_token_length) {
  if (vocab.size() != scores.size())
    throw Error(AMMON_E_VALIDATION, "tokenizer: " + std::to_string(vocab.size()) +
                                        " pieces but " + std::to_string(scores.size()) +
                                        " scores");
  BpeTokenizer t;
  t.vocab_ = std::move(vocab);
  t.scores_ = std::move(scores);
  t.max_token_length_ = max_token_length;
  t.sorted_.reserve(t.vocab_.size());
  for (size_t i = 0; i < t.vocab_.size(); ++i) t.sorted_.emplace_back(t.vocab_[i], (int32_t)i);
  // bytewise order, stable: equal pieces keep id order
  std::stable_sort(t.sorted_.begin(), t.sorted_.end(),
                   [](const auto &a, const auto &b) { return a.first < b.first; });
  return t;
}

BpeTokenizer BpeTokenizer::from_path(const std::string &path, size_t vocab_size) {
  FILE *f = std::fopen(path.c_str(), "rb");
  if (!f) throw Error(AMMON_E_VALIDATION, "open tokenizer " + path);
  struct Closer {
    FILE *f;
    ~Closer() { std::fclose(f); }
  } closer{f};
  uint32_t max_len = 0;
  if (!read_exact(f, &max_len, 4))
    throw Error(AMMON_E_VALIDATION, "read tokenizer max_token_length");
  std::vector<std::string> vocab;
  std::vector<float> scores;
  vocab.reserve(vocab_size);
  scores.reserve(vocab_size);
  for (size_t i = 0; i < vocab_size; ++i) {
    float score;
    int32_t len;
    if (!read_exact(f, &score, 4))
      throw Error(AMMON_E_VALIDATION, "read tokenizer score " + std::to_string(i));
    if (!read_exact(f, &len, 4))
      throw Error(AMMON_E_VALIDATION, "read tokenizer length " + std::to_string(i));
    if (len < 0)
      throw Error(AMMON_E_VALIDATION, "tokenizer piece " + std::to_string(i) +
                                          " has negative length " + std::to_string(len));
    std::string buf((size_t)len, '\0');
    if (len && !read_exact(f, &buf[0], (size_t)len))
      throw Error(AMMON_E_VALIDATION, "read tokenizer piece " + std::to_string(i));
    scores.push_back(score);
    vocab.push_back(utf8_lossy(buf));
  }
  return from_parts(std::move(vocab), std::move(scores), max_len);
}

// The Rust slice binary search: the loop count depends only on the length;
// among equal keys it settles on the last.
int32_t BpeTokenizer::lookup(const std::string &s) const {
  size_t size = sorted_.size();
  if (size == 0) return -1;
  size_t base = 0;
  while (size > 1) {
    const size_t half = size / 2, mid = base + half;
    if (!(s < sorted_[mid].first)) base = mid;  // element <= key
    size -= half;
  }
  return sorted_[base].first == s ? sorted_[base].second : -1;
}

std::vector<int32_t> BpeTokenizer::encode(const std::string &text, bool bos, bool eos) const {
  std::vector<int32_t> tokens;
  if (bos) tokens.push_back(bos_id());
  if (!text.empty()) {
    const int32_t dummy = lookup(" ");
    if (dummy >= 0) tokens.push_back(dummy);
  }
  const unsigned char *b = (const unsigned char *)text.data();
  const size_t n = text.size();
  for (size_t i = 0; i < n;) {
    const size_t start = i++;
    while (i < n && (b[i] & 0xC0) == 0x80 && i - start < 4) ++i;
    const std::string piece = text.substr(start, i - start);
    if (utf8_valid(piece)) {
      const int32_t id = lookup(piece);
      if (id >= 0) {
        tokens.push_back(id);
        continue;
      }
    }
    for (size_t k = start; k < i; ++k) tokens.push_back((int32_t)b[k] + 3);
  }
  auto piece_of = [&](int32_t id) -> const std::string & {
    if (id < 0 || (size_t)id >= vocab_.size())
      throw Error(AMMON_E_VALIDATION, "tokenizer: token id " + std::to_string(id) +
                                          " outside the vocabulary of " +
                                          std::to_string(vocab_.size()));
    return vocab_[(size_t)id];
  };
  for (;;) {
    float best_score = -1e10f;
    int32_t best_id = -1;
    size_t best_idx = SIZE_MAX;
    for (size_t i = 0; i + 1 < tokens.size(); ++i) {
      const int32_t id = lookup(piece_of(tokens[i]) + piece_of(tokens[i + 1]));
      if (id >= 0 && scores_[(size_t)id] > best_score) {
        best_score = scores_[(size_t)id];
        best_id = id;
        best_idx = i;
      }
    }
    if (best_idx == SIZE_MAX) break;
    tokens[best_idx] = best_id;
    tokens.erase(tokens.begin() + (ptrdiff_t)best_idx + 1);
  }
  if (eos) tokens.push_back(eos_id());
  return tokens;
}

std::string BpeTokenizer::decode(int32_t prev_token, int32_t token) const {
  std::string piece;
  if (token >= 0 && (size_t)token < vocab_.size()) piece = vocab_[(size_t)token];
  if (prev_token == bos_id() && !piece.empty() && piece[0] == ' ') piece.erase(0, 1);
  unsigned byte;
  if (parse_byte_token(piece, &byte)) return latin1_char(byte);
  return piece;
}

std::string decode_tokens(const Tokenizer &tokenizer, int32_t first,
                          const std::vector<int32_t> &tokens) {
  std::string text;
  int32_t prev = first;
  for (int32_t t : tokens) {
    text += tokenizer.decode(prev, t);
    prev = t;
  }
  return text;
}

GenerateOutput generate(AutoregressiveModel &model, const Tokenizer &tokenizer,
                        const std::string &prompt, const GenerateOptions &options) {
  const std::vector<int32_t> prompt_tokens = tokenizer.encode(prompt, options.bos, options.eos);
  if (prompt_tokens.empty())
    throw Error(AMMON_E_VALIDATION, "expected at least one prompt token");
  GenerateTokenOutput out =
      generate_tokens(model, prompt_tokens, options.max_new_tokens, options.stop_on);
  GenerateOutput g;
  g.text = decode_tokens(tokenizer, prompt_tokens[0], out.tokens);
  g.tokens = std::move(out.tokens);
  g.prompt_tokens = out.prompt_tokens;
  g.tokens_per_second = out.tokens_per_second;
  return g;
}

}  // namespace ammon

// ---- C ABI (include/ammon/ammon_tokenizer.h) --------------------------------------------
#include "../runtime/internal.h"
#include "ammon/ammon_tokenizer.h"

struct ammon_bpe {
  ammon::BpeTokenizer tok;
};

namespace {

template <typename F>
ammon_status tok_guarded(F &&fn) {
  try {
    fn();
    return AMMON_OK;
  } catch (const ammon::Error &e) {
    return ammon_rt::set_error(e.status(), "%s", e.what());
  } catch (const std::bad_alloc &) {
    return ammon_rt::set_error(AMMON_E_OOM, "tokenizer: out of host memory");
  } catch (const std::exception &e) {
    return ammon_rt::set_error(AMMON_E_VALIDATION, "%s", e.what());
  }
}

}  // namespace

extern "C" {

ammon_status ammon_bpe_load(const char *path, uint32_t vocab_size, ammon_bpe **out) {
  AMMON_CHECK(path && out, "bpe_load: NULL argument");
  return tok_guarded([&] {
    *out = new ammon_bpe{ammon::BpeTokenizer::from_path(path, vocab_size)};
  });
}

ammon_status ammon_bpe_from_parts(const char *const *pieces, const uint32_t *lengths,
                                  const float *scores, uint32_t n, uint32_t max_token_length,
                                  ammon_bpe **out) {
  AMMON_CHECK(out && (n == 0 || (pieces && lengths && scores)), "bpe_from_parts: NULL argument");
  return tok_guarded([&] {
    std::vector<std::string> vocab;
    vocab.reserve(n);
    for (uint32_t i = 0; i < n; ++i) {
      if (!pieces[i] && lengths[i])
        throw ammon::Error(AMMON_E_VALIDATION, "bpe_from_parts: NULL piece " + std::to_string(i));
      vocab.emplace_back(pieces[i] ? pieces[i] : "", lengths[i]);
    }
    *out = new ammon_bpe{ammon::BpeTokenizer::from_parts(
        std::move(vocab), std::vector<float>(scores, scores + n), max_token_length)};
  });
}

ammon_status ammon_bpe_destroy(ammon_bpe *t) {
  delete t;
  return AMMON_OK;
}

uint32_t ammon_bpe_vocab_size(const ammon_bpe *t) { return t ? (uint32_t)t->tok.vocab_size() : 0; }

uint32_t ammon_bpe_max_token_length(const ammon_bpe *t) {
  return t ? t->tok.max_token_length() : 0;
}

ammon_status ammon_bpe_encode(const ammon_bpe *t, const char *text, size_t text_len, int bos,
                              int eos, int32_t *ids, size_t capacity, size_t *n_ids) {
  AMMON_CHECK(t && n_ids && (text || text_len == 0) && (ids || capacity == 0),
              "bpe_encode: NULL argument");
  return tok_guarded([&] {
    const std::vector<int32_t> v =
        t->tok.encode(std::string(text ? text : "", text_len), bos != 0, eos != 0);
    std::copy(v.begin(), v.begin() + (ptrdiff_t)std::min(capacity, v.size()), ids);
    *n_ids = v.size();
  });
}

ammon_status ammon_bpe_decode(const ammon_bpe *t, int32_t prev_token, int32_t token, char *out,
                              size_t capacity, size_t *len) {
  AMMON_CHECK(t && len && (out || capacity == 0), "bpe_decode: NULL argument");
  return tok_guarded([&] {
    const std::string s = t->tok.decode(prev_token, token);
    if (capacity) {
      const size_t k = std::min(capacity - 1, s.size());
      std::memcpy(out, s.data(), k);
      out[k] = '\0';
    }
    *len = s.size();
  });
}

}  // extern "C"

namespace ammon {
const BpeTokenizer &bpe_of(const ammon_bpe *t) { return t->tok; }
}  // namespace ammon
