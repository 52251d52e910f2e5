// generate.cpp -- greedy decode over AutoregressiveModel (reference
// src/generate.rs:43-91) and sample_argmax (reference src/tokenizer.rs:179-189).
#include <chrono>

#include "ammon/ammon.hpp"

namespace ammon {

int32_t sample_argmax(const float *logits, size_t n) {
  size_t best = 0;
  float best_p = logits[0];
  for (size_t i = 1; i < n; ++i)
    if (logits[i] > best_p) {
      best = i;
      best_p = logits[i];
    }
  return (int32_t)best;
}

GenerateTokenOutput generate_tokens(AutoregressiveModel &model,
                                    const std::vector<int32_t> &prompt_tokens,
                                    uint32_t max_new_tokens, std::optional<int32_t> stop_on) {
  if (prompt_tokens.empty()) throw Error(AMMON_E_VALIDATION, "expected at least one prompt token");
  const uint32_t limit = std::min(max_new_tokens, model.max_seq_len());
  const uint32_t last = limit > 0 ? limit - 1 : 0;  // saturating_sub(1)
  GenerateTokenOutput out;
  out.prompt_tokens = prompt_tokens.size();
  uint32_t token = (uint32_t)prompt_tokens[0];
  uint32_t pos = 0;
  using clock = std::chrono::steady_clock;
  std::optional<clock::time_point> start;
  while (pos < last) {
    const std::vector<float> &logits = model.step(token, pos);
    const int32_t next = (size_t)pos < prompt_tokens.size() - 1
                             ? prompt_tokens[pos + 1]
                             : sample_argmax(logits.data(), logits.size());
    pos += 1;
    if (stop_on && *stop_on == next) break;
    out.tokens.push_back(next);
    token = (uint32_t)next;
    if (!start) start = clock::now();
  }
  const double elapsed =
      start ? std::chrono::duration<double>(clock::now() - *start).count() : 0.0;
  const double gen = pos > 0 ? (double)(pos - 1) : 0.0;
  out.tokens_per_second = elapsed > 0.0 ? gen / elapsed : 0.0;
  return out;
}

}  // namespace ammon
