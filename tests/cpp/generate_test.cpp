// generate_test.cpp -- host-only checks of ammon::generate_tokens and
// ammon::sample_argmax against the reference's loop (src/generate.rs:43-91)
// and argmax rule (src/tokenizer.rs:179-189).  A scripted model stands in
// for the device model, so no GPU is needed.
#include <algorithm>
#include <cmath>
#include <vector>

#include "ammon/ammon.hpp"
#include "check.hpp"

namespace {

// Logits whose argmax after token t at position p is (t + p + 1) % vocab;
// records every (token, pos) step() sees.
class ScriptedModel : public ammon::AutoregressiveModel {
 public:
  ScriptedModel(size_t vocab, uint32_t max_seq) : vocab_(vocab), max_seq_(max_seq), logits_(vocab) {}
  size_t vocab_size() const override { return vocab_; }
  uint32_t max_seq_len() const override { return max_seq_; }
  const std::vector<float> &step(uint32_t token, uint32_t pos) override {
    calls.push_back({token, pos});
    std::fill(logits_.begin(), logits_.end(), 0.f);
    logits_[(token + pos + 1) % vocab_] = 1.f;
    return logits_;
  }
  std::vector<std::pair<uint32_t, uint32_t>> calls;

 private:
  size_t vocab_;
  uint32_t max_seq_;
  std::vector<float> logits_;
};

// The reference loop, written out for the expected values.
std::vector<int32_t> expected(const std::vector<int32_t> &prompt, uint32_t max_new, uint32_t max_seq,
                              size_t vocab, int stop_on) {
  const uint32_t m = std::min(max_new, max_seq);
  std::vector<int32_t> out;
  uint32_t token = (uint32_t)prompt[0], pos = 0;
  while (pos + 1 < m) {
    const int32_t next = pos < prompt.size() - 1 ? prompt[pos + 1] : (int32_t)((token + pos + 1) % vocab);
    ++pos;
    if (next == stop_on) break;
    out.push_back(next);
    token = (uint32_t)next;
  }
  return out;
}

}  // namespace

TEST(generate_forces_prompt_then_follows_argmax) {
  ScriptedModel m(11, 64);
  const std::vector<int32_t> prompt = {3, 7, 2};
  auto o = ammon::generate_tokens(m, prompt, 10);
  CHECK(o.tokens == expected(prompt, 10, 64, 11, -1));
  CHECK(o.tokens.size() == 9);  // max_new - 1 steps
  CHECK(o.prompt_tokens == 3);
  CHECK(m.calls.size() == 9);
  CHECK(m.calls[0] == std::make_pair(3u, 0u));
  CHECK(m.calls[1] == std::make_pair(7u, 1u));  // forced prompt token fed back
}

TEST(generate_is_capped_by_max_seq) {
  ScriptedModel m(5, 6);
  auto o = ammon::generate_tokens(m, {1}, 100);
  CHECK(o.tokens.size() == 5);  // min(max_new, max_seq) - 1
  CHECK(o.tokens == expected({1}, 100, 6, 5, -1));
}

TEST(generate_stop_on_breaks_before_push) {
  ScriptedModel m(7, 64);
  const std::vector<int32_t> want = expected({2}, 20, 64, 7, -1);
  const int32_t stop = want[3];
  const size_t first = std::find(want.begin(), want.end(), stop) - want.begin();
  auto o = ammon::generate_tokens(m, {2}, 20, stop);
  CHECK(o.tokens == expected({2}, 20, 64, 7, stop));
  CHECK(o.tokens.size() == first);  // everything before the first stop token
}

TEST(generate_needs_a_prompt_token) {
  ScriptedModel m(7, 64);
  CHECK_THROWS_WITH(ammon::generate_tokens(m, {}, 5), "at least one prompt token");
}

TEST(generate_with_one_step_budget_does_nothing) {
  ScriptedModel m(7, 64);
  auto o = ammon::generate_tokens(m, {4, 5}, 1);
  CHECK(o.tokens.empty());
  CHECK(m.calls.empty());
  CHECK(o.tokens_per_second == 0.0);
}

// src/tokenizer.rs:225-228 and the NaN rule of :179-189
TEST(sample_argmax_first_index_of_max) {
  const float a[] = {1, 3, 3, 2};
  CHECK(ammon::sample_argmax(a, 4) == 1);
  const float nan_first[] = {NAN, 5, 6};
  CHECK(ammon::sample_argmax(nan_first, 3) == 0);
  const float nan_later[] = {1, NAN, 0.5f, 2};
  CHECK(ammon::sample_argmax(nan_later, 4) == 3);
  const float zeros[] = {-0.0f, 0.0f};
  CHECK(ammon::sample_argmax(zeros, 2) == 0);
}

int main(int argc, char **argv) { return check::run_all(argc, argv); }
