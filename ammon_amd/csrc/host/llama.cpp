// llama.cpp -- the llama2.c-convention test model built from the C++ modules,
// and its C entry points (include/ammon/ammon_model.h).
//
// Graph (the one Ammon's modules imply; the reference leaves it to
// architecture crates, README.md:5):
//   x = embed(token)
//   per layer: CausalAttentionBlock (x += attn), SwiGluBlock (x += ffn)
//   logits = Wcls . rmsnorm(x, w_final)          (one fused launch)
// One token is recorded once into a Scheme and replayed as a HIP graph; the
// DecodeStep parcel is the only per-token input.  A second scheme appends the
// device greedy step (argmax + prompt forcing + DecodeStep update) so tokens
// can be generated back to back without host round trips.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <memory>

#include "../runtime/internal.h"
#include "ammon/ammon.hpp"
#include "ammon/ammon_model.h"
#include "ammon/ammon_tokenizer.h"

namespace ammon {

const BpeTokenizer &bpe_of(const ammon_bpe *t);  // host/tokenizer.cpp
namespace {

class LlamaModel : public AutoregressiveModel {
 public:
  LlamaModel(const Runtime &rt, const ammon_llama_config &c, const ammon_llama_weights &w);
  ~LlamaModel() override;

  size_t vocab_size() const override { return c_.vocab; }
  uint32_t max_seq_len() const override { return c_.max_seq; }
  const std::vector<float> &step(uint32_t token, uint32_t pos) override;

  GenerateTokenOutput generate_device(const std::vector<int32_t> &prompt, uint32_t max_new,
                                      std::optional<int32_t> stop_on, float *last_logits);
  GenerateTokenOutput generate_prefill(const std::vector<int32_t> &prompt, uint32_t max_new,
                                       std::optional<int32_t> stop_on, float *last_logits);
  void prefill(const int32_t *tokens, uint32_t n, uint32_t start, float *logits);
  void decode(uint32_t token, uint32_t start_pos, uint32_t n_steps, int32_t *tokens);
  KvLayer kv_layer(uint32_t l) const { return cache_.layer(l); }
  void read_tokens(uint32_t start, uint32_t n, int32_t *out);
  ammon_stream stream() const { return stream_; }
  float *device_logits() const { return (float *)logits_.data(); }
  uint32_t launches() const { return (uint32_t)token_scheme_->ir_node_count(); }
  // Host logits of the most recent step() (what generate_tokens last saw).
  const std::vector<float> &last_logits() const { return host_logits_; }

 private:
  // greedy: end with the LM head fused with the greedy step (n_prompt
  // forced tokens) instead of the plain LM head
  void record_token(Scheme &s, bool greedy = false, uint32_t n_prompt = 0);
  void ensure_decode_scheme(uint32_t n_prompt);
  void ensure_prefill(uint32_t n);
  const float *rope_table();
  void deposit(uint32_t token, uint32_t pos, ammon_stream stream);

  Runtime rt_;
  ammon_llama_config c_;
  uint32_t head_, q_dim_, kv_dim_;
  TensorView tok_emb_, rms_final_, wcls_;
  std::vector<CausalAttentionBlockWeights> attn_w_;
  std::vector<SwiGluBlockWeights> ffn_w_;
  Embedding embed_;
  CausalAttentionBlock attn_;
  SwiGluBlock ffn_;
  Linear lm_head_;
  KvCache cache_;
  Tensor x_, logits_, step_, prompt_, tokens_, scratch_;
  ammon_stream stream_ = nullptr;  // both schemes replay here, in order
  std::unique_ptr<Scheme> token_scheme_, decode_scheme_;
  Tensor rope_table_;
  uint32_t decode_prompt_ = 0xffffffffu;
  ammon_decode_step *pinned_step_ = nullptr;
  float *pinned_logits_ = nullptr;
  std::vector<float> host_logits_;
  // prompt prefill scratch, [capacity, width] rows
  uint32_t pf_cap_ = 0;
  Tensor pf_ids_, pf_x_, pf_xn_, pf_q_, pf_att_, pf_hb_, pf_partial_, pf_ws_;
};

DType dt(ammon_dtype d) { return (DType)d; }

TensorView view(const void *base, DType d, size_t layer, std::vector<uint32_t> dims) {
  Shape s = Shape::from_dims(std::move(dims));
  return TensorView((char *)base + layer * s.numel() * dtype_size(d), s, d);
}

AttentionOptions attention_options(const ammon_llama_config &c) {
  AttentionOptions o;
  o.theta = c.theta;
  o.eps = c.eps;
  o.split_len = c.split_len;
  return o;
}

uint32_t checked_head(const ammon_llama_config &c) {
  if (c.n_heads == 0 || c.dim % c.n_heads != 0)
    throw Error(AMMON_E_VALIDATION, "llama: dim is not divisible by n_heads");
  if (c.n_kv_heads == 0 || c.n_heads % c.n_kv_heads != 0)
    throw Error(AMMON_E_VALIDATION, "llama: n_heads is not a multiple of n_kv_heads");
  if (c.vocab == 0 || c.max_seq == 0 || c.n_layers == 0 || c.hidden == 0)
    throw Error(AMMON_E_VALIDATION, "llama: empty configuration");
  return c.dim / c.n_heads;
}

LlamaModel::LlamaModel(const Runtime &rt, const ammon_llama_config &c, const ammon_llama_weights &w)
    : rt_(rt),
      c_(c),
      head_(checked_head(c)),
      q_dim_(head_ * c.n_heads),
      kv_dim_(head_ * c.n_kv_heads),
      embed_(rt),
      attn_(rt, c.dim, c.n_heads, c.max_seq, attention_options(c)),
      ffn_(rt, c.dim, c.hidden, c.eps),
      lm_head_(rt),
      cache_(rt, c.n_layers, c.max_seq, c.n_kv_heads, head_, dt(c.kv_dtype)) {
  const DType wd = dt(c.w_dtype);
  if (!w.tok_emb || !w.rms_att || !w.rms_ffn || !w.wq || !w.wk || !w.wv || !w.wo || !w.w1 ||
      !w.w2 || !w.w3 || !w.rms_final || !w.wcls)
    throw Error(AMMON_E_VALIDATION, "llama: a weight pointer is NULL");
  tok_emb_ = view(w.tok_emb, wd, 0, {c.vocab, c.dim});
  rms_final_ = view(w.rms_final, DType::F32, 0, {c.dim});
  wcls_ = view(w.wcls, wd, 0, {c.vocab, c.dim});
  for (uint32_t l = 0; l < c.n_layers; ++l) {
    attn_w_.push_back(CausalAttentionBlockWeights{
        view(w.rms_att, DType::F32, l, {c.dim}), view(w.wq, wd, l, {q_dim_, c.dim}),
        view(w.wk, wd, l, {kv_dim_, c.dim}), view(w.wv, wd, l, {kv_dim_, c.dim}),
        view(w.wo, wd, l, {c.dim, q_dim_})});
    ffn_w_.push_back(SwiGluBlockWeights{
        view(w.rms_ffn, DType::F32, l, {c.dim}), view(w.w1, wd, l, {c.hidden, c.dim}),
        view(w.w3, wd, l, {c.hidden, c.dim}), view(w.w2, wd, l, {c.dim, c.hidden})});
  }
  x_ = Tensor::zeros(rt, Shape::vector(c.dim), DType::F32);
  logits_ = Tensor::zeros(rt, Shape::vector(c.vocab), DType::F32);
  step_ = DecodeStep::parcel(rt);
  prompt_ = Tensor::zeros(rt, Shape::vector(c.max_seq), DType::I32);
  tokens_ = Tensor::zeros(rt, Shape::vector(c.max_seq), DType::I32);
  scratch_ = Tensor::zeros(
      rt,
      Shape::vector((uint32_t)(std::max(ammon_argmax_scratch_bytes(c.vocab),
                                        ammon_greedy_lm_head_scratch_bytes(rt.raw())) / 4)),
      DType::F32);
  check(ammon_alloc_host(rt.raw(), sizeof(ammon_decode_step), (void **)&pinned_step_), "llama");
  check(ammon_alloc_host(rt.raw(), sizeof(float) * c.vocab, (void **)&pinned_logits_), "llama");
  host_logits_.resize(c.vocab);
  check(ammon_stream_create(rt.raw(), &stream_), "llama stream");
  token_scheme_ = std::make_unique<Scheme>(rt, c.use_graph != 0, stream_);
  record_token(*token_scheme_);
}

LlamaModel::~LlamaModel() {
  decode_scheme_.reset();
  token_scheme_.reset();
  if (stream_) ammon_stream_destroy(rt_.raw(), stream_);
  if (pinned_step_) ammon_free_host(rt_.raw(), pinned_step_);
  if (pinned_logits_) ammon_free_host(rt_.raw(), pinned_logits_);
}

void LlamaModel::record_token(Scheme &s, bool greedy, uint32_t n_prompt) {
  embed_.record(s, tok_emb_, step_, x_.view());
  for (uint32_t l = 0; l < c_.n_layers; ++l) {
    const std::string layer = "layer" + std::to_string(l);
    attn_.record_group(s, layer + "/attn", x_.view(), attn_w_[l], cache_.layer(l), step_);
    ffn_.record_group(s, layer + "/ffn", x_.view(), ffn_w_[l]);
  }
  if (greedy)
    kernels::greedy_lm_head(s, "greedy_lm_head", wcls_, x_.view(), rms_final_, logits_.view(),
                            scratch_.view(), prompt_.view(), n_prompt, step_, tokens_.view(),
                            c_.eps);
  else
    lm_head_.record_normed(s, wcls_, x_.view(), rms_final_, logits_.view(), c_.eps);
}

void LlamaModel::ensure_decode_scheme(uint32_t n_prompt) {
  if (decode_scheme_ && decode_prompt_ == n_prompt) return;
  auto s = std::make_unique<Scheme>(rt_, c_.use_graph != 0, stream_);
  record_token(*s, true, n_prompt);
  decode_scheme_ = std::move(s);
  decode_prompt_ = n_prompt;
}

void LlamaModel::deposit(uint32_t token, uint32_t pos, ammon_stream stream) {
  // The pinned staging slot is reused per token: wait for the previous
  // deposit on this stream before overwriting it.
  check(ammon_stream_synchronize(rt_.raw(), stream), "deposit");
  pinned_step_->token = token;
  pinned_step_->position = pos;
  check(ammon_memcpy(rt_.raw(), step_.data(), pinned_step_, sizeof(ammon_decode_step),
                     AMMON_COPY_H2D, stream),
        "deposit");
}

const std::vector<float> &LlamaModel::step(uint32_t token, uint32_t pos) {
  if (token >= c_.vocab)
    throw Error(AMMON_E_VALIDATION, "step: token " + std::to_string(token) + " >= vocab " +
                                        std::to_string(c_.vocab));
  if (pos >= c_.max_seq)
    throw Error(AMMON_E_VALIDATION, "step: position " + std::to_string(pos) + " >= max_seq " +
                                        std::to_string(c_.max_seq));
  deposit(token, pos, stream_);
  token_scheme_->submit();
  check(ammon_memcpy(rt_.raw(), pinned_logits_, logits_.data(), sizeof(float) * c_.vocab,
                     AMMON_COPY_D2H, stream_),
        "logits");
  check(ammon_stream_synchronize(rt_.raw(), stream_), "step");
  std::memcpy(host_logits_.data(), pinned_logits_, sizeof(float) * c_.vocab);
  return host_logits_;
}

GenerateTokenOutput LlamaModel::generate_device(const std::vector<int32_t> &prompt,
                                                uint32_t max_new, std::optional<int32_t> stop_on,
                                                float *last_logits) {
  if (prompt.empty()) throw Error(AMMON_E_VALIDATION, "expected at least one prompt token");
  for (int32_t t : prompt)
    if (t < 0 || (uint32_t)t >= c_.vocab)
      throw Error(AMMON_E_VALIDATION, "prompt token " + std::to_string(t) + " outside the vocab");
  const uint32_t limit = std::min(max_new, c_.max_seq);
  const uint32_t steps = limit > 0 ? limit - 1 : 0;
  const uint32_t n_prompt = (uint32_t)std::min<size_t>(prompt.size(), c_.max_seq);
  ensure_decode_scheme(n_prompt);
  ammon_stream st = stream_;
  check(ammon_memcpy(rt_.raw(), prompt_.data(), prompt.data(), sizeof(int32_t) * n_prompt,
                     AMMON_COPY_H2D, st),
        "prompt upload");
  deposit((uint32_t)prompt[0], 0, st);
  ammon_event e0 = nullptr, e1 = nullptr;
  check(ammon_event_create(rt_.raw(), &e0), "event");
  check(ammon_event_create(rt_.raw(), &e1), "event");
  for (uint32_t i = 0; i < steps; ++i) {
    decode_scheme_->submit();
    if (i == 0) check(ammon_event_record(rt_.raw(), e0, st), "event");
  }
  check(ammon_event_record(rt_.raw(), e1, st), "event");
  check(ammon_stream_synchronize(rt_.raw(), st), "generate");
  float ms = 0.f;
  if (steps > 1) check(ammon_event_elapsed_ms(rt_.raw(), e0, e1, &ms), "event");
  ammon_event_destroy(rt_.raw(), e0);
  ammon_event_destroy(rt_.raw(), e1);

  std::vector<int32_t> all(steps);
  if (steps)
    check(ammon_memcpy(rt_.raw(), all.data(), tokens_.data(), sizeof(int32_t) * steps,
                       AMMON_COPY_D2H, st),
          "tokens");
  if (last_logits)
    check(ammon_memcpy(rt_.raw(), last_logits, logits_.data(), sizeof(float) * c_.vocab,
                       AMMON_COPY_D2H, st),
          "logits");
  check(ammon_stream_synchronize(rt_.raw(), st), "generate");
  GenerateTokenOutput out;
  out.prompt_tokens = prompt.size();
  for (int32_t t : all) {
    if (stop_on && *stop_on == t) break;
    out.tokens.push_back(t);
  }
  out.tokens_per_second = (steps > 1 && ms > 0.f) ? (double)(steps - 1) / (ms * 1e-3) : 0.0;
  return out;
}

void LlamaModel::decode(uint32_t token, uint32_t start_pos, uint32_t n_steps, int32_t *tokens) {
  if (token >= c_.vocab) throw Error(AMMON_E_VALIDATION, "decode: token outside the vocab");
  if ((uint64_t)start_pos + n_steps > c_.max_seq)
    throw Error(AMMON_E_VALIDATION, "decode: start_pos + n_steps exceeds max_seq");
  ensure_decode_scheme(0);
  deposit(token, start_pos, stream_);
  for (uint32_t i = 0; i < n_steps; ++i) decode_scheme_->submit();
  if (tokens) {
    check(ammon_memcpy(rt_.raw(), tokens, (int32_t *)tokens_.data() + start_pos,
                       sizeof(int32_t) * n_steps, AMMON_COPY_D2H, stream_),
          "tokens");
    check(ammon_stream_synchronize(rt_.raw(), stream_), "decode");
  }
}

const float *LlamaModel::rope_table() {
  if (!rope_table_.data()) {
    std::vector<float> table(ammon_rope_table_bytes(head_, c_.max_seq) / sizeof(float));
    check(ammon_rope_table_host(c_.theta, head_, c_.max_seq, table.data()), "rope table");
    rope_table_ = Tensor::from_f32(rt_, Shape::vector((uint32_t)table.size()), table);
  }
  return (const float *)rope_table_.data();
}

void LlamaModel::ensure_prefill(uint32_t n) {
  if (n <= pf_cap_) return;
  const uint32_t cap = std::max(n, 16u);
  pf_ids_ = Tensor::zeros(rt_, Shape::vector(cap), DType::I32);
  pf_x_ = Tensor::zeros(rt_, Shape::from_dims({cap, c_.dim}), DType::F32);
  pf_xn_ = Tensor::zeros(rt_, Shape::from_dims({cap, c_.dim}), DType::F32);
  pf_q_ = Tensor::zeros(rt_, Shape::from_dims({cap, q_dim_}), DType::F32);
  pf_att_ = Tensor::zeros(rt_, Shape::from_dims({cap, q_dim_}), DType::F32);
  pf_hb_ = Tensor::zeros(rt_, Shape::from_dims({cap, c_.hidden}), DType::F32);
  // split-reduction partial sums of the QKV, wo and w2 GEMMs
  const uint32_t ws_rows = std::max(c_.dim, q_dim_ + 2 * c_.n_kv_heads * head_);
  pf_ws_ = Tensor::zeros(
      rt_, Shape::vector((uint32_t)(ammon_prefill_gemm_workspace_bytes(ws_rows, cap) / 4)),
      DType::F32);
  pf_cap_ = cap;
}

// Positions start..start+n-1 through every layer at once: embed rows, then
// per layer rmsnorm rows, QKV GEMM (RoPE + cache stores at start + t),
// token-batched attention, wo GEMM + residual, rmsnorm rows, gate/up GEMM +
// SwiGLU, w2 GEMM + residual; the final norm and LM head for the last row.
void LlamaModel::prefill(const int32_t *tokens, uint32_t n, uint32_t start, float *logits) {
  if (n == 0) throw Error(AMMON_E_VALIDATION, "prefill: no tokens");
  if ((uint64_t)start + n > c_.max_seq)
    throw Error(AMMON_E_VALIDATION, "prefill: start_pos + n exceeds max_seq");
  for (uint32_t i = 0; i < n; ++i)
    if (tokens[i] < 0 || (uint32_t)tokens[i] >= c_.vocab)
      throw Error(AMMON_E_VALIDATION, "prefill: token " + std::to_string(tokens[i]) +
                                          " outside the vocab");
  ensure_prefill(n);
  ammon_runtime *rt = rt_.raw();
  ammon_stream st = stream_;
  const ammon_dtype wd = c_.w_dtype, kvd = c_.kv_dtype;
  const uint32_t ctx = start + n;
  // split: as many units as the device holds twice, over the context
  const uint32_t target = 2u * (uint32_t)std::max(rt->info.compute_units, 1);
  uint32_t split = 16;
  while (split < AMMON_ATTENTION_MAX_SPLIT &&
         ((uint64_t)c_.n_kv_heads * n * ammon_attention_splits(ctx, split) > target ||
          ammon_attention_splits(ctx, split) > AMMON_ATTENTION_MAX_SPLITS))
    split *= 2;
  // attention partials [n][q_heads][splits over ctx][head + 2], grown on demand
  const size_t part_bytes = ammon_attention_prefill_scratch_bytes(n, c_.n_heads, head_, ctx, split);
  if (!pf_partial_.data() || pf_partial_.nbytes() < part_bytes)
    pf_partial_ = Tensor::zeros(rt_, Shape::vector((uint32_t)(part_bytes / 4)), DType::F32);
  float *x = (float *)pf_x_.data(), *xn = (float *)pf_xn_.data();
  float *q = (float *)pf_q_.data(), *att = (float *)pf_att_.data(), *hb = (float *)pf_hb_.data();
  const float *table = rope_table();
  deposit((uint32_t)tokens[0], start, st);
  check(ammon_memcpy(rt, pf_ids_.data(), tokens, sizeof(int32_t) * n, AMMON_COPY_H2D, st),
        "prefill ids");
  check(ammon_embed_rows(rt, st, tok_emb_.data(), wd, c_.vocab, c_.dim,
                         (const uint32_t *)pf_ids_.data(), n, x),
        "prefill embed");
  const ammon_decode_step *step = (const ammon_decode_step *)step_.data();
  for (uint32_t l = 0; l < c_.n_layers; ++l) {
    const CausalAttentionBlockWeights &aw = attn_w_[l];
    const SwiGluBlockWeights &fw = ffn_w_[l];
    KvLayer kv = cache_.layer(l);
    check(ammon_rmsnorm(rt, st, x, aw.norm.data(), AMMON_F32, xn, n, c_.dim, c_.eps),
          "prefill rmsnorm");
    check(ammon_prefill_qkv_rope_store_ws(rt, st, xn, n, aw.query.data(), aw.key.data(),
                                          aw.value.data(), wd, c_.dim, c_.n_heads, c_.n_kv_heads,
                                          head_, q, kv.key.data(), kv.value.data(), kvd,
                                          c_.max_seq, step, table, pf_ws_.data(), pf_ws_.nbytes()),
          "prefill qkv");
    check(ammon_attention_prefill(rt, st, q, n, c_.n_heads, kv.key.data(), kv.value.data(), kvd,
                                  c_.n_kv_heads, head_, c_.max_seq, step, ctx, split,
                                  (float *)pf_partial_.data(), part_bytes, att),
          "prefill attention");
    check(ammon_prefill_gemm_ws(rt, st, aw.output.data(), wd, c_.dim, q_dim_, att, n, x, x,
                                pf_ws_.data(), pf_ws_.nbytes()),
          "prefill wo");
    check(ammon_rmsnorm(rt, st, x, fw.norm.data(), AMMON_F32, xn, n, c_.dim, c_.eps),
          "prefill rmsnorm");
    check(ammon_prefill_gate_up_swiglu(rt, st, xn, n, fw.gate.data(), fw.up.data(), wd, c_.dim,
                                       c_.hidden, hb),
          "prefill gate/up");
    check(ammon_prefill_gemm_ws(rt, st, fw.down.data(), wd, c_.dim, c_.hidden, hb, n, x, x,
                                pf_ws_.data(), pf_ws_.nbytes()),
          "prefill w2");
  }
  check(ammon_gemv_rmsnorm(rt, st, x + (size_t)(n - 1) * c_.dim, rms_final_.data(), AMMON_F32,
                           c_.eps, wcls_.data(), wd, c_.vocab, c_.dim, (float *)logits_.data()),
        "prefill lm head");
  // the DecodeStep a one-by-one pass would leave: the last token at its position
  deposit((uint32_t)tokens[n - 1], start + n - 1, st);
  if (logits) {
    check(ammon_memcpy(rt, logits, logits_.data(), sizeof(float) * c_.vocab, AMMON_COPY_D2H, st),
          "prefill logits");
  }
  check(ammon_stream_synchronize(rt, st), "prefill");
}

GenerateTokenOutput LlamaModel::generate_prefill(const std::vector<int32_t> &prompt,
                                                 uint32_t max_new, std::optional<int32_t> stop_on,
                                                 float *last_logits) {
  if (prompt.empty()) throw Error(AMMON_E_VALIDATION, "expected at least one prompt token");
  const uint32_t limit = std::min(max_new, c_.max_seq);
  const uint32_t steps = limit > 0 ? limit - 1 : 0;
  const uint32_t n_prompt = (uint32_t)std::min<size_t>(prompt.size(), c_.max_seq);
  // every step is a forced prompt token: nothing to prefill ahead of
  if (steps < n_prompt) return generate_device(prompt, max_new, stop_on, last_logits);
  ensure_decode_scheme(n_prompt);
  ammon_runtime *rt = rt_.raw();
  ammon_stream st = stream_;
  prefill(prompt.data(), n_prompt, 0, nullptr);
  check(ammon_memcpy(rt, prompt_.data(), prompt.data(), sizeof(int32_t) * n_prompt,
                     AMMON_COPY_H2D, st),
        "prompt upload");
  // forced tokens of positions 0..n-2, as the stepped loop records them
  if (n_prompt > 1)
    check(ammon_memcpy(rt, tokens_.data(), prompt.data() + 1, sizeof(int32_t) * (n_prompt - 1),
                       AMMON_COPY_H2D, st),
          "prompt tokens");
  // the greedy step of position n-1 on the prefilled logits
  check(ammon_greedy_next(rt, st, (const float *)logits_.data(), c_.vocab, scratch_.data(),
                          (const int32_t *)prompt_.data(), n_prompt,
                          (ammon_decode_step *)step_.data(), (int32_t *)tokens_.data(), c_.max_seq),
        "prefill greedy");
  ammon_event e0 = nullptr, e1 = nullptr;
  check(ammon_event_create(rt, &e0), "event");
  check(ammon_event_create(rt, &e1), "event");
  check(ammon_event_record(rt, e0, st), "event");
  for (uint32_t pos = n_prompt; pos < steps; ++pos) decode_scheme_->submit();
  check(ammon_event_record(rt, e1, st), "event");
  check(ammon_stream_synchronize(rt, st), "generate");
  float ms = 0.f;
  const uint32_t decoded = steps - n_prompt;
  if (decoded > 0) check(ammon_event_elapsed_ms(rt, e0, e1, &ms), "event");
  ammon_event_destroy(rt, e0);
  ammon_event_destroy(rt, e1);
  std::vector<int32_t> all(steps);
  if (steps)
    check(ammon_memcpy(rt, all.data(), tokens_.data(), sizeof(int32_t) * steps, AMMON_COPY_D2H, st),
          "tokens");
  if (last_logits)
    check(ammon_memcpy(rt, last_logits, logits_.data(), sizeof(float) * c_.vocab, AMMON_COPY_D2H,
                       st),
          "logits");
  check(ammon_stream_synchronize(rt, st), "generate");
  GenerateTokenOutput out;
  out.prompt_tokens = prompt.size();
  for (int32_t t : all) {
    if (stop_on && *stop_on == t) break;
    out.tokens.push_back(t);
  }
  out.tokens_per_second = (decoded > 0 && ms > 0.f) ? (double)decoded / (ms * 1e-3) : 0.0;
  return out;
}

void LlamaModel::read_tokens(uint32_t start, uint32_t n, int32_t *out) {
  if ((uint64_t)start + n > c_.max_seq)
    throw Error(AMMON_E_VALIDATION, "tokens: range exceeds max_seq");
  check(ammon_stream_synchronize(rt_.raw(), stream_), "tokens");
  if (!n) return;
  check(ammon_memcpy(rt_.raw(), out, (int32_t *)tokens_.data() + start, sizeof(int32_t) * n,
                     AMMON_COPY_D2H, stream_),
        "tokens");
  check(ammon_stream_synchronize(rt_.raw(), stream_), "tokens");
}

}  // namespace
}  // namespace ammon

// ---- C entry points -------------------------------------------------------------------------
struct ammon_llama {
  std::unique_ptr<ammon::LlamaModel> model;
  ammon::Runtime rt;
};

namespace {

template <typename F>
ammon_status guarded(F &&fn) {
  try {
    fn();
    return AMMON_OK;
  } catch (const ammon::Error &e) {
    return ammon_rt::set_error(e.status(), "%s", e.what());
  } catch (const std::exception &e) {
    return ammon_rt::set_error(AMMON_E_HIP, "%s", e.what());
  }
}

// The C++ layer holds its own runtime reference for the model's lifetime.
ammon::Runtime runtime_for(ammon_runtime *rt) {
  return ammon::Runtime::create(rt->device);
}

}  // namespace

extern "C" {

ammon_status ammon_llama_create(ammon_runtime *rt, const ammon_llama_config *cfg,
                                const ammon_llama_weights *w, ammon_llama **out) {
  AMMON_CHECK(rt && cfg && w && out, "llama_create: NULL argument");
  return guarded([&] {
    auto *m = new ammon_llama();
    try {
      m->rt = runtime_for(rt);
      m->model = std::make_unique<ammon::LlamaModel>(m->rt, *cfg, *w);
    } catch (...) {
      delete m;
      throw;
    }
    *out = m;
  });
}

ammon_status ammon_llama_destroy(ammon_llama *m) {
  delete m;
  return AMMON_OK;
}

ammon_status ammon_llama_step(ammon_llama *m, uint32_t token, uint32_t pos, float *logits) {
  AMMON_CHECK(m && logits, "llama_step: NULL argument");
  return guarded([&] {
    const std::vector<float> &l = m->model->step(token, pos);
    std::memcpy(logits, l.data(), l.size() * sizeof(float));
  });
}

static ammon_status fill_output(const ammon::GenerateTokenOutput &o, int32_t *out_tokens,
                                uint32_t *n_out, double *tps) {
  std::copy(o.tokens.begin(), o.tokens.end(), out_tokens);
  *n_out = (uint32_t)o.tokens.size();
  if (tps) *tps = o.tokens_per_second;
  return AMMON_OK;
}

ammon_status ammon_llama_generate_tokens(ammon_llama *m, const int32_t *prompt, uint32_t n_prompt,
                                         uint32_t max_new_tokens, int has_stop, int32_t stop_on,
                                         int32_t *out_tokens, uint32_t *n_out,
                                         double *tokens_per_second, float *last_logits) {
  AMMON_CHECK(m && out_tokens && n_out, "llama_generate_tokens: NULL argument");
  AMMON_CHECK(n_prompt > 0 && prompt, "expected at least one prompt token");
  return guarded([&] {
    std::vector<int32_t> p(prompt, prompt + n_prompt);
    for (int32_t t : p)
      if (t < 0 || (size_t)t >= m->model->vocab_size())
        throw ammon::Error(AMMON_E_VALIDATION, "prompt token outside the vocab");
    auto o = ammon::generate_tokens(*m->model, p, max_new_tokens,
                                    has_stop ? std::optional<int32_t>(stop_on) : std::nullopt);
    if (last_logits && !m->model->last_logits().empty())
      std::memcpy(last_logits, m->model->last_logits().data(),
                  m->model->last_logits().size() * sizeof(float));
    fill_output(o, out_tokens, n_out, tokens_per_second);
  });
}

ammon_status ammon_llama_generate_tokens_device(ammon_llama *m, const int32_t *prompt,
                                                uint32_t n_prompt, uint32_t max_new_tokens,
                                                int has_stop, int32_t stop_on,
                                                int32_t *out_tokens, uint32_t *n_out,
                                                double *tokens_per_second, float *last_logits) {
  AMMON_CHECK(m && out_tokens && n_out, "llama_generate_tokens_device: NULL argument");
  AMMON_CHECK(n_prompt > 0 && prompt, "expected at least one prompt token");
  return guarded([&] {
    std::vector<int32_t> p(prompt, prompt + n_prompt);
    auto o = m->model->generate_device(
        p, max_new_tokens, has_stop ? std::optional<int32_t>(stop_on) : std::nullopt, last_logits);
    fill_output(o, out_tokens, n_out, tokens_per_second);
  });
}

ammon_status ammon_llama_prefill(ammon_llama *m, const int32_t *tokens, uint32_t n,
                                 uint32_t start_pos, float *logits) {
  AMMON_CHECK(m && (tokens || n == 0), "llama_prefill: NULL argument");
  return guarded([&] { m->model->prefill(tokens, n, start_pos, logits); });
}

ammon_status ammon_llama_generate_tokens_prefill(ammon_llama *m, const int32_t *prompt,
                                                 uint32_t n_prompt, uint32_t max_new_tokens,
                                                 int has_stop, int32_t stop_on,
                                                 int32_t *out_tokens, uint32_t *n_out,
                                                 double *tokens_per_second, float *last_logits) {
  AMMON_CHECK(m && out_tokens && n_out, "llama_generate_tokens_prefill: NULL argument");
  AMMON_CHECK(n_prompt > 0 && prompt, "expected at least one prompt token");
  return guarded([&] {
    std::vector<int32_t> p(prompt, prompt + n_prompt);
    auto o = m->model->generate_prefill(
        p, max_new_tokens, has_stop ? std::optional<int32_t>(stop_on) : std::nullopt, last_logits);
    fill_output(o, out_tokens, n_out, tokens_per_second);
  });
}

ammon_status ammon_llama_generate_text(ammon_llama *m, const ammon_bpe *t, const char *prompt,
                                       size_t prompt_len, uint32_t max_new_tokens, int bos,
                                       int eos, int has_stop, int32_t stop_on, int loop,
                                       char *text, size_t text_capacity, size_t *text_len,
                                       int32_t *tokens, uint32_t token_capacity,
                                       uint32_t *n_tokens, double *tokens_per_second) {
  AMMON_CHECK(m && t && text_len && n_tokens && (prompt || prompt_len == 0) &&
                  (text || text_capacity == 0) && (tokens || token_capacity == 0),
              "llama_generate_text: NULL argument");
  AMMON_CHECK(loop >= 0 && loop <= 2, "llama_generate_text: loop must be 0, 1 or 2");
  return guarded([&] {
    const ammon::BpeTokenizer &tok = ammon::bpe_of(t);
    const std::vector<int32_t> ids =
        tok.encode(std::string(prompt ? prompt : "", prompt_len), bos != 0, eos != 0);
    if (ids.empty()) throw ammon::Error(AMMON_E_VALIDATION, "expected at least one prompt token");
    for (int32_t id : ids)
      if (id < 0 || (size_t)id >= m->model->vocab_size())
        throw ammon::Error(AMMON_E_VALIDATION, "prompt token " + std::to_string(id) +
                                                   " outside the model's vocab");
    const std::optional<int32_t> stop = has_stop ? std::optional<int32_t>(stop_on) : std::nullopt;
    const ammon::GenerateTokenOutput o =
        loop == 0 ? ammon::generate_tokens(*m->model, ids, max_new_tokens, stop)
        : loop == 1 ? m->model->generate_device(ids, max_new_tokens, stop, nullptr)
                    : m->model->generate_prefill(ids, max_new_tokens, stop, nullptr);
    const std::string s = ammon::decode_tokens(tok, ids[0], o.tokens);
    if (text_capacity) {
      const size_t k = std::min(text_capacity - 1, s.size());
      std::memcpy(text, s.data(), k);
      text[k] = '\0';
    }
    *text_len = s.size();
    std::copy(o.tokens.begin(),
              o.tokens.begin() + (ptrdiff_t)std::min<size_t>(token_capacity, o.tokens.size()),
              tokens);
    *n_tokens = (uint32_t)o.tokens.size();
    if (tokens_per_second) *tokens_per_second = o.tokens_per_second;
  });
}

ammon_status ammon_llama_decode(ammon_llama *m, uint32_t token, uint32_t start_pos,
                                uint32_t n_steps, int32_t *tokens) {
  AMMON_CHECK(m != nullptr, "llama_decode: NULL model");
  return guarded([&] { m->model->decode(token, start_pos, n_steps, tokens); });
}

ammon_status ammon_llama_tokens(ammon_llama *m, uint32_t start, uint32_t n, int32_t *tokens) {
  AMMON_CHECK(m && (tokens || n == 0), "llama_tokens: NULL argument");
  return guarded([&] { m->model->read_tokens(start, n, tokens); });
}

ammon_status ammon_llama_kv_layer(ammon_llama *m, uint32_t layer, void **key, void **value) {
  AMMON_CHECK(m && key && value, "llama_kv_layer: NULL argument");
  return guarded([&] {
    ammon::KvLayer l = m->model->kv_layer(layer);
    *key = l.key.data();
    *value = l.value.data();
  });
}

ammon_status ammon_llama_stream(ammon_llama *m, ammon_stream *stream) {
  AMMON_CHECK(m && stream, "llama_stream: NULL argument");
  *stream = m->model->stream();
  return AMMON_OK;
}

ammon_status ammon_llama_logits(ammon_llama *m, float **device_logits) {
  AMMON_CHECK(m && device_logits, "llama_logits: NULL argument");
  *device_logits = m->model->device_logits();
  return AMMON_OK;
}

ammon_status ammon_llama_launches(ammon_llama *m, uint32_t *n) {
  AMMON_CHECK(m && n, "llama_launches: NULL argument");
  *n = m->model->launches();
  return AMMON_OK;
}

}  // extern "C"
