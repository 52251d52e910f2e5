// modules.cpp -- Ammon's modules (reference src/modules.rs) over the C ABI.
//
// Ownership follows the reference (src/modules.rs:1-3): callers own
// activations, weights, the KV cache and the DecodeStep parcel; modules own
// their decode scratch; nothing here submits -- record() only appends
// validated launches to a Scheme.
//
// The per-block launch sequences are the fused rewrite of
// Blocks::record_attention / record_ffn (src/blocks.rs:172-278):
//   attention: [rmsnorm + wq|wk|wv + rope_store + cache_store] -> attn_partial
//              -> attn_combine -> [wo + residual]            (10 -> 4 launches)
//   SwiGLU:    [rmsnorm + w1|w3 + swiglu] -> [w2 + residual]  (6 -> 2 launches)
#include <sstream>

#include "ammon/ammon.hpp"

namespace ammon {
namespace {

[[noreturn]] void fail(const std::string &msg) { throw Error(AMMON_E_VALIDATION, msg); }

ammon_dtype abi(DType d) { return (ammon_dtype)d; }

void need(bool ok, const std::string &msg) {
  if (!ok) fail(msg);
}

std::string dims(const TensorView &v) { return v.shape().str(); }

}  // namespace

// ---- KvCache ----------------------------------------------------------------------
KvCache::KvCache(const Runtime &rt, uint32_t layers, uint32_t seq_len, uint32_t kv_heads,
                 uint32_t head_size, DType dtype)
    : rt_(rt), layers_(layers), seq_(seq_len), kv_heads_(kv_heads), head_(head_size),
      dtype_(dtype) {
  need(dtype == DType::F32 || dtype == DType::BF16, "KvCache: dtype must be f32 or bf16");
  const Shape shape = Shape::from_dims({layers, kv_heads, seq_len, head_size});
  key_ = Tensor::zeros(rt, shape, dtype);
  value_ = Tensor::zeros(rt, shape, dtype);
}

KvLayer KvCache::layer(uint32_t layer) const {
  need(layer < layers_, "KvCache::layer: layer " + std::to_string(layer) + " of " +
                            std::to_string(layers_));
  const std::vector<uint32_t> d = {kv_heads_, seq_, head_};
  return KvLayer{key_.view().narrow(0, layer, 1).reshape(d),
                 value_.view().narrow(0, layer, 1).reshape(d)};
}

std::vector<uint8_t> KvCache::layer_to_host_reference_order(uint32_t layer, bool value) const {
  need(layer < layers_, "KvCache: layer " + std::to_string(layer) + " of " +
                            std::to_string(layers_));
  const Tensor &src = value ? value_ : key_;
  const size_t layer_bytes = (size_t)kv_heads_ * seq_ * head_ * dtype_size(dtype_);
  std::vector<uint8_t> head_major(layer_bytes), pos_major(layer_bytes);
  check(ammon_memcpy(rt_.raw(), head_major.data(), (const char *)src.data() + layer * layer_bytes,
                     layer_bytes, AMMON_COPY_D2H, nullptr),
        "KvCache download");
  check(ammon_stream_synchronize(rt_.raw(), nullptr), "KvCache download");
  check(ammon_kv_unpermute(head_major.data(), pos_major.data(), kv_heads_, seq_, head_,
                           (uint32_t)dtype_size(dtype_)),
        "KvCache unpermute");
  return pos_major;
}

// ---- Embedding ------------------------------------------------------------------------
Embedding::Embedding(const Runtime &rt) : rt_(rt) {}

void Embedding::record(Scheme &s, TensorView table, const Tensor &step, TensorView x) const {
  kernels::embed(s, "embed", table, step, x);
}

void Embedding::record_group(Scheme &s, const std::string &label, TensorView table,
                             const Tensor &step, TensorView x) const {
  s.group(label, [&](Scheme &g) { record(g, table, step, x); });
}

// ---- RmsNorm ------------------------------------------------------------------------------
RmsNorm::RmsNorm(const Runtime &rt, float eps) : rt_(rt), eps_(eps) {}

void RmsNorm::record(Scheme &s, TensorView x, TensorView weight, TensorView out) const {
  kernels::rmsnorm(s, "rmsnorm", x, weight, out, eps_);
}

void RmsNorm::record_inplace(Scheme &s, TensorView x, TensorView weight) const {
  kernels::rmsnorm_inplace(s, "rmsnorm", x, weight, eps_);
}

// ---- Linear -----------------------------------------------------------------------------------
Linear::Linear(const Runtime &rt) : rt_(rt) {}

void Linear::record(Scheme &s, TensorView weight, TensorView x, TensorView out) const {
  TensorKernels::prepare(rt_).matmul_into(s, "linear", weight, x, out);
}

void Linear::record_normed(Scheme &s, TensorView weight, TensorView x, TensorView norm_weight,
                           TensorView out, float eps) const {
  const std::string k = "linear";
  need(weight.shape().rank() == 2, k + ": parameter `weight`: expected rank 2, got " + dims(weight));
  const uint32_t d = weight.shape().dim(0), n = weight.shape().dim(1);
  need(x.numel() == n && x.dtype() == DType::F32, k + ": parameter `x` must be f32 [" +
                                                      std::to_string(n) + "]");
  need(norm_weight.numel() == n, k + ": parameter `norm` must have " + std::to_string(n) +
                                     " elements");
  need(out.numel() == d && out.dtype() == DType::F32,
       k + ": parameter `out` must be f32 [" + std::to_string(d) + "]");
  ammon_runtime *rt = s.runtime().raw();
  s.record("linear", [=](ammon_stream stream) {
    return ammon_gemv_rmsnorm(rt, stream, (const float *)x.data(), norm_weight.data(),
                              abi(norm_weight.dtype()), eps, weight.data(), abi(weight.dtype()), d,
                              n, (float *)out.data());
  });
}

// ---- CausalAttentionBlock ---------------------------------------------------------------------
CausalAttentionBlock::CausalAttentionBlock(const Runtime &rt, uint32_t hidden, uint32_t query_heads,
                                           uint32_t seq_len, AttentionOptions opts)
    : rt_(rt), hidden_(hidden), q_heads_(query_heads), seq_(seq_len), opts_(opts) {
  // reference src/modules.rs:209-211
  if (query_heads == 0 || hidden % query_heads != 0) {
    std::ostringstream os;
    os << "hidden " << hidden << " is not divisible by query_heads " << query_heads;
    fail(os.str());
  }
  need(seq_len > 0, "CausalAttentionBlock: seq_len must be positive");
  head_ = hidden / query_heads;
  need(head_ <= AMMON_ATTENTION_MAX_HEAD, "attention: head size " + std::to_string(head_) +
                                              " exceeds " +
                                              std::to_string(AMMON_ATTENTION_MAX_HEAD));
  need(head_ % 2 == 0, "attention: head size " + std::to_string(head_) + " must be even for RoPE");
  xb_ = Tensor::zeros(rt, Shape::from_dims({query_heads, head_}), DType::F32);
  q_ = Tensor::zeros(rt, Shape::from_dims({query_heads, head_}), DType::F32);
  // Scratch for the most splits any shape will use: the split length grows
  // with kv_heads and with fewer units per CU, so kv_heads = 1 at two units
  // per CU bounds the count.
  const uint32_t min_split =
      opts_.split_len ? opts_.split_len : ammon_attention_default_split(rt.raw(), 1, seq_len);
  max_splits_ = ammon_attention_splits(seq_len, min_split);
  partial_ = Tensor::zeros(rt, Shape::from_dims({query_heads, max_splits_, head_ + 2}), DType::F32);
  table_ = kernels::rope_table(rt, opts.theta, head_, seq_len);
}

uint32_t CausalAttentionBlock::split_len_for(uint32_t kv_heads, DType kv_dtype) const {
  if (opts_.split_len) return opts_.split_len;
  return ammon_attention_default_split_for(rt_.raw(), q_heads_, kv_heads, head_,
                                           (ammon_dtype)kv_dtype, seq_);
}

void CausalAttentionBlock::record(Scheme &s, TensorView x, const CausalAttentionBlockWeights &w,
                                  const KvLayer &cache, const Tensor &step) const {
  // Shape contract (reference src/blocks.rs:183-215).
  const std::string k = "attention";
  need(x.shape().rank() == 1 && x.numel() == hidden_ && x.dtype() == DType::F32,
       k + ": parameter `x` must be f32 [" + std::to_string(hidden_) + "], got " + dims(x));
  need(w.query.shape().rank() == 2 && w.key.shape().rank() == 2 && w.value.shape().rank() == 2 &&
           w.output.shape().rank() == 2,
       k + ": projection weights must be rank 2");
  const uint32_t q_dim = q_heads_ * head_;
  need(w.query.shape().dim(0) == q_dim && w.query.shape().dim(1) == hidden_,
       k + ": parameter `wq` must be [" + std::to_string(q_dim) + ", " + std::to_string(hidden_) +
           "], got " + dims(w.query));
  const uint32_t kv_dim = w.key.shape().dim(0);
  need(w.value.shape().dim(0) == kv_dim, "attention: wk and wv row counts differ");
  need(kv_dim <= q_dim && kv_dim % 2 == 0, "attention: kv width must be even and no wider than q");
  need(w.key.shape().dim(1) == hidden_ && w.value.shape().dim(1) == hidden_,
       k + ": wk / wv must have " + std::to_string(hidden_) + " columns");
  need(w.output.shape().dim(0) == hidden_ && w.output.shape().dim(1) == q_dim,
       k + ": parameter `wo` must be [" + std::to_string(hidden_) + ", " + std::to_string(q_dim) +
           "], got " + dims(w.output));
  need(w.query.dtype() == w.key.dtype() && w.key.dtype() == w.value.dtype(),
       k + ": wq, wk and wv must share a dtype");
  need(w.norm.numel() == hidden_, k + ": parameter `norm` must have " + std::to_string(hidden_) +
                                      " elements");
  need(kv_dim % head_ == 0, k + ": kv width " + std::to_string(kv_dim) +
                                " is not a multiple of head " + std::to_string(head_));
  const uint32_t kv_heads = kv_dim / head_;
  const std::vector<uint32_t> cache_dims = {kv_heads, seq_, head_};
  need(cache.key.shape() == Shape::from_dims(cache_dims) && cache.value.shape() == cache.key.shape(),
       k + ": cache layer must be [" + std::to_string(kv_heads) + ", " + std::to_string(seq_) +
           ", " + std::to_string(head_) + "] (kv_heads, seq, head), got " + dims(cache.key));
  need(cache.key.dtype() == cache.value.dtype(), k + ": key and value caches differ in dtype");
  need(step.nbytes() >= sizeof(ammon_decode_step), k + ": parameter `step` is not a DecodeStep");
  const uint32_t split = split_len_for(kv_heads, cache.key.dtype());
  need(ammon_attention_splits(seq_, split) <= max_splits_, k + ": split scratch too small");

  ammon_runtime *rt = s.runtime().raw();
  const auto *st = (const ammon_decode_step *)step.data();
  const uint32_t hidden = hidden_, q_heads = q_heads_, head = head_, seq = seq_;
  const float eps = opts_.eps;
  float *q = (float *)q_.data();
  float *xb = (float *)xb_.data();
  float *partial = (float *)partial_.data();
  const size_t partial_bytes = partial_.nbytes();
  const float *table = (const float *)table_->data();
  s.record("qkv_rope_store", [=](ammon_stream stream) {
    return ammon_qkv_rope_store(rt, stream, (const float *)x.data(), w.norm.data(),
                                abi(w.norm.dtype()), eps, w.query.data(), w.key.data(),
                                w.value.data(), abi(w.query.dtype()), hidden, q_heads, kv_heads,
                                head, q, cache.key.data(), cache.value.data(),
                                abi(cache.key.dtype()), seq, st, table);
  });
  if (ammon_attention_splits(seq, split) == 1) {
    // one split covers the cache: pass 1 writes the output, no merge launch
    s.record("attention", [=](ammon_stream stream) {
      return ammon_attention_decode(rt, stream, q, q_heads, cache.key.data(), cache.value.data(),
                                    abi(cache.key.dtype()), kv_heads, head, seq, st, split,
                                    partial, partial_bytes, xb);
    });
  } else {
    s.record("attn_partial", [=](ammon_stream stream) {
      return ammon_attention_partial(rt, stream, q, q_heads, cache.key.data(), cache.value.data(),
                                     abi(cache.key.dtype()), kv_heads, head, seq, st, split,
                                     partial);
    });
    // the merge also brings the first tile of wo's rows into L2 for the
    // output projection that follows, from position 4096 on (measured at the
    // Llama-3-8B shape: 12-13 us per token gained at 4096 and 8000 positions,
    // 37-64 us lost at 2048 and below)
    const void *wo = w.output.data();
    const ammon_dtype wo_dt = abi(w.output.dtype());
    s.record("attn_combine", [=](ammon_stream stream) {
      return ammon_attention_combine_warm(rt, stream, partial, q_heads, head, seq, st, split, xb,
                                          wo, wo_dt, hidden, q_heads * head, 0, 4096);
    });
  }
  s.record("wo_residual", [=](ammon_stream stream) {
    return ammon_gemv(rt, stream, w.output.data(), abi(w.output.dtype()), hidden, q_heads * head,
                      xb, (float *)x.data(), (const float *)x.data());
  });
}

void CausalAttentionBlock::record_group(Scheme &s, const std::string &label, TensorView x,
                                        const CausalAttentionBlockWeights &w, const KvLayer &cache,
                                        const Tensor &step) const {
  s.group(label, [&](Scheme &g) { record(g, x, w, cache, step); });
}

// ---- SwiGluBlock ------------------------------------------------------------------------------
SwiGluBlock::SwiGluBlock(const Runtime &rt, uint32_t hidden, uint32_t intermediate, float eps)
    : rt_(rt), hidden_(hidden), inter_(intermediate), eps_(eps) {
  need(hidden > 0 && intermediate > 0, "SwiGluBlock: empty shape");
  hb_ = Tensor::zeros(rt, Shape::vector(intermediate), DType::F32);
}

void SwiGluBlock::record(Scheme &s, TensorView x, const SwiGluBlockWeights &w) const {
  const std::string k = "ffn";
  need(x.shape().rank() == 1 && x.numel() == hidden_ && x.dtype() == DType::F32,
       k + ": parameter `x` must be f32 [" + std::to_string(hidden_) + "], got " + dims(x));
  const Shape up_shape = Shape::from_dims({inter_, hidden_});
  need(w.gate.shape() == up_shape, k + ": parameter `w1` must be " + up_shape.str() + ", got " +
                                       dims(w.gate));
  need(w.up.shape() == up_shape, k + ": parameter `w3` must be " + up_shape.str() + ", got " +
                                     dims(w.up));
  need(w.down.shape() == Shape::from_dims({hidden_, inter_}),
       k + ": parameter `w2` must be [" + std::to_string(hidden_) + ", " + std::to_string(inter_) +
           "], got " + dims(w.down));
  need(w.gate.dtype() == w.up.dtype(), k + ": w1 and w3 must share a dtype");
  need(w.norm.numel() == hidden_, k + ": parameter `norm` must have " + std::to_string(hidden_) +
                                      " elements");
  ammon_runtime *rt = s.runtime().raw();
  const uint32_t hidden = hidden_, inter = inter_;
  const float eps = eps_;
  float *hb = (float *)hb_.data();
  s.record("gate_up_swiglu", [=](ammon_stream stream) {
    return ammon_gate_up_swiglu(rt, stream, (const float *)x.data(), w.norm.data(),
                                abi(w.norm.dtype()), eps, w.gate.data(), w.up.data(),
                                abi(w.gate.dtype()), hidden, inter, hb);
  });
  s.record("w2_residual", [=](ammon_stream stream) {
    return ammon_gemv(rt, stream, w.down.data(), abi(w.down.dtype()), hidden, inter, hb,
                      (float *)x.data(), (const float *)x.data());
  });
}

void SwiGluBlock::record_group(Scheme &s, const std::string &label, TensorView x,
                               const SwiGluBlockWeights &w) const {
  s.group(label, [&](Scheme &g) { record(g, x, w); });
}

}  // namespace ammon
