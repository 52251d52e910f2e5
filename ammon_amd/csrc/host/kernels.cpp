// kernels.cpp -- the kernel-recorder tier of the C++ host layer.
//
// Each recorder checks the reference kernel's tensor contract (the
// `#[tensor(shape = [...])]` declarations of src/kernels.rs: rank and symbol
// agreement, reported as "<kernel>: parameter `p`: ...") and records one
// C-ABI launch.  Validation runs before the scheme changes.
#include <map>
#include <mutex>
#include <sstream>
#include <tuple>

#include "ammon/ammon.hpp"

namespace ammon {
namespace {

[[noreturn]] void fail(const std::string &msg) { throw Error(AMMON_E_VALIDATION, msg); }

void expect_rank(const std::string &k, const TensorView &v, const char *param, size_t rank) {
  if (v.shape().rank() != rank) {
    std::ostringstream os;
    os << k << ": parameter `" << param << "`: expected rank " << rank << ", got rank "
       << v.shape().rank() << " " << v.shape().str();
    fail(os.str());
  }
}

void expect_dim(const std::string &k, const TensorView &v, const char *param, size_t axis,
                const char *symbol, uint32_t want) {
  if (v.shape().dim(axis) != want) {
    std::ostringstream os;
    os << k << ": parameter `" << param << "`: dimension " << axis << " (`" << symbol << "`) is "
       << v.shape().dim(axis) << ", expected " << want;
    fail(os.str());
  }
}

void expect_float(const std::string &k, const TensorView &v, const char *param) {
  if (v.dtype() != DType::F32 && v.dtype() != DType::BF16)
    fail(k + ": parameter `" + std::string(param) + "` must be f32 or bf16");
}

void expect_f32(const std::string &k, const TensorView &v, const char *param) {
  if (v.dtype() != DType::F32) fail(k + ": parameter `" + std::string(param) + "` must be f32");
}

void expect_step(const std::string &k, const Tensor &step) {
  if (step.nbytes() < sizeof(ammon_decode_step)) fail(k + ": parameter `step` is not a DecodeStep");
}

ammon_dtype abi(DType d) { return (ammon_dtype)d; }

const ammon_decode_step *step_ptr(const Tensor &step) {
  return (const ammon_decode_step *)step.data();
}

}  // namespace

namespace kernels {

void embed(Scheme &s, const std::string &label, TensorView table, const Tensor &step, TensorView x) {
  const std::string k = "embed";
  expect_rank(k, table, "embed", 2);
  expect_rank(k, x, "x", 1);
  expect_dim(k, x, "x", 0, "dim", table.shape().dim(1));
  expect_float(k, table, "embed");
  expect_f32(k, x, "x");
  expect_step(k, step);
  ammon_runtime *rt = s.runtime().raw();
  const auto *st = step_ptr(step);
  const uint32_t vocab = table.shape().dim(0), dim = table.shape().dim(1);
  s.record(label, [=](ammon_stream stream) {
    return ammon_embed(rt, stream, table.data(), abi(table.dtype()), vocab, dim, st,
                       (float *)x.data());
  });
}

void gemv(Scheme &s, const std::string &label, TensorView x, TensorView w, TensorView xout,
          const Tensor &step) {
  const std::string k = "gemv";
  expect_rank(k, x, "x", 1);
  expect_rank(k, w, "w", 2);
  expect_rank(k, xout, "xout", 2);
  const uint32_t d = w.shape().dim(0), n = w.shape().dim(1);
  expect_dim(k, x, "x", 0, "n", n);
  expect_dim(k, xout, "xout", 1, "d", d);
  expect_f32(k, x, "x");
  expect_float(k, w, "w");
  expect_f32(k, xout, "xout");
  expect_step(k, step);
  ammon_runtime *rt = s.runtime().raw();
  const auto *st = step_ptr(step);
  const uint32_t seq = xout.shape().dim(0);
  s.record(label, [=](ammon_stream stream) {
    return ammon_gemv_at_position(rt, stream, w.data(), abi(w.dtype()), d, n,
                                  (const float *)x.data(), (float *)xout.data(), seq, st);
  });
}

static void rms_common(Scheme &s, const std::string &label, const std::string &k, TensorView x,
                       TensorView weight, TensorView out, float eps) {
  if (x.shape().rank() != 1 && x.shape().rank() != 2) expect_rank(k, x, "x", 1);
  const uint32_t dim = x.shape().dim(x.shape().rank() - 1);
  const uint32_t rows = x.shape().rank() == 2 ? x.shape().dim(0) : 1;
  expect_rank(k, weight, "weight", 1);
  expect_dim(k, weight, "weight", 0, "dim", dim);
  if (!(out.shape() == x.shape())) fail(k + ": parameter `o`: shape " + out.shape().str() +
                                        " differs from `x` " + x.shape().str());
  expect_f32(k, x, "x");
  expect_f32(k, out, "o");
  expect_float(k, weight, "weight");
  ammon_runtime *rt = s.runtime().raw();
  s.record(label, [=](ammon_stream stream) {
    return ammon_rmsnorm(rt, stream, (const float *)x.data(), weight.data(), abi(weight.dtype()),
                         (float *)out.data(), rows, dim, eps);
  });
}

void rmsnorm(Scheme &s, const std::string &label, TensorView x, TensorView weight, TensorView out,
             float eps) {
  rms_common(s, label, "rmsnorm", x, weight, out, eps);
}

void rmsnorm_inplace(Scheme &s, const std::string &label, TensorView x, TensorView weight,
                     float eps) {
  rms_common(s, label, "rmsnorm_inplace", x, weight, x, eps);
}

static void check_rope(const std::string &k, const TensorView &q, const TensorView &cache,
                       const TensorView &table) {
  expect_rank(k, q, "q", 2);
  expect_rank(k, cache, "k", 3);
  const uint32_t head = q.shape().dim(1);
  expect_dim(k, cache, "k", 2, "head", head);
  expect_rank(k, table, "table", 3);
  expect_dim(k, table, "table", 0, "seq", cache.shape().dim(1));
  expect_dim(k, table, "table", 1, "head / 2", head / 2);
  expect_f32(k, q, "q");
  expect_f32(k, table, "table");
  expect_float(k, cache, "k");
}

void rope(Scheme &s, const std::string &label, TensorView q, TensorView kc, const Tensor &step,
          TensorView table) {
  const std::string k = "rope";
  check_rope(k, q, kc, table);
  expect_step(k, step);
  ammon_runtime *rt = s.runtime().raw();
  const auto *st = step_ptr(step);
  const uint32_t q_heads = q.shape().dim(0), head = q.shape().dim(1);
  const uint32_t kv_heads = kc.shape().dim(0), seq = kc.shape().dim(1);
  s.record(label, [=](ammon_stream stream) {
    return ammon_rope(rt, stream, (float *)q.data(), q_heads, kv_heads, head, kc.data(),
                      abi(kc.dtype()), seq, st, (const float *)table.data());
  });
}

void rope_store(Scheme &s, const std::string &label, TensorView q, TensorView k_proj,
                TensorView kc, const Tensor &step, TensorView table) {
  const std::string k = "rope_store";
  check_rope(k, q, kc, table);
  expect_rank(k, k_proj, "k_proj", 1);
  expect_dim(k, k_proj, "k_proj", 0, "kv_dim", kc.shape().dim(0) * kc.shape().dim(2));
  expect_f32(k, k_proj, "k_proj");
  expect_step(k, step);
  ammon_runtime *rt = s.runtime().raw();
  const auto *st = step_ptr(step);
  const uint32_t q_heads = q.shape().dim(0), head = q.shape().dim(1);
  const uint32_t kv_heads = kc.shape().dim(0), seq = kc.shape().dim(1);
  s.record(label, [=](ammon_stream stream) {
    return ammon_rope_store(rt, stream, (float *)q.data(), q_heads, (const float *)k_proj.data(),
                            kv_heads, head, kc.data(), abi(kc.dtype()), seq, st,
                            (const float *)table.data());
  });
}

void cache_store(Scheme &s, const std::string &label, TensorView src, TensorView dst,
                 const Tensor &step) {
  const std::string k = "cache_store";
  expect_rank(k, src, "src", 1);
  expect_rank(k, dst, "dst", 3);
  expect_dim(k, src, "src", 0, "kv_dim", dst.shape().dim(0) * dst.shape().dim(2));
  expect_f32(k, src, "src");
  expect_float(k, dst, "dst");
  expect_step(k, step);
  ammon_runtime *rt = s.runtime().raw();
  const auto *st = step_ptr(step);
  const uint32_t kv_heads = dst.shape().dim(0), seq = dst.shape().dim(1),
                 head = dst.shape().dim(2);
  s.record(label, [=](ammon_stream stream) {
    return ammon_cache_store(rt, stream, (const float *)src.data(), kv_heads, head, dst.data(),
                             abi(dst.dtype()), seq, st);
  });
}

void attention_partial(Scheme &s, const std::string &label, TensorView q, TensorView key,
                       TensorView value, TensorView partial, const Tensor &step,
                       uint32_t split_len) {
  const std::string k = "attention_partial";
  expect_rank(k, q, "q", 2);
  expect_rank(k, key, "key_cache", 3);
  expect_rank(k, value, "value_cache", 3);
  expect_rank(k, partial, "partial", 3);
  const uint32_t q_heads = q.shape().dim(0), head = q.shape().dim(1);
  const uint32_t kv_heads = key.shape().dim(0), seq = key.shape().dim(1);
  expect_dim(k, key, "key_cache", 2, "head", head);
  if (!(value.shape() == key.shape()) || value.dtype() != key.dtype())
    fail(k + ": parameter `value_cache` differs from `key_cache`");
  expect_dim(k, partial, "partial", 0, "q_heads", q_heads);
  expect_dim(k, partial, "partial", 1, "splits", ammon_attention_splits(seq, split_len));
  expect_dim(k, partial, "partial", 2, "slot", head + 2);
  expect_f32(k, q, "q");
  expect_f32(k, partial, "partial");
  expect_step(k, step);
  ammon_runtime *rt = s.runtime().raw();
  const auto *st = step_ptr(step);
  s.record(label, [=](ammon_stream stream) {
    return ammon_attention_partial(rt, stream, (const float *)q.data(), q_heads, key.data(),
                                   value.data(), abi(key.dtype()), kv_heads, head, seq, st,
                                   split_len, (float *)partial.data());
  });
}

void attention_combine(Scheme &s, const std::string &label, TensorView partial, TensorView out,
                       const Tensor &step, uint32_t seq, uint32_t split_len) {
  const std::string k = "attention_combine";
  expect_rank(k, partial, "partial", 3);
  expect_rank(k, out, "xb", 2);
  const uint32_t q_heads = out.shape().dim(0), head = out.shape().dim(1);
  expect_dim(k, partial, "partial", 0, "q_heads", q_heads);
  expect_dim(k, partial, "partial", 1, "splits", ammon_attention_splits(seq, split_len));
  expect_dim(k, partial, "partial", 2, "slot", head + 2);
  expect_f32(k, partial, "partial");
  expect_f32(k, out, "xb");
  expect_step(k, step);
  ammon_runtime *rt = s.runtime().raw();
  const auto *st = step_ptr(step);
  s.record(label, [=](ammon_stream stream) {
    return ammon_attention_combine(rt, stream, (const float *)partial.data(), q_heads, head, seq,
                                   st, split_len, (float *)out.data());
  });
}

void swiglu(Scheme &s, const std::string &label, TensorView hb, TensorView hb2) {
  const std::string k = "swiglu";
  expect_rank(k, hb, "hb", 1);
  expect_rank(k, hb2, "hb2", 1);
  expect_dim(k, hb2, "hb2", 0, "hidden", hb.shape().dim(0));
  expect_f32(k, hb, "hb");
  expect_f32(k, hb2, "hb2");
  ammon_runtime *rt = s.runtime().raw();
  const uint32_t n = hb.numel_u32();
  s.record(label, [=](ammon_stream stream) {
    return ammon_swiglu(rt, stream, (float *)hb.data(), (const float *)hb2.data(), n);
  });
}

void argmax(Scheme &s, const std::string &label, TensorView logits, TensorView scratch,
            TensorView out) {
  const std::string k = "argmax";
  expect_rank(k, logits, "logits", 1);
  expect_f32(k, logits, "logits");
  const uint32_t n = logits.numel_u32();
  if (scratch.nbytes() < ammon_argmax_scratch_bytes(n)) fail(k + ": scratch too small");
  if (out.nbytes() < 4) fail(k + ": parameter `out` is empty");
  ammon_runtime *rt = s.runtime().raw();
  s.record(label, [=](ammon_stream stream) {
    return ammon_argmax(rt, stream, (const float *)logits.data(), n, scratch.data(),
                        (int32_t *)out.data());
  });
}

void greedy_next(Scheme &s, const std::string &label, TensorView logits, TensorView scratch,
                 TensorView prompt, uint32_t n_prompt, const Tensor &step, TensorView tokens) {
  const std::string k = "greedy_next";
  expect_rank(k, logits, "logits", 1);
  expect_f32(k, logits, "logits");
  expect_step(k, step);
  const uint32_t n = logits.numel_u32();
  if (scratch.nbytes() < ammon_argmax_scratch_bytes(n)) fail(k + ": scratch too small");
  if (prompt.numel() < n_prompt) fail(k + ": prompt shorter than n_prompt");
  ammon_runtime *rt = s.runtime().raw();
  ammon_decode_step *st = (ammon_decode_step *)step.data();
  const uint32_t max_tokens = tokens.numel_u32();
  s.record(label, [=](ammon_stream stream) {
    return ammon_greedy_next(rt, stream, (const float *)logits.data(), n, scratch.data(),
                             (const int32_t *)prompt.data(), n_prompt, st,
                             (int32_t *)tokens.data(), max_tokens);
  });
}

void greedy_lm_head(Scheme &s, const std::string &label, TensorView weight, TensorView x,
                    TensorView norm_weight, TensorView logits, TensorView scratch,
                    TensorView prompt, uint32_t n_prompt, const Tensor &step, TensorView tokens,
                    float eps) {
  const std::string k = "greedy_lm_head";
  expect_rank(k, weight, "weight", 2);
  expect_f32(k, x, "x");
  expect_f32(k, logits, "logits");
  expect_step(k, step);
  const uint32_t d = weight.shape().dim(0), n = weight.shape().dim(1);
  if (x.numel() != n) fail(k + ": parameter `x` must have " + std::to_string(n) + " elements");
  if (norm_weight.numel() != n)
    fail(k + ": parameter `norm` must have " + std::to_string(n) + " elements");
  if (logits.numel() != d) fail(k + ": parameter `logits` must have " + std::to_string(d) + " elements");
  ammon_runtime *rt = s.runtime().raw();
  if (scratch.nbytes() < ammon_greedy_lm_head_scratch_bytes(rt)) fail(k + ": scratch too small");
  if (prompt.numel() < n_prompt) fail(k + ": prompt shorter than n_prompt");
  ammon_decode_step *st = (ammon_decode_step *)step.data();
  const uint32_t max_tokens = tokens.numel_u32();
  const ammon_dtype wd = weight.dtype() == DType::BF16 ? AMMON_BF16 : AMMON_F32;
  const ammon_dtype nd = norm_weight.dtype() == DType::BF16 ? AMMON_BF16 : AMMON_F32;
  const size_t scratch_bytes = scratch.nbytes();
  s.record(label, [=](ammon_stream stream) {
    return ammon_greedy_lm_head(rt, stream, (const float *)x.data(), norm_weight.data(), nd, eps,
                                weight.data(), wd, d, n, (float *)logits.data(), scratch.data(),
                                scratch_bytes, (const int32_t *)prompt.data(), n_prompt, st,
                                (int32_t *)tokens.data(), max_tokens);
  });
}

std::shared_ptr<Tensor> rope_table(const Runtime &rt, float theta, uint32_t head, uint32_t seq) {
  // Shared per (device, theta, head, seq) like the reference's prepared
  // kernels (weak entries; the table is freed with its last user).
  using Key = std::tuple<int, float, uint32_t, uint32_t>;
  static std::mutex mu;
  static std::map<Key, std::weak_ptr<Tensor>> cache;
  std::lock_guard<std::mutex> lock(mu);
  const Key key{rt.info().device, theta, head, seq};
  auto it = cache.find(key);
  if (it != cache.end())
    if (auto t = it->second.lock()) return t;
  std::vector<float> host(ammon_rope_table_bytes(head, seq) / sizeof(float));
  check(ammon_rope_table_host(theta, head, seq, host.data()), "rope table");
  auto t = std::make_shared<Tensor>(
      Tensor::from_host(rt, Shape::from_dims({seq, head / 2, 2}), DType::F32, host.data()));
  cache[key] = t;
  return t;
}

}  // namespace kernels

// ---- TensorKernels ------------------------------------------------------------------------
TensorKernels TensorKernels::prepare(const Runtime &rt) {
  if (!rt) throw Error(AMMON_E_VALIDATION, "TensorKernels::prepare: no runtime");
  return TensorKernels{};
}

void TensorKernels::add_into(Scheme &s, const std::string &label, TensorView a, TensorView b,
                             TensorView out) const {
  const std::string k = "add";
  if (!(a.shape() == b.shape()) || !(a.shape() == out.shape()))
    fail(k + ": operands " + a.shape().str() + ", " + b.shape().str() + " -> " +
         out.shape().str() + " differ");
  expect_f32(k, a, "a");
  expect_f32(k, b, "b");
  expect_f32(k, out, "out");
  ammon_runtime *rt = s.runtime().raw();
  const uint32_t n = a.numel_u32();
  s.record(label, [=](ammon_stream stream) {
    return ammon_add(rt, stream, (const float *)a.data(), (const float *)b.data(),
                     (float *)out.data(), n);
  });
}

void TensorKernels::matmul_into(Scheme &s, const std::string &label, TensorView a, TensorView b,
                                TensorView out) const {
  const std::string k = "matmul";
  expect_rank(k, a, "a", 2);
  const uint32_t d = a.shape().dim(0), n = a.shape().dim(1);
  if (b.numel() != n) fail(k + ": parameter `b` has " + std::to_string(b.numel()) +
                           " elements, expected `n` = " + std::to_string(n));
  if (out.numel() != d) fail(k + ": parameter `out` has " + std::to_string(out.numel()) +
                             " elements, expected `d` = " + std::to_string(d));
  expect_float(k, a, "a");
  expect_f32(k, b, "b");
  expect_f32(k, out, "out");
  ammon_runtime *rt = s.runtime().raw();
  s.record(label, [=](ammon_stream stream) {
    return ammon_gemv(rt, stream, a.data(), abi(a.dtype()), d, n, (const float *)b.data(),
                      (float *)out.data(), nullptr);
  });
}

}  // namespace ammon
