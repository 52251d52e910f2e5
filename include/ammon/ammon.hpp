// ammon.hpp -- C++ host layer mirroring koubaa/ammon's public API over the
// C ABI in ammon.h.
//
// Reference surface -> here:
//   gpu::create_runtime (src/gpu.rs:6-13)          -> ammon::create_runtime
//   goldy Tensor / TensorView / TensorShape          -> ammon::Tensor / TensorView / Shape
//   goldy Scheme record / submit / replay            -> ammon::Scheme (launch list, replayed
//                                                       as a HIP graph)
//   kernels::DecodeStep (src/kernels.rs:10-33)        -> ammon::DecodeStep
//   kernels::*Kernel::record (src/kernels.rs)         -> ammon::kernels::* recorders
//   kernels::TensorKernels (src/kernels.rs:490-534)   -> ammon::TensorKernels
//   modules::* (src/modules.rs:1-333)                 -> ammon::Embedding, RmsNorm, Linear,
//                                                       CausalAttentionBlock, SwiGluBlock,
//                                                       KvCache, KvLayer, *Weights
//   model::AutoregressiveModel (src/model.rs:7-11)    -> ammon::AutoregressiveModel
//   generate::generate_tokens (src/generate.rs:43-91) -> ammon::generate_tokens
//   tokenizer::sample_argmax (src/tokenizer.rs:179)   -> ammon::sample_argmax
//
// Errors are thrown as ammon::Error (the reference's GoldyError / anyhow
// results).  A failed record throws before the scheme changes, as a failed
// Goldy record leaves the IR node count unchanged.
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "ammon/ammon.h"

namespace ammon {

class Error : public std::runtime_error {
 public:
  Error(ammon_status status, const std::string &msg) : std::runtime_error(msg), status_(status) {}
  ammon_status status() const { return status_; }

 private:
  ammon_status status_;
};

// Throws ammon::Error with the library's message when `st` is not AMMON_OK.
void check(ammon_status st, const std::string &context = {});

// Storage dtypes.  F32 / BF16 are the ABI's ammon_dtype values; U32 / I32
// are host-layer index types (DecodeStep parcels, token ids).
enum class DType { F32 = AMMON_F32, BF16 = AMMON_BF16, U32 = 2, I32 = 3 };
size_t dtype_size(DType d);

// ---- runtime -----------------------------------------------------------------
// A shared handle to the per-device ammon_runtime (prepared kernels, stream).
class Runtime {
 public:
  Runtime() = default;
  static Runtime create(int device = 0);
  ammon_runtime *raw() const { return rt_.get(); }
  explicit operator bool() const { return (bool)rt_; }
  const ammon_device_info &info() const { return info_; }
  bool operator==(const Runtime &o) const { return rt_ == o.rt_; }

 private:
  std::shared_ptr<ammon_runtime> rt_;
  ammon_device_info info_ = {};
};

Runtime create_runtime(int device = 0);

// ---- tensors -------------------------------------------------------------------
struct Shape {
  std::vector<uint32_t> dims;

  static Shape vector(uint32_t n) { return Shape{{n}}; }
  static Shape matrix(uint32_t rows, uint32_t cols) { return Shape{{rows, cols}}; }
  static Shape from_dims(std::vector<uint32_t> d);
  size_t rank() const { return dims.size(); }
  uint32_t dim(size_t i) const;
  uint64_t numel() const;
  std::string str() const;
  bool operator==(const Shape &o) const { return dims == o.dims; }
};

// Non-owning device view: pointer, shape, storage dtype.
class TensorView {
 public:
  TensorView() = default;
  TensorView(void *ptr, Shape shape, DType dtype) : ptr_(ptr), shape_(std::move(shape)), dtype_(dtype) {}
  void *data() const { return ptr_; }
  const Shape &shape() const { return shape_; }
  DType dtype() const { return dtype_; }
  uint64_t numel() const { return shape_.numel(); }
  uint32_t numel_u32() const;
  size_t nbytes() const { return numel() * dtype_size(dtype_); }
  // Sub-range [start, start + len) along `axis` of a contiguous view
  // (Goldy TensorView::narrow).
  TensorView narrow(size_t axis, uint32_t start, uint32_t len) const;
  // Same storage, new dims with the same element count (TensorView::reshape).
  TensorView reshape(std::vector<uint32_t> dims) const;

 private:
  void *ptr_ = nullptr;
  Shape shape_;
  DType dtype_ = DType::F32;
};

// Owning device tensor (Goldy Tensor).  Move-only; freed on destruction.
class Tensor {
 public:
  Tensor() = default;
  Tensor(Tensor &&o) noexcept;
  Tensor &operator=(Tensor &&o) noexcept;
  Tensor(const Tensor &) = delete;
  Tensor &operator=(const Tensor &) = delete;
  ~Tensor();

  static Tensor zeros(const Runtime &rt, Shape shape, DType dtype);
  static Tensor from_f32(const Runtime &rt, Shape shape, const std::vector<float> &data);
  static Tensor from_host(const Runtime &rt, Shape shape, DType dtype, const void *data);

  TensorView view() const { return TensorView(ptr_, shape_, dtype_); }
  void *data() const { return ptr_; }
  const Shape &shape() const { return shape_; }
  DType dtype() const { return dtype_; }
  size_t nbytes() const { return shape_.numel() * dtype_size(dtype_); }
  // Synchronous copies (the reference's submit + host take).
  std::vector<float> to_f32() const;
  void to_host(void *dst) const;
  void upload(const void *src);

 private:
  Runtime rt_;
  void *ptr_ = nullptr;
  Shape shape_;
  DType dtype_ = DType::F32;
};

// ---- control parcel --------------------------------------------------------------
// DecodeStep (reference src/kernels.rs:10-33): {token, position} in device
// memory, rewritten per step by a deposit so recorded launches never change.
struct DecodeStep {
  uint32_t token = 0;
  uint32_t position = 0;

  // A one-element device parcel initialised to {0, 0} (DecodeStep::parcel).
  static Tensor parcel(const Runtime &rt);
  // Asynchronous deposit into `parcel` on `stream` (MemoryExchange deposit).
  static void deposit(const Runtime &rt, const Tensor &parcel, DecodeStep value,
                      ammon_stream stream = nullptr);
  static DecodeStep read(const Runtime &rt, const Tensor &parcel);
};

// ---- scheme ------------------------------------------------------------------------
// A recorded launch list.  record() validates the launch immediately (nothing
// is kept if it throws) and appends it; submit() replays the list on the
// scheme's stream -- captured into a HIP graph the first time and relaunched
// as that graph afterwards (the reference's record-once / replay-many).
class Scheme {
 public:
  using Launch = std::function<ammon_status(ammon_stream)>;

  // Replays on `stream` when given (not owned), else on a stream of its own.
  explicit Scheme(const Runtime &rt, bool use_graph = true, ammon_stream stream = nullptr);
  ~Scheme();
  Scheme(const Scheme &) = delete;
  Scheme &operator=(const Scheme &) = delete;

  void record(const std::string &label, Launch launch);
  // Records `fn`'s launches under a group label (Scheme::group).
  void group(const std::string &label, const std::function<void(Scheme &)> &fn);
  void submit();
  void synchronize();

  size_t ir_node_count() const { return nodes_.size(); }
  const std::vector<std::string> &labels() const { return labels_; }
  const Runtime &runtime() const { return rt_; }
  ammon_stream stream() const { return stream_; }

  struct ReplayStats {
    size_t records = 0;        // launches recorded
    size_t captures = 0;       // graph (re)captures
    size_t submits = 0;        // submits
  };
  const ReplayStats &replay_stats() const { return stats_; }

 private:
  void drop_graph();

  Runtime rt_;
  ammon_stream stream_ = nullptr;
  bool owns_stream_ = false;
  bool use_graph_;
  ammon_graph graph_ = nullptr;
  std::vector<Launch> nodes_;
  std::vector<std::string> labels_;
  std::string prefix_;
  ReplayStats stats_;
};

// ---- kernel recorders --------------------------------------------------------------
// The reference's `<Kernel>::prepare(runtime)?.record(scheme, label, ...)`
// tier.  Each validates the tensor shape contract (rank / symbol agreement,
// messages naming the parameter and the symbol) and records one C-ABI launch.
namespace kernels {
void embed(Scheme &s, const std::string &label, TensorView table, const Tensor &step, TensorView x);
// Position-strided serial-definition GEMV (src/kernels.rs:49-73):
// xout[step.position, :] = w x, with x [n], w [d, n], xout [seq, d].
void gemv(Scheme &s, const std::string &label, TensorView x, TensorView w, TensorView xout,
          const Tensor &step);
void rmsnorm(Scheme &s, const std::string &label, TensorView x, TensorView weight, TensorView out,
             float eps = 1e-5f);
void rmsnorm_inplace(Scheme &s, const std::string &label, TensorView x, TensorView weight,
                     float eps = 1e-5f);
void rope(Scheme &s, const std::string &label, TensorView q, TensorView k, const Tensor &step,
          TensorView table);
void rope_store(Scheme &s, const std::string &label, TensorView q, TensorView k_proj, TensorView k,
                const Tensor &step, TensorView table);
void cache_store(Scheme &s, const std::string &label, TensorView src, TensorView dst,
                 const Tensor &step);
void attention_partial(Scheme &s, const std::string &label, TensorView q, TensorView key,
                       TensorView value, TensorView partial, const Tensor &step, uint32_t split_len);
void attention_combine(Scheme &s, const std::string &label, TensorView partial, TensorView out,
                       const Tensor &step, uint32_t seq, uint32_t split_len);
void swiglu(Scheme &s, const std::string &label, TensorView hb, TensorView hb2);
void argmax(Scheme &s, const std::string &label, TensorView logits, TensorView scratch,
            TensorView out);
void greedy_next(Scheme &s, const std::string &label, TensorView logits, TensorView scratch,
                 TensorView prompt, uint32_t n_prompt, const Tensor &step, TensorView tokens);
// Final norm + LM head fused with the greedy step (ammon_greedy_lm_head):
// logits = W rmsnorm(x), then the argmax / prompt forcing / DecodeStep
// update of greedy_next.
void greedy_lm_head(Scheme &s, const std::string &label, TensorView weight, TensorView x,
                    TensorView norm_weight, TensorView logits, TensorView scratch,
                    TensorView prompt, uint32_t n_prompt, const Tensor &step, TensorView tokens,
                    float eps);
// Host cos/sin table for RoPE with the reference's fp32 formula, cached per
// (device, theta, head, seq) and shared by every block that asks for it.
std::shared_ptr<Tensor> rope_table(const Runtime &rt, float theta, uint32_t head, uint32_t seq);
}  // namespace kernels

// Goldy add / semantic matmul (reference kernels::TensorKernels).
class TensorKernels {
 public:
  static TensorKernels prepare(const Runtime &rt);
  // out = a + b
  void add_into(Scheme &s, const std::string &label, TensorView a, TensorView b, TensorView out) const;
  // out = a @ b with a [d, n] and b [n] (batch-1 GEMV)
  void matmul_into(Scheme &s, const std::string &label, TensorView a, TensorView b,
                   TensorView out) const;
};

// ---- modules (reference src/modules.rs) -----------------------------------------------

struct CausalAttentionBlockWeights {  // src/modules.rs:11-19
  TensorView norm, query, key, value, output;
};

struct SwiGluBlockWeights {  // src/modules.rs:21-28
  TensorView norm, gate, up, down;
};

// One layer of the KV cache.  Layout here is head-major [kv_heads, seq, head]
// (the reference's is [seq, kv_heads, head]).
struct KvLayer {  // src/modules.rs:30-35
  TensorView key, value;
};

class KvCache {  // src/modules.rs:37-71
 public:
  KvCache(const Runtime &rt, uint32_t layers, uint32_t seq_len, uint32_t kv_heads,
          uint32_t head_size, DType dtype = DType::F32);
  KvLayer layer(uint32_t layer) const;
  uint32_t layers() const { return layers_; }
  uint32_t seq_len() const { return seq_; }
  uint32_t kv_heads() const { return kv_heads_; }
  uint32_t head_size() const { return head_; }
  DType dtype() const { return dtype_; }
  // Host copy of one layer in the reference's [seq, kv_heads, head] order.
  std::vector<uint8_t> layer_to_host_reference_order(uint32_t layer, bool value) const;

 private:
  Runtime rt_;
  Tensor key_, value_;
  uint32_t layers_, seq_, kv_heads_, head_;
  DType dtype_;
};

class Embedding {  // src/modules.rs:99-132
 public:
  explicit Embedding(const Runtime &rt);
  void record(Scheme &s, TensorView table, const Tensor &step, TensorView x) const;
  void record_group(Scheme &s, const std::string &label, TensorView table, const Tensor &step,
                    TensorView x) const;

 private:
  Runtime rt_;
};

class RmsNorm {  // src/modules.rs:134-164
 public:
  explicit RmsNorm(const Runtime &rt, float eps = 1e-5f);
  void record(Scheme &s, TensorView x, TensorView weight, TensorView out) const;
  void record_inplace(Scheme &s, TensorView x, TensorView weight) const;

 private:
  Runtime rt_;
  float eps_;
};

class Linear {  // src/modules.rs:166-187
 public:
  explicit Linear(const Runtime &rt);
  void record(Scheme &s, TensorView weight, TensorView x, TensorView out) const;
  // RMSNorm prologue fused into the projection (e.g. final norm + LM head).
  void record_normed(Scheme &s, TensorView weight, TensorView x, TensorView norm_weight,
                     TensorView out, float eps = 1e-5f) const;

 private:
  Runtime rt_;
};

struct AttentionOptions {
  float theta = AMMON_DEFAULT_ROPE_THETA;  // reference hard-wires 10000 (src/blocks.rs:234)
  float eps = 1e-5f;                       // reference literal (src/kernels.rs:94)
  uint32_t split_len = 0;                  // 0: pick per device and cache shape
};

// Pre-norm causal attention block (src/modules.rs:189-274): RMSNorm, QKV,
// RoPE, attention, output projection, residual into x.  Recorded as four
// launches: norm+QKV+RoPE+KV store, split attention, LSE merge, wo +
// residual (three when one split covers the cache: the attention pass then
// writes the merged output).
class CausalAttentionBlock {
 public:
  CausalAttentionBlock(const Runtime &rt, uint32_t hidden, uint32_t query_heads, uint32_t seq_len,
                       AttentionOptions opts = {});
  void record(Scheme &s, TensorView x, const CausalAttentionBlockWeights &w, const KvLayer &cache,
              const Tensor &step) const;
  void record_group(Scheme &s, const std::string &label, TensorView x,
                    const CausalAttentionBlockWeights &w, const KvLayer &cache,
                    const Tensor &step) const;
  // The split length record() uses for a cache of kv_heads heads in kv_dtype.
  uint32_t split_len_for(uint32_t kv_heads, DType kv_dtype) const;

 private:
  Runtime rt_;
  uint32_t hidden_, q_heads_, head_, seq_;
  AttentionOptions opts_;
  Tensor xb_, q_, partial_;
  std::shared_ptr<Tensor> table_;
  uint32_t max_splits_;
};

// Pre-norm SwiGLU block (src/modules.rs:276-333): RMSNorm, gated MLP,
// residual.  Recorded as two launches: norm+gate/up+SwiGLU, down + residual.
class SwiGluBlock {
 public:
  SwiGluBlock(const Runtime &rt, uint32_t hidden, uint32_t intermediate, float eps = 1e-5f);
  void record(Scheme &s, TensorView x, const SwiGluBlockWeights &w) const;
  void record_group(Scheme &s, const std::string &label, TensorView x,
                    const SwiGluBlockWeights &w) const;

 private:
  Runtime rt_;
  uint32_t hidden_, inter_;
  float eps_;
  Tensor hb_;
};

// ---- model contract and greedy loop ------------------------------------------------------
class AutoregressiveModel {  // src/model.rs:7-11
 public:
  virtual ~AutoregressiveModel() = default;
  virtual size_t vocab_size() const = 0;
  virtual uint32_t max_seq_len() const = 0;
  // Logits [vocab] for (token, pos); valid until the next step.
  virtual const std::vector<float> &step(uint32_t token, uint32_t pos) = 0;
};

struct GenerateTokenOutput {  // src/generate.rs:28-33
  std::vector<int32_t> tokens;
  size_t prompt_tokens = 0;
  double tokens_per_second = 0.0;
};

// First index of the maximum under a strict `>`; NaN never wins
// (src/tokenizer.rs:179-189).
int32_t sample_argmax(const float *logits, size_t n);

// The reference's greedy loop (src/generate.rs:43-91), host argmax per step.
GenerateTokenOutput generate_tokens(AutoregressiveModel &model,
                                    const std::vector<int32_t> &prompt_tokens,
                                    uint32_t max_new_tokens,
                                    std::optional<int32_t> stop_on = std::nullopt);

// ---- tokenizer and text generation ------------------------------------------------------
// String <-> token ids (src/tokenizer.rs:11-16).  Strings are UTF-8 bytes.
class Tokenizer {
 public:
  virtual ~Tokenizer() = default;
  virtual size_t vocab_size() const = 0;
  virtual std::vector<int32_t> encode(const std::string &text, bool bos, bool eos) const = 0;
  virtual std::string decode(int32_t prev_token, int32_t token) const = 0;
};

// SentencePiece-style BPE over a llama2.c tokenizer.bin (src/tokenizer.rs:
// 18-177): pieces, merge scores, dummy-prefix encoding with byte fallback
// (byte b -> id b + 3) and greedy highest-score pair merging.
class BpeTokenizer : public Tokenizer {
 public:
  // tokenizer.bin: u32 max_token_length, then per piece f32 score, i32
  // length, bytes (pieces are read as UTF-8 with invalid sequences replaced
  // by U+FFFD, as the reference's from_utf8_lossy).
  static BpeTokenizer from_path(const std::string &path, size_t vocab_size);
  static BpeTokenizer from_parts(std::vector<std::string> vocab, std::vector<float> scores,
                                 uint32_t max_token_length);
  uint32_t max_token_length() const { return max_token_length_; }
  static int32_t bos_id() { return 1; }
  static int32_t eos_id() { return 2; }

  size_t vocab_size() const override { return vocab_.size(); }
  std::vector<int32_t> encode(const std::string &text, bool bos, bool eos) const override;
  std::string decode(int32_t prev_token, int32_t token) const override;
  const std::string &piece(int32_t id) const { return vocab_.at((size_t)id); }

 private:
  int32_t lookup(const std::string &s) const;  // -1 when absent
  std::vector<std::string> vocab_;
  std::vector<float> scores_;
  uint32_t max_token_length_ = 0;
  std::vector<std::pair<std::string, int32_t>> sorted_;
};

struct GenerateOptions {  // src/generate.rs:8-26
  uint32_t max_new_tokens = 50;
  bool bos = true;
  bool eos = false;
  std::optional<int32_t> stop_on;  // stop when chosen after the prompt
};

struct GenerateOutput {  // src/generate.rs:35-41
  std::string text;
  std::vector<int32_t> tokens;
  size_t prompt_tokens = 0;
  double tokens_per_second = 0.0;
};

// Text of a token sequence as the reference's generate assembles it
// (src/generate.rs:106-113): decode(prev, token) with prev starting at
// `first`.
std::string decode_tokens(const Tokenizer &tokenizer, int32_t first,
                          const std::vector<int32_t> &tokens);

// The reference's text generation (src/generate.rs:93-118): encode the
// prompt, run generate_tokens, decode the tokens after the first prompt token.
GenerateOutput generate(AutoregressiveModel &model, const Tokenizer &tokenizer,
                        const std::string &prompt, const GenerateOptions &options = {});

}  // namespace ammon
