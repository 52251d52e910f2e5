// core.cpp -- runtime handle, tensors, DecodeStep parcel and Scheme of the
// C++ host layer.  Uses only the public C ABI (ammon.h).
#include <cstring>
#include <sstream>

#include "ammon/ammon.hpp"

namespace ammon {

void check(ammon_status st, const std::string &context) {
  if (st == AMMON_OK) return;
  std::string msg = ammon_last_error();
  throw Error(st, context.empty() ? msg : context + ": " + msg);
}

size_t dtype_size(DType d) { return d == DType::BF16 ? 2 : 4; }

// ---- runtime -------------------------------------------------------------------
Runtime Runtime::create(int device) {
  ammon_runtime *raw = nullptr;
  check(ammon_runtime_create(device, &raw), "create runtime");
  Runtime r;
  r.rt_ = std::shared_ptr<ammon_runtime>(raw, [](ammon_runtime *p) { ammon_runtime_release(p); });
  check(ammon_runtime_info(raw, &r.info_), "runtime info");
  return r;
}

Runtime create_runtime(int device) { return Runtime::create(device); }

// ---- shapes and views --------------------------------------------------------------
Shape Shape::from_dims(std::vector<uint32_t> d) {
  if (d.empty()) throw Error(AMMON_E_VALIDATION, "shape must have at least one dimension");
  return Shape{std::move(d)};
}

uint32_t Shape::dim(size_t i) const {
  if (i >= dims.size()) {
    std::ostringstream os;
    os << "dimension " << i << " out of range for rank " << dims.size();
    throw Error(AMMON_E_VALIDATION, os.str());
  }
  return dims[i];
}

uint64_t Shape::numel() const {
  uint64_t n = 1;
  for (uint32_t d : dims) n *= d;
  return n;
}

std::string Shape::str() const {
  std::ostringstream os;
  os << "[";
  for (size_t i = 0; i < dims.size(); ++i) os << (i ? ", " : "") << dims[i];
  os << "]";
  return os.str();
}

uint32_t TensorView::numel_u32() const {
  const uint64_t n = numel();
  if (n > 0xffffffffull) throw Error(AMMON_E_VALIDATION, "tensor has more than 2^32 elements");
  return (uint32_t)n;
}

TensorView TensorView::narrow(size_t axis, uint32_t start, uint32_t len) const {
  const uint32_t extent = shape_.dim(axis);
  if ((uint64_t)start + len > extent) {
    std::ostringstream os;
    os << "narrow [" << start << ", " << start + len << ") exceeds axis " << axis << " of "
       << shape_.str();
    throw Error(AMMON_E_VALIDATION, os.str());
  }
  uint64_t inner = 1;
  for (size_t i = axis + 1; i < shape_.rank(); ++i) inner *= shape_.dims[i];
  Shape s = shape_;
  s.dims[axis] = len;
  return TensorView((char *)ptr_ + (size_t)start * inner * dtype_size(dtype_), s, dtype_);
}

TensorView TensorView::reshape(std::vector<uint32_t> dims) const {
  Shape s = Shape::from_dims(std::move(dims));
  if (s.numel() != numel()) {
    throw Error(AMMON_E_VALIDATION, "cannot reshape " + shape_.str() + " to " + s.str());
  }
  return TensorView(ptr_, s, dtype_);
}

// ---- tensors ---------------------------------------------------------------------------
Tensor::Tensor(Tensor &&o) noexcept { *this = std::move(o); }

Tensor &Tensor::operator=(Tensor &&o) noexcept {
  if (this != &o) {
    if (ptr_) ammon_free(rt_.raw(), ptr_);
    rt_ = std::move(o.rt_);
    ptr_ = o.ptr_;
    shape_ = std::move(o.shape_);
    dtype_ = o.dtype_;
    o.ptr_ = nullptr;
  }
  return *this;
}

Tensor::~Tensor() {
  if (ptr_ && rt_) ammon_free(rt_.raw(), ptr_);
}

Tensor Tensor::zeros(const Runtime &rt, Shape shape, DType dtype) {
  Tensor t;
  t.rt_ = rt;
  t.shape_ = std::move(shape);
  t.dtype_ = dtype;
  const size_t bytes = t.nbytes();
  check(ammon_alloc(rt.raw(), bytes, &t.ptr_), "Tensor::zeros");
  if (bytes) {
    // Zero with a fill kernel (4-byte words), then wait so the tensor is ready.
    const size_t words = bytes / 4, tail = bytes % 4;
    if (words) check(ammon_fill(rt.raw(), nullptr, t.ptr_, AMMON_F32, words, 0.0f), "Tensor::zeros");
    if (tail) {
      const uint32_t z = 0;
      check(ammon_memcpy(rt.raw(), (char *)t.ptr_ + words * 4, &z, tail, AMMON_COPY_H2D, nullptr),
            "Tensor::zeros");
    }
    check(ammon_stream_synchronize(rt.raw(), nullptr), "Tensor::zeros");
  }
  return t;
}

Tensor Tensor::from_host(const Runtime &rt, Shape shape, DType dtype, const void *data) {
  Tensor t = zeros(rt, std::move(shape), dtype);
  t.upload(data);
  return t;
}

Tensor Tensor::from_f32(const Runtime &rt, Shape shape, const std::vector<float> &data) {
  if (data.size() != shape.numel())
    throw Error(AMMON_E_VALIDATION, "from_f32: " + std::to_string(data.size()) +
                                        " values for shape " + shape.str());
  return from_host(rt, std::move(shape), DType::F32, data.data());
}

void Tensor::upload(const void *src) {
  if (!nbytes()) return;
  check(ammon_memcpy(rt_.raw(), ptr_, src, nbytes(), AMMON_COPY_H2D, nullptr), "upload");
  check(ammon_stream_synchronize(rt_.raw(), nullptr), "upload");
}

void Tensor::to_host(void *dst) const {
  if (!nbytes()) return;
  // Work queued on any stream of this runtime's device must be complete;
  // callers synchronise their scheme before reading.
  check(ammon_memcpy(rt_.raw(), dst, ptr_, nbytes(), AMMON_COPY_D2H, nullptr), "download");
  check(ammon_stream_synchronize(rt_.raw(), nullptr), "download");
}

std::vector<float> Tensor::to_f32() const {
  const size_t n = shape_.numel();
  std::vector<float> out(n);
  if (dtype_ == DType::BF16) {
    std::vector<uint16_t> raw(n);
    to_host(raw.data());
    for (size_t i = 0; i < n; ++i) {
      const uint32_t u = (uint32_t)raw[i] << 16;
      std::memcpy(&out[i], &u, 4);
    }
  } else if (dtype_ == DType::F32) {
    to_host(out.data());
  } else {
    throw Error(AMMON_E_VALIDATION, "to_f32: tensor is not floating point");
  }
  return out;
}

// ---- DecodeStep parcel -----------------------------------------------------------------
Tensor DecodeStep::parcel(const Runtime &rt) { return Tensor::zeros(rt, Shape::vector(2), DType::U32); }

void DecodeStep::deposit(const Runtime &rt, const Tensor &parcel, DecodeStep value,
                         ammon_stream stream) {
  if (parcel.nbytes() < sizeof(ammon_decode_step))
    throw Error(AMMON_E_VALIDATION, "deposit: parcel is smaller than a DecodeStep");
  const ammon_decode_step v = {value.token, value.position};
  check(ammon_memcpy(rt.raw(), parcel.data(), &v, sizeof v, AMMON_COPY_H2D, stream), "deposit");
  // `v` lives on this stack frame: wait for the copy before returning.
  check(ammon_stream_synchronize(rt.raw(), stream), "deposit");
}

DecodeStep DecodeStep::read(const Runtime &rt, const Tensor &parcel) {
  ammon_decode_step v = {0, 0};
  check(ammon_memcpy(rt.raw(), &v, parcel.data(), sizeof v, AMMON_COPY_D2H, nullptr), "read step");
  check(ammon_stream_synchronize(rt.raw(), nullptr), "read step");
  return DecodeStep{v.token, v.position};
}

// ---- Scheme ------------------------------------------------------------------------------
Scheme::Scheme(const Runtime &rt, bool use_graph, ammon_stream stream)
    : rt_(rt), stream_(stream), use_graph_(use_graph) {
  if (!stream_) {
    check(ammon_stream_create(rt_.raw(), &stream_), "Scheme stream");
    owns_stream_ = true;
  }
}

Scheme::~Scheme() {
  drop_graph();
  if (owns_stream_ && stream_) ammon_stream_destroy(rt_.raw(), stream_);
}

void Scheme::drop_graph() {
  if (graph_) ammon_graph_destroy(rt_.raw(), graph_);
  graph_ = nullptr;
}

void Scheme::record(const std::string &label, Launch launch) {
  const std::string full = prefix_.empty() ? label : prefix_ + "/" + label;
  const ammon_status st = launch(AMMON_STREAM_VALIDATE);
  if (st != AMMON_OK) throw Error(st, full + ": " + ammon_last_error());
  nodes_.push_back(std::move(launch));
  labels_.push_back(full);
  stats_.records += 1;
  drop_graph();
}

void Scheme::group(const std::string &label, const std::function<void(Scheme &)> &fn) {
  const std::string saved = prefix_;
  prefix_ = saved.empty() ? label : saved + "/" + label;
  try {
    fn(*this);
  } catch (...) {
    prefix_ = saved;
    throw;
  }
  prefix_ = saved;
}

void Scheme::submit() {
  stats_.submits += 1;
  if (use_graph_ && !graph_ && !nodes_.empty()) {
    if (ammon_capture_begin(rt_.raw(), stream_) == AMMON_OK) {
      ammon_status bad = AMMON_OK;
      std::string where;
      for (size_t i = 0; i < nodes_.size() && bad == AMMON_OK; ++i) {
        bad = nodes_[i](stream_);
        if (bad != AMMON_OK) where = labels_[i] + ": " + ammon_last_error();
      }
      ammon_graph g = nullptr;
      const ammon_status end = ammon_capture_end(rt_.raw(), stream_, &g);
      if (bad != AMMON_OK) {
        if (g) ammon_graph_destroy(rt_.raw(), g);
        throw Error(bad, where);
      }
      if (end == AMMON_OK) {
        graph_ = g;
        stats_.captures += 1;
      } else {
        use_graph_ = false;  // capture unsupported here: replay eagerly
      }
    } else {
      use_graph_ = false;
    }
  }
  if (graph_) {
    check(ammon_graph_launch(rt_.raw(), graph_, stream_), "scheme replay");
    return;
  }
  for (size_t i = 0; i < nodes_.size(); ++i) check(nodes_[i](stream_), labels_[i]);
}

void Scheme::synchronize() { check(ammon_stream_synchronize(rt_.raw(), stream_), "scheme sync"); }

}  // namespace ammon
