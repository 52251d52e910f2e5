// kernels_test.cpp -- the reference's kernel tests (tests/kernels.rs) restated
// against the C++ recorder tier (ammon::kernels, ammon::TensorKernels) on a
// gfx950 device.  Each test records launches into a Scheme, submits, and
// reads the results back; the validation tests check the error text names
// the parameter and that a failed record leaves the scheme unchanged.
//
// Layout differences from the reference: KV caches here are head-major
// [kv_heads, seq, head] (the reference's is [seq, kv_heads, head]); with one
// kv head both are [seq, head] in memory.
#include <cmath>
#include <cstdio>
#include <vector>

#include "ammon/ammon.hpp"
#include "check.hpp"

using ammon::DecodeStep;
using ammon::DType;
using ammon::Scheme;
using ammon::Shape;
using ammon::Tensor;
using ammon::TensorKernels;

namespace {

ammon::Runtime &runtime() {
  static ammon::Runtime rt = ammon::create_runtime(0);
  return rt;
}

// DecodeStep parcel holding {token, position} (tests/kernels.rs:17-21).
Tensor step_buf(uint32_t token, uint32_t position) {
  Tensor t = DecodeStep::parcel(runtime());
  DecodeStep::deposit(runtime(), t, DecodeStep{token, position});
  ammon::check(ammon_stream_synchronize(runtime().raw(), nullptr), "step_buf");
  return t;
}

Tensor f32(Shape s, std::vector<float> v) { return Tensor::from_f32(runtime(), std::move(s), v); }

std::vector<float> run_and_read(Scheme &s, const Tensor &t) {
  s.submit();
  s.synchronize();
  return t.to_f32();
}

}  // namespace

// tests/kernels.rs:36-52
TEST(embed_gathers_selected_row) {
  Tensor table = f32(Shape::matrix(2, 2), {1, 2, 3, 4});
  Tensor step = step_buf(1, 0);
  Tensor x = Tensor::zeros(runtime(), Shape::vector(2), DType::F32);
  Scheme s(runtime());
  ammon::kernels::embed(s, "embed", table.view(), step, x.view());
  CHECK((run_and_read(s, x) == std::vector<float>{3, 4}));
}

// tests/kernels.rs:54-81: RoPE at position 0 rotates by zero
TEST(rope_at_pos_zero_is_identity) {
  Tensor q = f32(Shape::matrix(1, 2), {1, 2});
  Tensor k = f32(Shape::from_dims({1, 1, 2}), {3, 4});
  Tensor step = step_buf(0, 0);
  auto table = ammon::kernels::rope_table(runtime(), AMMON_DEFAULT_ROPE_THETA, 2, 1);
  Scheme s(runtime());
  ammon::kernels::rope(s, "rope", q.view(), k.view(), step, table->view());
  CHECK((run_and_read(s, q) == std::vector<float>{1, 2}));
  CHECK((k.to_f32() == std::vector<float>{3, 4}));
}

// tests/kernels.rs:83-97
TEST(gemv_identity) {
  Tensor x = f32(Shape::vector(2), {1, 2});
  Tensor w = f32(Shape::matrix(2, 2), {1, 0, 0, 1});
  Tensor out = Tensor::zeros(runtime(), Shape::matrix(1, 2), DType::F32);
  Tensor step = step_buf(0, 0);
  Scheme s(runtime());
  ammon::kernels::gemv(s, "gemv", x.view(), w.view(), out.view(), step);
  CHECK((run_and_read(s, out) == std::vector<float>{1, 2}));
}

// tests/kernels.rs:99-123: the position-strided gemv writes row `position`
TEST(gemv_writes_cache_row_at_position) {
  Tensor x = f32(Shape::vector(2), {1, 2});
  Tensor w = f32(Shape::matrix(2, 2), {1, 0, 0, 1});
  Tensor out = Tensor::zeros(runtime(), Shape::matrix(4, 2), DType::F32);
  Tensor step = step_buf(0, 2);
  Scheme s(runtime());
  ammon::kernels::gemv(s, "gemv_row", x.view(), w.view(), out.view(), step);
  CHECK((run_and_read(s, out) == std::vector<float>{0, 0, 0, 0, 1, 2, 0, 0}));
}

// tests/kernels.rs:125-146
TEST(gemv_rejects_rank1_output) {
  Tensor x = f32(Shape::vector(2), {1, 2});
  Tensor w = f32(Shape::matrix(2, 2), {1, 0, 0, 1});
  Tensor out = f32(Shape::vector(2), {0, 0});
  Tensor step = step_buf(0, 0);
  Scheme s(runtime());
  const size_t before = s.ir_node_count();
  CHECK_THROWS_WITH(ammon::kernels::gemv(s, "gemv_rank1", x.view(), w.view(), out.view(), step),
                    "expected rank 2");
  CHECK(s.ir_node_count() == before);
}

// tests/kernels.rs:148-161
TEST(swiglu_of_zero_is_zero) {
  Tensor hb = f32(Shape::vector(2), {0, 0});
  Tensor hb2 = f32(Shape::vector(2), {5, 7});
  Scheme s(runtime());
  ammon::kernels::swiglu(s, "swiglu", hb.view(), hb2.view());
  CHECK((run_and_read(s, hb) == std::vector<float>{0, 0}));
}

// tests/kernels.rs:163-182
TEST(rmsnorm_matches_llama3_cuda_formula) {
  Tensor x = f32(Shape::vector(4), {1, 1, 1, 1});
  Tensor w = f32(Shape::vector(4), {1, 1, 1, 1});
  Tensor o = Tensor::zeros(runtime(), Shape::vector(4), DType::F32);
  Scheme s(runtime());
  ammon::kernels::rmsnorm(s, "rms", x.view(), w.view(), o.view());
  const float scale = 1.0f / std::sqrt(1.0f + 1e-5f);
  for (float v : run_and_read(s, o)) CHECK_NEAR(v, scale, 1e-5);
}

// tests/kernels.rs:184-222: one record, two deposits, two replays
TEST(deposit_feeds_embed_without_rerecord) {
  Tensor table = f32(Shape::matrix(2, 2), {10, 20, 30, 40});
  Tensor step = step_buf(0, 0);
  Tensor x = f32(Shape::vector(2), {0, 0});
  Scheme worker(runtime());
  ammon::kernels::embed(worker, "embed", table.view(), step, x.view());
  for (uint32_t token : {0u, 1u}) {
    DecodeStep::deposit(runtime(), step, DecodeStep{token, 0}, worker.stream());
    worker.submit();
    worker.synchronize();
    const std::vector<float> got = x.to_f32();
    CHECK((got == (token == 0 ? std::vector<float>{10, 20} : std::vector<float>{30, 40})));
  }
  CHECK(worker.replay_stats().records == 1);
  CHECK(worker.replay_stats().captures == 1);
  CHECK(worker.replay_stats().submits == 2);
}

// tests/kernels.rs:224-237
TEST(tensor_add_into_is_elementwise) {
  Tensor a = f32(Shape::vector(2), {1, 2});
  Tensor b = f32(Shape::vector(2), {3, 4});
  Tensor out = Tensor::zeros(runtime(), Shape::vector(2), DType::F32);
  Scheme s(runtime());
  TensorKernels::prepare(runtime()).add_into(s, "add", a.view(), b.view(), out.view());
  CHECK((run_and_read(s, out) == std::vector<float>{4, 6}));
}

// tests/kernels.rs:239-283: position 1, head 2 -> rotation by 1 rad; row 0 untouched
TEST(rope_store_writes_rotated_k_from_scratch) {
  Tensor q = f32(Shape::matrix(1, 2), {1, 0});
  Tensor k_proj = f32(Shape::vector(2), {0, 1});
  Tensor k = f32(Shape::from_dims({1, 2, 2}), {7, 8, 0, 0});  // [kv_heads, seq, head]
  Tensor step = step_buf(0, 1);
  auto table = ammon::kernels::rope_table(runtime(), AMMON_DEFAULT_ROPE_THETA, 2, 2);
  Scheme s(runtime());
  ammon::kernels::rope_store(s, "rope_store", q.view(), k_proj.view(), k.view(), step,
                             table->view());
  const std::vector<float> qv = run_and_read(s, q), kv = k.to_f32();
  const double c = std::cos(1.0), sn = std::sin(1.0);
  CHECK_NEAR(qv[0], c, 1e-5);
  CHECK_NEAR(qv[1], sn, 1e-5);
  CHECK(kv[0] == 7 && kv[1] == 8);  // row 0 untouched
  CHECK_NEAR(kv[2], -sn, 1e-5);
  CHECK_NEAR(kv[3], c, 1e-5);
}

// tests/kernels.rs:285-307
TEST(cache_store_writes_row_at_position) {
  Tensor v = f32(Shape::vector(2), {9, 8});
  Tensor cache = Tensor::zeros(runtime(), Shape::from_dims({1, 4, 2}), DType::F32);
  Tensor step = step_buf(0, 2);
  Scheme s(runtime());
  ammon::kernels::cache_store(s, "cache_store", v.view(), cache.view(), step);
  CHECK((run_and_read(s, cache) == std::vector<float>{0, 0, 0, 0, 9, 8, 0, 0}));
}

// tests/kernels.rs:309-340: matmul_into (identity weights) then cache_store
TEST(semantic_gemv_then_cache_store_matches_serial_identity) {
  Tensor x = f32(Shape::vector(2), {5, 6});
  Tensor w = f32(Shape::matrix(2, 2), {1, 0, 0, 1});
  Tensor proj = Tensor::zeros(runtime(), Shape::vector(2), DType::F32);
  Tensor cache = Tensor::zeros(runtime(), Shape::from_dims({1, 3, 2}), DType::F32);
  Tensor step = step_buf(0, 1);
  Scheme s(runtime());
  TensorKernels::prepare(runtime()).matmul_into(s, "proj", w.view(), x.view(), proj.view());
  ammon::kernels::cache_store(s, "store", proj.view(), cache.view(), step);
  CHECK((run_and_read(s, cache) == std::vector<float>{0, 0, 5, 6, 0, 0}));
}

// tests/kernels.rs:342-355
TEST(tensor_matmul_into_is_gemv) {
  Tensor a = f32(Shape::matrix(2, 2), {1, 0, 0, 1});
  Tensor b = f32(Shape::vector(2), {1, 2});
  Tensor out = Tensor::zeros(runtime(), Shape::vector(2), DType::F32);
  Scheme s(runtime());
  TensorKernels::prepare(runtime()).matmul_into(s, "matmul", a.view(), b.view(), out.view());
  CHECK((run_and_read(s, out) == std::vector<float>{1, 2}));
}

// tests/kernels.rs:357-378
TEST(rope_rejects_rank2_kv_cache) {
  Tensor q = f32(Shape::matrix(1, 2), {1, 2});
  Tensor k = f32(Shape::matrix(1, 2), {3, 4});
  Tensor step = step_buf(0, 0);
  auto table = ammon::kernels::rope_table(runtime(), AMMON_DEFAULT_ROPE_THETA, 2, 1);
  Scheme s(runtime());
  const size_t before = s.ir_node_count();
  CHECK_THROWS_WITH(ammon::kernels::rope(s, "rope_rank2", q.view(), k.view(), step, table->view()),
                    "parameter `k`: expected rank 3");
  CHECK(s.ir_node_count() == before);
}

// tests/kernels.rs:540-556
TEST(embed_rejects_dim_mismatch) {
  Tensor table = f32(Shape::matrix(2, 2), {1, 2, 3, 4});
  Tensor x = f32(Shape::vector(3), {0, 0, 0});
  Tensor step = step_buf(0, 0);
  Scheme s(runtime());
  const size_t before = s.ir_node_count();
  CHECK_THROWS_WITH(ammon::kernels::embed(s, "embed_dim", table.view(), step, x.view()), "`dim`");
  CHECK(s.ir_node_count() == before);
}

// An eager scheme (no graph) replays the same launches.
TEST(eager_scheme_matches_graph_replay) {
  Tensor table = f32(Shape::matrix(3, 2), {1, 2, 3, 4, 5, 6});
  Tensor step = step_buf(2, 0);
  Tensor xg = Tensor::zeros(runtime(), Shape::vector(2), DType::F32);
  Tensor xe = Tensor::zeros(runtime(), Shape::vector(2), DType::F32);
  Scheme g(runtime(), true), e(runtime(), false);
  ammon::kernels::embed(g, "embed", table.view(), step, xg.view());
  ammon::kernels::embed(e, "embed", table.view(), step, xe.view());
  CHECK((run_and_read(g, xg) == std::vector<float>{5, 6}));
  CHECK((run_and_read(e, xe) == std::vector<float>{5, 6}));
  CHECK(e.replay_stats().captures == 0);
}

int main(int argc, char **argv) { return check::run_all(argc, argv); }
