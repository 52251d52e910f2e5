// ops.cpp -- C-ABI kernel entry points: validate, pick the variant, launch.
//
// Each entry point replaces one reference kernel record + dispatch (or one
// fused group of them); the reference file:line is given in ammon.h.  All
// validation happens before anything is enqueued, so a failed call leaves
// the stream untouched -- the counterpart of a failed Goldy record leaving
// the scheme's IR unchanged (reference tests/kernels.rs:125-146).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "internal.h"

using namespace ammon_rt;

namespace {

using DeviceGuard = ammon_rt::DeviceScope;

inline uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

inline bool valid_dtype(ammon_dtype d) { return d == AMMON_F32 || d == AMMON_BF16; }
inline size_t dsize(ammon_dtype d) { return d == AMMON_BF16 ? 2 : 4; }

inline bool overlaps(const void *a, size_t abytes, const void *b, size_t bbytes) {
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  return a0 < b0 + bbytes && b0 < a0 + abytes;
}

template <typename P>
ammon_status launch3(ammon_runtime *rt, ammon_stream s, hipFunction_t f, uint32_t gx, uint32_t gy,
                     uint32_t gz, uint32_t shmem, P &params, const char *what) {
  if (gx == 0 || gy == 0 || gz == 0) return AMMON_OK;
  DeviceGuard guard(rt->device);
  hipStream_t st = s ? (hipStream_t)s : rt->stream;
  void *args[] = {&params};
  hipError_t e = hipModuleLaunchKernel(f, gx, gy, gz, kWorkgroup, 1, 1, shmem, st, args, nullptr);
  if (e != hipSuccess) return hip_error(e, what);
  return AMMON_OK;
}

template <typename P>
ammon_status launch(ammon_runtime *rt, ammon_stream s, hipFunction_t f, uint32_t gx, uint32_t gy,
                    uint32_t shmem, P &params, const char *what) {
  return launch3(rt, s, f, gx, gy, 1, shmem, params, what);
}

// The attention kernels take the DecodeStep pointer as a leading scalar
// argument (preloaded into SGPRs), then the parameter struct.
ammon_status launch_att(ammon_runtime *rt, ammon_stream s, hipFunction_t f, uint32_t gx,
                        uint32_t gy, uint32_t gz, ammon_k_attention &params, const char *what) {
  DeviceGuard guard(rt->device);
  hipStream_t st = s ? (hipStream_t)s : rt->stream;
  void *args[] = {&params.step, &params};
  hipError_t e = hipModuleLaunchKernel(f, gx, gy, gz, kWorkgroup, 1, 1, 0, st, args, nullptr);
  if (e != hipSuccess) return hip_error(e, what);
  return AMMON_OK;
}

#define REQUIRE_RT()                                              \
  do {                                                            \
    if (!rt) return set_error(AMMON_E_VALIDATION, "runtime is NULL"); \
  } while (0)

#define VALIDATE_ONLY()                                  \
  do {                                                   \
    if (stream == AMMON_STREAM_VALIDATE) return AMMON_OK; \
  } while (0)

// ---- GEMV family --------------------------------------------------------------
struct GemvArgs {
  int mode;
  const void *w0, *w1, *w2;
  ammon_dtype w_dtype;
  uint32_t d, n, rows;
  const float *x;
  const void *norm_w;
  ammon_dtype norm_dtype;
  float eps;
  const float *residual;
  float *y;
  void *k_cache, *v_cache;
  const ammon_decode_step *step;
  const float *table;
  uint32_t kv_dim, head, seq;
  ammon_dtype kv_dtype;
  float *cand_v;       // PLAIN_ARGMAX: candidate arrays of cand_cap entries
  uint32_t *cand_i;
  uint32_t cand_cap;
};

// The wide GEMV variant applies: a long bf16 matrix in 16-byte chunks with
// no epilogue beyond the argmax candidates.
static bool gemv_wide(const GemvArgs &a, int vec_ok) {
  return vec_ok && a.w_dtype == AMMON_BF16 && a.rows >= kGemvWideMinRows &&
         (uint64_t)a.n * 2 <= kGemvWideMaxRowBytes &&
         (a.mode == AMMON_GEMV_PLAIN || a.mode == AMMON_GEMV_PLAIN_ARGMAX);
}

// Validates and packs a GEMV: *p receives the kernel parameters, *lds_out
// the bytes of LDS its x staging needs, *vec_out whether the 16-byte-chunk
// (vector) kernels apply.
ammon_status gemv_pack(ammon_runtime *rt, const GemvArgs &a, const char *what, ammon_k_gemv *out,
                       size_t *lds_out, int *vec_out) {
  AMMON_CHECK(valid_dtype(a.w_dtype), "%s: unknown weight dtype %d", what, (int)a.w_dtype);
  AMMON_CHECK(a.w0 && a.x && a.y, "%s: NULL weight, x or y", what);
  AMMON_CHECK(a.n > 0 && a.d > 0, "%s: empty matrix (d=%u, n=%u)", what, a.d, a.n);
  AMMON_CHECK(!a.norm_w || valid_dtype(a.norm_dtype), "%s: unknown norm dtype", what);
  AMMON_CHECK(!a.norm_w || (std::isfinite(a.eps) && a.eps >= 0.f), "%s: eps must be finite and >= 0", what);
  // x staged in LDS, zero-padded to whole tiles of 64 lanes x kGemvTileChunks
  // chunks of 16 bytes (8 bf16 or 4 fp32 weights; 1 weight on the scalar path).
  const bool bf = a.w_dtype == AMMON_BF16;
  const uint32_t ch_v = bf ? 8 : 4;
  const uintptr_t wbits = (uintptr_t)a.w0 | (uintptr_t)a.w1 | (uintptr_t)a.w2;
  const int vec_ok = (a.n % ch_v == 0) && (wbits & 15u) == 0;
  const uint64_t tile_elems = 64ull * kGemvTileChunks * (vec_ok ? ch_v : 1);
  const size_t shmem = (size_t)((a.n + tile_elems - 1) / tile_elems * tile_elems) * sizeof(float);
  AMMON_CHECK(shmem <= (size_t)rt->info.max_shared_per_block,
              "%s: reduction length n=%u needs %zu bytes of LDS; the device allows %d", what, a.n,
              shmem, rt->info.max_shared_per_block);
  // y must not overlap x: x is staged by every workgroup while others write y.
  size_t ybytes = (size_t)a.d * 4;
  AMMON_CHECK(!overlaps(a.x, (size_t)a.n * 4, a.y, ybytes), "%s: y overlaps x", what);
  if (a.residual)
    AMMON_CHECK(!overlaps(a.x, (size_t)a.n * 4, a.residual, ybytes), "%s: residual overlaps x", what);

  ammon_k_gemv &p = *out;
  p = ammon_k_gemv{};
  p.w0 = a.w0;
  p.w1 = a.w1;
  p.w2 = a.w2;
  p.x = a.x;
  p.norm_w = a.norm_w;
  p.residual = a.residual;
  p.y = a.y;
  p.k_cache = a.k_cache;
  p.v_cache = a.v_cache;
  p.step = (const ammon_k_step *)a.step;
  p.table = a.table;
  p.d = a.d;
  p.n = a.n;
  p.rows = a.rows;
  const uint32_t rows_per_wg =
      (gemv_wide(a, vec_ok) ? kGemvWideRowsPerWave : kGemvRowsPerWave) * kGemvWaves;
  p.row_blocks = cdiv(a.rows, rows_per_wg);
  p.norm_dtype = (uint32_t)a.norm_dtype;
  p.eps = a.eps;
  p.kv_dim = a.kv_dim;
  p.head = a.head;
  p.seq = a.seq;
  p.kv_dtype = (uint32_t)a.kv_dtype;
  p.cand_v = a.cand_v;
  p.cand_i = a.cand_i;
  *lds_out = shmem;
  *vec_out = vec_ok;
  return AMMON_OK;
}

// The most weight bytes a merge launch warms for the next GEMV.
constexpr uint64_t kWarmMaxBytes = 20ull << 20;

// Grid: at most gemv_wgs_per_cu resident workgroups per CU (fewer if LDS
// bounds it); among 2..max per CU pick the count whose grid-stride split of
// the row blocks wastes the least (blocks / (grid * blocks per workgroup)).
uint32_t gemv_grid(ammon_runtime *rt, hipFunction_t fn, size_t lds, uint32_t row_blocks, int mode) {
  const uint32_t cus = (uint32_t)std::max(rt->info.compute_units, 1);
  const uint32_t resident = occupancy(rt, fn, lds);
  const uint32_t max_per_cu = std::max<uint32_t>(1, std::min(rt->gemv_wgs_per_cu, resident));
  uint32_t grid = std::min<uint32_t>(row_blocks, cus * max_per_cu);
  double best = -1.0;
  for (uint32_t w = max_per_cu; w >= 1; --w) {
    const uint32_t g = std::min<uint32_t>(row_blocks, cus * w);
    const uint32_t per_wg = cdiv(row_blocks, g);
    const double eff = (double)row_blocks / ((double)g * per_wg);
    if (eff > best + 1e-9) {
      best = eff;
      grid = g;
    }
    if (w == 1 || w <= max_per_cu / 2) break;
  }
  // QKV: at most two workgroups per CU, even with a ragged last round: at
  // the Llama-3-8B shape (768 row blocks) 512 workgroups measured 10.4-10.6
  // us against 11.5-11.6 for 768 (x requested ahead of the weights)
  if (mode == AMMON_GEMV_QKV && max_per_cu > 2) grid = std::min<uint32_t>(row_blocks, cus * 2);
  return grid;
}

// The grid of a RESIDUAL-mode GEMV of rows x n weights at w (its vector
// kernel when w is 16-byte aligned and n a whole number of chunks) and, in
// *tile_row_bytes, the bytes of each row its first tile covers.
uint32_t gemv_grid_for(ammon_runtime *rt, const void *w, ammon_dtype dt, uint32_t n,
                       uint32_t rows, uint64_t *tile_row_bytes) {
  const bool bf = dt == AMMON_BF16;
  const uint32_t ch_v = bf ? 8 : 4;
  const int vec = (n % ch_v == 0) && (((uintptr_t)w) & 15u) == 0;
  const uint64_t tile_elems = 64ull * kGemvTileChunks * (vec ? ch_v : 1);
  *tile_row_bytes = tile_elems * dsize(dt);
  const size_t lds = (size_t)((n + tile_elems - 1) / tile_elems * tile_elems) * sizeof(float);
  return gemv_grid(rt, rt->k.gemv[bf ? 1 : 0][vec][AMMON_GEMV_RESIDUAL], lds,
                   cdiv(rows, kGemvRowsPerWave * kGemvWaves), AMMON_GEMV_RESIDUAL);
}

// Validates, packs and launches a GEMV; *grid_out (optional) receives the
// workgroup count (PLAIN_ARGMAX writes one candidate per workgroup).
ammon_status gemv_check_and_launch(ammon_runtime *rt, ammon_stream stream, const GemvArgs &a,
                                   const char *what, uint32_t *grid_out = nullptr) {
  ammon_k_gemv p;
  size_t shmem = 0;
  int vec = 0;
  const ammon_status status = gemv_pack(rt, a, what, &p, &shmem, &vec);
  if (status != AMMON_OK || stream == AMMON_STREAM_VALIDATE) return status;
  const int dt = a.w_dtype == AMMON_BF16 ? 1 : 0;
  size_t lds = shmem;
  // PLAIN_ARGMAX reduces the workgroup's candidates in x's LDS
  if (a.mode == AMMON_GEMV_PLAIN_ARGMAX) lds = std::max<size_t>(lds, 2 * kWorkgroup * 4);
  hipFunction_t fn = gemv_wide(a, vec)                  ? rt->k.gemv_wide[a.mode == AMMON_GEMV_PLAIN_ARGMAX]
                     : a.mode == AMMON_GEMV_PLAIN_ARGMAX ? rt->k.gemv_argmax[dt][vec]
                                                         : rt->k.gemv[dt][vec][a.mode];
  uint32_t grid = gemv_grid(rt, fn, lds, p.row_blocks, a.mode);
  if (a.mode == AMMON_GEMV_PLAIN_ARGMAX)
    AMMON_CHECK(grid <= a.cand_cap, "%s: scratch holds %u candidates, the launch needs %u", what,
                a.cand_cap, grid);
  if (grid_out) *grid_out = grid;
  // the GEMV kernels' leading scalar arguments (preloaded into SGPRs), then
  // the parameter struct
  DeviceGuard guard(rt->device);
  hipStream_t st = stream ? (hipStream_t)stream : rt->stream;
  void *args[] = {&p.w0, &p.w1,   &p.w2,      &p.n,  &p.rows, &p.row_blocks,
                  &p.d,  &p.kv_dim, &grid, &p};
  hipError_t e = hipModuleLaunchKernel(fn, grid, 1, 1, kWorkgroup, 1, 1, (uint32_t)lds, st, args,
                                       nullptr);
  if (e != hipSuccess) return hip_error(e, what);
  return AMMON_OK;
}

// ---- attention ------------------------------------------------------------------
int att_chunk_index(ammon_dtype kv, uint32_t head, const void *k, const void *v) {
  // CH = 8 (bf16 only), 4, 2, 1 -> index 0..3; the widest that divides head
  // and keeps the cache bases aligned to a chunk.
  const uintptr_t bits = (uintptr_t)k | (uintptr_t)v;
  const size_t es = dsize(kv);
  const int chs[4] = {8, 4, 2, 1};
  for (int i = (kv == AMMON_BF16 ? 0 : 1); i < 4; ++i) {
    const uint32_t ch = (uint32_t)chs[i];
    if (head % ch == 0 && (bits % (ch * es)) == 0 && head / ch <= 64) return i;
  }
  return -1;
}

int att_group_index(uint32_t g) {
  if (g <= 1) return 0;
  if (g <= 2) return 1;
  if (g <= 4) return 2;
  if (g <= 8) return 3;
  return -1;
}

// Pass-1 variant for a cache layout, or NULL when no chunk width fits.
// split_len 0: the kernel a split of 128 positions would take (occupancy
// queries before the split is chosen).
hipFunction_t attention_kernel(ammon_runtime *rt, ammon_dtype kv_dtype, uint32_t q_heads,
                               uint32_t kv_heads, uint32_t head, const void *k, const void *v,
                               uint32_t split_len) {
  const int ci = att_chunk_index(kv_dtype, head, k, v);
  if (ci < 0) return nullptr;
  const int gi = att_group_index(q_heads / kv_heads);
  const int dt = kv_dtype == AMMON_BF16 ? 1 : 0;
  const uint32_t g = q_heads / kv_heads;
  // head 128, widest chunk, power-of-two group: the compile-time variant
  const bool h128 = head == 128 && ci == (dt ? 0 : 1) && (g & (g - 1)) == 0;
  if (h128 && dt) {
    // LDS chunk buffers: one for a split of one 64-position chunk, else two
    // (a split of up to two chunks is requested whole at the start; longer
    // ones stream through the ring)
    const uint32_t chunks = split_len ? (split_len + 63) / 64 : 2;
    return rt->k.att_partial_staged[chunks >= 2 ? 1 : 0][gi];
  }
  return h128 ? rt->k.att_partial_h128_f32[gi] : rt->k.att_partial[dt][ci][gi];
}

ammon_status attention_check(ammon_runtime *rt, const char *what, uint32_t q_heads,
                             uint32_t kv_heads, uint32_t head, uint32_t seq, uint32_t split_len) {
  (void)rt;
  AMMON_CHECK(q_heads > 0 && kv_heads > 0 && head > 0 && seq > 0,
              "%s: empty shape (q_heads=%u, kv_heads=%u, head=%u, seq=%u)", what, q_heads,
              kv_heads, head, seq);
  AMMON_CHECK(head <= AMMON_ATTENTION_MAX_HEAD, "%s: head size %u exceeds %u", what, head,
              AMMON_ATTENTION_MAX_HEAD);
  AMMON_CHECK(q_heads % kv_heads == 0, "%s: q_heads %u is not a multiple of kv_heads %u", what,
              q_heads, kv_heads);
  AMMON_CHECK(q_heads / kv_heads <= 8, "%s: %u query heads per kv head exceeds 8", what,
              q_heads / kv_heads);
  AMMON_CHECK(split_len >= 1 && split_len <= AMMON_ATTENTION_MAX_SPLIT,
              "%s: split length %u outside [1, %u]", what, split_len, AMMON_ATTENTION_MAX_SPLIT);
  AMMON_CHECK(ammon_attention_splits(seq, split_len) <= AMMON_ATTENTION_MAX_SPLITS,
              "%s: %u splits exceed %u; use a longer split", what,
              ammon_attention_splits(seq, split_len), AMMON_ATTENTION_MAX_SPLITS);
  return AMMON_OK;
}

}  // namespace

extern "C" {

// ---- embed ---------------------------------------------------------------------
static ammon_status embed_impl(ammon_runtime *rt, ammon_stream stream, const void *table,
                               ammon_dtype dt, uint32_t vocab, uint32_t dim,
                               const ammon_decode_step *step, const uint32_t *ids, uint32_t rows,
                               float *x, const char *what) {
  REQUIRE_RT();
  AMMON_CHECK(valid_dtype(dt), "%s: unknown table dtype %d", what, (int)dt);
  AMMON_CHECK(table && x, "%s: NULL table or x", what);
  AMMON_CHECK(ids || step, "%s: no token source", what);
  AMMON_CHECK(vocab > 0 && dim > 0, "%s: empty table (vocab=%u, dim=%u)", what, vocab, dim);
  VALIDATE_ONLY();
  ammon_k_embed p = {table, (const ammon_k_step *)step, ids, x, vocab, dim, rows, (uint32_t)dt};
  const uint32_t per_lane = dt == AMMON_BF16 ? 8 : 4;
  const uint32_t gx = std::min<uint32_t>(cdiv(dim, (uint64_t)kWorkgroup * per_lane), 64);
  return launch(rt, stream, rt->k.embed, gx, rows, 0, p, what);
}

ammon_status ammon_embed(ammon_runtime *rt, ammon_stream stream, const void *table,
                         ammon_dtype table_dtype, uint32_t vocab, uint32_t dim,
                         const ammon_decode_step *step, float *x) {
  AMMON_CHECK(step != nullptr, "embed: parameter `step` is NULL");
  return embed_impl(rt, stream, table, table_dtype, vocab, dim, step, nullptr, 1, x, "embed");
}

ammon_status ammon_embed_rows(ammon_runtime *rt, ammon_stream stream, const void *table,
                              ammon_dtype table_dtype, uint32_t vocab, uint32_t dim,
                              const uint32_t *ids, uint32_t rows, float *x) {
  AMMON_CHECK(ids != nullptr, "embed_rows: parameter `ids` is NULL");
  AMMON_CHECK(rows <= 65535, "embed_rows: %u rows exceed 65535", rows);
  return embed_impl(rt, stream, table, table_dtype, vocab, dim, nullptr, ids, rows, x,
                    "embed_rows");
}

// ---- rmsnorm ----------------------------------------------------------------------
ammon_status ammon_rmsnorm(ammon_runtime *rt, ammon_stream stream, const float *x,
                           const void *weight, ammon_dtype weight_dtype, float *out,
                           uint32_t rows, uint32_t dim, float eps) {
  REQUIRE_RT();
  AMMON_CHECK(x && weight && out, "rmsnorm: NULL x, weight or out");
  AMMON_CHECK(valid_dtype(weight_dtype), "rmsnorm: unknown weight dtype %d", (int)weight_dtype);
  AMMON_CHECK(dim > 0, "rmsnorm: `dim` is 0");
  AMMON_CHECK(std::isfinite(eps) && eps >= 0.f, "rmsnorm: eps must be finite and >= 0");
  AMMON_CHECK(out == x || !overlaps(x, (size_t)rows * dim * 4, out, (size_t)rows * dim * 4),
              "rmsnorm: out partially overlaps x");
  VALIDATE_ONLY();
  ammon_k_rmsnorm p = {x, weight, out, rows, dim, (uint32_t)weight_dtype, eps};
  return launch(rt, stream, rt->k.rmsnorm, rows, 1, 0, p, "rmsnorm");
}

// ---- rope / cache store ----------------------------------------------------------------
static ammon_status rope_impl(ammon_runtime *rt, ammon_stream stream, float *q, uint32_t q_heads,
                              const float *k_proj, uint32_t kv_heads, uint32_t head,
                              void *k_cache, ammon_dtype kv_dtype, uint32_t seq,
                              const ammon_decode_step *step, const float *table,
                              const char *what) {
  REQUIRE_RT();
  AMMON_CHECK(q && k_cache && step && table, "%s: NULL q, k cache, step or table", what);
  AMMON_CHECK(valid_dtype(kv_dtype), "%s: unknown kv dtype %d", what, (int)kv_dtype);
  AMMON_CHECK(head >= 2 && head % 2 == 0, "%s: head size %u must be even", what, head);
  AMMON_CHECK(q_heads > 0 && kv_heads > 0 && seq > 0, "%s: empty shape", what);
  const uint64_t q_numel = (uint64_t)q_heads * head, kv_dim = (uint64_t)kv_heads * head;
  AMMON_CHECK(kv_dim <= q_numel, "%s: kv width must be even and no wider than q", what);
  VALIDATE_ONLY();
  ammon_k_rope p = {q, k_proj, k_cache, (const ammon_k_step *)step, table,
                    (uint32_t)q_numel, (uint32_t)kv_dim, head, seq, (uint32_t)kv_dtype};
  return launch(rt, stream, rt->k.rope, cdiv(q_numel / 2, kWorkgroup), 1, 0, p, what);
}

ammon_status ammon_rope_store(ammon_runtime *rt, ammon_stream stream, float *q,
                              uint32_t q_heads, const float *k_proj, uint32_t kv_heads,
                              uint32_t head, void *k_cache, ammon_dtype kv_dtype, uint32_t seq,
                              const ammon_decode_step *step, const float *table) {
  AMMON_CHECK(k_proj != nullptr, "rope_store: parameter `k_proj` is NULL");
  return rope_impl(rt, stream, q, q_heads, k_proj, kv_heads, head, k_cache, kv_dtype, seq, step,
                   table, "rope_store");
}

ammon_status ammon_rope(ammon_runtime *rt, ammon_stream stream, float *q, uint32_t q_heads,
                        uint32_t kv_heads, uint32_t head, void *k_cache, ammon_dtype kv_dtype,
                        uint32_t seq, const ammon_decode_step *step, const float *table) {
  return rope_impl(rt, stream, q, q_heads, nullptr, kv_heads, head, k_cache, kv_dtype, seq, step,
                   table, "rope");
}

ammon_status ammon_cache_store(ammon_runtime *rt, ammon_stream stream, const float *src,
                               uint32_t kv_heads, uint32_t head, void *cache,
                               ammon_dtype kv_dtype, uint32_t seq,
                               const ammon_decode_step *step) {
  REQUIRE_RT();
  AMMON_CHECK(src && cache && step, "cache_store: NULL src, cache or step");
  AMMON_CHECK(valid_dtype(kv_dtype), "cache_store: unknown dtype %d", (int)kv_dtype);
  AMMON_CHECK(kv_heads > 0 && head > 0 && seq > 0, "cache_store: empty shape");
  VALIDATE_ONLY();
  const uint32_t kv_dim = kv_heads * head;
  ammon_k_cache_store p = {src, cache, (const ammon_k_step *)step, kv_dim, head, seq,
                           (uint32_t)kv_dtype};
  return launch(rt, stream, rt->k.cache_store, cdiv(kv_dim, kWorkgroup), 1, 0, p, "cache_store");
}

// ---- attention ---------------------------------------------------------------------------
}  // extern "C"

namespace {
// Pass 1; with `single_out` (a decode whose split covers the whole cache) it
// writes the merged output itself and no pass 2 is needed.
ammon_status attention_pass1(ammon_runtime *rt, ammon_stream stream, const float *q,
                             uint32_t q_heads, const void *k_cache, const void *v_cache,
                             ammon_dtype kv_dtype, uint32_t kv_heads, uint32_t head, uint32_t seq,
                             const ammon_decode_step *step, uint32_t split_len, float *partial,
                             float *single_out) {
  AMMON_CHECK(q && k_cache && v_cache && step && partial,
              "attention_partial: NULL q, cache, step or partial");
  AMMON_CHECK(valid_dtype(kv_dtype), "attention_partial: unknown kv dtype %d", (int)kv_dtype);
  ammon_status st = attention_check(rt, "attention_partial", q_heads, kv_heads, head, seq, split_len);
  if (st != AMMON_OK) return st;
  hipFunction_t f =
      attention_kernel(rt, kv_dtype, q_heads, kv_heads, head, k_cache, v_cache, split_len);
  AMMON_CHECK(f, "attention_partial: head %u needs an even width above 64", head);
  VALIDATE_ONLY();
  const uint32_t splits = ammon_attention_splits(seq, split_len);
  ammon_k_attention p = {q, k_cache, v_cache, (const ammon_k_step *)step, partial, single_out,
                         q_heads, kv_heads, head, seq, split_len, splits, 0, seq,
                         single_out ? 1u : 0u, nullptr, 0, 0, 0, 0, 0};
  return launch_att(rt, stream, f, splits, kv_heads, 1, p, "attention_partial");
}
}  // namespace

extern "C" {

ammon_status ammon_attention_partial(ammon_runtime *rt, ammon_stream stream, const float *q,
                                     uint32_t q_heads, const void *k_cache, const void *v_cache,
                                     ammon_dtype kv_dtype, uint32_t kv_heads, uint32_t head,
                                     uint32_t seq, const ammon_decode_step *step,
                                     uint32_t split_len, float *partial) {
  REQUIRE_RT();
  return attention_pass1(rt, stream, q, q_heads, k_cache, v_cache, kv_dtype, kv_heads, head, seq,
                         step, split_len, partial, nullptr);
}

ammon_status ammon_attention_combine(ammon_runtime *rt, ammon_stream stream,
                                     const float *partial, uint32_t q_heads, uint32_t head,
                                     uint32_t seq, const ammon_decode_step *step,
                                     uint32_t split_len, float *out) {
  return ammon_attention_combine_warm(rt, stream, partial, q_heads, head, seq, step, split_len,
                                      out, nullptr, AMMON_BF16, 0, 0, 0, 0);
}

ammon_status ammon_attention_combine_warm(ammon_runtime *rt, ammon_stream stream,
                                          const float *partial, uint32_t q_heads, uint32_t head,
                                          uint32_t seq, const ammon_decode_step *step,
                                          uint32_t split_len, float *out, const void *next_w,
                                          ammon_dtype next_dtype, uint32_t next_rows,
                                          uint32_t next_n, uint32_t warm_row_bytes,
                                          uint32_t min_position) {
  REQUIRE_RT();
  AMMON_CHECK(partial && step && out, "attention_combine: NULL partial, step or out");
  AMMON_CHECK(q_heads > 0 && head > 0 && seq > 0,
              "attention_combine: empty shape (q_heads=%u, head=%u, seq=%u)", q_heads, head, seq);
  AMMON_CHECK(head <= AMMON_ATTENTION_MAX_HEAD, "attention_combine: head size %u exceeds %u",
              head, AMMON_ATTENTION_MAX_HEAD);
  AMMON_CHECK(split_len >= 1 && split_len <= AMMON_ATTENTION_MAX_SPLIT,
              "attention_combine: split length %u outside [1, %u]", split_len,
              AMMON_ATTENTION_MAX_SPLIT);
  AMMON_CHECK(ammon_attention_splits(seq, split_len) <= AMMON_ATTENTION_MAX_SPLITS,
              "attention_combine: %u splits exceed %u", ammon_attention_splits(seq, split_len),
              AMMON_ATTENTION_MAX_SPLITS);
  if (next_w) {
    AMMON_CHECK(valid_dtype(next_dtype), "attention_combine: unknown next weight dtype %d",
                (int)next_dtype);
    AMMON_CHECK(next_rows > 0 && next_n > 0, "attention_combine: empty next matrix (%u x %u)",
                next_rows, next_n);
  }
  VALIDATE_ONLY();
  ammon_k_attention p = {nullptr, nullptr, nullptr, (const ammon_k_step *)step, (float *)partial,
                         out, q_heads, 1, head, seq, split_len,
                         ammon_attention_splits(seq, split_len), 0, seq, 0, nullptr, 0, 0, 0, 0, 0};
  const uint32_t grid = q_heads * cdiv(head, 8);
  if (next_w) {
    // The next GEMV (a RESIDUAL-mode ammon_gemv of next_rows x next_n) gives
    // row block j (kGemvRowsPerWave * kGemvWaves rows) to workgroup j % its
    // grid, which runs on XCD (j % grid) % 8, and requests each row's first
    // tile (64 lanes x kGemvTileChunks chunks) first; merge workgroup i
    // runs on XCD i % 8.  So merge workgroup i warms block i when every block
    // has a workgroup of its own and both grids are whole multiples of the 8
    // XCDs.  Warming half a tile bought nothing when measured (a wave waits
    // for the slowest of its loads), and more than ~20 MB overflows the 8
    // XCDs' 4 MB L2s.  A workgroup warms whole blocks (its buffer covers
    // rows_per_wg rows), so a ragged last block would reach past the matrix:
    // such a matrix is not warmed.
    const uint64_t row_bytes = (uint64_t)next_n * dsize(next_dtype);
    const uint32_t rows_per_wg = kGemvRowsPerWave * kGemvWaves;
    const uint32_t blocks = cdiv(next_rows, rows_per_wg);
    uint64_t tile_row_bytes = 0;
    const uint32_t gemv_grid =
        gemv_grid_for(rt, next_w, next_dtype, next_n, next_rows, &tile_row_bytes);
    const uint64_t want = warm_row_bytes ? warm_row_bytes : tile_row_bytes;
    const uint64_t bytes = std::min<uint64_t>(want, row_bytes) / 128 * 128;
    if (next_rows % rows_per_wg == 0 && gemv_grid % 8 == 0 && grid % 8 == 0 &&
        blocks == gemv_grid && blocks <= grid &&
        bytes > 0 && (uint64_t)rows_per_wg * row_bytes < (1ull << 31) &&
        bytes / 128 * rows_per_wg <= (uint64_t)kWorkgroup * 4 &&
        (uint64_t)blocks * rows_per_wg * bytes <= kWarmMaxBytes) {
      p.warm = next_w;
      p.warm_row_bytes = (uint32_t)row_bytes;
      p.warm_rows = rows_per_wg;
      p.warm_bytes = (uint32_t)bytes;
      p.warm_blocks = blocks;
      p.warm_min_pos = min_position;
    }
  }
  return launch_att(rt, stream, rt->k.att_combine, q_heads, cdiv(head, 8), 1, p,
                    "attention_combine");
}

uint32_t ammon_attention_default_split_for(ammon_runtime *rt, uint32_t q_heads,
                                           uint32_t kv_heads, uint32_t head,
                                           ammon_dtype kv_dtype, uint32_t seq) {
  // Two units per CU where two pass-1 workgroups of this shape's kernel fit
  // on a CU; one where only one does (the generic bf16 kernel of an 8:1
  // group): one round of long units, not two rounds of short ones.  A
  // two-buffer head-128 8:1 kernel that fit once per CU measured it on the
  // 70B-shaped layer at 32768 positions: 0.635-0.636 against 0.639-0.642 ms
  // per step.
  //
  // The matrix-core kernels (bf16 cache, head 128, power-of-two group)
  // score 64-position chunks, so a split never goes below one chunk: a
  // shorter one leaves most of each workgroup's chunk past its split
  // (32 q / 8 kv heads, 1024 positions: 8.6 us at split 64 against 10.0 at
  // 16; 2048: 9.7 against 10.6 at 32).
  uint32_t per_cu = 2, min_split = 16;
  if (rt && kv_heads > 0 && q_heads % kv_heads == 0 && q_heads / kv_heads <= 8 && head > 0 &&
      head <= AMMON_ATTENTION_MAX_HEAD && valid_dtype(kv_dtype)) {
    DeviceGuard guard(rt->device);
    hipFunction_t f =
        attention_kernel(rt, kv_dtype, q_heads, kv_heads, head, nullptr, nullptr, 0);
    if (f) per_cu = std::min<uint32_t>(occupancy(rt, f, 0), 2);
    const uint32_t g = q_heads / kv_heads;
    if (kv_dtype == AMMON_BF16 && head == 128 && (g & (g - 1)) == 0) min_split = 64;
  }
  return default_split(rt, kv_heads, seq, per_cu, min_split);
}

ammon_status ammon_attention_decode(ammon_runtime *rt, ammon_stream stream, const float *q,
                                    uint32_t q_heads, const void *k_cache, const void *v_cache,
                                    ammon_dtype kv_dtype, uint32_t kv_heads, uint32_t head,
                                    uint32_t seq, const ammon_decode_step *step,
                                    uint32_t split_len, float *partial, size_t partial_bytes,
                                    float *out) {
  REQUIRE_RT();
  AMMON_CHECK(partial_bytes >= ammon_attention_scratch_bytes(q_heads, head, seq, split_len),
              "attention: partial scratch must be %zu bytes ([%u, %u, %u] fp32)",
              ammon_attention_scratch_bytes(q_heads, head, seq, split_len), q_heads,
              ammon_attention_splits(seq, split_len), head + 2);
  ammon_status st = ammon_attention_partial(rt, AMMON_STREAM_VALIDATE, q, q_heads, k_cache,
                                            v_cache, kv_dtype, kv_heads, head, seq, step,
                                            split_len, partial);
  if (st != AMMON_OK) return st;
  st = ammon_attention_combine(rt, AMMON_STREAM_VALIDATE, partial, q_heads, head, seq, step,
                               split_len, out);
  if (st != AMMON_OK) return st;
  VALIDATE_ONLY();
  if (ammon_attention_splits(seq, split_len) == 1)  // one launch: pass 1 writes out
    return attention_pass1(rt, stream, q, q_heads, k_cache, v_cache, kv_dtype, kv_heads, head,
                           seq, step, split_len, partial, out);
  st = ammon_attention_partial(rt, stream, q, q_heads, k_cache, v_cache, kv_dtype, kv_heads, head,
                               seq, step, split_len, partial);
  if (st != AMMON_OK) return st;
  return ammon_attention_combine(rt, stream, partial, q_heads, head, seq, step, split_len, out);
}

// ---- prompt prefill ---------------------------------------------------------------------
size_t ammon_attention_prefill_scratch_bytes(uint32_t tokens, uint32_t q_heads, uint32_t head,
                                             uint32_t ctx, uint32_t split_len) {
  return (size_t)tokens * ammon_attention_scratch_bytes(q_heads, head, ctx, split_len);
}

ammon_status ammon_attention_prefill(ammon_runtime *rt, ammon_stream stream, const float *q,
                                     uint32_t tokens, uint32_t q_heads, const void *k_cache,
                                     const void *v_cache, ammon_dtype kv_dtype, uint32_t kv_heads,
                                     uint32_t head, uint32_t seq, const ammon_decode_step *step,
                                     uint32_t ctx, uint32_t split_len, float *partial,
                                     size_t partial_bytes, float *out) {
  REQUIRE_RT();
  AMMON_CHECK(q && k_cache && v_cache && step && partial && out,
              "attention_prefill: NULL q, cache, step, partial or out");
  AMMON_CHECK(valid_dtype(kv_dtype), "attention_prefill: unknown kv dtype %d", (int)kv_dtype);
  AMMON_CHECK(tokens > 0, "attention_prefill: no query tokens");
  ammon_status st = attention_check(rt, "attention_prefill", q_heads, kv_heads, head, seq, split_len);
  if (st != AMMON_OK) return st;
  AMMON_CHECK(ctx >= 1 && ctx <= seq, "attention_prefill: ctx %u outside [1, seq=%u]", ctx, seq);
  const size_t need = ammon_attention_prefill_scratch_bytes(tokens, q_heads, head, ctx, split_len);
  AMMON_CHECK(partial_bytes >= need, "attention_prefill: partial scratch must be %zu bytes", need);
  const size_t qbytes = (size_t)tokens * q_heads * head * 4;
  AMMON_CHECK(!overlaps(out, qbytes, q, qbytes) && !overlaps(out, qbytes, partial, need) &&
                  !overlaps(q, qbytes, partial, need),
              "attention_prefill: q, partial and out must not overlap");
  hipFunction_t f =
      attention_kernel(rt, kv_dtype, q_heads, kv_heads, head, k_cache, v_cache, split_len);
  AMMON_CHECK(f, "attention_prefill: head %u needs an even width above 64", head);
  VALIDATE_ONLY();
  // the partial layout and the grid cover ctx positions: [tokens][q_heads][splits][head + 2];
  // a token at position >= ctx (the host cannot see step->position) gets the
  // out-of-range treatment -- NaN output, no partial -- like one past seq
  const uint32_t splits = ammon_attention_splits(ctx, split_len);
  ammon_k_attention p = {q, k_cache, v_cache, (const ammon_k_step *)step, partial, out,
                         q_heads, kv_heads, head, seq, split_len, splits, 0, ctx, 0, nullptr, 0, 0, 0, 0, 0};
  st = launch_att(rt, stream, f, splits, kv_heads, tokens, p, "attention_prefill");
  if (st != AMMON_OK) return st;
  return launch_att(rt, stream, rt->k.att_combine_waves, cdiv(q_heads, kWaves), 1, tokens, p,
                    "attention_prefill");
}

namespace {

struct GemmArgs {
  int mode;
  const void *w0, *w1, *w2;
  ammon_dtype w_dtype;
  uint32_t d, n, rows, tokens;
  const float *x;
  const float *residual;
  float *y;
  size_t y_bytes;
  void *k_cache, *v_cache;
  const ammon_decode_step *step;
  const float *table;
  uint32_t kv_dim, head, seq;
  ammon_dtype kv_dtype;
  void *ws;  // PLAIN / RESIDUAL: optional workspace for a split reduction
  size_t ws_bytes;
};

ammon_status gemm_check_and_launch(ammon_runtime *rt, ammon_stream stream, const GemmArgs &a,
                                   const char *what) {
  AMMON_CHECK(valid_dtype(a.w_dtype), "%s: unknown weight dtype %d", what, (int)a.w_dtype);
  AMMON_CHECK(a.w0 && a.x && a.y, "%s: NULL weight, x or y", what);
  AMMON_CHECK(a.n > 0 && a.d > 0 && a.tokens > 0, "%s: empty shape (d=%u, n=%u, tokens=%u)", what,
              a.d, a.n, a.tokens);
  AMMON_CHECK(a.n % 8 == 0, "%s: reduction length %u must be a multiple of 8", what, a.n);
  AMMON_CHECK((uint64_t)a.n * 32 * 4 < (1ull << 31), "%s: reduction length %u too large", what,
              a.n);
  AMMON_CHECK(a.rows < (1u << 31), "%s: too many rows", what);
  const uintptr_t bits = (uintptr_t)a.w0 | (uintptr_t)a.w1 | (uintptr_t)a.w2 | (uintptr_t)a.x;
  AMMON_CHECK((bits & 15u) == 0, "%s: weights and x must be 16-byte aligned", what);
  const size_t xbytes = (size_t)a.tokens * a.n * 4;
  AMMON_CHECK(!overlaps(a.x, xbytes, a.y, a.y_bytes), "%s: y overlaps x", what);
  if (a.residual)
    AMMON_CHECK(!overlaps(a.x, xbytes, a.residual, a.y_bytes), "%s: residual overlaps x", what);
  if (a.ws) {
    AMMON_CHECK(!overlaps(a.ws, a.ws_bytes, a.x, xbytes) && !overlaps(a.ws, a.ws_bytes, a.y, a.y_bytes) &&
                    !(a.residual && overlaps(a.ws, a.ws_bytes, a.residual, a.y_bytes)),
                "%s: workspace overlaps x, y or residual", what);
    AMMON_CHECK(((uintptr_t)a.ws & 15u) == 0, "%s: workspace must be 16-byte aligned", what);
  }
  VALIDATE_ONLY();
  ammon_k_gemm p = {};
  p.w0 = a.w0;
  p.w1 = a.w1;
  p.w2 = a.w2;
  p.x = a.x;
  p.residual = a.residual;
  p.y = a.y;
  p.k_cache = a.k_cache;
  p.v_cache = a.v_cache;
  p.step = (const ammon_k_step *)a.step;
  p.table = a.table;
  p.d = a.d;
  p.n = a.n;
  p.rows = a.rows;
  p.tokens = a.tokens;
  p.kv_dim = a.kv_dim;
  p.head = a.head;
  p.seq = a.seq;
  p.kv_dtype = (uint32_t)a.kv_dtype;
  // bf16 W: register-blocked tiles of 64 or 32 tokens x 4 waves x 4 or 2
  // 16-row tiles per wave, the reduction optionally split into 2..8 ranges
  // (plain / residual with a workspace).  Take the largest tile whose grid,
  // split into ranges of at least 16 chunks, gives at least 3/4 of a
  // workgroup per CU, with the smallest split that does; else (64+ tokens,
  // or a splittable reduction) the smallest tile split into ranges of at
  // least 8 chunks; below 64 tokens a projection that fills the device no
  // way keeps the 16/32-token tiles below, whose reduction split over the
  // waves suits few rows.  Measured on the Llama-3-8B projections at
  // 16..512 tokens (e.g. w2 at 512 tokens: 64-row x 64-token tiles split in
  // two 197 us, unsplit 128-row x 64-token tiles 253 us).
  const uint32_t cus = (uint32_t)std::max(rt->info.compute_units, 1);
  if (a.w_dtype == AMMON_BF16 && rt->gemm_big != 0) {
    const uint32_t covered = a.mode == AMMON_GEMV_SWIGLU ? a.d : a.rows;
    const uint32_t per4 = a.mode == AMMON_GEMV_SWIGLU ? 128 : 256;  // RT 4: rows per workgroup
    auto wgs = [&](int t64, int rt4) {
      return (uint64_t)cdiv(covered, rt4 ? per4 : per4 / 2) * cdiv(a.tokens, t64 ? 64 : 32);
    };
    const uint32_t chunks = (uint32_t)cdiv(a.n, 64);
    const bool splittable = a.ws && a.mode != AMMON_GEMV_SWIGLU;
    // the most ranges of at least `len` chunks the workspace holds
    auto kmax_of = [&](uint32_t len) {
      uint32_t k = 1;
      if (splittable)
        while (k < 8 && chunks / (k * 2) >= len &&
               (uint64_t)k * 2 * a.tokens * a.rows * 4 <= a.ws_bytes)
          k *= 2;
      return k;
    };
    uint32_t kmax = kmax_of(16);
    const uint64_t need = ((uint64_t)cus * 3 + 3) / 4;
    int t64 = -1, rt4 = 0;
    if (rt->gemm_big > 0) {
      t64 = rt->gemm_big / 10 == 4;
      rt4 = rt->gemm_big % 10 == 4;
    } else {
      const int order[4][2] = {{1, 1}, {1, 0}, {0, 1}, {0, 0}};
      for (const auto &o : order)
        if ((a.tokens >= 64 || !o[0]) && wgs(o[0], o[1]) * kmax >= need) {
          t64 = o[0];
          rt4 = o[1];
          break;
        }
      if (t64 < 0 && (a.tokens >= 64 || splittable)) {
        t64 = rt4 = 0;
        kmax = kmax_of(8);
      }
    }
    if (t64 >= 0) {
      const uint64_t tiles = cdiv(a.tokens, t64 ? 64 : 32);
      const uint64_t groups = cdiv(cdiv(covered, rt4 ? per4 : per4 / 2), 8);
      uint32_t ksplit = 1;
      while (ksplit < kmax && wgs(t64, rt4) * ksplit < need) ksplit *= 2;
      if (ksplit > 1) {
        p.ws = (float *)a.ws;
        p.ksplit = ksplit;
        p.kchunks = cdiv(chunks, ksplit);
      }
      AMMON_CHECK(groups * 8 * tiles * ksplit < (1ull << 31), "%s: grid too large", what);
      ammon_status st = launch(rt, stream, rt->k.gemm_big[t64 ? 0 : 1][rt4 ? 0 : 1][a.mode],
                               (uint32_t)(groups * 8 * tiles * ksplit), 1, 0, p, what);
      if (st != AMMON_OK || ksplit == 1) return st;
      // the ranges' sums (QKV: per row pair, then the rotation and stores)
      const bool qkv = a.mode == AMMON_GEMV_QKV;
      const uint64_t elems = (uint64_t)a.tokens * (qkv ? a.rows / 2 : a.d);
      const uint32_t blocks = (uint32_t)std::min<uint64_t>(cdiv(elems, kWorkgroup), cus * 4ull);
      return launch(rt, stream, qkv ? rt->k.gemm_reduce_qkv : rt->k.gemm_reduce, blocks, 1, 0, p,
                    what);
    }
  }
  // 64 virtual rows x 16 tokens per workgroup for short prompts, x 32 beyond;
  // 16 rows (the reduction split over the four waves) when 64-row tiles
  // would occupy at most half of the CUs -- measured at the Llama-3-8B
  // shape: the 4096-row projections run 1.2-1.9x faster split at up to 48
  // tokens and the 6144-row QKV 1.1-1.5x up to 32 tokens, while QKV at 48
  // tokens and the 28672 gate/up rows lose, every split x chunk being
  // staged for a quarter of the rows.  The kernel maps a 1-D grid of
  // (row-block groups of 8) x token tiles x 8.
  const int wide = a.tokens > 16 ? 1 : 0;
  const uint64_t tiles = cdiv(a.tokens, wide ? 32 : 16);
  const int split = rt->gemm_split >= 0 ? rt->gemm_split
                                        : ((uint64_t)cdiv(a.rows, 64) * tiles * 4 <= 2 * cus ? 1 : 0);
  hipFunction_t f = rt->k.gemm[a.w_dtype == AMMON_BF16 ? 1 : 0][wide][split][a.mode];
  const uint64_t groups = cdiv(a.rows, (split ? 16 : 64) * 8);
  AMMON_CHECK(groups * 8 * tiles < (1ull << 31), "%s: grid too large", what);
  return launch(rt, stream, f, (uint32_t)(groups * 8 * tiles), 1, 0, p, what);
}

}  // namespace

size_t ammon_prefill_gemm_workspace_bytes(uint32_t rows, uint32_t tokens) {
  return (size_t)8 * tokens * rows * sizeof(float);
}

ammon_status ammon_prefill_gemm(ammon_runtime *rt, ammon_stream stream, const void *w,
                                ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x,
                                uint32_t tokens, float *y, const float *residual) {
  return ammon_prefill_gemm_ws(rt, stream, w, w_dtype, d, n, x, tokens, y, residual, nullptr, 0);
}

ammon_status ammon_prefill_gemm_ws(ammon_runtime *rt, ammon_stream stream, const void *w,
                                   ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x,
                                   uint32_t tokens, float *y, const float *residual,
                                   void *workspace, size_t workspace_bytes) {
  REQUIRE_RT();
  GemmArgs a = {};
  a.mode = residual ? AMMON_GEMV_RESIDUAL : AMMON_GEMV_PLAIN;
  a.w0 = w;
  a.w_dtype = w_dtype;
  a.d = d;
  a.n = n;
  a.rows = d;
  a.tokens = tokens;
  a.x = x;
  a.residual = residual;
  a.y = y;
  a.y_bytes = (size_t)tokens * d * 4;
  a.ws = workspace;
  a.ws_bytes = workspace ? workspace_bytes : 0;
  return gemm_check_and_launch(rt, stream, a, "prefill_gemm");
}

ammon_status ammon_prefill_qkv_rope_store(ammon_runtime *rt, ammon_stream stream, const float *x,
                                          uint32_t tokens, const void *wq, const void *wk,
                                          const void *wv, ammon_dtype w_dtype, uint32_t dim,
                                          uint32_t q_heads, uint32_t kv_heads, uint32_t head,
                                          float *q, void *k_cache, void *v_cache,
                                          ammon_dtype kv_dtype, uint32_t seq,
                                          const ammon_decode_step *step, const float *table) {
  return ammon_prefill_qkv_rope_store_ws(rt, stream, x, tokens, wq, wk, wv, w_dtype, dim, q_heads,
                                         kv_heads, head, q, k_cache, v_cache, kv_dtype, seq, step,
                                         table, nullptr, 0);
}

ammon_status ammon_prefill_qkv_rope_store_ws(ammon_runtime *rt, ammon_stream stream, const float *x,
                                          uint32_t tokens, const void *wq, const void *wk,
                                          const void *wv, ammon_dtype w_dtype, uint32_t dim,
                                          uint32_t q_heads, uint32_t kv_heads, uint32_t head,
                                          float *q, void *k_cache, void *v_cache,
                                          ammon_dtype kv_dtype, uint32_t seq,
                                          const ammon_decode_step *step, const float *table,
                                             void *workspace, size_t workspace_bytes) {
  REQUIRE_RT();
  AMMON_CHECK(wq && wk && wv, "prefill_qkv: NULL wq, wk or wv");
  AMMON_CHECK(k_cache && v_cache && step && table, "prefill_qkv: NULL cache, step or table");
  AMMON_CHECK(valid_dtype(kv_dtype), "prefill_qkv: unknown kv dtype %d", (int)kv_dtype);
  AMMON_CHECK(head >= 16 && head % 16 == 0, "prefill_qkv: head size %u must be a multiple of 16",
              head);
  AMMON_CHECK(q_heads > 0 && kv_heads > 0 && seq > 0, "prefill_qkv: empty shape");
  const uint64_t q_dim = (uint64_t)q_heads * head, kv_dim = (uint64_t)kv_heads * head;
  AMMON_CHECK(kv_dim <= q_dim, "attention: kv width must be even and no wider than q");
  AMMON_CHECK(q_dim + 2 * kv_dim < (1ull << 31), "prefill_qkv: too many rows");
  AMMON_CHECK(!overlaps(k_cache, (size_t)kv_dim * seq * dsize(kv_dtype), v_cache,
                        (size_t)kv_dim * seq * dsize(kv_dtype)),
              "prefill_qkv: key and value caches overlap");
  GemmArgs a = {};
  a.mode = AMMON_GEMV_QKV;
  a.w0 = wq;
  a.w1 = wk;
  a.w2 = wv;
  a.w_dtype = w_dtype;
  a.d = (uint32_t)q_dim;
  a.n = dim;
  a.rows = (uint32_t)(q_dim + 2 * kv_dim);
  a.tokens = tokens;
  a.x = x;
  a.y = q;
  a.y_bytes = (size_t)tokens * q_dim * 4;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.step = step;
  a.table = table;
  a.kv_dim = (uint32_t)kv_dim;
  a.head = head;
  a.seq = seq;
  a.kv_dtype = kv_dtype;
  a.ws = workspace;
  a.ws_bytes = workspace ? workspace_bytes : 0;
  const size_t cache_bytes = (size_t)kv_dim * seq * dsize(kv_dtype);
  AMMON_CHECK(!workspace || (!overlaps(workspace, workspace_bytes, k_cache, cache_bytes) &&
                             !overlaps(workspace, workspace_bytes, v_cache, cache_bytes)),
              "prefill_qkv: workspace overlaps a cache");
  return gemm_check_and_launch(rt, stream, a, "prefill_qkv_rope_store");
}

ammon_status ammon_prefill_gate_up_swiglu(ammon_runtime *rt, ammon_stream stream, const float *x,
                                          uint32_t tokens, const void *w1, const void *w3,
                                          ammon_dtype w_dtype, uint32_t dim, uint32_t hidden,
                                          float *hb) {
  REQUIRE_RT();
  AMMON_CHECK(w1 && w3, "prefill_gate_up_swiglu: NULL w1 or w3");
  AMMON_CHECK((uint64_t)hidden * 2 < (1ull << 31), "prefill_gate_up_swiglu: too many rows");
  GemmArgs a = {};
  a.mode = AMMON_GEMV_SWIGLU;
  a.w0 = w1;
  a.w1 = w3;
  a.w_dtype = w_dtype;
  a.d = hidden;
  a.n = dim;
  a.rows = 2 * hidden;
  a.tokens = tokens;
  a.x = x;
  a.y = hb;
  a.y_bytes = (size_t)tokens * hidden * 4;
  return gemm_check_and_launch(rt, stream, a, "prefill_gate_up_swiglu");
}

// ---- elementwise ---------------------------------------------------------------------------
ammon_status ammon_swiglu(ammon_runtime *rt, ammon_stream stream, float *hb, const float *hb2,
                          uint32_t n) {
  REQUIRE_RT();
  AMMON_CHECK(n == 0 || (hb && hb2), "swiglu: NULL hb or hb2");
  VALIDATE_ONLY();
  ammon_k_elementwise p = {hb, nullptr, hb2, n};
  return launch(rt, stream, rt->k.swiglu, cdiv(n, kWorkgroup), 1, 0, p, "swiglu");
}

ammon_status ammon_add(ammon_runtime *rt, ammon_stream stream, const float *a, const float *b,
                       float *out, uint32_t n) {
  REQUIRE_RT();
  AMMON_CHECK(n == 0 || (a && b && out), "add: NULL operand");
  VALIDATE_ONLY();
  ammon_k_elementwise p = {out, a, b, n};
  return launch(rt, stream, rt->k.add, cdiv(n, kWorkgroup), 1, 0, p, "add");
}

// ---- GEMV family ------------------------------------------------------------------------
ammon_status ammon_gemv(ammon_runtime *rt, ammon_stream stream, const void *w,
                        ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x, float *y,
                        const float *residual) {
  REQUIRE_RT();
  GemvArgs a = {};
  a.mode = residual ? AMMON_GEMV_RESIDUAL : AMMON_GEMV_PLAIN;
  a.w0 = w;
  a.w_dtype = w_dtype;
  a.d = d;
  a.n = n;
  a.rows = d;
  a.x = x;
  a.residual = residual;
  a.y = y;
  return gemv_check_and_launch(rt, stream, a, "gemv");
}

ammon_status ammon_gemv_at_position(ammon_runtime *rt, ammon_stream stream, const void *w,
                                    ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x,
                                    float *xout, uint32_t seq, const ammon_decode_step *step) {
  REQUIRE_RT();
  AMMON_CHECK(step != nullptr, "gemv_at_position: parameter `step` is NULL");
  AMMON_CHECK(seq > 0, "gemv_at_position: `seq` is 0");
  AMMON_CHECK(!overlaps(x, (size_t)n * 4, xout, (size_t)seq * d * 4),
              "gemv_at_position: xout overlaps x");
  GemvArgs a = {};
  a.mode = AMMON_GEMV_PLAIN;
  a.w0 = w;
  a.w_dtype = w_dtype;
  a.d = d;
  a.n = n;
  a.rows = d;
  a.x = x;
  a.y = xout;
  a.step = step;
  a.seq = seq;
  return gemv_check_and_launch(rt, stream, a, "gemv_at_position");
}

ammon_status ammon_gemv_rmsnorm(ammon_runtime *rt, ammon_stream stream, const float *x,
                                const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                const void *w, ammon_dtype w_dtype, uint32_t d, uint32_t n,
                                float *y) {
  REQUIRE_RT();
  AMMON_CHECK(norm_weight != nullptr, "gemv_rmsnorm: parameter `norm_weight` is NULL");
  GemvArgs a = {};
  a.mode = AMMON_GEMV_PLAIN;
  a.w0 = w;
  a.w_dtype = w_dtype;
  a.d = d;
  a.n = n;
  a.rows = d;
  a.x = x;
  a.norm_w = norm_weight;
  a.norm_dtype = norm_dtype;
  a.eps = eps;
  a.y = y;
  return gemv_check_and_launch(rt, stream, a, "gemv_rmsnorm");
}

ammon_status ammon_qkv_rope_store(ammon_runtime *rt, ammon_stream stream, const float *x,
                                  const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                  const void *wq, const void *wk, const void *wv,
                                  ammon_dtype w_dtype, uint32_t dim, uint32_t q_heads,
                                  uint32_t kv_heads, uint32_t head, float *q, void *k_cache,
                                  void *v_cache, ammon_dtype kv_dtype, uint32_t seq,
                                  const ammon_decode_step *step, const float *table) {
  REQUIRE_RT();
  AMMON_CHECK(wq && wk && wv, "qkv: NULL wq, wk or wv");
  AMMON_CHECK(k_cache && v_cache && step && table, "qkv: NULL cache, step or table");
  AMMON_CHECK(valid_dtype(kv_dtype), "qkv: unknown kv dtype %d", (int)kv_dtype);
  AMMON_CHECK(head >= 2 && head % 2 == 0, "qkv: head size %u must be even", head);
  AMMON_CHECK(q_heads > 0 && kv_heads > 0 && seq > 0, "qkv: empty shape");
  const uint64_t q_dim = (uint64_t)q_heads * head, kv_dim = (uint64_t)kv_heads * head;
  AMMON_CHECK(kv_dim <= q_dim, "attention: kv width must be even and no wider than q");
  AMMON_CHECK(q_dim + 2 * kv_dim < (1ull << 31), "qkv: too many rows");
  AMMON_CHECK(!overlaps(k_cache, (size_t)kv_dim * seq * dsize(kv_dtype), v_cache,
                        (size_t)kv_dim * seq * dsize(kv_dtype)),
              "qkv: key and value caches overlap");
  GemvArgs a = {};
  a.mode = AMMON_GEMV_QKV;
  a.w0 = wq;
  a.w1 = wk;
  a.w2 = wv;
  a.w_dtype = w_dtype;
  a.d = (uint32_t)q_dim;
  a.n = dim;
  a.rows = (uint32_t)(q_dim + 2 * kv_dim);
  a.x = x;
  a.norm_w = norm_weight;
  a.norm_dtype = norm_dtype;
  a.eps = eps;
  a.y = q;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.step = step;
  a.table = table;
  a.kv_dim = (uint32_t)kv_dim;
  a.head = head;
  a.seq = seq;
  a.kv_dtype = kv_dtype;
  return gemv_check_and_launch(rt, stream, a, "qkv_rope_store");
}

ammon_status ammon_gate_up_swiglu(ammon_runtime *rt, ammon_stream stream, const float *x,
                                  const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                  const void *w1, const void *w3, ammon_dtype w_dtype,
                                  uint32_t dim, uint32_t hidden, float *hb) {
  REQUIRE_RT();
  AMMON_CHECK(w1 && w3, "gate_up_swiglu: NULL w1 or w3");
  AMMON_CHECK((uint64_t)hidden * 2 < (1ull << 31), "gate_up_swiglu: too many rows");
  GemvArgs a = {};
  a.mode = AMMON_GEMV_SWIGLU;
  a.w0 = w1;
  a.w1 = w3;
  a.w_dtype = w_dtype;
  a.d = hidden;
  a.n = dim;
  a.rows = 2 * hidden;
  a.x = x;
  a.norm_w = norm_weight;
  a.norm_dtype = norm_dtype;
  a.eps = eps;
  a.y = hb;
  return gemv_check_and_launch(rt, stream, a, "gate_up_swiglu");
}

// ---- argmax ---------------------------------------------------------------------------------
static uint32_t argmax_blocks(uint32_t n) {
  return std::max<uint32_t>(1, std::min<uint32_t>(256, cdiv(n, (uint64_t)kWorkgroup * 2)));
}

size_t ammon_argmax_scratch_bytes(uint32_t n) { return (size_t)argmax_blocks(n) * 8; }

static ammon_status argmax_impl(ammon_runtime *rt, ammon_stream stream, const float *logits,
                                uint32_t n, void *scratch, int32_t *out, const int32_t *prompt,
                                uint32_t n_prompt, ammon_decode_step *step, int32_t *tokens,
                                uint32_t max_tokens, const char *what) {
  REQUIRE_RT();
  AMMON_CHECK(logits && scratch, "%s: NULL logits or scratch", what);
  AMMON_CHECK(n > 0, "%s: empty logits", what);
  VALIDATE_ONLY();
  const uint32_t blocks = argmax_blocks(n);
  ammon_k_argmax p = {};
  p.logits = logits;
  p.cand_v = (float *)scratch;
  p.cand_i = (uint32_t *)((char *)scratch + (size_t)blocks * 4);
  p.out = out;
  p.step = (ammon_k_step *)step;
  p.prompt = prompt;
  p.tokens = tokens;
  p.n = n;
  p.blocks = blocks;
  p.n_prompt = n_prompt;
  p.max_tokens = max_tokens;
  ammon_status st = launch(rt, stream, rt->k.argmax_partial, blocks, 1, 0, p, what);
  if (st != AMMON_OK) return st;
  return launch(rt, stream, rt->k.argmax_final, 1, 1, 0, p, what);
}

ammon_status ammon_argmax(ammon_runtime *rt, ammon_stream stream, const float *logits,
                          uint32_t n, void *scratch, int32_t *out) {
  AMMON_CHECK(out != nullptr, "argmax: parameter `out` is NULL");
  return argmax_impl(rt, stream, logits, n, scratch, out, nullptr, 0, nullptr, nullptr, 0,
                     "argmax");
}

size_t ammon_greedy_lm_head_scratch_bytes(ammon_runtime *rt) {
  if (!rt) return 0;
  return (size_t)std::max(rt->info.compute_units, 1) * rt->gemv_wgs_per_cu * 8;
}

ammon_status ammon_greedy_lm_head(ammon_runtime *rt, ammon_stream stream, const float *x,
                                  const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                  const void *w, ammon_dtype w_dtype, uint32_t vocab,
                                  uint32_t dim, float *logits, void *scratch,
                                  size_t scratch_bytes, const int32_t *prompt, uint32_t n_prompt,
                                  ammon_decode_step *step, int32_t *tokens, uint32_t max_tokens) {
  REQUIRE_RT();
  AMMON_CHECK(norm_weight && scratch && step, "greedy_lm_head: NULL norm weight, scratch or step");
  AMMON_CHECK(n_prompt == 0 || prompt != nullptr, "greedy_lm_head: NULL prompt");
  AMMON_CHECK(scratch_bytes >= ammon_greedy_lm_head_scratch_bytes(rt),
              "greedy_lm_head: scratch must be %zu bytes", ammon_greedy_lm_head_scratch_bytes(rt));
  const uint32_t cap = (uint32_t)std::min<size_t>(scratch_bytes / 8, 0xffffffffu);
  GemvArgs a = {};
  a.mode = AMMON_GEMV_PLAIN_ARGMAX;
  a.w0 = w;
  a.w_dtype = w_dtype;
  a.d = vocab;
  a.n = dim;
  a.rows = vocab;
  a.x = x;
  a.norm_w = norm_weight;
  a.norm_dtype = norm_dtype;
  a.eps = eps;
  a.y = logits;
  a.cand_v = (float *)scratch;
  a.cand_i = (uint32_t *)((char *)scratch + (size_t)cap * 4);
  a.cand_cap = cap;
  uint32_t grid = 0;
  ammon_status st = gemv_check_and_launch(rt, stream, a, "greedy_lm_head", &grid);
  if (st != AMMON_OK || stream == AMMON_STREAM_VALIDATE) return st;
  ammon_k_argmax p = {};
  p.logits = logits;
  p.cand_v = a.cand_v;
  p.cand_i = a.cand_i;
  p.step = (ammon_k_step *)step;
  p.prompt = prompt;
  p.tokens = tokens;
  p.n = vocab;
  p.blocks = grid;
  p.n_prompt = n_prompt;
  p.max_tokens = max_tokens;
  return launch(rt, stream, rt->k.argmax_final, 1, 1, 0, p, "greedy_lm_head");
}

ammon_status ammon_greedy_next(ammon_runtime *rt, ammon_stream stream, const float *logits,
                               uint32_t n, void *scratch, const int32_t *prompt,
                               uint32_t n_prompt, ammon_decode_step *step, int32_t *tokens,
                               uint32_t max_tokens) {
  AMMON_CHECK(step != nullptr, "greedy_next: parameter `step` is NULL");
  AMMON_CHECK(n_prompt == 0 || prompt != nullptr, "greedy_next: NULL prompt");
  return argmax_impl(rt, stream, logits, n, scratch, nullptr, prompt, n_prompt, step, tokens,
                     max_tokens, "greedy_next");
}

// ---- fills -------------------------------------------------------------------------------------
ammon_status ammon_fill(ammon_runtime *rt, ammon_stream stream, void *dst, ammon_dtype dtype,
                        size_t count, float value) {
  REQUIRE_RT();
  AMMON_CHECK(valid_dtype(dtype), "fill: unknown dtype %d", (int)dtype);
  AMMON_CHECK(count == 0 || dst, "fill: NULL destination");
  VALIDATE_ONLY();
  ammon_k_fill p = {};
  p.dst = dst;
  p.count = count;
  p.dtype = (uint32_t)dtype;
  if (dtype == AMMON_BF16) {
    uint32_t u;
    std::memcpy(&u, &value, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u)
      p.bits = (u >> 16) | 0x40u;
    else
      p.bits = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  } else {
    std::memcpy(&p.bits, &value, 4);
  }
  const uint32_t grid = (uint32_t)std::min<uint64_t>(cdiv(count, kWorkgroup),
                                                     (uint64_t)rt->info.compute_units * 32);
  return launch(rt, stream, rt->k.fill_const, grid, 1, 0, p, "fill");
}

ammon_status ammon_fill_normal(ammon_runtime *rt, ammon_stream stream, void *dst,
                               ammon_dtype dtype, size_t count, uint64_t seed,
                               uint64_t stream_id, float mean, float std) {
  REQUIRE_RT();
  AMMON_CHECK(valid_dtype(dtype), "fill_normal: unknown dtype %d", (int)dtype);
  AMMON_CHECK(count == 0 || dst, "fill_normal: NULL destination");
  VALIDATE_ONLY();
  ammon_k_fill p = {};
  p.dst = dst;
  p.count = count;
  p.seed = seed;
  p.stream = stream_id;
  p.mean = mean;
  p.std = std;
  p.dtype = (uint32_t)dtype;
  const uint32_t grid = (uint32_t)std::min<uint64_t>(cdiv((count + 1) / 2, kWorkgroup),
                                                     (uint64_t)rt->info.compute_units * 32);
  return launch(rt, stream, rt->k.fill_normal, grid, 1, 0, p, "fill_normal");
}

ammon_status ammon_checksum(ammon_runtime *rt, ammon_stream stream, const void *src, size_t bytes,
                            uint64_t *out) {
  REQUIRE_RT();
  AMMON_CHECK(out != nullptr && (bytes == 0 || src != nullptr), "checksum: NULL src or out");
  AMMON_CHECK(bytes % 8 == 0, "checksum: %zu bytes is not a whole number of 64-bit words", bytes);
  AMMON_CHECK(((uintptr_t)src & 15) == 0 && ((uintptr_t)out & 7) == 0,
              "checksum: src must be 16-byte and out 8-byte aligned");
  VALIDATE_ONLY();
  // zero the two result words with a kernel (capturable), then fold
  ammon_status st = ammon_fill(rt, stream, out, AMMON_F32, 4, 0.f);
  if (st != AMMON_OK || bytes == 0) return st;
  ammon_k_checksum p = {src, (uint64_t)bytes, (unsigned long long *)out};
  // one workgroup per CU: the whole device then sweeps the buffer in one
  // contiguous window, which streamed fastest in a sweep of 1-16 workgroups
  // per CU (4 GiB: 7.15 TB/s at one per CU, 5.8 at four)
  const uint32_t grid = (uint32_t)std::min<uint64_t>(
      std::max<uint64_t>(cdiv(bytes / 16, (uint64_t)kWorkgroup * 8), 1),
      (uint64_t)std::max(rt->info.compute_units, 1));
  return launch(rt, stream, rt->k.checksum, grid, 1, 0, p, "checksum");
}

ammon_status ammon_stream_read(ammon_runtime *rt, ammon_stream stream, const void *src,
                               size_t bytes) {
  REQUIRE_RT();
  AMMON_CHECK(bytes == 0 || src != nullptr, "stream_read: NULL src");
  AMMON_CHECK(((uintptr_t)src & 15) == 0, "stream_read: src must be 16-byte aligned");
  VALIDATE_ONLY();
  if (bytes == 0) return AMMON_OK;
  // two workgroups per CU, each a contiguous share in 16 KiB windows: the
  // fastest read of 32 MiB - 3.5 GiB in a chained sweep of layouts (one share
  // or a device-wide sweep per window; 1, 2 or 4 workgroups per CU; 4 or 8
  // loads in flight per lane)
  const uint64_t win = (uint64_t)kWorkgroup * 4 * 16;
  const uint32_t cus = (uint32_t)std::max(rt->info.compute_units, 1);
  const uint32_t grid = (uint32_t)std::min<uint64_t>(2ull * cus, cdiv((uint64_t)bytes, win));
  const uint64_t share = cdiv(cdiv((uint64_t)bytes, (uint64_t)grid), win) * win;
  AMMON_CHECK(share <= (1ull << 31), "stream_read: %zu bytes exceed %llu per workgroup", bytes,
              (unsigned long long)(1ull << 31));
  ammon_k_stream_read p = {src, (uint64_t)bytes, share};
  return launch(rt, stream, rt->k.stream_read, grid, 1, 0, p, "stream_read");
}

}  // extern "C"
