/*
 * ammon_oracle.c -- CPU restatement of koubaa/ammon's decode-layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY: the parity reference for ammon_amd's HIP path and
 * the cpu_baseline of bench.py.  Nothing in the product links or calls it.
 *
 * Every function names the reference file:line it restates.  The reference's
 * arithmetic is fp32; this file is compiled with -ffp-contract=off so every
 * `a * b + c` below rounds twice, as written.  OpenMP parallelises only over
 * independent outputs (GEMV rows, attention (head, split) pairs), so each
 * output keeps its serial summation order and results do not depend on the
 * thread count.
 *
 * Pinned by tests/test_oracle.py against: the reference's known-answer
 * tests (tests/kernels.rs), its f64 attention reference
 * (tests/kernels.rs:400-427) on its own xorshift inputs, numpy/scipy f64
 * closed forms, torch's bf16 rounding, and an f64 brute-force model.
 */
#include "ammon_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- bf16 ------------------------------------------------------------------
 * Round-to-nearest-even truncation of the fp32 pattern; NaN stays NaN (quiet
 * bit set).  The reference is fp32-only; bf16 storage is an extension of
 * the HIP path, and both sides round with this rule. */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}

void orc_bf16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = orc_bf16_to_f32(src[i]);
}

static inline float load_elem(const void *base, int dtype, size_t i) {
  if (dtype == ORC_BF16) return orc_bf16_to_f32(((const uint16_t *)base)[i]);
  return ((const float *)base)[i];
}

static inline void store_elem(void *base, int dtype, size_t i, float v) {
  if (dtype == ORC_BF16)
    ((uint16_t *)base)[i] = orc_f32_to_bf16(v);
  else
    ((float *)base)[i] = v;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---- seeded inputs ---------------------------------------------------------- */
static inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

void orc_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream,
                     float mean, float std) {
  const uint64_t key = splitmix64(seed ^ splitmix64(stream + 0x632BE59BD9B4E019ull));
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (size_t c = 0; c < (n + 1) / 2; ++c) {
    uint64_t bits = splitmix64(key ^ (c * 0xD1B54A32D192ED03ull));
    double u1 = ((double)(bits >> 32) + 0.5) * (1.0 / 4294967296.0);
    double u2 = ((double)(bits & 0xffffffffull) + 0.5) * (1.0 / 4294967296.0);
    double r = sqrt(-2.0 * log(u1));
    double z0 = r * cos(two_pi * u2);
    double z1 = r * sin(two_pi * u2);
    dst[2 * c] = (float)((double)mean + (double)std * z0);
    if (2 * c + 1 < n) dst[2 * c + 1] = (float)((double)mean + (double)std * z1);
  }
}

/* reference tests/kernels.rs:380-390 */
void orc_pseudo_random(float *dst, size_t n, uint32_t seed) {
  uint32_t state = seed * 2654435761u + 1u;
  for (size_t i = 0; i < n; ++i) {
    state ^= state << 13;
    state ^= state >> 17;
    state ^= state << 5;
    dst[i] = (float)(state % 2001u) / 1000.0f - 1.0f;
  }
}

/* ---- kernels -------------------------------------------------------------- */

/* embed: reference src/kernels.rs:35-47, x[i] = table[token * dim + i].
 * `ids` holds one token per row (the reference reads step[0].token). */
void orc_embed(const void *table, int dtype, uint32_t vocab, uint32_t dim,
               const uint32_t *ids, uint32_t rows, float *x) {
  (void)vocab;
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t i = 0; i < dim; ++i)
      x[(size_t)r * dim + i] = load_elem(table, dtype, (size_t)ids[r] * dim + i);
}

/* rmsnorm: reference src/kernels.rs:75-101.  Lane l of 256 sums x_j^2 over
 * j = l, l+256, ...; the lane sums are then folded by a pairwise tree
 * (workgroup_sum, src/kernels.rs:92); then ss/dim + 1e-5, 1/sqrt, and
 * o = w * (s * x) in that multiplication order (src/kernels.rs:93-98). */
void orc_rmsnorm(const float *x, const void *w, int w_dtype, float *out,
                 uint32_t rows, uint32_t dim, float eps) {
  for (uint32_t r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * dim;
    float *orow = out + (size_t)r * dim;
    float lanes[256];
    for (uint32_t l = 0; l < 256; ++l) {
      float ss = 0.0f;
      for (uint32_t j = l; j < dim; j += 256) {
        float v = xr[j];
        ss = ss + v * v;
      }
      lanes[l] = ss;
    }
    for (uint32_t stride = 128; stride > 0; stride >>= 1)
      for (uint32_t l = 0; l < stride; ++l) lanes[l] = lanes[l] + lanes[l + stride];
    float ss = lanes[0];
    ss = ss / (float)dim;
    ss = ss + eps;
    ss = 1.0f / sqrtf(ss);
    for (uint32_t j = 0; j < dim; ++j) orow[j] = load_elem(w, w_dtype, j) * (ss * xr[j]);
  }
}

/* RoPE cos/sin per (pos, pair-within-head), computed with the reference's
 * fp32 formula (src/kernels.rs:195-199): for i = 2p, hd = i % head,
 * freq = 1 / powf(theta, hd / head), val = pos * freq, (cosf, sinf)(val).
 * Layout: table[(pos * (head/2) + p) * 2 + {0: cos, 1: sin}]. */
void orc_rope_table(float theta, uint32_t head, uint32_t seq, float *table) {
  const uint32_t half = head / 2;
  for (uint32_t pos = 0; pos < seq; ++pos)
    for (uint32_t p = 0; p < half; ++p) {
      uint32_t hd = (2 * p) % head;
      float freq = 1.0f / powf(theta, (float)hd / (float)head);
      float val = (float)pos * freq;
      table[((size_t)pos * half + p) * 2 + 0] = cosf(val);
      table[((size_t)pos * half + p) * 2 + 1] = sinf(val);
    }
}

/* rope_store: reference src/kernels.rs:174-210.  Pair i = 2p over the whole
 * query width rotates q in place; pairs with i < kv_dim also write the
 * rotated key projection into K[pos] (position-major row of kv_dim). */
/* rope_store with the rotated k row written at k_row[0 .. kv_dim). */
static void rope_store_row(float *q, const float *k_proj, void *k_row, int kv_dtype,
                           uint32_t q_numel, uint32_t kv_dim, uint32_t head, uint32_t pos,
                           const float *table) {
  const uint32_t half = head / 2;
  const size_t k_base = 0;
  for (uint32_t i = 0; i < q_numel; i += 2) {
    uint32_t hd = i % head;
    const float *cs = table + ((size_t)pos * half + hd / 2) * 2;
    float fcr = cs[0], fci = cs[1];
    float q0 = q[i], q1 = q[i + 1];
    q[i] = q0 * fcr - q1 * fci;
    q[i + 1] = q0 * fci + q1 * fcr;
    if (i < kv_dim) {
      float k0 = k_proj[i], k1 = k_proj[i + 1];
      store_elem(k_row, kv_dtype, k_base + i, k0 * fcr - k1 * fci);
      store_elem(k_row, kv_dtype, k_base + i + 1, k0 * fci + k1 * fcr);
    }
  }
}

void orc_rope_store(float *q, const float *k_proj, void *k_cache, int kv_dtype,
                    uint32_t q_numel, uint32_t kv_dim, uint32_t head,
                    uint32_t seq, uint32_t pos, const float *table) {
  (void)seq;
  rope_store_row(q, k_proj, (char *)k_cache + (size_t)pos * kv_dim * (kv_dtype == ORC_BF16 ? 2 : 4),
                 kv_dtype, q_numel, kv_dim, head, pos, table);
}

/* cache_store: reference src/kernels.rs:212-226, V[pos * row + i] = v[i]. */
void orc_cache_store(const float *v, void *v_cache, int kv_dtype,
                     uint32_t kv_dim, uint32_t seq, uint32_t pos) {
  (void)seq;
  for (uint32_t i = 0; i < kv_dim; ++i)
    store_elem(v_cache, kv_dtype, (size_t)pos * kv_dim + i, v[i]);
}

/* reference src/blocks.rs:317-320 with ATTENTION_SPLIT = 8 (src/kernels.rs:229) */
uint32_t orc_attention_splits(uint32_t seq, uint32_t split_len) {
  uint32_t s = (seq + split_len - 1) / split_len;
  return s ? s : 1;
}

/* attention_partial: reference src/kernels.rs:228-345, split length 8.
 * Per (h, s): 16 lanes per position, lane l summing dims l, l+16, ..., then
 * the 16 lane sums in order (:279-299); score = sum / sqrt(head) (a
 * division, :298); m = running max (:302-308); p = exp(score - m) (:310);
 * acc over `ways = 128 / head` groups folded in order (:314-336);
 * l = sum of p in order (:337-344).  Dead splits (8 s > pos) are skipped. */
void orc_attention_partial(const float *q, const void *k_cache,
                           const void *v_cache, int kv_dtype, uint32_t q_heads,
                           uint32_t kv_heads, uint32_t head, uint32_t seq,
                           uint32_t pos, float *partial) {
  const uint32_t SPLIT = 8;
  const uint32_t splits = orc_attention_splits(seq, SPLIT);
  const uint32_t kv_mul = q_heads / kv_heads;
  const uint32_t kv_dim = kv_heads * head;
  const uint32_t slot = head + 2;
  const float root = sqrtf((float)head);
#pragma omp parallel for schedule(static) collapse(2)
  for (uint32_t h = 0; h < q_heads; ++h)
    for (uint32_t s = 0; s < splits; ++s) {
      const uint32_t t0 = s * SPLIT;
      if (t0 > pos) continue;
      uint32_t n = pos + 1 - t0;
      if (n > SPLIT) n = SPLIT;
      const uint32_t head_base = (h / kv_mul) * head;
      const float *qs = q + (size_t)h * head;
      float scores[8] = {0}, probs[8] = {0};
      for (uint32_t p = 0; p < n; ++p) {
        const size_t k_base = (size_t)(t0 + p) * kv_dim + head_base;
        float sum = 0.0f;
        for (uint32_t l = 0; l < 16; ++l) {
          float dot = 0.0f;
          for (uint32_t i = l; i < head; i += 16)
            dot = dot + qs[i] * load_elem(k_cache, kv_dtype, k_base + i);
          sum = sum + dot;
        }
        scores[p] = sum / root;
      }
      float m = scores[0];
      for (uint32_t j = 1; j < n; ++j)
        if (scores[j] > m) m = scores[j];
      for (uint32_t j = 0; j < n; ++j) probs[j] = expf(scores[j] - m);
      const uint32_t ways = 128 / head;
      float *out = partial + ((size_t)h * splits + s) * slot;
      for (uint32_t i = 0; i < head; ++i) {
        float total = 0.0f;
        for (uint32_t w = 0; w < ways; ++w) {
          float acc = 0.0f;
          for (uint32_t j = w; j < n; j += ways)
            acc = acc + probs[j] * load_elem(v_cache, kv_dtype,
                                             (size_t)(t0 + j) * kv_dim + head_base + i);
          total = (w == 0) ? acc : total + acc;
        }
        out[i] = total;
      }
      float l = 0.0f;
      for (uint32_t j = 0; j < n; ++j) l = l + probs[j];
      out[head] = m;
      out[head + 1] = l;
    }
}

/* attention_combine: reference src/kernels.rs:347-410.  live = pos/8 + 1;
 * M = max of the live split maxima (:369-378); `ways = 256 / head` groups
 * each sum j = way, way+ways, ... of acc_j e^{m_j - M} and l_j e^{m_j - M}
 * (:380-394); the group sums are folded in order and divided (:401-408). */
void orc_attention_combine(const float *partial, uint32_t q_heads,
                           uint32_t head, uint32_t seq, uint32_t pos,
                           float *out) {
  const uint32_t splits = orc_attention_splits(seq, 8);
  const uint32_t slot = head + 2;
  const uint32_t live = pos / 8 + 1;
  const uint32_t ways = 256 / head;
  for (uint32_t h = 0; h < q_heads; ++h) {
    const float *base = partial + (size_t)h * splits * slot;
    float m = base[head];
    for (uint32_t s = 0; s < live; ++s) {
      float v = base[(size_t)s * slot + head];
      if (v > m) m = v;
    }
    float sums[256] = {0};
    for (uint32_t w = 0; w < ways; ++w) {
      float l = 0.0f;
      for (uint32_t j = w; j < live; j += ways) {
        const float *o = base + (size_t)j * slot;
        float wt = expf(o[head] - m);
        l = l + o[head + 1] * wt;
      }
      sums[w] = l;
    }
    float norm = sums[0];
    for (uint32_t w = 1; w < ways; ++w) norm = norm + sums[w];
    for (uint32_t i = 0; i < head; ++i) {
      float total = 0.0f;
      for (uint32_t w = 0; w < ways; ++w) {
        float acc = 0.0f;
        for (uint32_t j = w; j < live; j += ways) {
          const float *o = base + (size_t)j * slot;
          float wt = expf(o[head] - m);
          acc = acc + o[i] * wt;
        }
        total = (w == 0) ? acc : total + acc;
      }
        out[(size_t)h * head + i] = total / norm;
    }
  }
}

/* Serial attention: reference src/kernels.rs:412-460.  The softmax is Goldy's
 * workgroup_softmax_in_place (not in the tree); restated as max, exp(s - max),
 * serial sum, divide. */
void orc_attention_serial(const float *q, const void *k_cache,
                          const void *v_cache, int kv_dtype, uint32_t q_heads,
                          uint32_t kv_heads, uint32_t head, uint32_t seq,
                          uint32_t pos, float *att, float *out) {
  const uint32_t kv_mul = q_heads / kv_heads;
  const uint32_t kv_dim = kv_heads * head;
  const float root = sqrtf((float)head);
  for (uint32_t h = 0; h < q_heads; ++h) {
    float *a = att + (size_t)h * seq;
    const uint32_t kv_head = h / kv_mul;
    for (uint32_t t = 0; t <= pos; ++t) {
      float score = 0.0f;
      const size_t k_base = (size_t)t * kv_dim + (size_t)kv_head * head;
      for (uint32_t i = 0; i < head; ++i)
        score = score + q[(size_t)h * head + i] * load_elem(k_cache, kv_dtype, k_base + i);
      a[t] = score / root;
    }
    float m = a[0];
    for (uint32_t t = 1; t <= pos; ++t)
      if (a[t] > m) m = a[t];
    float sum = 0.0f;
    for (uint32_t t = 0; t <= pos; ++t) {
      a[t] = expf(a[t] - m);
      sum = sum + a[t];
    }
    for (uint32_t t = 0; t <= pos; ++t) a[t] = a[t] / sum;
    for (uint32_t i = 0; i < head; ++i) {
      float acc = 0.0f;
      for (uint32_t t = 0; t <= pos; ++t)
        acc = acc + a[t] * load_elem(v_cache, kv_dtype,
                                     (size_t)t * kv_dim + (size_t)kv_head * head + i);
      out[(size_t)h * head + i] = acc;
    }
  }
}

/* swiglu: reference src/kernels.rs:462-476. */
void orc_swiglu(float *hb, const float *hb2, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) {
    float val = hb[i];
    val = val * (1.0f / (1.0f + expf(-val)));
    val = val * hb2[i];
    hb[i] = val;
  }
}

/* GEMV: the serial definition, reference src/kernels.rs:54-73
 * (y_i = sum_j W[i*n + j] x_j, j ascending).  Several rows are interleaved
 * per thread for instruction-level parallelism; each row's order is
 * unchanged. */

/* Summation order of every GEMV row: 0 = the reference's (j ascending),
 * 1 = j descending.  The descending order is not the reference's; it exists
 * so a test can run the oracle against itself with one valid change of fp32
 * summation order (how far two correct implementations drift apart). */
static int g_gemv_order = 0;
void orc_set_gemv_order(int descending) { g_gemv_order = descending ? 1 : 0; }

/* Rows [r0, r0 + nr) (nr <= 4) of the serial gemv, j in the configured order. */
static void gemv_rows_scalar(const void *w, int w_dtype, uint32_t r0, uint32_t nr, uint32_t n,
                             const float *x, float *y) {
  float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t k = 0; k < n; ++k) {
    const uint32_t j = g_gemv_order ? n - 1 - k : k;
    const float xj = x[j];
    for (uint32_t r = 0; r < nr; ++r) {
      const size_t i = (size_t)(r0 + r) * n + j;
      const float wv = w_dtype == ORC_BF16 ? orc_bf16_to_f32(((const uint16_t *)w)[i])
                                           : ((const float *)w)[i];
      s[r] = s[r] + wv * xj;
    }
  }
  for (uint32_t r = 0; r < nr; ++r) y[r0 + r] = s[r];
}

#if defined(__x86_64__) && defined(__GNUC__)
#include <immintrin.h>
#define ORC_HAVE_AVX2_GEMV 1
/* 32 rows [r0, r0 + 32) of the serial gemv with AVX2: each 8-float vector
 * holds 8 rows' running sums, and every 8 x 8 block of W is transposed in
 * registers so the sums advance one column at a time -- every row keeps the
 * serial order (s = s + w_rj * x_j, j in the configured order, one rounding
 * for the product and one for the sum), so the results equal the scalar
 * loop's bit for bit.  Rows past d read row r0's data and are not stored.
 * Columns past the last whole block of 8 run through the scalar tail, in
 * order. */
__attribute__((target("avx2"))) static void gemv_rows32_avx2(const void *w, int w_dtype,
                                                             uint32_t r0, uint32_t d, uint32_t n,
                                                             const float *x, float *y) {
  const uint32_t n8 = n & ~7u;
  const int desc = g_gemv_order;
  __m256 acc[4];
  size_t row[32];
  for (int r = 0; r < 32; ++r) row[r] = (size_t)(r0 + r < d ? r0 + r : r0) * n;
  for (int g = 0; g < 4; ++g) acc[g] = _mm256_setzero_ps();
  /* descending: the tail columns come first, highest column first */
  if (desc) {
    for (uint32_t j = n; j-- > n8;) {
      const float xj = x[j];
      for (int g = 0; g < 4; ++g) {
        float t[8];
        _mm256_storeu_ps(t, acc[g]);
        for (int r = 0; r < 8; ++r) {
          const size_t i = row[8 * g + r] + j;
          const float wv = w_dtype == ORC_BF16 ? orc_bf16_to_f32(((const uint16_t *)w)[i])
                                               : ((const float *)w)[i];
          t[r] = t[r] + wv * xj;
        }
        acc[g] = _mm256_loadu_ps(t);
      }
    }
  }
  for (uint32_t bi = 0; bi < n8 / 8; ++bi) {
    const uint32_t j0 = desc ? n8 - 8 * (bi + 1) : 8 * bi;
    __m256 xb[8];
    for (int k = 0; k < 8; ++k) xb[k] = _mm256_set1_ps(x[j0 + k]);
    for (int g = 0; g < 4; ++g) {
      __m256 v[8];
      for (int r = 0; r < 8; ++r) {
        const size_t i = row[8 * g + r] + j0;
        if (w_dtype == ORC_BF16) {
          const __m128i h = _mm_loadu_si128((const __m128i *)((const uint16_t *)w + i));
          v[r] = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
        } else {
          v[r] = _mm256_loadu_ps((const float *)w + i);
        }
      }
      /* 8 x 8 transpose: c[k] = (v[0][k], ..., v[7][k]) */
      const __m256 t0 = _mm256_unpacklo_ps(v[0], v[1]), t1 = _mm256_unpackhi_ps(v[0], v[1]);
      const __m256 t2 = _mm256_unpacklo_ps(v[2], v[3]), t3 = _mm256_unpackhi_ps(v[2], v[3]);
      const __m256 t4 = _mm256_unpacklo_ps(v[4], v[5]), t5 = _mm256_unpackhi_ps(v[4], v[5]);
      const __m256 t6 = _mm256_unpacklo_ps(v[6], v[7]), t7 = _mm256_unpackhi_ps(v[6], v[7]);
      const __m256 u0 = _mm256_shuffle_ps(t0, t2, 0x44), u1 = _mm256_shuffle_ps(t0, t2, 0xEE);
      const __m256 u2 = _mm256_shuffle_ps(t1, t3, 0x44), u3 = _mm256_shuffle_ps(t1, t3, 0xEE);
      const __m256 u4 = _mm256_shuffle_ps(t4, t6, 0x44), u5 = _mm256_shuffle_ps(t4, t6, 0xEE);
      const __m256 u6 = _mm256_shuffle_ps(t5, t7, 0x44), u7 = _mm256_shuffle_ps(t5, t7, 0xEE);
      __m256 c[8];
      c[0] = _mm256_permute2f128_ps(u0, u4, 0x20);
      c[1] = _mm256_permute2f128_ps(u1, u5, 0x20);
      c[2] = _mm256_permute2f128_ps(u2, u6, 0x20);
      c[3] = _mm256_permute2f128_ps(u3, u7, 0x20);
      c[4] = _mm256_permute2f128_ps(u0, u4, 0x31);
      c[5] = _mm256_permute2f128_ps(u1, u5, 0x31);
      c[6] = _mm256_permute2f128_ps(u2, u6, 0x31);
      c[7] = _mm256_permute2f128_ps(u3, u7, 0x31);
      __m256 a = acc[g];
      if (desc) {
        for (int k = 7; k >= 0; --k) a = _mm256_add_ps(a, _mm256_mul_ps(c[k], xb[k]));
      } else {
        for (int k = 0; k < 8; ++k) a = _mm256_add_ps(a, _mm256_mul_ps(c[k], xb[k]));
      }
      acc[g] = a;
    }
  }
  float out[32];
  for (int g = 0; g < 4; ++g) _mm256_storeu_ps(out + 8 * g, acc[g]);
  if (!desc) {
    for (uint32_t j = n8; j < n; ++j) {
      const float xj = x[j];
      for (int r = 0; r < 32; ++r) {
        const size_t i = row[r] + j;
        const float wv = w_dtype == ORC_BF16 ? orc_bf16_to_f32(((const uint16_t *)w)[i])
                                             : ((const float *)w)[i];
        out[r] = out[r] + wv * xj;
      }
    }
  }
  for (uint32_t r = 0; r < 32 && r0 + r < d; ++r) y[r0 + r] = out[r];
}
#endif

/* gemv: reference serial definition src/kernels.rs:54-73,
 * y_i = sum_j W[i*n + j] x_j accumulated in j order, one fp32 rounding per
 * product and per sum.  OpenMP over blocks of output rows only. */
void orc_gemv(const void *w, int w_dtype, uint32_t d, uint32_t n,
              const float *x, float *y) {
#ifdef ORC_HAVE_AVX2_GEMV
  if (__builtin_cpu_supports("avx2")) {
    const int64_t blocks = ((int64_t)d + 31) / 32;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < blocks; ++b)
      gemv_rows32_avx2(w, w_dtype, (uint32_t)b * 32, d, n, x, y);
    return;
  }
#endif
  orc_gemv_scalar(w, w_dtype, d, n, x, y);
}

/* The same, one scalar chain per row (the portable path, and the check of
 * the vector path). */
void orc_gemv_scalar(const void *w, int w_dtype, uint32_t d, uint32_t n,
                     const float *x, float *y) {
  const int64_t blocks = ((int64_t)d + 3) / 4;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < blocks; ++b) {
    const uint32_t r0 = (uint32_t)b * 4;
    gemv_rows_scalar(w, w_dtype, r0, (d - r0) < 4 ? (d - r0) : 4, n, x, y);
  }
}

/* residual add: reference src/kernels.rs:506-516 (Goldy add_into), out = a + b. */
void orc_add(const float *a, const float *b, float *out, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* sample_argmax: reference src/tokenizer.rs:179-189 -- first index of the
 * maximum under a strict `>`; NaN never wins, and a NaN logits[0] gives 0. */
int32_t orc_sample_argmax(const float *logits, uint32_t n) {
  uint32_t best = 0;
  float best_p = logits[0];
  for (uint32_t i = 1; i < n; ++i)
    if (logits[i] > best_p) {
      best = i;
      best_p = logits[i];
    }
  return (int32_t)best;
}

/* ---- test model ------------------------------------------------------------
 * The graph Ammon's modules imply (its own graph lives in architecture crates,
 * reference README.md:5): x = embed(tok); per layer the attention block
 * (src/blocks.rs:219-257) and the SwiGLU block (src/blocks.rs:267-276);
 * logits = Wcls . rmsnorm(x, w_final). */
struct orc_model {
  orc_config c;
  orc_weights w;
  uint32_t head, q_dim, kv_dim, splits;
  float *x, *xb, *xb2, *q, *kp, *v, *hb, *hb2, *partial, *table;
  void *key, *value; /* [L, seq, kv_heads, head] */
  /* The K / V rows the latest step computed, per layer [L, kv_dim] in the
   * cache dtype, and whether a step stores them into the cache (1, the
   * reference's behaviour) or leaves the cache untouched (0: a test has
   * written the rows at the position itself). */
  void *krow, *vrow;
  int store_kv;
};

static size_t esize(int dtype) { return dtype == ORC_BF16 ? 2 : 4; }

orc_model *orc_model_create(const orc_config *cfg, const orc_weights *w) {
  orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
  m->c = *cfg;
  m->w = *w;
  m->head = cfg->dim / cfg->n_heads;
  m->q_dim = m->head * cfg->n_heads;
  m->kv_dim = m->head * cfg->n_kv_heads;
  m->splits = orc_attention_splits(cfg->max_seq, 8);
  m->x = (float *)calloc(cfg->dim, 4);
  m->xb = (float *)calloc(cfg->dim > m->q_dim ? cfg->dim : m->q_dim, 4);
  m->xb2 = (float *)calloc(cfg->dim, 4);
  m->q = (float *)calloc(m->q_dim, 4);
  m->kp = (float *)calloc(m->kv_dim, 4);
  m->v = (float *)calloc(m->kv_dim, 4);
  m->hb = (float *)calloc(cfg->hidden, 4);
  m->hb2 = (float *)calloc(cfg->hidden, 4);
  m->partial = (float *)calloc((size_t)cfg->n_heads * m->splits * (m->head + 2), 4);
  m->table = (float *)malloc((size_t)cfg->max_seq * (m->head / 2) * 2 * 4);
  orc_rope_table(cfg->theta, m->head, cfg->max_seq, m->table);
  size_t kv_elems = (size_t)cfg->n_layers * cfg->max_seq * m->kv_dim;
  m->key = calloc(kv_elems, esize(cfg->kv_dtype));
  m->value = calloc(kv_elems, esize(cfg->kv_dtype));
  m->krow = calloc((size_t)cfg->n_layers * m->kv_dim, esize(cfg->kv_dtype));
  m->vrow = calloc((size_t)cfg->n_layers * m->kv_dim, esize(cfg->kv_dtype));
  m->store_kv = 1;
  return m;
}

void orc_model_destroy(orc_model *m) {
  if (!m) return;
  free(m->x); free(m->xb); free(m->xb2); free(m->q); free(m->kp); free(m->v);
  free(m->hb); free(m->hb2); free(m->partial); free(m->table);
  free(m->key); free(m->value); free(m->krow); free(m->vrow);
  free(m);
}

static const void *layer_ptr(const void *base, int dtype, uint32_t l, size_t per_layer) {
  return (const char *)base + (size_t)l * per_layer * esize(dtype);
}

void orc_model_set_kv_store(orc_model *m, int on) { m->store_kv = on ? 1 : 0; }

void *orc_model_key_row(orc_model *m, uint32_t layer) {
  return (char *)m->krow + (size_t)layer * m->kv_dim * esize(m->c.kv_dtype);
}

void *orc_model_value_row(orc_model *m, uint32_t layer) {
  return (char *)m->vrow + (size_t)layer * m->kv_dim * esize(m->c.kv_dtype);
}

void *orc_model_key_cache(orc_model *m, uint32_t layer) {
  return (char *)m->key + (size_t)layer * m->c.max_seq * m->kv_dim * esize(m->c.kv_dtype);
}

void *orc_model_value_cache(orc_model *m, uint32_t layer) {
  return (char *)m->value + (size_t)layer * m->c.max_seq * m->kv_dim * esize(m->c.kv_dtype);
}

void orc_model_step(orc_model *m, uint32_t token, uint32_t pos, float *logits) {
  const orc_config *c = &m->c;
  const orc_weights *w = &m->w;
  const int wd = c->w_dtype;
  const uint32_t dim = c->dim;
  orc_embed(w->tok_emb, wd, c->vocab, dim, &token, 1, m->x);
  for (uint32_t l = 0; l < c->n_layers; ++l) {
    void *kc = orc_model_key_cache(m, l);
    void *vc = orc_model_value_cache(m, l);
    /* attention block: src/blocks.rs:219-257 */
    orc_rmsnorm(m->x, w->rms_att + (size_t)l * dim, ORC_F32, m->xb, 1, dim, c->eps);
    orc_gemv(layer_ptr(w->wq, wd, l, (size_t)m->q_dim * dim), wd, m->q_dim, dim, m->xb, m->q);
    orc_gemv(layer_ptr(w->wk, wd, l, (size_t)m->kv_dim * dim), wd, m->kv_dim, dim, m->xb, m->kp);
    orc_gemv(layer_ptr(w->wv, wd, l, (size_t)m->kv_dim * dim), wd, m->kv_dim, dim, m->xb, m->v);
    /* rope_store + cache_store (src/blocks.rs:226-239): the rows in the
     * cache dtype, then into the cache at pos */
    const size_t row_bytes = (size_t)m->kv_dim * esize(c->kv_dtype);
    char *krow = (char *)m->krow + (size_t)l * row_bytes;
    char *vrow = (char *)m->vrow + (size_t)l * row_bytes;
    rope_store_row(m->q, m->kp, krow, c->kv_dtype, m->q_dim, m->kv_dim, m->head, pos, m->table);
    for (uint32_t i = 0; i < m->kv_dim; ++i) store_elem(vrow, c->kv_dtype, i, m->v[i]);
    if (m->store_kv) {
      memcpy((char *)kc + (size_t)pos * row_bytes, krow, row_bytes);
      memcpy((char *)vc + (size_t)pos * row_bytes, vrow, row_bytes);
    }
    orc_attention_partial(m->q, kc, vc, c->kv_dtype, c->n_heads, c->n_kv_heads, m->head,
                          c->max_seq, pos, m->partial);
    orc_attention_combine(m->partial, c->n_heads, m->head, c->max_seq, pos, m->xb);
    orc_gemv(layer_ptr(w->wo, wd, l, (size_t)dim * m->q_dim), wd, dim, m->q_dim, m->xb, m->xb2);
    orc_add(m->x, m->xb2, m->x, dim);
    /* SwiGLU block: src/blocks.rs:267-276 */
    orc_rmsnorm(m->x, w->rms_ffn + (size_t)l * dim, ORC_F32, m->xb, 1, dim, c->eps);
    orc_gemv(layer_ptr(w->w1, wd, l, (size_t)c->hidden * dim), wd, c->hidden, dim, m->xb, m->hb);
    orc_gemv(layer_ptr(w->w3, wd, l, (size_t)c->hidden * dim), wd, c->hidden, dim, m->xb, m->hb2);
    orc_swiglu(m->hb, m->hb2, c->hidden);
    orc_gemv(layer_ptr(w->w2, wd, l, (size_t)dim * c->hidden), wd, dim, c->hidden, m->hb, m->xb);
    orc_add(m->x, m->xb, m->x, dim);
  }
  orc_rmsnorm(m->x, w->rms_final, ORC_F32, m->xb, 1, dim, c->eps);
  orc_gemv(w->wcls, wd, c->vocab, dim, m->xb, logits);
}

/* generate_tokens: reference src/generate.rs:43-91.  M = min(max_new, max_seq);
 * steps pos = 0 .. M-2; prompt tokens are forced while pos < P-1; the output
 * holds the chosen next tokens (prompt[1..] then argmax picks) and stops
 * before pushing `stop_on`. */
int orc_generate_tokens(orc_model *m, const int32_t *prompt, uint32_t n_prompt,
                        uint32_t max_new_tokens, int has_stop, int32_t stop_on,
                        int32_t *out_tokens, uint32_t *n_out,
                        float *last_logits) {
  if (n_prompt == 0) return 1;
  uint32_t limit = max_new_tokens < m->c.max_seq ? max_new_tokens : m->c.max_seq;
  float *logits = (float *)malloc(sizeof(float) * m->c.vocab);
  const uint32_t last = limit > 0 ? limit - 1 : 0; /* saturating_sub(1) */
  uint32_t token = (uint32_t)prompt[0];
  uint32_t pos = 0, count = 0;
  while (pos < last) {
    orc_model_step(m, token, pos, logits);
    int32_t next = (pos < n_prompt - 1) ? prompt[pos + 1]
                                        : orc_sample_argmax(logits, m->c.vocab);
    pos += 1;
    if (has_stop && next == stop_on) break;
    out_tokens[count++] = next;
    token = (uint32_t)next;
  }
  if (last_logits) memcpy(last_logits, logits, sizeof(float) * m->c.vocab);
  free(logits);
  *n_out = count;
  return 0;
}
