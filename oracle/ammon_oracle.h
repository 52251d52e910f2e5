/*
 * ammon_oracle.h -- CPU restatement of koubaa/ammon's decode-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity reference for the
 * HIP path in ammon_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only to check results or as
 * the reported CPU baseline -- never as a product code path.
 *
 * Layouts follow the reference, not the GPU build:
 *   - KV cache per layer is position-major [seq, kv_heads, head]
 *     (reference src/modules.rs:37-71);
 *   - weights are row-major [out, in] (reference src/modules.rs:166);
 *   - attention scratch is [q_heads, splits, head + 2]
 *     (reference src/modules.rs:223-227).
 * All arithmetic is fp32 with no FMA contraction (built with
 * -ffp-contract=off), following the order the reference kernels use.
 * bf16 values are stored as uint16_t and widened exactly.
 */
#ifndef AMMON_ORACLE_H
#define AMMON_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_BF16 = 1 };

/* ---- bf16 ---------------------------------------------------------------- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n);
void orc_bf16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* ---- seeded inputs ------------------------------------------------------- */
/* Counter-based normal generator: element i of (seed, stream) is a
 * Box-Muller draw from splitmix64(seed, stream, i / 2). */
void orc_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream,
                     float mean, float std);
/* The reference tests' xorshift32 generator (tests/kernels.rs:380-390). */
void orc_pseudo_random(float *dst, size_t n, uint32_t seed);

/* ---- kernels --------------------------------------------------------------- */
void orc_embed(const void *table, int dtype, uint32_t vocab, uint32_t dim,
               const uint32_t *ids, uint32_t rows, float *x);
void orc_rmsnorm(const float *x, const void *w, int w_dtype, float *out,
                 uint32_t rows, uint32_t dim, float eps);
void orc_rope_table(float theta, uint32_t head, uint32_t seq, float *table);
void orc_rope_store(float *q, const float *k_proj, void *k_cache, int kv_dtype,
                    uint32_t q_numel, uint32_t kv_dim, uint32_t head,
                    uint32_t seq, uint32_t pos, const float *table);
void orc_cache_store(const float *v, void *v_cache, int kv_dtype,
                     uint32_t kv_dim, uint32_t seq, uint32_t pos);
uint32_t orc_attention_splits(uint32_t seq, uint32_t split_len);
void orc_attention_partial(const float *q, const void *k_cache,
                           const void *v_cache, int kv_dtype, uint32_t q_heads,
                           uint32_t kv_heads, uint32_t head, uint32_t seq,
                           uint32_t pos, float *partial);
void orc_attention_combine(const float *partial, uint32_t q_heads,
                           uint32_t head, uint32_t seq, uint32_t pos,
                           float *out);
void orc_attention_serial(const float *q, const void *k_cache,
                          const void *v_cache, int kv_dtype, uint32_t q_heads,
                          uint32_t kv_heads, uint32_t head, uint32_t seq,
                          uint32_t pos, float *att, float *out);
void orc_swiglu(float *hb, const float *hb2, uint32_t n);
void orc_gemv(const void *w, int w_dtype, uint32_t d, uint32_t n,
              const float *x, float *y);
/* The same with one scalar chain per row (no vector instructions): the
 * check of the vector path, bit-identical to it. */
void orc_gemv_scalar(const void *w, int w_dtype, uint32_t d, uint32_t n,
                     const float *x, float *y);
/* Summation order of every GEMV row: 0 (default) = the reference's, j
 * ascending; 1 = j descending.  Only for measuring how far two valid
 * summation orders drift apart; process-wide, not thread-safe. */
void orc_set_gemv_order(int descending);
void orc_add(const float *a, const float *b, float *out, uint32_t n);
int32_t orc_sample_argmax(const float *logits, uint32_t n);

/* ---- llama2.c-convention test model -------------------------------------- */
typedef struct {
  uint32_t dim, n_layers, n_heads, n_kv_heads, hidden, vocab, max_seq;
  float theta, eps;
  int w_dtype;  /* matrices and embedding table */
  int kv_dtype; /* KV cache storage */
} orc_config;

typedef struct {
  const void *tok_emb;     /* [vocab, dim]                 */
  const float *rms_att;    /* [L, dim]                     */
  const float *rms_ffn;    /* [L, dim]                     */
  const void *wq;          /* [L, n_heads*head, dim]       */
  const void *wk;          /* [L, n_kv_heads*head, dim]    */
  const void *wv;          /* [L, n_kv_heads*head, dim]    */
  const void *wo;          /* [L, dim, n_heads*head]       */
  const void *w1;          /* [L, hidden, dim]             */
  const void *w2;          /* [L, dim, hidden]             */
  const void *w3;          /* [L, hidden, dim]             */
  const float *rms_final;  /* [dim]                        */
  const void *wcls;        /* [vocab, dim]                 */
} orc_weights;

typedef struct orc_model orc_model;

orc_model *orc_model_create(const orc_config *cfg, const orc_weights *w);
void orc_model_destroy(orc_model *m);
void orc_model_step(orc_model *m, uint32_t token, uint32_t pos, float *logits);
/* Pointer to the layer-l key / value cache ([seq, kv_heads, head]). */
/* Test hooks: the K / V rows (cache dtype, [kv_dim]) that the latest step
 * computed for `layer`, and whether steps store them into the cache (1,
 * the default, as the reference does) or leave it untouched (0). */
void *orc_model_key_row(orc_model *m, uint32_t layer);
void *orc_model_value_row(orc_model *m, uint32_t layer);
void orc_model_set_kv_store(orc_model *m, int on);
void *orc_model_key_cache(orc_model *m, uint32_t layer);
void *orc_model_value_cache(orc_model *m, uint32_t layer);
/* Greedy loop with the reference's semantics; returns 0 on success. */
int orc_generate_tokens(orc_model *m, const int32_t *prompt, uint32_t n_prompt,
                        uint32_t max_new_tokens, int has_stop, int32_t stop_on,
                        int32_t *out_tokens, uint32_t *n_out,
                        float *last_logits);

int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
