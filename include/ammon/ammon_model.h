/*
 * ammon_model.h -- C entry points of the C++ host layer's test model.
 *
 * The reference owns no model graph: architecture crates build it out of
 * Ammon's modules (reference README.md:5).  This header exposes the minimal
 * llama2.c-convention model the C++ layer builds from its own modules
 * (Embedding, CausalAttentionBlock, SwiGluBlock, Linear with the final norm)
 * together with the reference's greedy loop, so that a foreign caller
 * (ctypes, a Rust FFI crate) can drive whole decode steps:
 *   x = embed(token); per layer attention block then SwiGLU block;
 *   logits = Wcls . rmsnorm(x, w_final).
 * Weights are caller-owned device pointers, stacked per layer.
 */
#ifndef AMMON_AMMON_MODEL_H
#define AMMON_AMMON_MODEL_H

#include "ammon/ammon.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ammon_llama ammon_llama;

typedef struct ammon_llama_config {
  uint32_t dim, n_layers, n_heads, n_kv_heads, hidden, vocab, max_seq;
  float theta; /* RoPE base; the reference's default is 10000 */
  float eps;   /* RMSNorm epsilon; the reference's literal is 1e-5 */
  ammon_dtype w_dtype;  /* embedding table and projection matrices */
  ammon_dtype kv_dtype; /* KV cache storage */
  uint32_t use_graph;   /* replay each token as a captured HIP graph */
  uint32_t split_len;   /* attention split length; 0 picks one sized to the
                           device and the shape's kernel
                           (ammon_attention_default_split_for) */
} ammon_llama_config;

typedef struct ammon_llama_weights {
  const void *tok_emb;    /* [vocab, dim]                  w_dtype */
  const float *rms_att;   /* [L, dim]                      fp32    */
  const float *rms_ffn;   /* [L, dim]                      fp32    */
  const void *wq;         /* [L, n_heads*head, dim]        w_dtype */
  const void *wk;         /* [L, n_kv_heads*head, dim]     w_dtype */
  const void *wv;         /* [L, n_kv_heads*head, dim]     w_dtype */
  const void *wo;         /* [L, dim, n_heads*head]        w_dtype */
  const void *w1;         /* [L, hidden, dim]              w_dtype */
  const void *w2;         /* [L, dim, hidden]              w_dtype */
  const void *w3;         /* [L, hidden, dim]              w_dtype */
  const float *rms_final; /* [dim]                         fp32    */
  const void *wcls;       /* [vocab, dim]                  w_dtype */
} ammon_llama_weights;

ammon_status ammon_llama_create(ammon_runtime *rt, const ammon_llama_config *cfg,
                                const ammon_llama_weights *w, ammon_llama **out);
ammon_status ammon_llama_destroy(ammon_llama *m);

/* AutoregressiveModel::step (reference src/model.rs:10): logits for
 * (token, pos) copied to `logits` (host, [vocab]). */
ammon_status ammon_llama_step(ammon_llama *m, uint32_t token, uint32_t pos, float *logits);

/* generate_tokens (reference src/generate.rs:43-91) with the host argmax per
 * step.  out_tokens holds up to max(min(max_new_tokens, max_seq) - 1, 0)
 * tokens; last_logits (nullable, [vocab]) receives the final step's logits. */
ammon_status ammon_llama_generate_tokens(ammon_llama *m, const int32_t *prompt,
                                         uint32_t n_prompt, uint32_t max_new_tokens,
                                         int has_stop, int32_t stop_on, int32_t *out_tokens,
                                         uint32_t *n_out, double *tokens_per_second,
                                         float *last_logits);

/* The same loop with the argmax, prompt forcing and DecodeStep update on the
 * device: the token graph is replayed back to back with no host round trip,
 * and the host reads the tokens once at the end (stop_on truncates the
 * result).  tokens_per_second follows the reference's formula (steps after
 * the first over the time they took). */
ammon_status ammon_llama_generate_tokens_device(ammon_llama *m, const int32_t *prompt,
                                                uint32_t n_prompt, uint32_t max_new_tokens,
                                                int has_stop, int32_t stop_on,
                                                int32_t *out_tokens, uint32_t *n_out,
                                                double *tokens_per_second, float *last_logits);

/* Prompt prefill (no counterpart in the reference, which steps the prompt
 * one token at a time, src/generate.rs:62-64): tokens[0..n) run at
 * positions start_pos.. in one pass per layer (GEMMs on matrix cores,
 * token-batched attention), filling the KV cache; the DecodeStep is left at
 * {tokens[n - 1], start_pos + n - 1} as after stepping them one by one.
 * logits (nullable, host, [vocab]) receives the last position's logits. */
ammon_status ammon_llama_prefill(ammon_llama *m, const int32_t *tokens, uint32_t n,
                                 uint32_t start_pos, float *logits);

/* generate_tokens_device with the prompt prefilled in one pass: the same
 * outputs (up to fp32 summation order in the prompt's projections), with
 * the prompt's positions in one launch per kernel instead of one decode
 * step each.  tokens_per_second covers the decode steps after the first
 * generated token. */
ammon_status ammon_llama_generate_tokens_prefill(ammon_llama *m, const int32_t *prompt,
                                                 uint32_t n_prompt, uint32_t max_new_tokens,
                                                 int has_stop, int32_t stop_on,
                                                 int32_t *out_tokens, uint32_t *n_out,
                                                 double *tokens_per_second, float *last_logits);

/* Enqueue `n_steps` device-greedy decode steps starting from (token,
 * start_pos) on the model's stream, without synchronising (the caller times
 * them with events).  tokens (nullable, host, [n_steps]) is filled after an
 * internal synchronisation only when non-NULL. */
ammon_status ammon_llama_decode(ammon_llama *m, uint32_t token, uint32_t start_pos,
                                uint32_t n_steps, int32_t *tokens);

/* Tokens the device greedy step wrote for positions [start, start + n)
 * (host array; synchronises the model's stream). */
ammon_status ammon_llama_tokens(ammon_llama *m, uint32_t start, uint32_t n, int32_t *tokens);

/* Device pointers of layer `layer`'s key and value caches ([kv_heads, seq,
 * head] in kv_dtype), the model's stream, and its logits buffer. */
ammon_status ammon_llama_kv_layer(ammon_llama *m, uint32_t layer, void **key, void **value);
ammon_status ammon_llama_stream(ammon_llama *m, ammon_stream *stream);
ammon_status ammon_llama_logits(ammon_llama *m, float **device_logits);
/* Number of kernel launches per token (greedy step excluded). */
ammon_status ammon_llama_launches(ammon_llama *m, uint32_t *n);

#ifdef __cplusplus
}
#endif
#endif
