/*
 * ammon_checkpoint.h -- llama2.c checkpoint loading into device memory.
 *
 * No counterpart in the reference (checkpoint loading belongs to the
 * architecture crates built on it).  Two public llama2.c layouts, fp32
 * weights stored [out, in] row-major:
 *   legacy (run.c): 7 int32 -- dim, hidden_dim, n_layers, n_heads,
 *     n_kv_heads, vocab_size (negative: separate classifier), seq_len --
 *     then token_embedding, rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3,
 *     rms_final, two RoPE tables [seq_len, head/2] (skipped), classifier;
 *   version 1 (export.py): uint32 magic 0x616b3432 ("ak42"), int32 version
 *     1, the 7 int32, uint8 shared_classifier, zero padding to 256 bytes,
 *     then rms_att, rms_ffn, rms_final, token_embedding, wq, wk, wv, wo, w1,
 *     w2, w3, classifier (when not shared).
 * The file is streamed through a pinned staging buffer; weights land in
 * w_dtype (bf16: round to nearest even), norm weights in fp32.
 */
#ifndef AMMON_AMMON_CHECKPOINT_H
#define AMMON_AMMON_CHECKPOINT_H

#include "ammon/ammon.h"
#include "ammon/ammon_model.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ammon_checkpoint ammon_checkpoint;

#define AMMON_CHECKPOINT_LEGACY 0u
#define AMMON_CHECKPOINT_V1 1u

/* Read and validate the header only (host, no device): the model shape in
 * cfg (theta 10000 and eps 1e-5, llama2.c's; w_dtype / kv_dtype fp32;
 * use_graph 1; split_len 0), the layout, whether the
 * classifier is the embedding table, and the file size the shape implies. */
ammon_status ammon_checkpoint_probe(const char *path, ammon_llama_config *cfg, uint32_t *format,
                                    uint32_t *shared_classifier, uint64_t *expected_bytes);
/* Load the whole checkpoint onto rt's device, weights in w_dtype. */
ammon_status ammon_checkpoint_load(ammon_runtime *rt, const char *path, ammon_dtype w_dtype,
                                   ammon_checkpoint **out);
/* The probe's config with w_dtype set to the loaded one, and the device
 * weight pointers (owned by the checkpoint; valid until ammon_checkpoint_free),
 * ready for ammon_llama_create. */
ammon_status ammon_checkpoint_config(const ammon_checkpoint *c, ammon_llama_config *cfg);
ammon_status ammon_checkpoint_weights(const ammon_checkpoint *c, ammon_llama_weights *w);
ammon_status ammon_checkpoint_free(ammon_checkpoint *c);

#ifdef __cplusplus
}
#endif
#endif
