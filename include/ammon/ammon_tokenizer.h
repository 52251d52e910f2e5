/*
 * ammon_tokenizer.h -- C ABI of the llama2.c-compatible BPE tokenizer and
 * text generation (reference src/tokenizer.rs:11-177, src/generate.rs:93-118).
 *
 * Host-only (no device work).  Text is UTF-8 bytes with an explicit length;
 * outputs that may not fit are truncated to the caller's capacity while the
 * full length is reported, so a caller can retry with a larger buffer.
 */
#ifndef AMMON_AMMON_TOKENIZER_H
#define AMMON_AMMON_TOKENIZER_H

#include "ammon/ammon.h"
#include "ammon/ammon_model.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ammon_bpe ammon_bpe;

/* BpeTokenizer::from_path (reference src/tokenizer.rs:28-57): a llama2.c
 * tokenizer.bin with `vocab_size` pieces. */
ammon_status ammon_bpe_load(const char *path, uint32_t vocab_size, ammon_bpe **out);
/* BpeTokenizer::from_parts (src/tokenizer.rs:59-73): piece i is
 * pieces[i][0..lengths[i]) (UTF-8), with merge score scores[i]. */
ammon_status ammon_bpe_from_parts(const char *const *pieces, const uint32_t *lengths,
                                  const float *scores, uint32_t n, uint32_t max_token_length,
                                  ammon_bpe **out);
ammon_status ammon_bpe_destroy(ammon_bpe *t);
uint32_t ammon_bpe_vocab_size(const ammon_bpe *t);
uint32_t ammon_bpe_max_token_length(const ammon_bpe *t);

/* Tokenizer::encode (src/tokenizer.rs:104-159): BOS (id 1) if bos, the
 * dummy-prefix piece " " for non-empty text, code points looked up or split
 * into byte tokens (byte + 3), then the highest-score adjacent merge
 * repeated; EOS (id 2) if eos.  Writes min(*n_ids, capacity) ids; *n_ids is
 * the full count. */
ammon_status ammon_bpe_encode(const ammon_bpe *t, const char *text, size_t text_len, int bos,
                              int eos, int32_t *ids, size_t capacity, size_t *n_ids);
/* Tokenizer::decode (src/tokenizer.rs:161-170): the piece of `token`
 * (without its leading space after BOS; "<0xNN>" pieces give the character
 * U+00NN).  Writes at most capacity - 1 bytes and a terminating NUL; *len is
 * the full length. */
ammon_status ammon_bpe_decode(const ammon_bpe *t, int32_t prev_token, int32_t token, char *out,
                              size_t capacity, size_t *len);

/* generate (reference src/generate.rs:93-118) on the test model: encode the
 * prompt, run the greedy loop, decode the tokens after the first prompt
 * token.  loop: 0 = the reference loop (host argmax per step), 1 = the
 * device greedy loop, 2 = device loop after a one-pass prompt prefill.
 * text: at most text_capacity - 1 bytes + NUL (*text_len = full length);
 * tokens (nullable): at most token_capacity ids (*n_tokens = full count). */
ammon_status ammon_llama_generate_text(ammon_llama *m, const ammon_bpe *t, const char *prompt,
                                       size_t prompt_len, uint32_t max_new_tokens, int bos,
                                       int eos, int has_stop, int32_t stop_on, int loop,
                                       char *text, size_t text_capacity, size_t *text_len,
                                       int32_t *tokens, uint32_t token_capacity,
                                       uint32_t *n_tokens, double *tokens_per_second);

#ifdef __cplusplus
}
#endif
#endif
