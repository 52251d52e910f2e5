/*
 * ammon.h -- C ABI of the MI355X (gfx950) decode-layer kernels.
 *
 * This is the boundary a host-language binding (a Rust FFI crate via bindgen,
 * or ctypes) links against.  It replaces the Goldy kernel tier of
 * koubaa/ammon: each `<Kernel>::prepare` + `record(...)` + dispatch of the
 * reference becomes one call here that validates its arguments and, if they
 * are valid, enqueues the kernel asynchronously on the given stream.
 *
 * Conventions
 *   - Device buffers are plain pointers owned by the caller (allocate them
 *     with ammon_alloc or any HIP allocator).  Sizes are element counts.
 *   - `stream` is a hipStream_t passed as void*; NULL means the runtime's own
 *     stream.  AMMON_STREAM_VALIDATE checks the arguments and returns
 *     without launching (record-time validation for a caller that records
 *     launches and replays them later).
 *   - Every call returns an ammon_status.  On failure nothing is launched and
 *     ammon_last_error() returns a message on the calling thread.
 *   - Storage dtypes: AMMON_F32, or AMMON_BF16 (bit patterns, round to nearest
 *     even when written).  Activations are always fp32.
 *   - KV caches are head-major per layer: [kv_heads, seq, head].  The
 *     reference is position-major [seq, kv_heads, head]
 *     (reference src/modules.rs:37-71); ammon_kv_unpermute converts.
 *   - Positions and token ids that live in device memory (ammon_decode_step)
 *     cannot be checked on the host; kernels that find position >= seq or
 *     token >= vocab write NaN to their activation output and touch no
 *     memory outside the caller's buffers.
 *
 * Reference paths below are relative to the koubaa/ammon tree.
 */
#ifndef AMMON_AMMON_H
#define AMMON_AMMON_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AMMON_ABI_VERSION 1

typedef enum ammon_status {
  AMMON_OK = 0,
  AMMON_E_VALIDATION = 1, /* argument / shape contract violated (GoldyError::Validation) */
  AMMON_E_HIP = 2,        /* HIP runtime error */
  AMMON_E_OOM = 3,        /* device allocation failed */
  AMMON_E_NO_DEVICE = 4   /* no usable gfx950 device */
} ammon_status;

typedef enum ammon_dtype { AMMON_F32 = 0, AMMON_BF16 = 1 } ammon_dtype;

typedef enum ammon_copy_kind {
  AMMON_COPY_H2D = 1,
  AMMON_COPY_D2H = 2,
  AMMON_COPY_D2D = 3
} ammon_copy_kind;

/* DecodeStep (reference src/kernels.rs:10-15): token and position, kept in
 * device memory so a recorded launch sequence never changes per token. */
typedef struct ammon_decode_step {
  uint32_t token;
  uint32_t position;
} ammon_decode_step;

typedef struct ammon_runtime ammon_runtime;
typedef void *ammon_stream;
typedef void *ammon_event;

#define AMMON_STREAM_VALIDATE ((ammon_stream)(uintptr_t)1)

/* Attention constants (reference src/kernels.rs:228-231): the reference's
 * split length and the widest supported head. */
#define AMMON_ATTENTION_SPLIT_REF 8u
#define AMMON_ATTENTION_MAX_HEAD 128u
#define AMMON_ATTENTION_MAX_SPLIT 1024u
#define AMMON_ATTENTION_MAX_SPLITS 4096u
/* Llama-2 / llama2.c default RoPE base (reference src/kernels.rs:7-8). */
#define AMMON_DEFAULT_ROPE_THETA 10000.0f

/* ---- runtime ------------------------------------------------------------ */

/* Device bootstrap and prepared-kernel cache: replaces create_runtime
 * (reference src/gpu.rs:6-13) and Blocks::shared / Blocks::prepare
 * (reference src/blocks.rs:72-104).  Runtimes are cached per device and
 * reference counted: a second create for the same device returns the same
 * runtime until every holder has released it. */
ammon_status ammon_runtime_create(int device, ammon_runtime **out);
ammon_status ammon_runtime_release(ammon_runtime *rt);
const char *ammon_last_error(void);
int ammon_abi_version(void);

typedef struct ammon_device_info {
  int device;
  int compute_units;
  int max_shared_per_block; /* bytes */
  int warp_size;
  size_t total_memory;
  char arch[64];
  char name[128];
} ammon_device_info;
ammon_status ammon_runtime_info(ammon_runtime *rt, ammon_device_info *out);

/* Memory, streams and events (Goldy Runtime / Buffer plumbing). */
ammon_status ammon_alloc(ammon_runtime *rt, size_t bytes, void **dptr);
ammon_status ammon_free(ammon_runtime *rt, void *dptr);
ammon_status ammon_alloc_host(ammon_runtime *rt, size_t bytes, void **hptr); /* pinned */
ammon_status ammon_free_host(ammon_runtime *rt, void *hptr);
ammon_status ammon_memcpy(ammon_runtime *rt, void *dst, const void *src, size_t bytes,
                          ammon_copy_kind kind, ammon_stream stream);
ammon_status ammon_stream_create(ammon_runtime *rt, ammon_stream *out);
ammon_status ammon_stream_destroy(ammon_runtime *rt, ammon_stream stream);
ammon_status ammon_stream_synchronize(ammon_runtime *rt, ammon_stream stream);
ammon_status ammon_event_create(ammon_runtime *rt, ammon_event *out);
ammon_status ammon_event_destroy(ammon_runtime *rt, ammon_event ev);
ammon_status ammon_event_record(ammon_runtime *rt, ammon_event ev, ammon_stream stream);
ammon_status ammon_event_synchronize(ammon_runtime *rt, ammon_event ev);
ammon_status ammon_event_elapsed_ms(ammon_runtime *rt, ammon_event start, ammon_event stop,
                                    float *ms);

/* Launch-list replay.  A caller that records a sequence of the kernel calls
 * below (the reference's Scheme record, src/blocks.rs:178-278) captures it
 * once -- begin, make the calls on `stream`, end -- and replays the
 * instantiated graph per token (the reference's Scheme::submit replay).
 * Kernels read the token/position from a device ammon_decode_step, so the
 * graph never changes between tokens. */
typedef void *ammon_graph;
ammon_status ammon_capture_begin(ammon_runtime *rt, ammon_stream stream);
ammon_status ammon_capture_end(ammon_runtime *rt, ammon_stream stream, ammon_graph *out);
ammon_status ammon_graph_launch(ammon_runtime *rt, ammon_graph graph, ammon_stream stream);
ammon_status ammon_graph_destroy(ammon_runtime *rt, ammon_graph graph);

/* Fill `count` elements with `value` (a kernel, not hipMemset, so it can be
 * captured in a graph). */
ammon_status ammon_fill(ammon_runtime *rt, ammon_stream stream, void *dst, ammon_dtype dtype,
                        size_t count, float value);
/* Seeded N(mean, std) fill for synthetic weights / KV contents: element i is
 * a Box-Muller draw from splitmix64 keyed by (seed, stream_id, i / 2). */
ammon_status ammon_fill_normal(ammon_runtime *rt, ammon_stream stream, void *dst,
                               ammon_dtype dtype, size_t count, uint64_t seed,
                               uint64_t stream_id, float mean, float std);

/* Storage checksum (no counterpart in the reference): out[0] = wrapping sum
 * and out[1] = xor of the little-endian 64-bit words of src[0, bytes) (bytes
 * a multiple of 8, src 16-byte aligned; out is 2 words of device memory).
 * Proves two copies of a tensor identical bit for bit (device-generated
 * weights against a host fixture) without moving them. */
ammon_status ammon_checksum(ammon_runtime *rt, ammon_stream stream, const void *src, size_t bytes,
                            uint64_t *out);
/* Streaming read (no counterpart in the reference): reads src[0, bytes) once
 * (src 16-byte aligned) and writes nothing.  A chain of these over distinct
 * buffers measures the floor of a launch that moves that many bytes -- the
 * benchmark's per-size read floor. */
ammon_status ammon_stream_read(ammon_runtime *rt, ammon_stream stream, const void *src,
                               size_t bytes);

/* ---- host utilities (no device needed) ----------------------------------- */

/* RoPE cos/sin table [seq, head/2, 2] with the reference's fp32 formula
 * (reference src/kernels.rs:195-199): freq = 1 / powf(theta, hd / head),
 * val = pos * freq.  Replaces the per-lane pow/cos/sin of rope_store. */
size_t ammon_rope_table_bytes(uint32_t head, uint32_t seq);
ammon_status ammon_rope_table_host(float theta, uint32_t head, uint32_t seq, float *table);
/* Head-major [kv_heads, seq, head] -> reference position-major
 * [seq, kv_heads, head] (host arrays, elem_bytes 2 or 4); and the inverse. */
ammon_status ammon_kv_unpermute(const void *head_major, void *pos_major, uint32_t kv_heads,
                                uint32_t seq, uint32_t head, uint32_t elem_bytes);
ammon_status ammon_kv_permute(const void *pos_major, void *head_major, uint32_t kv_heads,
                              uint32_t seq, uint32_t head, uint32_t elem_bytes);
/* Flash-decoding split count and scratch size ([q_heads, splits, head + 2]
 * fp32; reference src/blocks.rs:317-320 with a caller-chosen split length). */
uint32_t ammon_attention_splits(uint32_t seq, uint32_t split_len);
size_t ammon_attention_scratch_bytes(uint32_t q_heads, uint32_t head, uint32_t seq,
                                     uint32_t split_len);
/* Split length the library picks for a kv-head count and cache length so that
 * kv_heads * splits fills the device at full context; a cache of at most 256
 * positions gets one split (the decode attention is then one launch). */
uint32_t ammon_attention_default_split(ammon_runtime *rt, uint32_t kv_heads, uint32_t seq);
/* The same choice for a full attention shape, which the model uses: the
 * unit count is sized to the pass-1 workgroups of that shape's kernel that
 * fit on a CU (two, or one for a kernel that fits only once), so a kernel
 * that runs one workgroup per CU gets one round of longer splits; and the
 * matrix-core kernels (bf16 cache, head 128, power-of-two group), which
 * score 64-position chunks, get splits of at least 64. */
uint32_t ammon_attention_default_split_for(ammon_runtime *rt, uint32_t q_heads,
                                           uint32_t kv_heads, uint32_t head,
                                           ammon_dtype kv_dtype, uint32_t seq);

/* ---- kernels ------------------------------------------------------------- */

/* embed (reference src/kernels.rs:35-47): x[dim] = table[step->token, :]. */
ammon_status ammon_embed(ammon_runtime *rt, ammon_stream stream, const void *table,
                         ammon_dtype table_dtype, uint32_t vocab, uint32_t dim,
                         const ammon_decode_step *step, float *x);
/* Batched gather: x[r, :] = table[ids[r], :] for `rows` device-resident ids
 * (an id >= vocab gives a NaN row). */
ammon_status ammon_embed_rows(ammon_runtime *rt, ammon_stream stream, const void *table,
                              ammon_dtype table_dtype, uint32_t vocab, uint32_t dim,
                              const uint32_t *ids, uint32_t rows, float *x);

/* rmsnorm / rmsnorm_inplace (reference src/kernels.rs:75-128), one
 * workgroup per row: out = w * (x / sqrt(mean(x^2) + eps)).  out == x is the
 * in-place form. */
ammon_status ammon_rmsnorm(ammon_runtime *rt, ammon_stream stream, const float *x,
                           const void *weight, ammon_dtype weight_dtype, float *out,
                           uint32_t rows, uint32_t dim, float eps);

/* rope_store (reference src/kernels.rs:174-210): rotate q [q_heads, head] in
 * place and write RoPE(k_proj) [kv_heads * head] into k_cache at
 * step->position.  `table` is ammon_rope_table_host's output in device
 * memory.  Requires kv_heads * head <= q_heads * head and even head. */
ammon_status ammon_rope_store(ammon_runtime *rt, ammon_stream stream, float *q,
                              uint32_t q_heads, const float *k_proj, uint32_t kv_heads,
                              uint32_t head, void *k_cache, ammon_dtype kv_dtype, uint32_t seq,
                              const ammon_decode_step *step, const float *table);
/* rope (reference src/kernels.rs:130-172): rotate q and the k_cache row at
 * step->position in place. */
ammon_status ammon_rope(ammon_runtime *rt, ammon_stream stream, float *q, uint32_t q_heads,
                        uint32_t kv_heads, uint32_t head, void *k_cache, ammon_dtype kv_dtype,
                        uint32_t seq, const ammon_decode_step *step, const float *table);
/* cache_store (reference src/kernels.rs:212-226): cache[:, pos, :] = src. */
ammon_status ammon_cache_store(ammon_runtime *rt, ammon_stream stream, const float *src,
                               uint32_t kv_heads, uint32_t head, void *cache,
                               ammon_dtype kv_dtype, uint32_t seq,
                               const ammon_decode_step *step);

/* attention_partial (reference src/kernels.rs:228-345): split-K pass over
 * the head-major cache, one workgroup per (split, kv head) serving all
 * q_heads / kv_heads query heads.  partial is [q_heads, splits, head + 2]
 * fp32 with splits = ammon_attention_splits(seq, split_len); splits past
 * step->position are not written. */
ammon_status ammon_attention_partial(ammon_runtime *rt, ammon_stream stream, const float *q,
                                     uint32_t q_heads, const void *k_cache, const void *v_cache,
                                     ammon_dtype kv_dtype, uint32_t kv_heads, uint32_t head,
                                     uint32_t seq, const ammon_decode_step *step,
                                     uint32_t split_len, float *partial);
/* attention_combine (reference src/kernels.rs:347-410): log-sum-exp merge of
 * the live splits into out [q_heads, head]. */
ammon_status ammon_attention_combine(ammon_runtime *rt, ammon_stream stream,
                                     const float *partial, uint32_t q_heads, uint32_t head,
                                     uint32_t seq, const ammon_decode_step *step,
                                     uint32_t split_len, float *out);
/* ammon_attention_combine, and while the merge runs (it reads ~1 MB and
 * leaves HBM mostly idle) it also reads the first warm_row_bytes of every
 * row of the next GEMV's weights next_w [next_rows, next_n] -- the output
 * projection that consumes out -- into the L2 of the XCD whose workgroup of
 * that GEMV (a RESIDUAL-mode ammon_gemv) reads them first; warm_row_bytes 0
 * means the GEMV's first tile of each row (4 KiB), next_w NULL no warming.
 * The warming happens only at step->position >= min_position (it paid at
 * 4096 positions and beyond and cost time at 2048 and below).  out is
 * bit-identical to ammon_attention_combine's.  Warming is skipped where
 * the two launches' workgroup-to-XCD maps do not line up or the bytes would
 * overflow the L2s.  No counterpart in the reference (its combine and
 * matmul are separate launches with no such hand-over). */
ammon_status ammon_attention_combine_warm(ammon_runtime *rt, ammon_stream stream,
                                          const float *partial, uint32_t q_heads, uint32_t head,
                                          uint32_t seq, const ammon_decode_step *step,
                                          uint32_t split_len, float *out, const void *next_w,
                                          ammon_dtype next_dtype, uint32_t next_rows,
                                          uint32_t next_n, uint32_t warm_row_bytes,
                                          uint32_t min_position);
/* Both passes (the reference's attn_partial + attn_combine pair,
 * src/blocks.rs:240-253).  When one split covers the cache
 * (ammon_attention_splits(seq, split_len) == 1) it is one launch: pass 1
 * writes out itself (the merge of a single split, bit for bit) and leaves
 * the partial scratch unwritten. */
ammon_status ammon_attention_decode(ammon_runtime *rt, ammon_stream stream, const float *q,
                                    uint32_t q_heads, const void *k_cache, const void *v_cache,
                                    ammon_dtype kv_dtype, uint32_t kv_heads, uint32_t head,
                                    uint32_t seq, const ammon_decode_step *step,
                                    uint32_t split_len, float *partial, size_t partial_bytes,
                                    float *out);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ammon_attention_decode with the split partials in a
 * library-owned device array of AMMON_NOALLOC_SCRATCH_BYTES per GPU instead
 * of a caller buffer.  Same kernels, same results; allocates nothing.  Fails
 * with AMMON_E_VALIDATION when ammon_attention_scratch_bytes(q_heads, head,
 * seq, split_len) exceeds the array.  All calls on one GPU share its array:
 * calls that can overlap on one GPU (unordered streams) race. */
#define AMMON_NOALLOC_SCRATCH_BYTES (4u << 20)
ammon_status ammon_attention_decode_noalloc(ammon_runtime *rt, ammon_stream stream,
                                            const float *q, uint32_t q_heads,
                                            const void *k_cache, const void *v_cache,
                                            ammon_dtype kv_dtype, uint32_t kv_heads,
                                            uint32_t head, uint32_t seq,
                                            const ammon_decode_step *step, uint32_t split_len,
                                            float *out);

/* swiglu (reference src/kernels.rs:462-476): hb = silu(hb) * hb2. */
ammon_status ammon_swiglu(ammon_runtime *rt, ammon_stream stream, float *hb, const float *hb2,
                          uint32_t n);
/* Residual add (reference TensorKernels::add_into, src/kernels.rs:506-516):
 * out = a + b; out may alias a or b. */
ammon_status ammon_add(ammon_runtime *rt, ammon_stream stream, const float *a, const float *b,
                       float *out, uint32_t n);

/* Dense projection (reference TensorKernels::matmul_into,
 * src/kernels.rs:518-528, defined by the serial gemv, src/kernels.rs:54-73):
 * y[d] = W[d, n] x[n], W row-major fp32 or bf16.  With residual != NULL,
 * y = residual + W x (residual may equal y: the wo / w2 + add_into pair of
 * src/blocks.rs:254-257,274-276).  With norm_weight != NULL, x is first
 * RMS-normalised (the rmsnorm + matmul pair; e.g. final norm + LM head). */
ammon_status ammon_gemv(ammon_runtime *rt, ammon_stream stream, const void *w,
                        ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x, float *y,
                        const float *residual);
/* The reference's position-strided gemv (src/kernels.rs:49-73; a test-only
 * serial definition there): xout[step->position, :] = W x with xout
 * [seq, d]. */
ammon_status ammon_gemv_at_position(ammon_runtime *rt, ammon_stream stream, const void *w,
                                    ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x,
                                    float *xout, uint32_t seq, const ammon_decode_step *step);
ammon_status ammon_gemv_rmsnorm(ammon_runtime *rt, ammon_stream stream, const float *x,
                                const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                const void *w, ammon_dtype w_dtype, uint32_t d, uint32_t n,
                                float *y);

/* Fused attention-block front (reference src/blocks.rs:219-239: rmsnorm, wq,
 * wk, wv, rope_store, cache_store) in one launch: q [q_heads * head] gets
 * RoPE(Wq xn); k_cache / v_cache get RoPE(Wk xn) / Wv xn at step->position.
 * norm_weight == NULL skips the normalisation. */
ammon_status ammon_qkv_rope_store(ammon_runtime *rt, ammon_stream stream, const float *x,
                                  const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                  const void *wq, const void *wk, const void *wv,
                                  ammon_dtype w_dtype, uint32_t dim, uint32_t q_heads,
                                  uint32_t kv_heads, uint32_t head, float *q, void *k_cache,
                                  void *v_cache, ammon_dtype kv_dtype, uint32_t seq,
                                  const ammon_decode_step *step, const float *table);

/* Fused SwiGLU-block front (reference src/blocks.rs:267-272: rmsnorm, w1,
 * w3, swiglu) in one launch: hb = silu(W1 xn) * (W3 xn). */
ammon_status ammon_gate_up_swiglu(ammon_runtime *rt, ammon_stream stream, const float *x,
                                  const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                  const void *w1, const void *w3, ammon_dtype w_dtype,
                                  uint32_t dim, uint32_t hidden, float *hb);

/* sample_argmax (reference src/tokenizer.rs:179-189) on device: first index
 * of the maximum, NaN never wins, NaN logits[0] gives 0.  `scratch` holds
 * ammon_argmax_scratch_bytes(n) bytes. */
size_t ammon_argmax_scratch_bytes(uint32_t n);
ammon_status ammon_argmax(ammon_runtime *rt, ammon_stream stream, const float *logits,
                          uint32_t n, void *scratch, int32_t *out);
/* Greedy step of generate_tokens (reference src/generate.rs:60-72) on device:
 * next = position + 1 < n_prompt ? prompt[position + 1] : argmax(logits);
 * tokens[position] = next (if position < max_tokens); step = {next,
 * position + 1}.  Lets a replayed token sequence run without host syncs. */
ammon_status ammon_greedy_next(ammon_runtime *rt, ammon_stream stream, const float *logits,
                               uint32_t n, void *scratch, const int32_t *prompt,
                               uint32_t n_prompt, ammon_decode_step *step, int32_t *tokens,
                               uint32_t max_tokens);

/* Final norm + LM head (ammon_gemv_rmsnorm into `logits`) fused with the
 * first pass of ammon_greedy_next, then its second pass: the same logits,
 * argmax and DecodeStep update as the two calls, with one launch fewer.
 * `scratch` holds ammon_greedy_lm_head_scratch_bytes(rt) bytes. */
size_t ammon_greedy_lm_head_scratch_bytes(ammon_runtime *rt);
ammon_status ammon_greedy_lm_head(ammon_runtime *rt, ammon_stream stream, const float *x,
                                  const void *norm_weight, ammon_dtype norm_dtype, float eps,
                                  const void *w, ammon_dtype w_dtype, uint32_t vocab,
                                  uint32_t dim, float *logits, void *scratch,
                                  size_t scratch_bytes, const int32_t *prompt, uint32_t n_prompt,
                                  ammon_decode_step *step, int32_t *tokens, uint32_t max_tokens);

/* ---- prompt prefill -------------------------------------------------------
 * No counterpart kernels in the reference, which feeds a prompt one decode
 * step per token (src/generate.rs:62-64).  These run `tokens` consecutive
 * positions step->position + t (t < tokens) at once with the decode path's
 * per-token arithmetic: the same formulas and fp32-grade products, the
 * projections as GEMMs on matrix cores (so only the fp32 summation order
 * differs from the GEMVs).  x, q, hb, y: row-major [tokens, width] fp32,
 * 16-byte aligned; the reduction length n (dim or hidden) a multiple of 8. */

/* The GEMV of ammon_gemv over rows of x: y[t] = W x[t] (+ residual[t]);
 * residual may equal y. */
ammon_status ammon_prefill_gemm(ammon_runtime *rt, ammon_stream stream, const void *w,
                                ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x,
                                uint32_t tokens, float *y, const float *residual);
/* ammon_prefill_gemm with a workspace of workspace_bytes (16-byte aligned,
 * not overlapping x, y or residual): with bf16 weights, projections whose
 * tiles alone would leave CUs idle (few rows, a long reduction, a short
 * prompt) split the reduction into ranges whose partial sums go to the
 * workspace and are added in range order by a second launch -- the result
 * is deterministic.  ammon_prefill_gemm_workspace_bytes(rows, tokens) gives
 * the size that allows every split (rows = d here; (q_heads + 2 kv_heads)
 * head for ammon_prefill_qkv_rope_store_ws). */
size_t ammon_prefill_gemm_workspace_bytes(uint32_t rows, uint32_t tokens);
ammon_status ammon_prefill_gemm_ws(ammon_runtime *rt, ammon_stream stream, const void *w,
                                   ammon_dtype w_dtype, uint32_t d, uint32_t n, const float *x,
                                   uint32_t tokens, float *y, const float *residual,
                                   void *workspace, size_t workspace_bytes);
/* ammon_qkv_rope_store over rows of an already normalised x: q [tokens,
 * q_heads * head]; rotated k and raw v rows go to the caches at positions
 * step->position + t.  head a multiple of 16. */
ammon_status ammon_prefill_qkv_rope_store(ammon_runtime *rt, ammon_stream stream, const float *x,
                                          uint32_t tokens, const void *wq, const void *wk,
                                          const void *wv, ammon_dtype w_dtype, uint32_t dim,
                                          uint32_t q_heads, uint32_t kv_heads, uint32_t head,
                                          float *q, void *k_cache, void *v_cache,
                                          ammon_dtype kv_dtype, uint32_t seq,
                                          const ammon_decode_step *step, const float *table);
/* ... with a workspace for a split reduction, as ammon_prefill_gemm_ws. */
ammon_status ammon_prefill_qkv_rope_store_ws(ammon_runtime *rt, ammon_stream stream, const float *x,
                                          uint32_t tokens, const void *wq, const void *wk,
                                          const void *wv, ammon_dtype w_dtype, uint32_t dim,
                                          uint32_t q_heads, uint32_t kv_heads, uint32_t head,
                                          float *q, void *k_cache, void *v_cache,
                                          ammon_dtype kv_dtype, uint32_t seq,
                                          const ammon_decode_step *step, const float *table,
                                             void *workspace, size_t workspace_bytes);
/* ammon_gate_up_swiglu over rows of an already normalised x: hb [tokens,
 * hidden]. */
ammon_status ammon_prefill_gate_up_swiglu(ammon_runtime *rt, ammon_stream stream, const float *x,
                                          uint32_t tokens, const void *w1, const void *w3,
                                          ammon_dtype w_dtype, uint32_t dim, uint32_t hidden,
                                          float *hb);
/* ammon_attention_decode for each of `tokens` query rows q [tokens, q_heads,
 * head] at positions step->position + t, which must be below ctx <= seq
 * (the scratch and the grid cover ctx positions); out [tokens, q_heads,
 * head].  `partial` holds ammon_attention_prefill_scratch_bytes bytes. */
size_t ammon_attention_prefill_scratch_bytes(uint32_t tokens, uint32_t q_heads, uint32_t head,
                                             uint32_t ctx, uint32_t split_len);
ammon_status ammon_attention_prefill(ammon_runtime *rt, ammon_stream stream, const float *q,
                                     uint32_t tokens, uint32_t q_heads, const void *k_cache,
                                     const void *v_cache, ammon_dtype kv_dtype, uint32_t kv_heads,
                                     uint32_t head, uint32_t seq, const ammon_decode_step *step,
                                     uint32_t ctx, uint32_t split_len, float *partial,
                                     size_t partial_bytes, float *out);

#ifdef __cplusplus
}
#endif
#endif
