/*
 * kernel_params.h -- argument blocks of the gfx950 kernels.
 *
 * Every kernel takes exactly one of these structs by value; the host packs it
 * and passes its address through hipModuleLaunchKernel's kernelParams.  The
 * header is plain C so that the host library (g++) and the device code
 * (hipcc, amdgcn) see the same layout.
 */
#ifndef AMMON_KERNEL_PARAMS_H
#define AMMON_KERNEL_PARAMS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage type codes; match ammon_dtype in include/ammon/ammon.h. */
#define AMMON_K_F32 0
#define AMMON_K_BF16 1

/* Device-resident control parcel: same layout as ammon_decode_step. */
typedef struct {
  uint32_t token;
  uint32_t position;
} ammon_k_step;

typedef struct {
  const void *table;        /* [vocab, dim] f32 or bf16 */
  const ammon_k_step *step; /* token source when ids == NULL */
  const uint32_t *ids;      /* [rows] or NULL */
  float *x;                 /* [rows, dim] */
  uint32_t vocab, dim, rows, dtype;
} ammon_k_embed;

typedef struct {
  const float *x;    /* [rows, dim] */
  const void *w;     /* [dim] f32 or bf16 */
  float *out;        /* [rows, dim]; may equal x */
  uint32_t rows, dim, w_dtype;
  float eps;
} ammon_k_rmsnorm;

typedef struct {
  float *q;                 /* [q_heads * head], rotated in place */
  const float *k_proj;      /* [kv_dim] (rope_store) or NULL (rope) */
  void *k_cache;            /* layer view [kv_heads, seq, head] */
  const ammon_k_step *step;
  const float *table;       /* [seq, head/2, 2] cos/sin */
  uint32_t q_numel, kv_dim, head, seq, kv_dtype;
} ammon_k_rope;

typedef struct {
  const float *src;         /* [kv_dim] */
  void *cache;              /* layer view [kv_heads, seq, head] */
  const ammon_k_step *step;
  uint32_t kv_dim, head, seq, dtype;
} ammon_k_cache_store;

/* Attention.  A grid z dimension runs several query tokens at consecutive
 * positions (prefill): token z reads q + z q_heads head, attends at
 * position step->position + z, and owns partial + z q_heads splits
 * (head + 2) and out + z q_heads head.  The kernels fold z into q, partial,
 * out and pos_add (0 for a single token). */
typedef struct {
  const float *q;           /* [q_heads, head] */
  const void *k_cache;      /* [kv_heads, seq, head] */
  const void *v_cache;      /* [kv_heads, seq, head] */
  const ammon_k_step *step;
  float *partial;           /* [q_heads, splits, head + 2] */
  float *out;               /* [q_heads, head] (combine) */
  uint32_t q_heads, kv_heads, head, seq, split_len, splits;
  uint32_t pos_add;         /* added to step->position */
  uint32_t limit;           /* positions at or past it (<= seq) are out of range:
                               NaN output, no partial (seq for decode; the
                               positions the grid and scratch cover for prefill) */
  uint32_t single_out;      /* pass 1 with splits == 1 writes out (the merge's
                               result) instead of the partial; no pass 2 */
  /* Merge only, optional (NULL: none): the next GEMV's weights.  Merge
   * workgroup i reads one dword of every 128-byte line of row block i
   * (rows [i warm_rows, +warm_rows), bytes [0, warm_bytes) of each, rows
   * warm_row_bytes apart) and discards it, so the lines wait in the L2 of
   * the XCD that runs the GEMV's workgroup i; only at positions of at
   * least warm_min_pos. */
  const void *warm;
  uint32_t warm_row_bytes, warm_rows, warm_bytes, warm_blocks, warm_min_pos;
} ammon_k_attention;

typedef struct {
  float *hb;                /* [n] in/out (swiglu) or out (add) */
  const float *a;           /* add: first operand */
  const float *b;           /* swiglu: hb2; add: second operand */
  uint32_t n;
} ammon_k_elementwise;

/* GEMV family.  Rows are "virtual": mode PLAIN/RESIDUAL index w0 rows
 * directly; SWIGLU interleaves w0 (gate) and w1 (up) rows; QKV runs over
 * [w0 (q); w1 (k); w2 (v)]. */
enum {
  AMMON_GEMV_PLAIN = 0,
  AMMON_GEMV_RESIDUAL = 1,
  AMMON_GEMV_SWIGLU = 2,
  AMMON_GEMV_QKV = 3,
  AMMON_GEMV_PLAIN_ARGMAX = 4 /* PLAIN, plus one argmax candidate per workgroup */
};

typedef struct {
  const void *w0, *w1, *w2; /* row-major [rows, n] matrices */
  const float *x;           /* [n] */
  const void *norm_w;       /* [n] RMSNorm weight or NULL (no prologue) */
  const float *residual;    /* RESIDUAL: y = residual + W x (may equal y) */
  float *y;                 /* PLAIN/RESIDUAL: [d]; SWIGLU: [d]; QKV: q out */
  void *k_cache, *v_cache;  /* QKV: layer views [kv_heads, seq, head] */
  const ammon_k_step *step; /* QKV */
  const float *table;       /* QKV: rope cos/sin */
  uint32_t d;               /* output rows (QKV: q_dim) */
  uint32_t n;               /* reduction length */
  uint32_t rows;            /* virtual rows: d, 2d (swiglu), q_dim + 2 kv_dim */
  uint32_t row_blocks;      /* ceil(rows / rows per workgroup) */
  uint32_t norm_dtype;
  float eps;
  uint32_t kv_dim, head, seq, kv_dtype; /* QKV */
  float *cand_v;            /* PLAIN_ARGMAX: [gridDim.x] (value, index) of the */
  uint32_t *cand_i;         /* first maximum over the workgroup's rows */
} ammon_k_gemv;

/* Prefill GEMM family: the GEMV modes over `tokens` rows of x at once
 * (Y[t] = W X[t]), on matrix cores.  QKV rotates and stores token t at
 * position step->position + t.  Virtual rows as for the GEMV family; a
 * 16-row wave tile never straddles q/k/v (q_dim, kv_dim multiples of 16). */
typedef struct {
  const void *w0, *w1, *w2; /* row-major [*, n] matrices */
  const float *x;           /* [tokens, n] */
  const float *residual;    /* RESIDUAL: [tokens, d] (may equal y) */
  float *y;                 /* [tokens, d]; QKV: q [tokens, q_dim] */
  void *k_cache, *v_cache;  /* QKV: layer views [kv_heads, seq, head] */
  const ammon_k_step *step; /* QKV */
  const float *table;       /* QKV: rope cos/sin [seq, head/2, 2] */
  uint32_t d, n, rows, tokens;
  uint32_t kv_dim, head, seq, kv_dtype; /* QKV */
  /* PLAIN / RESIDUAL, register-blocked tiles: the reduction split into
   * ksplit ranges of kchunks 64-wide chunks; range s writes its partial
   * sums to ws[s][tokens][d], summed in order by ammon_gemm_reduce */
  float *ws;
  uint32_t ksplit, kchunks;
} ammon_k_gemm;

typedef struct {
  const float *logits;      /* [n] */
  float *cand_v;            /* [blocks] candidate values */
  uint32_t *cand_i;         /* [blocks] candidate indices */
  int32_t *out;             /* argmax result (final pass) */
  ammon_k_step *step;       /* greedy feedback (final pass) or NULL */
  const int32_t *prompt;    /* greedy feedback: forced tokens */
  int32_t *tokens;          /* greedy feedback: tokens[pos] = next */
  uint32_t n, blocks, n_prompt, max_tokens;
} ammon_k_argmax;

typedef struct {
  const void *src;          /* bytes, a multiple of 8, 16-byte aligned */
  uint64_t bytes;
  unsigned long long *out;  /* [2]: wrapping sum, xor of the 64-bit words; zeroed first */
} ammon_k_checksum;

typedef struct {
  const void *src;          /* 16-byte aligned */
  uint64_t bytes;
  uint64_t share;           /* bytes per workgroup: a multiple of 16 KiB, < 2^32 */
} ammon_k_stream_read;

typedef struct {
  void *dst;
  uint64_t count, seed, stream;
  float mean, std;
  uint32_t dtype;
  uint32_t bits; /* fill: raw 32-bit pattern (f32) or 16-bit (bf16) */
} ammon_k_fill;

#ifdef __cplusplus
}
#endif
#endif
