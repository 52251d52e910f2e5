// token.hip -- persistent decode-token kernel: one cooperative launch per
// token runs the whole decode step of the reference's recorded scheme
// (embed, per layer the attention block src/blocks.rs:172-259 and the FFN
// block src/blocks.rs:261-278, final norm + LM head, and the greedy step of
// src/generate.rs:60-72) with the same per-row, per-unit arithmetic as the
// standalone kernels (gemv_impl.h, attention_impl.h, argmax_impl.h).
//
// Why: one launch per fused kernel costs a ramp-up and a drain of the whole
// device each time (~4 us against 5-40 us kernels).  Here every workgroup
// stays resident for the token; dependent phases are separated by grid-wide
// barriers, and before a workgroup waits at a barrier it already requests
// the weight tiles of its next GEMV pass (weights never depend on the
// activations), so HBM keeps streaming while the barrier completes.
//
// Data between phases: every phase writes its own slice of the activation
// buffers (per layer, per residual step) with agent-scope stores that write
// through to the device coherence point (st_out), and every read of a value
// another workgroup produced in this launch -- x for a GEMV's LDS staging,
// the residual, q, the K/V rows (the newest is stored by the QKV phase), the
// split partials, the logits and the argmax candidates -- is an agent-scope
// load (ld_in, ld_in4, AMMON_HANDOFF_CPOL; device_common.h).  Agent-scope
// loads are coherent per location, so no L1 or L2 line -- whether cached by
// an earlier read or shared with a neighbouring slice written by another
// workgroup -- can supply a stale value, and the barrier needs no L2
// writeback or invalidate (each costs several microseconds across the
// device).  Order: a producer's waves wait for their stores to complete
// (s_waitcnt vmcnt(0): stores are counted there and complete at the
// coherence point) before the workgroup counts itself in; a consumer issues
// its loads only after its poll has seen the full count (the loads follow
// the poll loop's exit and the workgroup barrier).  Read-only inputs
// (weights, norm weights, the RoPE table) and the DecodeStep (written by the
// previous launch) use plain loads.
//
// Barrier: GridSync (grid_sync.h), hierarchical counters with bounded
// polls.  Workgroup 0 waits at the final barrier (the greedy step needs
// every candidate) and then zeroes the counters for the next launch.  With a
// trace buffer every workgroup stamps the device clock at each barrier
// (phase timing and load balance without a profiler).
//
// Requires all gridDim.x workgroups to be co-resident (cooperative launch).
// results cross workgroups within the launch: agent-scope stores and loads
#define AMMON_AGENT_HANDOFF 1
#include "argmax_impl.h"
#include "attention_impl.h"
#include "gemv_impl.h"
#include "grid_sync.h"

namespace {

template <typename KV>
AMMON_DEV size_t kv_layer_elems(const ammon_k_token &P) {
  return (size_t)P.kv_heads * P.seq * P.head;
}

}  // namespace

// WT: weight storage, KV: cache storage, GMAX: q heads per kv head.
template <typename WT, typename KV, int GMAX>
AMMON_DEV void decode_token(const ammon_k_token &P) {
  constexpr int CH = 16 / sizeof(WT);  // 16-byte weight chunks
  constexpr int RPW = 2, U = AMMON_TOKEN_GEMV_U;
  constexpr int ACH = 16 / sizeof(KV);  // attention: 16-byte K/V chunks, head 128
  extern __shared__ float4 lds4[];
  float *lds = (float *)lds4;
  __shared__ float red[AMMON_WAVES];

  const uint32_t wg = blockIdx.x, G = gridDim.x;
  GridSync bar{P.sync, G, 0, P.spin_limit, P.trace, P.trace_slots};
  const uint32_t head = P.head, q_dim = P.q_heads * head, kv_dim = P.kv_heads * head;
  const uint32_t rows_per_block = AMMON_WAVES * RPW;
  auto blocks = [&](uint32_t rows) { return (rows + rows_per_block - 1) / rows_per_block; };
  const uint32_t kvt = (uint32_t)sizeof(KV) == 2 ? AMMON_K_BF16 : AMMON_K_F32;

  // ---- embed: x = table[token] (NaN row for a token outside the vocab) ----
  {
    const uint32_t token = P.step->token;
    const bool ok = token < P.vocab;
    for (uint32_t i = wg * AMMON_WG + threadIdx.x; i < P.dim; i += G * AMMON_WG) {
      float v = __uint_as_float(0x7fc00000u);
      if (ok) {
        const size_t at = (size_t)token * P.dim + i;
        v = sizeof(WT) == 2 ? bf16_to_f32(((const uint16_t *)P.tok_emb)[at])
                            : ((const float *)P.tok_emb)[at];
      }
      st_out(P.x + i, v);
    }
  }
  bar.arrive();

  for (uint32_t l = 0; l < P.n_layers; ++l) {
    const size_t kv_off = (size_t)l * kv_layer_elems<KV>(P);
    KV *kc = (KV *)P.k_cache + kv_off;
    KV *vc = (KV *)P.v_cache + kv_off;
    float *x_in = P.x + (size_t)(2 * l) * P.x_stride;   // layer input
    float *x_mid = x_in + P.x_stride;                   // after the attention residual
    float *x_out = x_mid + P.x_stride;                  // after the FFN residual
    float *q = P.q + (size_t)l * P.q_stride;
    float *att = P.att + (size_t)l * P.q_stride;
    float *hb = P.hb + (size_t)l * P.hb_stride;
    float *partial = P.partial + (size_t)l * P.partial_stride;

    // ---- norm + QKV + RoPE + K/V store -----------------------------------
    {
      ammon_k_gemv g{};
      g.w0 = (const WT *)P.wq + (size_t)l * q_dim * P.dim;
      g.w1 = (const WT *)P.wk + (size_t)l * kv_dim * P.dim;
      g.w2 = (const WT *)P.wv + (size_t)l * kv_dim * P.dim;
      g.x = x_in;
      g.norm_w = P.rms_att + (size_t)l * P.dim;
      g.norm_dtype = AMMON_K_F32;
      g.eps = P.eps;
      g.y = q;
      g.k_cache = kc;
      g.v_cache = vc;
      g.step = P.step;
      g.table = P.table;
      g.d = q_dim;
      g.n = P.dim;
      g.rows = q_dim + 2 * kv_dim;
      g.row_blocks = blocks(g.rows);
      g.kv_dim = kv_dim;
      g.head = head;
      g.seq = P.seq;
      g.kv_dtype = kvt;
      GemvPass<WT, CH, RPW, U, AMMON_GEMV_QKV> pass;
      pass.begin(g, wg, G);
      bar.wait();  // x final (embed or the previous layer's down projection)
      pass.run(lds4, red);
    }
    bar.arrive();

    // ---- split-K attention ---------------------------------------------------
    ammon_k_attention a{};
    a.q = q;
    a.k_cache = kc;
    a.v_cache = vc;
    a.step = P.step;
    a.partial = partial;
    a.out = att;
    a.q_heads = P.q_heads;
    a.kv_heads = P.kv_heads;
    a.head = head;
    a.seq = P.seq;
    a.limit = P.seq;
    a.split_len = P.split_len;
    a.splits = P.splits;
    {
      const uint32_t units = P.kv_heads * P.splits;
      bar.wait();  // q and the new K/V rows written
      for (uint32_t u = wg; u < units; u += G) {
        if constexpr (sizeof(KV) == 2) {  // the standalone kernels' choice per KV type
          AttnPartialMfma<GMAX, 4> unit;
          if (unit.begin(a, u % P.splits, u / P.splits)) unit.run(a, lds);
        } else {
          AttnPartial<KV, ACH, GMAX, 128, true> unit;
          if (unit.begin(a, u % P.splits, u / P.splits)) unit.run(a, lds);
        }
      }
    }
    bar.arrive();

    // ---- merge, output projection + residual --------------------------------
    {
      ammon_k_gemv g{};
      g.w0 = (const WT *)P.wo + (size_t)l * P.dim * q_dim;
      g.x = att;
      g.residual = x_in;
      g.y = x_mid;
      g.d = P.dim;
      g.n = q_dim;
      g.rows = P.dim;
      g.row_blocks = blocks(g.rows);
      GemvPass<WT, CH, RPW, U, AMMON_GEMV_RESIDUAL> pass;
      pass.begin(g, wg, G);
      bar.wait();  // partials written
      const uint32_t slices = (head + 31) / 32;
      for (uint32_t u = wg; u < P.q_heads * slices; u += G)
        attention_combine_unit(a, u / slices, u % slices, lds);
      bar.arrive();
      bar.wait();  // attention output final
      pass.run(lds4, red);
    }
    bar.arrive();

    // ---- norm + gate/up + SwiGLU -------------------------------------------
    {
      ammon_k_gemv g{};
      g.w0 = (const WT *)P.w1 + (size_t)l * P.hidden * P.dim;
      g.w1 = (const WT *)P.w3 + (size_t)l * P.hidden * P.dim;
      g.x = x_mid;
      g.norm_w = P.rms_ffn + (size_t)l * P.dim;
      g.norm_dtype = AMMON_K_F32;
      g.eps = P.eps;
      g.y = hb;
      g.d = P.hidden;
      g.n = P.dim;
      g.rows = 2 * P.hidden;
      g.row_blocks = blocks(g.rows);
      GemvPass<WT, CH, RPW, U, AMMON_GEMV_SWIGLU> pass;
      pass.begin(g, wg, G);
      bar.wait();  // x after the attention residual
      pass.run(lds4, red);
    }
    bar.arrive();

    // ---- down projection + residual ----------------------------------------
    {
      ammon_k_gemv g{};
      g.w0 = (const WT *)P.w2 + (size_t)l * P.dim * P.hidden;
      g.x = hb;
      g.residual = x_mid;
      g.y = x_out;
      g.d = P.dim;
      g.n = P.hidden;
      g.rows = P.dim;
      g.row_blocks = blocks(g.rows);
      GemvPass<WT, CH, RPW, U, AMMON_GEMV_RESIDUAL> pass;
      pass.begin(g, wg, G);
      bar.wait();  // hb final
      pass.run(lds4, red);
    }
    bar.arrive();
  }

  // ---- final norm + LM head ------------------------------------------------
  {
    ammon_k_gemv g{};
    g.w0 = P.wcls;
    g.x = P.x + (size_t)(2 * P.n_layers) * P.x_stride;
    g.norm_w = P.rms_final;
    g.norm_dtype = AMMON_K_F32;
    g.eps = P.eps;
    g.y = P.logits;
    g.d = P.vocab;
    g.n = P.dim;
    g.rows = P.vocab;
    g.row_blocks = blocks(g.rows);
    GemvPass<WT, CH, RPW, U, AMMON_GEMV_PLAIN> pass;
    pass.begin(g, wg, G);
    bar.wait();  // x after the last layer
    pass.run(lds4, red);
  }
  bar.arrive();

  float *sv = lds;
  uint32_t *si = (uint32_t *)(lds + AMMON_WG);
  if (P.greedy) {
    // argmax pass 1: one candidate per workgroup over a contiguous slice
    bar.wait();  // logits final
    const uint32_t per = (P.vocab + G - 1) / G;
    const uint32_t lo = wg * per, hi = min(P.vocab, lo + per);
    float v = 0.f;
    uint32_t idx = ARGMAX_NONE;
    for (uint32_t i = lo + threadIdx.x; i < hi; i += AMMON_WG) {
      const float xl = ld_in(P.logits + i);
      if (xl == xl) cand_merge(v, idx, xl, i);
    }
    block_cand_reduce(v, idx, sv, si);
    if (threadIdx.x == 0) {
      st_out(P.cand_v + wg, v);
      st_out(P.cand_i + wg, idx);
    }
    bar.arrive();
  }
  if (wg != 0) return;  // the others are done with the counters
  bar.wait();
  if (P.greedy) {
    // argmax pass 2 and the greedy step (reference src/generate.rs:60-72):
    // next = pos + 1 < n_prompt ? prompt[pos + 1] : argmax; tokens[pos] = next
    float v = 0.f;
    uint32_t idx = ARGMAX_NONE;
    for (uint32_t b = threadIdx.x; b < G; b += AMMON_WG)
      cand_merge(v, idx, ld_in(P.cand_v + b), ld_in(P.cand_i + b));
    block_cand_reduce(v, idx, sv, si);
    if (threadIdx.x == 0) {
      const float first = ld_in(P.logits);
      const int32_t best = (first != first || idx == ARGMAX_NONE) ? 0 : (int32_t)idx;
      if (P.argmax_out) *P.argmax_out = best;
      const uint32_t pos = P.step->position;
      const int32_t next = (P.prompt && pos + 1 < P.n_prompt) ? P.prompt[pos + 1] : best;
      if (P.tokens && pos < P.max_tokens) P.tokens[pos] = next;
      P.step->token = (uint32_t)next;
      P.step->position = pos + 1;
    }
  }
  // every workgroup has arrived for the last time: zero the counters for the
  // next launch (the error word is left for the host)
  if (threadIdx.x < 9) __hip_atomic_store(P.sync + 64 * threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

#define TOKEN_KERNEL(NAME, WT, KV, GMAX)                                          \
  extern "C" __global__ __launch_bounds__(AMMON_WG, 1) void NAME(ammon_k_token p) { \
    decode_token<WT, KV, GMAX>(p);                                              \
  }

// bf16 weights, head 128; bf16 or fp32 KV cache; 1, 2, 4 or 8 q heads per kv head
TOKEN_KERNEL(ammon_token_bf16_kvbf16_g1, uint16_t, uint16_t, 1)
TOKEN_KERNEL(ammon_token_bf16_kvbf16_g2, uint16_t, uint16_t, 2)
TOKEN_KERNEL(ammon_token_bf16_kvbf16_g4, uint16_t, uint16_t, 4)
TOKEN_KERNEL(ammon_token_bf16_kvbf16_g8, uint16_t, uint16_t, 8)
TOKEN_KERNEL(ammon_token_bf16_kvf32_g1, uint16_t, float, 1)
TOKEN_KERNEL(ammon_token_bf16_kvf32_g2, uint16_t, float, 2)
TOKEN_KERNEL(ammon_token_bf16_kvf32_g4, uint16_t, float, 4)
TOKEN_KERNEL(ammon_token_bf16_kvf32_g8, uint16_t, float, 8)
