// block.hip -- the reference's recorded attention block (src/blocks.rs:172-259)
// and SwiGLU block (src/blocks.rs:261-278) each as ONE launch, built from the
// same per-row and per-unit code as the standalone kernels (gemv_impl.h,
// attention_impl.h), so the results are bit-identical to the launch list.
//
// Why: at batch 1 every kernel boundary costs a drain and a ramp of the
// whole device (3-5 us against 8-40 us kernels), and the attention block is
// four short launches.  Here all workgroups are resident for the block and
// the dependent phases are separated by grid barriers (grid_sync.h), and a
// workgroup requests, before it waits, the next phase's inputs that do not
// depend on the phase in progress.
//
// Measured at the Llama-3-8B shape (context 8192, one MI355X): the
// attention block takes 40 us against 34 us for its four launches and the
// SwiGLU block 65-66 us against 63 us for its two -- each barrier plus the
// loads of another workgroup's results costs about what a kernel boundary
// costs, whatever the staging loads' cache policy, and the prefetch ahead of
// a barrier does not shorten the phase after it.  The model therefore
// records the separate launches unless asked for one launch per block
// (ammon_llama_config.one_launch_blocks).
//
// Attention block, one workgroup per CU slot (2 per CU):
//   1. norm + QKV GEMV + RoPE; q and the position's K/V rows stored.
//      A workgroup done with its rows then requests its attention unit's
//      K/V (every row but the position's, not stored yet): HBM keeps
//      streaming through the barrier.
//   2. barrier; q (and the chunk holding the new row) are requested, the
//      unit scores, accumulates and stores its split partial, then requests
//      its first two Wo tiles (at 2 workgroups per CU, about all of Wo),
//      which stream through the next two barriers and the merge.
//   3. barrier; the log-sum-exp merge, one (q head, 8-dim slice) per
//      workgroup.
//   4. barrier; the Wo GEMV + residual, its first tiles already in registers.
// SwiGLU block: norm + gate/up GEMV + SwiGLU; the first two W2 tiles
// requested; barrier; W2 GEMV + residual.
//
// Handoff between workgroups inside the launch: agent-scope stores and loads
// (AMMON_AGENT_HANDOFF, device_common.h).  The launch ends with a final
// arrival whose completing workgroup zeroes the barrier counters.
//
// Requires gridDim.x workgroups to be co-resident; the host sizes the grid
// from the occupancy of this code object (2 per CU), and a barrier that
// waits too long gives up and flags the launch instead of hanging.
#define AMMON_AGENT_HANDOFF 1
#include "attention_impl.h"
#include "gemv_impl.h"
#include "grid_sync.h"

namespace {

// the standalone bf16 GEMV's tiling (gemv.hip, ammon_gemv_bf16_v_*)
template <int MODE>
using Bf16Pass = GemvPass<uint16_t, 8, 2, 4, MODE>;

// K/V chunk buffers of the attention unit: two 64-position chunks
// prefetched for 1-2 q heads per kv head; one for 4-8, whose accumulators
// leave no room for a second under two workgroups per CU
template <int GMAX>
constexpr int kv_bufs() {
  return GMAX <= 2 ? 2 : 1;
}

template <int GMAX>
AMMON_DEV void attention_block(const ammon_k_attn_block &P) {
  extern __shared__ float4 lds4[];
  float *lds = (float *)lds4;
  __shared__ float red[AMMON_WAVES];
  const uint32_t wg = blockIdx.x, G = gridDim.x;
  GridSync bar{P.sync, G, 0, P.spin_limit, nullptr, 0};
  const ammon_k_attention &a = P.att;
  const uint32_t units = a.kv_heads * a.splits;

  {  // 1. norm + QKV + RoPE + K/V store
    Bf16Pass<AMMON_GEMV_QKV> qkv;
    qkv.begin(P.qkv, wg, G);
    qkv.run(lds4, red);
  }
  // requested ahead of the barrier: the first attention unit's older K/V rows
  AttnPartialMfma<GMAX, kv_bufs<GMAX>()> unit;
  const bool first = wg < units && unit.prefetch(a, wg % a.splits, wg / a.splits);
  bar.sync_all();  // q and the position's K/V rows stored

  // 2. split-K attention
  if (first) {
    unit.finish(a);
    unit.run(a, lds);
  }
  for (uint32_t u = wg + G; u < units; u += G) {
    AttnPartialMfma<GMAX, kv_bufs<GMAX>()> more;
    if (more.begin(a, u % a.splits, u / a.splits)) more.run(a, lds);
  }
  // requested ahead of the next two barriers and the merge: the first Wo
  // tiles (two per workgroup: about all of Wo at 2 workgroups per CU)
  Bf16Pass<AMMON_GEMV_RESIDUAL> wo;
  wo.begin(P.wo, wg, G);
  bar.sync_all();  // partials stored

  // 3. merge
  const uint32_t slices = a.head / 8;
  for (uint32_t u = wg; u < a.q_heads * slices; u += G)
    attention_combine_unit<8>(a, u / slices, u % slices, lds);
  bar.sync_all();  // attention output stored

  // 4. output projection + residual
  wo.run(lds4, red);
  bar.arrive_final();
}

AMMON_DEV void ffn_block(const ammon_k_ffn_block &P) {
  extern __shared__ float4 lds4[];
  __shared__ float red[AMMON_WAVES];
  const uint32_t wg = blockIdx.x, G = gridDim.x;
  GridSync bar{P.sync, G, 0, P.spin_limit, nullptr, 0};
  {  // norm + gate/up + SwiGLU
    Bf16Pass<AMMON_GEMV_SWIGLU> gate_up;
    gate_up.begin(P.gate_up, wg, G);
    gate_up.run(lds4, red);
  }
  Bf16Pass<AMMON_GEMV_RESIDUAL> down;
  down.begin(P.down, wg, G);  // first W2 tiles, ahead of the barrier
  bar.sync_all();             // hb stored
  down.run(lds4, red);
  bar.arrive_final();
}

}  // namespace

// bf16 weights and KV cache, head 128; 1, 2 or 4 q heads per kv head (8
// needs more registers than two workgroups per CU leave: the launch list)
#define ATTN_BLOCK(NAME, GMAX)                                                        \
  extern "C" __global__ __launch_bounds__(AMMON_WG, 2) void NAME(ammon_k_attn_block p) { \
    attention_block<GMAX>(p);                                                         \
  }
ATTN_BLOCK(ammon_attn_block_bf16_g1, 1)
ATTN_BLOCK(ammon_attn_block_bf16_g2, 2)
ATTN_BLOCK(ammon_attn_block_bf16_g4, 4)

extern "C" __global__ __launch_bounds__(AMMON_WG, 2) void ammon_ffn_block_bf16(ammon_k_ffn_block p) {
  ffn_block(p);
}
