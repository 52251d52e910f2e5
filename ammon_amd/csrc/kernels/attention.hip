// attention.hip -- standalone split-K decode attention kernels over the
// units in attention_impl.h: pass 1 on a (splits, kv heads) grid, pass 2 on
// a (q heads, head / 8) grid; a z dimension runs consecutive query tokens
// (prefill).
//
// Every kernel takes the DecodeStep pointer first, as a scalar argument that
// this code object asks to have preloaded into SGPRs at wave launch
// (-amdgpu-kernarg-preload-count): the position load, which every request of
// the unit waits for, then goes out without a kernel-argument load before it.
// The parameter struct follows (its copy of the pointer is ignored).
#include "attention_impl.h"

#define ATT_KERNEL(NAME) \
  extern "C" __global__ __launch_bounds__(AMMON_WG) void NAME(const ammon_k_step *step, \
                                                             ammon_k_attention p_)
// ... with registers for at least OCC workgroups per CU
#define ATT_KERNEL_OCC(NAME, OCC)                                                           \
  extern "C" __global__ __launch_bounds__(AMMON_WG, OCC) void NAME(const ammon_k_step *step, \
                                                                  ammon_k_attention p_)
#define ATT_PARAMS(p0)     \
  ammon_k_attention p0 = p_; \
  p0.step = step

#define ATT_PARTIAL(NAME, KV, CH, GMAX, HEAD, EXACT)                             \
  ATT_KERNEL(NAME) {                                                            \
    ATT_PARAMS(p0);                                                             \
    __shared__ float lds[att_lds_floats(GMAX, CH)];                             \
    const ammon_k_attention p = attention_token(p0, blockIdx.z);                \
    AttnPartial<KV, CH, GMAX, HEAD, EXACT> unit;                                \
    if (unit.begin(p, blockIdx.x, blockIdx.y))                                  \
      unit.run(p, lds);                                                         \
    else                                                                        \
      direct_out_nan(p, blockIdx.y);                                            \
  }

#define ATT_PARTIAL_G(PREFIX, KV, CH)                  \
  ATT_PARTIAL(PREFIX##_g1, KV, CH, 1, 0, false)        \
  ATT_PARTIAL(PREFIX##_g2, KV, CH, 2, 0, false)        \
  ATT_PARTIAL(PREFIX##_g4, KV, CH, 4, 0, false)        \
  ATT_PARTIAL(PREFIX##_g8, KV, CH, 8, 0, false)

// generic: any head <= 128 and group size <= 8
ATT_PARTIAL_G(ammon_attention_partial_f32_c4, float, 4)
ATT_PARTIAL_G(ammon_attention_partial_f32_c2, float, 2)
ATT_PARTIAL_G(ammon_attention_partial_f32_c1, float, 1)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c8, uint16_t, 8)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c4, uint16_t, 4)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c2, uint16_t, 2)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c1, uint16_t, 1)

// head 128 with a power-of-two group (Llama-3 shapes): compile-time layout
#define ATT_PARTIAL_H128(PREFIX, KV, CH)               \
  ATT_PARTIAL(PREFIX##_g1, KV, CH, 1, 128, true)       \
  ATT_PARTIAL(PREFIX##_g2, KV, CH, 2, 128, true)       \
  ATT_PARTIAL(PREFIX##_g4, KV, CH, 4, 128, true)       \
  ATT_PARTIAL(PREFIX##_g8, KV, CH, 8, 128, true)

ATT_PARTIAL_H128(ammon_attention_partial_h128_f32_c4, float, 4)

// bf16 K/V, head 128: K/V staged in an LDS ring of NCH 64-position chunk
// buffers by 16-byte buffer-to-LDS requests (AttnPartialMfmaStaged)
// (two per CU, as the two-buffer ring's LDS allows: left to itself the
// compiler put the score tiles in the accumulator registers and copied them
// out: 192 copy instructions in the 4:1 kernel)
#define ATT_PARTIAL_STAGED(NAME, GMAX, NCH)                                          \
  ATT_KERNEL_OCC(NAME, 2) {                                                         \
    ATT_PARAMS(p0);                                                                 \
    __shared__ float lds[att_staged_lds_floats(GMAX, NCH)];                         \
    const ammon_k_attention p = attention_token(p0, blockIdx.z);                    \
    AttnPartialMfmaStaged<GMAX, NCH> unit;                                          \
    if (unit.begin(p, blockIdx.x, blockIdx.y, lds))                                 \
      unit.run(p, lds);                                                             \
    else                                                                            \
      direct_out_nan(p, blockIdx.y);                                                \
  }
#define ATT_PARTIAL_STAGED_G(NCH)                                            \
  ATT_PARTIAL_STAGED(ammon_attention_partial_h128_bf16_lds##NCH##_g1, 1, NCH) \
  ATT_PARTIAL_STAGED(ammon_attention_partial_h128_bf16_lds##NCH##_g2, 2, NCH) \
  ATT_PARTIAL_STAGED(ammon_attention_partial_h128_bf16_lds##NCH##_g4, 4, NCH) \
  ATT_PARTIAL_STAGED(ammon_attention_partial_h128_bf16_lds##NCH##_g8, 8, NCH)
ATT_PARTIAL_STAGED_G(1)
ATT_PARTIAL_STAGED_G(2)

// Merge units of 8 dims: 512 workgroups at the Llama-3-8B shape (32 q
// heads); measured 3.7 us per launch against 4.2 for 32-dim units.
ATT_KERNEL(ammon_attention_combine) {
  ATT_PARAMS(p);
  __shared__ float lds[COMB_LDS_FLOATS_W(8)];
  attention_combine_unit<8>(attention_token(p, blockIdx.z), blockIdx.x, blockIdx.y, lds);
}

// Pass 2 for many query tokens: grid (ceil(q_heads / 4), 1, tokens), one
// wave per (token, q head); the same arithmetic as ammon_attention_combine.
ATT_KERNEL(ammon_attention_combine_waves) {
  ATT_PARAMS(p);
  const ammon_k_attention t = attention_token(p, blockIdx.z);
  const uint32_t h = blockIdx.x * AMMON_WAVES + (threadIdx.x >> 6);
  if (h < t.q_heads) attention_combine_wave(t, h);
}
