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

// bf16 K/V: q.k on matrix cores with two chunk buffers, one for the 4:1
// group (the Llama-3 shape): at split 128 every workgroup requesting both of
// its chunks at once delays all first chunks -- one buffer measured 0.1-0.7
// us faster per launch at positions 1023..8191 (four buffers no faster than
// two).  One for the 8:1 group too: 242 VGPRs fit two workgroups per CU,
// where two buffers (256 VGPRs + 70 AGPRs) fit one, and the Llama-3-70B
// layer at 32768 positions then steps in 0.623-0.625 ms against 0.635-0.636
// (each at its best split: 512 against 1024)
#define ATT_PARTIAL_MFMA(NAME, GMAX, NBUF)                                           \
  ATT_KERNEL(NAME) {                                                                \
    ATT_PARAMS(p0);                                                                 \
    __shared__ float lds[att_lds_floats(GMAX, 8)];                                  \
    const ammon_k_attention p = attention_token(p0, blockIdx.z);                    \
    AttnPartialMfma<GMAX, NBUF> unit;                                               \
    if (unit.begin(p, blockIdx.x, blockIdx.y))                                      \
      unit.run(p, lds);                                                             \
    else                                                                            \
      direct_out_nan(p, blockIdx.y);                                                \
  }
ATT_PARTIAL_MFMA(ammon_attention_partial_h128_bf16_c8_g1, 1, 2)
ATT_PARTIAL_MFMA(ammon_attention_partial_h128_bf16_c8_g2, 2, 2)
ATT_PARTIAL_MFMA(ammon_attention_partial_h128_bf16_c8_g4, 4, 1)
ATT_PARTIAL_MFMA(ammon_attention_partial_h128_bf16_c8_g8, 8, 1)
ATT_PARTIAL_H128(ammon_attention_partial_h128_f32_c4, float, 4)


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
