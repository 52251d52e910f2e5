// embed.hip -- embedding row gather (reference src/kernels.rs:35-47).
//
// x[r, i] = table[token_r * dim + i], token_r = ids[r] or step->token.
// Grid: (x-blocks over the row, rows).  Each lane moves one 16-byte chunk of
// the table row (4 fp32 or 8 bf16) when the row is 16-byte aligned, else one
// element.  bf16 widens exactly, so the gather is bit-exact.  A token outside
// [0, vocab) -- which the reference would read out of bounds -- fills the row
// with NaN instead of touching memory past the table.
#include "device_common.h"

extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_embed(ammon_k_embed p) {
  const uint32_t row = blockIdx.y;
  const uint32_t token = p.ids ? p.ids[row] : p.step->token;
  float *x = p.x + (size_t)row * p.dim;
  const uint32_t stride = blockDim.x * gridDim.x;
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (token >= p.vocab) {
    for (uint32_t i = tid; i < p.dim; i += stride) x[i] = __uint_as_float(0x7fc00000u);
    return;
  }
  if (p.dtype == AMMON_K_BF16) {
    const uint16_t *src = (const uint16_t *)p.table + (size_t)token * p.dim;
    if ((p.dim & 7u) == 0 && ((((uintptr_t)src) | ((uintptr_t)x)) & 15u) == 0) {
      const uint32_t nv = p.dim / 8;
      for (uint32_t c = tid; c < nv; c += stride) {
        float f[8];
        Chunk<uint16_t, 8>::widen(Chunk<uint16_t, 8>::load(src + (size_t)c * 8), f);
        float4 *dst = (float4 *)(x + (size_t)c * 8);
        dst[0] = make_float4(f[0], f[1], f[2], f[3]);
        dst[1] = make_float4(f[4], f[5], f[6], f[7]);
      }
    } else {
      for (uint32_t i = tid; i < p.dim; i += stride) x[i] = bf16_to_f32(src[i]);
    }
  } else {
    const float *src = (const float *)p.table + (size_t)token * p.dim;
    if ((p.dim & 3u) == 0 && ((((uintptr_t)src) | ((uintptr_t)x)) & 15u) == 0) {
      const uint32_t nv = p.dim / 4;
      for (uint32_t c = tid; c < nv; c += stride)
        ((float4 *)x)[c] = ((const float4 *)src)[c];
    } else {
      for (uint32_t i = tid; i < p.dim; i += stride) x[i] = src[i];
    }
  }
}
