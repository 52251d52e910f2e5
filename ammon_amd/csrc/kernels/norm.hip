// norm.hip -- RMSNorm, one workgroup per row (reference src/kernels.rs:75-128).
//
// ss = sum x_j^2 (lanes stride the row in 16-byte chunks; wave64 butterfly,
// then the four wave totals in order), s = 1 / sqrt(ss / dim + eps), and
// o_j = w_j * (s * x_j) in the reference's multiplication order.  out may
// alias x (the reference's rmsnorm_inplace): each lane rewrites only the
// elements it read, after the barrier inside block_sum.
#include "device_common.h"

extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_rmsnorm(ammon_k_rmsnorm p) {
  __shared__ float red[AMMON_WAVES];
  const uint32_t row = blockIdx.x;
  const float *x = p.x + (size_t)row * p.dim;
  float *out = p.out + (size_t)row * p.dim;
  const uintptr_t wbits = p.w_dtype == AMMON_K_F32 ? (uintptr_t)p.w : 0;
  const bool vec = (p.dim & 3u) == 0 &&
                   ((((uintptr_t)x) | ((uintptr_t)out) | wbits) & 15u) == 0;
  float ss = 0.f;
  if (vec) {
    for (uint32_t c = threadIdx.x; c < p.dim / 4; c += AMMON_WG) {
      float4 v = ((const float4 *)x)[c];
      ss += v.x * v.x;
      ss += v.y * v.y;
      ss += v.z * v.z;
      ss += v.w * v.w;
    }
  } else {
    for (uint32_t j = threadIdx.x; j < p.dim; j += AMMON_WG) ss += x[j] * x[j];
  }
  ss = block_sum(ss, red);
  ss = ss / (float)p.dim;
  ss = ss + p.eps;
  const float s = 1.0f / sqrtf(ss);
  if (vec) {
    for (uint32_t c = threadIdx.x; c < p.dim / 4; c += AMMON_WG) {
      float4 v = ((const float4 *)x)[c];
      float w[4];
      if (p.w_dtype == AMMON_K_BF16) {
        const uint16_t *wb = (const uint16_t *)p.w + (size_t)c * 4;
        w[0] = bf16_to_f32(wb[0]); w[1] = bf16_to_f32(wb[1]);
        w[2] = bf16_to_f32(wb[2]); w[3] = bf16_to_f32(wb[3]);
      } else {
        float4 wv = ((const float4 *)p.w)[c];
        w[0] = wv.x; w[1] = wv.y; w[2] = wv.z; w[3] = wv.w;
      }
      ((float4 *)out)[c] = make_float4(w[0] * (s * v.x), w[1] * (s * v.y),
                                       w[2] * (s * v.z), w[3] * (s * v.w));
    }
  } else {
    for (uint32_t j = threadIdx.x; j < p.dim; j += AMMON_WG)
      out[j] = load_elem(p.w, p.w_dtype, j) * (s * x[j]);
  }
}
