// gemv.hip -- standalone GEMV kernels (plain, residual, SwiGLU and QKV
// modes, optional RMSNorm prologue) over the pass in gemv_impl.h: one launch
// = one pass with the workgroups of the grid, x staged in dynamic LDS.
#include "gemv_impl.h"

// The fields the first weight requests depend on come first as scalar
// arguments, which this code object asks to have preloaded into SGPRs at
// wave launch (-amdgpu-kernarg-preload-count): the requests then go out
// without waiting for a kernel-argument load.  The parameter struct follows
// (its copies of these fields are ignored).
#define GEMV_KERNEL(NAME, WT, CH, RPW, U, MODE)                                          \
  extern "C" __global__ __launch_bounds__(AMMON_WG) void NAME(                          \
      const void *w0, const void *w1, const void *w2, uint32_t n, uint32_t rows,        \
      uint32_t row_blocks, uint32_t d, uint32_t kv_dim, uint32_t nwg, ammon_k_gemv p0) { \
    extern __shared__ float4 xs4[];                                                     \
    __shared__ float red[AMMON_WAVES];                                                  \
    ammon_k_gemv p = p0;                                                                \
    p.w0 = w0;                                                                          \
    p.w1 = w1;                                                                          \
    p.w2 = w2;                                                                          \
    p.n = n;                                                                            \
    p.rows = rows;                                                                      \
    p.row_blocks = row_blocks;                                                          \
    p.d = d;                                                                            \
    p.kv_dim = kv_dim;                                                                  \
    GemvPass<WT, CH, RPW, U, MODE> pass;                                                \
    pass.begin(p, blockIdx.x, nwg, xs4);                                                \
    pass.run(xs4, red);                                                                 \
  }

#define GEMV_MODES(PREFIX, WT, CH, RPW, U)                                    \
  GEMV_KERNEL(PREFIX##_plain, WT, CH, RPW, U, AMMON_GEMV_PLAIN)               \
  GEMV_KERNEL(PREFIX##_residual, WT, CH, RPW, U, AMMON_GEMV_RESIDUAL)         \
  GEMV_KERNEL(PREFIX##_swiglu, WT, CH, RPW, U, AMMON_GEMV_SWIGLU)             \
  GEMV_KERNEL(PREFIX##_qkv, WT, CH, RPW, U, AMMON_GEMV_QKV)                     \
  GEMV_KERNEL(PREFIX##_plain_argmax, WT, CH, RPW, U, AMMON_GEMV_PLAIN_ARGMAX)

GEMV_MODES(ammon_gemv_bf16_v, uint16_t, 8, 2, 4)
// Long bf16 matrices without an epilogue (the LM head): 4 rows per wave
// (128256 x 4096: 155 vs 160 us per launch; slower for the per-layer
// projections)
GEMV_KERNEL(ammon_gemv_bf16_w_plain, uint16_t, 8, 4, 4, AMMON_GEMV_PLAIN)
GEMV_KERNEL(ammon_gemv_bf16_w_plain_argmax, uint16_t, 8, 4, 4, AMMON_GEMV_PLAIN_ARGMAX)
GEMV_MODES(ammon_gemv_bf16_s, uint16_t, 1, 2, 4)
GEMV_MODES(ammon_gemv_f32_v, float, 4, 2, 4)
GEMV_MODES(ammon_gemv_f32_s, float, 1, 2, 4)
