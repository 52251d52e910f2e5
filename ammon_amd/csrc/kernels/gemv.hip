// gemv.hip -- standalone GEMV kernels (plain, residual, SwiGLU and QKV
// modes, optional RMSNorm prologue) over the pass in gemv_impl.h: one launch
// = one pass with the workgroups of the grid, x staged in dynamic LDS.
#include "gemv_impl.h"

#define GEMV_KERNEL(NAME, WT, CH, RPW, U, MODE)                                 \
  extern "C" __global__ __launch_bounds__(AMMON_WG) void NAME(ammon_k_gemv p) { \
    extern __shared__ float4 xs4[];                                            \
    __shared__ float red[AMMON_WAVES];                                         \
    GemvPass<WT, CH, RPW, U, MODE> pass;                                       \
    pass.begin(p, blockIdx.x, gridDim.x);                                      \
    pass.run(xs4, red);                                                        \
  }

#define GEMV_MODES(PREFIX, WT, CH, RPW, U)                                    \
  GEMV_KERNEL(PREFIX##_plain, WT, CH, RPW, U, AMMON_GEMV_PLAIN)               \
  GEMV_KERNEL(PREFIX##_residual, WT, CH, RPW, U, AMMON_GEMV_RESIDUAL)         \
  GEMV_KERNEL(PREFIX##_swiglu, WT, CH, RPW, U, AMMON_GEMV_SWIGLU)             \
  GEMV_KERNEL(PREFIX##_qkv, WT, CH, RPW, U, AMMON_GEMV_QKV)                     \
  GEMV_KERNEL(PREFIX##_plain_argmax, WT, CH, RPW, U, AMMON_GEMV_PLAIN_ARGMAX)

GEMV_MODES(ammon_gemv_bf16_v, uint16_t, 8, 2, 4)
GEMV_MODES(ammon_gemv_bf16_s, uint16_t, 1, 2, 4)
GEMV_MODES(ammon_gemv_f32_v, float, 4, 2, 4)
GEMV_MODES(ammon_gemv_f32_s, float, 1, 2, 4)
