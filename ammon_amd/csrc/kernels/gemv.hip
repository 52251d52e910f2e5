// gemv.hip -- bandwidth-bound batch-1 GEMV family with fused prologue and
// epilogues (replaces the reference's Goldy matmul_into, src/kernels.rs:518-528,
// whose definition is the serial gemv, src/kernels.rs:54-73, and the
// surrounding rmsnorm / rope_store / cache_store / swiglu / add_into launches
// of src/blocks.rs:219-276).
//
// y_i = sum_j W[i, j] x_j with W row-major [rows, n] in fp32 or bf16.
//
// Workgroup of 4 wave64s.  x (optionally RMS-normalised) is staged once per
// workgroup in LDS as fp32.  Each wave owns RPW consecutive "virtual rows"
// per row block; lane l streams the 16-byte chunks l, l+64, ... of each of
// its rows (coalesced 1 KiB per wave per load instruction), keeping U chunk
// loads per row in flight, multiplies them against the matching LDS slice
// of x and reduces each row with a wave64 butterfly.  Row blocks are
// distributed grid-stride so x is staged once per resident workgroup.  No
// MFMA: at batch 1 the arithmetic intensity is ~1 flop/byte.
//
// Modes (virtual rows):
//   PLAIN     y[r] = dot_r; with a step, y[position * d + r] (reference gemv)
//   RESIDUAL  y[r] = residual[r] + dot_r            (y may alias residual)
//   SWIGLU    rows interleave gate (w0) and up (w1): r = 2i -> gate row i,
//             r = 2i+1 -> up row i; y[i] = silu(gate) * up in the reference's
//             order (src/kernels.rs:472-475)
//   QKV       rows run over [Wq; Wk; Wv]; (2i, 2i+1) pairs of q and k rows are
//             rotated with the cos/sin table at step->position; q goes to y,
//             rotated k and raw v go to the head-major caches at that position
//             (src/kernels.rs:174-226).
#include "device_common.h"

// The RMSNorm prologue sums squares with the same per-lane chunking and
// reduction order as ammon_rmsnorm, so its normalised x matches the
// standalone kernel bit for bit when the row is 16-byte aligned.
template <typename WT, int CH, int RPW, int MODE>
AMMON_DEV void gemv_body(const ammon_k_gemv &p) {
  constexpr int U = (CH >= 4) ? (16 / RPW > 0 ? 16 / RPW : 1) : 4;
  extern __shared__ float xs[];
  __shared__ float red[AMMON_WAVES];
  const uint32_t n = p.n;
  const uint32_t tid = threadIdx.x;

  // ---- stage x, optional RMSNorm prologue --------------------------------
  float ss = 0.f;
  const bool xvec = (n & 3u) == 0 && (((uintptr_t)p.x) & 15u) == 0;
  if (xvec) {
    for (uint32_t c = tid; c < n / 4; c += AMMON_WG) {
      float4 v = ((const float4 *)p.x)[c];
      ((float4 *)xs)[c] = v;
      ss += v.x * v.x;
      ss += v.y * v.y;
      ss += v.z * v.z;
      ss += v.w * v.w;
    }
  } else {
    for (uint32_t j = tid; j < n; j += AMMON_WG) {
      const float v = p.x[j];
      xs[j] = v;
      ss += v * v;
    }
  }
  if (p.norm_w) {
    ss = block_sum(ss, red);
    ss = ss / (float)n;
    ss = ss + p.eps;
    const float s = 1.0f / sqrtf(ss);
    for (uint32_t j = tid; j < n; j += AMMON_WG)
      xs[j] = load_elem(p.norm_w, p.norm_dtype, j) * (s * xs[j]);
  }
  __syncthreads();

  // ---- stream rows -------------------------------------------------------
  using C = Chunk<WT, CH>;
  const uint32_t lane = tid & 63, wave = tid >> 6;
  const uint32_t nch = n / CH;
  uint32_t pos = 0;
  if (MODE == AMMON_GEMV_QKV) pos = p.step->position;
  // PLAIN with a step: the reference's position-strided gemv
  // (src/kernels.rs:49-73) writes row `position` of a [seq, d] output.
  float *yout = p.y;
  bool write_ok = true;
  if (MODE == AMMON_GEMV_PLAIN && p.step) {
    const uint32_t ps = p.step->position;
    write_ok = ps < p.seq;
    yout = p.y + (size_t)(write_ok ? ps : 0) * p.d;
  }

  for (uint32_t blk = blockIdx.x; blk < p.row_blocks; blk += gridDim.x) {
    const uint32_t r0 = (blk * AMMON_WAVES + wave) * RPW;
    const WT *wrow[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      uint32_t vr = r0 + k;
      if (vr >= p.rows) vr = 0;  // row past the end: read row 0, discard
      const WT *base;
      size_t row;
      if (MODE == AMMON_GEMV_SWIGLU) {
        base = (const WT *)((vr & 1u) ? p.w1 : p.w0);
        row = vr >> 1;
      } else if (MODE == AMMON_GEMV_QKV) {
        if (vr < p.d) {
          base = (const WT *)p.w0;
          row = vr;
        } else if (vr < p.d + p.kv_dim) {
          base = (const WT *)p.w1;
          row = vr - p.d;
        } else {
          base = (const WT *)p.w2;
          row = vr - p.d - p.kv_dim;
        }
      } else {
        base = (const WT *)p.w0;
        row = vr;
      }
      wrow[k] = base + row * n;
    }

    float acc[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) acc[k] = 0.f;

    for (uint32_t c0 = 0; c0 < nch; c0 += 64 * U) {
      typename C::V w[RPW][U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t c = c0 + u * 64 + lane;
#pragma unroll
        for (int k = 0; k < RPW; ++k)
          w[k][u] = (c < nch) ? C::load(wrow[k] + (size_t)c * CH) : C::zero();
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t c = c0 + u * 64 + lane;
        if (c < nch) {
          float xv[CH];
#pragma unroll
          for (int e = 0; e < CH; ++e) xv[e] = xs[c * CH + e];
#pragma unroll
          for (int k = 0; k < RPW; ++k) {
            float wf[CH];
            C::widen(w[k][u], wf);
            float s = acc[k];
#pragma unroll
            for (int e = 0; e < CH; ++e) s += wf[e] * xv[e];
            acc[k] = s;
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < RPW; ++k) acc[k] = wave_sum(acc[k]);

    // ---- epilogues (lane k handles row k / pair k) ------------------------
    if (MODE == AMMON_GEMV_PLAIN || MODE == AMMON_GEMV_RESIDUAL) {
#pragma unroll
      for (int k = 0; k < RPW; ++k) {
        const uint32_t vr = r0 + k;
        if ((uint32_t)k == lane && vr < p.rows) {
          if (MODE == AMMON_GEMV_RESIDUAL)
            p.y[vr] = p.residual[vr] + acc[k];
          else if (write_ok)
            yout[vr] = acc[k];
        }
      }
    } else if (MODE == AMMON_GEMV_SWIGLU) {
#pragma unroll
      for (int k = 0; k < RPW; k += 2) {
        const uint32_t vr = r0 + k;
        if ((uint32_t)k == lane && vr < p.rows) {
          const float gate = acc[k], up = acc[k + 1];
          float v = gate * (1.0f / (1.0f + expf(-gate)));
          v = v * up;
          p.y[vr >> 1] = v;
        }
      }
    } else {  // QKV
#pragma clang fp contract(off)
#pragma unroll
      for (int k = 0; k < RPW; k += 2) {
        const uint32_t vr = r0 + k;
        if ((uint32_t)k != lane || vr >= p.rows) continue;
        const float a0 = acc[k], a1 = acc[k + 1];
        if (pos >= p.seq) {  // out-of-range position: poison q, touch no cache
          if (vr < p.d) p.y[vr] = p.y[vr + 1] = __uint_as_float(0x7fc00000u);
          continue;
        }
        if (vr < p.d + p.kv_dim) {
          const uint32_t rr = vr < p.d ? vr : vr - p.d;
          const uint32_t hd = rr % p.head;
          const float *cs = p.table + ((size_t)pos * (p.head / 2) + hd / 2) * 2;
          const float fcr = cs[0], fci = cs[1];
          const float o0 = a0 * fcr - a1 * fci;
          const float o1 = a0 * fci + a1 * fcr;
          if (vr < p.d) {
            p.y[vr] = o0;
            p.y[vr + 1] = o1;
          } else {
            const size_t dst = ((size_t)(rr / p.head) * p.seq + pos) * p.head + hd;
            store_elem(p.k_cache, p.kv_dtype, dst, o0);
            store_elem(p.k_cache, p.kv_dtype, dst + 1, o1);
          }
        } else {
          const uint32_t rv = vr - p.d - p.kv_dim;
          const size_t dst = ((size_t)(rv / p.head) * p.seq + pos) * p.head + rv % p.head;
          store_elem(p.v_cache, p.kv_dtype, dst, a0);
          store_elem(p.v_cache, p.kv_dtype, dst + 1, a1);
        }
      }
    }
  }
}

#define GEMV_KERNEL(NAME, WT, CH, RPW, MODE)                                    \
  extern "C" __global__ __launch_bounds__(AMMON_WG) void NAME(ammon_k_gemv p) { \
    gemv_body<WT, CH, RPW, MODE>(p);                                           \
  }

#define GEMV_MODES(PREFIX, WT, CH, RPW)                                    \
  GEMV_KERNEL(PREFIX##_plain, WT, CH, RPW, AMMON_GEMV_PLAIN)               \
  GEMV_KERNEL(PREFIX##_residual, WT, CH, RPW, AMMON_GEMV_RESIDUAL)         \
  GEMV_KERNEL(PREFIX##_swiglu, WT, CH, RPW, AMMON_GEMV_SWIGLU)             \
  GEMV_KERNEL(PREFIX##_qkv, WT, CH, RPW, AMMON_GEMV_QKV)

GEMV_MODES(ammon_gemv_bf16_v, uint16_t, 8, 2)
GEMV_MODES(ammon_gemv_bf16_s, uint16_t, 1, 2)
GEMV_MODES(ammon_gemv_f32_v, float, 4, 2)
GEMV_MODES(ammon_gemv_f32_s, float, 1, 2)
