// device_common.h -- shared gfx950 device helpers: bf16 conversion, 16-byte
// chunk loads, wave64 and workgroup reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kernel_params.h"

#define AMMON_DEV __device__ __forceinline__
#define AMMON_WG 256
#define AMMON_WAVES (AMMON_WG / 64)

// ---- bf16 ------------------------------------------------------------------
AMMON_DEV float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
AMMON_DEV float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
AMMON_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even; NaN stays a (quiet) NaN.
AMMON_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

AMMON_DEV void store_elem(void *base, uint32_t dtype, size_t i, float v) {
  if (dtype == AMMON_K_BF16)
    ((uint16_t *)base)[i] = f32_to_bf16(v);
  else
    ((float *)base)[i] = v;
}

// Results pass between kernels at kernel boundaries only: outputs are plain
// stores (st_out) and inputs another kernel wrote are plain loads (ld_in,
// ld_in4).
// Weight matrices are streamed once per token: nontemporal buffer loads
// (aux 2 = nt).  Measured at the Llama-3-8B shape: gate/up 40.7 -> 38.0 us,
// LM head 178 -> 163 us.
#define AMMON_WEIGHT_CPOL 2
template <typename T>
AMMON_DEV void st_out_t(T *p, T v) {
  *p = v;
}
template <typename T>
AMMON_DEV T ld_in(const T *p) {
  return *p;
}
// ... four floats at a 16-byte-aligned address
AMMON_DEV float4 ld_in4(const float *p) { return *(const float4 *)p; }
AMMON_DEV void st_out(float *p, float v) { st_out_t(p, v); }
AMMON_DEV void st_out(uint32_t *p, uint32_t v) { st_out_t(p, v); }
AMMON_DEV void st_out(int32_t *p, int32_t v) { st_out_t(p, v); }
// Elements i and i + 1 (i even) of an fp32 / bf16 array as one store.
AMMON_DEV void store_pair_out(void *base, uint32_t dtype, size_t i, float a, float b) {
  if (dtype == AMMON_K_BF16) {
    const uint32_t w = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
    st_out_t((uint32_t *)((uint16_t *)base + i), w);
  } else {
    const uint64_t w = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
    st_out_t((uint64_t *)((float *)base + i), w);
  }
}

AMMON_DEV float load_elem(const void *base, uint32_t dtype, size_t i) {
  if (dtype == AMMON_K_BF16) return bf16_to_f32(((const uint16_t *)base)[i]);
  return ((const float *)base)[i];
}

// s_waitcnt that waits until at most N vector-memory operations of this wave
// are outstanding (expcnt and lgkmcnt left at their maxima; gfx9 encoding:
// vmcnt bits 3:0 and 15:14).  Loads complete in order, so this is how a
// wave waits for the requests it issued before its last N.
template <int N> AMMON_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// ---- chunk loads -----------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Buffer resource (V#) over [base, base + bytes): raw buffer loads at byte
// offsets >= bytes return zero and touch no memory, which replaces
// per-lane bounds branches.  Dword 3 is the gfx9-family raw-buffer format.
#define AMMON_BUFFER_DWORD3 0x00020000
AMMON_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, AMMON_BUFFER_DWORD3);
}
#define AMMON_OOB 0x80000000u  // a byte offset past every buffer used here

// Chunk<T, CH>: CH consecutive elements of storage type T (float or bf16
// stored as uint16_t) loaded with one vector load and widened to fp32.
// load_buf reads the chunk at byte offset `off` of a buffer resource.
template <typename T, int CH> struct Chunk;

template <> struct Chunk<uint16_t, 8> {
  using V = u32x4;
  template <int CPOL = 0>
  static AMMON_DEV V load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL);
  }
  static AMMON_DEV V load(const uint16_t *p) { return *(const V *)p; }
  static AMMON_DEV V load_nt(const uint16_t *p) { return __builtin_nontemporal_load((const V *)p); }
  static AMMON_DEV V zero() { return V{0u, 0u, 0u, 0u}; }
  static AMMON_DEV void widen(V v, float *f) {
    f[0] = bf16_lo(v[0]); f[1] = bf16_hi(v[0]);
    f[2] = bf16_lo(v[1]); f[3] = bf16_hi(v[1]);
    f[4] = bf16_lo(v[2]); f[5] = bf16_hi(v[2]);
    f[6] = bf16_lo(v[3]); f[7] = bf16_hi(v[3]);
  }
};

template <> struct Chunk<uint16_t, 4> {
  using V = u32x2;
  template <int CPOL = 0>
  static AMMON_DEV V load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CPOL);
  }
  static AMMON_DEV V load(const uint16_t *p) { return *(const V *)p; }
  static AMMON_DEV V load_nt(const uint16_t *p) { return __builtin_nontemporal_load((const V *)p); }
  static AMMON_DEV V zero() { return V{0u, 0u}; }
  static AMMON_DEV void widen(V v, float *f) {
    f[0] = bf16_lo(v[0]); f[1] = bf16_hi(v[0]);
    f[2] = bf16_lo(v[1]); f[3] = bf16_hi(v[1]);
  }
};

template <> struct Chunk<uint16_t, 2> {
  using V = uint32_t;
  template <int CPOL = 0>
  static AMMON_DEV V load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL);
  }
  static AMMON_DEV V load(const uint16_t *p) { return *(const uint32_t *)p; }
  static AMMON_DEV V load_nt(const uint16_t *p) {
    return __builtin_nontemporal_load((const uint32_t *)p);
  }
  static AMMON_DEV V zero() { return 0u; }
  static AMMON_DEV void widen(V v, float *f) { f[0] = bf16_lo(v); f[1] = bf16_hi(v); }
};

template <> struct Chunk<uint16_t, 1> {
  using V = uint16_t;
  template <int CPOL = 0>
  static AMMON_DEV V load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, CPOL);
  }
  static AMMON_DEV V load(const uint16_t *p) { return *p; }
  static AMMON_DEV V load_nt(const uint16_t *p) { return *p; }
  static AMMON_DEV V zero() { return 0; }
  static AMMON_DEV void widen(V v, float *f) { f[0] = bf16_to_f32(v); }
};

template <> struct Chunk<float, 4> {
  using V = f32x4;
  template <int CPOL = 0>
  static AMMON_DEV V load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL));
  }
  static AMMON_DEV V load(const float *p) { return *(const V *)p; }
  static AMMON_DEV V load_in(const float *p) {  // another kernel's output (ld_in4)
    const float4 v = ld_in4(p);
    return V{v.x, v.y, v.z, v.w};
  }
  static AMMON_DEV V load_nt(const float *p) { return __builtin_nontemporal_load((const V *)p); }
  static AMMON_DEV V zero() { return V{0.f, 0.f, 0.f, 0.f}; }
  static AMMON_DEV void widen(V v, float *f) { f[0] = v[0]; f[1] = v[1]; f[2] = v[2]; f[3] = v[3]; }
};

template <> struct Chunk<float, 2> {
  using V = f32x2;
  template <int CPOL = 0>
  static AMMON_DEV V load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CPOL));
  }
  static AMMON_DEV V load(const float *p) { return *(const V *)p; }
  static AMMON_DEV V load_in(const float *p) {  // another kernel's output (8-byte load)
    const uint64_t a = ld_in((const uint64_t *)p);
    return V{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32))};
  }
  static AMMON_DEV V load_nt(const float *p) { return __builtin_nontemporal_load((const V *)p); }
  static AMMON_DEV V zero() { return V{0.f, 0.f}; }
  static AMMON_DEV void widen(V v, float *f) { f[0] = v[0]; f[1] = v[1]; }
};

template <> struct Chunk<float, 1> {
  using V = float;
  template <int CPOL = 0>
  static AMMON_DEV V load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL));
  }
  static AMMON_DEV V load(const float *p) { return *p; }
  static AMMON_DEV V load_in(const float *p) { return ld_in(p); }  // another kernel's output
  static AMMON_DEV V load_nt(const float *p) { return *p; }
  static AMMON_DEV V zero() { return 0.f; }
  static AMMON_DEV void widen(V v, float *f) { f[0] = v; }
};

// ---- reductions --------------------------------------------------------------
// DPP reductions inside 16-lane rows.  Each step is one VALU op reading a
// permuted neighbour: quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1]
// (xor 2), row_half_mirror (pairs quads 0/1, 2/3) and row_mirror (pairs
// half rows).  After the steps up to WIDTH every lane of a WIDTH-lane group
// holds the group's total; both operands of each add hold identically
// associated partial sums, so the lanes agree bit for bit.
#define AMMON_DPP_XOR1 0xB1
#define AMMON_DPP_XOR2 0x4E
#define AMMON_DPP_HALF_MIRROR 0x141
#define AMMON_DPP_MIRROR 0x140

template <int CTRL> AMMON_DEV float dpp_get(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

AMMON_DEV float lane_get(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Whole-wave reductions (call with all 64 lanes active): the four DPP
// steps give each 16-lane row its total, the row totals are read into
// scalar registers and combined as (r0 + r1) + (r2 + r3).  Every lane gets
// the identical, deterministically associated value.  Narrower widths use
// an xor butterfly.
template <int WIDTH = 64> AMMON_DEV float wave_sum(float v) {
  if constexpr (WIDTH == 64) {
    v += dpp_get<AMMON_DPP_XOR1>(v);
    v += dpp_get<AMMON_DPP_XOR2>(v);
    v += dpp_get<AMMON_DPP_HALF_MIRROR>(v);
    v += dpp_get<AMMON_DPP_MIRROR>(v);
    return (lane_get(v, 0) + lane_get(v, 16)) + (lane_get(v, 32) + lane_get(v, 48));
  } else {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
  }
}

template <int WIDTH = 64> AMMON_DEV float wave_max(float v) {
  if constexpr (WIDTH == 64) {
    v = fmaxf(v, dpp_get<AMMON_DPP_XOR1>(v));
    v = fmaxf(v, dpp_get<AMMON_DPP_XOR2>(v));
    v = fmaxf(v, dpp_get<AMMON_DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_get<AMMON_DPP_MIRROR>(v));
    return fmaxf(fmaxf(lane_get(v, 0), lane_get(v, 16)), fmaxf(lane_get(v, 32), lane_get(v, 48)));
  } else {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
  }
}

// Sum over aligned groups of `width` lanes (width in {1, 2, 4, 8, 16}).
AMMON_DEV float group_sum16(float v, uint32_t width) {
  if (width >= 2) v += dpp_get<AMMON_DPP_XOR1>(v);
  if (width >= 4) v += dpp_get<AMMON_DPP_XOR2>(v);
  if (width >= 8) v += dpp_get<AMMON_DPP_HALF_MIRROR>(v);
  if (width >= 16) v += dpp_get<AMMON_DPP_MIRROR>(v);
  return v;
}

// Sum over a 256-thread workgroup; `red` must hold AMMON_WAVES floats.  The
// wave totals are added in wave order.  Contains barriers: call uniformly.
AMMON_DEV float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < AMMON_WAVES; ++w) t += red[w];
  __syncthreads();
  return t;
}

AMMON_DEV float block_max(float v, float *red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < AMMON_WAVES; ++w) t = fmaxf(t, red[w]);
  __syncthreads();
  return t;
}
