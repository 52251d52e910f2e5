// misc.hip -- elementwise SwiGLU and residual add, the greedy argmax with
// DecodeStep feedback, and fills for synthetic weights and scratch clearing.
#include "argmax_impl.h"

// hb = silu(hb) * hb2 in the reference's order (src/kernels.rs:462-476).
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_swiglu(ammon_k_elementwise p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.n) return;
  float val = p.hb[i];
  val = val * (1.0f / (1.0f + expf(-val)));
  val = val * p.b[i];
  p.hb[i] = val;
}

// out = a + b (Goldy add_into as used for residuals, src/blocks.rs:256-257).
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_add(ammon_k_elementwise p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.n) return;
  p.hb[i] = p.a[i] + p.b[i];
}

// ---- argmax (candidate order in argmax_impl.h) -------------------------------
// Pass 1: one candidate per workgroup.
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_argmax_partial(ammon_k_argmax p) {
  float v = 0.f;
  uint32_t idx = ARGMAX_NONE;
  for (uint32_t i = blockIdx.x * AMMON_WG + threadIdx.x; i < p.n; i += gridDim.x * AMMON_WG) {
    const float x = p.logits[i];
    if (x == x) cand_merge(v, idx, x, i);
  }
  __shared__ float sv[AMMON_WG];
  __shared__ uint32_t si[AMMON_WG];
  block_cand_reduce(v, idx, sv, si);
  if (threadIdx.x == 0) {
    p.cand_v[blockIdx.x] = v;
    p.cand_i[blockIdx.x] = idx;
  }
}

// Pass 2 (one workgroup): fold the candidates, apply the logits[0] rule, and
// optionally feed the choice back into the device DecodeStep with the greedy
// loop's prompt forcing (reference src/generate.rs:60-72):
//   next = pos + 1 < n_prompt ? prompt[pos + 1] : argmax;  tokens[pos] = next;
//   step = {next, pos + 1}.
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_argmax_final(ammon_k_argmax p) {
  float v = 0.f;
  uint32_t idx = ARGMAX_NONE;
  for (uint32_t b = threadIdx.x; b < p.blocks; b += AMMON_WG) cand_merge(v, idx, p.cand_v[b], p.cand_i[b]);
  __shared__ float sv[AMMON_WG];
  __shared__ uint32_t si[AMMON_WG];
  block_cand_reduce(v, idx, sv, si);
  if (threadIdx.x != 0) return;
  const float first = p.logits[0];
  int32_t best = (first != first || idx == ARGMAX_NONE) ? 0 : (int32_t)idx;
  if (p.out) *p.out = best;
  if (p.step) {
    const uint32_t pos = p.step->position;
    const int32_t next = (pos + 1 < p.n_prompt) ? p.prompt[pos + 1] : best;
    if (p.tokens && pos < p.max_tokens) p.tokens[pos] = next;
    p.step->token = (uint32_t)next;
    p.step->position = pos + 1;
  }
}

// ---- storage checksum ------------------------------------------------------------
// (wrapping sum, xor) of a buffer's little-endian 64-bit words.  Both are
// associative and commutative, so the workgroups fold their results into
// out[] with 64-bit atomics in any order and the answer is exact.  Each lane
// keeps CK_U 16-byte loads in flight per sweep and does two integer ops per
// word, so the kernel is a plain streaming read of the buffer.
#define CK_U 8
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_checksum(ammon_k_checksum p) {
  const u32x4 *src = (const u32x4 *)p.src;
  const uint64_t n16 = p.bytes / 16;
  const uint64_t stride = (uint64_t)gridDim.x * AMMON_WG;
  unsigned long long s = 0, x = 0;
  auto fold = [&](u32x4 v) {
    const unsigned long long a = ((unsigned long long)v[1] << 32) | v[0];
    const unsigned long long b = ((unsigned long long)v[3] << 32) | v[2];
    s += a + b;
    x ^= a ^ b;
  };
  uint64_t i = (uint64_t)blockIdx.x * AMMON_WG + threadIdx.x;
  for (; i + (CK_U - 1) * stride < n16; i += CK_U * stride) {
    u32x4 v[CK_U];
#pragma unroll
    for (int u = 0; u < CK_U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < CK_U; ++u) fold(v[u]);
  }
  for (; i < n16; i += stride) fold(src[i]);
  // an 8-byte tail word
  if (blockIdx.x == 0 && threadIdx.x == 0 && (p.bytes & 8)) {
    const unsigned long long t = ((const unsigned long long *)p.src)[p.bytes / 8 - 1];
    s += t;
    x ^= t;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    s += __shfl_xor(s, off, 64);
    x ^= __shfl_xor(x, off, 64);
  }
  // one atomic pair per workgroup: the waves' sums meet in LDS first (every
  // atomic on the two result words is serialized at one address)
  __shared__ unsigned long long ws[AMMON_WAVES], wx[AMMON_WAVES];
  const uint32_t wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    ws[wave] = s;
    wx[wave] = x;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < AMMON_WAVES; ++w) {
      s += ws[w];
      x ^= wx[w];
    }
    atomicAdd(p.out, s);
    atomicXor(p.out + 1, x);
  }
}

// ---- streaming read ------------------------------------------------------------
// Reads src[0, bytes) once and keeps nothing: the floor for a launch that
// moves that many bytes.  Workgroup w reads bytes [w share, (w + 1) share)
// in windows of 16 KiB (four 16-byte loads per lane, 1 KiB contiguous per
// wave and load), requesting the next window before folding the current one;
// the loads go through a buffer resource bounded to the share, so a tail
// past the buffer reads zero without touching memory.  The folded value is
// consumed by an empty asm statement: no store, no atomic.
#define SR_WIN 4
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_stream_read(ammon_k_stream_read p) {
  constexpr uint32_t win_bytes = AMMON_WG * SR_WIN * 16;
  const uint64_t start = (uint64_t)blockIdx.x * p.share;
  const uint32_t len =
      start >= p.bytes ? 0u : (uint32_t)(p.bytes - start < p.share ? p.bytes - start : p.share);
  const __amdgpu_buffer_rsrc_t r =
      make_rsrc((const char *)p.src + (start >= p.bytes ? 0 : start), len);
  const uint32_t rounds = (uint32_t)(p.share / win_bytes);
  uint32_t off = threadIdx.x * 16u;
  u32x4 a[SR_WIN], b[SR_WIN];
  u32x4 x = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int u = 0; u < SR_WIN; ++u)
    a[u] = __builtin_amdgcn_raw_buffer_load_b128(r, off + u * AMMON_WG * 16u, 0, AMMON_WEIGHT_CPOL);
  for (uint32_t k = 1; k < rounds; ++k) {
    off += win_bytes;
#pragma unroll
    for (int u = 0; u < SR_WIN; ++u)
      b[u] = __builtin_amdgcn_raw_buffer_load_b128(r, off + u * AMMON_WG * 16u, 0, AMMON_WEIGHT_CPOL);
#pragma unroll
    for (int u = 0; u < SR_WIN; ++u) {
      x ^= a[u];
      a[u] = b[u];
    }
  }
#pragma unroll
  for (int u = 0; u < SR_WIN; ++u) x ^= a[u];
  const uint32_t f = x[0] ^ x[1] ^ x[2] ^ x[3];
  asm volatile("" ::"v"(f));
}

// ---- fills -----------------------------------------------------------------
AMMON_DEV uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Counter-based N(mean, std): element 2c and 2c+1 are the Box-Muller pair of
// splitmix64(key ^ c * K).  Used for synthetic weights and KV contents.
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_fill_normal(ammon_k_fill p) {
#pragma clang fp contract(off)
  const uint64_t key = splitmix64(p.seed ^ splitmix64(p.stream + 0x632BE59BD9B4E019ull));
  const double two_pi = 6.283185307179586476925286766559;
  const uint64_t pairs = (p.count + 1) / 2;
  for (uint64_t c = (uint64_t)blockIdx.x * AMMON_WG + threadIdx.x; c < pairs;
       c += (uint64_t)gridDim.x * AMMON_WG) {
    const uint64_t bits = splitmix64(key ^ (c * 0xD1B54A32D192ED03ull));
    const double u1 = ((double)(bits >> 32) + 0.5) * (1.0 / 4294967296.0);
    const double u2 = ((double)(bits & 0xffffffffull) + 0.5) * (1.0 / 4294967296.0);
    const double r = sqrt(-2.0 * log(u1));
    double sn, cn;
    sincos(two_pi * u2, &sn, &cn);
    const float z0 = (float)((double)p.mean + (double)p.std * (r * cn));
    const float z1 = (float)((double)p.mean + (double)p.std * (r * sn));
    store_elem(p.dst, p.dtype, 2 * c, z0);
    if (2 * c + 1 < p.count) store_elem(p.dst, p.dtype, 2 * c + 1, z1);
  }
}

// Constant fill with a raw bit pattern (32-bit for f32, 16-bit for bf16).
// Used instead of hipMemsetAsync so the launch can sit inside a graph.
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_fill_const(ammon_k_fill p) {
  for (uint64_t i = (uint64_t)blockIdx.x * AMMON_WG + threadIdx.x; i < p.count;
       i += (uint64_t)gridDim.x * AMMON_WG) {
    if (p.dtype == AMMON_K_BF16)
      ((uint16_t *)p.dst)[i] = (uint16_t)p.bits;
    else
      ((uint32_t *)p.dst)[i] = p.bits;
  }
}
