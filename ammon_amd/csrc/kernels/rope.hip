// rope.hip -- RoPE and KV-cache stores on the head-major cache.
//
// The cache is laid out per layer as [kv_heads, seq, head]: element d of kv
// head g at position t lives at (g * seq + t) * head + d, so one head's
// positions are contiguous head-sized rows (the attention kernels stream
// them).  The reference layout is position-major [seq, kv_heads, head]
// (reference src/modules.rs:37-71); only the address changes, not the values.
//
// cos/sin come from a host-built table [seq, head/2, 2] computed with the
// reference's fp32 formula (reference src/kernels.rs:195-199), so the
// rotation below is plain fp32 multiply/subtract.  Contraction is off in
// these functions: each product rounds before the add, as the CPU restatement
// does, which makes the stored K bit-exact given the same projection.
#include "device_common.h"

// One lane per pair i = 2p of the query width (reference src/kernels.rs:174-210):
// rotate q in place; pairs with i < kv_dim also write rotated k_proj into
// K[pos].  With k_proj == NULL the K row at pos is rotated in place instead
// (the reference's test-only `rope`, src/kernels.rs:130-172).
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_rope(ammon_k_rope p) {
#pragma clang fp contract(off)
  const uint32_t i = 2u * (blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= p.q_numel) return;
  const uint32_t pos = p.step->position;
  if (pos >= p.seq) return;  // out-of-range position: no access past the cache
  const uint32_t hd = i % p.head;
  const float *cs = p.table + ((size_t)pos * (p.head / 2) + hd / 2) * 2;
  const float fcr = cs[0], fci = cs[1];
  const float q0 = p.q[i], q1 = p.q[i + 1];
  p.q[i] = q0 * fcr - q1 * fci;
  p.q[i + 1] = q0 * fci + q1 * fcr;
  if (i < p.kv_dim) {
    const uint32_t g = i / p.head;
    const size_t dst = ((size_t)g * p.seq + pos) * p.head + hd;
    float k0, k1;
    if (p.k_proj) {
      k0 = p.k_proj[i];
      k1 = p.k_proj[i + 1];
    } else {
      k0 = load_elem(p.k_cache, p.kv_dtype, dst);
      k1 = load_elem(p.k_cache, p.kv_dtype, dst + 1);
    }
    store_elem(p.k_cache, p.kv_dtype, dst, k0 * fcr - k1 * fci);
    store_elem(p.k_cache, p.kv_dtype, dst + 1, k0 * fci + k1 * fcr);
  }
}

// cache[pos] = src (reference src/kernels.rs:212-226), one lane per element.
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_cache_store(ammon_k_cache_store p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.kv_dim) return;
  const uint32_t pos = p.step->position;
  if (pos >= p.seq) return;
  const uint32_t g = i / p.head, d = i % p.head;
  store_elem(p.cache, p.dtype, ((size_t)g * p.seq + pos) * p.head + d, p.src[i]);
}
