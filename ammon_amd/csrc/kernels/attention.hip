// attention.hip -- split-K decode attention with GQA head sharing and a
// log-sum-exp merge (reference flash-decoding pair, src/kernels.rs:228-410).
//
// Pass 1, one workgroup per (split s, kv head g): positions
// [s*S, s*S + S) clipped to t <= pos, for all G = q_heads / kv_heads query
// heads of that kv head.  Each K and V byte is loaded once from HBM into
// registers and used for all G heads (the reference re-reads it per q head).
// A lane owns CH consecutive dims of one position (16-byte loads for bf16
// head 128), so a wave covers 64 / P2 positions per pass over the head-major
// cache [kv_heads, seq, head].  Scores land in LDS, the split max and
// exp-sums are wave reductions, and the V accumulation is reduced across the
// lanes of a wave (butterfly) and then across the four waves (LDS, wave
// order).  Writes partial[h, s, :] = (sum_t e^{score_t - m} V_t, m, l) with
// the reference's layout [q_heads, splits, head + 2].  Splits that start past
// pos write nothing.
//
// Pass 2, one workgroup per q head: M = max m_s over live splits,
// out = sum_s acc_s e^{m_s - M} / sum_s l_s e^{m_s - M}.
#include "device_common.h"

#define ATT_SMAX 1024      // positions per split
#define ATT_MAX_SPLITS 4096
#define ATT_MAX_HEAD 128

template <typename KV, int CH, int GMAX>
AMMON_DEV void attention_partial_body(const ammon_k_attention &p) {
  constexpr int U = 4;  // position rounds with loads in flight per lane
  __shared__ float s_p[GMAX][ATT_SMAX];
  __shared__ float s_red[AMMON_WAVES][GMAX * ATT_MAX_HEAD];
  __shared__ float s_ml[2][GMAX];

  const uint32_t split = blockIdx.x, g = blockIdx.y;
  const uint32_t pos = p.step->position;
  if (pos >= p.seq) return;
  const uint32_t t0 = split * p.split_len;
  if (t0 > pos) return;  // dead split
  const uint32_t n = min(p.split_len, pos + 1 - t0);
  const uint32_t G = p.q_heads / p.kv_heads;
  const uint32_t head = p.head;
  const uint32_t LP = head / CH;
  uint32_t P2 = 1;
  while (P2 < LP) P2 <<= 1;
  const uint32_t PW = 64 / P2;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t sub = lane & (P2 - 1), slot = lane / P2;
  const bool active = sub < LP;
  const uint32_t round = AMMON_WAVES * PW;

  float qr[GMAX][CH];
#pragma unroll
  for (int j = 0; j < GMAX; ++j)
#pragma unroll
    for (int c = 0; c < CH; ++c)
      qr[j][c] = ((uint32_t)j < G && active)
                     ? p.q[(size_t)(g * G + j) * head + sub * CH + c]
                     : 0.f;

  const KV *kb = (const KV *)p.k_cache + ((size_t)g * p.seq + t0) * head + sub * CH;
  const KV *vb = (const KV *)p.v_cache + ((size_t)g * p.seq + t0) * head + sub * CH;
  const float root = sqrtf((float)head);
  using C = Chunk<KV, CH>;

  // Scores.
  for (uint32_t base = 0; base < n; base += round * U) {
    typename C::V raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t tl = base + u * round + wave * PW + slot;
      raw[u] = (tl < n && active) ? C::load(kb + (size_t)tl * head) : C::zero();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t tl = base + u * round + wave * PW + slot;
      float kf[CH];
      C::widen(raw[u], kf);
      float d[GMAX];
#pragma unroll
      for (int j = 0; j < GMAX; ++j) {
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) s += qr[j][c] * kf[c];
        d[j] = s;
      }
      for (uint32_t off = P2 >> 1; off > 0; off >>= 1)
#pragma unroll
        for (int j = 0; j < GMAX; ++j) d[j] += __shfl_xor(d[j], off, 64);
      if (sub == 0 && tl < n)
#pragma unroll
        for (int j = 0; j < GMAX; ++j)
          if ((uint32_t)j < G) s_p[j][tl] = d[j] / root;
    }
  }
  __syncthreads();

  // Split max and exp-sum per query head.
  for (uint32_t j = wave; j < G; j += AMMON_WAVES) {
    float m = -INFINITY;
    for (uint32_t t = lane; t < n; t += 64) m = fmaxf(m, s_p[j][t]);
    m = wave_max(m);
    float l = 0.f;
    for (uint32_t t = lane; t < n; t += 64) {
      const float e = expf(s_p[j][t] - m);
      s_p[j][t] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      s_ml[0][j] = m;
      s_ml[1][j] = l;
    }
  }
  __syncthreads();

  // Probability-weighted V.
  float acc[GMAX][CH];
#pragma unroll
  for (int j = 0; j < GMAX; ++j)
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[j][c] = 0.f;
  for (uint32_t base = 0; base < n; base += round * U) {
    typename C::V raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t tl = base + u * round + wave * PW + slot;
      raw[u] = (tl < n && active) ? C::load(vb + (size_t)tl * head) : C::zero();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t tl = base + u * round + wave * PW + slot;
      if (tl < n) {
        float vf[CH];
        C::widen(raw[u], vf);
#pragma unroll
        for (int j = 0; j < GMAX; ++j) {
          const float pj = ((uint32_t)j < G) ? s_p[j][tl] : 0.f;
#pragma unroll
          for (int c = 0; c < CH; ++c) acc[j][c] += pj * vf[c];
        }
      }
    }
  }
  for (uint32_t off = P2; off < 64; off <<= 1)
#pragma unroll
    for (int j = 0; j < GMAX; ++j)
#pragma unroll
      for (int c = 0; c < CH; ++c) acc[j][c] += __shfl_xor(acc[j][c], off, 64);
  if (slot == 0 && active)
#pragma unroll
    for (int j = 0; j < GMAX; ++j)
      if ((uint32_t)j < G)
#pragma unroll
        for (int c = 0; c < CH; ++c) s_red[wave][j * head + sub * CH + c] = acc[j][c];
  __syncthreads();

  const uint32_t slot_w = head + 2;
  for (uint32_t idx = threadIdx.x; idx < G * head; idx += AMMON_WG) {
    const uint32_t j = idx / head, d = idx % head;
    float total = s_red[0][idx];
#pragma unroll
    for (int w = 1; w < AMMON_WAVES; ++w) total += s_red[w][idx];
    p.partial[((size_t)(g * G + j) * p.splits + split) * slot_w + d] = total;
  }
  if (threadIdx.x < G) {
    const uint32_t j = threadIdx.x;
    float *o = p.partial + ((size_t)(g * G + j) * p.splits + split) * slot_w;
    o[head] = s_ml[0][j];
    o[head + 1] = s_ml[1][j];
  }
}

#define ATT_PARTIAL(NAME, KV, CH, GMAX)                                          \
  extern "C" __global__ __launch_bounds__(AMMON_WG) void NAME(ammon_k_attention p) { \
    attention_partial_body<KV, CH, GMAX>(p);                                     \
  }

#define ATT_PARTIAL_G(PREFIX, KV, CH)          \
  ATT_PARTIAL(PREFIX##_g1, KV, CH, 1)          \
  ATT_PARTIAL(PREFIX##_g2, KV, CH, 2)          \
  ATT_PARTIAL(PREFIX##_g4, KV, CH, 4)          \
  ATT_PARTIAL(PREFIX##_g8, KV, CH, 8)

ATT_PARTIAL_G(ammon_attention_partial_f32_c4, float, 4)
ATT_PARTIAL_G(ammon_attention_partial_f32_c2, float, 2)
ATT_PARTIAL_G(ammon_attention_partial_f32_c1, float, 1)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c8, uint16_t, 8)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c4, uint16_t, 4)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c2, uint16_t, 2)
ATT_PARTIAL_G(ammon_attention_partial_bf16_c1, uint16_t, 1)

extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_attention_combine(ammon_k_attention p) {
  __shared__ float s_w[ATT_MAX_SPLITS];
  __shared__ float s_acc[AMMON_WG];
  __shared__ float red[AMMON_WAVES];
  const uint32_t h = blockIdx.x;
  const uint32_t head = p.head, slot = head + 2;
  float *out = p.out + (size_t)h * head;
  const uint32_t pos = p.step->position;
  if (pos >= p.seq) {
    for (uint32_t d = threadIdx.x; d < head; d += AMMON_WG) out[d] = __uint_as_float(0x7fc00000u);
    return;
  }
  const uint32_t live = pos / p.split_len + 1;
  const float *base = p.partial + (size_t)h * p.splits * slot;

  float m = -INFINITY;
  for (uint32_t s = threadIdx.x; s < live; s += AMMON_WG) m = fmaxf(m, base[(size_t)s * slot + head]);
  const float M = block_max(m, red);
  for (uint32_t s = threadIdx.x; s < live; s += AMMON_WG)
    s_w[s] = expf(base[(size_t)s * slot + head] - M);
  __syncthreads();
  float l = 0.f;
  for (uint32_t s = threadIdx.x; s < live; s += AMMON_WG) l += base[(size_t)s * slot + head + 1] * s_w[s];
  const float L = block_sum(l, red);

  const uint32_t ways = AMMON_WG / head;
  const uint32_t way = threadIdx.x / head, d = threadIdx.x % head;
  float acc = 0.f;
  if (way < ways)
    for (uint32_t s = way; s < live; s += ways) acc += base[(size_t)s * slot + d] * s_w[s];
  s_acc[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < head) {
    float total = s_acc[threadIdx.x];
    for (uint32_t w = 1; w < ways; ++w) total += s_acc[w * head + threadIdx.x];
    out[threadIdx.x] = total / L;
  }
}
