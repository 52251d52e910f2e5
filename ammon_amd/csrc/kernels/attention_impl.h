// attention_impl.h -- split-K decode attention with GQA head sharing and a
// log-sum-exp merge (reference flash-decoding pair, src/kernels.rs:228-410),
// as workgroup-level units shared by the standalone kernels (attention.hip)
// and the persistent decode-token kernel (token.hip).
//
// Pass 1, one workgroup per (split s, kv head g): positions
// [s*S, s*S + S) clipped to t <= pos, for all G = q_heads / kv_heads query
// heads of that kv head.  Each K and V byte is loaded once from HBM into
// registers and used for all G heads (the reference re-reads it per q head).
// A lane owns CH consecutive dims of one position (16-byte loads for bf16
// head 128), so a wave covers 64 / P2 positions per pass over the head-major
// cache [kv_heads, seq, head].  Each group of lanes keeps an online softmax
// over the positions it sees; the groups are merged once at the end (LDS).
// Writes partial[h, s, :] = (sum_t e^{score_t - m} V_t, m, l) with
// the reference's layout [q_heads, splits, head + 2].  Splits that start past
// pos write nothing.
//
// Pass 2, one workgroup per (q head, 8- or 32-dim slice): M = max m_s over live splits,
// out = sum_s acc_s e^{m_s - M} / sum_s l_s e^{m_s - M}.
//
// The reference uses fixed 8-position splits (src/kernels.rs:228-229); here
// the split length is a launch parameter chosen to fill the device.
#pragma once

#include "device_common.h"

#define ATT_ROUNDS 4         // position rounds per chunk held in registers
#define ATT_MAX_SPLITS 4096
#define ATT_MAX_HEAD 128

// Sum over aligned groups of `width` lanes (a power of two <= 64): DPP
// inside 16-lane rows, shuffles across rows.
AMMON_DEV float group_sum(float v, uint32_t width) {
  v = group_sum16(v, width < 16 ? width : 16);
  for (uint32_t off = 16; off < width; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// A decode with a single split needs no merge pass: the merge of one split
// is out = acc * e^0 / (l * e^0) = acc / l exactly (the combine's fmaf(x, 1,
// 0) and +0 leave x unchanged), so pass 1 writes out itself when the launch
// asks for it (single_out).
AMMON_DEV bool direct_out(const ammon_k_attention &p) {
  return p.single_out && p.splits == 1 && p.out != nullptr;
}

// ... and for a position out of range (no unit runs), the merge's NaN output
// for kv head g's query heads.
AMMON_DEV void direct_out_nan(const ammon_k_attention &p, uint32_t g) {
  if (!direct_out(p)) return;
  const uint32_t gq = p.q_heads / p.kv_heads;
  for (uint32_t i = threadIdx.x; i < gq * p.head; i += AMMON_WG)
    st_out(p.out + (size_t)g * gq * p.head + i, __uint_as_float(0x7fc00000u));
}

// One workgroup = one (split, kv head).  The split's positions are processed
// in chunks of ATT_ROUNDS rounds; a round is 4 waves x (64 / P2) positions,
// P2 lanes per position (the power of two >= head / CH), so each group of P2
// lanes -- a "slot" -- sees one position per round.  Chunks are
// double-buffered in registers: the next chunk's K and V loads are in flight
// while the current one is processed.  After the q.k reduction every lane of
// a slot holds its position's score (the reference's dot / sqrt(head)), so
// each slot runs its own online softmax (running max, exp-sum and V
// accumulator per query head) with no LDS traffic and no barrier inside the
// split.  At the end the slots' states are merged through LDS: M = max of
// the slot maxima, acc = sum_s acc_s e^{m_s - M}, l = sum_s l_s e^{m_s - M}.
// HEAD > 0 fixes the head width at compile time (then the lane layout and
// the DPP reduction steps are constants); EXACT_G means q_heads / kv_heads
// equals GMAX.  The generic instantiations (HEAD 0) read both at run time.
template <int W> AMMON_DEV float group_sum_c(float v) {
  static_assert(W >= 2 && W <= 64 && (W & (W - 1)) == 0, "power of two");
  v += dpp_get<AMMON_DPP_XOR1>(v);
  if (W >= 4) v += dpp_get<AMMON_DPP_XOR2>(v);
  if (W >= 8) v += dpp_get<AMMON_DPP_HALF_MIRROR>(v);
  if (W >= 16) v += dpp_get<AMMON_DPP_MIRROR>(v);
  if (W >= 32) v += __shfl_xor(v, 16, 64);
  if (W >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

constexpr uint32_t ceil_pow2(uint32_t v) {
  uint32_t p = 2;
  while (p < v) p <<= 1;
  return p;
}

// LDS floats one partial unit needs: the per-lane accumulators of the final
// cross-slot merge (one padded row of GMAX * CH floats per lane) and the
// slots' (m, l) per head.
constexpr uint32_t att_lds_floats(int GMAX, int CH) {
  return AMMON_WG * (GMAX * CH + 1) + 2 * (AMMON_WG / 2) * GMAX;
}

// Unit (split, g) of pass 1, in two steps: begin() requests q and the K and
// V of the split's first two chunks; run() scores, accumulates, merges the
// slots and writes the partial (lds holds att_lds_floats(GMAX, CH) floats).
// begin() returns false for a dead split (start past the position) or an
// out-of-range position, which write nothing; the result is uniform per
// workgroup.
template <typename KV, int CH, int GMAX, int HEAD, bool EXACT_G>
struct AttnPartial {
  static constexpr int R = ATT_ROUNDS;
  static constexpr int QCH = CH >= 4 ? 4 : CH;
  static constexpr uint32_t P2C = HEAD > 0 ? ceil_pow2(HEAD / CH) : 0;
  using C = Chunk<KV, CH>;
  using QC = Chunk<float, QCH>;
  using VT = typename C::V;

  uint32_t split, g, pos, t0, n, G, head, lg_p2, P2, lg_pw, PW, lane, wave, sub, slot, round,
      chunk;
  bool active;
  __amdgpu_buffer_rsrc_t kres, vres;
  float qr[GMAX][CH];
  VT kA[R], vA[R], kB[R], vB[R];

  AMMON_DEV uint32_t off_of(uint32_t t) const {
    return (t < n && active) ? (t * head + sub * CH) * (uint32_t)sizeof(KV) : AMMON_OOB;
  }
  // Positions past the split read zero without touching memory, so loads
  // are issued unconditionally and the wait counts stay exact.
  AMMON_DEV void load_chunk(uint32_t c0, VT (&kr)[R], VT (&vr)[R]) const {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t off = off_of(c0 + r * round + wave * PW + slot);
      // the row at the position may have been stored earlier in this launch
      kr[r] = C::template load_buf<AMMON_HANDOFF_CPOL>(kres, off);
      vr[r] = C::template load_buf<AMMON_HANDOFF_CPOL>(vres, off);
    }
  }

  AMMON_DEV bool begin(const ammon_k_attention &p, uint32_t split_, uint32_t g_) {
    split = split_;
    g = g_;
    pos = p.step->position + p.pos_add;
    if (pos >= p.limit) return false;
    t0 = split * p.split_len;
    if (t0 > pos) return false;  // dead split: writes nothing
    n = min(p.split_len, pos + 1 - t0);
    G = EXACT_G ? (uint32_t)GMAX : p.q_heads / p.kv_heads;
    head = HEAD > 0 ? (uint32_t)HEAD : p.head;
    const uint32_t LP = head / CH;
    lg_p2 = 1;
    while ((1u << lg_p2) < LP) ++lg_p2;
    P2 = HEAD > 0 ? P2C : (1u << lg_p2);
    if (HEAD > 0) lg_p2 = __builtin_ctz(P2C > 0 ? P2C : 2);
    lg_pw = 6 - lg_p2;
    PW = 1u << lg_pw;
    lane = threadIdx.x & 63;
    wave = threadIdx.x >> 6;
    sub = lane & (P2 - 1);
    slot = lane / P2;
    active = sub < LP;
    round = AMMON_WAVES * PW;
    chunk = R * round;
    // Buffer resources over this split's valid positions: inactive lanes and
    // positions past the split read zero through an out-of-range offset.
    const uint32_t es = (uint32_t)sizeof(KV);
    kres = make_rsrc((const KV *)p.k_cache + ((size_t)g * p.seq + t0) * head, n * head * es);
    vres = make_rsrc((const KV *)p.v_cache + ((size_t)g * p.seq + t0) * head, n * head * es);
    // q first: loads complete in order, so the first chunk then waits only
    // for q and that chunk's K/V
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
      const bool ok = (uint32_t)j < G && active;
      const float *qp = p.q + (size_t)(g * G + (ok ? j : 0)) * head + sub * CH;
#pragma unroll
      for (int c = 0; c < CH; c += QCH) {
        float f[QCH];
        QC::widen(ok ? QC::load_in(qp + c) : QC::zero(), f);
#pragma unroll
        for (int e = 0; e < QCH; ++e) qr[j][c + e] = f[e];
      }
    }
    load_chunk(0, kA, vA);
    load_chunk(chunk, kB, vB);
    return true;
  }

  AMMON_DEV void run(const ammon_k_attention &p, float *lds) {
    float(*s_red)[GMAX * CH + 1] = (float(*)[GMAX * CH + 1])lds;
    float(*s_m)[GMAX] = (float(*)[GMAX])(lds + AMMON_WG * (GMAX * CH + 1));
    float(*s_l)[GMAX] = (float(*)[GMAX])(lds + AMMON_WG * (GMAX * CH + 1) + (AMMON_WG / 2) * GMAX);
    // Softmax in base 2: e^(s - m) = 2^(s log2e - m log2e), one v_exp_f32
    // per weight (results below 2^-126 flush to zero, far below fp32
    // resolution of the sums).  The running maxima are kept in base-2 units
    // and converted back (x ln 2) when the partial is written.
    const float scale2 = 1.4426950408889634f / sqrtf((float)head);

    float acc[GMAX][CH];
    float m_run[GMAX], l_run[GMAX];
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
      m_run[j] = -INFINITY;
      l_run[j] = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c) acc[j][c] = 0.f;
    }

    auto compute_chunk = [&](uint32_t c0, VT (&kr)[R], VT (&vr)[R]) {
      // scores of this slot's R positions (-inf past the split)
      float sc[R][GMAX];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t t = c0 + r * round + wave * PW + slot;
        float kf[CH];
        C::widen(kr[r], kf);
#pragma unroll
        for (int j = 0; j < GMAX; ++j) {
          float d = 0.f;
#pragma unroll
          for (int c = 0; c < CH; ++c) d += qr[j][c] * kf[c];
          if constexpr (HEAD > 0)
            d = group_sum_c<P2C>(d);
          else
            d = group_sum(d, P2);
          // score (reference src/kernels.rs:298: dot / sqrt(head)) in base-2
          // units: d * log2(e) / sqrt(head)
          sc[r][j] = t < n ? d * scale2 : -INFINITY;
        }
      }
      // online softmax update of the slot's state
#pragma unroll
      for (int j = 0; j < GMAX; ++j) {
        if (!EXACT_G && (uint32_t)j >= G) continue;
        float mc = m_run[j];
#pragma unroll
        for (int r = 0; r < R; ++r) mc = fmaxf(mc, sc[r][j]);
        if (mc == -INFINITY) continue;  // nothing seen yet
        const float a = __builtin_amdgcn_exp2f(m_run[j] - mc);
        float l = l_run[j] * a;
#pragma unroll
        for (int c = 0; c < CH; ++c) acc[j][c] *= a;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float e = __builtin_amdgcn_exp2f(sc[r][j] - mc);  // 0 for -inf scores
          l += e;
          float vf[CH];
          C::widen(vr[r], vf);
#pragma unroll
          for (int c = 0; c < CH; ++c) acc[j][c] += e * vf[c];
        }
        l_run[j] = l;
        m_run[j] = mc;
      }
    };

    // Steady state: both buffers are refilled two chunks ahead.  The last
    // (at most three) chunks run without prefetches: a load past the split
    // would return only zeros, but the merge below reuses its registers and
    // would first wait for it to come back.
    uint32_t c0 = 0;
    for (; c0 + 3 * chunk < n; c0 += 2 * chunk) {
      compute_chunk(c0, kA, vA);
      load_chunk(c0 + 2 * chunk, kA, vA);
      compute_chunk(c0 + chunk, kB, vB);
      load_chunk(c0 + 3 * chunk, kB, vB);
    }
    if (c0 < n) {
      compute_chunk(c0, kA, vA);
      if (c0 + 2 * chunk < n) load_chunk(c0 + 2 * chunk, kA, vA);
      if (c0 + chunk < n) {
        compute_chunk(c0 + chunk, kB, vB);
        if (c0 + 2 * chunk < n) compute_chunk(c0 + 2 * chunk, kA, vA);
      }
    }

    // merge the 4 * PW slots of the workgroup through LDS
#pragma unroll
    for (int j = 0; j < GMAX; ++j)
#pragma unroll
      for (int c = 0; c < CH; ++c) s_red[threadIdx.x][j * CH + c] = acc[j][c];
    const uint32_t slots = AMMON_WAVES * PW;
    const uint32_t slot_id = wave * PW + slot;
    if (sub == 0) {
#pragma unroll
      for (int j = 0; j < GMAX; ++j) {
        s_m[slot_id][j] = m_run[j];
        s_l[slot_id][j] = l_run[j];
      }
    }
    __syncthreads();
    const uint32_t slot_w = head + 2;
    for (uint32_t idx = threadIdx.x; idx < G * head; idx += AMMON_WG) {
      const uint32_t j = idx / head, d = idx - j * head;
      const uint32_t sb = d / CH, c = d % CH;  // lane sub and element (CH is a constant)
      float M = -INFINITY;
      for (uint32_t s = 0; s < slots; ++s) M = fmaxf(M, s_m[s][j]);
      float total = 0.f, L = 0.f;
      for (uint32_t s = 0; s < slots; ++s) {
        const float ms = s_m[s][j];
        const float w = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - M);
        // thread of (wave s / PW, slot s % PW, sub sb)
        const uint32_t t = ((s >> lg_pw) << 6) + ((s & (PW - 1)) << lg_p2) + sb;
        total += s_red[t][j * CH + c] * w;
        L += s_l[s][j] * w;
      }
      if (direct_out(p)) {  // the only split: the merge's result, total / L
        st_out(p.out + (size_t)(g * G + j) * head + d, total / L);
        continue;
      }
      float *o = p.partial + ((size_t)(g * G + j) * p.splits + split) * slot_w;
      st_out(o + d, total);
      if (d == 0) {
        st_out(o + head, M * 0.6931471805599453f);  // back to natural-log units
        st_out(o + head + 1, L);
      }
    }
  }
};

// Pass 1 on matrix cores, for bf16 K/V and head 128 (Llama-style shapes):
// the same unit as AttnPartial with q.k on v_mfma_f32_16x16x32_bf16.
//
// Chunks of 64 positions, NBUF-buffered in registers (the next NBUF - 1
// chunks' K and V are in flight while one is processed, so compute on the
// first chunks of a split overlaps the arrival of the rest; a split of
// NBUF * 64 positions is requested in one go).  Wave w scores positions
// [16w, 16w + 16) of a chunk as one 16x16 tile S^T[t][h] = sum_d K[t][d]
// q[h][d] (A = K rows as stored, B = q^T, heads as the 16 columns; heads
// >= G are zero).  q is split into bf16 hi + lo parts (two MFMAs per 32
// dims), so the products keep ~16 mantissa bits of q and accumulate in
// fp32.  The chunk's scores go to LDS; one wave per head takes the chunk
// max, rescales the running state and turns scores into weights 2^(s - m)
// (one exponential per position and head); then every lane accumulates 8
// dims of V for its 4 positions of the chunk with the weights read from
// LDS.  All slots share the workgroup's running max, so the final merge
// across lanes and waves is a plain sum.  The partial format is the VALU
// unit's: (sum_t e^{s_t - m} V_t, m, l).
template <int GMAX, int NBUF = 2>
struct AttnPartialMfma {
  static_assert(GMAX >= 1 && GMAX <= 16, "q heads per kv head");
  static_assert(NBUF >= 1 && NBUF <= 4, "chunk buffers");
  static constexpr uint32_t HEAD = 128, CHUNK = 64;
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef float f32x8 __attribute__((ext_vector_type(8)));

  uint32_t split, g, pos, t0, n, lane, wave;
  __amdgpu_buffer_rsrc_t kres, vres;
  // q^T (B operand): lane l holds head l % 16, dims 32(l/16) + 8kk..+7 as fp32
  float4 qraw[4][2];
  // per chunk buffer: K row (l % 16) of the wave's tile, dims 32(l/16) + 8kk;
  // V rows of the lane's 4 positions 16w + 4k + l/16, dims 8(l % 16)..+7
  u32x4 kb[NBUF][4], vb[NBUF][4];

  // Positions past the split read zero without touching memory, so loads
  // are issued unconditionally and the wait counts stay exact.
  // Rows at or past `rows` (of the split) read as zero.
  AMMON_DEV void load_chunk(uint32_t c0, u32x4 (&kr)[4], u32x4 (&vr)[4], uint32_t rows) const {
    const uint32_t tk = c0 + 16 * wave + (lane & 15);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t off = tk < rows ? (tk * HEAD + 32 * (lane >> 4) + 8 * kk) * 2 : AMMON_OOB;
      kr[kk] = __builtin_amdgcn_raw_buffer_load_b128(kres, off, 0, AMMON_HANDOFF_CPOL);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t tv = c0 + 16 * wave + 4 * k + (lane >> 4);
      const uint32_t off = tv < rows ? (tv * HEAD + 8 * (lane & 15)) * 2 : AMMON_OOB;
      vr[k] = __builtin_amdgcn_raw_buffer_load_b128(vres, off, 0, AMMON_HANDOFF_CPOL);
    }
  }
  AMMON_DEV void load_chunk(uint32_t c0, u32x4 (&kr)[4], u32x4 (&vr)[4]) const {
    load_chunk(c0, kr, vr, n);
  }

  // The unit's split and cache resources; false for a dead split (start past
  // the position) or an out-of-range position, which write nothing.
  AMMON_DEV bool setup(const ammon_k_attention &p, uint32_t split_, uint32_t g_) {
    split = split_;
    g = g_;
    pos = p.step->position + p.pos_add;
    if (pos >= p.limit) return false;
    t0 = split * p.split_len;
    if (t0 > pos) return false;  // dead split: writes nothing
    n = min(p.split_len, pos + 1 - t0);
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kres = make_rsrc((const uint16_t *)p.k_cache + ((size_t)g * p.seq + t0) * HEAD, n * HEAD * 2);
    vres = make_rsrc((const uint16_t *)p.v_cache + ((size_t)g * p.seq + t0) * HEAD, n * HEAD * 2);
    return true;
  }

  // Lanes of score columns h >= GMAX load head 0's q: those columns are
  // never stored, and unconditional loads leave no branch whose join would
  // wait for the first loads before the K/V requests go out.
  AMMON_DEV void load_q(const ammon_k_attention &p) {
    const uint32_t h = lane & 15;
    const float *qp = p.q + (size_t)(g * GMAX + (h < GMAX ? h : 0)) * HEAD + 32 * (lane >> 4);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      qraw[kk][0] = ld_in4(qp + 8 * kk);
      qraw[kk][1] = ld_in4(qp + 8 * kk + 4);
    }
  }

  AMMON_DEV bool begin(const ammon_k_attention &p, uint32_t split_, uint32_t g_) {
    if (!setup(p, split_, g_)) return false;
    // q first: loads complete in order, so the first chunk's MFMAs then wait
    // only for q and that chunk, not for the later chunk's K/V as well
    load_q(p);
#pragma unroll
    for (int b = 0; b < NBUF; ++b) load_chunk(b * CHUNK, kb[b], vb[b]);
    // keep run()'s q conversion below the requests: scheduled among them,
    // it waited for q before the later K/V requests went out
    __builtin_amdgcn_sched_barrier(0);
    return true;
  }

  // begin() in two steps, for a caller whose q and newest K/V row are stored
  // by other workgroups of the same launch: prefetch() -- before they are --
  // requests the first NBUF chunks with every row except the position's
  // (which may not exist yet); finish() -- once they are -- requests q and,
  // if the position's row lies in a prefetched chunk, that chunk again in
  // full.  run() then sees exactly what begin() would have loaded.
  AMMON_DEV bool prefetch(const ammon_k_attention &p, uint32_t split_, uint32_t g_) {
    if (!setup(p, split_, g_)) return false;
    const uint32_t before = t0 + n - 1 == pos ? n - 1 : n;  // rows older than the position
#pragma unroll
    for (int b = 0; b < NBUF; ++b) load_chunk(b * CHUNK, kb[b], vb[b], before);
    return true;
  }
  AMMON_DEV void finish(const ammon_k_attention &p) {
    load_q(p);
    if (t0 + n - 1 == pos) {
      const uint32_t cb = (pos - t0) / CHUNK;  // chunk of the position's row
#pragma unroll
      for (int b = 0; b < NBUF; ++b)
        if ((uint32_t)b == cb) load_chunk(b * CHUNK, kb[b], vb[b]);
    }
  }

  // lds: att_lds_floats(GMAX, 8) floats.
  AMMON_DEV void run(const ammon_k_attention &p, float *lds) {
    float(*s_red)[GMAX * 8 + 1] = (float(*)[GMAX * 8 + 1])lds;      // final merge
    float *s_s = lds + AMMON_WG * (GMAX * 8 + 1);                     // [CHUNK][GMAX]
    float *s_scale = s_s + CHUNK * GMAX;                              // [GMAX]
    float *s_ml = s_scale + GMAX;                                     // [2][GMAX]
    const float scale2 = 1.4426950408889634f / sqrtf((float)HEAD);  // log2(e)/sqrt(head)

    // q^T as bf16 hi + lo B operands
    bf16x8 qhi[4], qlo[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const float4 a = qraw[kk][0], b = qraw[kk][1];
      const f32x8 f = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      // v_cvt_pk_bf16_f32 (round to nearest even); hi + lo = q to ~16 bits
      qhi[kk] = __builtin_convertvector(f, bf16x8);
      qlo[kk] = __builtin_convertvector(f - __builtin_convertvector(qhi[kk], f32x8), bf16x8);
    }

    float acc[GMAX][8];
#pragma unroll
    for (int j = 0; j < GMAX; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    // running max / sum of the heads this wave owns: h = wave + 4i
    constexpr int HW = (GMAX + AMMON_WAVES - 1) / AMMON_WAVES;
    float m_run[HW], l_run[HW];
#pragma unroll
    for (int i = 0; i < HW; ++i) {
      m_run[i] = -INFINITY;
      l_run[i] = 0.f;
    }

    auto process = [&](uint32_t c0, u32x4 (&kr)[4], u32x4 (&vr)[4]) {
      // scores of this wave's 16-position tile
      f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8 a = __builtin_bit_cast(bf16x8, kr[kk]);
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qhi[kk], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qlo[kk], st, 0, 0, 0);
      }
      if (c0 > 0) __syncthreads();  // previous chunk's weights consumed
      // D layout: lane l holds S^T[4(l/16) + r][l % 16] of the tile
      if ((lane & 15) < GMAX) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t pl = 16 * wave + 4 * (lane >> 4) + r;  // position in chunk
          // score (reference src/kernels.rs:298: dot / sqrt(head)), base-2 units
          s_s[pl * GMAX + (lane & 15)] = c0 + pl < n ? st[r] * scale2 : -INFINITY;
        }
      }
      __syncthreads();
      // one wave per head: chunk max, running rescale, weights
#pragma unroll
      for (int i = 0; i < HW; ++i) {
        const uint32_t h = wave + AMMON_WAVES * i;
        if (h >= GMAX) continue;  // wave-uniform
        const float a0 = s_s[lane * GMAX + h];
        const float mc = wave_max(a0);
        const float m_new = fmaxf(m_run[i], mc);
        // m_new is finite: every chunk holds at least one valid position
        const float sc = __builtin_amdgcn_exp2f(m_run[i] - m_new);  // 0 on the first chunk
        const float e0 = __builtin_amdgcn_exp2f(a0 - m_new);
        s_s[lane * GMAX + h] = e0;
        const float ls = wave_sum(e0);
        l_run[i] = l_run[i] * sc + ls;
        m_run[i] = m_new;
        if (lane == 0) s_scale[h] = sc;
      }
      __syncthreads();
      // V: lane l accumulates dims 8(l % 16)..+7 of positions 16w + 4k + l/16
#pragma unroll
      for (int j = 0; j < GMAX; ++j) {
        const float sc = s_scale[j];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] *= sc;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t pl = 16 * wave + 4 * k + (lane >> 4);
        float vf[8];
        Chunk<uint16_t, 8>::widen(vr[k], vf);
#pragma unroll
        for (int j = 0; j < GMAX; ++j) {
          const float w = s_s[pl * GMAX + j];
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[j][e] += w * vf[e];
        }
      }
    };

    // Buffers keep fixed roles (unrolled); each is refilled NBUF chunks
    // ahead.  Steady state while every refill lies inside the split; the
    // last 2 NBUF - 1 chunks at most run in two passes, the second without
    // prefetches: a load past the split returns only zeros, but the merge
    // below reuses its registers and would first wait for it to come back.
    const uint32_t nch = (n + CHUNK - 1) / CHUNK;
    uint32_t c = 0;  // chunk index
    for (; c + 2 * NBUF <= nch; c += NBUF) {
#pragma unroll
      for (int b = 0; b < NBUF; ++b) {
        process((c + b) * CHUNK, kb[b], vb[b]);
        load_chunk((c + b + NBUF) * CHUNK, kb[b], vb[b]);
      }
    }
#pragma unroll
    for (int b = 0; b < NBUF; ++b) {
      if (c + b < nch) {
        process((c + b) * CHUNK, kb[b], vb[b]);
        if (c + b + NBUF < nch) load_chunk((c + b + NBUF) * CHUNK, kb[b], vb[b]);
      }
    }
#pragma unroll
    for (int b = 0; b < NBUF; ++b)
      if (c + NBUF + b < nch) process((c + NBUF + b) * CHUNK, kb[b], vb[b]);

    // merge: plain sums over the 16 position slots (4 per wave) of the group
    __syncthreads();
#pragma unroll
    for (int j = 0; j < GMAX; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_red[threadIdx.x][j * 8 + e] = acc[j][e];
#pragma unroll
    for (int i = 0; i < HW; ++i) {
      const uint32_t h = wave + AMMON_WAVES * i;
      if (h < GMAX && lane == 0) {
        s_ml[h] = m_run[i];
        s_ml[GMAX + h] = l_run[i];
      }
    }
    __syncthreads();
    const uint32_t slot_w = HEAD + 2;
    for (uint32_t idx = threadIdx.x; idx < GMAX * HEAD; idx += AMMON_WG) {
      const uint32_t j = idx / HEAD, d = idx % HEAD;
      const uint32_t sb = d / 8, e = d % 8;
      float total = 0.f;
#pragma unroll
      for (uint32_t s = 0; s < 16; ++s) total += s_red[(s >> 2) * 64 + (s & 3) * 16 + sb][j * 8 + e];
      if (direct_out(p)) {  // the only split: the merge's result, total / l
        st_out(p.out + (size_t)(g * GMAX + j) * HEAD + d, total / s_ml[GMAX + j]);
        continue;
      }
      float *o = p.partial + ((size_t)(g * GMAX + j) * p.splits + split) * slot_w;
      st_out(o + d, total);
      if (d == 0) {
        st_out(o + HEAD, s_ml[j] * 0.6931471805599453f);  // back to natural-log units
        st_out(o + HEAD + 1, s_ml[GMAX + j]);
      }
    }
  }
};

// Query token z of a multi-token (prefill) grid: its q, partial and output
// slices and its position offset (identity for z = 0).
AMMON_DEV ammon_k_attention attention_token(const ammon_k_attention &p, uint32_t z) {
  ammon_k_attention t = p;
  const size_t qn = (size_t)p.q_heads * p.head;
  t.q = p.q + z * qn;
  t.partial = p.partial + (size_t)z * p.q_heads * p.splits * (p.head + 2);
  if (p.out) t.out = p.out + z * qn;
  t.pos_add = p.pos_add + z;
  return t;
}

// Pass 2: the log-sum-exp merge.  Its arithmetic, per output dim d:
//   M     = max of the live splits' m_s;  w_s = e^{m_s - M}
//   a_j   = fma chain over s = j, j + 64, j + 128, ... < live of (o_s[d], w_s),
//   l_j   = the same chain of (l_s, w_s), both from 0, for split lanes j < 64
//   total = ((0 + a_0) + a_1) + ... + a_63,  L likewise;  out[d] = total / L
// (lanes without a live split add +0).  Two layouts compute exactly this:
//
// Units (q head, head / 32 or head / 8 dim slices) of a workgroup: lane
// (split lane sl, dim quarter) covers splits sl, sl + 64, ...; with up to
// COMB_ROUNDS * 64 live splits it loads each split's max, sum and its dims in
// one round trip and keeps them in registers while the workgroup max M
// forms (more splits take a second pass over the buffer); the split lanes
// are summed through LDS.  Every workgroup of a head computes the same M.
// Used where the split count is large (decode at long context).
//
// attention_combine_wave: one wave per q head, lane l owning dims 2l and
// 2l + 1, walking the split lanes in order.  Used for many query tokens with
// few live splits each (prefill), where a workgroup per 32 dims would be
// mostly idle lanes.
#define COMB_SPLIT_LANES 64
#define COMB_ROUNDS 4
// LDS floats of one combine unit over SLICE dims: per split lane the slice
// + 1 pad, its sum, and the block reduction slots.
#define COMB_LDS_FLOATS_W(SLICE) (COMB_SPLIT_LANES * ((SLICE) + 1) + COMB_SPLIT_LANES + AMMON_WAVES)
#define COMB_LDS_FLOATS COMB_LDS_FLOATS_W(32)

// Unit (q head h, SLICE-dim slice) of pass 2 (SLICE 32 or 8: each lane
// owns SLICE / 4 dims of one split lane; the per-dim arithmetic does not
// depend on SLICE); lds holds COMB_LDS_FLOATS_W(SLICE) floats.
template <int SLICE = 32>
AMMON_DEV void attention_combine_unit(const ammon_k_attention &p, uint32_t h, uint32_t slice,
                                      float *lds) {
  static_assert(SLICE == 32 || SLICE == 8, "slice width");
  constexpr int DQ = SLICE / 4;  // dims per lane
  float(*s_acc)[SLICE + 1] = (float(*)[SLICE + 1])lds;
  float *s_l = lds + COMB_SPLIT_LANES * (SLICE + 1);
  float *red = s_l + COMB_SPLIT_LANES;
  const uint32_t head = p.head, slot = head + 2;
  const uint32_t d0 = slice * SLICE;
  float *out = p.out + (size_t)h * head;
  const float *base = p.partial + (size_t)h * p.splits * slot;
  const uint32_t sl = threadIdx.x >> 2;         // split lane, 0..63
  const uint32_t dq = (threadIdx.x & 3) * DQ;  // DQ dims of the slice
  // With at most COMB_ROUNDS * 64 splits in the buffer, every split's max,
  // sum and dims are requested before the position is known (entries of
  // dead splits are loaded and then ignored), so the position load and the
  // partials take one round trip instead of two.
  const bool one_trip = p.splits <= COMB_ROUNDS * COMB_SPLIT_LANES;
  float mv[COMB_ROUNDS], lv[COMB_ROUNDS], dv[COMB_ROUNDS][DQ];
  if (one_trip) {
#pragma unroll
    for (int r = 0; r < COMB_ROUNDS; ++r) {
      const uint32_t s = sl + r * COMB_SPLIT_LANES;
      const float *row = base + (size_t)(s < p.splits ? s : 0) * slot;
      mv[r] = ld_in(row + head);
      lv[r] = ld_in(row + head + 1);
#pragma unroll
      for (int k = 0; k < DQ; ++k) {
        const uint32_t d = d0 + dq + k;
        dv[r][k] = d < head ? ld_in(row + d) : 0.f;
      }
    }
  }
  const uint32_t pos = p.step->position + p.pos_add;
  if (pos >= p.limit) {
    if (threadIdx.x < SLICE && d0 + threadIdx.x < head)
      st_out(out + d0 + threadIdx.x, __uint_as_float(0x7fc00000u));
    return;
  }
  const uint32_t live = min(pos / p.split_len + 1, p.splits);

  float a[DQ];
#pragma unroll
  for (int k = 0; k < DQ; ++k) a[k] = 0.f;
  float l = 0.f;
  if (one_trip) {
#pragma unroll
    for (int r = 0; r < COMB_ROUNDS; ++r)
      if (sl + r * COMB_SPLIT_LANES >= live) mv[r] = -INFINITY;
    float m = mv[0];
#pragma unroll
    for (int r = 1; r < COMB_ROUNDS; ++r) m = fmaxf(m, mv[r]);
    const float M = block_max(m, red);
#pragma unroll
    for (int r = 0; r < COMB_ROUNDS; ++r) {
      if (sl + r * COMB_SPLIT_LANES >= live) break;
      const float w = expf(mv[r] - M);
      if ((threadIdx.x & 3) == 0) l = fmaf(lv[r], w, l);
#pragma unroll
      for (int k = 0; k < DQ; ++k) a[k] = fmaf(dv[r][k], w, a[k]);
    }
  } else {
    float m = -INFINITY;
    for (uint32_t s = threadIdx.x; s < live; s += AMMON_WG)
      m = fmaxf(m, ld_in(base + (size_t)s * slot + head));
    const float M = block_max(m, red);
    for (uint32_t s = sl; s < live; s += COMB_SPLIT_LANES) {
      const float *row = base + (size_t)s * slot;
      const float w = expf(ld_in(row + head) - M);
      if ((threadIdx.x & 3) == 0) l = fmaf(ld_in(row + head + 1), w, l);
#pragma unroll
      for (int k = 0; k < DQ; ++k) {
        const uint32_t d = d0 + dq + k;
        if (d < head) a[k] = fmaf(ld_in(row + d), w, a[k]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < DQ; ++k) s_acc[sl][dq + k] = a[k];
  if ((threadIdx.x & 3) == 0) s_l[sl] = l;
  __syncthreads();
  if (threadIdx.x < SLICE) {
    float total = 0.f, L = 0.f;
    for (uint32_t s = 0; s < COMB_SPLIT_LANES; ++s) {
      total += s_acc[s][threadIdx.x];
      L += s_l[s];
    }
    const uint32_t d = d0 + threadIdx.x;
    if (d < head) st_out(out + d, total / L);
  }
}

// The merge above for q head h by one wave (call with the whole wave).
AMMON_DEV void attention_combine_wave(const ammon_k_attention &p, uint32_t h) {
#pragma clang fp contract(off)
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t head = p.head, slot = head + 2;
  const bool mine = 2 * lane < head;
  float *out = p.out + (size_t)h * head + 2 * lane;
  const uint32_t pos = p.step->position + p.pos_add;
  if (pos >= p.limit) {
    if (mine) {
      st_out(out, __uint_as_float(0x7fc00000u));
      st_out(out + 1, __uint_as_float(0x7fc00000u));
    }
    return;
  }
  const uint32_t live = min(pos / p.split_len + 1, p.splits);
  const float *base = p.partial + (size_t)h * p.splits * slot;
  float m = -INFINITY;
  for (uint32_t s = lane; s < live; s += COMB_SPLIT_LANES) m = fmaxf(m, base[(size_t)s * slot + head]);
  const float M = wave_max(m);
  const uint32_t d = mine ? 2 * lane : 0;
  float t0 = 0.f, t1 = 0.f, L = 0.f;
  const uint32_t lanes = min(live, (uint32_t)COMB_SPLIT_LANES);
  for (uint32_t j = 0; j < lanes; ++j) {
    float a0 = 0.f, a1 = 0.f, l = 0.f;
    for (uint32_t s = j; s < live; s += COMB_SPLIT_LANES) {
      const float *row = base + (size_t)s * slot;
      const float w = expf(row[head] - M);
      l = fmaf(row[head + 1], w, l);
      a0 = fmaf(row[d], w, a0);
      a1 = fmaf(row[d + 1], w, a1);
    }
    t0 = t0 + a0;
    t1 = t1 + a1;
    L = L + l;
  }
  if (lanes < COMB_SPLIT_LANES) {  // the idle split lanes' +0
    t0 = t0 + 0.f;
    t1 = t1 + 0.f;
    L = L + 0.f;
  }
  if (mine) {
    st_out(out, t0 / L);
    st_out(out + 1, t1 / L);
  }
}
