// attention_impl.h -- split-K decode attention with GQA head sharing and a
// log-sum-exp merge (reference flash-decoding pair, src/kernels.rs:228-410),
// as workgroup-level units run by the kernels of attention.hip.
//
// Pass 1, one workgroup per (split s, kv head g): positions
// [s*S, s*S + S) clipped to t <= pos, for all G = q_heads / kv_heads query
// heads of that kv head.  Each K and V byte is loaded once from HBM and used
// for all G heads (the reference re-reads it per q head).  Two units run it:
// AttnPartial (VALU, K/V in registers; fp32 caches and heads other than
// 128), where a lane owns CH consecutive dims of one position and each group
// of lanes keeps an online softmax over the positions it sees, merged once
// at the end; and AttnPartialMfmaStaged (matrix cores, K/V staged in LDS;
// bf16 caches of head 128), below.  Both write partial[h, s, :] =
// (sum_t e^{score_t - m} V_t, m, l) with the reference's layout [q_heads,
// splits, head + 2]; splits that start past pos write nothing.
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
      kr[r] = C::template load_buf<0>(kres, off);
      vr[r] = C::template load_buf<0>(vres, off);
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

// Compiler-level ordering of LDS accesses between the lanes of one wave: the
// wave's LDS operations execute in program order, so a value one lane writes
// is visible to another lane's later read once the compiler keeps the two in
// that order (no hardware barrier is needed inside a wave).
AMMON_DEV void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Pass 1 entirely on matrix cores, with K/V staged in LDS by the load unit,
// for bf16 K/V and head 128 (Llama-style shapes).
//
// Staging.  Every K and V request is a 16-byte buffer load written straight
// into LDS (buffer_load_dwordx4 ... lds), so no VGPRs are held while the
// bytes are in flight.  The LDS holds a ring of NCH chunk buffers of 64
// positions (32 KiB each: K and V, 4 waves x 4 requests x 1 KiB); at the
// start a workgroup requests its first NCH chunks, and each chunk buffer is
// refilled with the chunk NCH ahead as soon as it is consumed.  Rows past
// the split's end read zero and touch no memory; the first NCH chunks are
// always requested, later ones only up to the split's last, so while it
// processes a chunk a wave has a known number of chunks (8 requests each)
// in flight behind it, and the waits are compile-time vmcnt values picked
// by that count.  Each wave
// reads back only the rows its own requests brought in, so no barrier is
// needed between the load unit and the consumer beyond the wave's own wait
// count.
//
// Arithmetic.  Wave w owns positions [16w, 16w + 16) of every chunk.
//   scores  S^T[t][h] = sum_d K[t][d] q[h][d] on v_mfma_f32_16x16x32_bf16
//           (A = K rows from LDS, B = q^T with q split into bf16 hi + lo:
//           ~16 bits of q, fp32 accumulation); heads >= G are padding;
//   softmax per wave and head, in base 2: running max m and sum l; the
//           weights P = 2^(s - m) are exact fp32 values;
//   values  O^T[d][h] += sum_t V[t][d] P[h][t] on v_mfma_f32_16x16x16_bf16
//           (A = V^T by transposing LDS reads, B = P^T straight from the score tile's
//           registers -- the score layout of a 16x16 tile is the 16x16x16
//           B-operand layout), with P split into three bf16 parts
//           (hi + mid + lo = P exactly), so every product is exact and only
//           the fp32 summation order differs from the serial definition.
// So the chunk loop has no workgroup barrier and little VALU work; the four
// waves' states are merged once at the end: M = max_w m_w,
// acc = sum_w acc_w 2^(m_w - M), l = sum_w l_w 2^(m_w - M).  The partial
// format is the other units': (sum_t e^{s_t - m} V_t, m, l).
//
// Rows land in LDS with their 16-byte pieces rotated so the operand reads
// are free of bank conflicts: K rows by the row index (the score operand
// reads one piece of 16 rows per lane group), V rows by 2 (row % 4) +
// 8 ((row / 4) % 2) slots (the transposing reads of the P.V operand take
// four rows' 32-byte runs per 16 lanes); row = the wave's position 0..15.
//
// LDS: att_staged_lds_floats(GMAX, NCH) floats (the merge's rows reuse the
// chunk buffers).
#define ATT_STAGED_OROW (ATT_MAX_HEAD + 4)  // merge row: 16-byte aligned, banks spread

// Max / sum over lanes l and l ^ 32 (resp. l ^ 16) with gfx950's lane-swap
// instructions (VALU, no LDS round trip): permlane32_swap(v, v) leaves the
// lane's own value in one result and its partner's in the other, so both
// lanes of a pair compute the same max and the same (commutative) sum.
AMMON_DEV float pair32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
AMMON_DEV float pair16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
AMMON_DEV float pair32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
AMMON_DEV float pair16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
constexpr uint32_t att_staged_lds_floats(int GMAX, int NCH) {
  const uint32_t ring = (uint32_t)NCH * 8192u;                      // NCH x 32 KiB
  const uint32_t merge = AMMON_WAVES * GMAX * ATT_STAGED_OROW;      // per-wave outputs
  // + the waves' maxima and sums, then the workgroup's per head
  return (ring > merge ? ring : merge) + 2 * AMMON_WAVES * GMAX + 2 * GMAX;
}

template <int GMAX, int NCH>
struct AttnPartialMfmaStaged {
  static_assert(GMAX >= 1 && GMAX <= 16, "q heads per kv head");
  static_assert(NCH >= 1 && NCH <= 4, "chunk buffers");
  static constexpr uint32_t HEAD = 128, CHUNK = 64;
  static constexpr int REQ = 8;  // requests per wave per chunk (4 K + 4 V)
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  typedef float f32x8 __attribute__((ext_vector_type(8)));

  uint32_t split, g, pos, t0, n, lane, wave;
  __amdgpu_buffer_rsrc_t kres, vres;
  float4 qraw[4][2];

  // The split, its cache resources and q; false for a dead split (start past
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

  // Ring buffer b's K (kv 0) or V (kv 1) block of request i of wave w, as
  // 16-byte slots: lane l's bytes land at slot l.
  AMMON_DEV static u32x4 *slot_base(float *lds, uint32_t b, uint32_t kv, uint32_t w, uint32_t i) {
    return (u32x4 *)lds + ((b * 2 + kv) * 16 + w * 4 + i) * 64;
  }

  // Request chunk c of the split into ring buffer b; every request of a
  // wave brings four whole 256-byte rows (1 KiB contiguous: a request that
  // gathered 16 rows x 16-byte pieces instead ran 1.1 us slower per 33.5 MB
  // launch).  K: request kk brings row r = 4kk + l / 16 of the wave's 16,
  // 16-byte piece (l % 16 + r) % 16 -- so the wave's K block is [row][slot],
  // slot s of row r holding dims 8((s + r) % 16)..+7, and the 16 lanes that
  // read one piece of 16 rows for the score MFMA hit 16 distinct slots.  V:
  // request i brings row r = 4i + l / 16, piece (l % 16 + rv(r)) % 16 with
  // rv(r) = 2 (r % 4) + 8 ((r / 4) % 2) -- slot s of row r holding dims
  // 8((s + rv(r)) % 16)..+7, so the transposing reads of v_frag (four rows'
  // 32-byte runs per 16 lanes, two lane groups per half-wave) fall on eight
  // distinct 32-byte bank ranges.  Rows at or past the split's end read as
  // zero.
  AMMON_DEV void stage(float *lds, uint32_t c, uint32_t b) const {
    const uint32_t c0 = c * CHUNK + 16 * wave;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t r = 4 * kk + (lane >> 4);
      const uint32_t tk = c0 + r;
      const uint32_t piece = ((lane & 15) + r) & 15;
      const uint32_t off = tk < n ? (tk * HEAD + 8 * piece) * 2 : AMMON_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          kres, (__attribute__((address_space(3))) void *)slot_base(lds, b, 0, wave, kk), 16,
          off, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t tv = c0 + 4 * i + (lane >> 4);
      const uint32_t piece = ((lane & 15) + 2 * (lane >> 4) + 8 * (i & 1)) & 15;
      const uint32_t off = tv < n ? (tv * HEAD + 8 * piece) * 2 : AMMON_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          vres, (__attribute__((address_space(3))) void *)slot_base(lds, b, 1, wave, i), 16,
          off, 0, 0, 0);
    }
  }

  // Lanes of score columns h >= GMAX load head 0's q: those columns are
  // never used, and unconditional loads keep the wait counts exact.
  AMMON_DEV void load_q(const ammon_k_attention &p) {
    const uint32_t h = lane & 15;
    const float *qp = p.q + (size_t)(g * GMAX + (h < GMAX ? h : 0)) * HEAD + 32 * (lane >> 4);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      qraw[kk][0] = ld_in4(qp + 8 * kk);
      qraw[kk][1] = ld_in4(qp + 8 * kk + 4);
    }
  }

  // q first (loads complete in order: the q conversion then waits for q
  // alone), then chunks 0..NCH - 1 -- unconditionally, so the count of
  // requests behind q is fixed (chunks past a short split read zero and
  // touch no memory).
  AMMON_DEV bool begin(const ammon_k_attention &p, uint32_t split_, uint32_t g_, float *lds) {
    if (!setup(p, split_, g_)) return false;
    load_q(p);
#pragma unroll
    for (int b = 0; b < NCH; ++b) stage(lds, b, b);
    __builtin_amdgcn_sched_barrier(0);
    return true;
  }

  // Wait until at most `extra` requests plus k whole chunks (REQ each) of
  // this wave are outstanding, k = 0..NCH - 1 (the chunks requested after
  // the one being processed).
  template <int EXTRA> AMMON_DEV static void wait_chunks(uint32_t k) {
    if (NCH > 3 && k == 3) wait_vmcnt<EXTRA + 3 * REQ>();
    else if (NCH > 2 && k == 2) wait_vmcnt<EXTRA + 2 * REQ>();
    else if (NCH > 1 && k == 1) wait_vmcnt<EXTRA + REQ>();
    else wait_vmcnt<EXTRA>();
  }

  // The V^T A fragment of dims 16nt..16nt+15 from the wave's staged V block:
  // lane l gets V[4(l / 16) + i][16nt + l % 16], i = 0..3, by one transposing
  // LDS read (ds_read_b64_tr_b16: within each 16-lane group, lane m receives
  // element m % 4 of the 8-byte blocks addressed by lanes m / 4 + 4i).  So
  // lane s of group g addresses row 4g + s / 4, dims 16nt + 4(s % 4)..+3.
  AMMON_DEV static i16x4 v_frag(const float *vblk, uint32_t lane, int nt) {
    const uint32_t s = lane & 15, g = lane >> 4, j = s >> 2, q = s & 3;
    const uint32_t r = 4 * g + j;
    const uint32_t slot = (2 * nt + (q >> 1) - (2 * j + 8 * (g & 1))) & 15;
    const uint16_t *a = (const uint16_t *)vblk + r * HEAD + slot * 8 + (q & 1) * 4;
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4 *)(a));
  }

  AMMON_DEV void run(const ammon_k_attention &p, float *lds) {
    const uint32_t ring = att_staged_lds_floats(GMAX, NCH) - 2 * AMMON_WAVES * GMAX - 2 * GMAX;
    float *s_m = lds + ring;                                       // [4][GMAX] wave maxima
    float *s_l = s_m + AMMON_WAVES * GMAX;                         // [4][GMAX] wave sums
    float *s_M = s_l + AMMON_WAVES * GMAX;                         // [GMAX] workgroup maxima
    float *s_L = s_M + GMAX;                                       // [GMAX] workgroup sums
    const float scale2 = 1.4426950408889634f / sqrtf((float)HEAD);  // log2(e)/sqrt(head)
    const uint32_t h = lane & 15, grp = lane >> 4;

    // q^T as bf16 hi + lo B operands
    bf16x8 qhi[4], qlo[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const float4 a = qraw[kk][0], b = qraw[kk][1];
      const f32x8 f = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      qhi[kk] = __builtin_convertvector(f, bf16x8);
      qlo[kk] = __builtin_convertvector(f - __builtin_convertvector(qhi[kk], f32x8), bf16x8);
    }

    // The score MFMA's A fragment kk of lane l: row l % 16 of the wave's K
    // block, dims 32(l / 16) + 8kk..+7 (q's B fragment kk holds the same
    // dims): piece 4(l / 16) + kk, at slot (piece - row) % 16 of that row.
    uint32_t kslot[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) kslot[kk] = 16 * h + ((4 * grp + kk - h) & 15);

    // O^T tiles: lane l holds dims 16nt + 4(l / 16) + r of head l % 16
    f32x4 o[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // running max / sum of head h (the lanes of one head agree)
    float m_run = -INFINITY, l_run = 0.f;

    const uint32_t nch = (n + CHUNK - 1) / CHUNK;
    // The split in blocks of up to NCH chunks (the whole split when it fits
    // the ring): all scores of a block first, then one max / exponential
    // pass, then the block's values -- the running state is rescaled once
    // per block, not per chunk.  Chunk c + NCH is requested once chunk c's
    // values are done, so when a block starts its chunks are requested and
    // the next block's are not: chunks [0, base_end) are, base_end = NCH for
    // the first block (chunks past a short split included) and the block's
    // end for the others.
    for (uint32_t c0b = 0; c0b < nch; c0b += NCH) {
      const uint32_t base_end = c0b == 0 ? (uint32_t)NCH : min(c0b + NCH, nch);
      float sb[NCH][4];
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const uint32_t c = c0b + i;
        if (c >= nch) {  // past the split (uniform)
#pragma unroll
          for (int r = 0; r < 4; ++r) sb[i][r] = -INFINITY;
          continue;
        }
        // K of chunk c landed: only its V and the block's later chunks may
        // be outstanding
        wait_chunks<4>(base_end - 1 - c);
        // two independent accumulation chains (q hi and q lo parts)
        f32x4 sh = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 a = __builtin_bit_cast(bf16x8, slot_base(lds, c % NCH, 0, wave, 0)[kslot[kk]]);
          sh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qhi[kk], sh, 0, 0, 0);
          sl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qlo[kk], sl, 0, 0, 0);
        }
        const f32x4 st = sh + sl;
        // lane l holds S^T[4(l / 16) + r][l % 16]: head h, positions
        // 16w + 4 grp + r of the chunk.  Score (reference
        // src/kernels.rs:298: dot / sqrt(head)) in base-2 units; past the
        // split: -inf.
        const uint32_t pl0 = c * CHUNK + 16 * wave + 4 * grp;
#pragma unroll
        for (int r = 0; r < 4; ++r) sb[i][r] = pl0 + r < n ? st[r] * scale2 : -INFINITY;
      }
      float mc = -INFINITY;
#pragma unroll
      for (int i = 0; i < NCH; ++i)
        mc = fmaxf(mc, fmaxf(fmaxf(sb[i][0], sb[i][1]), fmaxf(sb[i][2], sb[i][3])));
      mc = pair32_max(pair16_max(mc));
      const float m_new = fmaxf(m_run, mc);
      // a wave with no position yet keeps (m, l, acc) = (-inf, 0, 0)
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float sc = __builtin_amdgcn_exp2f(m_run - m_use);
      f32x4 pr[NCH];
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[i][r] = __builtin_amdgcn_exp2f(sb[i][r] - m_use);
        ls += (pr[i][0] + pr[i][1]) + (pr[i][2] + pr[i][3]);
      }
      ls = pair32_sum(pair16_sum(ls));
      l_run = l_run * sc + ls;
      m_run = m_new;
      // rescale the running tiles (none before the first block; a multiply
      // by exactly 1 is skipped)
      if (c0b > 0 && !__all(sc == 1.0f)) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) o[nt] *= sc;
      }
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const uint32_t c = c0b + i;
        if (c >= nch) continue;  // uniform
        // P^T as three bf16 parts with hi + mid + lo = P exactly
        i16x4 pp[3];
        const bf16x4 phi = __builtin_convertvector(pr[i], bf16x4);
        const f32x4 r1 = pr[i] - __builtin_convertvector(phi, f32x4);
        const bf16x4 pmid = __builtin_convertvector(r1, bf16x4);
        pp[0] = __builtin_bit_cast(i16x4, phi);
        pp[1] = __builtin_bit_cast(i16x4, pmid);
        pp[2] = __builtin_bit_cast(
            i16x4, __builtin_convertvector(r1 - __builtin_convertvector(pmid, f32x4), bf16x4));
        // V of chunk c landed: the block's later chunks and the refills for
        // its earlier ones (chunks up to min(c + NCH, nch)) may be
        // outstanding
        wait_chunks<0>(max(base_end, min(c + NCH, nch)) - 1 - c);
        const float *vblk = (const float *)slot_base(lds, c % NCH, 1, wave, 0);
        i16x4 va[8];
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) va[nt] = v_frag(vblk, lane, nt);
        // part-major: eight independent accumulation chains per part
#pragma unroll
        for (int part = 0; part < 3; ++part)
#pragma unroll
          for (int nt = 0; nt < 8; ++nt)
            o[nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[nt], pp[part], o[nt], 0, 0, 0);
        // refill buffer c % NCH with chunk c + NCH once this wave's reads
        // of it have returned (lgkmcnt(0); vmcnt and expcnt at their maxima)
        if (c + NCH < nch) {
          wave_lds_order();
          __builtin_amdgcn_s_waitcnt(0xC07F);
          stage(lds, c + NCH, c % NCH);
        }
      }
    }

    // every request has landed (zero-filled chunks of a short split too)
    // before the ring's LDS is reused below
    wait_vmcnt<0>();
    if (lane < GMAX) {
      s_m[wave * GMAX + lane] = m_run;
      s_l[wave * GMAX + lane] = l_run;
    }
    __syncthreads();
    // this wave's tiles, scaled to the workgroup max, as rows [w][h][d]
    // (16-byte writes); wave 0 also leaves each head's max and sum
    if (h < GMAX) {
      float M = s_m[h];
#pragma unroll
      for (int w = 1; w < AMMON_WAVES; ++w) M = fmaxf(M, s_m[w * GMAX + h]);
      // M is finite: a live split's first position is wave 0's
      const float f = __builtin_amdgcn_exp2f(m_run - M);
      float4 *row = (float4 *)(lds + (wave * GMAX + h) * ATT_STAGED_OROW + 4 * grp);
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
        row[4 * nt] = make_float4(o[nt][0] * f, o[nt][1] * f, o[nt][2] * f, o[nt][3] * f);
      if (wave == 0 && grp == 0) {
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < AMMON_WAVES; ++w)
          L += s_l[w * GMAX + h] * __builtin_amdgcn_exp2f(s_m[w * GMAX + h] - M);
        s_M[h] = M;
        s_L[h] = L;
      }
    }
    __syncthreads();
    const uint32_t slot_w = HEAD + 2;
    for (uint32_t idx = threadIdx.x; idx < GMAX * HEAD; idx += AMMON_WG) {
      const uint32_t j = idx / HEAD, d = idx % HEAD;
      float total = 0.f;
#pragma unroll
      for (int w = 0; w < AMMON_WAVES; ++w) total += lds[(w * GMAX + j) * ATT_STAGED_OROW + d];
      const float M = s_M[j], L = s_L[j];
      if (direct_out(p)) {  // the only split: the merge's result, total / l
        st_out(p.out + (size_t)(g * GMAX + j) * HEAD + d, total / L);
        continue;
      }
      float *o_ = p.partial + ((size_t)(g * GMAX + j) * p.splits + split) * slot_w;
      st_out(o_ + d, total);
      if (d == 0) {
        st_out(o_ + HEAD, M * 0.6931471805599453f);  // back to natural-log units
        st_out(o_ + HEAD + 1, L);
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

// Lines per lane of the merge's L2 warming (AMMON_WG * WARM_LINES lines, 128
// bytes each, per workgroup at most).
#define WARM_LINES 4

// The warming loads of merge workgroup b (one dword per 128-byte line of
// the next GEMV's row block b, see ammon_k_attention::warm).  The values
// are kept, unused, until warm_sink at the workgroup's end, so no wait for
// them is placed before then; they are issued after the merge's own loads,
// and loads complete in order, so the merge's waits leave them in flight.
// The WARM_LINES loads are issued unconditionally (with nothing to warm they
// read as zero and touch no memory), so every path has the same count in
// flight and the compiler's wait counts stay exact.
AMMON_DEV void warm_issue(const ammon_k_attention &p, uint32_t b, uint32_t pos,
                          uint32_t (&v)[WARM_LINES]) {
  // (not when the merge streams its partials after this point: its waits
  // would then wait for these loads too)
  const bool on = p.warm != nullptr && b < p.warm_blocks && pos >= p.warm_min_pos &&
                  p.splits <= COMB_ROUNDS * COMB_SPLIT_LANES;  // uniform
  const uint32_t per_row = on ? p.warm_bytes / 128 : 1;
  const uint32_t lines = on ? per_row * p.warm_rows : 0;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(
      on ? (const char *)p.warm + (size_t)b * p.warm_rows * p.warm_row_bytes : (const char *)p.partial,
      on ? p.warm_rows * p.warm_row_bytes : 0);
#pragma unroll
  for (int i = 0; i < WARM_LINES; ++i) {
    const uint32_t l = threadIdx.x + i * AMMON_WG;
    const uint32_t off = l < lines ? (l / per_row) * p.warm_row_bytes + (l % per_row) * 128
                                   : AMMON_OOB;
    v[i] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  }
}
AMMON_DEV void warm_sink(const uint32_t (&v)[WARM_LINES]) {
  asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]));
}

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
  uint32_t wv[WARM_LINES];
  warm_issue(p, blockIdx.x + gridDim.x * blockIdx.y, pos, wv);
  if (pos >= p.limit) {
    if (threadIdx.x < SLICE && d0 + threadIdx.x < head)
      st_out(out + d0 + threadIdx.x, __uint_as_float(0x7fc00000u));
    warm_sink(wv);
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
  warm_sink(wv);
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
