// prefill.hip -- multi-token GEMMs for prompt prefill, on matrix cores.
//
// The reference feeds a prompt one decode step per token
// (src/generate.rs:62-64), so each projection is a GEMV (src/kernels.rs:
// 518-528, serial definition :54-73) per token.  Prefill runs T consecutive
// positions through one GEMM per projection, Y[t] = W X[t], with the decode
// GEMV's fused epilogues: PLAIN, RESIDUAL (y = residual + W x), SWIGLU (gate
// rows in waves 0-1, the matching up rows in waves 2-3, paired through LDS:
// silu(gate) * up as src/kernels.rs:472-475) and QKV (RoPE on
// (2i, 2i+1) pairs of q and k rows at position step->position + t, then the
// head-major K/V cache stores of src/kernels.rs:174-226).
//
// Tiling.  A workgroup owns 64 virtual rows (16 per wave) x 16 NT tokens
// (NT 16-token column tiles) and walks the reduction in KC-wide chunks: NT = 1,
// KC = 512 for prompts of up to 16 tokens (twice the W bytes in flight per
// wave: x staging waits on the loads issued before it, so the W chunk after
// the current one is all a wave keeps in flight), NT = 2, KC = 256 beyond.  On
// each 32-wide step a wave multiplies its 16 x 32 slice of W (the A operand,
// as stored: lane l holds row l % 16, k 8(l / 16)..+7) by the tokens' x (the
// B operand, lane l: token l % 16, the same k) with 16x16 MFMAs; lane l then
// holds rows 4(l / 16)..+3 of token l % 16 of the result.
//
//   bf16 W: v_mfma_f32_16x16x32_bf16.  x is fp32, so each x is split into
//     three bf16 parts hi + mid + lo (each the bf16 rounding of what the
//     previous parts left): the parts sum to x exactly, every W x part
//     product is exact in fp32, and the three MFMAs accumulate in fp32 --
//     fp32-grade results; only the summation order differs from the GEMV.
//   fp32 W: v_mfma_f32_16x16x4_f32, eight per 32-wide step (lane group
//     l / 16 supplies k 8(l / 16) + e on the e-th), exact fp32 products.
//
// W streams from HBM through per-wave buffer resources (rows past the
// matrix and k past the row read as zero without touching memory), two
// chunks in flight per wave.  x is read from L2 (it is small and every
// workgroup of the pass reads it), one chunk ahead in registers, split /
// packed, and staged in LDS in the B-operand order: quad (step s, column
// tile c, part q, lane l) at ((s * NT + c) * XQ + q) * 64 + l, so every
// operand read is a conflict-free ds_read_b128.  Column tiles past the last
// token are skipped.
//
// Launch: a 1-D grid of ceil(row blocks / 8) * 8 * token tiles workgroups of
// 256 threads.  Workgroups go to the 8 XCDs round robin (id % 8), each XCD
// with its own L2, so the id -> (row block, token tile) map keeps all token
// tiles of a row block on one XCD and adjacent in dispatch order: W is
// fetched from HBM about once and re-read from that XCD's L2.
#include "device_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));


// WQ: 16-byte W loads per lane per step; XQ: LDS quads per lane per (step,
// column tile) -- three bf16 parts of 8 x values, or 8 fp32 x values.
template <typename WT> struct GemmTraits;
template <> struct GemmTraits<uint16_t> {
  static constexpr int WQ = 1, XQ = 3;
};
template <> struct GemmTraits<float> {
  static constexpr int WQ = 2, XQ = 2;
};

// NT 16-token column tiles per workgroup, KC-wide reduction chunks; KS
// waves share a row tile, each taking every KS-th 32-wide step (KS = 4: one
// 16-row tile per workgroup, the four partial sums added in wave order).
template <typename WT, int MODE, uint32_t NT, uint32_t KC, uint32_t KS>
struct GemmTile {
  static constexpr int WQ = GemmTraits<WT>::WQ, XQ = GemmTraits<WT>::XQ;
  static constexpr uint32_t ES = sizeof(WT);
  static constexpr uint32_t S = KC / 32;     // 32-wide steps per chunk
  static constexpr uint32_t SW = S / KS;     // of which each wave takes
  static constexpr uint32_t RBW = 16 * AMMON_WAVES / KS;  // virtual rows per workgroup
  static constexpr uint32_t TB = 16 * NT;    // tokens per workgroup
  static constexpr uint32_t KG = KC / 8;     // 8-wide k groups per chunk
  static constexpr uint32_t XU = TB * KG / AMMON_WG;  // x units per thread per chunk
  static_assert(TB * KG % AMMON_WG == 0, "x units per thread");

  ammon_k_gemm p;  // by value: a reference to the kernel argument would live in scratch
  uint32_t lane, wave, kw, vr0, tok0, row_bytes;
  // W source of this wave: row lane % 16 of resource r0.  SWIGLU, KS = 1:
  // waves 0-1 take gate rows i0..i0+15 / +16..+31 of the workgroup's 32
  // hidden rows, waves 2-3 the same up rows; KS = 4: rows 0-7 of the tile
  // are gate rows i0..i0+7 (r0), rows 8-15 the same up rows (r1).  vr0 is
  // then the first hidden row.
  __amdgpu_buffer_rsrc_t r0, r1;

  AMMON_DEV GemmTile(const ammon_k_gemm &p_, uint32_t rb, uint32_t tt) : p(p_) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kw = wave % KS;
    vr0 = rb * RBW + 16 * (wave / KS);
    tok0 = tt * TB;
    row_bytes = p.n * ES;
    auto rsrc = [&](const void *base, uint32_t first, uint32_t limit, uint32_t count) {
      const uint32_t valid = first < limit ? min(count, limit - first) : 0;
      return make_rsrc((const WT *)base + (size_t)(valid ? first : 0) * p.n, valid * row_bytes);
    };
    r1 = r0 = make_rsrc(p.w0, 0);
    if (MODE == AMMON_GEMV_SWIGLU && KS == 1) {
      vr0 = rb * (RBW / 2) + 16 * (wave & 1);
      r0 = rsrc(wave >= 2 ? p.w1 : p.w0, vr0, p.d, 16);
    } else if (MODE == AMMON_GEMV_SWIGLU) {
      vr0 = rb * (RBW / 2);
      r0 = rsrc(p.w0, vr0, p.d, 8);
      r1 = rsrc(p.w1, vr0, p.d, 8);
    } else if (MODE == AMMON_GEMV_QKV) {
      const uint32_t kvd = p.kv_dim;
      if (vr0 < p.d)
        r0 = rsrc(p.w0, vr0, p.d, 16);
      else if (vr0 < p.d + kvd)
        r0 = rsrc(p.w1, vr0 - p.d, kvd, 16);
      else
        r0 = rsrc(p.w2, vr0 - p.d - kvd, kvd, 16);
    } else {
      r0 = rsrc(p.w0, vr0, p.rows, 16);
    }
  }

  // W quads of this wave's steps of chunk `ch` (k past the row end read as
  // zero).
  AMMON_DEV void load_w(uint32_t ch, u32x4 (&w)[SW][WQ]) const {
#pragma unroll
    for (uint32_t j = 0; j < SW; ++j) {
      const uint32_t k = ch * KC + 32 * (j * KS + kw) + 8 * (lane >> 4);
      const bool ok = k < p.n;
#pragma unroll
      for (int q = 0; q < WQ; ++q) {
        if (MODE == AMMON_GEMV_SWIGLU && KS > 1) {
          // gate lanes read r0, up lanes r1; each lane's other one out of range
          const uint32_t off = (lane & 7) * row_bytes + (k + 4 * q) * ES;
          const bool up = (lane & 15) >= 8;
          const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r0, ok && !up ? off : AMMON_OOB, 0, 0);
          const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r1, ok && up ? off : AMMON_OOB, 0, 0);
          w[j][q] = a | b;
        } else {
          const uint32_t off = (lane & 15) * row_bytes + (k + 4 * q) * ES;
          w[j][q] = __builtin_amdgcn_raw_buffer_load_b128(r0, ok ? off : AMMON_OOB, 0, 0);
        }
      }
    }
  }

  // x unit u = tid + 256 m of chunk `ch` (8 consecutive k of one token):
  // the 64 units of each group u / 64 are 8 tokens x 8 consecutive k groups,
  // so a wave's loads read 8 rows of x, 256 contiguous bytes each; the unit
  // is B-fragment lane l = t % 16 + 16 (kg % 4) of step kg / 4 and column
  // tile t / 16.  Tokens and k past the end read as zero (no branches).
  AMMON_DEV static void unit(uint32_t u, uint32_t &s, uint32_t &c, uint32_t &l, uint32_t &t,
                             uint32_t &kg) {
    const uint32_t g = u >> 6, ln = u & 63;
    t = 8 * (g % (TB / 8)) + (ln >> 3);
    kg = 8 * (g / (TB / 8)) + (ln & 7);
    s = kg >> 2;
    c = t >> 4;
    l = (t & 15) + 16 * (kg & 3);
  }

  AMMON_DEV void load_x(uint32_t ch, u32x4 (&x)[XU][2]) const {
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x + (size_t)tok0 * p.n, (min(p.tokens - tok0, TB)) * p.n * 4);
#pragma unroll
    for (uint32_t m = 0; m < XU; ++m) {
      uint32_t s, c, l, t, kg;
      unit(threadIdx.x + AMMON_WG * m, s, c, l, t, kg);
      const uint32_t k = ch * KC + 8 * kg;
      const uint32_t off = k < p.n ? (t * p.n + k) * 4 : AMMON_OOB;
      x[m][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
      x[m][1] = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0);
    }
  }

  // LDS slot of B-fragment lane l of (step s, column tile c, part q), lanes
  // XOR-swizzled within their 16-quad row as in BigTile::quad below
  // (conflict-free operand reads and staging writes).
  AMMON_DEV static uint32_t quad(uint32_t s, uint32_t c, uint32_t q, uint32_t l) {
    const uint32_t pos = (((l & 15) ^ ((l >> 4) | 4 * (s & 1))) & 15) | (l & 48);
    return ((s * NT + c) * XQ + q) * 64 + pos;
  }

  // Split / pack the x chunk into LDS in B-operand order.
  AMMON_DEV void stage(const u32x4 (&x)[XU][2], u32x4 *xs) const {
#pragma unroll
    for (uint32_t m = 0; m < XU; ++m) {
      uint32_t s, c, l, t, kg;
      unit(threadIdx.x + AMMON_WG * m, s, c, l, t, kg);
      if constexpr (sizeof(WT) == 2) {
        const f32x4 a = __builtin_bit_cast(f32x4, x[m][0]), b = __builtin_bit_cast(f32x4, x[m][1]);
        const f32x8 f = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        const bf16x8 hi = __builtin_convertvector(f, bf16x8);
        const f32x8 r1 = f - __builtin_convertvector(hi, f32x8);
        const bf16x8 mid = __builtin_convertvector(r1, bf16x8);
        const f32x8 r2 = r1 - __builtin_convertvector(mid, f32x8);
        const bf16x8 lo = __builtin_convertvector(r2, bf16x8);
        xs[quad(s, c, 0, l)] = __builtin_bit_cast(u32x4, hi);
        xs[quad(s, c, 1, l)] = __builtin_bit_cast(u32x4, mid);
        xs[quad(s, c, 2, l)] = __builtin_bit_cast(u32x4, lo);
      } else {
        xs[quad(s, c, 0, l)] = x[m][0];
        xs[quad(s, c, 1, l)] = x[m][1];
      }
    }
  }

  AMMON_DEV void compute(const u32x4 (&w)[SW][WQ], const u32x4 *xs, f32x4 (&acc)[NT]) const {
#pragma unroll
    for (uint32_t j = 0; j < SW; ++j) {
      const uint32_t s = j * KS + kw;
#pragma unroll
      for (uint32_t c = 0; c < NT; ++c) {
        if (tok0 + 16 * c >= p.tokens) continue;  // uniform
        if constexpr (sizeof(WT) == 2) {
          const bf16x8 a = __builtin_bit_cast(bf16x8, w[j][0]);
#pragma unroll
          for (int q = 0; q < 3; ++q) {
            const bf16x8 b = __builtin_bit_cast(bf16x8, xs[quad(s, c, q, lane)]);
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const f32x4 a = __builtin_bit_cast(f32x4, w[j][q]);
            const f32x4 b = __builtin_bit_cast(f32x4, xs[quad(s, c, q, lane)]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc[c], 0, 0, 0);
          }
        }
      }
    }
  }

  // Lane l holds rows 4(l / 16) + r of the wave tile, token tok0 + 16c + l % 16.
  // KS = 1: contains barriers (SWIGLU), call uniformly; KS > 1: wave 0 only,
  // with the summed partials.  xs is free by then.
  AMMON_DEV void epilogue(f32x4 (&acc)[NT], u32x4 *xs) const {
    const uint32_t rq = 4 * (lane >> 4);
    float *ex = (float *)xs;
    if (MODE == AMMON_GEMV_SWIGLU && KS > 1) {
      // gate rows sit in lanes 0-31, the matching up rows 32 lanes higher
#pragma unroll
      for (uint32_t c = 0; c < NT; ++c) {
        float up[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) up[r] = __shfl_xor(acc[c][r], 32);
        const uint32_t t = tok0 + 16 * c + (lane & 15);
        if (lane >= 32 || t >= p.tokens) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t i = vr0 + rq + r;
          if (i >= p.d) continue;
          const float gate = acc[c][r];
          float v = gate * (1.0f / (1.0f + expf(-gate)));
          v = v * up[r];
          p.y[(size_t)t * p.d + i] = v;
        }
      }
      return;
    }
    if (MODE == AMMON_GEMV_SWIGLU) {
      // waves 2-3 hand their up rows to waves 0-1 through LDS, same lane layout
      __syncthreads();
      if (wave >= 2) {
#pragma unroll
        for (uint32_t c = 0; c < NT; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) ex[((((wave - 2) * NT + c) * 4) + r) * 64 + lane] = acc[c][r];
      }
      __syncthreads();
      if (wave >= 2) return;
    }
#pragma unroll
    for (uint32_t c = 0; c < NT; ++c) {
      const uint32_t t = tok0 + 16 * c + (lane & 15);
      if (MODE == AMMON_GEMV_SWIGLU) {
        if (t >= p.tokens) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t i = vr0 + rq + r;
          if (i >= p.d) continue;
          const float gate = acc[c][r], up = ex[(((wave * NT + c) * 4) + r) * 64 + lane];
          float v = gate * (1.0f / (1.0f + expf(-gate)));
          v = v * up;
          p.y[(size_t)t * p.d + i] = v;
        }
      } else if (MODE == AMMON_GEMV_QKV) {
#pragma clang fp contract(off)
        if (t >= p.tokens) continue;
        const uint32_t pos = p.step->position + t;
        const uint32_t kvd = p.kv_dim;
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          const uint32_t vr = vr0 + rq + r;
          if (vr >= p.rows) continue;
          const float a0 = acc[c][r], a1 = acc[c][r + 1];
          if (pos >= p.seq) {  // out-of-range position: poison q, touch no cache
            if (vr < p.d) {
              p.y[(size_t)t * p.d + vr] = __uint_as_float(0x7fc00000u);
              p.y[(size_t)t * p.d + vr + 1] = __uint_as_float(0x7fc00000u);
            }
            continue;
          }
          if (vr < p.d + kvd) {
            const uint32_t rr = vr < p.d ? vr : vr - p.d;
            const uint32_t hd = rr % p.head;
            const float *cs = p.table + ((size_t)pos * (p.head / 2) + hd / 2) * 2;
            const float fcr = cs[0], fci = cs[1];
            const float o0 = a0 * fcr - a1 * fci;
            const float o1 = a0 * fci + a1 * fcr;
            if (vr < p.d) {
              p.y[(size_t)t * p.d + vr] = o0;
              p.y[(size_t)t * p.d + vr + 1] = o1;
            } else {
              store_pair_out(p.k_cache, p.kv_dtype, ((size_t)(rr / p.head) * p.seq + pos) * p.head + hd,
                             o0, o1);
            }
          } else {
            const uint32_t rv = vr - p.d - kvd;
            store_pair_out(p.v_cache, p.kv_dtype,
                           ((size_t)(rv / p.head) * p.seq + pos) * p.head + rv % p.head, a0, a1);
          }
        }
      } else {
        if (t >= p.tokens) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t vr = vr0 + rq + r;
          if (vr >= p.rows) continue;
          const size_t at = (size_t)t * p.d + vr;
          p.y[at] = MODE == AMMON_GEMV_RESIDUAL ? p.residual[at] + acc[c][r] : acc[c][r];
        }
      }
    }
  }
};

template <typename WT, int MODE, uint32_t NT, uint32_t KC, uint32_t KS>
AMMON_DEV void gemm(const ammon_k_gemm &p) {
  using T = GemmTile<WT, MODE, NT, KC, KS>;
  constexpr uint32_t S = T::S, SW = T::SW;
  __shared__ u32x4 xs[S * NT * T::XQ * 64];
  static_assert(S * NT * T::XQ * 64 * 4 >= (KS - 1) * NT * 4 * 64, "room for the partial sums");
  // XCD-aware tile map: id = (row block group, token tile, XCD), row block =
  // group * 8 + XCD
  const uint32_t tiles = (p.tokens + T::TB - 1) / T::TB;
  const uint32_t q = blockIdx.x >> 3;
  const uint32_t rb = (q / tiles) * 8 + (blockIdx.x & 7u), tt = q % tiles;
  if (rb * T::RBW >= p.rows) return;  // padding of the last group (uniform)
  T tile(p, rb, tt);
  f32x4 acc[NT];
#pragma unroll
  for (uint32_t c = 0; c < NT; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t chunks = (p.n + KC - 1) / KC;
  u32x4 wa[SW][T::WQ], wb[SW][T::WQ];
  u32x4 xr[T::XU][2];
  tile.load_w(0, wa);
  tile.load_w(1, wb);
  tile.load_x(0, xr);
  // Two W buffers with fixed roles (unrolled); x one chunk ahead.
  for (uint32_t ch = 0; ch < chunks; ch += 2) {
    __syncthreads();  // the previous chunk's operands are consumed
    tile.stage(xr, xs);
    __syncthreads();
    if (ch + 1 < chunks) tile.load_x(ch + 1, xr);
    tile.compute(wa, xs, acc);
    tile.load_w(ch + 2, wa);
    if (ch + 1 >= chunks) break;
    __syncthreads();
    tile.stage(xr, xs);
    __syncthreads();
    if (ch + 2 < chunks) tile.load_x(ch + 2, xr);
    tile.compute(wb, xs, acc);
    tile.load_w(ch + 3, wb);
  }
  if (KS > 1) {
    // waves 1..KS-1 hand their partial sums to wave 0, added in wave order
    float *ex = (float *)xs;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (wave > 0) {
#pragma unroll
      for (uint32_t c = 0; c < NT; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) ex[(((wave - 1) * NT + c) * 4 + r) * 64 + lane] = acc[c][r];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (uint32_t w = 1; w < KS; ++w)
#pragma unroll
      for (uint32_t c = 0; c < NT; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[c][r] += ex[(((w - 1) * NT + c) * 4 + r) * 64 + lane];
  }
  tile.epilogue(acc, xs);
}

// QKV epilogue of virtual rows (v, v + 1) of token t: rotate q and k pairs
// with the cos/sin table at position step->position + t; q to y, k and raw
// v rows to the head-major caches (src/kernels.rs:174-226); a position past
// the cache poisons q and touches no cache.
AMMON_DEV void qkv_store_pair(const ammon_k_gemm &p, uint32_t t, uint32_t v, float a0, float a1) {
#pragma clang fp contract(off)
  const uint32_t pos = p.step->position + t;
  const uint32_t kvd = p.kv_dim;
  if (pos >= p.seq) {
    if (v < p.d) {
      p.y[(size_t)t * p.d + v] = __uint_as_float(0x7fc00000u);
      p.y[(size_t)t * p.d + v + 1] = __uint_as_float(0x7fc00000u);
    }
    return;
  }
  if (v < p.d + kvd) {
    const uint32_t rr = v < p.d ? v : v - p.d;
    const uint32_t hd = rr % p.head;
    const float *cs = p.table + ((size_t)pos * (p.head / 2) + hd / 2) * 2;
    const float fcr = cs[0], fci = cs[1];
    const float o0 = a0 * fcr - a1 * fci;
    const float o1 = a0 * fci + a1 * fcr;
    if (v < p.d) {
      p.y[(size_t)t * p.d + v] = o0;
      p.y[(size_t)t * p.d + v + 1] = o1;
    } else {
      store_pair_out(p.k_cache, p.kv_dtype, ((size_t)(rr / p.head) * p.seq + pos) * p.head + hd,
                     o0, o1);
    }
  } else {
    const uint32_t rv = v - p.d - kvd;
    store_pair_out(p.v_cache, p.kv_dtype,
                   ((size_t)(rv / p.head) * p.seq + pos) * p.head + rv % p.head, a0, a1);
  }
}

// ---- long prompts: register-blocked tiles ----------------------------------
// For prompts of 64 tokens and more a workgroup owns 64 tokens (4 column
// tiles) x 4 waves x RT 16-row tiles per wave.  Every B fragment (x part)
// read from LDS feeds RT MFMAs and every A fragment (W) 12, so a wave issues
// 3 NT RT MFMAs per 32-wide step against 3 NT LDS and RT global 16-byte
// reads per lane (the 16-row tiles above: 6 MFMAs per 6 LDS reads), and the
// x chunk is staged once for 64 RT rows.  W streams six steps (three chunks)
// ahead of use in registers and x two chunks ahead, so a workgroup's chain
// of chunks is not paced by memory latency; x is staged in three LDS
// buffers, one barrier per chunk.  The
// arithmetic per output is the 16-row tiles' (W x hi, W x mid, W x lo per
// step, fp32 accumulation) in the same order.  SWIGLU: a wave's first RT/2
// tiles are gate rows, the last RT/2 the same up rows, paired in registers.
template <int MODE, uint32_t RT, uint32_t NT_>
struct BigTile {
  static constexpr uint32_t NT = NT_, TB = 16 * NT, KC = 64, S = KC / 32;
  static constexpr uint32_t RW = 16 * RT;                // virtual rows per wave
  static constexpr uint32_t RBW = RW * AMMON_WAVES;      // virtual rows per workgroup
  static constexpr uint32_t KG = KC / 8;
  static constexpr uint32_t XU = TB * KG / AMMON_WG;     // x units per thread per chunk
  static constexpr uint32_t QUADS = S * NT * 3 * 64;     // LDS quads per x buffer
  static_assert(RT == 1 || RT % 2 == 0, "gate/up tile pairs");

  ammon_k_gemm p;  // by value (see GemmTile)
  uint32_t lane, tok0, row_bytes;
  uint32_t kbeg, kend;  // this workgroup's reduction range
  uint32_t vr[RT];  // first virtual row (SWIGLU: hidden row) of each tile
  __amdgpu_buffer_rsrc_t r[RT];

  AMMON_DEV BigTile(const ammon_k_gemm &p_, uint32_t rb, uint32_t tt, uint32_t ks) : p(p_) {
    lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    tok0 = tt * TB;
    row_bytes = p.n * 2;
    kbeg = p.ksplit > 1 ? ks * p.kchunks * KC : 0;
    kend = p.ksplit > 1 ? min(kbeg + p.kchunks * KC, p.n) : p.n;
    auto rsrc = [&](const void *base, uint32_t first, uint32_t limit) {
      const uint32_t valid = first < limit ? min(16u, limit - first) : 0;
      return make_rsrc((const uint16_t *)base + (size_t)(valid ? first : 0) * p.n,
                       valid * row_bytes);
    };
#pragma unroll
    for (uint32_t j = 0; j < RT; ++j) {
      if (MODE == AMMON_GEMV_SWIGLU) {
        const uint32_t h = rb * (RBW / 2) + wave * (RW / 2) + 16 * (j % (RT / 2));
        vr[j] = h;
        r[j] = rsrc(j < RT / 2 ? p.w0 : p.w1, h, p.d);
      } else {
        const uint32_t v = rb * RBW + wave * RW + 16 * j;
        vr[j] = v;
        if (MODE == AMMON_GEMV_QKV) {
          const uint32_t kvd = p.kv_dim;
          if (v < p.d)
            r[j] = rsrc(p.w0, v, p.d);
          else if (v < p.d + kvd)
            r[j] = rsrc(p.w1, v - p.d, kvd);
          else
            r[j] = rsrc(p.w2, v - p.d - kvd, kvd);
        } else {
          r[j] = rsrc(p.w0, v, p.rows);
        }
      }
    }
  }

  // W of the range's 32-wide step g (k past the range reads zero).
  AMMON_DEV void load_w(uint32_t g, u32x4 (&a)[RT]) const {
    const uint32_t k = kbeg + 32 * g + 8 * (lane >> 4);
    const uint32_t off = k < kend ? (lane & 15) * row_bytes + k * 2 : AMMON_OOB;
#pragma unroll
    for (uint32_t j = 0; j < RT; ++j) a[j] = __builtin_amdgcn_raw_buffer_load_b128(r[j], off, 0, 0);
  }

  // x unit u (8 consecutive k of one token) of a chunk: the 64 units of
  // each group u / 64 are 8 tokens x the chunk's 8 k groups, so each wave's
  // two 16-byte loads per unit cover 8 rows of x, 256 contiguous bytes each
  // (B-fragment order, 16 tokens x 4 k groups per load, made the 512-token
  // gate/up GEMM 15% slower); the unit is B-fragment lane l = t % 16 +
  // 16 (kg % 4) of step kg / 4 and column tile t / 16.
  AMMON_DEV static void unit(uint32_t u, uint32_t &s, uint32_t &c, uint32_t &l, uint32_t &t,
                             uint32_t &kg) {
    const uint32_t g = u >> 6, ln = u & 63;
    t = 8 * g + (ln >> 3);
    kg = ln & 7;
    s = kg >> 2;
    c = t >> 4;
    l = (t & 15) + 16 * (kg & 3);
  }

  AMMON_DEV void load_x(uint32_t ch, u32x4 (&x)[XU][2]) const {
    const __amdgpu_buffer_rsrc_t xr =
        make_rsrc(p.x + (size_t)tok0 * p.n, (min(p.tokens - tok0, TB)) * p.n * 4);
#pragma unroll
    for (uint32_t m = 0; m < XU; ++m) {
      uint32_t s, c, l, t, kg;
      unit(threadIdx.x + AMMON_WG * m, s, c, l, t, kg);
      const uint32_t k = kbeg + ch * KC + 8 * kg;
      const uint32_t off = k < kend ? (t * p.n + k) * 4 : AMMON_OOB;
      x[m][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
      x[m][1] = __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0);
    }
  }

  // LDS slot of B-fragment lane l of (step s, column tile c, part q): the
  // fragment's 64 quads, with lane l's position within its 16-quad row
  // XOR-swizzled by its k group and the step's parity.  LDS serves a
  // 16-byte access 8 lanes (128 bytes) at a time: the operand reads' 8
  // lanes stay within one 8-quad run, and a staging write's 8 lanes (one
  // token, 8 k groups over two steps) get the 8 distinct values of
  // (k group | 4 (step & 1)) in the low three bits, so neither conflicts
  // (an XOR by 4 (k group) ^ 2 step left the writes 2-way conflicted).
  AMMON_DEV static uint32_t quad(uint32_t s, uint32_t c, uint32_t q, uint32_t l) {
    const uint32_t pos = (((l & 15) ^ ((l >> 4) | 4 * (s & 1))) & 15) | (l & 48);
    return ((s * NT + c) * 3 + q) * 64 + pos;
  }

  AMMON_DEV void stage(const u32x4 (&x)[XU][2], u32x4 *xs) const {
#pragma unroll
    for (uint32_t m = 0; m < XU; ++m) {
      uint32_t s, c, l, t, kg;
      unit(threadIdx.x + AMMON_WG * m, s, c, l, t, kg);
      const f32x4 a = __builtin_bit_cast(f32x4, x[m][0]), b = __builtin_bit_cast(f32x4, x[m][1]);
      const f32x8 f = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
      const bf16x8 hi = __builtin_convertvector(f, bf16x8);
      const f32x8 r1 = f - __builtin_convertvector(hi, f32x8);
      const bf16x8 mid = __builtin_convertvector(r1, bf16x8);
      const f32x8 r2 = r1 - __builtin_convertvector(mid, f32x8);
      const bf16x8 lo = __builtin_convertvector(r2, bf16x8);
      xs[quad(s, c, 0, l)] = __builtin_bit_cast(u32x4, hi);
      xs[quad(s, c, 1, l)] = __builtin_bit_cast(u32x4, mid);
      xs[quad(s, c, 2, l)] = __builtin_bit_cast(u32x4, lo);
    }
  }

  // Step s of the staged chunk: per column tile the three x parts, each
  // against every row tile.  Straight-line code: a column tile past the
  // last token multiplies staged zeros rather than branching, so the LDS
  // reads of the whole step can be issued ahead of the MFMAs.
  AMMON_DEV void compute(uint32_t s, const u32x4 *xs, const u32x4 (&a)[RT],
                         f32x4 (&acc)[RT][NT]) const {
#pragma unroll
    for (uint32_t c = 0; c < NT; ++c) {
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const bf16x8 b = __builtin_bit_cast(bf16x8, xs[quad(s, c, q, lane)]);
#pragma unroll
        for (uint32_t j = 0; j < RT; ++j)
          acc[j][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, a[j]), b, acc[j][c], 0, 0, 0);
      }
    }
  }

  // Lane l holds rows 4(l / 16)..+3 of each tile for token tok0 + 16c + l % 16.
  AMMON_DEV void epilogue(const f32x4 (&acc)[RT][NT], uint32_t ks) const {
    const uint32_t rq = 4 * (lane >> 4);
#pragma unroll
    for (uint32_t c = 0; c < NT; ++c) {
      const uint32_t t = tok0 + 16 * c + (lane & 15);
      if (t >= p.tokens) continue;
      if (MODE != AMMON_GEMV_SWIGLU && p.ksplit > 1) {
        float *w = p.ws + ((size_t)ks * p.tokens + t) * p.rows;  // this range's partial sums
#pragma unroll
        for (uint32_t j = 0; j < RT; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t v = vr[j] + rq + i;
            if (v < p.rows) w[v] = acc[j][c][i];
          }
      } else if (MODE == AMMON_GEMV_SWIGLU) {
#pragma unroll
        for (uint32_t j = 0; j < RT / 2; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t h = vr[j] + rq + i;
            if (h >= p.d) continue;
            const float gate = acc[j][c][i], up = acc[j + RT / 2][c][i];
            float v = gate * (1.0f / (1.0f + expf(-gate)));
            v = v * up;
            p.y[(size_t)t * p.d + h] = v;
          }
      } else if (MODE == AMMON_GEMV_QKV) {
#pragma unroll
        for (uint32_t j = 0; j < RT; ++j)
#pragma unroll
          for (int i = 0; i < 4; i += 2) {
            const uint32_t v = vr[j] + rq + i;
            if (v < p.rows) qkv_store_pair(p, t, v, acc[j][c][i], acc[j][c][i + 1]);
          }
      } else {
#pragma unroll
        for (uint32_t j = 0; j < RT; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t v = vr[j] + rq + i;
            if (v >= p.rows) continue;
            const size_t at = (size_t)t * p.d + v;
            p.y[at] = MODE == AMMON_GEMV_RESIDUAL ? p.residual[at] + acc[j][c][i] : acc[j][c][i];
          }
      }
    }
  }
};

template <int MODE, uint32_t RT, uint32_t NT>
AMMON_DEV void gemm_big(const ammon_k_gemm &p) {
  using T = BigTile<MODE, RT, NT>;
  __shared__ u32x4 xs[3][T::QUADS];
  // id = ((row-block group, reduction range), token tile, XCD): the token
  // tiles of a row block and range are adjacent on one XCD
  const uint32_t tiles = (p.tokens + T::TB - 1) / T::TB;
  const uint32_t ksplit = p.ksplit > 1 ? p.ksplit : 1;
  const uint32_t q = blockIdx.x >> 3;
  const uint32_t tt = q % tiles, ks = (q / tiles) % ksplit;
  const uint32_t rb = (q / tiles / ksplit) * 8 + (blockIdx.x & 7u);
  const uint32_t covered = MODE == AMMON_GEMV_SWIGLU ? p.d : p.rows;
  const uint32_t per = MODE == AMMON_GEMV_SWIGLU ? T::RBW / 2 : T::RBW;
  if (rb * per >= covered) return;  // padding of the last group (uniform)
  T tile(p, rb, tt, ks);
  f32x4 acc[RT][T::NT];
#pragma unroll
  for (uint32_t j = 0; j < RT; ++j)
#pragma unroll
    for (uint32_t c = 0; c < T::NT; ++c) acc[j][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t chunks = (tile.kend - tile.kbeg + T::KC - 1) / T::KC;
  // rings: W of steps 2ch .. 2ch + 5 (a0..a5), x of chunks ch .. ch + 2
  // (x0..x2), LDS buffer ch % 3
  u32x4 a0[RT], a1[RT], a2[RT], a3[RT], a4[RT], a5[RT];
  u32x4 x0[T::XU][2], x1[T::XU][2], x2[T::XU][2];
  // issue order pinned as the loop's (see below)
  tile.load_w(0, a0);
  __builtin_amdgcn_sched_barrier(0);
  tile.load_w(1, a1);
  __builtin_amdgcn_sched_barrier(0);
  tile.load_x(0, x0);
  __builtin_amdgcn_sched_barrier(0);
  tile.load_w(2, a2);
  __builtin_amdgcn_sched_barrier(0);
  tile.load_w(3, a3);
  __builtin_amdgcn_sched_barrier(0);
  tile.load_x(1, x1);
  __builtin_amdgcn_sched_barrier(0);
  tile.load_w(4, a4);
  __builtin_amdgcn_sched_barrier(0);
  tile.load_w(5, a5);
  __builtin_amdgcn_sched_barrier(0);
  // Chunk c: stage its x (loaded two chunks ago) into LDS buffer c % 3,
  // then request x of chunk c + 2 and, as each step's W is used, the W six
  // steps on.  Buffer c % 3 was last read for chunk c - 3, which every wave
  // finished before the barrier of chunk c - 2.  Requests past the end read
  // zero without touching memory; they are issued anyway so that every path
  // into the loop has the same loads in flight in the same order (the
  // compiler's wait counts then leave the prefetches outstanding).
  // The scheduling barriers pin the issue order of the phases: the memory
  // counters complete in order, so a load moved later would make every
  // older prefetch wait for it.
#define BIG_CHUNK(C, XS, XC, XN, WA, WB)                 \
  {                                                      \
    tile.stage(XC, xs[XS]);                              \
    __syncthreads();                                     \
    tile.load_x((C) + 2, XN);                            \
    __builtin_amdgcn_sched_barrier(0);                   \
    tile.compute(0, xs[XS], WA, acc);                    \
    __builtin_amdgcn_sched_barrier(0);                   \
    tile.load_w(2 * (C) + 6, WA);                        \
    __builtin_amdgcn_sched_barrier(0);                   \
    tile.compute(1, xs[XS], WB, acc);                    \
    __builtin_amdgcn_sched_barrier(0);                   \
    tile.load_w(2 * (C) + 7, WB);                        \
    __builtin_amdgcn_sched_barrier(0);                   \
  }
  // Whole rounds of three chunks: one or two chunks past the end multiply
  // zeros (adding nothing), which keeps the loop body free of exits.
  for (uint32_t ch = 0; ch < chunks; ch += 3) {
    BIG_CHUNK(ch, 0, x0, x2, a0, a1)
    BIG_CHUNK(ch + 1, 1, x1, x0, a2, a3)
    BIG_CHUNK(ch + 2, 2, x2, x1, a4, a5)
  }
#undef BIG_CHUNK
  tile.epilogue(acc, ks);
}

}  // namespace

#define GEMM_KERNEL(NAME, WT, MODE, NT, KC, KS)                                    \
  extern "C" __global__ __launch_bounds__(AMMON_WG) void NAME(ammon_k_gemm p) { \
    gemm<WT, MODE, NT, KC, KS>(p);                                               \
  }
#define GEMM_MODE4(DT, WT, SUFFIX, NT, KC, KS)                                         \
  GEMM_KERNEL(ammon_gemm_##DT##_plain_##SUFFIX, WT, AMMON_GEMV_PLAIN, NT, KC, KS)       \
  GEMM_KERNEL(ammon_gemm_##DT##_residual_##SUFFIX, WT, AMMON_GEMV_RESIDUAL, NT, KC, KS) \
  GEMM_KERNEL(ammon_gemm_##DT##_swiglu_##SUFFIX, WT, AMMON_GEMV_SWIGLU, NT, KC, KS)     \
  GEMM_KERNEL(ammon_gemm_##DT##_qkv_##SUFFIX, WT, AMMON_GEMV_QKV, NT, KC, KS)
// t16 / t32: up to 16 / 32 tokens per workgroup; k4: one 16-row tile per
// workgroup, the reduction split over its four waves
#define GEMM_MODES(DT, WT, KC16)              \
  GEMM_MODE4(DT, WT, t16, 1, KC16, 1)         \
  GEMM_MODE4(DT, WT, t32, 2, 256, 1)          \
  GEMM_MODE4(DT, WT, t16_k4, 1, KC16, 4)      \
  GEMM_MODE4(DT, WT, t32_k4, 2, 256, 4)

GEMM_MODES(bf16, uint16_t, 512)
GEMM_MODES(f32, float, 256)

// long prompts, bf16 W: 16 NT-token tiles, RT 16-row tiles per wave.  OCC:
// workgroups per CU the registers must allow (the LDS allows 2 of the
// 64-token tiles' 72 KiB, 4 of the 32-token tiles' 36 KiB); left to itself
// the compiler gave the 64-row-per-wave tiles 288 registers (one wave per
// SIMD) and shuffled the SwiGLU tile's accumulators between register files.
#define GEMM_BIG_KERNEL(NAME, MODE, RT, NT, OCC)                                        \
  extern "C" __global__ __launch_bounds__(AMMON_WG, OCC) void NAME(ammon_k_gemm p) { \
    gemm_big<MODE, RT, NT>(p);                                                        \
  }
#define GEMM_BIG_MODES(SUFFIX, RT, NT, OCC)                                                 \
  GEMM_BIG_KERNEL(ammon_gemm_bf16_plain_##SUFFIX, AMMON_GEMV_PLAIN, RT, NT, OCC)            \
  GEMM_BIG_KERNEL(ammon_gemm_bf16_residual_##SUFFIX, AMMON_GEMV_RESIDUAL, RT, NT, OCC)      \
  GEMM_BIG_KERNEL(ammon_gemm_bf16_swiglu_##SUFFIX, AMMON_GEMV_SWIGLU, RT, NT, OCC)          \
  GEMM_BIG_KERNEL(ammon_gemm_bf16_qkv_##SUFFIX, AMMON_GEMV_QKV, RT, NT, OCC)
GEMM_BIG_MODES(t64_r4, 4, 4, 2)
GEMM_BIG_MODES(t64_r2, 2, 4, 2)
GEMM_BIG_MODES(t32_r4, 4, 2, 2)
GEMM_BIG_MODES(t32_r2, 2, 2, 4)

// y[t][r] = (residual[t][r] +) the split ranges' partial sums added in range
// order: grid-stride over tokens x d.
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_gemm_reduce(ammon_k_gemm p) {
  const size_t total = (size_t)p.tokens * p.d;
  for (size_t i = (size_t)blockIdx.x * AMMON_WG + threadIdx.x; i < total;
       i += (size_t)gridDim.x * AMMON_WG) {
    float acc = p.ws[i];
    for (uint32_t s = 1; s < p.ksplit; ++s) acc = acc + p.ws[s * total + i];
    p.y[i] = p.residual ? p.residual[i] + acc : acc;
  }
}

// QKV: each (token, row pair) sums its split partial sums in range order,
// then the QKV epilogue: grid-stride over tokens x rows / 2.
extern "C" __global__ __launch_bounds__(AMMON_WG) void ammon_gemm_reduce_qkv(ammon_k_gemm p) {
  const uint32_t pairs = p.rows / 2;
  const size_t total = (size_t)p.tokens * p.rows, n = (size_t)p.tokens * pairs;
  for (size_t i = (size_t)blockIdx.x * AMMON_WG + threadIdx.x; i < n;
       i += (size_t)gridDim.x * AMMON_WG) {
    const uint32_t t = (uint32_t)(i / pairs), v = 2 * (uint32_t)(i % pairs);
    const size_t at = (size_t)t * p.rows + v;
    float a0 = p.ws[at], a1 = p.ws[at + 1];
    for (uint32_t s = 1; s < p.ksplit; ++s) {
      a0 = a0 + p.ws[s * total + at];
      a1 = a1 + p.ws[s * total + at + 1];
    }
    qkv_store_pair(p, t, v, a0, a1);
  }
}
