// gemv_impl.h -- the bandwidth-bound batch-1 GEMV pass of the GEMV kernels
// (gemv.hip).  Replaces the reference's Goldy matmul_into
// (src/kernels.rs:518-528), whose definition is the serial gemv
// (src/kernels.rs:54-73), with the surrounding rmsnorm / rope_store /
// cache_store / swiglu / add_into launches of src/blocks.rs:219-276 fused in.
//
// y_i = sum_j W[i, j] x_j with W row-major [rows, n] in fp32 or bf16.
//
// Workgroup of 4 wave64s.  x (optionally RMS-normalised) is staged once per
// workgroup in LDS as fp32, zero-padded to whole tiles.  Each wave owns RPW
// consecutive "virtual rows" per row block; lane l streams the 16-byte
// chunks l, l+64, ... of each of its rows (coalesced 1 KiB per wave per load
// instruction), keeping U chunk loads per row in flight, multiplies them
// against the matching LDS slice of x and reduces each row across the wave.
// Row blocks are distributed over the workgroups of the pass (workgroup wg
// of nwg takes blocks wg, wg + nwg, ...), so x is staged once per
// workgroup.  No MFMA: at batch 1 the arithmetic intensity is ~1 flop/byte.
//
// Modes (virtual rows):
//   PLAIN     y[r] = dot_r; with a step, y[position * d + r] (reference gemv)
//   RESIDUAL  y[r] = residual[r] + dot_r            (y may alias residual)
//   SWIGLU    rows interleave gate (w0) and up (w1): r = 2i -> gate row i,
//             r = 2i+1 -> up row i; y[i] = silu(gate) * up in the reference's
//             order (src/kernels.rs:472-475)
//   PLAIN_ARGMAX  PLAIN, and each workgroup writes the (value, lowest index)
//             of the maximum over its rows (NaN never wins) to cand_v/cand_i
//             [wg]: pass 1 of the greedy argmax fused into the LM head
//   QKV       rows run over [Wq; Wk; Wv]; (2i, 2i+1) pairs of q and k rows are
//             rotated with the cos/sin table at step->position; q goes to y,
//             rotated k and raw v go to the head-major caches at that position
//             (src/kernels.rs:174-226).
//
// The pass runs in two steps: begin() requests the first two tiles (weights
// only, which depend on nothing an earlier kernel wrote), run() stages x,
// then multiplies and keeps streaming.  Work is a sequence of
// tiles per workgroup: tile = (row block, chunk range) of RPW rows per wave
// x 64*U chunks, software-pipelined through two register buffers -- the
// next tile's loads are in flight while the current one is multiplied.
//
// Outputs (y, K/V rows) go through st_out and inputs an earlier kernel
// wrote (x, the residual) through ld_in (device_common.h).
//
// The RMSNorm prologue sums squares with the same per-lane chunking and
// reduction order as ammon_rmsnorm, so its normalised x matches the
// standalone kernel bit for bit when the rows are 16-byte aligned.
#pragma once

#include "argmax_impl.h"
#include "device_common.h"

template <typename WT, int CH, int RPW, int U, int MODE>
struct GemvPass {
  using C = Chunk<WT, CH>;
  using V = typename C::V;

  // x staging (run()): up to XREG 16-byte chunks of x (and of the norm
  // weight) per lane through registers; longer x without a norm by 16-byte
  // buffer loads straight into LDS; anything else by a loop in run().
  static constexpr int XREG = 4;
  enum XPath { X_REG, X_DMA, X_LOOP };

  ammon_k_gemv p;
  uint32_t wg, nwg;
  uint32_t n, tiles, wave_u, row_bytes;
  uint32_t blk, ti, blk1, ti1;
  XPath xpath;
  float pre_a[RPW], pre_b[RPW];
  float4 xr[XREG], wr[XREG];  // x and the fp32 norm weight (X_REG)
  uint2 wb[XREG];             // ... or the bf16 norm weight's raw bits
  V bufA[RPW][U], bufB[RPW][U];

  static constexpr uint32_t tile_chunks = 64 * U;

  // Row pointer of virtual row r0 + k; rows past the end read row 0.  The
  // wave index is made wave-uniform so row selection stays in scalar
  // registers, and rows start even (RPW is even), so in SWIGLU mode the
  // gate/up choice is k's parity -- a compile-time select, never a memory
  // read of the argument block that would have to wait behind the loads in
  // flight.
  AMMON_DEV const WT *row_ptr(uint32_t b, int k) const {
    const uint32_t r0 = (b * AMMON_WAVES + wave_u) * RPW;
    const uint32_t vr = r0 + k;
    const bool ok = vr < p.rows;
    if (MODE == AMMON_GEMV_SWIGLU) {
      const WT *base = (const WT *)((k & 1) ? p.w1 : p.w0);
      return base + (size_t)(ok ? (r0 >> 1) + (k >> 1) : 0) * n;
    } else if (MODE == AMMON_GEMV_QKV) {
      const uint32_t r = ok ? vr : 0;
      const WT *w0 = (const WT *)p.w0, *w1 = (const WT *)p.w1, *w2 = (const WT *)p.w2;
      if (r < p.d) return w0 + (size_t)r * n;
      if (r < p.d + p.kv_dim) return w1 + (size_t)(r - p.d) * n;
      return w2 + (size_t)(r - p.d - p.kv_dim) * n;
    }
    return (const WT *)p.w0 + (size_t)(ok ? vr : 0) * n;
  }

  // Loads of tile (b, t) through per-row buffer resources: chunks past the
  // row end, and every chunk of a tile past the last row block, read as zero
  // without touching memory.  No branches, so the wait counts of the two
  // in-flight tiles stay exact.
  AMMON_DEV void load_tile(uint32_t b, uint32_t t, V (&buf)[RPW][U]) const {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t bytes = b < p.row_blocks ? row_bytes : 0;
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const __amdgpu_buffer_rsrc_t r = make_rsrc(row_ptr(b, k), bytes);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t c = t * tile_chunks + u * 64 + lane;
        buf[k][u] = C::template load_buf<AMMON_WEIGHT_CPOL>(r, c * (uint32_t)(CH * sizeof(WT)));
      }
    }
  }

  // Epilogue operands of row block b: QKV -> (cos, sin) of row pair k
  // (k even) at step->position; RESIDUAL -> residual[row k].
  AMMON_DEV void epi_load(uint32_t b, uint32_t pos, float (&ea)[RPW], float (&eb)[RPW]) const {
    const uint32_t r0 = (b * AMMON_WAVES + wave_u) * RPW;
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      ea[k] = 0.f;
      eb[k] = 0.f;
      const uint32_t vr = r0 + k;
      if (vr >= p.rows) continue;
      if (MODE == AMMON_GEMV_RESIDUAL) {
        ea[k] = ld_in(p.residual + vr);
      } else if (MODE == AMMON_GEMV_QKV && (k & 1) == 0 && pos < p.seq &&
                 vr < p.d + p.kv_dim) {
        const uint32_t rr = vr < p.d ? vr : vr - p.d;
        const uint32_t hd = rr % p.head;
        const float *cs = p.table + ((size_t)pos * (p.head / 2) + hd / 2) * 2;
        ea[k] = cs[0];
        eb[k] = cs[1];
      }
    }
  }

  AMMON_DEV static void advance(uint32_t &b, uint32_t &t, uint32_t tiles_, uint32_t nwg_) {
    if (++t == tiles_) {
      t = 0;
      b += nwg_;
    }
  }

  // LDS layout of x in 16-byte quads.  With 8-element chunks a lane needs
  // two quads; they are stored as two planes of 64 quads per 64 chunks, so
  // each ds_read_b128 of a wave covers 1 KiB of consecutive addresses
  // (conflict-free) instead of a 32-byte lane stride.
  AMMON_DEV static uint32_t xq(uint32_t q) {
    if (CH == 8) return (q & ~127u) | ((q & 1u) << 6) | ((q >> 1) & 63u);
    return q;
  }

  // Request x (and the norm weight) for staging: the registers of the
  // X_REG path, or the buffer-to-LDS loads of the X_DMA path (wave w fills
  // groups w, w + 4, ... of GQ quads: with 8-element chunks the two planes
  // of a group are two loads, even quads then odd, each lane's 16 bytes
  // landing at slot `lane` of its plane; quads past n read as zero).
  AMMON_DEV void request_x(float4 *xs4) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const bool xvec = (n & 3u) == 0 && (((uintptr_t)p.x) & 15u) == 0;
    // norm weights read four at a time: 8-byte (bf16) or 16-byte (fp32) loads
    const bool wvec = p.norm_w == nullptr ||
                      (((uintptr_t)p.norm_w) & (p.norm_dtype == AMMON_K_BF16 ? 7u : 15u)) == 0;
    if (!p.norm_w && xvec && n / 4 > XREG * AMMON_WG) {
      xpath = X_DMA;
      const __amdgpu_buffer_rsrc_t xres = make_rsrc(p.x, n * 4u);
      constexpr uint32_t GQ = CH == 8 ? 128 : 64;
      static_assert(tile_chunks * CH / 4 % GQ == 0, "whole groups per tile");
      const uint32_t groups = tiles * tile_chunks * CH / 4 / GQ;
      for (uint32_t g = wave_u; g < groups; g += AMMON_WAVES) {
#pragma unroll
        for (uint32_t pl = 0; pl < GQ / 64; ++pl) {
          const uint32_t q = g * GQ + (GQ == 128 ? 2 * lane + pl : lane);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              xres, (__attribute__((address_space(3))) void *)(xs4 + g * GQ + pl * 64), 16,
              q < n / 4 ? q * 16 : AMMON_OOB, 0, 0, 0);
        }
      }
    } else if (xvec && wvec && n / 4 <= XREG * AMMON_WG) {
      xpath = X_REG;
#pragma unroll
      for (int i = 0; i < XREG; ++i) {
        const uint32_t c = tid + i * AMMON_WG;
        if (c < n / 4) {
          xr[i] = ld_in4(p.x + 4 * c);
          // raw loads only (widened in run()): nothing here waits for a load
          if (p.norm_w) {
            if (p.norm_dtype == AMMON_K_BF16)
              wb[i] = ((const uint2 *)p.norm_w)[c];
            else
              wr[i] = ((const float4 *)p.norm_w)[c];
          }
        }
      }
    } else {
      xpath = X_LOOP;
    }
  }

  // Request x (into registers or LDS) and then the first two tiles of
  // workgroup wg_ of nwg_.  x first: it is small and shared by every
  // workgroup, so it arrives ahead of the weights and its staging (and the
  // norm) runs while the weights stream in.
  AMMON_DEV void begin(const ammon_k_gemv &params, uint32_t wg_, uint32_t nwg_, float4 *xs4) {
    p = params;
    wg = wg_;
    nwg = nwg_;
    n = p.n;
    const uint32_t nch = n / CH;
    tiles = (nch + tile_chunks - 1) / tile_chunks;  // per row block
    wave_u = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    row_bytes = n * (uint32_t)sizeof(WT);
    blk = wg;
    ti = 0;
    blk1 = blk;
    ti1 = ti;
    advance(blk1, ti1, tiles, nwg);
    request_x(xs4);
    load_tile(blk, ti, bufA);
    load_tile(blk1, ti1, bufB);
  }

  // Stage x (with the optional RMSNorm prologue) into xs4 -- at least
  // tiles * 64*U*CH floats -- then stream the remaining tiles and write the
  // outputs.  red holds AMMON_WAVES floats.  Contains barriers: call
  // uniformly.
  AMMON_DEV void run(float4 *xs4, float *red) {
    float *xs = (float *)xs4;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    // The first block's epilogue operands are requested before x is staged,
    // so a one-block workgroup does not wait on them after its last tile.
    uint32_t pos = 0;
    if (MODE == AMMON_GEMV_QKV) pos = p.step->position;
    epi_load(wg, pos, pre_a, pre_b);

    auto xi = [&](uint32_t j) -> uint32_t { return xq(j >> 2) * 4 + (j & 3u); };

    // ---- stage x, optional RMSNorm prologue ------------------------------
    // x was requested in begin(), ahead of the weight tiles.
    const bool xvec = (n & 3u) == 0 && (((uintptr_t)p.x) & 15u) == 0;
    const bool wvec = p.norm_w == nullptr ||
                      (((uintptr_t)p.norm_w) & (p.norm_dtype == AMMON_K_BF16 ? 7u : 15u)) == 0;
    if (xpath == X_DMA) {
      // this wave's x requests have landed: only the two tiles' requests
      // (issued after them) may be outstanding
      wait_vmcnt<2 * RPW * U>();
    } else if (xpath == X_REG) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < XREG; ++i) {
        const uint32_t c = tid + i * AMMON_WG;
        if (c < n / 4) {
          ss += xr[i].x * xr[i].x;
          ss += xr[i].y * xr[i].y;
          ss += xr[i].z * xr[i].z;
          ss += xr[i].w * xr[i].w;
        }
      }
      float s = 1.f;
      if (p.norm_w) {
        ss = block_sum(ss, red);
        ss = ss / (float)n;
        ss = ss + p.eps;
        s = 1.0f / sqrtf(ss);
      }
#pragma unroll
      for (int i = 0; i < XREG; ++i) {
        const uint32_t c = tid + i * AMMON_WG;
        if (c < n / 4) {
          float4 v = xr[i];
          if (p.norm_w) {
            const float4 w4 = p.norm_dtype == AMMON_K_BF16
                                  ? make_float4(bf16_lo(wb[i].x), bf16_hi(wb[i].x),
                                                bf16_lo(wb[i].y), bf16_hi(wb[i].y))
                                  : wr[i];
            v = make_float4(w4.x * (s * v.x), w4.y * (s * v.y), w4.z * (s * v.z),
                            w4.w * (s * v.w));
          }
          xs4[xq(c)] = v;
        }
      }
    } else {
      float ss = 0.f;
      if (xvec) {
        // 16-byte loads, several in flight per lane
#pragma unroll 4
        for (uint32_t c = tid; c < n / 4; c += AMMON_WG) {
          const float4 v = ld_in4(p.x + 4 * c);
          xs4[xq(c)] = v;
          ss += v.x * v.x;
          ss += v.y * v.y;
          ss += v.z * v.z;
          ss += v.w * v.w;
        }
      } else {
        for (uint32_t j = tid; j < n; j += AMMON_WG) {
          const float v = ld_in(p.x + j);
          xs[xi(j)] = v;
          ss += v * v;
        }
      }
      if (p.norm_w) {
        ss = block_sum(ss, red);
        ss = ss / (float)n;
        ss = ss + p.eps;
        const float s = 1.0f / sqrtf(ss);
        if (xvec && wvec) {
          // each lane scales the quads it staged, 16-byte weight loads
          // several in flight (a scalar pass, one load per element, made the
          // dim-8192 layer + LM head step 0.662 ms against 0.647)
#pragma unroll 4
          for (uint32_t c = tid; c < n / 4; c += AMMON_WG) {
            float4 w4;
            if (p.norm_dtype == AMMON_K_BF16) {
              const uint2 wb = ((const uint2 *)p.norm_w)[c];
              w4 = make_float4(bf16_lo(wb.x), bf16_hi(wb.x), bf16_lo(wb.y), bf16_hi(wb.y));
            } else {
              w4 = ((const float4 *)p.norm_w)[c];
            }
            const float4 v = xs4[xq(c)];
            xs4[xq(c)] = make_float4(w4.x * (s * v.x), w4.y * (s * v.y), w4.z * (s * v.z),
                                     w4.w * (s * v.w));
          }
        } else {
          for (uint32_t j = tid; j < n; j += AMMON_WG)
            xs[xi(j)] = load_elem(p.norm_w, p.norm_dtype, j) * (s * xs[xi(j)]);
        }
      }
    }
    // zero padding up to whole tiles (the matching weight chunks read as 0)
    for (uint32_t j = n + tid; j < tiles * tile_chunks * CH; j += AMMON_WG) xs[xi(j)] = 0.f;
    __syncthreads();

    // PLAIN with a step: the reference's position-strided gemv
    // (src/kernels.rs:49-73) writes row `position` of a [seq, d] output.
    float *yout = p.y;
    bool write_ok = true;
    if (MODE == AMMON_GEMV_PLAIN && p.step) {
      const uint32_t ps = p.step->position;
      write_ok = ps < p.seq;
      yout = p.y + (size_t)(write_ok ? ps : 0) * p.d;
    }

    float acc[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) acc[k] = 0.f;
    float cand_v = 0.f;  // PLAIN_ARGMAX: this lane's best row so far
    uint32_t cand_i = ARGMAX_NONE;

    auto compute = [&](uint32_t ti_, V (&buf)[RPW][U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t c = ti_ * tile_chunks + u * 64 + lane;
        float xv[CH];
        if (CH >= 4) {
#pragma unroll
          for (int h = 0; h < CH / 4; ++h) {
            const float4 v = xs4[xq(c * (CH / 4) + h)];
            xv[4 * h] = v.x;
            xv[4 * h + 1] = v.y;
            xv[4 * h + 2] = v.z;
            xv[4 * h + 3] = v.w;
          }
        } else {
          xv[0] = xs[c];
        }
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
          float wf[CH];
          C::widen(buf[k][u], wf);
          float s = acc[k];
#pragma unroll
          for (int e = 0; e < CH; ++e) s += wf[e] * xv[e];
          acc[k] = s;
        }
      }
    };

    // Row-block epilogue (lane k handles row k / pair k).
    auto finish = [&](uint32_t blk_) {
      const uint32_t r0 = (blk_ * AMMON_WAVES + wave_u) * RPW;
      float ea[RPW], eb[RPW];
      if (blk_ == wg) {
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
          ea[k] = pre_a[k];
          eb[k] = pre_b[k];
        }
      } else {
        epi_load(blk_, pos, ea, eb);
      }
#pragma unroll
      for (int k = 0; k < RPW; ++k) acc[k] = wave_sum(acc[k]);
      if (MODE == AMMON_GEMV_PLAIN || MODE == AMMON_GEMV_RESIDUAL ||
          MODE == AMMON_GEMV_PLAIN_ARGMAX) {
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
          const uint32_t vr = r0 + k;
          if ((uint32_t)k == lane && vr < p.rows) {
            if (MODE == AMMON_GEMV_RESIDUAL) {
              st_out(p.y + vr, ea[k] + acc[k]);
            } else if (MODE == AMMON_GEMV_PLAIN_ARGMAX) {
              st_out(p.y + vr, acc[k]);
              if (acc[k] == acc[k]) cand_merge(cand_v, cand_i, acc[k], vr);
            } else if (write_ok) {
              st_out(yout + vr, acc[k]);
            }
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
            st_out(p.y + (vr >> 1), v);
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
            if (vr < p.d) {
              st_out(p.y + vr, __uint_as_float(0x7fc00000u));
              st_out(p.y + vr + 1, __uint_as_float(0x7fc00000u));
            }
            continue;
          }
          if (vr < p.d + p.kv_dim) {
            const uint32_t rr = vr < p.d ? vr : vr - p.d;
            const uint32_t hd = rr % p.head;
            const float fcr = ea[k], fci = eb[k];
            const float o0 = a0 * fcr - a1 * fci;
            const float o1 = a0 * fci + a1 * fcr;
            if (vr < p.d) {
              st_out(p.y + vr, o0);
              st_out(p.y + vr + 1, o1);
            } else {
              const size_t dst = ((size_t)(rr / p.head) * p.seq + pos) * p.head + hd;
              store_pair_out(p.k_cache, p.kv_dtype, dst, o0, o1);
            }
          } else {
            const uint32_t rv = vr - p.d - p.kv_dim;
            const size_t dst = ((size_t)(rv / p.head) * p.seq + pos) * p.head + rv % p.head;
            store_pair_out(p.v_cache, p.kv_dtype, dst, a0, a1);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < RPW; ++k) acc[k] = 0.f;
    };

    // Two-stage pipeline: compute one buffer, then refill it with the tile
    // two ahead, so the other buffer's loads stay in flight meanwhile.
    // Unrolled so each buffer keeps a fixed role.  The steady state runs
    // while both refills are real tiles (loads unconditional, so the wait
    // counts stay exact); the last one to three tiles run without refills
    // past the end -- those would return only zeros, yet the wave could not
    // retire before they came back.
    uint32_t blk2 = blk1, ti2 = ti1;
    advance(blk2, ti2, tiles, nwg);
    auto shift = [&] {
      blk = blk1;
      ti = ti1;
      blk1 = blk2;
      ti1 = ti2;
      advance(blk2, ti2, tiles, nwg);
    };
    const uint32_t total = (wg < p.row_blocks ? (p.row_blocks - 1 - wg) / nwg + 1 : 0) * tiles;
    uint32_t i = 0;
    for (; i + 3 < total; i += 2) {
      compute(ti, bufA);
      if (ti + 1 == tiles) finish(blk);
      load_tile(blk2, ti2, bufA);
      shift();
      compute(ti, bufB);
      if (ti + 1 == tiles) finish(blk);
      load_tile(blk2, ti2, bufB);
      shift();
    }
    if (i < total) {
      compute(ti, bufA);
      if (ti + 1 == tiles) finish(blk);
      if (i + 2 < total) load_tile(blk2, ti2, bufA);
      shift();
      if (i + 1 < total) {
        compute(ti, bufB);
        if (ti + 1 == tiles) finish(blk);
        shift();
        if (i + 2 < total) {
          compute(ti, bufA);
          if (ti + 1 == tiles) finish(blk);
        }
      }
    }
    if (MODE == AMMON_GEMV_PLAIN_ARGMAX) {
      // the workgroup's candidate; x's LDS is free once every wave is done
      __syncthreads();
      float *sv = xs;
      uint32_t *si = (uint32_t *)(xs + AMMON_WG);
      block_cand_reduce(cand_v, cand_i, sv, si);
      if (threadIdx.x == 0) {
        st_out(p.cand_v + wg, cand_v);
        st_out(p.cand_i + wg, cand_i);
      }
    }
  }
};
