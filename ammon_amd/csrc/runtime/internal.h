// internal.h -- shared state of the C-ABI implementation (host side only).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../kernel_params.h"
#include "ammon/ammon.h"

namespace ammon_rt {

// Attention partial variants: [kv dtype][chunk index][G index].
constexpr int kAttChunks = 4;  // CH = 8, 4, 2, 1
constexpr int kAttGroups = 4;  // GMAX = 1, 2, 4, 8
// GEMV variants: [weight dtype][vector?][mode].
constexpr int kGemvModes = 4;

struct Kernels {
  hipFunction_t embed = nullptr;
  hipFunction_t rmsnorm = nullptr;
  hipFunction_t rope = nullptr;
  hipFunction_t cache_store = nullptr;
  hipFunction_t att_partial[2][kAttChunks][kAttGroups] = {};
  // head-128 specialisations: [dtype][group index], widest chunk only
  // head 128, power-of-two group: fp32 caches on VALU; bf16 caches on
  // matrix cores with K/V staged in an LDS ring of 1 or 2 chunk buffers
  hipFunction_t att_partial_h128_f32[kAttGroups] = {};
  hipFunction_t att_partial_staged[2][kAttGroups] = {};
  hipFunction_t att_combine = nullptr;
  hipFunction_t att_combine_waves = nullptr;  // one wave per (token, q head)
  hipFunction_t gemv[2][2][kGemvModes] = {};
  hipFunction_t gemv_argmax[2][2] = {};  // PLAIN_ARGMAX: [dtype][vector?]
  hipFunction_t gemv_wide[2] = {};       // bf16 vector, kGemvWideRowsPerWave: [plain, argmax]
  hipFunction_t swiglu = nullptr;
  hipFunction_t add = nullptr;
  hipFunction_t argmax_partial = nullptr;
  hipFunction_t argmax_final = nullptr;
  hipFunction_t fill_normal = nullptr;
  hipFunction_t fill_const = nullptr;
  hipFunction_t checksum = nullptr;
  hipFunction_t stream_read = nullptr;
  // prefill GEMMs on matrix cores: [weight dtype][16 / 32-token tiles]
  // [row tile per wave / split over the workgroup's waves][mode]
  hipFunction_t gemm[2][2][2][kGemvModes] = {};
  hipFunction_t gemm_reduce = nullptr;      // split-reduction sum
  hipFunction_t gemm_reduce_qkv = nullptr;  // ... with the QKV epilogue
  // bf16, register-blocked tiles: [64 tokens, 32 tokens][RT 4, RT 2][mode]
  hipFunction_t gemm_big[2][2][kGemvModes] = {};
};

// LDS per compute unit on gfx950 (bytes); bounds resident GEMV workgroups.
constexpr uint32_t kLdsPerCu = 160 * 1024;

// GEMV rows per wave and waves per workgroup (must match gemv.hip).
constexpr uint32_t kGemvRowsPerWave = 2;
// the wide variant (plain / plain_argmax, bf16, 16-byte chunks) for matrices
// of at least kGemvWideMinRows rows of at most kGemvWideMaxRowBytes: the LM
// head at 128256 x 4096 runs 155 against 160 us per launch; at 128256 x
// 8192 the 2-row kernel (up to four workgroups per CU where the wide one's
// registers allow two) is ~36 us faster
constexpr uint32_t kGemvWideRowsPerWave = 4;
constexpr uint32_t kGemvWideMinRows = 65536;
constexpr uint64_t kGemvWideMaxRowBytes = 8192;
constexpr uint32_t kGemvTileChunks = 4;  // U: chunks per lane per tile
constexpr uint32_t kGemvWaves = 4;
constexpr uint32_t kWorkgroup = 256;
constexpr uint32_t kWaves = kWorkgroup / 64;

// Resident workgroups of `f` per CU at 256 threads and `shmem` bytes of
// dynamic LDS (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor, cached).
uint32_t occupancy(ammon_runtime *rt, hipFunction_t f, size_t shmem);
// Attention split length for about units_per_cu pass-1 units per CU at the
// cache length, at least min_split (one split for caches of at most 256
// positions).
uint32_t default_split(ammon_runtime *rt, uint32_t kv_heads, uint32_t seq,
                       uint32_t units_per_cu, uint32_t min_split = 16);

// Makes `device` current for the scope's lifetime.
struct DeviceScope {
  int prev = -1;
  explicit DeviceScope(int device) {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != device) {
      prev = cur;
      (void)hipSetDevice(device);
    }
  }
  ~DeviceScope() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
  DeviceScope(const DeviceScope &) = delete;
  DeviceScope &operator=(const DeviceScope &) = delete;
};

ammon_status set_error(ammon_status st, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
ammon_status hip_error(hipError_t e, const char *what);

// Looks up this device's copy of the library scratch used by
// ammon_attention_decode_noalloc (runtime/noalloc.hip); call once per device
// with that device current.
ammon_status noalloc_init(int device);

}  // namespace ammon_rt

struct ammon_runtime {
  int device = 0;
  int refs = 0;
  hipStream_t stream = nullptr;
  std::vector<hipModule_t> modules;
  ammon_rt::Kernels k;
  ammon_device_info info = {};
  uint32_t gemv_wgs_per_cu = 4;
  int gemm_split = -1;  // prefill GEMM reduction split: -1 by shape, 0 never, 1 always
  // prefill GEMM register-blocked tiles (bf16, >= 64 tokens): -1 by shape,
  // 0 never, else 10 * tokens-per-tile / 16 + 16-row tiles per wave
  // (44, 42, 24, 22)
  int gemm_big = -1;
  std::mutex occ_mu;
  std::map<std::pair<hipFunction_t, size_t>, uint32_t> occ_cache;
};

#define AMMON_HIP(expr)                                            \
  do {                                                             \
    hipError_t _e = (expr);                                        \
    if (_e != hipSuccess) return ammon_rt::hip_error(_e, #expr);   \
  } while (0)

#define AMMON_CHECK(cond, ...)                                                \
  do {                                                                        \
    if (!(cond)) return ammon_rt::set_error(AMMON_E_VALIDATION, __VA_ARGS__); \
  } while (0)
