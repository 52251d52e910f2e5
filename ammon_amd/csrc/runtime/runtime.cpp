// runtime.cpp -- device bootstrap, per-device prepared-kernel cache, memory,
// streams, events and host utilities of the C ABI.
//
// The reference prepares its kernels once per Goldy runtime and shares them
// through a global mutex-guarded cache of weak references keyed by the
// runtime (reference src/blocks.rs:72-86,322).  Here the cache is keyed by
// device ordinal: the first ammon_runtime_create for a device loads the
// embedded gfx950 code objects with hipModuleLoadData and resolves every
// kernel once; later creates share it; the last release unloads it.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "internal.h"

// Code objects embedded by blobs.s (one per kernels/*.hip).
#define AMMON_BLOB(name) extern "C" const char ammon_co_##name[], ammon_co_##name##_end[];
AMMON_BLOB(embed)
AMMON_BLOB(norm)
AMMON_BLOB(rope)
AMMON_BLOB(attention)
AMMON_BLOB(gemv)
AMMON_BLOB(misc)
AMMON_BLOB(prefill)

namespace ammon_rt {

static thread_local std::string g_last_error;

ammon_status set_error(ammon_status st, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

ammon_status hip_error(hipError_t e, const char *what) {
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    return set_error(AMMON_E_OOM, "%s: %s", what, hipGetErrorString(e));
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
    return set_error(AMMON_E_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
  return set_error(AMMON_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

uint32_t occupancy(ammon_runtime *rt, hipFunction_t f, size_t shmem) {
  std::lock_guard<std::mutex> lock(rt->occ_mu);
  const auto key = std::make_pair(f, shmem);
  auto it = rt->occ_cache.find(key);
  if (it != rt->occ_cache.end()) return it->second;
  int blocks = 0;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, f, 256, shmem) != hipSuccess ||
      blocks < 1)
    blocks = 1;
  rt->occ_cache[key] = (uint32_t)blocks;
  return (uint32_t)blocks;
}

static std::mutex g_mu;
static std::map<int, ammon_runtime *> g_runtimes;

static ammon_status resolve(hipModule_t mod, const char *name, hipFunction_t *out) {
  hipError_t e = hipModuleGetFunction(out, mod, name);
  if (e != hipSuccess) return set_error(AMMON_E_HIP, "kernel %s not found: %s", name, hipGetErrorString(e));
  return AMMON_OK;
}

static ammon_status load_kernels(ammon_runtime *rt) {
  struct Blob {
    const char *name;
    const char *data;
  } blobs[] = {{"embed", ammon_co_embed}, {"norm", ammon_co_norm},
               {"rope", ammon_co_rope},   {"attention", ammon_co_attention},
               {"gemv", ammon_co_gemv},   {"misc", ammon_co_misc},
               {"prefill", ammon_co_prefill}};
  constexpr int kModules = (int)(sizeof(blobs) / sizeof(blobs[0]));
  hipModule_t mods[kModules];
  for (int i = 0; i < kModules; ++i) {
    hipError_t e = hipModuleLoadData(&mods[i], blobs[i].data);
    if (e != hipSuccess)
      return set_error(AMMON_E_HIP, "load code object %s: %s", blobs[i].name, hipGetErrorString(e));
    rt->modules.push_back(mods[i]);
  }
  Kernels &k = rt->k;
  ammon_status st;
#define R(mod, name, dst) \
  if ((st = resolve(mods[mod], name, &(dst))) != AMMON_OK) return st;
  R(0, "ammon_embed", k.embed);
  R(1, "ammon_rmsnorm", k.rmsnorm);
  R(2, "ammon_rope", k.rope);
  R(2, "ammon_cache_store", k.cache_store);
  R(3, "ammon_attention_combine", k.att_combine);
  R(3, "ammon_attention_combine_waves", k.att_combine_waves);
  const char *dtn[2] = {"f32", "bf16"};
  const int chs[kAttChunks] = {8, 4, 2, 1};
  const int gs[kAttGroups] = {1, 2, 4, 8};
  for (int d = 0; d < 2; ++d)
    for (int c = 0; c < kAttChunks; ++c) {
      if (d == 0 && chs[c] == 8) continue;  // no 8-wide fp32 chunk
      for (int g = 0; g < kAttGroups; ++g) {
        char name[96];
        snprintf(name, sizeof name, "ammon_attention_partial_%s_c%d_g%d", dtn[d], chs[c], gs[g]);
        R(3, name, k.att_partial[d][c][g]);
      }
    }
  for (int g = 0; g < kAttGroups; ++g) {
    char name[96];
    snprintf(name, sizeof name, "ammon_attention_partial_h128_f32_c4_g%d", gs[g]);
    R(3, name, k.att_partial_h128_f32[g]);
  }
  for (int b = 0; b < 2; ++b)
    for (int g = 0; g < kAttGroups; ++g) {
      char name[96];
      snprintf(name, sizeof name, "ammon_attention_partial_h128_bf16_lds%d_g%d", 1 << b, gs[g]);
      R(3, name, k.att_partial_staged[b][g]);
    }
  const char *modes[kGemvModes] = {"plain", "residual", "swiglu", "qkv"};
  for (int d = 0; d < 2; ++d)
    for (int v = 0; v < 2; ++v)
      for (int m = 0; m < kGemvModes; ++m) {
        char name[96];
        snprintf(name, sizeof name, "ammon_gemv_%s_%s_%s", dtn[d], v ? "v" : "s", modes[m]);
        R(4, name, k.gemv[d][v][m]);
      }
  for (int d = 0; d < 2; ++d)
    for (int v = 0; v < 2; ++v) {
      char name[96];
      snprintf(name, sizeof name, "ammon_gemv_%s_%s_plain_argmax", dtn[d], v ? "v" : "s");
      R(4, name, k.gemv_argmax[d][v]);
    }
  R(4, "ammon_gemv_bf16_w_plain", k.gemv_wide[0]);
  R(4, "ammon_gemv_bf16_w_plain_argmax", k.gemv_wide[1]);
  R(5, "ammon_swiglu", k.swiglu);
  R(5, "ammon_add", k.add);
  R(5, "ammon_argmax_partial", k.argmax_partial);
  R(5, "ammon_argmax_final", k.argmax_final);
  R(5, "ammon_fill_normal", k.fill_normal);
  R(5, "ammon_fill_const", k.fill_const);
  R(5, "ammon_checksum", k.checksum);
  R(5, "ammon_stream_read", k.stream_read);
  for (int d = 0; d < 2; ++d)
    for (int t = 0; t < 2; ++t)
      for (int s = 0; s < 2; ++s)
        for (int m = 0; m < kGemvModes; ++m) {
          char name[96];
          snprintf(name, sizeof name, "ammon_gemm_%s_%s_t%d%s", dtn[d], modes[m], t ? 32 : 16,
                   s ? "_k4" : "");
          R(6, name, k.gemm[d][t][s][m]);
        }
  R(6, "ammon_gemm_reduce", k.gemm_reduce);
  R(6, "ammon_gemm_reduce_qkv", k.gemm_reduce_qkv);
  for (int t = 0; t < 2; ++t)
    for (int r = 0; r < 2; ++r)
      for (int m = 0; m < kGemvModes; ++m) {
        char name[96];
        snprintf(name, sizeof name, "ammon_gemm_bf16_%s_t%d_r%d", modes[m], t ? 32 : 64,
                 r ? 2 : 4);
        R(6, name, k.gemm_big[t][r][m]);
      }
#undef R
  return AMMON_OK;
}

static void destroy(ammon_runtime *rt) {
  // Teardown is best effort: errors here have no caller to report to.
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(rt->device);
  if (rt->stream) (void)hipStreamDestroy(rt->stream);
  for (hipModule_t m : rt->modules) (void)hipModuleUnload(m);
  (void)hipSetDevice(prev);
  delete rt;
}

static ammon_status create(int device, ammon_runtime **out) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return set_error(AMMON_E_NO_DEVICE, "no HIP device available (%s)", hipGetErrorString(e));
  if (device < 0 || device >= count)
    return set_error(AMMON_E_NO_DEVICE, "device %d out of range (%d devices)", device, count);
  AMMON_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  AMMON_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(AMMON_E_NO_DEVICE, "device %d is %s; libammon_amd targets gfx950 only", device,
                     prop.gcnArchName);
  ammon_runtime *rt = new ammon_runtime();
  rt->device = device;
  rt->info.device = device;
  rt->info.compute_units = prop.multiProcessorCount;
  rt->info.max_shared_per_block = (int)prop.sharedMemPerBlock;
  int optin = 0;
  if (hipDeviceGetAttribute(&optin, hipDeviceAttributeSharedMemPerBlockOptin, device) == hipSuccess &&
      optin > rt->info.max_shared_per_block)
    rt->info.max_shared_per_block = optin;
  rt->info.warp_size = prop.warpSize;
  rt->info.total_memory = prop.totalGlobalMem;
  std::snprintf(rt->info.arch, sizeof rt->info.arch, "%.63s", prop.gcnArchName);
  std::snprintf(rt->info.name, sizeof rt->info.name, "%.127s", prop.name);
  if (const char *env = std::getenv("AMMON_GEMM_SPLIT")) {
    const int v = std::atoi(env);
    if (v == 0 || v == 1) rt->gemm_split = v;
  }
  if (const char *env = std::getenv("AMMON_GEMM_BIG")) {
    const int v = std::atoi(env);
    if (v == 0 || v == 44 || v == 42 || v == 24 || v == 22) rt->gemm_big = v;
  }
  if (const char *env = std::getenv("AMMON_GEMV_WGS_PER_CU")) {
    int v = std::atoi(env);
    if (v > 0 && v <= 64) rt->gemv_wgs_per_cu = (uint32_t)v;
  }
  ammon_status st = load_kernels(rt);
  if (st == AMMON_OK) st = noalloc_init(device);  // device is current
  if (st == AMMON_OK) {
    e = hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking);
    if (e != hipSuccess) st = hip_error(e, "hipStreamCreateWithFlags");
  }
  if (st != AMMON_OK) {
    destroy(rt);
    return st;
  }
  *out = rt;
  return AMMON_OK;
}

}  // namespace ammon_rt

using namespace ammon_rt;

extern "C" {

int ammon_abi_version(void) { return AMMON_ABI_VERSION; }

const char *ammon_last_error(void) { return g_last_error.c_str(); }

ammon_status ammon_runtime_create(int device, ammon_runtime **out) {
  AMMON_CHECK(out != nullptr, "ammon_runtime_create: out is NULL");
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_runtimes.find(device);
  if (it != g_runtimes.end()) {
    it->second->refs += 1;
    *out = it->second;
    return AMMON_OK;
  }
  ammon_runtime *rt = nullptr;
  ammon_status st = create(device, &rt);
  if (st != AMMON_OK) return st;
  rt->refs = 1;
  g_runtimes[device] = rt;
  *out = rt;
  return AMMON_OK;
}

ammon_status ammon_runtime_release(ammon_runtime *rt) {
  AMMON_CHECK(rt != nullptr, "ammon_runtime_release: runtime is NULL");
  std::lock_guard<std::mutex> lock(g_mu);
  if (--rt->refs > 0) return AMMON_OK;
  g_runtimes.erase(rt->device);
  destroy(rt);
  return AMMON_OK;
}

ammon_status ammon_runtime_info(ammon_runtime *rt, ammon_device_info *out) {
  AMMON_CHECK(rt && out, "ammon_runtime_info: NULL argument");
  *out = rt->info;
  return AMMON_OK;
}

ammon_status ammon_alloc(ammon_runtime *rt, size_t bytes, void **dptr) {
  AMMON_CHECK(rt && dptr, "ammon_alloc: NULL argument");
  AMMON_HIP(hipSetDevice(rt->device));
  *dptr = nullptr;
  if (bytes == 0) return AMMON_OK;
  AMMON_HIP(hipMalloc(dptr, bytes));
  return AMMON_OK;
}

ammon_status ammon_free(ammon_runtime *rt, void *dptr) {
  AMMON_CHECK(rt != nullptr, "ammon_free: runtime is NULL");
  if (!dptr) return AMMON_OK;
  AMMON_HIP(hipSetDevice(rt->device));
  AMMON_HIP(hipFree(dptr));
  return AMMON_OK;
}

ammon_status ammon_alloc_host(ammon_runtime *rt, size_t bytes, void **hptr) {
  AMMON_CHECK(rt && hptr, "ammon_alloc_host: NULL argument");
  AMMON_HIP(hipSetDevice(rt->device));
  *hptr = nullptr;
  if (bytes == 0) return AMMON_OK;
  AMMON_HIP(hipHostMalloc(hptr, bytes, hipHostMallocDefault));
  return AMMON_OK;
}

ammon_status ammon_free_host(ammon_runtime *rt, void *hptr) {
  AMMON_CHECK(rt != nullptr, "ammon_free_host: runtime is NULL");
  if (!hptr) return AMMON_OK;
  AMMON_HIP(hipHostFree(hptr));
  return AMMON_OK;
}

static hipStream_t pick(ammon_runtime *rt, ammon_stream s) {
  return s ? (hipStream_t)s : rt->stream;
}

ammon_status ammon_memcpy(ammon_runtime *rt, void *dst, const void *src, size_t bytes,
                          ammon_copy_kind kind, ammon_stream stream) {
  AMMON_CHECK(rt != nullptr, "ammon_memcpy: runtime is NULL");
  AMMON_CHECK(stream != AMMON_STREAM_VALIDATE, "ammon_memcpy: validate-only stream");
  if (bytes == 0) return AMMON_OK;
  AMMON_CHECK(dst && src, "ammon_memcpy: NULL pointer");
  hipMemcpyKind k;
  switch (kind) {
    case AMMON_COPY_H2D: k = hipMemcpyHostToDevice; break;
    case AMMON_COPY_D2H: k = hipMemcpyDeviceToHost; break;
    case AMMON_COPY_D2D: k = hipMemcpyDeviceToDevice; break;
    default: return set_error(AMMON_E_VALIDATION, "ammon_memcpy: bad copy kind %d", (int)kind);
  }
  AMMON_HIP(hipSetDevice(rt->device));
  AMMON_HIP(hipMemcpyAsync(dst, src, bytes, k, pick(rt, stream)));
  return AMMON_OK;
}

ammon_status ammon_stream_create(ammon_runtime *rt, ammon_stream *out) {
  AMMON_CHECK(rt && out, "ammon_stream_create: NULL argument");
  AMMON_HIP(hipSetDevice(rt->device));
  hipStream_t s;
  AMMON_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = (ammon_stream)s;
  return AMMON_OK;
}

ammon_status ammon_stream_destroy(ammon_runtime *rt, ammon_stream stream) {
  AMMON_CHECK(rt && stream && stream != AMMON_STREAM_VALIDATE, "ammon_stream_destroy: bad stream");
  AMMON_HIP(hipStreamDestroy((hipStream_t)stream));
  return AMMON_OK;
}

ammon_status ammon_stream_synchronize(ammon_runtime *rt, ammon_stream stream) {
  AMMON_CHECK(rt != nullptr, "ammon_stream_synchronize: runtime is NULL");
  AMMON_CHECK(stream != AMMON_STREAM_VALIDATE, "ammon_stream_synchronize: validate-only stream");
  AMMON_HIP(hipStreamSynchronize(pick(rt, stream)));
  return AMMON_OK;
}

ammon_status ammon_event_create(ammon_runtime *rt, ammon_event *out) {
  AMMON_CHECK(rt && out, "ammon_event_create: NULL argument");
  AMMON_HIP(hipSetDevice(rt->device));
  hipEvent_t ev;
  AMMON_HIP(hipEventCreate(&ev));
  *out = (ammon_event)ev;
  return AMMON_OK;
}

ammon_status ammon_event_destroy(ammon_runtime *rt, ammon_event ev) {
  AMMON_CHECK(rt && ev, "ammon_event_destroy: NULL argument");
  AMMON_HIP(hipEventDestroy((hipEvent_t)ev));
  return AMMON_OK;
}

ammon_status ammon_event_record(ammon_runtime *rt, ammon_event ev, ammon_stream stream) {
  AMMON_CHECK(rt && ev, "ammon_event_record: NULL argument");
  AMMON_CHECK(stream != AMMON_STREAM_VALIDATE, "ammon_event_record: validate-only stream");
  AMMON_HIP(hipEventRecord((hipEvent_t)ev, pick(rt, stream)));
  return AMMON_OK;
}

ammon_status ammon_event_synchronize(ammon_runtime *rt, ammon_event ev) {
  AMMON_CHECK(rt && ev, "ammon_event_synchronize: NULL argument");
  AMMON_HIP(hipEventSynchronize((hipEvent_t)ev));
  return AMMON_OK;
}

ammon_status ammon_event_elapsed_ms(ammon_runtime *rt, ammon_event start, ammon_event stop,
                                    float *ms) {
  AMMON_CHECK(rt && start && stop && ms, "ammon_event_elapsed_ms: NULL argument");
  AMMON_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return AMMON_OK;
}

// ---- launch-list capture -------------------------------------------------------

struct GraphHandle {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

ammon_status ammon_capture_begin(ammon_runtime *rt, ammon_stream stream) {
  AMMON_CHECK(rt != nullptr, "capture_begin: runtime is NULL");
  AMMON_CHECK(stream != AMMON_STREAM_VALIDATE, "capture_begin: validate-only stream");
  AMMON_HIP(hipSetDevice(rt->device));
  AMMON_HIP(hipStreamBeginCapture(pick(rt, stream), hipStreamCaptureModeThreadLocal));
  return AMMON_OK;
}

ammon_status ammon_capture_end(ammon_runtime *rt, ammon_stream stream, ammon_graph *out) {
  AMMON_CHECK(rt && out, "capture_end: NULL argument");
  AMMON_CHECK(stream != AMMON_STREAM_VALIDATE, "capture_end: validate-only stream");
  GraphHandle *g = new GraphHandle();
  hipError_t e = hipStreamEndCapture(pick(rt, stream), &g->graph);
  if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return hip_error(e, "capture_end");
  }
  *out = (ammon_graph)g;
  return AMMON_OK;
}

ammon_status ammon_graph_launch(ammon_runtime *rt, ammon_graph graph, ammon_stream stream) {
  AMMON_CHECK(rt && graph, "graph_launch: NULL argument");
  AMMON_CHECK(stream != AMMON_STREAM_VALIDATE, "graph_launch: validate-only stream");
  AMMON_HIP(hipGraphLaunch(((GraphHandle *)graph)->exec, pick(rt, stream)));
  return AMMON_OK;
}

ammon_status ammon_graph_destroy(ammon_runtime *rt, ammon_graph graph) {
  AMMON_CHECK(rt != nullptr, "graph_destroy: runtime is NULL");
  if (!graph) return AMMON_OK;
  GraphHandle *g = (GraphHandle *)graph;
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
  return AMMON_OK;
}

// ---- host utilities ----------------------------------------------------------

size_t ammon_rope_table_bytes(uint32_t head, uint32_t seq) {
  return (size_t)seq * (head / 2) * 2 * sizeof(float);
}

// The reference's per-lane formula (src/kernels.rs:195-199), evaluated once
// per (position, pair) on the host in fp32 with libm's powf / cosf / sinf.
ammon_status ammon_rope_table_host(float theta, uint32_t head, uint32_t seq, float *table) {
  AMMON_CHECK(table != nullptr, "rope table: output is NULL");
  AMMON_CHECK(head >= 2 && head % 2 == 0, "rope table: head %u must be even and >= 2", head);
  AMMON_CHECK(theta > 0.0f, "rope table: theta must be positive");
  const uint32_t half = head / 2;
  for (uint32_t pos = 0; pos < seq; ++pos)
    for (uint32_t p = 0; p < half; ++p) {
      const uint32_t hd = (2 * p) % head;
      const float freq = 1.0f / powf(theta, (float)hd / (float)head);
      const float val = (float)pos * freq;
      table[((size_t)pos * half + p) * 2 + 0] = cosf(val);
      table[((size_t)pos * half + p) * 2 + 1] = sinf(val);
    }
  return AMMON_OK;
}

static ammon_status kv_move(const void *src, void *dst, uint32_t kv_heads, uint32_t seq,
                            uint32_t head, uint32_t elem, bool to_pos_major) {
  AMMON_CHECK(src && dst, "kv permute: NULL argument");
  AMMON_CHECK(elem == 2 || elem == 4, "kv permute: elem_bytes must be 2 or 4");
  const size_t row = (size_t)head * elem;
  for (uint32_t g = 0; g < kv_heads; ++g)
    for (uint32_t t = 0; t < seq; ++t) {
      const size_t hm = ((size_t)g * seq + t) * row;
      const size_t pm = ((size_t)t * kv_heads + g) * row;
      if (to_pos_major)
        std::memcpy((char *)dst + pm, (const char *)src + hm, row);
      else
        std::memcpy((char *)dst + hm, (const char *)src + pm, row);
    }
  return AMMON_OK;
}

ammon_status ammon_kv_unpermute(const void *head_major, void *pos_major, uint32_t kv_heads,
                                uint32_t seq, uint32_t head, uint32_t elem_bytes) {
  return kv_move(head_major, pos_major, kv_heads, seq, head, elem_bytes, true);
}

ammon_status ammon_kv_permute(const void *pos_major, void *head_major, uint32_t kv_heads,
                              uint32_t seq, uint32_t head, uint32_t elem_bytes) {
  return kv_move(pos_major, head_major, kv_heads, seq, head, elem_bytes, false);
}

uint32_t ammon_attention_splits(uint32_t seq, uint32_t split_len) {
  if (split_len == 0) return 0;
  const uint32_t s = (uint32_t)(((uint64_t)seq + split_len - 1) / split_len);
  return s ? s : 1;
}

size_t ammon_attention_scratch_bytes(uint32_t q_heads, uint32_t head, uint32_t seq,
                                     uint32_t split_len) {
  return (size_t)q_heads * ammon_attention_splits(seq, split_len) * (head + 2) * sizeof(float);
}

// Aim for about two workgroups per CU at full context: the partial kernel
// pipelines two chunks of K and V (64 positions of a 128-wide bf16 head
// each) through registers, so a workgroup overlaps its own loads and
// arithmetic.  Splits stay between 16 and AMMON_ATTENTION_MAX_SPLIT
// positions and the count under AMMON_ATTENTION_MAX_SPLITS.  A cache of at
// most kSingleSplitSeq positions takes one split: the decode is then one
// launch (pass 1 writes the merged output), which at that size saves more
// than the split-level parallelism costs (the 6-layer dim-288 fp32 decoder
// at 256 positions: 7921 against 7056 tokens/s).
static constexpr uint32_t kSingleSplitSeq = 256;
uint32_t ammon_attention_default_split(ammon_runtime *rt, uint32_t kv_heads, uint32_t seq) {
  return ammon_rt::default_split(rt, kv_heads, seq, 2);
}

}  // extern "C"

namespace ammon_rt {

// The shortest power-of-two split from min_split (a power of two) up whose
// kv_heads * splits units fit in units_per_cu units per CU (and under the
// split-count limit).
uint32_t default_split(ammon_runtime *rt, uint32_t kv_heads, uint32_t seq,
                       uint32_t units_per_cu, uint32_t min_split) {
  if (seq >= 1 && seq <= kSingleSplitSeq) return seq;
  const uint32_t cus = rt ? (uint32_t)rt->info.compute_units : 256u;
  const uint64_t target_wgs = (uint64_t)std::max(units_per_cu, 1u) * (cus ? cus : 256u);
  uint32_t split = std::min<uint32_t>(std::max<uint32_t>(min_split, 1), AMMON_ATTENTION_MAX_SPLIT);
  while (split < AMMON_ATTENTION_MAX_SPLIT &&
         ((uint64_t)kv_heads * ammon_attention_splits(seq, split) > target_wgs ||
          ammon_attention_splits(seq, split) > AMMON_ATTENTION_MAX_SPLITS))
    split *= 2;
  return split;
}

}  // namespace ammon_rt
