// noalloc.hip -- the decode attention pair (split partials + log-sum-exp
// merge) with a library-owned scratch buffer, for callers that cannot
// allocate device memory: code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc.
//
// ammon_attention_decode takes its split partials [q_heads, splits, head + 2]
// fp32 from a caller buffer.  ammon_attention_decode_noalloc runs the same
// two kernels with the partials in `scratch`, a file-scope device array of
// AMMON_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until
// the process ends.  Its device address is looked up once per device, with
// that device current, when ammon_runtime_create first sets the device up;
// host code uses only that address, never the array's name (which on the
// host is a stand-in symbol, not device memory).
//
// The entry point allocates nothing: no hipMalloc, hipFree or allocating
// library routine.  Nothing in the scratch needs to start at zero (the merge
// uses only the splits the partial pass wrote for the current position).
// Every call on one GPU shares that GPU's array, so calls that can overlap on
// one GPU (different streams, no ordering between them) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.h"

static __device__ __align__(256) unsigned char scratch[AMMON_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices] = {};
}  // namespace

namespace ammon_rt {

// Called by runtime set-up with `device` current.
ammon_status noalloc_init(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(AMMON_E_NO_DEVICE, "device %d beyond the %d the scratch table covers", device,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device]) return AMMON_OK;
  void *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
  if (!ptr) return set_error(AMMON_E_HIP, "hipGetSymbolAddress(scratch) returned NULL");
  g_scratch[device] = ptr;
  return AMMON_OK;
}

}  // namespace ammon_rt

extern "C" ammon_status ammon_attention_decode_noalloc(
    ammon_runtime *rt, ammon_stream stream, const float *q, uint32_t q_heads,
    const void *k_cache, const void *v_cache, ammon_dtype kv_dtype, uint32_t kv_heads,
    uint32_t head, uint32_t seq, const ammon_decode_step *step, uint32_t split_len, float *out) {
  AMMON_CHECK(rt != nullptr, "runtime is NULL");
  AMMON_CHECK(split_len >= 1 && split_len <= AMMON_ATTENTION_MAX_SPLIT,
              "attention_decode_noalloc: split length %u outside [1, %u]", split_len,
              AMMON_ATTENTION_MAX_SPLIT);
  const size_t need = ammon_attention_scratch_bytes(q_heads, head, seq, split_len);
  AMMON_CHECK(need <= AMMON_NOALLOC_SCRATCH_BYTES,
              "attention_decode_noalloc: the split partials need %zu bytes ([%u, %u, %u] fp32), "
              "above the %u-byte library scratch; use a longer split or ammon_attention_decode "
              "with a caller buffer",
              need, q_heads, ammon_attention_splits(seq, split_len), head + 2,
              (unsigned)AMMON_NOALLOC_SCRATCH_BYTES);
  void *ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (rt->device >= 0 && rt->device < kMaxDevices) ptr = g_scratch[rt->device];
  }
  AMMON_CHECK(ptr != nullptr, "attention_decode_noalloc: scratch of device %d not set up",
              rt->device);
  return ammon_attention_decode(rt, stream, q, q_heads, k_cache, v_cache, kv_dtype, kv_heads,
                                head, seq, step, split_len, (float *)ptr, need, out);
}
