// grid_sync.h -- grid-wide barrier for kernels whose workgroups are all
// co-resident and hand results to each other inside one launch (the fused
// attention / SwiGLU blocks and the persistent decode-token kernel).
//
// Counters (sync words, AMMON_TOKEN_SYNC_WORDS, zero before a launch): 8
// group counters at sync[64 (1 + grp)] (grp = blockIdx % 8, each on its own
// 256-byte line) and a top counter at sync[0].  Every wave waits for its
// stores to complete, thread 0 counts the workgroup into its group; the
// last arrival of a group bumps the top counter; waiters poll the top
// counter until it reaches 8 k for the k-th barrier.  Polls are bounded: a
// wait that exceeds spin_limit polls sets sync[AMMON_TOKEN_SYNC_ERR] and
// lets the kernel run to its end instead of hanging (results are then
// invalid and the host reports it).  Requires gridDim.x >= 8.
//
// arrive_final() is a last arrival without a wait: the workgroup whose count
// completes it (every other workgroup has passed all earlier waits by then)
// zeroes the counters for the next launch; the error word is left for the
// host.
//
// With a trace buffer, thread 0 of every workgroup stamps the device clock
// when it arrives at and when it leaves each barrier.
#pragma once

#include "device_common.h"

struct GridSync {
  uint32_t *sync;
  uint32_t nwg;
  uint32_t k;  // barriers passed by this workgroup
  uint32_t spin_limit;
  uint64_t *trace;
  uint32_t trace_slots;

  AMMON_DEV void stamp(uint32_t half) const {
    if (trace && k - 1 < trace_slots)
      trace[(size_t)(2 * (k - 1) + half) * nwg + blockIdx.x] = __builtin_amdgcn_s_memrealtime();
  }

  AMMON_DEV uint32_t poll(const uint32_t *a) const {
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Count this workgroup in once its stores have completed; true in the
  // workgroup (thread 0) whose count completed the barrier.
  AMMON_DEV bool count_in() {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are at the coherence point
    __syncthreads();
    ++k;
    bool last = false;
    if (threadIdx.x == 0) {
      const uint32_t grp = blockIdx.x & 7u;
      const uint32_t per = (nwg - grp + 7u) / 8u;  // workgroups in this group
      const uint32_t old =
          __hip_atomic_fetch_add(sync + 64 * (1 + grp), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old + 1 == per * k)
        last = __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 ==
               8u * k;
      stamp(0);
    }
    return last;
  }

  AMMON_DEV void arrive() { (void)count_in(); }

  // Wait until every workgroup has arrived k times.
  AMMON_DEV void wait() {
    if (threadIdx.x == 0) {
      const uint32_t target = 8u * k;
      uint32_t it = 0;
      if (poll(sync + AMMON_TOKEN_SYNC_ERR) == 0) {
        while (poll(sync) < target) {
          if (++it > spin_limit) {
            __hip_atomic_store(sync + AMMON_TOKEN_SYNC_ERR, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
      stamp(1);
    }
    __syncthreads();
  }

  AMMON_DEV void sync_all() {
    arrive();
    wait();
  }

  // The launch's last barrier, without a wait: the completing workgroup
  // zeroes the counters (nobody polls them any more).
  AMMON_DEV void arrive_final() {
    if (count_in() && threadIdx.x == 0) {
#pragma unroll
      for (uint32_t i = 0; i < 9; ++i)
        __hip_atomic_store(sync + 64 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
};
