// argmax_impl.h -- candidate merge of the parallel greedy argmax, shared by
// misc.hip and the LM-head GEMV (gemv_impl.h).
//
// sample_argmax (reference src/tokenizer.rs:179-189) returns the first index
// of the maximum under a strict `>` scan from logits[0]: NaN never wins, and a
// NaN logits[0] yields 0.  In parallel: every non-NaN element is a candidate,
// candidates combine by (larger value, then lower index) -- a total order, so
// the tree shape cannot change the answer -- and the NaN-logits[0] case is
// applied at the end.  +0 and -0 compare equal, as in the scan.
#pragma once

#include "device_common.h"

#define ARGMAX_NONE 0xffffffffu

AMMON_DEV void cand_merge(float &v, uint32_t &i, float v2, uint32_t i2) {
  if (i2 == ARGMAX_NONE) return;
  if (i == ARGMAX_NONE || v2 > v || (!(v > v2) && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// Workgroup reduction of the candidates; sv / si hold AMMON_WG entries of
// LDS.  Contains barriers: call uniformly.
AMMON_DEV void block_cand_reduce(float &v, uint32_t &i, float *sv, uint32_t *si) {
  sv[threadIdx.x] = v;
  si[threadIdx.x] = i;
  __syncthreads();
  for (uint32_t s = AMMON_WG / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      float a = sv[threadIdx.x];
      uint32_t ai = si[threadIdx.x];
      cand_merge(a, ai, sv[threadIdx.x + s], si[threadIdx.x + s]);
      sv[threadIdx.x] = a;
      si[threadIdx.x] = ai;
    }
    __syncthreads();
  }
  v = sv[0];
  i = si[0];
}

