// Block-level log-sum-exp merge of one row-head's split partials (the body
// of the stand-alone merge kernel, merge.hip).
// Semantics follow the reference merge (src/attention_shared.cu:295-335):
//   M = max_j m_j,  L = sum_{l_j > 0} e^{m_j - M} l_j,
//   N[d] = sum_{l_j > 0} e^{m_j - M} n_j[d],
// so an all-empty row-head gives M = -inf, L = 0, N = 0 with no NaN.  The
// optional output is out[rh * dim + d] = L > 0 ? N[d] / L : 0 (fp32 or fp16).
//
// kMergeThreads threads (threads tid < kMergeThreads of the calling block do
// the work; every thread of the block must call it, for the barriers).
// Phase 1: the (m_j, l_j) pairs are read in parallel, reduced to M and L, and
// the per-split factors f_j = e^{m_j - M} (0 for l_j <= 0) kept in LDS.
// Phase 2: threads are laid out as (split group, dim); each sums its share
// of the splits with all loads independent, and the groups are added
// through LDS.  Two dependent memory round trips, any split count.
#pragma once
#include <cstdint>
#include "device_common.h"

namespace kvb {

constexpr int kMergeThreads = 256;
constexpr int kMergeMaxFactors = 4096;  // splits per LDS pass

struct MergeSmem {
  float f[kMergeMaxFactors];
  float red[2][kMergeThreads / 64];
  float part[kMergeThreads];
};

// out_type: 0 none, 1 fp32, 2 fp16.
__device__ __forceinline__ void merge_row_head(MergeSmem& sm, uint32_t tid, uint32_t rh, uint32_t dim,
                                               uint32_t splits, const float* __restrict__ scratch,
                                               float* __restrict__ m, float* __restrict__ l,
                                               float* __restrict__ n, void* __restrict__ out, int out_type) {
  const bool active = tid < uint32_t(kMergeThreads);
  const uint32_t wave = tid >> 6;
  const uint32_t stride = dim + 2;
  const float* base = scratch + size_t(rh) * splits * stride;

  float mx = neg_inf();
  if (active)
    for (uint32_t j = tid; j < splits; j += kMergeThreads) mx = fmaxf(mx, base[size_t(j) * stride]);
  mx = wave_max(mx);
  if (active && (tid & 63) == 0) sm.red[0][wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(sm.red[0][0], sm.red[0][1]), fmaxf(sm.red[0][2], sm.red[0][3]));

  const uint32_t groups = dim >= uint32_t(kMergeThreads) ? 1u : uint32_t(kMergeThreads) / dim;
  const uint32_t grp = tid / dim, d = tid % dim;
  float lsum = 0.f, nacc = 0.f;
  for (uint32_t j0 = 0; j0 < splits; j0 += kMergeMaxFactors) {
    const uint32_t cnt = splits - j0 < uint32_t(kMergeMaxFactors) ? splits - j0 : uint32_t(kMergeMaxFactors);
    if (active) {
      for (uint32_t j = tid; j < cnt; j += kMergeThreads) {
        const float* p = base + size_t(j0 + j) * stride;
        const float lj = p[1];
        float f = 0.f;
        if (lj > 0.f) {
          f = exp_e(p[0] - mx);
          lsum = fmaf(f, lj, lsum);
        }
        sm.f[j] = f;
      }
    }
    __syncthreads();
    if (active && grp < groups) {
#pragma unroll 8
      for (uint32_t j = grp; j < cnt; j += groups) {
        const float f = sm.f[j];
        if (f != 0.f) nacc = fmaf(f, base[size_t(j0 + j) * stride + 2 + d], nacc);
      }
    }
    __syncthreads();
  }
  lsum = wave_sum(lsum);
  if (active && (tid & 63) == 0) sm.red[1][wave] = lsum;
  if (active) sm.part[tid] = nacc;
  __syncthreads();
  lsum = (sm.red[1][0] + sm.red[1][1]) + (sm.red[1][2] + sm.red[1][3]);
  if (tid == 0) {
    m[rh] = mx;
    l[rh] = lsum;
  }
  if (tid < dim) {
    float nd = 0.f;
    for (uint32_t gi = 0; gi < groups; ++gi) nd += sm.part[gi * dim + tid];
    n[size_t(rh) * dim + tid] = nd;
    if (out_type != 0) {
      const float o = lsum > 0.f ? nd / lsum : 0.f;
      if (out_type == 1) static_cast<float*>(out)[size_t(rh) * dim + tid] = o;
      else static_cast<_Float16*>(out)[size_t(rh) * dim + tid] = (_Float16)o;
    }
  }
  __syncthreads();  // LDS reuse by a following call
}

}  // namespace kvb
