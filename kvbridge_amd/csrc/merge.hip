// Log-sum-exp merge of split partials, optionally fused with normalization.
// Semantics follow the reference merge (src/attention_shared.cu:295-335):
//   M = max_j m_j,  L = sum_{l_j > 0} e^{m_j - M} l_j,
//   N[d] = sum_{l_j > 0} e^{m_j - M} n_j[d],
// so an all-empty row-head gives M = -inf, L = 0, N = 0 with no NaN.  The
// optional output is out[rh * dim + d] = L > 0 ? N[d] / L : 0 (fp32 or fp16).
//
// One 256-thread work-group per row-head.  Phase 1: the (m_j, l_j) pairs are
// read in parallel, reduced to M and L, and the per-split factors
// f_j = e^{m_j - M} (0 for l_j <= 0) are kept in LDS.  Phase 2: threads are
// laid out as (split group, dim); each sums its share of the splits with all
// loads independent, and the groups are added through LDS.  Two dependent
// memory round trips in total, independent of the split count.
#include "kernels.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxFactors = 4096;  // splits handled per LDS pass

template <int kOut>  // 0 none, 1 fp32, 2 fp16
__global__ __launch_bounds__(kThreads) void merge_kernel(
    uint32_t dim, uint32_t splits, const float* __restrict__ scratch, float* __restrict__ m,
    float* __restrict__ l, float* __restrict__ n, void* __restrict__ out) {
  __shared__ float f_s[kMaxFactors];
  __shared__ float red_s[2][kThreads / 64];
  __shared__ float part_s[kThreads];
  const uint32_t tid = threadIdx.x, wave = tid >> 6;
  const uint32_t rh = blockIdx.x;
  const uint32_t stride = dim + 2;
  const float* base = scratch + size_t(rh) * splits * stride;

  // Phase 1: M over all splits.
  float mx = neg_inf();
  for (uint32_t j = tid; j < splits; j += kThreads) mx = fmaxf(mx, base[size_t(j) * stride]);
  mx = wave_max(mx);
  if ((tid & 63) == 0) red_s[0][wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red_s[0][0], red_s[0][1]), fmaxf(red_s[0][2], red_s[0][3]));

  // Phase 2 layout: G split groups x dim threads (dim <= 256).
  const uint32_t groups = dim >= kThreads ? 1u : kThreads / dim;
  const uint32_t grp = tid / dim, d = tid % dim;
  float lsum = 0.f, nacc = 0.f;
  for (uint32_t j0 = 0; j0 < splits; j0 += kMaxFactors) {
    const uint32_t cnt = splits - j0 < uint32_t(kMaxFactors) ? splits - j0 : uint32_t(kMaxFactors);
    for (uint32_t j = tid; j < cnt; j += kThreads) {
      const float* p = base + size_t(j0 + j) * stride;
      const float lj = p[1];
      float f = 0.f;
      if (lj > 0.f) {
        f = exp_e(p[0] - mx);
        lsum = fmaf(f, lj, lsum);
      }
      f_s[j] = f;
    }
    __syncthreads();
    if (grp < groups) {
#pragma unroll 8
      for (uint32_t j = grp; j < cnt; j += groups) {
        const float f = f_s[j];
        if (f != 0.f) nacc = fmaf(f, base[size_t(j0 + j) * stride + 2 + d], nacc);
      }
    }
    __syncthreads();
  }
  lsum = wave_sum(lsum);
  if ((tid & 63) == 0) red_s[1][wave] = lsum;
  part_s[tid] = nacc;
  __syncthreads();
  lsum = (red_s[1][0] + red_s[1][1]) + (red_s[1][2] + red_s[1][3]);
  if (tid == 0) {
    m[rh] = mx;
    l[rh] = lsum;
  }
  if (tid < dim) {
    float nd = 0.f;
    for (uint32_t gi = 0; gi < groups; ++gi) nd += part_s[gi * dim + tid];
    n[size_t(rh) * dim + tid] = nd;
    if constexpr (kOut != 0) {
      const float o = lsum > 0.f ? nd / lsum : 0.f;
      if constexpr (kOut == 1) static_cast<float*>(out)[size_t(rh) * dim + tid] = o;
      else static_cast<_Float16*>(out)[size_t(rh) * dim + tid] = (_Float16)o;
    }
  }
}

}  // namespace

hipError_t launch_merge(uint32_t row_heads, uint32_t dim, uint32_t splits, const float* scratch,
                        float* m, float* l, float* n, void* out, int out_type,
                        hipStream_t stream) {
  const dim3 grid(row_heads), block(kThreads);
  switch (out_type) {
    case 1:
      hipLaunchKernelGGL(merge_kernel<1>, grid, block, 0, stream, dim, splits, scratch, m, l, n, out);
      break;
    case 2:
      hipLaunchKernelGGL(merge_kernel<2>, grid, block, 0, stream, dim, splits, scratch, m, l, n, out);
      break;
    default:
      hipLaunchKernelGGL(merge_kernel<0>, grid, block, 0, stream, dim, splits, scratch, m, l, n, out);
      break;
  }
  return hipGetLastError();
}

hipError_t preload_merge() {
  hipFuncAttributes attr{};
  hipError_t e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&merge_kernel<0>));
  if (e != hipSuccess) return e;
  e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&merge_kernel<1>));
  if (e != hipSuccess) return e;
  return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&merge_kernel<2>));
}

}  // namespace kvb
