// Log-sum-exp merge of split partials, optionally fused with normalization.
// Semantics follow the reference merge (src/attention_shared.cu:295-335):
//   M = max_j m_j,  L = sum_{l_j > 0} e^{m_j - M} l_j,
//   N[d] = sum_{l_j > 0} e^{m_j - M} n_j[d]   (accumulated in split order),
// so an all-empty row-head gives M = -inf, L = 0, N = 0 with no NaN.  The
// optional output is out[rh * dim + d] = L > 0 ? N[d] / L : 0 (fp32 or fp16).
//
// One wave per row-head, four row-heads per 256-thread block.  Lane j first
// holds split j's (m, l) to form the per-split factor e^{m_j - M}; the
// numerator loop then reads that factor from lane j with a scalar readlane,
// so the only memory traffic in the loop is the coalesced n_j row.
#include "kernels.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr int kWavesPerBlock = 4;

template <int kOut>  // 0 none, 1 fp32, 2 fp16
__global__ __launch_bounds__(64 * kWavesPerBlock) void merge_kernel(
    uint32_t row_heads, uint32_t dim, uint32_t splits, const float* __restrict__ scratch,
    float* __restrict__ m, float* __restrict__ l, float* __restrict__ n, void* __restrict__ out) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t rh = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (rh >= row_heads) return;
  const uint32_t stride = dim + 2;
  const float* base = scratch + size_t(rh) * splits * stride;

  float mx = neg_inf();
  for (uint32_t j = lane; j < splits; j += 64) mx = fmaxf(mx, base[size_t(j) * stride]);
  mx = wave_max(mx);

  float lsum = 0.f;
  float nacc[4] = {0.f, 0.f, 0.f, 0.f};  // dims lane, lane+64, lane+128, lane+192
  for (uint32_t j0 = 0; j0 < splits; j0 += 64) {
    const uint32_t j = j0 + lane;
    float f = 0.f;
    if (j < splits) {
      const float lj = base[size_t(j) * stride + 1];
      if (lj > 0.f) {
        f = exp_e(base[size_t(j) * stride] - mx);
        lsum = fmaf(f, lj, lsum);
      }
    }
    const uint32_t cnt = splits - j0 < 64u ? splits - j0 : 64u;
    for (uint32_t jj = 0; jj < cnt; ++jj) {
      const float fj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), jj));
      if (fj == 0.f) continue;  // split with l <= 0 (or an underflowed factor) adds nothing
      const float* nj = base + size_t(j0 + jj) * stride + 2;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t d = lane + 64u * c;
        if (d < dim) nacc[c] = fmaf(fj, nj[d], nacc[c]);
      }
    }
  }
  lsum = wave_sum(lsum);
  if (lane == 0) {
    m[rh] = mx;
    l[rh] = lsum;
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint32_t d = lane + 64u * c;
    if (d >= dim) continue;
    n[size_t(rh) * dim + d] = nacc[c];
    if constexpr (kOut != 0) {
      const float o = lsum > 0.f ? nacc[c] / lsum : 0.f;
      if constexpr (kOut == 1) static_cast<float*>(out)[size_t(rh) * dim + d] = o;
      else static_cast<_Float16*>(out)[size_t(rh) * dim + d] = (_Float16)o;
    }
  }
}

}  // namespace

hipError_t launch_merge(uint32_t row_heads, uint32_t dim, uint32_t splits, const float* scratch,
                        float* m, float* l, float* n, void* out, int out_type,
                        hipStream_t stream) {
  const dim3 grid((row_heads + kWavesPerBlock - 1) / kWavesPerBlock);
  const dim3 block(64 * kWavesPerBlock);
  switch (out_type) {
    case 1:
      hipLaunchKernelGGL(merge_kernel<1>, grid, block, 0, stream, row_heads, dim, splits, scratch, m, l, n, out);
      break;
    case 2:
      hipLaunchKernelGGL(merge_kernel<2>, grid, block, 0, stream, row_heads, dim, splits, scratch, m, l, n, out);
      break;
    default:
      hipLaunchKernelGGL(merge_kernel<0>, grid, block, 0, stream, row_heads, dim, splits, scratch, m, l, n, out);
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
