// Stand-alone log-sum-exp merge (+ optional normalization) kernel: one
// 256-thread work-group per row-head running merge_row_head (merge_block.h),
// whose header states the semantics (reference src/attention_shared.cu:295-335).
#include "kernels.h"
#include "merge_block.h"

namespace kvb {
namespace {

__global__ __launch_bounds__(kMergeThreads) void merge_kernel(
    uint32_t dim, uint32_t splits, const float* __restrict__ scratch, float* __restrict__ m,
    float* __restrict__ l, float* __restrict__ n, void* __restrict__ out, int out_type) {
  __shared__ MergeSmem sm;
  merge_row_head(sm, threadIdx.x, blockIdx.x, dim, splits, scratch, m, l, n, out, out_type);
}

}  // namespace

hipError_t launch_merge(uint32_t row_heads, uint32_t dim, uint32_t splits, const float* scratch,
                        float* m, float* l, float* n, void* out, int out_type,
                        hipStream_t stream) {
  hipLaunchKernelGGL(merge_kernel, dim3(row_heads), dim3(kMergeThreads), 0, stream, dim, splits, scratch, m, l,
                     n, out, out_type);
  return hipGetLastError();
}

hipError_t preload_merge() {
  hipFuncAttributes attr{};
  return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&merge_kernel));
}

}  // namespace kvb
