// Stand-alone log-sum-exp merge (+ optional normalization) kernels, one
// 256-thread work-group per row-head (reference src/attention_shared.cu:295-335;
// the semantics are stated in merge_rows.h and merge_block.h).  Dims 64, 128
// and 256 run merge_rows (16-byte loads of split groups, one memory round
// trip per 64 splits); any other dim runs merge_row_head.
#include "kernels.h"
#include "merge_block.h"
#include "merge_rows.h"

namespace kvb {
namespace {

__global__ __launch_bounds__(kMergeThreads) void merge_kernel(
    uint32_t dim, uint32_t splits, const float* __restrict__ scratch, float* __restrict__ m,
    float* __restrict__ l, float* __restrict__ n, void* __restrict__ out, int out_type) {
  __shared__ MergeSmem sm;
  merge_row_head(sm, threadIdx.x, blockIdx.x, dim, splits, scratch, m, l, n, out, out_type);
}

constexpr int kRowsWaves = kMergeThreads / 64;

template <int D>
__global__ __launch_bounds__(kMergeThreads) void merge_rows_kernel(
    uint32_t splits, const float* __restrict__ scratch, float* __restrict__ m, float* __restrict__ l,
    float* __restrict__ n, void* __restrict__ out, int out_type) {
  using L = MergeRowsLayout<D, kRowsWaves, 1>;
  __shared__ __attribute__((aligned(16))) float lds[L::kFloats];
  const size_t rh = blockIdx.x;
  const float* const base = scratch + rh * splits * (D + 2);
  merge_rows<D, kRowsWaves, 1, false>(
      1u, splits, [&](uint32_t) { return base; }, lds,
      [&](uint32_t, uint32_t q, float4 nv, float mv, float lv) {
        if (q == 0) {
          m[rh] = mv;
          l[rh] = lv;
        }
        float* const nd = n + rh * D + 4u * q;  // caller buffers need only 4-byte alignment
        nd[0] = nv.x;
        nd[1] = nv.y;
        nd[2] = nv.z;
        nd[3] = nv.w;
        if (out_type != 0) {
          const float o[4] = {lv > 0.f ? nv.x / lv : 0.f, lv > 0.f ? nv.y / lv : 0.f, lv > 0.f ? nv.z / lv : 0.f,
                              lv > 0.f ? nv.w / lv : 0.f};
          if (out_type == 1) {
            float* const od = static_cast<float*>(out) + rh * D + 4u * q;
            for (int i = 0; i < 4; ++i) od[i] = o[i];
          } else {
            _Float16* const oh = static_cast<_Float16*>(out) + rh * D + 4u * q;
            for (int i = 0; i < 4; ++i) oh[i] = (_Float16)o[i];
          }
        }
      });
}

}  // namespace

hipError_t launch_merge(uint32_t row_heads, uint32_t dim, uint32_t splits, const float* scratch,
                        float* m, float* l, float* n, void* out, int out_type,
                        hipStream_t stream) {
  const dim3 grid(row_heads), block(kMergeThreads);
  switch (dim) {
    case 64:
      hipLaunchKernelGGL(merge_rows_kernel<64>, grid, block, 0, stream, splits, scratch, m, l, n, out, out_type);
      break;
    case 128:
      hipLaunchKernelGGL(merge_rows_kernel<128>, grid, block, 0, stream, splits, scratch, m, l, n, out, out_type);
      break;
    case 256:
      hipLaunchKernelGGL(merge_rows_kernel<256>, grid, block, 0, stream, splits, scratch, m, l, n, out, out_type);
      break;
    default:
      hipLaunchKernelGGL(merge_kernel, grid, block, 0, stream, dim, splits, scratch, m, l, n, out, out_type);
  }
  return hipGetLastError();
}

hipError_t preload_merge() {
  const void* fns[] = {reinterpret_cast<const void*>(&merge_kernel),
                       reinterpret_cast<const void*>(&merge_rows_kernel<64>),
                       reinterpret_cast<const void*>(&merge_rows_kernel<128>),
                       reinterpret_cast<const void*>(&merge_rows_kernel<256>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvb
