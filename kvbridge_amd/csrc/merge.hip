// Stand-alone log-sum-exp merge (+ optional normalization) kernels, one
// 256-thread work-group per row-head (reference src/attention_shared.cu:295-335;
// the semantics are stated in merge_rows.h and merge_block.h).  Dims 64, 128
// and 256 run merge_rows (16-byte loads of split groups, one memory round
// trip per 64 splits), or above 64 splits merge_wide_kernel (1024 threads,
// one pass of up to 256-1024 splits); any other dim runs merge_row_head.
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

// More than 64 splits: one 1024-thread work-group per row-head takes up to
// 16 splits per thread in one pass (256 / 512 / 1024 splits per pass at dim
// 256 / 128 / 64) instead of merge_rows' 64-split passes.  Threads are
// (split group g, quad e) as in merge_rows: group g sums splits g, g + G, ...
// of its quad in increasing order with 16-byte loads issued before the
// pass's factors are known; the split maxima come first (one strided pass
// over m_j), factors f_j = e^(m_j - M) (0 where l_j = 0) are shared through
// LDS, and the group sums are added in group order.  Same semantics as
// merge_rows (merge_rows.h), deterministic for a given S and D.
constexpr int kWideThreads = 1024;

template <int D>
__global__ __launch_bounds__(kWideThreads) void merge_wide_kernel(
    uint32_t S, const float* __restrict__ scratch, float* __restrict__ m, float* __restrict__ l,
    float* __restrict__ n, void* __restrict__ out, int out_type) {
  constexpr uint32_t W = D + 2;
  constexpr uint32_t Q = D / 4;                   // quads of a row-head
  constexpr uint32_t G = kWideThreads / Q;        // split groups
  constexpr uint32_t K = 16;                      // splits per thread per pass
  constexpr uint32_t PS = G * K;                  // splits per pass
  constexpr uint32_t NWV = kWideThreads / 64;     // waves
  static_assert(PS <= uint32_t(kWideThreads), "one factor per thread");
  __shared__ float fs[PS];
  __shared__ float red[2][NWV];
  __shared__ float4 part[G][Q];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t g = tid / Q, q = tid % Q;
  const size_t rh = blockIdx.x;
  const float* const base = scratch + rh * S * W;
  const __amdgpu_buffer_rsrc_t rs = merge_detail::rows_rsrc(base, S * W * 4u);

  // M = max_j m_j.
  float mx = neg_inf();
  for (uint32_t j = tid; j < S; j += kWideThreads) mx = fmaxf(mx, base[size_t(j) * W]);
  mx = wave_max(mx);
  if (lane == 0) red[0][wave] = mx;
  __syncthreads();
  float M = red[0][0];
#pragma unroll
  for (uint32_t w = 1; w < NWV; ++w) M = fmaxf(M, red[0][w]);

  float L = 0.f;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  const uint32_t passes = (S + PS - 1u) / PS;
  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t j0 = p * PS;
    merge_detail::u32x4 v[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
      const uint32_t j = j0 + g + G * k;
      v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, int(((j < S ? j : S - 1u) * W + 2u + 4u * q) * 4u), 0, 0);
    }
    float fl = 0.f;
    if (tid < PS) {
      const uint32_t j = j0 + tid;
      float f = 0.f;
      if (j < S) {
        const float mj = base[size_t(j) * W], lj = base[size_t(j) * W + 1];
        f = lj > 0.f ? exp_e(mj - M) : 0.f;
        fl = f * lj;
      }
      fs[tid] = f;
    }
    fl = wave_sum(fl);
    __syncthreads();  // fs ready; red[0] no longer read
    if (lane == 0) red[1][wave] = fl;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
      const uint32_t jl = g + G * k;
      if (j0 + jl < S) {
        const float f = fs[jl];
        acc.x = fmaf(f, __uint_as_float(v[k][0]), acc.x);
        acc.y = fmaf(f, __uint_as_float(v[k][1]), acc.y);
        acc.z = fmaf(f, __uint_as_float(v[k][2]), acc.z);
        acc.w = fmaf(f, __uint_as_float(v[k][3]), acc.w);
      }
    }
    __syncthreads();  // red[1] complete, fs free for the next pass
#pragma unroll
    for (uint32_t w = 0; w < NWV; ++w) L += red[1][w];
    __syncthreads();  // red[1] read before the next pass rewrites it
  }
  part[g][q] = acc;
  __syncthreads();
  if (g == 0) {
    float4 nv = part[0][q];
#pragma unroll 4
    for (uint32_t gg = 1; gg < G; ++gg) {
      const float4 x = part[gg][q];
      nv.x += x.x;
      nv.y += x.y;
      nv.z += x.z;
      nv.w += x.w;
    }
    if (q == 0) {
      m[rh] = M;
      l[rh] = L;
    }
    float* const nd = n + rh * D + 4u * q;
    nd[0] = nv.x;
    nd[1] = nv.y;
    nd[2] = nv.z;
    nd[3] = nv.w;
    if (out_type != 0) {
      const float o[4] = {L > 0.f ? nv.x / L : 0.f, L > 0.f ? nv.y / L : 0.f, L > 0.f ? nv.z / L : 0.f,
                          L > 0.f ? nv.w / L : 0.f};
      if (out_type == 1) {
        float* const od = static_cast<float*>(out) + rh * D + 4u * q;
        for (int i = 0; i < 4; ++i) od[i] = o[i];
      } else {
        _Float16* const oh = static_cast<_Float16*>(out) + rh * D + 4u * q;
        for (int i = 0; i < 4; ++i) oh[i] = (_Float16)o[i];
      }
    }
  }
}

}  // namespace

hipError_t launch_merge(uint32_t row_heads, uint32_t dim, uint32_t splits, const float* scratch,
                        float* m, float* l, float* n, void* out, int out_type,
                        hipStream_t stream) {
  const dim3 grid(row_heads), block(kMergeThreads);
  if (splits > 64u && (dim == 64 || dim == 128 || dim == 256)) {
    const dim3 wblock(kWideThreads);
    switch (dim) {
      case 64:
        hipLaunchKernelGGL(merge_wide_kernel<64>, grid, wblock, 0, stream, splits, scratch, m, l, n, out, out_type);
        break;
      case 128:
        hipLaunchKernelGGL(merge_wide_kernel<128>, grid, wblock, 0, stream, splits, scratch, m, l, n, out, out_type);
        break;
      default:
        hipLaunchKernelGGL(merge_wide_kernel<256>, grid, wblock, 0, stream, splits, scratch, m, l, n, out, out_type);
    }
    return hipGetLastError();
  }
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
                       reinterpret_cast<const void*>(&merge_rows_kernel<256>),
                       reinterpret_cast<const void*>(&merge_wide_kernel<64>),
                       reinterpret_cast<const void*>(&merge_wide_kernel<128>),
                       reinterpret_cast<const void*>(&merge_wide_kernel<256>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvb
