// Stand-alone log-sum-exp merge (+ optional normalization) kernels, one
// 256-thread work-group per row-head (reference src/attention_shared.cu:295-335;
// the semantics are stated in merge_rows.h and merge_block.h).  Dims 64, 128
// and 256 run merge_rows (16-byte loads of split groups, one memory round
// trip per 64 splits), or above 64 splits merge_slices_kernel (a row-head's
// dims over several work-groups, one round trip per 256 splits); any other
// dim runs merge_row_head.
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

// More than 64 splits, spread over the chip: each row-head's D dims are cut
// into slices of DS dims, one 256-thread work-group per (row-head, slice)
// (row_heads x D / DS work-groups instead of one per row-head).  Threads are
// (split group g, quad q of the slice); a pass covers 256 splits: thread t
// loads m and l of split j0 + t, group g the 16-byte numerator quads of
// splits g, g + G, ... (K = 256 / G of them), and every load of a pass is
// issued before anything waits, so a call of at most 256 splits costs one
// memory round trip (more splits take their maxima in a strided pass
// first).  M = max_j m_j, f_j = e^(m_j - M) (0 where l_j = 0) shared through
// LDS, L = sum_j f_j l_j, the group sums added in group order; slice 0
// writes m and l.  Deterministic for a given S, D and DS (DS is chosen from
// the shape alone).
constexpr uint32_t kSliceThreads = 256;

template <int D, int DS>
__global__ __launch_bounds__(kSliceThreads) void merge_slices_kernel(
    uint32_t S, const float* __restrict__ scratch, float* __restrict__ m, float* __restrict__ l,
    float* __restrict__ n, void* __restrict__ out, int out_type) {
  constexpr uint32_t W = D + 2;
  constexpr uint32_t QD = DS / 4;              // quads of a slice
  constexpr uint32_t G = kSliceThreads / QD;   // split groups
  constexpr uint32_t PS = kSliceThreads;       // splits per pass
  constexpr uint32_t K = PS / G;               // numerator quads per thread per pass
  constexpr uint32_t NWV = kSliceThreads / 64;
  static_assert(D % DS == 0 && DS % 4 == 0 && K * G == PS, "slice shape");
  __shared__ float fs[PS];
  __shared__ float red[2][NWV];
  __shared__ float4 part[G][QD];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t g = tid / QD, q = tid % QD;
  const size_t rh = blockIdx.x;
  const uint32_t col = blockIdx.y * uint32_t(DS) + 4u * q;  // the thread's first column
  const float* const base = scratch + rh * S * W;
  const __amdgpu_buffer_rsrc_t rs = merge_detail::rows_rsrc(base, S * W * 4u);
  const uint32_t passes = (S + PS - 1u) / PS;
  auto block_max = [&](float x) __attribute__((always_inline)) {
    x = wave_max(x);
    if (lane == 0) red[0][wave] = x;
    __syncthreads();
    float r = red[0][0];
#pragma unroll
    for (uint32_t w = 1; w < NWV; ++w) r = fmaxf(r, red[0][w]);
    return r;
  };

  float M = neg_inf();
  if (passes > 1u) {
    float mx = neg_inf();
    for (uint32_t j = tid; j < S; j += kSliceThreads) mx = fmaxf(mx, base[size_t(j) * W]);
    M = block_max(mx);
  }
  float L = 0.f;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t j0 = p * PS;
    const uint32_t jt = j0 + tid;
    float mj = neg_inf(), lj = 0.f;
    if (jt < S) {
      mj = base[size_t(jt) * W];
      lj = base[size_t(jt) * W + 1];
    }
    merge_detail::u32x4 v[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
      const uint32_t j = j0 + g + G * k;
      v[k] = merge_detail::u32x4{0u, 0u, 0u, 0u};  // splits past S: no load (not read below)
      if (j < S) v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, int((j * W + 2u + col) * 4u), 0, 0);
    }
    if (passes == 1u) M = block_max(mj);
    const float f = jt < S && lj > 0.f ? exp_e(mj - M) : 0.f;
    fs[tid] = f;
    const float fl = wave_sum(f * lj);
    __syncthreads();  // fs ready; red[0] no longer read
    if (lane == 0) red[1][wave] = fl;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
      const uint32_t jl = g + G * k;
      if (j0 + jl < S) {
        const float fk = fs[jl];
        acc.x = fmaf(fk, __uint_as_float(v[k][0]), acc.x);
        acc.y = fmaf(fk, __uint_as_float(v[k][1]), acc.y);
        acc.z = fmaf(fk, __uint_as_float(v[k][2]), acc.z);
        acc.w = fmaf(fk, __uint_as_float(v[k][3]), acc.w);
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
    if (blockIdx.y == 0 && q == 0) {
      m[rh] = M;
      l[rh] = L;
    }
    float* const nd = n + rh * D + col;
    nd[0] = nv.x;
    nd[1] = nv.y;
    nd[2] = nv.z;
    nd[3] = nv.w;
    if (out_type != 0) {
      const float o[4] = {L > 0.f ? nv.x / L : 0.f, L > 0.f ? nv.y / L : 0.f, L > 0.f ? nv.z / L : 0.f,
                          L > 0.f ? nv.w / L : 0.f};
      if (out_type == 1) {
        float* const od = static_cast<float*>(out) + rh * D + col;
        for (int i = 0; i < 4; ++i) od[i] = o[i];
      } else {
        _Float16* const oh = static_cast<_Float16*>(out) + rh * D + col;
        for (int i = 0; i < 4; ++i) oh[i] = (_Float16)o[i];
      }
    }
  }
}

// Slice width: the widest of 64 / 32 / 16 dims that still gives 512
// work-groups (two per compute unit of a whole MI355X), else 16.  The width
// sets the split groups the sums are added in, so it is chosen from the
// shape alone, not from the device's compute-unit count: the same call gives
// the same bits on a partitioned device.
constexpr uint64_t kSliceGroupsWanted = 512;

template <int D>
hipError_t launch_merge_slices(uint32_t row_heads, uint32_t splits, const float* scratch, float* m, float* l,
                               float* n, void* out, int out_type, hipStream_t stream) {
  const uint64_t want = kSliceGroupsWanted;
  const dim3 block(kSliceThreads);
  if (uint64_t(row_heads) * (D / 64) >= want)
    hipLaunchKernelGGL((merge_slices_kernel<D, 64>), dim3(row_heads, D / 64), block, 0, stream, splits, scratch,
                       m, l, n, out, out_type);
  else if (uint64_t(row_heads) * (D / 32) >= want)
    hipLaunchKernelGGL((merge_slices_kernel<D, 32>), dim3(row_heads, D / 32), block, 0, stream, splits, scratch,
                       m, l, n, out, out_type);
  else
    hipLaunchKernelGGL((merge_slices_kernel<D, 16>), dim3(row_heads, D / 16), block, 0, stream, splits, scratch,
                       m, l, n, out, out_type);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_merge(uint32_t row_heads, uint32_t dim, uint32_t splits, const float* scratch,
                        float* m, float* l, float* n, void* out, int out_type,
                        hipStream_t stream) {
  const dim3 grid(row_heads), block(kMergeThreads);
  if (splits > 64u && (dim == 64 || dim == 128 || dim == 256)) {
    switch (dim) {
      case 64: return launch_merge_slices<64>(row_heads, splits, scratch, m, l, n, out, out_type, stream);
      case 128: return launch_merge_slices<128>(row_heads, splits, scratch, m, l, n, out, out_type, stream);
      default: return launch_merge_slices<256>(row_heads, splits, scratch, m, l, n, out, out_type, stream);
    }
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
                       reinterpret_cast<const void*>(&merge_slices_kernel<64, 64>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<64, 32>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<64, 16>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<128, 64>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<128, 32>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<128, 16>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<256, 64>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<256, 32>),
                       reinterpret_cast<const void*>(&merge_slices_kernel<256, 16>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvb
