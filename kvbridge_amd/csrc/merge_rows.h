// Log-sum-exp merge of the split partials of up to RM row-heads by one
// work-group of 64 * NW threads, with the reference merge semantics
// (src/attention_shared.cu:295-335):
//   M = max_j m_j,  L = sum_{l_j > 0} e^{m_j - M} l_j,
//   N[d] = sum_{l_j > 0} e^{m_j - M} n_j[d],
// so an all-empty row-head gives M = -inf, L = 0, N = 0 with no NaN.
//
// Partial j of row-head r is row_base(r)[j * (D + 2) + c]: c = 0 max, 1
// denominator, 2.. numerator.  Threads are (split group g, quad e): quad e
// is four consecutive numerator columns of one row-head, and group g sums
// the splits j = g, g + G, g + 2G, ... of its quad in increasing order with
// 16-byte loads; the G group sums are then added in group order.  Splits go
// in passes of PS = G * K (<= 64): in each pass every numerator load of the
// thread is issued before the pass's (m_j, l_j) loads, so a pass costs one
// memory round trip.  The factors e^{m_j - M} of a pass are computed by one
// wave per row-head (lane = split) and shared through LDS; L is a wave tree
// per pass, added in pass order.  The result is deterministic: it depends
// only on S, D and the thread layout.
//
// AGENT: partials written by other work-groups of the running kernel (any
// XCD) -- every load uses the agent-scope coherent policy (sc1).
#pragma once
#include <cstdint>

#include "device_common.h"

namespace kvb {

template <int D, int NW, int RM>
struct MergeRowsLayout {
  static constexpr uint32_t kT = 64u * NW;
  static constexpr uint32_t kQ = D / 4;        // quads per row-head
  static constexpr uint32_t kQT = RM * kQ;     // quads of RM row-heads
  static_assert(kQT <= kT, "merge_rows needs a thread per quad");
  static constexpr uint32_t kG = kT / kQT;     // split groups
  static constexpr uint32_t kK = kG >= 4 ? 64u / kG : 16u;  // splits per thread per pass (<= 16 loads)
  static constexpr uint32_t kPS = kG * kK;     // splits per pass (<= 64)
  static_assert(kPS <= 64, "one wave computes a pass's factors");
  // LDS floats: factors [RM][kPS], (M, L, pad) [RM][4], group sums [kG][kQT] float4
  static constexpr uint32_t kFloats = RM * kPS + 4 * RM + 4 * kG * kQT;
};

namespace merge_detail {

constexpr int kAuxPlain = 0;
constexpr int kAuxAgent = 16;  // sc1: the cache policy of an agent-scope atomic load

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, int(bytes), 0x00020000);
}

template <bool AGENT>
__device__ __forceinline__ float load1(const float* p) {
  if constexpr (AGENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else return *p;
}

}  // namespace merge_detail

// R <= RM row-heads, S >= 1 splits.  row_base(r) -> const float* (r < R).
// emit(r, q, N (float4: columns 4q..4q+3), M, L) is called once per quad
// of every row-head, by the thread that owns it.  lds: kFloats floats,
// 16-byte aligned.  Every thread of the work-group must call this.
template <int D, int NW, int RM, bool AGENT, typename RowBase, typename Emit>
__device__ __forceinline__ void merge_rows(uint32_t R, uint32_t S, RowBase row_base, float* lds, Emit emit) {
  using L = MergeRowsLayout<D, NW, RM>;
  using merge_detail::u32x4;
  constexpr uint32_t W = D + 2;
  constexpr int aux = AGENT ? merge_detail::kAuxAgent : merge_detail::kAuxPlain;
  float* const fs = lds;                                                   // [RM][kPS]
  float* const ml = lds + RM * L::kPS;                                     // [RM][4]: M, L
  float4* const part = reinterpret_cast<float4*>(lds + RM * L::kPS + 4 * RM);  // [kG][kQT]
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t g = tid / L::kQT, e = tid % L::kQT;
  const uint32_t r = e / L::kQ, q = e % L::kQ;
  const bool mine = g < L::kG && r < R;
  const uint32_t rr = mine ? r : 0u;
  const __amdgpu_buffer_rsrc_t rs = merge_detail::rows_rsrc(row_base(rr), S * W * 4u);
  const uint32_t passes = (S + L::kPS - 1u) / L::kPS;

  // Maxima over every split first when there is more than one pass.
  if (passes > 1u) {
    for (uint32_t h = wave; h < R; h += NW) {
      const float* b = row_base(h);
      float mx = neg_inf();
      for (uint32_t j = lane; j < S; j += 64u) mx = fmaxf(mx, merge_detail::load1<AGENT>(b + size_t(j) * W));
      mx = wave_max(mx);
      if (lane == 0) ml[4 * h] = mx;
    }
    __syncthreads();
  }

  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t j0 = p * L::kPS;
    const uint32_t jmax = S - 1u;
    u32x4 v[L::kK];
#pragma unroll
    for (uint32_t k = 0; k < L::kK; ++k) {
      const uint32_t j = j0 + g + L::kG * k;
      v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, int(((j < jmax ? j : jmax) * W + 2u + 4u * q) * 4u), 0, aux);
    }
    for (uint32_t h = wave; h < R; h += NW) {
      const float* b = row_base(h);
      const uint32_t j = j0 + lane;
      const bool in = lane < L::kPS && j < S;
      const float* pj = b + size_t(in ? j : 0u) * W;
      const float mj = merge_detail::load1<AGENT>(pj);
      const float lj = merge_detail::load1<AGENT>(pj + 1);
      const float mx = passes > 1u ? ml[4 * h] : wave_max(in ? mj : neg_inf());
      const float f = in && lj > 0.f ? exp_e(mj - mx) : 0.f;
      const float lsum = wave_sum(f * lj);
      if (lane < L::kPS) fs[h * L::kPS + lane] = f;
      if (lane == 0) {
        ml[4 * h] = mx;
        ml[4 * h + 1] = p == 0 ? lsum : ml[4 * h + 1] + lsum;
      }
    }
    __syncthreads();
    if (mine) {
      const float* fr = fs + r * L::kPS;
#pragma unroll
      for (uint32_t k = 0; k < L::kK; ++k) {
        const uint32_t jl = g + L::kG * k;
        if (j0 + jl < S) {
          const float f = fr[jl];
          acc.x = fmaf(f, __uint_as_float(v[k][0]), acc.x);
          acc.y = fmaf(f, __uint_as_float(v[k][1]), acc.y);
          acc.z = fmaf(f, __uint_as_float(v[k][2]), acc.z);
          acc.w = fmaf(f, __uint_as_float(v[k][3]), acc.w);
        }
      }
    }
    __syncthreads();
  }
  if (g < L::kG) part[g * L::kQT + e] = acc;
  __syncthreads();
  if (g == 0 && r < R) {
    float4 nsum = part[e];
#pragma unroll
    for (uint32_t gg = 1; gg < L::kG; ++gg) {
      const float4 x = part[gg * L::kQT + e];
      nsum.x += x.x;
      nsum.y += x.y;
      nsum.z += x.z;
      nsum.w += x.w;
    }
    emit(r, q, nsum, ml[4 * r], ml[4 * r + 1]);
  }
}

}  // namespace kvb
