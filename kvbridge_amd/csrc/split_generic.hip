// Generic split-partial kernel: any valid Shape (dim 1..256, any page size,
// any begin, int8 or fp32 KV, any GQA group).  It is the fallback behind
// launch_attention for shapes the tiled MFMA kernel does not cover; the
// arithmetic follows the per-split semantics of the reference
// src/attention_shared.cu:42-209 / :213-293 (visible = k_pos <= q_pos, score =
// (q . k_code) * k_scale * scale, weights exp(score - split max), numerator
// weighted by v_scale), evaluated as an online softmax over 256-token chunks
// so that one work-group can cover a split of any length.
//
// Grid: x = row * q_heads + head, y = split, z = sequence of a batched call.
// Block: 256 threads (4 waves).
#include "kernels.h"
#include "batch.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float block_max(float x, float* red) {
  x = wave_max(x);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red is reused; previous readers must be done
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = fmaxf(r, red[w]);
  return r;
}
__device__ __forceinline__ float block_sum(float x, float* red) {
  x = wave_sum(x);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r += red[w];
  return r;
}

template <bool kInt8>
__device__ __forceinline__ float kv_value(const void* base, uint32_t i) {
  if constexpr (kInt8) return float(static_cast<const int8_t*>(base)[i]);
  else return static_cast<const float*>(base)[i];
}

template <bool kInt8, bool VARLEN>
__global__ __launch_bounds__(kThreads) void split_generic_kernel(SplitArgs a) {
  if constexpr (VARLEN) rebase_sequence(a, blockIdx.z);
  __shared__ float q_s[256];
  __shared__ float pw_s[kThreads];
  __shared__ uint32_t vbase_s[kThreads];
  __shared__ float red_s[2][kWaves];

  const uint32_t tid = threadIdx.x;
  const uint32_t rh = blockIdx.x, split = blockIdx.y;
  const uint32_t row = rh / a.q_heads, head = rh % a.q_heads;
  const uint32_t kv = head / a.group;
  const uint32_t D = a.dim, P = a.page_tokens;

  const uint64_t s0_64 = uint64_t(a.begin) + uint64_t(split) * a.split_tokens;
  const uint32_t s0 = s0_64 < a.end ? uint32_t(s0_64) : a.end;
  const uint32_t s1 = uint64_t(s0) + a.split_tokens < a.end ? s0 + a.split_tokens : a.end;
  const int64_t qpos = a.q_positions[row];

  if (tid < D) q_s[tid] = a.q[size_t(rh) * D + tid];
  __syncthreads();

  float m_run = neg_inf(), l_run = 0.f, acc = 0.f;
  for (uint32_t c0 = s0; c0 < s1; c0 += kThreads) {
    const uint32_t t = c0 + tid;
    float score = neg_inf(), vsc = 0.f;
    uint32_t vb = 0;
    if (t < s1 && a.k_positions[t] <= qpos) {
      uint32_t page = a.page_table[t / P];
      page = page < a.pages ? page : a.pages - 1;
      const uint32_t slot = t % P;
      const uint32_t si = (page * a.kv_heads + kv) * P + slot;
      float dot = 0.f;
      for (uint32_t d = 0; d < D; ++d) dot = fmaf(q_s[d], kv_value<kInt8>(a.k, si * D + d), dot);
      const float ks = kInt8 ? a.k_scales[si] : 1.f;
      vsc = kInt8 ? a.v_scales[si] : 1.f;
      score = dot * ks * a.scale;
      vb = (page * a.kv_heads + kv) * D * P + slot;
    }
    const float cmax = block_max(score, red_s[0]);
    const float m_new = fmaxf(m_run, cmax);
    const float m_use = m_new == neg_inf() ? 0.f : m_new;
    const float alpha = exp_e(m_run - m_use);  // m_run = -inf -> 0
    const float w = exp_e(score - m_use);       // score = -inf -> 0
    const float csum = block_sum(w, red_s[1]);
    l_run = l_run * alpha + csum;
    m_run = m_new;
    pw_s[tid] = w * vsc;
    vbase_s[tid] = vb;
    __syncthreads();
    if (tid < D) {
      float part = 0.f;
      const uint32_t cnt = s1 - c0 < uint32_t(kThreads) ? s1 - c0 : uint32_t(kThreads);
      for (uint32_t j = 0; j < cnt; ++j) {
        const float p = pw_s[j];
        if (p != 0.f) part = fmaf(p, kv_value<kInt8>(a.v, vbase_s[j] + tid * P), part);
      }
      acc = fmaf(acc, alpha, part);
    }
    __syncthreads();
  }
  const size_t out = (size_t(rh) * a.splits + split) * (size_t(D) + 2);
  if (tid == 0) {
    a.scratch[out] = m_run;
    a.scratch[out + 1] = l_run;
  }
  if (tid < D) a.scratch[out + 2 + tid] = acc;
}

}  // namespace

hipError_t launch_split_generic(const SplitArgs& a, bool int8, hipStream_t stream) {
  const bool varlen = a.seq_starts != nullptr;
  const dim3 grid(a.rows * a.q_heads, a.splits, varlen ? a.batch : 1u);
  if (int8 && varlen)
    hipLaunchKernelGGL((split_generic_kernel<true, true>), grid, dim3(kThreads), 0, stream, a);
  else if (int8)
    hipLaunchKernelGGL((split_generic_kernel<true, false>), grid, dim3(kThreads), 0, stream, a);
  else if (varlen)
    hipLaunchKernelGGL((split_generic_kernel<false, true>), grid, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((split_generic_kernel<false, false>), grid, dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t preload_generic() {
  const void* fns[] = {reinterpret_cast<const void*>(&split_generic_kernel<true, false>),
                       reinterpret_cast<const void*>(&split_generic_kernel<false, false>),
                       reinterpret_cast<const void*>(&split_generic_kernel<true, true>),
                       reinterpret_cast<const void*>(&split_generic_kernel<false, true>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvb
