// Paged INT8 KV append (the write side of the cache format the split kernels
// read, include/kvbridge/attention_common.h): each new token's K and V rows
// of one kv head are quantized to symmetric int8 with a per-(token, kv head)
// fp32 scale and stored into its physical slot of the page pool:
//   scale = absmax / 127 (1 when absmax == 0, all codes 0),
//   code  = clamp(rint(x / scale), -127, 127)      (round half to even),
//   K codes token-major  k[((page*kv_heads + kv)*P + slot)*D + d],
//   V codes dim-major    v[((page*kv_heads + kv)*D + d)*P + slot],
//   scales               k_scales / v_scales[(page*kv_heads + kv)*P + slot].
// The division is IEEE round-to-nearest fp32 (HIP's default fp32 division),
// so codes and scales are bitwise those of any correctly rounded fp32
// implementation of the same formula.
//
// One wave per (token, kv head); lane i holds dims i, i+64, ... (D <= 256).
// Slot ids at or past the pool's capacity (pages * page_tokens) are skipped
// (padding entries of a slot mapping).  Grid: x = tokens / 4 (4 waves per
// work-group), y = kv heads.
#include "kernels.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr int kWaves = 4;

template <class T>
__device__ __forceinline__ float to_f32(T x) {
  if constexpr (std::is_same<T, float>::value) return x;
  else return float(x);
}

template <class T>
__device__ __forceinline__ void quantize_row(const T* __restrict__ src, uint32_t D, uint32_t lane, int8_t (&code)[4],
                                             float& scale) {
  float x[4];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    x[i] = d < D ? to_f32(src[d]) : 0.f;
    amax = fmaxf(amax, fabsf(x[i]));
  }
  amax = wave_max(amax);
  scale = amax == 0.f ? 1.f : amax / 127.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float c = __builtin_rintf(x[i] / scale);
    c = fminf(fmaxf(c, -127.f), 127.f);
    code[i] = int8_t(int(c));
  }
}

template <class T>
__global__ __launch_bounds__(64 * kWaves) void append_kernel(AppendArgs a) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t t = blockIdx.x * kWaves + wave;
  if (t >= a.tokens) return;
  const uint32_t kv = blockIdx.y;
  const uint32_t id = a.slots[t];
  if (id >= a.pages * a.page_tokens) return;  // padding entry
  const uint32_t page = id / a.page_tokens, slot = id % a.page_tokens;
  const uint32_t D = a.dim, P = a.page_tokens;
  const size_t row = (size_t(page) * a.kv_heads + kv) * P + slot;  // token row of this (page, kv)
  const T* ksrc = static_cast<const T*>(a.k_new) + size_t(t) * a.k_stride + size_t(kv) * D;
  const T* vsrc = static_cast<const T*>(a.v_new) + size_t(t) * a.v_stride + size_t(kv) * D;
  int8_t kc[4], vc[4];
  float ks, vs;
  quantize_row(ksrc, D, lane, kc, ks);
  quantize_row(vsrc, D, lane, vc, vs);
  int8_t* kdst = a.k + row * D;
  int8_t* vdst = a.v + (size_t(page) * a.kv_heads + kv) * D * P + slot;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    if (d < D) {
      kdst[d] = kc[i];
      vdst[size_t(d) * P] = vc[i];
    }
  }
  if (lane == 0) {
    a.k_scales[row] = ks;
    a.v_scales[row] = vs;
  }
}

}  // namespace

hipError_t launch_append(const AppendArgs& a, hipStream_t stream) {
  if (a.tokens == 0) return hipSuccess;
  const dim3 grid((a.tokens + kWaves - 1) / kWaves, a.kv_heads);
  switch (a.src_type) {
    case 1: hipLaunchKernelGGL(append_kernel<float>, grid, dim3(64 * kWaves), 0, stream, a); break;
    case 2: hipLaunchKernelGGL(append_kernel<_Float16>, grid, dim3(64 * kWaves), 0, stream, a); break;
    case 3: hipLaunchKernelGGL(append_kernel<__bf16>, grid, dim3(64 * kWaves), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t preload_append() {
  const void* fns[] = {reinterpret_cast<const void*>(&append_kernel<float>),
                       reinterpret_cast<const void*>(&append_kernel<_Float16>),
                       reinterpret_cast<const void*>(&append_kernel<__bf16>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvb
