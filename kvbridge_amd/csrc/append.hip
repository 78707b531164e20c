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
// implementation of the same formula.  Slot ids at or past the pool's
// capacity (pages * page_tokens) are skipped (padding entries of a slot
// mapping).  Two kernels, same results:
//
// append_row_kernel (few tokens, e.g. one decode step): one wave per
// (token, kv head); lane i holds dims i, i+64, ... (D <= 256), the absmax
// is a wave reduction.  Grid: x = tokens / 4 (4 waves per work-group), y =
// kv heads.
//
// append_tile_kernel (prefill-sized appends): one work-group per (64
// consecutive new tokens, kv head), lane = token, wave w = a quarter of the
// dims.  Each wave reads its dims of the tokens' rows twice (absmax, then
// quantize; the second read hits the cache); the four partial absmaxes meet
// in LDS.  K codes go out in 16-byte pieces of each token's row, V codes one
// dim at a time: lane i writes token i's byte of the dim row, so tokens that
// fill consecutive slots of a page -- a prefill chunk -- make one contiguous
// 64-byte store per dim instead of 64 single-byte stores strided by
// page_tokens (arbitrary slots still work: every lane has its own address).
// VEC: 16-byte source loads and K stores (host-checked alignment and sizes;
// then every quarter is a multiple of 16 dims).
#include "kernels.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr int kWaves = 4;
constexpr uint32_t kTileMin = 256;  // tokens from which the tile kernel is used

template <class T>
__device__ __forceinline__ float to_f32(T x) {
  if constexpr (std::is_same<T, float>::value) return x;
  else return float(x);
}

__device__ __forceinline__ int8_t quantize(float x, float scale) {
  float c = __builtin_rintf(x / scale);
  c = fminf(fmaxf(c, -127.f), 127.f);
  return int8_t(int(c));
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
  for (int i = 0; i < 4; ++i) code[i] = quantize(x[i], scale);
}

template <class T>
__global__ __launch_bounds__(64 * kWaves) void append_row_kernel(AppendArgs a) {
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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 consecutive source elements of a row as floats (VEC: 16-byte loads).
template <class T, bool VEC>
__device__ __forceinline__ void load16(const T* __restrict__ p, float (&x)[16]) {
  if constexpr (VEC) {
    constexpr int kPer = 16 / int(sizeof(T));  // elements per 16-byte load
#pragma unroll
    for (int c = 0; c < 16 / kPer; ++c) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(p + kPer * c);
      const T* e = reinterpret_cast<const T*>(&w);
#pragma unroll
      for (int i = 0; i < kPer; ++i) x[kPer * c + i] = to_f32(e[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = to_f32(p[i]);
  }
}

// Absmax of src[d0 .. d1).
template <class T, bool VEC>
__device__ __forceinline__ float part_absmax(const T* __restrict__ src, uint32_t d0, uint32_t d1) {
  float amax = 0.f;
  uint32_t d = d0;
  for (; d + 16u <= d1; d += 16u) {
    float x[16];
    load16<T, VEC>(src + d, x);
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
  }
  for (; d < d1; ++d) amax = fmaxf(amax, fabsf(to_f32(src[d])));
  return amax;
}

template <class T, bool VEC>
__global__ __launch_bounds__(64 * kWaves) void append_tile_kernel(AppendArgs a) {
  __shared__ float amax_s[2][kWaves][64];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t kv = blockIdx.y;
  const uint32_t t = blockIdx.x * 64u + lane;
  const uint32_t D = a.dim, P = a.page_tokens, cap = a.pages * a.page_tokens;
  const uint32_t dq = VEC ? D / kWaves : (D + kWaves - 1) / kWaves;  // dims per wave
  const uint32_t d0 = wave * dq < D ? wave * dq : D, d1 = d0 + dq < D ? d0 + dq : D;
  const bool live = t < a.tokens;
  const uint32_t id = live ? a.slots[t] : cap;
  const T* ksrc = static_cast<const T*>(a.k_new) + size_t(live ? t : 0u) * a.k_stride + size_t(kv) * D;
  const T* vsrc = static_cast<const T*>(a.v_new) + size_t(live ? t : 0u) * a.v_stride + size_t(kv) * D;
  amax_s[0][wave][lane] = live ? part_absmax<T, VEC>(ksrc, d0, d1) : 0.f;
  amax_s[1][wave][lane] = live ? part_absmax<T, VEC>(vsrc, d0, d1) : 0.f;
  __syncthreads();
  if (id >= cap) return;  // past the last token, or a padding entry
  float kamax = amax_s[0][0][lane], vamax = amax_s[1][0][lane];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    kamax = fmaxf(kamax, amax_s[0][w][lane]);
    vamax = fmaxf(vamax, amax_s[1][w][lane]);
  }
  const float ks = kamax == 0.f ? 1.f : kamax / 127.f;
  const float vs = vamax == 0.f ? 1.f : vamax / 127.f;
  const size_t row = (size_t(id / P) * a.kv_heads + kv) * P + id % P;  // token row of this (page, kv)
  if (wave == 0) {
    a.k_scales[row] = ks;
    a.v_scales[row] = vs;
  }
  int8_t* const kdst = a.k + row * D;
  int8_t* const vdst = a.v + (size_t(id / P) * a.kv_heads + kv) * D * P + id % P;
  uint32_t d = d0;
  for (; d + 16u <= d1; d += 16u) {
    float x[16];
    load16<T, VEC>(ksrc + d, x);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i / 4] |= (uint32_t(uint8_t(quantize(x[i], ks))) << (8 * (i % 4)));
    if constexpr (VEC) {
      *reinterpret_cast<u32x4*>(kdst + d) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) kdst[d + i] = int8_t(w[i / 4] >> (8 * (i % 4)));
    }
    load16<T, VEC>(vsrc + d, x);
#pragma unroll
    for (int i = 0; i < 16; ++i) vdst[size_t(d + i) * P] = quantize(x[i], vs);
  }
  for (; d < d1; ++d) {
    kdst[d] = quantize(to_f32(ksrc[d]), ks);
    vdst[size_t(d) * P] = quantize(to_f32(vsrc[d]), vs);
  }
}

template <class T>
hipError_t launch_typed(const AppendArgs& a, hipStream_t stream) {
  if (a.tokens < kTileMin) {
    hipLaunchKernelGGL(append_row_kernel<T>, dim3((a.tokens + kWaves - 1) / kWaves, a.kv_heads),
                       dim3(64 * kWaves), 0, stream, a);
    return hipGetLastError();
  }
  // 16-byte loads and K stores: sources, strides, rows and the K pool aligned.
  const uint32_t es = sizeof(T);
  const bool vec = reinterpret_cast<uintptr_t>(a.k_new) % 16 == 0 && reinterpret_cast<uintptr_t>(a.v_new) % 16 == 0 &&
                   (uint64_t(a.k_stride) * es) % 16 == 0 && (uint64_t(a.v_stride) * es) % 16 == 0 &&
                   a.dim % (16u * kWaves) == 0 && reinterpret_cast<uintptr_t>(a.k) % 16 == 0;
  const dim3 grid((a.tokens + 63u) / 64u, a.kv_heads);
  if (vec) hipLaunchKernelGGL((append_tile_kernel<T, true>), grid, dim3(64 * kWaves), 0, stream, a);
  else hipLaunchKernelGGL((append_tile_kernel<T, false>), grid, dim3(64 * kWaves), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_append(const AppendArgs& a, hipStream_t stream) {
  if (a.tokens == 0) return hipSuccess;
  switch (a.src_type) {
    case 1: return launch_typed<float>(a, stream);
    case 2: return launch_typed<_Float16>(a, stream);
    case 3: return launch_typed<__bf16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t preload_append() {
  const void* fns[] = {reinterpret_cast<const void*>(&append_row_kernel<float>),
                       reinterpret_cast<const void*>(&append_row_kernel<_Float16>),
                       reinterpret_cast<const void*>(&append_row_kernel<__bf16>),
                       reinterpret_cast<const void*>(&append_tile_kernel<float, true>),
                       reinterpret_cast<const void*>(&append_tile_kernel<float, false>),
                       reinterpret_cast<const void*>(&append_tile_kernel<_Float16, true>),
                       reinterpret_cast<const void*>(&append_tile_kernel<_Float16, false>),
                       reinterpret_cast<const void*>(&append_tile_kernel<__bf16, true>),
                       reinterpret_cast<const void*>(&append_tile_kernel<__bf16, false>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvb
