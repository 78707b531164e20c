// Device helpers shared by the gfx950 kernels: exponent, wave64 reductions
// built from DPP row rotations and the gfx950 permlane swaps (pure VALU, no
// LDS traffic), and the exact INT8 -> f16 conversion used by the MFMA kernel.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace kvb {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// PV weight scaling of the int8-digit kernels: p = round(w * v_scale * 2^kp)
// with kp = 21 - exponent(v_max * kVmaxMargin) stays below 2^21 - 1 (w <= 1),
// so its top 7-bit digit is at most 127.  Without the margin a v_max just
// below a power of two could round p up to 2^21.
constexpr float kVmaxMargin = 1.0f + 1.0f / 1048576.0f;  // 1 + 2^-20

// e^x as 2^(x * log2 e) on the hardware base-2 exponential (v_exp_f32).
// exp(-inf) = 0.  Callers never pass NaN-producing (-inf) - (-inf).
__device__ __forceinline__ float exp_e(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }

// DPP row rotation by N lanes inside each 16-lane row.
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xF, 0xF, false));
}
// Broadcast lane J of each 16-lane row to the whole row (DPP row_newbcast).
template <int J>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + J, 0xF, 0xF, false));
}

// Combine x across the four 16-lane rows (lanes l, l^16, l^32, l^48) with the
// gfx950 permlane swaps.  The swap returns {row-pair mirror A, B}; op(A, B)
// is symmetric, so every lane ends with the same combination.
__device__ __forceinline__ float rows_max(float x) {
  auto p = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  x = fmaxf(__int_as_float(p[0]), __int_as_float(p[1]));
  auto q = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(q[0]), __int_as_float(q[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  auto p = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  x = __int_as_float(p[0]) + __int_as_float(p[1]);
  auto q = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float(q[0]) + __int_as_float(q[1]);
}
// Max over all 64 lanes, result in every lane.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, row_ror<8>(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<2>(x));
  x = fmaxf(x, row_ror<1>(x));
  return rows_max(x);
}
__device__ __forceinline__ float wave_sum(float x) {
  x += row_ror<8>(x);
  x += row_ror<4>(x);
  x += row_ror<2>(x);
  x += row_ror<1>(x);
  return rows_sum(x);
}

// Eight signed INT8 codes (two dwords) -> eight exactly equal f16 values.
// Flipping the sign bit turns code b into the unsigned byte u = b + 128; the
// f16 bit pattern 0x6400 | u is the value 1024 + u, so subtracting 1152 gives
// b exactly (every integer below 2048 is representable).  v_perm_b32 builds
// two such halves per instruction from the flipped dword and the 0x64 bytes.
__device__ __forceinline__ f16x8 i8x8_to_f16(uint32_t lo, uint32_t hi) {
  const uint32_t a = lo ^ 0x80808080u, b = hi ^ 0x80808080u;
  const uint32_t w0 = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
  const uint32_t w1 = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
  const uint32_t w2 = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
  const uint32_t w3 = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
  const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const f16x2 h0 = __builtin_bit_cast(f16x2, w0) - bias;
  const f16x2 h1 = __builtin_bit_cast(f16x2, w1) - bias;
  const f16x2 h2 = __builtin_bit_cast(f16x2, w2) - bias;
  const f16x2 h3 = __builtin_bit_cast(f16x2, w3) - bias;
  return f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// First t in [lo, hi) with kpos[t] > x, or hi (k_positions are nondecreasing).
// 64-ary search by the whole wave: each round samples 64 evenly spaced
// positions and keeps the sub-interval where the predicate flips.
__device__ inline uint32_t visible_end(const int64_t* __restrict__ kpos, uint32_t lo, uint32_t hi, int64_t x,
                                uint32_t lane) {
  while (hi - lo > 64u) {
    const uint32_t stride = (hi - lo + 63u) / 64u;
    const uint64_t t = uint64_t(lo) + uint64_t(lane) * stride;
    const bool p = t < hi && kpos[t] <= x;
    const uint32_t c = uint32_t(__popcll(__ballot(p)));
    if (c == 0) return lo;
    const uint64_t nhi = uint64_t(lo) + uint64_t(c) * stride;
    lo = lo + (c - 1u) * stride + 1u;
    hi = nhi < hi ? uint32_t(nhi) : hi;
  }
  const uint32_t t = lo + lane;
  const bool p = t < hi && kpos[t] <= x;
  return lo + uint32_t(__popcll(__ballot(p)));
}

__device__ __forceinline__ uint32_t clampu(uint32_t x, uint32_t lo, uint32_t hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

}  // namespace kvb
