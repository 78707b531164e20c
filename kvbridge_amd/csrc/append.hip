// Paged INT8 KV append (the write side of the cache format the split kernels
// read, include/kvbridge/attention_common.h): each new token's K and V rows
// of one kv head are quantized to symmetric int8 with a per-(token, kv head)
// fp32 scale and stored into its physical slot of the page pool:
//   scale = absmax / 127 (1 when absmax == 0, all codes 0),
//   code  = clamp(rint(x / scale), -127, 127)      (round half to even),
// with fp32 IEEE semantics throughout, max and clamp as fmaxf / fminf:
// non-finite sources give defined codes in every kernel -- NaN elements are
// left out of the absmax, an infinite element makes the scale infinite
// (finite elements then quantize to 0), and a NaN quotient (a NaN element,
// or infinity over an infinite scale) clamps to -127;
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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr uint32_t kTileMin = 256;  // tokens from which the tile kernel is used

template <class T>
__device__ __forceinline__ float to_f32(T x) {
  if constexpr (std::is_same<T, float>::value) return x;
  else return float(x);
}

// clamp(rint(x / scale), -127, 127) with x / scale the correctly rounded
// fp32 quotient, without the IEEE division sequence in the common case.
// q = x * rcp(scale) is within 1.25 * 2^-22 relative of x / scale
// (v_rcp_f32 is accurate to 1 ulp, the product adds half an ulp), i.e.
// within 4e-5 absolute for |q| <= 128, and the correctly rounded quotient is
// within half an ulp (<= 2^-18) of the exact one.  So wherever q lies more
// than 2^-13 away from a half-integer, the rounded quotient has the same
// nearest integer and is no tie: rint(q) is the answer.  The rest (about one
// element in 4,000, and any non-finite q, e.g. a subnormal scale) take the
// division.
__device__ __forceinline__ int8_t quantize(float x, float scale) {
  const float q = x * __builtin_amdgcn_rcpf(scale);
  float c = __builtin_rintf(q);
  if (!(fabsf(q - c) <= 0.5f - 0x1p-14f)) c = __builtin_rintf(x / scale);
  c = fminf(fmaxf(c, -127.f), 127.f);
  return int8_t(int(c));
}

constexpr float kRoundMagic = 12582912.f;  // 1.5 * 2^23

// The per-token scale absmax / 127 (1 for an all-zero row), bitwise the IEEE
// fp32 quotient: for finite absmax, q0 = RN(a * RN(1/127)) is within an ulp
// and one residual step fma(fma(-q0, 127, a), RN(1/127), q0) gives the
// correctly rounded quotient -- checked for every non-negative finite fp32
// value by tests/cpp/scale_div_check.c -- in three instructions instead of
// the division sequence.  An infinite absmax keeps the quotient (infinity).
__device__ __forceinline__ float scale_of(float amax) {
  constexpr float kInv127 = 1.0f / 127.0f;
  const float q0 = __fmul_rn(amax, kInv127);
  const float q = fmaf(fmaf(-q0, 127.f, amax), kInv127, q0);
  return amax == 0.f ? 1.f : (amax <= 3.4028234663852886e38f ? q : amax);
}

// |x| max of a lane's W 16-byte words of N elements of type T, as the bit
// pattern of a non-negative fp32 value (exact: max picks an element), NaN
// elements ignored like fmaxf does (as in the row and tile kernels).
// Non-negative floats order like their bit patterns, so the maxima are
// unsigned integer maxima of the patterns with the sign cleared (fp16 / bf16:
// two elements an instruction); a NaN (pattern above infinity's) wins that
// max, and such a lane (rare) is redone element by element.  nonfinite: the
// words hold an infinity or a NaN.
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
template <class T, uint32_t N, uint32_t W>
__device__ __forceinline__ uint32_t lane_absmax_bits(const u32x4 (&w)[W], bool& nonfinite) {
  auto slow = [&]() {
    float a = 0.f;
#pragma unroll
    for (uint32_t j = 0; j < W; ++j) {
      const T* e = reinterpret_cast<const T*>(&w[j]);
#pragma unroll
      for (uint32_t i = 0; i < N; ++i) a = fmaxf(a, fabsf(to_f32(e[i])));
    }
    return __float_as_uint(a);
  };
  if constexpr (sizeof(T) == 2) {
    constexpr uint16_t kInf = std::is_same<T, _Float16>::value ? 0x7c00u : 0x7f80u;
    u16x2 m = __builtin_bit_cast(u16x2, w[0][0] & 0x7fff7fffu);
#pragma unroll
    for (uint32_t j = 0; j < W; ++j)
#pragma unroll
      for (int k = (j == 0 ? 1 : 0); k < 4; ++k) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[j][k] & 0x7fff7fffu));
    const uint16_t b = m[0] > m[1] ? m[0] : m[1];
    nonfinite = b >= kInf;
    if (b > kInf) return slow();
    if constexpr (std::is_same<T, _Float16>::value) return __float_as_uint(float(__builtin_bit_cast(_Float16, b)));
    else return uint32_t(b) << 16;
  } else {
    uint32_t m = w[0][0] & 0x7fffffffu;
#pragma unroll
    for (uint32_t j = 0; j < W; ++j)
#pragma unroll
      for (int k = (j == 0 ? 1 : 0); k < 4; ++k) m = max(m, w[j][k] & 0x7fffffffu);
    nonfinite = m >= 0x7f800000u;
    if (m > 0x7f800000u) return slow();
    return m;
  }
}

// The codes of a lane's W words of N elements of one row, quantize()
// bitwise, with r the hardware reciprocal of the scale (within one ulp of
// 1/scale) and M = 1.5 * 2^23 (RN(q + M) holds rint(q), half to even, in its
// low mantissa bits).
//  - fp16 / bf16 sources: the quotient as q0 = RN(x * r), residual
//    fma(-q0, scale, x), q = fma(residual, r, q0) -- equal to the IEEE
//    quotient RN(x / scale) for every fp16 and bf16 row maximum a with scale
//    RN(a / 127) >= 2^-100, every such r and every source value |x| <= a
//    (exhaustive: tests/cpp/quant_fmadiv_check.c), so no element needs a
//    check.
//  - fp32 sources: with r_lo = RN(r * (1 - 2^-21)) and r_hi = RN(r * (1 +
//    2^-21)) the products x * r_lo and x * r_hi bracket RN(x / scale); fma(x,
//    r, M) rounds the exact product to the nearest integer, and rounding to
//    the nearest integer is monotone, so where both ends give the same
//    integer it is rint(RN(x / scale)) (tests/cpp/quant_bracket_check.c).
//    The ends are compared by sums of absolute differences of their low 16
//    bits (the two integers differ by at most 1), in two chains; a lane where
//    some pair differs (a quotient within ~2^-21 relative of a half-integer,
//    e.g. an exact tie) divides.
// A lane whose words hold a non-finite element, or whose row's reciprocal is
// not finite or scale below 2^-100 (force), takes the division and the clamp
// of quantize() (a NaN quotient gives -127).
template <class T, uint32_t N, uint32_t W>
__device__ __forceinline__ void quantize_lane(const u32x4 (&w)[W], float scale, float r_lo, float r_hi, bool force,
                                              uint32_t (&t)[W * N]) {
  uint32_t amb0 = force ? 1u : 0u, amb1 = 0u;
  const float r = r_lo;  // fp16 / bf16: the reciprocal itself (recip_of)
#pragma unroll
  for (uint32_t j = 0; j < W; ++j) {
    const T* e = reinterpret_cast<const T*>(&w[j]);
#pragma unroll
    for (uint32_t i = 0; i < N; ++i) {
      const float x = to_f32(e[i]);
      if constexpr (sizeof(T) == 2) {
        // RN(x * r + 0): an fma (fp16 x read in place by the mixed-precision
        // form); the +0 addend only turns a -0 product into +0, which gives
        // the same code, and keeps the compiler from making it a multiply.
        const float q0 = fmaf(x, r, 0.0f);
        const float q = fmaf(fmaf(-q0, scale, x), r, q0);
        t[N * j + i] = __float_as_uint(q + kRoundMagic);
      } else {
        const float lo = fmaf(x, r_lo, kRoundMagic);
        const float hi = fmaf(x, r_hi, kRoundMagic);
        if (i & 1u) amb1 = __builtin_amdgcn_sad_u16(__float_as_uint(lo), __float_as_uint(hi), amb1);
        else amb0 = __builtin_amdgcn_sad_u16(__float_as_uint(lo), __float_as_uint(hi), amb0);
        t[N * j + i] = __float_as_uint(lo);
      }
    }
  }
  if ((amb0 | amb1) != 0u) {  // rare: one branch per lane and row
#pragma unroll
    for (uint32_t j = 0; j < W; ++j) {
      const T* e = reinterpret_cast<const T*>(&w[j]);
#pragma unroll
      for (uint32_t i = 0; i < N; ++i)
        t[N * j + i] = __float_as_uint(fminf(fmaxf(__builtin_rintf(to_f32(e[i]) / scale), -127.f), 127.f) + kRoundMagic);
    }
  }
}

// The reciprocal terms of quantize_lane for one row's scale (fp16 / bf16: r
// in r_lo; fp32: the bracket), and force where the reciprocal is not finite
// or the scale is below 2^-100 (the range the CPU checks cover; subnormal
// scales in particular never reach the hardware reciprocal's fast path).
template <class T>
__device__ __forceinline__ void recip_of(float scale, float& r_lo, float& r_hi, bool& force) {
  const float r = __builtin_amdgcn_rcpf(scale);
  if constexpr (sizeof(T) == 2) {
    r_lo = r_hi = r;
    force = !(r <= 3.4028234663852886e38f) || !(scale >= 0x1p-100f);
  } else {
    r_lo = r * (1.0f - 0x1p-21f);
    r_hi = r * (1.0f + 0x1p-21f);
    force = !(r_hi <= 3.4028234663852886e38f) || !(scale >= 0x1p-100f);
  }
}

// Max over aligned groups of L lanes (L a power of two, 4..64), in every lane
// of the group, of non-negative fp32 bit patterns (unsigned maxima): DPP
// quad permutes and row mirrors inside a 16-lane row (each folded into one
// v_max_u32), then the gfx950 permlane swaps across rows.
template <uint32_t L>
__device__ __forceinline__ uint32_t group_max_bits(uint32_t x) {
  static_assert(L >= 4 && L <= 64 && (L & (L - 1)) == 0, "group size");
  auto dpp = [](uint32_t v, auto ctrl) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  x = max(x, dpp(x, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  x = max(x, dpp(x, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  if constexpr (L >= 8) x = max(x, dpp(x, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  if constexpr (L >= 16) x = max(x, dpp(x, std::integral_constant<int, 0x140>{}));  // row_mirror
  if constexpr (L >= 32) {
    auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = max(uint32_t(p[0]), uint32_t(p[1]));
  }
  if constexpr (L >= 64) {
    auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    x = max(uint32_t(p[0]), uint32_t(p[1]));
  }
  return x;
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
  scale = scale_of(amax);
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
  const float ks = scale_of(kamax);
  const float vs = scale_of(vamax);
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

// append_stream_kernel (prefill-sized appends from 16-byte aligned rows, dim
// 64/128/256): one work-group of eight waves per (64 new tokens, kv head).
// Wave w holds tokens 8w .. 8w + 7, eight lanes per token row: word j of a
// lane is elements 16 / sizeof(T) * (8j + sub) .. of its row (sub = lane %
// 8), so every load instruction reads whole 128-byte lines and every row is
// read once.  The row absmax is a three-step DPP max over the eight lanes,
// and the per-row work (scale, reciprocal) is shared by twice the elements
// per lane of a sixteen-lane split (the same kernel with sixteen lanes per
// row and a checked bracket rounding ran 6.62 us against 5.09 us at 4,096
// fp16 tokens, its divisions at exact fp16 ties included).  K codes go out
// as 8-byte (fp16 / bf16) or 4-byte pieces of each word.  V codes are
// transposed through LDS ([dim][64 tokens], 68-byte rows) and stored 16
// tokens per 16-byte store where those 16 tokens fill 16 consecutive slots
// of one page starting on a 16-slot boundary (a prefill chunk); any other
// group of 16 is stored byte by byte.
// The pool stores are non-temporal (streaming): the codes are not read again
// by this launch, and cached write-back stores measured slower (4,096 /
// 16,384 / 65,536 tokens at d128: 8.2 / 23.2 / 86.8 us against 7.9 / 21.9 /
// 69.4 us).  The source loads stay cached: non-temporal loads were slower.
// Eight waves of eight tokens rather than four of sixteen: the work-group's
// arithmetic (absmax, scale, codes) is a dependent chain per token row, and
// twice the waves per SIMD hide each other's latency (4,096 tokens at d128:
// 6.54 against 7.21 us).
constexpr int kStreamWaves = 8;
template <class T, int D, bool P2>  // P2: page_tokens is a power of two
__global__ __launch_bounds__(64 * kStreamWaves) void append_stream_kernel(AppendArgs a) {
  constexpr uint32_t EPL = 16 / sizeof(T);  // elements per 16-byte word
  constexpr uint32_t LPR = 8;               // lanes per row
  constexpr uint32_t WPL = D / EPL / LPR;   // words per lane and row
  static_assert(WPL >= 1 && D % (EPL * LPR) == 0, "row split");
  constexpr uint32_t TPW = 64u / LPR;       // tokens per wave
  static_assert(TPW * kStreamWaves == 64u, "64 tokens per work-group");
  // V codes [d][token] with 68-byte rows: a lane's code bytes go to dim rows
  // EPL apart, so the lanes of a token row hit different LDS banks (64-byte
  // rows put them all on one bank).
  constexpr uint32_t VR = 68;
  __shared__ __attribute__((aligned(16))) uint8_t vt[D * VR];
  __shared__ uint32_t ids[64];
  __shared__ uint32_t grp_ok[4];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t kv = blockIdx.x, t0 = blockIdx.y * 64u;  // the kv heads of a tile are consecutive work-groups
  const uint32_t P = a.page_tokens, cap = a.pages * a.page_tokens;
  const uint32_t psh = __builtin_ctz(P);
  auto page_of = [&](uint32_t id) { return P2 ? id >> psh : id / P; };
  auto slot_of = [&](uint32_t id) { return P2 ? id & (P - 1u) : id % P; };
  const uint32_t sub = lane % LPR, r = TPW * wave + lane / LPR;  // r: token of the tile
  // Word j of a lane holds elements EPL * (LPR * j + sub) .. + EPL - 1 of its
  // row, so each load instruction reads whole 128-byte lines of the rows.
  auto elem0 = [&](uint32_t j) { return EPL * (LPR * j + sub); };
  // Every source load of the wave first (they do not depend on the slot
  // ids), so they are all in flight together; then the slot ids.
  u32x4 wk[WPL], wv[WPL];
  {
    const uint32_t t = t0 + r;
#pragma unroll
    for (uint32_t j = 0; j < WPL; ++j) {
      if (t < a.tokens) {
        wk[j] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.k_new) + size_t(t) * a.k_stride +
                                                size_t(kv) * D + elem0(j));
        wv[j] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.v_new) + size_t(t) * a.v_stride +
                                                size_t(kv) * D + elem0(j));
      } else {
        wk[j] = wv[j] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  if (wave == 0) {
    const uint32_t t = t0 + lane;
    const uint32_t id = t < a.tokens ? a.slots[t] : cap;
    ids[lane] = id;
    const uint32_t id0 = __shfl(id, int(lane & ~15u));
    const bool ok = id < cap && id == id0 + (lane & 15u) && id0 % 16u == 0u;
    const uint64_t b = __ballot(ok);
    if ((lane & 15u) == 0u) grp_ok[lane >> 4] = ((b >> (lane & ~15u)) & 0xffffull) == 0xffffull ? 1u : 0u;
  }
  __syncthreads();
  {
    const uint32_t id = ids[r];
    bool knf, vnf;
    const uint32_t ka = group_max_bits<LPR>(lane_absmax_bits<T, EPL, WPL>(wk, knf));  // the row's lanes are an aligned group
    const uint32_t va = group_max_bits<LPR>(lane_absmax_bits<T, EPL, WPL>(wv, vnf));
    const float ks = scale_of(__uint_as_float(ka));
    const float vs = scale_of(__uint_as_float(va));
    float klo, khi, vlo, vhi;
    bool kf, vf;
    recip_of<T>(ks, klo, khi, kf);
    recip_of<T>(vs, vlo, vhi, vf);
    uint32_t tk[WPL * EPL], tv[WPL * EPL];
    quantize_lane<T, EPL, WPL>(wk, ks, klo, khi, kf || knf, tk);
    quantize_lane<T, EPL, WPL>(wv, vs, vlo, vhi, vf || vnf, tv);
#pragma unroll
    for (uint32_t j = 0; j < WPL; ++j)
#pragma unroll
      for (uint32_t e = 0; e < EPL; ++e) vt[(elem0(j) + e) * VR + r] = uint8_t(tv[EPL * j + e]);
    if (id < cap) {
      const size_t row = (size_t(page_of(id)) * a.kv_heads + kv) * P + slot_of(id);
#pragma unroll
      for (uint32_t j = 0; j < WPL; ++j) {
        uint32_t kw[EPL / 4];
#pragma unroll
        for (uint32_t e = 0; e < EPL / 4; ++e) {  // low bytes of four codes
          const uint32_t* const c = tk + EPL * j + 4 * e;
          kw[e] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(c[3], c[2], 0x0c0c0400u),
                                        __builtin_amdgcn_perm(c[1], c[0], 0x0c0c0400u), 0x05040100u);
        }
        int8_t* const kdst = a.k + row * D + elem0(j);
        if constexpr (EPL == 8) __builtin_nontemporal_store(u32x2{kw[0], kw[1]}, reinterpret_cast<u32x2*>(kdst));
        else __builtin_nontemporal_store(kw[0], reinterpret_cast<uint32_t*>(kdst));
      }
      if (sub == 0) {
        __builtin_nontemporal_store(ks, a.k_scales + row);
        __builtin_nontemporal_store(vs, a.v_scales + row);
      }
    }
  }
  __syncthreads();
  // V: item (d, group q) of D * 4, one per thread at D = 128.
  for (uint32_t it = threadIdx.x; it < D * 4u; it += 64u * kStreamWaves) {
    const uint32_t d = it >> 2, q = it & 3u;
    const uint8_t* const src = vt + d * VR + 16u * q;
    if (grp_ok[q]) {
      const uint32_t id = ids[16u * q];
      int8_t* const dst = a.v + (size_t(page_of(id)) * a.kv_heads + kv) * D * P + size_t(d) * P + slot_of(id);
      const uint32_t* const s4 = reinterpret_cast<const uint32_t*>(src);  // 4-byte aligned rows
      __builtin_nontemporal_store(u32x4{s4[0], s4[1], s4[2], s4[3]}, reinterpret_cast<u32x4*>(dst));
    } else {
#pragma unroll 4
      for (uint32_t j = 0; j < 16u; ++j) {
        const uint32_t id = ids[16u * q + j];
        if (id < cap) a.v[(size_t(page_of(id)) * a.kv_heads + kv) * D * P + size_t(d) * P + slot_of(id)] = int8_t(src[j]);
      }
    }
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
  // Row-streaming kernel: 16-byte aligned sources and strides, aligned K and V
  // pools, whole 16-slot groups in a page.
  const bool stream_ok = vec && reinterpret_cast<uintptr_t>(a.v) % 16 == 0 && a.page_tokens % 16 == 0 &&
                         (a.tokens + 63u) / 64u <= 65535u;  // tiles on grid.y
  const dim3 sgrid(a.kv_heads, (a.tokens + 63u) / 64u);
  if (stream_ok) {
    const bool p2 = (a.page_tokens & (a.page_tokens - 1u)) == 0u;
    auto go = [&](auto dc) {
      constexpr int DD = decltype(dc)::value;
      if (p2) hipLaunchKernelGGL((append_stream_kernel<T, DD, true>), sgrid, dim3(64 * kStreamWaves), 0, stream, a);
      else hipLaunchKernelGGL((append_stream_kernel<T, DD, false>), sgrid, dim3(64 * kStreamWaves), 0, stream, a);
    };
    if (a.dim == 64) { go(std::integral_constant<int, 64>{}); return hipGetLastError(); }
    if (a.dim == 128) { go(std::integral_constant<int, 128>{}); return hipGetLastError(); }
    if (a.dim == 256) { go(std::integral_constant<int, 256>{}); return hipGetLastError(); }
  }
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
                       reinterpret_cast<const void*>(&append_tile_kernel<__bf16, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<float, 64, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<float, 64, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<float, 128, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<float, 128, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<float, 256, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<float, 256, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<_Float16, 64, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<_Float16, 64, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<_Float16, 128, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<_Float16, 128, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<_Float16, 256, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<_Float16, 256, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<__bf16, 64, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<__bf16, 64, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<__bf16, 128, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<__bf16, 128, false>),
                       reinterpret_cast<const void*>(&append_stream_kernel<__bf16, 256, true>),
                       reinterpret_cast<const void*>(&append_stream_kernel<__bf16, 256, false>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvb
