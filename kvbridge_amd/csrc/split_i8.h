// Integer-MFMA split-partial kernel for paged INT8 KV with few grouped
// head-rows per KV head (head_rows = rows * q_heads/kv_heads <= 8).
//
// The INT8 codes are never converted: both contractions run on
// v_mfma_i32_16x16x64_i8 with the raw K and V bytes as the A operand.
//  * QK: Q of each head-row is scaled by a power of two to a 23-bit integer
//    and split into three int8 digits (q = hi*2^16 + mid*2^8 + lo, exact).
//    The digits of all head-rows sit side by side in the 16 MFMA columns
//    (column = digit * HS + head), so one MFMA per 64 dims gives all three
//    digit dot products for 16 tokens.
//  * PV: the weights w * v_scale are scaled by 2^kp to integers below 2^21
//    and split into three 7-bit digits (p = d0*2^14 + d1*2^7 + d2); the
//    per-digit integer numerators accumulate exactly in int32.
// Digit recombination and the softmax run in a transposed view where each
// lane owns one token of the tile for every head-row (data moves through a
// small per-wave LDS exchange area), so no VALU work is spent on padding
// columns.
//
// Two passes per chunk of up to 4 tiles: the K images of the chunk are
// streamed first (scores kept in registers, exact chunk maximum), then the V
// images; the int32 numerators therefore never need an online rescale and
// are folded into fp32 once per chunk.
//
// Staging: K and V bytes go from HBM straight into VGPRs, already in the
// MFMA operand layout, with non-temporal 16-byte buffer loads (per-lane
// constant voffset; the descriptor is rebased per tile on its page, so
// every access is bounded by the page).  Each wave keeps a ring of NB item
// slots in registers and issues item j+NB-1 before computing item j; items
// run in fixed chunks (K images of 4 tiles, then their V images) so every
// ring slot is a compile-time register set and the issue is unconditional
// (an item past the wave's last tile gets a zero-sized descriptor and moves
// no data), which lets the compiler's wait-count pass keep exact
// per-register waits.  Eight waves per work-group (two per SIMD) where the
// state fits in 256 registers.
//
// Partial layout and semantics are those of every split kernel here:
// scratch[((row*q_heads + head)*splits + split)*(dim+2) + col], col 0 = split
// max score (natural log units), 1 = sum of exp(score - max), 2.. =
// sum of exp(score - max) * v_scale * v_code -- except in the single launch
// whose merge takes the short path, which packs the same values differently
// in the same scratch (PackedPartials below).
#pragma once
#include <cstdint>

#include "kernels.h"
#include "batch.h"
#include "device_common.h"
#include "lds_stream.h"
#include "merge_rows.h"

namespace kvb {
namespace {

using lds::static_for;
using lds::u32x4_t;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kTileTokens = 64;
constexpr int kChunk = 4;                    // tiles per two-pass chunk
constexpr float kLn2 = 0.6931471805599453f;
constexpr int32_t kRsrcWord3 = 0x00020000;   // raw 32-bit buffer, gfx9 dword3

// ---- loads.  Compiler builtins, so that its wait-count pass tracks every
// loaded register (in-order vmcnt; exact for this static schedule).
constexpr int kAuxNT = 2;  // non-temporal
__device__ __forceinline__ u32x4_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), kAuxNT);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, int(voff), int(soff), kAuxNT);
}
__device__ __forceinline__ u32x4_t gload16(const int8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ uint32_t gload4(const float* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// One item in registers: the K image (d[mb * D/64 + j] = 16 bytes of K row
// 16*(m/4) + 4*mb + m%4, dims 64*j + 16*g ..; with PAIR the half-row layout
// below) plus k- and v-scale of token lane, or the V image (d[mb] = V row
// 16*mb + m, slots 16g .. 16g+15), which reuses its tile's scales.
template <int D>
struct Slot {
  u32x4_t d[D / 16];
  uint32_t ks, vs;
};

struct IssueCtx {
  __amdgpu_buffer_rsrc_t rk, rv, rks, rvs;  // whole-array descriptors (small-page path)
  uint32_t voff_k, voff_v, voff_s;          // per-lane constant offsets (page-tile path)
  const int8_t* k;
  const int8_t* v;
  const float* ks;
  const float* vs;
  const uint32_t* table;
  uint32_t kv, kv_heads, P, lg_p, pages, lp_lo, lp_hi, lane, ptab;
  uint32_t kv_bytes, sc_bytes;  // small-page path: whole-array sizes (< 4 GiB)
};

typedef const __attribute__((address_space(4))) uint32_t* const_u32_ptr;

// Physical page of logical page lp (uniform), clamped to the split's pages
// and to the pool; the first 64 come from the wave's page-table window.
__device__ __forceinline__ uint32_t page_of(const IssueCtx& c, uint32_t lp) {
  lp = clampu(lp, c.lp_lo, c.lp_hi);
  const uint32_t rel = lp - c.lp_lo;
  uint32_t x = rel < 64u ? uint32_t(__builtin_amdgcn_readlane(int(c.ptab), int(rel)))
                         : ((const_u32_ptr)(c.table))[lp];  // scalar load
  x = uint32_t(__builtin_amdgcn_readfirstlane(int(x)));
  return x < c.pages ? x : c.pages - 1u;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), kRsrcWord3);
}

// Issue one item (D/16 + 2 loads for K, D/16 for V, unconditionally: an
// item past the wave's last tile gets zero-sized descriptors, so its loads
// return 0 and move no data).  PT: page_tokens is a power of two >= 64, the tile lies in one page
// and the descriptors are rebased on it (any pool size).  Otherwise
// page_tokens is 16 or 32: every 16-token group lies in one page and lanes
// address their group's page through whole-array descriptors.
// PAIR (K image of the paired-row QK layout): MFMA row m of M-block mb is
// half m%2 of token 8*mb + m/2, so the 16 lanes of a k-block read 8 rows x
// 2 segments of one 128-byte line each instead of 16 rows.
template <int D, bool PT, bool IS_V, bool PAIR>
__device__ __forceinline__ void issue_item(const IssueCtx& c, uint32_t tile, bool real, Slot<D>& s) {
  const uint32_t t0 = tile * kTileTokens;
  if constexpr (PT) {
    const uint64_t slab = page_of(c, t0 >> c.lg_p) * uint64_t(c.kv_heads) + c.kv;
    const uint32_t slot0 = t0 & (c.P - 1u);
    const uint64_t tok = slab * c.P + slot0;
    if constexpr (!IS_V && PAIR) {
      const __amdgpu_buffer_rsrc_t r = rsrc(c.k + tok * D, real ? 64u * D : 0u);
#pragma unroll
      for (uint32_t mb = 0; mb < 8; ++mb) s.d[mb] = bload16(r, c.voff_k + 1024u * mb, 0u);
    } else if constexpr (!IS_V) {
      const __amdgpu_buffer_rsrc_t r = rsrc(c.k + tok * D, real ? 64u * D : 0u);
      static_for<0, 4>([&](auto mbc) __attribute__((always_inline)) {
        constexpr uint32_t mb = decltype(mbc)::value;
        static_for<0, D / 64>([&](auto jc) __attribute__((always_inline)) {
          constexpr uint32_t j = decltype(jc)::value;
          s.d[mb * (D / 64) + j] = bload16(r, c.voff_k + (4 * mb * D + 64 * j), 0u);
        });
      });
    } else {
      const __amdgpu_buffer_rsrc_t r = rsrc(c.v + slab * D * c.P + slot0, real ? D * c.P - slot0 : 0u);
#pragma unroll
      for (uint32_t mb = 0; mb < D / 16; ++mb) s.d[mb] = bload16(r, c.voff_v, 16u * mb * c.P);
    }
    if constexpr (!IS_V) {  // the tile's V item reuses these
      s.ks = bload4(rsrc(c.ks + tok, real ? 256u : 0u), c.voff_s, 0u);
      s.vs = bload4(rsrc(c.vs + tok, real ? 256u : 0u), c.voff_s, 0u);
    }
  } else {
    const uint32_t lane = c.lane, m = lane & 15u, g = lane >> 4;
    uint32_t slab[4];  // slab of token group q (tokens t0+16q ..), uniform
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) slab[q] = page_of(c, (t0 + 16u * q) >> c.lg_p) * c.kv_heads + c.kv;
    auto pick = [&](uint32_t q) __attribute__((always_inline)) {
      return q == 0 ? slab[0] : (q == 1 ? slab[1] : (q == 2 ? slab[2] : slab[3]));
    };
    const __amdgpu_buffer_rsrc_t none = rsrc(c.k, 0u);
    if constexpr (!IS_V && PAIR) {
      const __amdgpu_buffer_rsrc_t r = real ? c.rk : none;
      static_for<0, 8>([&](auto mbc) __attribute__((always_inline)) {
        constexpr uint32_t mb = decltype(mbc)::value;
        constexpr uint32_t q = mb >> 1;  // 16-token group of tokens 8*mb ..
        const uint32_t row = pick(q) * c.P + ((t0 + 16u * q) & (c.P - 1u)) + 8u * (mb & 1u) + (m >> 1);
        s.d[mb] = bload16(r, row * uint32_t(D) + 64u * (m & 1u) + 16u * g, 0u);
      });
    } else if constexpr (!IS_V) {
      const uint32_t grp = m >> 2;
      const uint32_t row = pick(grp) * c.P + ((t0 + 16u * grp) & (c.P - 1u)) + (m & 3u);
      const uint32_t voff = row * uint32_t(D) + 16u * g;
      const __amdgpu_buffer_rsrc_t r = real ? c.rk : none;
      static_for<0, 4>([&](auto mbc) __attribute__((always_inline)) {
        constexpr uint32_t mb = decltype(mbc)::value;
        static_for<0, D / 64>([&](auto jc) __attribute__((always_inline)) {
          constexpr uint32_t j = decltype(jc)::value;
          s.d[mb * (D / 64) + j] = bload16(r, voff + (4 * mb * D + 64 * j), 0u);
        });
      });
    } else {
      const uint32_t voff = (pick(g) * uint32_t(D) + m) * c.P + ((t0 + 16u * g) & (c.P - 1u));
      const __amdgpu_buffer_rsrc_t r = real ? c.rv : none;
#pragma unroll
      for (uint32_t mb = 0; mb < D / 16; ++mb) s.d[mb] = bload16(r, voff, 16u * mb * c.P);
    }
    if constexpr (!IS_V) {  // the tile's V item reuses these
      const uint32_t si = (pick(g) * c.P + ((t0 + 16u * g) & (c.P - 1u)) + m) * 4u;
      s.ks = bload4(real ? c.rks : none, si, 0u);
      s.vs = bload4(real ? c.rvs : none, si, 0u);
    }
  }
}

template <int D, int NW, int HS>
struct I8Layout {
  static constexpr int NC = (3 * HS + 15) / 16;       // MFMA column tiles
  static constexpr uint32_t kExchCol = 272;           // int32 column of 64 tokens + pad
  static constexpr uint32_t kDigCol = 80;             // int8 column of 64 tokens + pad
  static constexpr uint32_t kExch = NC * 16 * kExchCol;
  static constexpr uint32_t kDig = NC * 16 * kDigCol;
  static constexpr uint32_t kWave = kExch + kDig;
  // Wave combine area after the exchange areas: [NW][HS] maxima, [NW][HS]
  // denominators, [NW][HS][D] numerators.
  static constexpr uint32_t kComb = NW * kWave;
  // Q digit area after it: [64 lanes][kQdBytes] (written before the main
  // loop, read by every wave; waves with no tiles reach the combine early,
  // so it must not overlap the combine area).
  static constexpr bool kPair = D == 128 && HS <= 4;  // paired-row QK layout
  static constexpr uint32_t kQdBytes = (kPair ? 2 : NC) * (kPair ? 1 : D / 64) * 16;
  static constexpr uint32_t kQd = kComb + NW * HS * (D + 2) * 4;
  static constexpr uint32_t kBytes = kQd + 64 * kQdBytes;
};

// Agent-scope (all XCDs) coherent load of a partial written by another
// work-group with an agent-scope atomic store.
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The single launch's short merge (at most 32 splits, one output column per
// thread) reads a packed partial layout of its own instead of the
// [row-head][split][m, l, n] rows above (same size, internal to the call):
//   m: scratch[rh*splits + j]             (RS = rows * q_heads * splits)
//   l: scratch[RS + rh*splits + j]
//   n: scratch[2*RS + (rh*splits + j)*D + d]
// so the merger's (m_j, l_j) of one row-head are one 128-byte line each
// instead of a line per split, and every 256-byte numerator request of a
// wave covers two whole 128-byte lines (numerator rows start 512-byte apart,
// at a 128-byte boundary when the scratch base has one) instead of three.
// The merge is bound by those line requests: agent-scope loads miss the
// L2, and one work-group issues all of them.
template <int D>
struct PackedPartials {
  const size_t rs;
  float* base;
  __device__ __forceinline__ PackedPartials(float* scratch, const SplitArgs& a)
      : rs(size_t(a.rows) * a.q_heads * a.splits), base(scratch) {}
  __device__ __forceinline__ float* m(size_t rh, uint32_t splits, uint32_t j) const { return base + rh * splits + j; }
  __device__ __forceinline__ float* l(size_t rh, uint32_t splits, uint32_t j) const { return base + rs + rh * splits + j; }
  __device__ __forceinline__ float* n(size_t rh, uint32_t splits, uint32_t j) const {
    return base + 2 * rs + (rh * splits + j) * D;
  }
};

// Whether the single launch's merge takes the short path (and so the packed
// layout): every work-group of the kernel evaluates the same condition.
template <int D, int NW>
__device__ __forceinline__ bool short_merge(uint32_t ns, uint32_t head_rows) {
  return ns <= 32u && head_rows * uint32_t(D) <= 64u * NW;
}

// Merge of all splits of one kv head's head-rows, by the last work-group,
// with the reference merge semantics (src/attention_shared.cu:295-335):
// M = max_j m_j; L = sum_{l_j > 0} e^{m_j - M} l_j; N[d] likewise (N summed
// in split order, L by a wave tree); an all-empty head-row gives M = -inf,
// L = 0, N = 0.  Optional normalized output out = L > 0 ? N / L : 0 (fp32 or
// fp16).  Splits 0 .. ns-1 are merged; a.splits is the partial stride.
// f_s: LDS [8][32] split factors (the merge_rows area when that runs),
// ml_s: LDS [8][2] (M, L).
template <int D, int NW, int HS>
__device__ __forceinline__ void fused_merge(const SplitArgs& a, uint32_t kv, uint32_t head_rows, uint32_t ns,
                                            const float* __restrict__ scratch, float* f_s, float* ml_s) {
  constexpr uint32_t W = D + 2;
  constexpr uint32_t kCh = 32;  // splits per pass
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t outs = head_rows * D;
  auto row_head = [&](uint32_t hh) __attribute__((always_inline)) {
    return size_t(hh / a.group) * a.q_heads + kv * a.group + hh % a.group;
  };
  // Common case (<= 32 splits, one output per thread; the packed partial
  // layout): straight-line code that requests every operand at once -- the
  // wave's (m_j, l_j) and the thread's 32 numerators, split indices clamped
  // instead of branched on -- so the merge costs one memory round trip.  The
  // 64 outputs of a wave lie in one head-row (64 divides D), so every wave
  // turns its own head-row's (m_j, l_j) into the factors e^{m_j - M} (lane j
  // holds split j) and reads them back with readlane: no LDS exchange and no
  // work-group barrier.
  if (short_merge<D, NW>(ns, head_rows)) {
    static_assert(D % 64 == 0, "a wave's outputs lie in one head-row");
    static_assert(kCh == 32, "the short merge covers 32 splits");
    if (64u * wave >= outs) return;
    const uint32_t jmax = ns - 1u;
    const uint32_t hh = (64u * wave) / D;
    const PackedPartials<D> pp(const_cast<float*>(scratch), a);
    const size_t rhh = row_head(hh);
    const uint32_t jl = lane < ns ? lane : jmax;
    const float mj = ld_agent(pp.m(rhh, a.splits, jl));
    const float lj = ld_agent(pp.l(rhh, a.splits, jl));
    const uint32_t d = tid % D;
    // Numerator j of column d through one descriptor over the head-row's
    // numerator rows, with the row offset in the instruction's scalar offset
    // (no per-load vector address arithmetic); agent-coherent cache policy.
    // Rows past ns - 1 re-read row ns - 1 and are masked below.
    const float* nb = pp.n(rhh, a.splits, 0) + d;
    float pre[kCh];
#pragma unroll
    for (uint32_t j = 0; j < kCh; ++j) pre[j] = ld_agent(nb + size_t(j < jmax ? j : jmax) * D);
    const bool in = lane < ns;
    const float mx = wave_max(in ? mj : neg_inf());
    const float f = in && lj > 0.f ? exp_e(mj - mx) : 0.f;
    const float lsum = wave_sum(f * lj);
    // The factors reach every lane as LDS broadcasts (this wave's own 32
    // floats of f_s), and the 32 products go into four interleaved sums
    // added as (s0 + s1) + (s2 + s3): a fixed order, four times shorter
    // dependency chains.
    float* const fw = f_s + wave * kCh;
    if (lane < kCh) fw[lane] = f;
    float fv[kCh];
#pragma unroll
    for (uint32_t q4 = 0; q4 < kCh / 4u; ++q4) {
      const float4 x = reinterpret_cast<const float4*>(fw)[q4];
      fv[4 * q4] = x.x;
      fv[4 * q4 + 1] = x.y;
      fv[4 * q4 + 2] = x.z;
      fv[4 * q4 + 3] = x.w;
    }
    float s4[4] = {0.f, 0.f, 0.f, 0.f};
    if (ns == kCh) {
#pragma unroll
      for (uint32_t j = 0; j < kCh; ++j) s4[j & 3u] = fmaf(fv[j], pre[j], s4[j & 3u]);
    } else {
#pragma unroll
      for (uint32_t j = 0; j < kCh; ++j) s4[j & 3u] = fmaf(fv[j], j <= jmax ? pre[j] : 0.f, s4[j & 3u]);
    }
    const float nacc = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    const size_t rh = row_head(hh);
    if (d == 0) {
      a.m[rh] = mx;
      a.l[rh] = lsum;
    }
    a.n[rh * D + d] = nacc;
    if (a.out_type != 0) {
      const float ov = lsum > 0.f ? nacc / lsum : 0.f;
      if (a.out_type == 1) static_cast<float*>(a.out)[rh * D + d] = ov;
      else static_cast<_Float16*>(a.out)[rh * D + d] = (_Float16)ov;
    }
    return;
  }
  // Otherwise, where a thread can own four columns of a head-row: merge_rows
  // (16-byte agent-coherent loads by split groups, one round trip per pass).
  if constexpr (uint32_t(HS) * D / 4u <= 64u * NW) {
    merge_rows<D, NW, HS, true>(
        head_rows, ns, [&](uint32_t hh) { return scratch + row_head(hh) * a.splits * W; }, f_s,
        [&](uint32_t hh, uint32_t q, float4 nv, float mv, float lv) {
          const size_t rh = row_head(hh);
          if (q == 0) {
            a.m[rh] = mv;
            a.l[rh] = lv;
          }
          float* const nd = a.n + rh * D + 4u * q;  // caller buffers need only 4-byte alignment
          nd[0] = nv.x;
          nd[1] = nv.y;
          nd[2] = nv.z;
          nd[3] = nv.w;
          if (a.out_type != 0) {
            const float o[4] = {lv > 0.f ? nv.x / lv : 0.f, lv > 0.f ? nv.y / lv : 0.f,
                                lv > 0.f ? nv.z / lv : 0.f, lv > 0.f ? nv.w / lv : 0.f};
            if (a.out_type == 1) {
              float* const od = static_cast<float*>(a.out) + rh * D + 4u * q;
              for (int i = 0; i < 4; ++i) od[i] = o[i];
            } else {
              _Float16* const oh = static_cast<_Float16*>(a.out) + rh * D + 4u * q;
              for (int i = 0; i < 4; ++i) oh[i] = (_Float16)o[i];
            }
          }
        });
    return;
  }
  // General case: passes of 32 splits; the running numerator goes through n.
  for (uint32_t j0 = 0; j0 < ns; j0 += kCh) {
    const uint32_t cnt = ns - j0 < kCh ? ns - j0 : kCh;
    for (uint32_t hh = wave; hh < head_rows; hh += NW) {
      const float* base = scratch + row_head(hh) * a.splits * W;
      const bool in = lane < cnt;  // lanes >= 32 idle
      const float mj = in ? ld_agent(base + size_t(j0 + lane) * W) : neg_inf();
      const float lj = in ? ld_agent(base + size_t(j0 + lane) * W + 1) : 0.f;
      float mx;
      if (j0 == 0) {  // M over every split (later passes reuse it)
        mx = mj;
        for (uint32_t j = kCh + lane; j < ns; j += 64u) mx = fmaxf(mx, ld_agent(base + size_t(j) * W));
        mx = wave_max(mx);
      } else {
        mx = ml_s[2 * hh];
      }
      const float f = lj > 0.f ? exp_e(mj - mx) : 0.f;
      const float lsum = wave_sum(f * lj);
      if (lane < kCh) f_s[hh * kCh + lane] = f;
      if (lane == 0) {
        ml_s[2 * hh] = mx;
        ml_s[2 * hh + 1] = (j0 == 0 ? 0.f : ml_s[2 * hh + 1]) + lsum;
      }
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < outs; idx += 64u * NW) {
      const uint32_t hh = idx / D, d = idx % D;
      const float* fh = f_s + hh * kCh;
      const size_t rh = row_head(hh);
      float nacc = 0.f;
      {
        const float* base = scratch + rh * a.splits * W + 2 + d;
        const uint32_t jm = j0 + cnt - 1u;
        float nv[kCh];
#pragma unroll
        for (uint32_t j = 0; j < kCh; ++j) nv[j] = ld_agent(base + size_t(j0 + j < jm ? j0 + j : jm) * W);
        if (j0 != 0) nacc = a.n[rh * D + d];
#pragma unroll
        for (uint32_t j = 0; j < kCh; ++j) nacc = fmaf(fh[j], j < cnt ? nv[j] : 0.f, nacc);
      }
      if (j0 + kCh < ns) {
        a.n[rh * D + d] = nacc;  // running numerator, re-read by this thread next pass
        continue;
      }
      const float lsum = ml_s[2 * hh + 1];
      if (d == 0) {
        a.m[rh] = ml_s[2 * hh];
        a.l[rh] = lsum;
      }
      a.n[rh * D + d] = nacc;
      if (a.out_type != 0) {
        const float o = lsum > 0.f ? nacc / lsum : 0.f;
        if (a.out_type == 1) static_cast<float*>(a.out)[rh * D + d] = o;
        else static_cast<_Float16*>(a.out)[rh * D + d] = (_Float16)o;
      }
    }
    __syncthreads();
  }
}

// VARLEN: batched call, grid.z = sequence (arguments rebased per work-group).
// The leading scalar arguments are everything the first KV request depends
// on; the translation units that instantiate this kernel are built with
// kernel-argument preloading for them (the dispatcher places them in SGPRs),
// so the page-table load is issued without waiting for a kernel-argument
// load.  They duplicate fields of a_in, which the kernel overrides with them.
//
// FENCE (one diagnostic instance, kvb_decode_attention_fused_fenced): the
// single launch with the formal agent-scope release fence before every
// ticket and an acquire fence after the merger's -- the ordering the other
// instances get from agent-scope atomic partials, without the L2 write-back
// and invalidate these fences add.
template <int D, int NW, int NB, bool PT, int HS, bool FUSED, bool VARLEN, bool FENCE>
__global__ __launch_bounds__(64 * NW) void split_i8_kernel(
    const uint32_t* __restrict__ table_in, const int8_t* __restrict__ kdata, const float* __restrict__ kscale,
    const float* __restrict__ vscale, uint32_t p_begin, uint32_t p_end, uint32_t p_split_tokens,
    uint32_t p_page_tokens, uint32_t p_kv_heads, uint32_t p_pages, SplitArgs a_in,
    const float* __restrict__ q_in, const int64_t* __restrict__ qpos_in, const int64_t* __restrict__ kpos_in,
    const int8_t* __restrict__ vdata, float* __restrict__ scratch_in) {
  SplitArgs a = a_in;
  a.begin = p_begin;
  a.end = p_end;
  a.split_tokens = p_split_tokens;
  a.page_tokens = p_page_tokens;
  a.kv_heads = p_kv_heads;
  a.pages = p_pages;
  if constexpr (VARLEN) rebase_sequence(a, blockIdx.z);
  const float* __restrict__ q = VARLEN ? a.q : q_in;
  const int64_t* __restrict__ qpos = VARLEN ? a.q_positions : qpos_in;
  const int64_t* __restrict__ kpos = VARLEN ? a.k_positions : kpos_in;
  const uint32_t* __restrict__ table = VARLEN ? a.page_table : table_in;
  float* __restrict__ scratch = VARLEN ? a.scratch : scratch_in;
  using L = I8Layout<D, NW, HS>;
  constexpr int NC = L::NC;  // MFMA column tiles of the digit columns (PV; QK unless PAIR)
  // Paired-row QK (dim 128, <= 4 head-rows): MFMA row m of M-block mb is
  // half m%2 (dims 64*(m%2) ..) of token 8*mb + m/2; column tile h of the Q
  // digits holds half h, so rows and tiles of equal half give the two half
  // dot products of a token, which add exactly in int32.  The K loads of a
  // k-block then read whole 64-byte half rows, two per 128-byte line.
  constexpr bool PAIR = L::kPair;
  constexpr int NCQ = PAIR ? 2 : NC;        // MFMA column tiles of the QK B operand
  constexpr int KS = PAIR ? 1 : D / 64;     // 64-dim steps per QK M-block
  __shared__ __attribute__((aligned(16))) uint8_t smem[L::kBytes];

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t n = lane & 15u, g = lane >> 4;
  const uint32_t split = blockIdx.x;
  const uint32_t kv = blockIdx.y;
  const uint32_t head_rows = a.rows * a.group;  // <= HS
  // Splits that take part in the fused merge.  A batched single-launch call
  // merges only the sequence's own splits (at least one, so that an empty
  // sequence still gets its empty result); work-groups past them write no
  // partial and take no ticket.  In a two-launch batched call they write the
  // empty partial (m = -inf, l = 0, n = 0) straight away, without loading
  // anything.
  uint32_t nsplit = a.splits;
  if constexpr (VARLEN) {
    nsplit = a.end > 0u ? (a.end - 1u) / a.split_tokens + 1u : 1u;
    if (split >= nsplit) {
      if constexpr (!FUSED) {
        constexpr uint32_t W = D + 2;
        for (uint32_t o = threadIdx.x; o < head_rows * W; o += 64u * NW) {
          const uint32_t hh = o / W, col = o % W;
          const uint32_t row2 = hh / a.group, head2 = kv * a.group + hh % a.group;
          scratch[((size_t(row2) * a.q_heads + head2) * a.splits + split) * W + col] = col == 0 ? neg_inf() : 0.f;
        }
      }
      return;
    }
  }

  const uint64_t s0_64 = uint64_t(a.begin) + uint64_t(split) * a.split_tokens;
  const uint32_t s0 = s0_64 < a.end ? uint32_t(s0_64) : a.end;
  const uint32_t s1 = uint64_t(s0) + a.split_tokens < a.end ? s0 + a.split_tokens : a.end;
  const uint32_t k_first = s0 / kTileTokens;

  IssueCtx c;
  c.k = kdata;
  c.v = vdata;
  c.ks = kscale;
  c.vs = vscale;
  c.table = table;
  c.kv = kv;
  c.kv_heads = a.kv_heads;
  c.P = a.page_tokens;
  c.pages = a.pages;
  c.lp_lo = s0 / a.page_tokens;
  c.lp_hi = s1 > s0 ? (s1 - 1u) / a.page_tokens : c.lp_lo;
  c.lane = lane;
  c.lg_p = 31u - __builtin_clz(a.page_tokens);  // page_tokens is a power of two
  {
    // Page-table window of the split (no load for an empty split, whose
    // lp_lo may be one past the last page).
    const uint32_t lp = c.lp_lo + lane;
    c.ptab = s1 > s0 && lp <= c.lp_hi ? table[lp] : 0u;
  }
  if constexpr (PT) {
    c.voff_k = PAIR ? 128u * (n >> 1) + 64u * (n & 1u) + 16u * g
                    : (16u * (n >> 2) + (n & 3u)) * uint32_t(D) + 16u * g;
    c.voff_v = n * a.page_tokens + 16u * g;
    c.voff_s = 4u * lane;
  } else {
    const uint32_t kv_bytes = a.pages * a.kv_heads * a.page_tokens * uint32_t(D);  // < 4 GiB (host check)
    const uint32_t sc_bytes = a.pages * a.kv_heads * a.page_tokens * 4u;
    c.rk = rsrc(kdata, kv_bytes);
    c.rv = rsrc(vdata, kv_bytes);
    c.rks = rsrc(kscale, sc_bytes);
    c.rvs = rsrc(vscale, sc_bytes);
  }

  // Per-wave LDS exchange areas (plain LDS accesses: the compiler inserts
  // the MFMA-result hazards and lgkmcnt waits).
  uint8_t* const wbase = smem + wave * L::kWave;

  // ---- everything the KV stream and the Q digits depend on is loaded in
  // one memory round trip: the page-table window (above), the split's last
  // key position, the query positions, and the Q elements this lane turns
  // into MFMA digit columns (straight into registers; no LDS staging and no
  // work-group barrier before the stream starts).
  const int64_t klast = s1 > s0 ? kpos[s1 - 1u] : 0;
  int64_t qp[HS];
#pragma unroll
  for (int r = 0; r < HS; ++r) qp[r] = qpos[uint32_t(r) < a.rows ? uint32_t(r) : 0u];
  // Lane (n, g) of MFMA column tile nc feeds a digit column: column
  // 16*nc + n (digit dg = col / HS of head-row col % HS), or with PAIR column
  // n of tile nc = half nc.  MFMA s of a 64-dim step takes dims 64*s + 16*g
  // .. +15 of Q and K alike (PAIR: dims 64*nc + 16*g ..), so the K loads
  // read whole 64-byte row segments.
  float qv[NCQ][16 * KS];
#pragma unroll
  for (int nc = 0; nc < NCQ; ++nc) {
    const uint32_t col = PAIR ? n : 16u * nc + n;
    const uint32_t h = col % HS;
    const bool valid = col < 3u * HS && h < head_rows;
    const uint32_t hq = valid ? h : 0u;
    const float* src = q + (size_t(hq / a.group) * a.q_heads + kv * a.group + hq % a.group) * D + 16u * g +
                       (PAIR ? 64u * nc : 0u);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 w = reinterpret_cast<const float4*>(src + 64 * s)[j];
        qv[nc][16 * s + 4 * j] = valid ? w.x : 0.f;
        qv[nc][16 * s + 4 * j + 1] = valid ? w.y : 0.f;
        qv[nc][16 * s + 4 * j + 2] = valid ? w.z : 0.f;
        qv[nc][16 * s + 4 * j + 3] = valid ? w.w : 0.f;
      }
    }
  }

  // ---- visibility per head-row: tokens [s0, eh[h]) (k_positions nondecreasing)
  uint32_t eh[HS];
  {
    uint32_t erow[HS];
#pragma unroll
    for (int r = 0; r < HS; ++r) {
      erow[r] = s0;
      if (s1 > s0 && uint32_t(r) < a.rows)
        erow[r] = klast <= qp[r] ? s1 : visible_end(kpos, s0, s1, qp[r], lane);
    }
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      const uint32_t r = uint32_t(h) / a.group;
      uint32_t e = s0;
#pragma unroll
      for (int rr = 0; rr < HS; ++rr)
        if (uint32_t(rr) == r) e = erow[rr];
      eh[h] = uint32_t(h) < head_rows ? __builtin_amdgcn_readfirstlane(e) : s0;
    }
  }
  uint32_t e_min = 0xffffffffu, e_max = s0;
#pragma unroll
  for (int h = 0; h < HS; ++h) {
    if (uint32_t(h) < head_rows) e_min = eh[h] < e_min ? eh[h] : e_min;
    e_max = eh[h] > e_max ? eh[h] : e_max;
  }

  // ---- the wave's tiles (round-robin over the work-group).  Items run in
  // chunks of 2*kChunk: K images of tiles 4c..4c+3, then their V images.
  // Items of tiles past the wave's last tile load nothing (zero-sized
  // descriptors); their stale slot contents are masked by tok_ok and zero
  // weights.
  const uint32_t k_vis = e_max > s0 ? (e_max - 1u) / kTileTokens : 0u;
  const uint32_t k_count = e_max > s0 ? k_vis + 1u - k_first : 0u;
  const uint32_t nt = k_count > wave ? (k_count - wave + NW - 1u) / NW : 0u;
  const uint32_t n_chunks = (nt + kChunk - 1u) / kChunk;
  auto tile_k = [&](uint32_t i) __attribute__((always_inline)) { return k_first + wave + i * NW; };
  // Item at chunk position POS (0 .. 2*kChunk-1) of chunk ch.
  auto issue = [&](auto posc, uint32_t ch, Slot<D>& slot) __attribute__((always_inline)) {
    constexpr uint32_t pos = decltype(posc)::value;
    const uint32_t i = ch * kChunk + pos % kChunk;
    issue_item<D, PT, (pos >= uint32_t(kChunk)), PAIR>(c, tile_k(i), i < nt, slot);
  };
  Slot<D> ring[NB];
  // Start streaming before the Q digits are built.
  static_for<0, NB - 1>([&](auto uc) __attribute__((always_inline)) { issue(uc, 0u, ring[decltype(uc)::value]); });

  // ---- Q digits (B operand of QK) and per-head score factors.  A column's
  // scale 2^kq comes from its head-row's whole Q row (with PAIR both tiles
  // of a lane hold the same column).  Every wave needs the same digits (its
  // lanes are the same MFMA columns), so the digit dwords are built once per
  // work-group: wave w builds dwords d = w, w + NW, ... of every lane and
  // stores them in the Q digit area of LDS; after one barrier (LDS only: the
  // first KV item stays in flight) each wave reads its lanes' digits back.
  i32x4 qd[NCQ][KS];
  float cql[HS];
  static_assert(L::kQdBytes == NCQ * KS * 16, "digit bytes per lane");
  uint8_t* const qd_s = smem + L::kQd + lane * L::kQdBytes;
  {
    int kq_lane = 0;
    auto col_kq = [&](float amax) __attribute__((always_inline)) {
      amax = rows_max(amax);
      int kq = 0;
      if (amax > 0.f) {
        kq = 22 - __builtin_amdgcn_frexp_expf(amax);  // |2^kq q| < 2^22: top digit in [-64, 64]
        kq = kq < -100 ? -100 : (kq > 100 ? 100 : kq);
      }
      return kq;
    };
    int kq_pair = 0;
    if constexpr (PAIR) {
      float amax = 0.f;
#pragma unroll
      for (int nc = 0; nc < NCQ; ++nc)
#pragma unroll
        for (int i = 0; i < 16 * KS; ++i) amax = fmaxf(amax, fabsf(qv[nc][i]));
      kq_pair = col_kq(amax);
    }
#pragma unroll
    for (int nc = 0; nc < NCQ; ++nc) {
      const uint32_t col = PAIR ? n : 16u * nc + n;
      const uint32_t dg = col / HS;
      const bool valid = col < 3u * HS && col % HS < head_rows;
      int kq = kq_pair;
      if constexpr (!PAIR) {
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 16 * KS; ++i) amax = fmaxf(amax, fabsf(qv[nc][i]));
        kq = col_kq(amax);
      }
      if (nc == 0) kq_lane = kq;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t dw = (uint32_t(nc) * KS + s) * 4u + j;  // digit dword of the lane
          if (dw % NW != wave) continue;                       // uniform: built by wave dw % NW
          uint32_t packed = 0;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int qi = int(__builtin_rintf(__builtin_amdgcn_ldexpf(qv[nc][16 * s + 4 * j + b], kq)));
            const int lo = int(int8_t(qi & 0xff));
            const int r1 = (qi - lo) >> 8;
            const int mid = int(int8_t(r1 & 0xff));
            const int hi = (r1 - mid) >> 8;
            const int d = dg == 0 ? hi : (dg == 1 ? mid : lo);
            packed |= (uint32_t(d) & 0xffu) << (8 * b);
          }
          *reinterpret_cast<uint32_t*>(qd_s + 4u * dw) = valid ? packed : 0u;
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int nc = 0; nc < NCQ; ++nc)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4_t w = *reinterpret_cast<const u32x4_t*>(qd_s + 16u * (uint32_t(nc) * KS + s));
        qd[nc][s] = i32x4{int(w[0]), int(w[1]), int(w[2]), int(w[3])};
      }
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      const int kq = __builtin_amdgcn_readlane(kq_lane, h);
      cql[h] = __builtin_amdgcn_ldexpf(a.scale, -kq) * kLog2e;
    }
  }

  uint8_t* const exch_w = wbase + n * L::kExchCol + 64u * g;              // C write base (MFMA view)
  uint8_t* const exch_w2 = wbase + n * L::kExchCol + 8u * g;              // PAIR: summed C write base
  const uint8_t* const exch_r = wbase + 4u * lane;                        // lane-as-token read base
  uint8_t* const dig_w = wbase + L::kExch + lane;                         // digit write (lane-as-token)
  const uint8_t* const dig_r = wbase + L::kExch + n * L::kDigCol + 16u * g;  // B operand read

  // State.  Lane-as-token view: sc, mx, lw, lrun per head-row.  MFMA view:
  // int32 digit numerators acc_i, fp32 numerators acc_f (head = lane & 15).
  float sc[kChunk][HS];
  float vsc[kChunk];  // v-scale of token lane, per tile of the chunk
  float mx[HS], lw[HS], lrun[HS];
  float m_run[HS], m_new[HS], mu[HS];
  float vmx = 0.f;
  int kp = 0;
  i32x4 acc_i[NC][D / 16];
  f32x4 acc_f[D / 16];
#pragma unroll
  for (int h = 0; h < HS; ++h) {
    mx[h] = neg_inf();
    lw[h] = 0.f;
    lrun[h] = 0.f;
    m_run[h] = neg_inf();
    m_new[h] = neg_inf();
    mu[h] = 0.f;
#pragma unroll
    for (int r = 0; r < kChunk; ++r) sc[r][h] = neg_inf();
  }
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) {
    acc_f[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nc = 0; nc < NC; ++nc) acc_i[nc][mb] = i32x4{0, 0, 0, 0};
  }

  // ---- pass 1 item: scores of chunk tile r (tile index i).
  auto process_k = [&](auto rc, uint32_t i, const Slot<D>& it) __attribute__((always_inline)) {
    constexpr uint32_t r = decltype(rc)::value;
    const uint32_t t0 = tile_k(i) * kTileTokens;
    const uint32_t tok = t0 + lane;
    const bool real = i < nt;
    const bool full = real && t0 >= s0 && t0 + kTileTokens <= e_min;
    const bool tok_ok = full || (real && tok >= s0 && tok < e_max);
    if constexpr (PAIR) {
      // Rows 4g+e of M-block mb: e even = half 0, e odd = half 1 of tokens
      // 8mb+2g (e < 2) and 8mb+2g+1; tile 0 gives the half-0 and tile 1 the
      // half-1 dot products, summed exactly here.
      static_for<0, 8>([&](auto mbc) __attribute__((always_inline)) {
        constexpr uint32_t mb = decltype(mbc)::value;
        const u32x4_t w = it.d[mb];
        const i32x4 av = {int(w[0]), int(w[1]), int(w[2]), int(w[3])};
        const i32x4 zero = {0, 0, 0, 0};
        const i32x4 c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, qd[0][0], zero, 0, 0, 0);
        const i32x4 c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, qd[1][0], zero, 0, 0, 0);
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t cw = {uint32_t(c0[0] + c1[1]), uint32_t(c0[2] + c1[3])};
        *reinterpret_cast<u32x2_t*>(exch_w2 + 32 * mb) = cw;
      });
    } else {
      static_for<0, NC>([&](auto ncc) __attribute__((always_inline)) {
        constexpr uint32_t nc = decltype(ncc)::value;
        static_for<0, 4>([&](auto mbc) __attribute__((always_inline)) {
          constexpr uint32_t mb = decltype(mbc)::value;
          i32x4 cc = {0, 0, 0, 0};
#pragma unroll
          for (int s = 0; s < D / 64; ++s) {
            const u32x4_t w = it.d[mb * (D / 64) + s];
            const i32x4 av = {int(w[0]), int(w[1]), int(w[2]), int(w[3])};
            cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, qd[nc][s], cc, 0, 0, 0);
          }
          const u32x4_t cw = {uint32_t(cc[0]), uint32_t(cc[1]), uint32_t(cc[2]), uint32_t(cc[3])};
          *reinterpret_cast<u32x4_t*>(exch_w + (nc * 16 * L::kExchCol + 16 * mb)) = cw;
        });
      });
    }
    int dv[HS][3];
    static_for<0, HS>([&](auto hc) __attribute__((always_inline)) {
      constexpr uint32_t h = decltype(hc)::value;
      static_for<0, 3>([&](auto dc) __attribute__((always_inline)) {
        constexpr uint32_t dg = decltype(dc)::value;
        constexpr uint32_t col = dg * HS + h;
        dv[h][dg] = *reinterpret_cast<const int*>(exch_r + col * L::kExchCol);
      });
    });
    const float ks_l = __uint_as_float(it.ks);
    const float vs_l = __uint_as_float(it.vs);
    vsc[r] = vs_l;  // for the tile's V item (which loads no scales)
    vmx = fmaxf(vmx, tok_ok ? fabsf(vs_l) : 0.f);
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      const float si = fmaf(fmaf(float(dv[h][0]), 256.f, float(dv[h][1])), 256.f, float(dv[h][2]));
      float s2 = si * (ks_l * cql[h]);
      if (!full && !(real && tok >= s0 && tok < eh[h])) s2 = neg_inf();
      if (uint32_t(h) >= head_rows) s2 = neg_inf();
      sc[r][h] = s2;
      mx[h] = fmaxf(mx[h], s2);
    }
  };

  // ---- pass 2 item: weights of chunk tile r, PV.
  auto process_v = [&](auto rc, uint32_t i, const Slot<D>& it) __attribute__((always_inline)) {
    constexpr uint32_t r = decltype(rc)::value;
    const uint32_t t0 = tile_k(i) * kTileTokens;
    const uint32_t tok = t0 + lane;
    const bool real = i < nt;
    const bool tok_ok = real && ((t0 >= s0 && t0 + kTileTokens <= e_min) || (tok >= s0 && tok < e_max));
    const float vs_l = tok_ok ? vsc[r] : 0.f;
    static_for<0, HS>([&](auto hc) __attribute__((always_inline)) {
      constexpr uint32_t h = decltype(hc)::value;
      const float w = __builtin_amdgcn_exp2f(sc[r][h] - mu[h]);  // w * 2^kp
      lw[h] += w;
      // p = w * v_scale rounded to an integer (0 <= p < 2^21) in one fma:
      // 1.5 * 2^23 + p lies in [2^23, 2^24), where the float's ulp is 1, so
      // its low 22 bits are p mod 2^22 (two's complement), and bits 0-6,
      // 7-13 and 14-21 are the three digits of p.
      const uint32_t pb = __float_as_uint(fmaf(w, vs_l, 12582912.f));
      const uint32_t d0 = (pb >> 14) & 0xffu;
      const uint32_t d1 = (pb >> 7) & 0x7fu;
      const uint32_t d2 = pb & 0x7fu;
      dig_w[h * L::kDigCol] = uint8_t(d0);
      dig_w[(HS + h) * L::kDigCol] = uint8_t(d1);
      dig_w[(2 * HS + h) * L::kDigCol] = uint8_t(d2);
    });
    u32x4_t bd[NC];
    static_for<0, NC>([&](auto ncc) __attribute__((always_inline)) {
      constexpr uint32_t nc = decltype(ncc)::value;
      bd[nc] = *reinterpret_cast<const u32x4_t*>(dig_r + nc * 16 * L::kDigCol);
    });
#pragma unroll
    for (int nc = 0; nc < NC; ++nc) {
      const i32x4 bv = {int(bd[nc][0]), int(bd[nc][1]), int(bd[nc][2]), int(bd[nc][3])};
#pragma unroll
      for (int mb = 0; mb < D / 16; ++mb) {
        const u32x4_t w = it.d[mb];
        const i32x4 av = {int(w[0]), int(w[1]), int(w[2]), int(w[3])};
        acc_i[nc][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, acc_i[nc][mb], 0, 0, 0);
      }
    }
  };

  // ---- chunk maximum and weight exponent kp (after the chunk's K items).
  auto chunk_max = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      const float mc = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_max(mx[h]))));
      m_new[h] = fmaxf(m_run[h], mc);
      mx[h] = neg_inf();
    }
    const float vmax = wave_max(vmx);
    vmx = 0.f;
    kp = 0;
    if (vmax > 0.f) {
      kp = 21 - __builtin_amdgcn_frexp_expf(vmax * kVmaxMargin);
      kp = kp < -100 ? -100 : (kp > 100 ? 100 : kp);
    }
#pragma unroll
    for (int h = 0; h < HS; ++h) mu[h] = (m_new[h] == neg_inf() ? 0.f : m_new[h]) - float(kp);
  };

  // ---- fold the chunk's int32 digit numerators into the fp32 state.
  auto fold = [&]() __attribute__((always_inline)) {
    float fh[HS];
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      fh[h] = m_run[h] == neg_inf() ? 0.f : __builtin_amdgcn_exp2f(m_run[h] - m_new[h]);
      lrun[h] = fmaf(lrun[h], fh[h], __builtin_amdgcn_ldexpf(lw[h], -kp));
      lw[h] = 0.f;
      m_run[h] = m_new[h];
    }
    float f_lane = 0.f;  // head (lane & 15) of the MFMA view
#pragma unroll
    for (int h = 0; h < HS; ++h)
      if (n == uint32_t(h)) f_lane = fh[h];
    const float inv = __builtin_amdgcn_ldexpf(1.f, -kp);
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // digit dg of head h is column dg*HS + h: tile (dg*HS+h)/16, lane shift (dg*HS)%16.
        const float x0 = float(acc_i[0][mb][e]);
        float x1, x2;
        if constexpr (HS <= 5) {
          x1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x0), 0x100 + HS, 0xF, 0xF, true));
          x2 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x0), 0x100 + 2 * HS, 0xF, 0xF, true));
        } else {
          x1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x0), 0x100 + (HS % 16), 0xF, 0xF, true));
          x2 = float(acc_i[NC - 1][mb][e]);  // column 2*HS + h = 16 + h for HS == 8
        }
        const float comb = fmaf(fmaf(x0, 128.f, x1), 128.f, x2);
        acc_f[mb][e] = fmaf(acc_f[mb][e], f_lane, comb * inv);
      }
#pragma unroll
      for (int nc = 0; nc < NC; ++nc) acc_i[nc][mb] = i32x4{0, 0, 0, 0};
    }
  };

  // ---- main loop: one chunk per iteration, items unrolled so that ring
  // slots (item % NB, NB divides 2*kChunk) are compile-time.
  static_assert((2 * kChunk) % NB == 0, "ring size must divide the chunk");
  for (uint32_t ch = 0; ch < n_chunks; ++ch) {
    static_for<0, 2 * kChunk>([&](auto uc) __attribute__((always_inline)) {
      constexpr uint32_t u = decltype(uc)::value;
      issue(std::integral_constant<uint32_t, (u + NB - 1) % (2 * kChunk)>(), ch + (u + NB - 1) / (2 * kChunk),
            ring[(u + NB - 1) % NB]);
      if constexpr (u < uint32_t(kChunk)) {
        process_k(std::integral_constant<uint32_t, u>(), ch * kChunk + u, ring[u % NB]);
        if constexpr (u == uint32_t(kChunk) - 1) chunk_max();
      } else {
        process_v(std::integral_constant<uint32_t, u - kChunk>(), ch * kChunk + (u - kChunk), ring[u % NB]);
        if constexpr (u == 2u * kChunk - 1) fold();
      }
    });
  }

  // ---- combine the waves through LDS and write the split partial.  Each
  // wave publishes its maxima, denominators and numerators in its own rows
  // of the combine area (disjoint from every exchange area, so no barrier is
  // needed before), then one barrier.  Each output then requests the NW
  // wave values of its column together (independent LDS loads, one latency)
  // and adds them in wave order; a wave with no visible token (m = -inf)
  // contributes factor 0 to its zero values, which leaves the sum unchanged.
  float* const wm_s = reinterpret_cast<float*>(smem + L::kComb);  // [NW][HS]
  float* const wl_s = wm_s + NW * HS;                              // [NW][HS]
  float* const wacc_s = wl_s + NW * HS;                            // [NW][HS][D]
#pragma unroll
  for (int h = 0; h < HS; ++h) {
    const float lsum = wave_sum(lrun[h]);
    if (lane == 0) {
      wm_s[wave * HS + h] = m_run[h] * kLn2;
      wl_s[wave * HS + h] = lsum;
    }
  }
  if (n < uint32_t(HS)) {
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) {
      float4 y;
      y.x = acc_f[mb][0];
      y.y = acc_f[mb][1];
      y.z = acc_f[mb][2];
      y.w = acc_f[mb][3];
      *reinterpret_cast<float4*>(&wacc_s[(wave * HS + n) * D + 16 * mb + 4 * g]) = y;
    }
  }
  __syncthreads();
  // One numerator column per thread and iteration (no branches: the LDS
  // loads of all waves are requested together); the thread of column 0 also
  // writes the head-row's maximum and denominator.
  constexpr uint32_t W = D + 2;
  for (uint32_t o = threadIdx.x; o < head_rows * uint32_t(D); o += 64u * NW) {
    // A wave's 64 columns lie in one head-row (64 divides D), so the NW
    // wave maxima, denominators and factors of its iteration are scalars:
    // lane w < NW reads wave w's pair and computes its factor once.
    const uint32_t hh = __builtin_amdgcn_readfirstlane(o / D), d = o % D;
    const uint32_t wl = lane < uint32_t(NW) ? lane : 0u;
    const float m_l = wm_s[wl * HS + hh], l_l = wl_s[wl * HS + hh];
    float mw[NW], lv[NW], xw[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      mw[w] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m_l), w));
      lv[w] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l_l), w));
      xw[w] = wacc_s[(w * HS + hh) * D + d];
    }
    float mm = mw[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mm = fmaxf(mm, mw[w]);
    const float f_l = m_l == neg_inf() ? 0.f : exp_e(m_l - mm);
    float val = 0.f, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f_l), w));
      val = fmaf(f, xw[w], val);
      lsum = fmaf(f, lv[w], lsum);
    }
    const uint32_t row2 = hh / a.group, head2 = kv * a.group + hh % a.group;
    const size_t rh = size_t(row2) * a.q_heads + head2;
    float* const dst = scratch + (rh * a.splits + split) * W;
    if constexpr (FUSED) {  // agent-coherent; the short merge's packed layout or the rows
      const bool packed = short_merge<D, NW>(nsplit, head_rows);
      const PackedPartials<D> pp(scratch, a);
      float* const pn = packed ? pp.n(rh, a.splits, split) : dst + 2;
      float* const pm = packed ? pp.m(rh, a.splits, split) : dst;
      float* const pl = packed ? pp.l(rh, a.splits, split) : dst + 1;
      __hip_atomic_store(pn + d, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(pm, mm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pl, lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      dst[2 + d] = val;
      if (d == 0) {
        dst[0] = mm;
        dst[1] = lsum;
      }
    }
  }

  // ---- fused merge: the last work-group to finish for this kv head merges
  // its splits (agent-scope release of every partial, then a ticket).
  if constexpr (FUSED) {
    __shared__ uint32_t last_s;
    // The partials were stored with agent-scope atomic stores (coherent
    // across XCDs, no L2 write-back needed) and are read back with
    // agent-scope atomic loads.  Every wave waits until its stores have
    // completed, the work-group synchronizes, and only then takes a ticket,
    // so the work-group that draws the last ticket sees every partial.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if constexpr (FENCE) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t t = __hip_atomic_fetch_add(a.counters + kv, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_s = t + 1u == nsplit ? 1u : 0u;
    }
    __syncthreads();
    if (last_s != 0u) {
      if constexpr (FENCE) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      static_assert(MergeRowsLayout<D, NW, (uint32_t(HS) * D / 4u <= 64u * NW ? HS : 1)>::kFloats * 4u <= L::kBytes,
                    "the merge's LDS fits the kernel's");
      float* f_s = reinterpret_cast<float*>(smem);  // [HS][32] split factors or the merge_rows area
      fused_merge<D, NW, HS>(a, kv, head_rows, nsplit, scratch, f_s, f_s + HS * 32);
      if (threadIdx.x == 0) __hip_atomic_store(a.counters + kv, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

#define KVB_I8_ARGS                                                                                        \
  a.page_table, static_cast<const int8_t*>(a.k), a.k_scales, a.v_scales, a.begin, a.end, a.split_tokens,     \
      a.page_tokens, a.kv_heads, a.pages, a, a.q, a.q_positions, a.k_positions, static_cast<const int8_t*>(a.v), \
      a.scratch

template <int D, int NW, int NB, int HS>
hipError_t launch_cfg(const SplitArgs& a, hipStream_t stream) {
  const bool pt = a.page_tokens >= kTileTokens, fused = a.counters != nullptr, varlen = a.seq_starts != nullptr;
  const dim3 grid(a.splits, a.kv_heads, varlen ? a.batch : 1u);
  const dim3 block(64 * NW);
  if (varlen && !pt) return hipErrorInvalidValue;  // batched calls need whole-tile pages (i8_supported)
  if (varlen && fused)
    hipLaunchKernelGGL((split_i8_kernel<D, NW, NB, true, HS, true, true, false>), grid, block, 0, stream, KVB_I8_ARGS);
  else if (varlen)
    hipLaunchKernelGGL((split_i8_kernel<D, NW, NB, true, HS, false, true, false>), grid, block, 0, stream, KVB_I8_ARGS);
  else if (pt && fused)
    hipLaunchKernelGGL((split_i8_kernel<D, NW, NB, true, HS, true, false, false>), grid, block, 0, stream, KVB_I8_ARGS);
  else if (pt)
    hipLaunchKernelGGL((split_i8_kernel<D, NW, NB, true, HS, false, false, false>), grid, block, 0, stream, KVB_I8_ARGS);
  else if (fused)
    hipLaunchKernelGGL((split_i8_kernel<D, NW, NB, false, HS, true, false, false>), grid, block, 0, stream, KVB_I8_ARGS);
  else
    hipLaunchKernelGGL((split_i8_kernel<D, NW, NB, false, HS, false, false, false>), grid, block, 0, stream, KVB_I8_ARGS);
  return hipGetLastError();
}

template <int D, int NW, int NB, int HS>
hipError_t preload_cfg() {
  const void* fns[] = {reinterpret_cast<const void*>(&split_i8_kernel<D, NW, NB, true, HS, false, false, false>),
                       reinterpret_cast<const void*>(&split_i8_kernel<D, NW, NB, false, HS, false, false, false>),
                       reinterpret_cast<const void*>(&split_i8_kernel<D, NW, NB, true, HS, true, false, false>),
                       reinterpret_cast<const void*>(&split_i8_kernel<D, NW, NB, false, HS, true, false, false>),
                       reinterpret_cast<const void*>(&split_i8_kernel<D, NW, NB, true, HS, false, true, false>),
                       reinterpret_cast<const void*>(&split_i8_kernel<D, NW, NB, true, HS, true, true, false>)};
  hipFuncAttributes attr{};
  for (const void* f : fns) {
    const hipError_t e = hipFuncGetAttributes(&attr, f);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Launch / preload of every (waves, ring) configuration of one dim; cfg =
// 10 * waves + ring slots (82 only for head_rows <= 4 and dim <= 128).
template <int D>
hipError_t launch_dim(const SplitArgs& a, int cfg, hipStream_t stream) {
  if (a.rows * a.group <= 4) {
    if constexpr (D <= 128) {
      if (cfg == 82) return launch_cfg<D, 8, 2, 4>(a, stream);
      if (cfg == 44) return launch_cfg<D, 4, 4, 4>(a, stream);
    }
    if (cfg == 12) return launch_cfg<D, 1, 2, 4>(a, stream);
    if (cfg == 14) return launch_cfg<D, 1, 4, 4>(a, stream);
    return cfg == 42 ? launch_cfg<D, 4, 2, 4>(a, stream) : launch_cfg<D, 2, 2, 4>(a, stream);
  }
  if constexpr (D <= 128) {
    if (cfg == 12) return launch_cfg<D, 1, 2, 8>(a, stream);
    return cfg == 42 ? launch_cfg<D, 4, 2, 8>(a, stream) : launch_cfg<D, 2, 2, 8>(a, stream);
  }
  return hipErrorInvalidValue;
}

template <int D>
hipError_t preload_dim() {
  hipError_t e = hipSuccess;
  if constexpr (D <= 128) {
    if (e == hipSuccess) e = preload_cfg<D, 8, 2, 4>();
    if (e == hipSuccess) e = preload_cfg<D, 4, 4, 4>();
    if (e == hipSuccess) e = preload_cfg<D, 4, 2, 8>();
    if (e == hipSuccess) e = preload_cfg<D, 2, 2, 8>();
  }
  if (e == hipSuccess) e = preload_cfg<D, 4, 2, 4>();
  if (e == hipSuccess) e = preload_cfg<D, 2, 2, 4>();
  if (e == hipSuccess) e = preload_cfg<D, 1, 2, 4>();
  if (e == hipSuccess) e = preload_cfg<D, 1, 4, 4>();
  if constexpr (D <= 128) {
    if (e == hipSuccess) e = preload_cfg<D, 1, 2, 8>();
  }
  return e;
}

}  // namespace
}  // namespace kvb
