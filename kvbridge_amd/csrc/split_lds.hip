// LDS-streamed MFMA split-partial kernel for paged INT8 KV (gfx950).
//
// Used where the int8-MFMA kernel (split_i8.h) does not apply, notably more
// than 8 head-rows per kv head (e.g. the reference's dense rows8/group6
// geometry).  One work-group per (split, kv_head, block of <= 16 head-rows);
// 64-token tiles split round-robin over the waves; QK and PV as
// v_mfma_f32_16x16x32_f16 with the KV tile (int8 codes converted exactly to
// f16) as the A operand and the head-rows as the 16 MFMA columns; Q and the
// softmax weights P carried as f16 hi + lo pairs (scaled by powers of two)
// so both products keep fp32-level accuracy; online softmax per wave and an
// LDS combine of the waves into the fp32 partial layout.
//
// What differs is how a tile reaches the MFMA operands.  Each wave owns a
// ring of NB tile buffers in LDS and fills them with gfx950's
// global_load_lds_dwordx4 (HBM -> LDS without passing through VGPRs), NB-1
// tiles ahead of the tile it computes.  Every load instruction moves 1 KiB
// of contiguous HBM; the lane -> 16-byte-chunk assignment applies an XOR
// swizzle so the MFMA-layout ds_read_b128 reads that follow are free of bank
// conflicts (checked for both 32- and 64-bank LDS).  LDS reads are issued
// with inline ds_read so the compiler does not add its conservative
// "wait for every LDS DMA" before them; instead each iteration issues a fixed
// number of vector-memory instructions (one tile; page ids come from a
// per-wave window of page-table entries via v_readlane), which makes "tile i
// has landed" an exact s_waitcnt vmcnt((NB-1) * loads_per_tile).
//
// Tile buffer (bytes):  K [64 tokens][D]   row r at r*D, chunk c at 16*(c ^ fK(r))
//                       V [D dims][64 B]   row d at d*64, chunk c at 16*(c ^ fV(d))
//                       k-scales [64], v-scales [64] floats, token order.
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "kernels.h"
#include "device_common.h"
#include "lds_stream.h"

namespace kvb {
namespace {

using namespace lds;

template <int D>
struct WaveState {
  f32x4 acc[D / 16];  // O[d = 16*mb + 4*g + e][h] in element e of acc[mb]
  float m;            // running max of head-row h
  float l;            // this lane's partial sum of weights
  int kexp;           // PV weights carried as w * v_scale * 2^kexp
};

// Compute one tile from LDS buffer at byte address `base` (+ BOFF immediate).
template <int D, uint32_t BOFF>
__device__ __forceinline__ void compute_tile(WaveState<D>& st, uint32_t base, const ReadOffsets<D>& o,
                                             uint32_t tile, const f16x8 (&qh)[D / 32],
                                             const f16x8 (&ql)[D / 32], bool qlo, float cq, bool full,
                                             uint32_t s0, uint32_t e_h, uint32_t e_max, uint32_t lane) {
  const uint32_t g = lane >> 4;
  const uint32_t t0 = tile * kTileTokens;
  // ---- LDS -> registers (one wait for the whole tile)
  uint4 kr[4][D / 64];
  uint4 vr[D / 16];
  static_for<0, 4>([&](auto mbc) {
    constexpr uint32_t mb = decltype(mbc)::value;
#pragma unroll
    for (int j = 0; j < D / 64; ++j) kr[mb][j] = ds_read16<BOFF + 4 * mb * D>(base + o.k[j]);
  });
  static_for<0, D / 16>([&](auto mbc) {
    constexpr uint32_t mb = decltype(mbc)::value;
    vr[mb] = ds_read16<BOFF + 1024 * mb>(base + o.v);
  });
  uint4 ks0 = ds_read16<BOFF>(base + o.sc), ks1 = ds_read16<BOFF + 16>(base + o.sc),
        ks2 = ds_read16<BOFF + 32>(base + o.sc), ks3 = ds_read16<BOFF + 48>(base + o.sc);
  uint4 vs0 = ds_read16<BOFF + 256>(base + o.sc), vs1 = ds_read16<BOFF + 272>(base + o.sc),
        vs2 = ds_read16<BOFF + 288>(base + o.sc), vs3 = ds_read16<BOFF + 304>(base + o.sc);
  wait_lds();
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int j = 0; j < D / 64; ++j) lds_fence(kr[mb][j]);
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) lds_fence(vr[mb]);
  lds_fence(ks0, ks1, ks2, ks3, vs0, vs1, vs2, vs3);
  const float ks[16] = {__uint_as_float(ks0.x), __uint_as_float(ks0.y), __uint_as_float(ks0.z), __uint_as_float(ks0.w),
                        __uint_as_float(ks1.x), __uint_as_float(ks1.y), __uint_as_float(ks1.z), __uint_as_float(ks1.w),
                        __uint_as_float(ks2.x), __uint_as_float(ks2.y), __uint_as_float(ks2.z), __uint_as_float(ks2.w),
                        __uint_as_float(ks3.x), __uint_as_float(ks3.y), __uint_as_float(ks3.z), __uint_as_float(ks3.w)};
  float vs[16] = {__uint_as_float(vs0.x), __uint_as_float(vs0.y), __uint_as_float(vs0.z), __uint_as_float(vs0.w),
                  __uint_as_float(vs1.x), __uint_as_float(vs1.y), __uint_as_float(vs1.z), __uint_as_float(vs1.w),
                  __uint_as_float(vs2.x), __uint_as_float(vs2.y), __uint_as_float(vs2.z), __uint_as_float(vs2.w),
                  __uint_as_float(vs3.x), __uint_as_float(vs3.y), __uint_as_float(vs3.z), __uint_as_float(vs3.w)};

  // ---- QK: c[mb][e] = S[token 16g + 4mb + e][h]
  f32x4 c[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    c[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const uint4 w = kr[mb][s / 2];
      const f16x8 a = (s & 1) ? i8x8_to_f16(w.z, w.w) : i8x8_to_f16(w.x, w.y);
      c[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[s], c[mb], 0, 0, 0);
      if (qlo) c[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[s], c[mb], 0, 0, 0);
    }
  }
  float sc[16];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int e = 0; e < 4; ++e) sc[4 * mb + e] = c[mb][e] * ks[4 * mb + e] * cq;
  if (!full) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t tok = t0 + 16u * g + uint32_t(j);
      if (!(tok >= s0 && tok < e_h)) sc[j] = neg_inf();
      if (!(tok >= s0 && tok < e_max)) vs[j] = 0.f;  // unused slots may hold anything
    }
  }
  float mx = sc[0], vmax = fabsf(vs[0]);
#pragma unroll
  for (int j = 1; j < 16; ++j) {
    mx = fmaxf(mx, sc[j]);
    vmax = fmaxf(vmax, fabsf(vs[j]));
  }
  mx = rows_max(mx);
  vmax = rows_max(vmax);  // every lane row sees all 64 tokens' scales
  const float m_new = fmaxf(st.m, mx);
  int k_new = st.kexp;
  if (vmax > 0.f) {
    const int kt = 15 - __builtin_amdgcn_frexp_expf(vmax);
    k_new = kt < k_new ? (kt < -100 ? -100 : kt) : k_new;
  }
  if (__ballot(m_new > st.m) != 0 || k_new != st.kexp) {
    const float alpha = st.m == neg_inf() ? 0.f : exp_e(st.m - m_new);
    const float f = __builtin_amdgcn_ldexpf(alpha, k_new - st.kexp);
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) st.acc[mb] *= f;
    st.l *= alpha;
  }
  st.m = m_new;
  st.kexp = k_new;
  const float m_use = m_new == neg_inf() ? 0.f : m_new;
  float p[16];
  float lsum = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float w = exp_e(sc[j] - m_use);
    lsum += w;
    p[j] = w * __builtin_amdgcn_ldexpf(vs[j], k_new);
  }
  st.l += lsum;
  f16x8 bh[2], bl[2];
#pragma unroll
  for (int js = 0; js < 2; ++js)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = p[8 * js + e];
      const _Float16 hi = (_Float16)x;
      bh[js][e] = hi;
      bl[js][e] = (_Float16)(x - (float)hi);
    }
  // ---- PV
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) {
    const uint4 w = vr[mb];
    const f16x8 a0 = i8x8_to_f16(w.x, w.y);
    const f16x8 a1 = i8x8_to_f16(w.z, w.w);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bh[0], st.acc[mb], 0, 0, 0);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bl[0], st.acc[mb], 0, 0, 0);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bh[1], st.acc[mb], 0, 0, 0);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bl[1], st.acc[mb], 0, 0, 0);
  }
}

static_assert(true, "");

template <int D, int NW, int NB>
struct Smem {
  static constexpr uint32_t kRing = NW * NB * Geo<D>::kBufBytes;
  static constexpr uint32_t kCombine = NW * 16 * (D + 2) * 4;
  static constexpr uint32_t kBytes = kRing > kCombine ? kRing : kCombine;
};

template <int D, int NW, int NB, bool PT>
__global__ __launch_bounds__(64 * NW) void split_lds_kernel(
    SplitArgs a, const float* __restrict__ q, const int64_t* __restrict__ qpos,
    const int64_t* __restrict__ kpos, const uint32_t* __restrict__ table,
    const int8_t* __restrict__ kdata, const int8_t* __restrict__ vdata,
    const float* __restrict__ kscale, const float* __restrict__ vscale, float* __restrict__ scratch) {
  using G = Geo<D>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[Smem<D, NW, NB>::kBytes];

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane & 15u, g = lane >> 4;
  const uint32_t head_rows = a.rows * a.group;
  // Work-group -> (split, kv head, block of 16 head-rows).  The blocks of one
  // (split, kv head) read the same KV tiles, so they get consecutive ids
  // congruent mod 8: dispatched together, and on the same XCD where
  // work-groups are dealt to the 8 XCDs round-robin, where the later blocks'
  // reads then hit that XCD's L2 (a locality choice only).
  const uint32_t hblocks = (head_rows + 15u) / 16u;
  const uint32_t id = blockIdx.x, xr = id % 8u, xt = id / 8u;
  const uint32_t hblock = xt % hblocks, unit = 8u * (xt / hblocks) + xr;
  if (unit >= a.splits * a.kv_heads) return;  // grid padding
  const uint32_t split = unit % a.splits, kv = unit / a.splits;
  const uint32_t hr = hblock * 16u + h;
  const bool hvalid = hr < head_rows;
  const uint32_t row = hvalid ? hr / a.group : 0u;
  const uint32_t head = kv * a.group + (hvalid ? hr % a.group : 0u);

  const uint64_t s0_64 = uint64_t(a.begin) + uint64_t(split) * a.split_tokens;
  const uint32_t s0 = s0_64 < a.end ? uint32_t(s0_64) : a.end;
  const uint32_t s1 = uint64_t(s0) + a.split_tokens < a.end ? s0 + a.split_tokens : a.end;
  const uint32_t k_first = s0 / kTileTokens;
  const uint32_t k_last = s1 > s0 ? (s1 - 1u) / kTileTokens : k_first;

  Ctx c;
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
  auto tile_of = [&](uint32_t i) {  // i-th tile of this wave, clamped: extra loads are harmless
    const uint32_t k = k_first + wave + i * NW;
    return k < k_last ? k : k_last;
  };
  uint8_t* ring = smem + wave * (NB * G::kBufBytes);
  const uint32_t ring_addr = lds_addr(ring);

  // ---- page-table window, then start streaming before anything else.
  {
    // No table load for an empty split (its lp_lo may be one past the last page).
    const uint32_t lp = c.lp_lo + lane;
    c.ptab = s1 > s0 && lp <= c.lp_hi ? table[lp] : 0u;
  }
  // Issue sequence: this wave's tiles in order, the last one repeated past the
  // end (so every step issues exactly one tile).
  PtCtx pc;
  IssuePos ip;
  if constexpr (PT) {
    const uint32_t kv_bytes = a.pages * a.kv_heads * a.page_tokens * uint32_t(D);
    const uint32_t sc_bytes = a.pages * a.kv_heads * a.page_tokens * 4u;
    pt_init<D>(pc, kdata, vdata, kscale, vscale, kv_bytes, sc_bytes, a.page_tokens, lane);
    ip.k = tile_of(0);
    ip.lp = ip.k * kTileTokens / a.page_tokens;
    ip.slot = ip.k * kTileTokens - ip.lp * a.page_tokens;
  }
  auto issue_next = [&](uint32_t seq, uint8_t* buf) __attribute__((always_inline)) {
    dma_group_mark();
    if constexpr (PT) {
      const uint32_t rel = ip.lp - c.lp_lo;
      uint32_t phys = rel < 64u ? __builtin_amdgcn_readlane(c.ptab, rel) : table[ip.lp];
      phys = phys < a.pages ? phys : a.pages - 1u;
      pt_issue<D>(pc, phys * a.kv_heads + kv, ip.slot, a.page_tokens, buf);
      if (ip.k + NW <= k_last) {
        ip.k += NW;
        ip.slot += kTileTokens * NW;
        while (ip.slot >= a.page_tokens) {
          ip.slot -= a.page_tokens;
          ++ip.lp;
        }
      }
    } else {
      issue_tile<D>(c, tile_of(seq), buf);
    }
  };
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) issue_next(j, ring + j * G::kBufBytes);

  // ---- visibility: tokens [s0, e_h) are visible to this lane's row.
  const uint32_t r_lo = hblock * 16u / a.group;
  const uint32_t r_hi = (hblock * 16u + 15u < head_rows ? hblock * 16u + 15u : head_rows - 1u) / a.group;
  uint32_t e_h = s0;
  if (s1 > s0) {
    const int64_t klast = kpos[s1 - 1u];
    bool all_visible = true;
    for (uint32_t r = r_lo; r <= r_hi; ++r) all_visible &= klast <= qpos[r];
    if (all_visible) {
      e_h = s1;
    } else {
      for (uint32_t r = r_lo; r <= r_hi; ++r) {
        const uint32_t e = visible_end(kpos, s0, s1, qpos[r], lane);
        if (row == r) e_h = e;
      }
    }
    if (!hvalid) e_h = s0;
  }
  uint32_t e_min = hvalid ? e_h : 0xffffffffu, e_max = e_h;
#define KVB_ROW_RED(N)                                                                          \
  {                                                                                             \
    const uint32_t o1 = uint32_t(__builtin_amdgcn_update_dpp(0, int(e_min), 0x120 + N, 0xF, 0xF, false)); \
    const uint32_t o2 = uint32_t(__builtin_amdgcn_update_dpp(0, int(e_max), 0x120 + N, 0xF, 0xF, false)); \
    e_min = o1 < e_min ? o1 : e_min;                                                            \
    e_max = o2 > e_max ? o2 : e_max;                                                            \
  }
  KVB_ROW_RED(8) KVB_ROW_RED(4) KVB_ROW_RED(2) KVB_ROW_RED(1)
#undef KVB_ROW_RED
  e_min = __builtin_amdgcn_readfirstlane(e_min);
  e_max = __builtin_amdgcn_readfirstlane(e_max);

  // ---- Q as 2^kq-scaled f16 hi + lo (B operand of QK).
  float qv[D / 4];
  if (hvalid) {
    const float4* qp = reinterpret_cast<const float4*>(q + (size_t(row) * a.q_heads + head) * D + g * (D / 4));
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
      const float4 x = qp[i];
      qv[4 * i] = x.x; qv[4 * i + 1] = x.y; qv[4 * i + 2] = x.z; qv[4 * i + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < D / 4; ++i) qv[i] = 0.f;
  }
  float qmax = 0.f;
#pragma unroll
  for (int i = 0; i < D / 4; ++i) qmax = fmaxf(qmax, fabsf(qv[i]));
  qmax = rows_max(qmax);
  int kq = 0;
  if (qmax > 0.f) {
    kq = 15 - __builtin_amdgcn_frexp_expf(qmax);
    kq = kq < -100 ? -100 : (kq > 100 ? 100 : kq);
  }
  const float cq = __builtin_amdgcn_ldexpf(a.scale, -kq);
  f16x8 qh[D / 32], ql[D / 32];
  bool any_lo = false;
#pragma unroll
  for (int s = 0; s < D / 32; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = __builtin_amdgcn_ldexpf(qv[8 * s + e], kq);
      const _Float16 hi = (_Float16)x;
      const _Float16 lo = (_Float16)(x - (float)hi);
      qh[s][e] = hi;
      ql[s][e] = lo;
      any_lo |= (lo != (_Float16)0.0f);
    }
  const bool qlo = __ballot(any_lo) != 0;

  WaveState<D> st;
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) st.acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = neg_inf();
  st.l = 0.f;
  st.kexp = 100;
  const ReadOffsets<D> ro = read_offsets<D>(lane);

  const uint32_t k_vis = e_max > s0 ? (e_max - 1u) / kTileTokens : 0u;
  const uint32_t k_count = e_max > s0 ? k_vis + 1u - k_first : 0u;
  const uint32_t nt = k_count > wave ? (k_count - wave + NW - 1u) / NW : 0u;
  auto is_full = [&](uint32_t k) { return k * kTileTokens >= s0 && (k + 1u) * kTileTokens <= e_min; };

  // ---- main loop, unrolled by NB so ring slots are compile-time.  Every step
  // issues exactly one tile (clamped past the end), so after tile i's loads
  // exactly (NB-1) tiles' worth of vector-memory instructions were issued.
  constexpr uint32_t kWait = (NB - 1) * G::kLoadsPerTile;
  auto step = [&](uint32_t i0, auto uc) {
    constexpr int u = decltype(uc)::value;
    const uint32_t i = i0 + u;
    if (i < nt) {
      issue_next(i + NB - 1, ring + ((u + NB - 1) % NB) * G::kBufBytes);
      if constexpr (NB > 1) wait_vm_keep<kWait, NB - 1>();  // tile i has landed in slot u
      else wait_vm<0>();
      const uint32_t k = tile_of(i);
      compute_tile<D, u * G::kBufBytes>(st, ring_addr, ro, k, qh, ql, qlo, cq, is_full(k), s0, e_h,
                                        e_max, lane);
    }
  };
  for (uint32_t i0 = 0; i0 < nt; i0 += NB) {
    step(i0, std::integral_constant<int, 0>{});
    if constexpr (NB > 1) step(i0, std::integral_constant<int, 1>{});
    if constexpr (NB > 2) step(i0, std::integral_constant<int, 2>{});
    if constexpr (NB > 3) step(i0, std::integral_constant<int, 3>{});
  }
  wait_vm<0>();

  // ---- combine the waves through LDS (reusing the ring) and write the partial.
  __syncthreads();
  float* wm_s = reinterpret_cast<float*>(smem);            // [NW][16]
  float* wl_s = wm_s + NW * 16;                            // [NW][16]
  float* wacc_s = wl_s + NW * 16;                          // [NW][16][D]
  const float l_h = rows_sum(st.l);
  if (g == 0) {
    wm_s[wave * 16 + h] = st.m;
    wl_s[wave * 16 + h] = l_h;
  }
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) {
    const f32x4 x = st.acc[mb];
    float4 y;
    y.x = __builtin_amdgcn_ldexpf(x[0], -st.kexp);
    y.y = __builtin_amdgcn_ldexpf(x[1], -st.kexp);
    y.z = __builtin_amdgcn_ldexpf(x[2], -st.kexp);
    y.w = __builtin_amdgcn_ldexpf(x[3], -st.kexp);
    *reinterpret_cast<float4*>(&wacc_s[(wave * 16 + h) * D + 16 * mb + 4 * g]) = y;
  }
  __syncthreads();
  const uint32_t nvalid = head_rows - hblock * 16u < 16u ? head_rows - hblock * 16u : 16u;
  constexpr uint32_t W = D + 2;
  for (uint32_t idx = threadIdx.x; idx < nvalid * W; idx += 64u * NW) {
    const uint32_t hh = idx / W, col = idx % W;
    float mm = wm_s[hh];
#pragma unroll
    for (int w = 1; w < NW; ++w) mm = fmaxf(mm, wm_s[w * 16 + hh]);
    float val = mm;
    if (col > 0) {
      val = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = wm_s[w * 16 + hh];
        if (mw == neg_inf()) continue;
        const float f = exp_e(mw - mm);
        val = fmaf(f, col == 1 ? wl_s[w * 16 + hh] : wacc_s[(w * 16 + hh) * D + col - 2], val);
      }
    }
    const uint32_t hr2 = hblock * 16u + hh;
    const uint32_t row2 = hr2 / a.group, head2 = kv * a.group + hr2 % a.group;
    scratch[((size_t(row2) * a.q_heads + head2) * a.splits + split) * W + col] = val;
  }
}

// Many head-row blocks over short splits (e.g. the reference's dense
// rows-8 / group-6 geometry, 48 head-rows = 3 blocks, 256-token splits): one
// work-group per (split, kv head) DMAs the split's whole tiles into LDS once
// (tile j by wave j % 4), and after one barrier wave w runs head-row blocks
// w, w + 4, ... over every tile with the online softmax of compute_tile.  A
// wave owns whole head-rows, so it writes their partials straight from its
// registers: no wave combine, and the KV bytes of a (split, kv head) are
// read once instead of once per block.  Requires splits that start on a
// tile boundary and hold at most TM tiles (host-checked).
constexpr int kRowsWaves = 4;

template <int D, int TM, bool PT>
__global__ __launch_bounds__(64 * kRowsWaves) void split_lds_rows_kernel(
    SplitArgs a, const float* __restrict__ q, const int64_t* __restrict__ qpos,
    const int64_t* __restrict__ kpos, const uint32_t* __restrict__ table,
    const int8_t* __restrict__ kdata, const int8_t* __restrict__ vdata,
    const float* __restrict__ kscale, const float* __restrict__ vscale, float* __restrict__ scratch) {
  using G = Geo<D>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[TM * G::kBufBytes];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane & 15u, g = lane >> 4;
  const uint32_t split = blockIdx.x, kv = blockIdx.y;
  const uint32_t head_rows = a.rows * a.group, hblocks = (head_rows + 15u) / 16u;

  const uint64_t s0_64 = uint64_t(a.begin) + uint64_t(split) * a.split_tokens;
  const uint32_t s0 = s0_64 < a.end ? uint32_t(s0_64) : a.end;
  const uint32_t s1 = uint64_t(s0) + a.split_tokens < a.end ? s0 + a.split_tokens : a.end;
  const uint32_t k_first = s0 / kTileTokens;
  const uint32_t ntiles = s1 > s0 ? (s1 - 1u) / kTileTokens + 1u - k_first : 0u;  // <= TM

  // ---- every tile of the split into LDS (tile j -> buffer j, by wave j % 4)
  if (ntiles > 0) {
    Ctx c;
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
    c.lp_hi = (s1 - 1u) / a.page_tokens;
    c.lane = lane;
    {
      const uint32_t lp = c.lp_lo + lane;
      c.ptab = lp <= c.lp_hi ? table[lp] : 0u;
    }
    PtCtx pc;
    if constexpr (PT) {
      const uint32_t kv_bytes = a.pages * a.kv_heads * a.page_tokens * uint32_t(D);
      const uint32_t sc_bytes = a.pages * a.kv_heads * a.page_tokens * 4u;
      pt_init<D>(pc, kdata, vdata, kscale, vscale, kv_bytes, sc_bytes, a.page_tokens, lane);
    }
    for (uint32_t j = wave; j < ntiles; j += kRowsWaves) {
      uint8_t* const buf = smem + j * G::kBufBytes;
      const uint32_t k = k_first + j;
      if constexpr (PT) {
        const uint32_t lp = k * kTileTokens / a.page_tokens;
        const uint32_t rel = lp - c.lp_lo;
        uint32_t phys = rel < 64u ? __builtin_amdgcn_readlane(c.ptab, rel) : table[lp];
        phys = phys < a.pages ? phys : a.pages - 1u;
        pt_issue<D>(pc, phys * a.kv_heads + kv, k * kTileTokens - lp * a.page_tokens, a.page_tokens, buf);
      } else {
        issue_tile<D>(c, k, buf);
      }
    }
  }
  wait_vm<0>();
  __syncthreads();

  const ReadOffsets<D> ro = read_offsets<D>(lane);
  const uint32_t base0 = lds_addr(smem);
  constexpr uint32_t W = D + 2;
  for (uint32_t hblock = wave; hblock < hblocks; hblock += kRowsWaves) {
    const uint32_t hr = hblock * 16u + h;
    const bool hvalid = hr < head_rows;
    const uint32_t row = hvalid ? hr / a.group : 0u;
    const uint32_t head = kv * a.group + (hvalid ? hr % a.group : 0u);

    // ---- visibility: tokens [s0, e_h) are visible to this lane's row.
    const uint32_t r_lo = hblock * 16u / a.group;
    const uint32_t r_hi = (hblock * 16u + 15u < head_rows ? hblock * 16u + 15u : head_rows - 1u) / a.group;
    uint32_t e_h = s0;
    if (s1 > s0) {
      const int64_t klast = kpos[s1 - 1u];
      bool all_visible = true;
      for (uint32_t r = r_lo; r <= r_hi; ++r) all_visible &= klast <= qpos[r];
      if (all_visible) {
        e_h = s1;
      } else {
        for (uint32_t r = r_lo; r <= r_hi; ++r) {
          const uint32_t e = visible_end(kpos, s0, s1, qpos[r], lane);
          if (row == r) e_h = e;
        }
      }
      if (!hvalid) e_h = s0;
    }
    uint32_t e_min = hvalid ? e_h : 0xffffffffu, e_max = e_h;
#define KVB_ROW_RED(N)                                                                                    \
  {                                                                                                       \
    const uint32_t o1 = uint32_t(__builtin_amdgcn_update_dpp(0, int(e_min), 0x120 + N, 0xF, 0xF, false)); \
    const uint32_t o2 = uint32_t(__builtin_amdgcn_update_dpp(0, int(e_max), 0x120 + N, 0xF, 0xF, false)); \
    e_min = o1 < e_min ? o1 : e_min;                                                                      \
    e_max = o2 > e_max ? o2 : e_max;                                                                      \
  }
    KVB_ROW_RED(8) KVB_ROW_RED(4) KVB_ROW_RED(2) KVB_ROW_RED(1)
#undef KVB_ROW_RED
    e_min = __builtin_amdgcn_readfirstlane(e_min);
    e_max = __builtin_amdgcn_readfirstlane(e_max);

    // ---- Q as 2^kq-scaled f16 hi + lo (B operand of QK).
    float qv[D / 4];
    if (hvalid) {
      const float4* qp = reinterpret_cast<const float4*>(q + (size_t(row) * a.q_heads + head) * D + g * (D / 4));
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        const float4 x = qp[i];
        qv[4 * i] = x.x;
        qv[4 * i + 1] = x.y;
        qv[4 * i + 2] = x.z;
        qv[4 * i + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < D / 4; ++i) qv[i] = 0.f;
    }
    float qmax = 0.f;
#pragma unroll
    for (int i = 0; i < D / 4; ++i) qmax = fmaxf(qmax, fabsf(qv[i]));
    qmax = rows_max(qmax);
    int kq = 0;
    if (qmax > 0.f) {
      kq = 15 - __builtin_amdgcn_frexp_expf(qmax);
      kq = kq < -100 ? -100 : (kq > 100 ? 100 : kq);
    }
    const float cq = __builtin_amdgcn_ldexpf(a.scale, -kq);
    f16x8 qh[D / 32], ql[D / 32];
    bool any_lo = false;
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = __builtin_amdgcn_ldexpf(qv[8 * s + e], kq);
        const _Float16 hi = (_Float16)x;
        const _Float16 lo = (_Float16)(x - (float)hi);
        qh[s][e] = hi;
        ql[s][e] = lo;
        any_lo |= (lo != (_Float16)0.0f);
      }
    const bool qlo = __ballot(any_lo) != 0;

    WaveState<D> st;
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) st.acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = neg_inf();
    st.l = 0.f;
    st.kexp = 100;
    const uint32_t k_vis = e_max > s0 ? (e_max - 1u) / kTileTokens : 0u;
    const uint32_t nvis = e_max > s0 ? k_vis + 1u - k_first : 0u;
    for (uint32_t j = 0; j < nvis; ++j) {
      const uint32_t k = k_first + j;
      const bool full = k * kTileTokens >= s0 && (k + 1u) * kTileTokens <= e_min;
      compute_tile<D, 0>(st, base0 + j * G::kBufBytes, ro, k, qh, ql, qlo, cq, full, s0, e_h, e_max, lane);
    }

    // ---- this block's partials, straight from the registers
    const float l_h = rows_sum(st.l);
    if (hvalid) {
      float* const dst = scratch + ((size_t(row) * a.q_heads + head) * a.splits + split) * W;
      if (g == 0) {
        dst[0] = st.m;
        dst[1] = l_h;
      }
#pragma unroll
      for (int mb = 0; mb < D / 16; ++mb) {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[2 + 16 * mb + 4 * g + e] = __builtin_amdgcn_ldexpf(st.acc[mb][e], -st.kexp);
      }
    }
  }
}

#define KVB_LDS_ARGS                                                                             \
  a, a.q, a.q_positions, a.k_positions, a.page_table, static_cast<const int8_t*>(a.k),             \
      static_cast<const int8_t*>(a.v), a.k_scales, a.v_scales, a.scratch

template <int D, int NW, int NB>
hipError_t launch_cfg(const SplitArgs& a, hipStream_t stream) {
  const uint64_t hblocks = (uint64_t(a.rows) * a.group + 15u) / 16u;
  const uint64_t units = uint64_t(a.splits) * a.kv_heads;  // (split, kv head) pairs
  const uint64_t groups = 8u * hblocks * ((units + 7u) / 8u);
  if (groups > 0x7fffffffull) return hipErrorInvalidValue;
  const dim3 grid(static_cast<uint32_t>(groups), 1u, 1u);
  if (a.page_tokens % kTileTokens == 0)
    hipLaunchKernelGGL((split_lds_kernel<D, NW, NB, true>), grid, dim3(64 * NW), 0, stream, KVB_LDS_ARGS);
  else
    hipLaunchKernelGGL((split_lds_kernel<D, NW, NB, false>), grid, dim3(64 * NW), 0, stream, KVB_LDS_ARGS);
  return hipGetLastError();
}

template <int D, int NW, int NB>
hipError_t preload_cfg() {
  hipFuncAttributes attr{};
  hipError_t e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_lds_kernel<D, NW, NB, true>));
  if (e != hipSuccess) return e;
  return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_lds_kernel<D, NW, NB, false>));
}

// (waves, buffers) per work-group by dim and tiles per split, as 10*NW + NB;
// LDS use is NW * NB * (128 * D + 512) bytes.  KVB_LDS_CFG="NW,NB" overrides
// (tuning sweeps).
int lds_config(const SplitArgs& a) {
  static const int forced = [] {
    const char* e = std::getenv("KVB_LDS_CFG");
    if (!e) return 0;
    return std::atoi(e) * 10 + std::atoi(e + 2);
  }();
  const uint32_t tiles = (a.split_tokens + kTileTokens - 1) / kTileTokens;
  int cfg = forced;
  if (a.dim == 128) {
    if (cfg != 41 && cfg != 81 && cfg != 23 && cfg != 42) cfg = tiles >= 16 ? 42 : 41;
  } else if (a.dim == 64) {
    if (cfg != 41 && cfg != 42 && cfg != 43) cfg = tiles >= 16 ? 43 : 41;
  } else {
    if (cfg != 41 && cfg != 22) cfg = tiles >= 16 ? 22 : 41;
  }
  return cfg;
}

}  // namespace

// Tiles of a split the rows kernel holds in LDS, by dim (about 135 KiB).
constexpr int kRowsTiles256 = 4, kRowsTiles128 = 8, kRowsTiles64 = 16;

int rows_tiles(uint32_t dim) {
  return dim == 256 ? kRowsTiles256 : (dim == 128 ? kRowsTiles128 : (dim == 64 ? kRowsTiles64 : 0));
}

// More than one head-row block and splits that start on a tile boundary and
// fit the rows kernel's LDS.
bool use_rows_kernel(const SplitArgs& a) {
  if (a.rows * a.group <= 16u || a.seq_starts != nullptr) return false;
  if (a.begin % kTileTokens != 0 || a.split_tokens % kTileTokens != 0) return false;
  return a.split_tokens / kTileTokens <= uint32_t(rows_tiles(a.dim));
}

template <int D, int TM>
hipError_t launch_rows(const SplitArgs& a, hipStream_t stream) {
  const dim3 grid(a.splits, a.kv_heads);
  if (a.page_tokens % kTileTokens == 0)
    hipLaunchKernelGGL((split_lds_rows_kernel<D, TM, true>), grid, dim3(64 * kRowsWaves), 0, stream, KVB_LDS_ARGS);
  else
    hipLaunchKernelGGL((split_lds_rows_kernel<D, TM, false>), grid, dim3(64 * kRowsWaves), 0, stream, KVB_LDS_ARGS);
  return hipGetLastError();
}

template <int D, int TM>
hipError_t preload_rows() {
  hipFuncAttributes attr{};
  hipError_t e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_lds_rows_kernel<D, TM, true>));
  if (e != hipSuccess) return e;
  return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_lds_rows_kernel<D, TM, false>));
}

hipError_t launch_split_lds(const SplitArgs& a, hipStream_t stream) {
  if (use_rows_kernel(a)) {
    switch (a.dim) {
      case 64: return launch_rows<64, kRowsTiles64>(a, stream);
      case 128: return launch_rows<128, kRowsTiles128>(a, stream);
      case 256: return launch_rows<256, kRowsTiles256>(a, stream);
      default: break;
    }
  }
  const int cfg = lds_config(a);
  switch (a.dim * 100 + cfg) {
    case 12841: return launch_cfg<128, 4, 1>(a, stream);
    case 12881: return launch_cfg<128, 8, 1>(a, stream);
    case 12823: return launch_cfg<128, 2, 3>(a, stream);
    case 12842: return launch_cfg<128, 4, 2>(a, stream);
    case 6441: return launch_cfg<64, 4, 1>(a, stream);
    case 6442: return launch_cfg<64, 4, 2>(a, stream);
    case 6443: return launch_cfg<64, 4, 3>(a, stream);
    case 25641: return launch_cfg<256, 4, 1>(a, stream);
    case 25622: return launch_cfg<256, 2, 2>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

const char* lds_kernel_name(const SplitArgs& a) {
  static thread_local char buf[96];
  if (use_rows_kernel(a) && rows_tiles(a.dim) > 0) {
    std::snprintf(buf, sizeof(buf), "split_lds_rows_kernel<%u,%d,%s>", a.dim, rows_tiles(a.dim),
                  a.page_tokens % kTileTokens == 0 ? "true" : "false");
    return buf;
  }
  const int cfg = lds_config(a);
  std::snprintf(buf, sizeof(buf), "split_lds_kernel<%u,%d,%d,%s>", a.dim, cfg / 10, cfg % 10,
                a.page_tokens % kTileTokens == 0 ? "true" : "false");
  return buf;
}

hipError_t preload_lds() {
  hipError_t e;
  if ((e = preload_cfg<128, 4, 1>()) != hipSuccess) return e;
  if ((e = preload_cfg<128, 8, 1>()) != hipSuccess) return e;
  if ((e = preload_cfg<128, 2, 3>()) != hipSuccess) return e;
  if ((e = preload_cfg<128, 4, 2>()) != hipSuccess) return e;
  if ((e = preload_cfg<64, 4, 1>()) != hipSuccess) return e;
  if ((e = preload_cfg<64, 4, 2>()) != hipSuccess) return e;
  if ((e = preload_cfg<64, 4, 3>()) != hipSuccess) return e;
  if ((e = preload_cfg<256, 4, 1>()) != hipSuccess) return e;
  if ((e = preload_cfg<256, 2, 2>()) != hipSuccess) return e;
  if ((e = preload_rows<64, kRowsTiles64>()) != hipSuccess) return e;
  if ((e = preload_rows<128, kRowsTiles128>()) != hipSuccess) return e;
  return preload_rows<256, kRowsTiles256>();
}

}  // namespace kvb
