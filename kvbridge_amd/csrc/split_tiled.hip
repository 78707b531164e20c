// Tiled MFMA split-partial kernel for paged INT8 KV (gfx950).
//
// One work-group per (split, kv_head, block of up to 16 head-rows).  A
// head-row is one (query row, grouped query head) pair sharing the KV head,
// so GQA reuse is in the MFMA N dimension: every K/V byte is read from HBM
// once per work-group and multiplied against all head-rows at once.  The
// work-group's NW waves take 64-token tiles of the split round-robin; each
// wave keeps an online softmax (max, sum, numerator) in registers and the
// waves are combined through LDS at the end into the fp32 partial layout
//   scratch[((row * q_heads + head) * splits + split) * (dim + 2) + col].
//
// Per 64-token tile a wave issues, per lane, D/16 16-byte loads of K and
// D/16 16-byte loads of V (the whole 64 x D K tile and D x 64 V tile with no
// byte read twice) plus one k-scale and one v-scale.  Loads for tile i+1 are
// in flight while tile i is computed (register double buffer); page-table
// entries are fetched two tiles ahead.
//
// Both contractions are v_mfma_f32_16x16x32_f16 with the KV tile as the A
// operand, so the layouts line up without any LDS transpose:
//   QK:  S[token, h] = sum_d K[token, d] * Q[h, d]     (M = 16 tokens, N = 16 head-rows, K = 32 dims)
//   PV:  O[d, h]     = sum_t V[d, t]     * P[h, t]     (M = 16 dims,   N = 16 head-rows, K = 32 tokens)
// MFMA 16x16 lane layout: A[i][k] in lane (i + 16 * kgroup), B[k][j] in lane
// (j + 16 * kgroup), C[i][j] in lane (j + 16 * (i / 4)) element i % 4.  The
// k order inside a lane is free as long as A and B agree, which is used to
// pick token orders such that the QK result (C layout) is already the PV B
// operand: lane (h, g) with g = lane / 16 owns tokens 16g .. 16g+15 of the
// tile in both, and the V A-operand of lane (d, g) is the 16 contiguous bytes
// V[d][16g .. 16g+15] of the dim-major page.
//
// Numerics.  INT8 codes are exact in f16.  Q is scaled per head-row by a
// power of two so its largest magnitude lies in [2^14, 2^15), then split into
// f16 hi + lo parts (lo is skipped when it is zero for the whole wave, i.e.
// for f16-exact Q).  Scores are (Q.K_code) * k_scale * scale in fp32.  The PV
// weight w * v_scale is scaled by a per-wave power of two (monotone, so the
// accumulator only ever needs an exact 2^-n rescale) and split into f16
// hi + lo, giving ~22-bit weights against fp32 accumulation.  Softmax
// reductions use DPP and permlane swaps, not LDS.
#include <cstdlib>

#include "kernels.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr uint32_t kTileTokens = 64;

template <int D>
struct Tile {
  uint4 k[D / 16];  // M-block mb (16 tokens) uses k[mb * D/64 .. +D/64): the lane's D/4-byte K slice
  uint4 v[D / 16];  // M-block mb (16 dims): 16 slots of V row 16*mb + lane%16
  float ks, vs;     // scales of token t0 + 16*g + lane%16
};

// Physical pages of the four 16-token groups of one tile.  Fetched with
// wave-uniform addresses, so they are scalar loads (counted by lgkmcnt, not
// vmcnt): waiting for them never waits for the tile loads in flight.
struct Pages {
  uint32_t g[4];
};

struct WaveCtx {
  const int8_t* __restrict__ kbase;
  const int8_t* __restrict__ vbase;
  const float* __restrict__ ks;
  const float* __restrict__ vs;
  const uint32_t* __restrict__ table;
  uint32_t kv, kv_heads, P, pages;
  uint32_t lp_lo, lp_hi;  // clamp range of logical pages (pages holding [s0, s1))
  uint32_t lane;
};

__device__ __forceinline__ Pages fetch_pages(const WaveCtx& c, uint32_t tile) {
  const uint32_t t0 = tile * kTileTokens;
  Pages p;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t lp = clampu((t0 + 16u * g) / c.P, c.lp_lo, c.lp_hi);
    p.g[g] = c.table[lp];
  }
  return p;
}

// The page of token group `grp` (0..3, per lane) from the four uniform
// values, clamped into the pool (the clamp sits here, at the use, so that
// fetching never waits for the scalar loads).
__device__ __forceinline__ uint32_t pick(const Pages& p, uint32_t grp, uint32_t pages) {
  const uint32_t lo = (grp & 1u) ? p.g[1] : p.g[0];
  const uint32_t hi = (grp & 1u) ? p.g[3] : p.g[2];
  const uint32_t x = (grp & 2u) ? hi : lo;
  return x < pages ? x : pages - 1u;
}

template <int D>
__device__ __forceinline__ void load_tile(Tile<D>& t, const WaveCtx& c, uint32_t tile, Pages pg) {
  const uint32_t t0 = tile * kTileTokens;
  const uint32_t lane = c.lane, g = lane >> 4, gk = (lane & 15u) >> 2;
  const uint32_t pk = pick(pg, gk, c.pages);
  const uint32_t pv = pick(pg, g, c.pages);
  // K: token row (t0 + 16*gk + 4*mb + lane%4), bytes [g*D/4, (g+1)*D/4).
  const uint32_t krow0 = (pk * c.kv_heads + c.kv) * c.P + (t0 + 16u * gk) % c.P + (lane & 3u);
  const int8_t* kp = c.kbase + size_t(krow0) * D + g * (D / 4);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int j = 0; j < D / 64; ++j)
      t.k[mb * (D / 64) + j] = *reinterpret_cast<const uint4*>(kp + size_t(4 * mb) * D + 16 * j);
  // V: dim row (16*mb + lane%16), slots [(t0 + 16*g) % P, +16).
  const uint32_t vslab = pv * c.kv_heads + c.kv;
  const int8_t* vp = c.vbase + (size_t(vslab) * D + (lane & 15u)) * c.P + (t0 + 16u * g) % c.P;
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb)
    t.v[mb] = *reinterpret_cast<const uint4*>(vp + size_t(16 * mb) * c.P);
  const uint32_t si = vslab * c.P + (t0 + 16u * g) % c.P + (lane & 15u);
  t.ks = c.ks[si];
  t.vs = c.vs[si];
}

template <int J>
__device__ __forceinline__ float bc(float x) { return row_bcast<J>(x); }

// Per-wave online-softmax state.
template <int D>
struct State {
  f32x4 acc[D / 16];  // O[d = 16*mb + 4*g + e][h] in element e of acc[mb]
  float m;            // running max of head-row h (same in the four rows of lanes)
  float l;            // this lane's partial sum of weights (16 tokens per tile)
  int kexp;           // PV weights are carried as w * v_scale * 2^kexp
};

template <int D>
__device__ __forceinline__ void compute_tile(State<D>& st, const Tile<D>& t, uint32_t tile,
                                             const f16x8 (&qh)[D / 32], const f16x8 (&ql)[D / 32],
                                             bool qlo, float cq, bool full, uint32_t s0,
                                             uint32_t e_h, uint32_t e_max, uint32_t lane) {
  const uint32_t g = lane >> 4;
  const uint32_t t0 = tile * kTileTokens;
  // ---- QK on MFMA: c[mb][e] = S[token 16g + 4mb + e][h]
  f32x4 c[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    c[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const uint4 w = t.k[mb * (D / 64) + s / 2];
      const f16x8 a = (s & 1) ? i8x8_to_f16(w.z, w.w) : i8x8_to_f16(w.x, w.y);
      c[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[s], c[mb], 0, 0, 0);
      if (qlo) c[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[s], c[mb], 0, 0, 0);
    }
  }
  // ---- scores: k_scale of token 16g + j is broadcast from lane j of the row.
  float sc[16];
#define KVB_SCORE(mb, e) sc[4 * mb + e] = c[mb][e] * bc<4 * mb + e>(t.ks) * cq;
  KVB_SCORE(0, 0) KVB_SCORE(0, 1) KVB_SCORE(0, 2) KVB_SCORE(0, 3)
  KVB_SCORE(1, 0) KVB_SCORE(1, 1) KVB_SCORE(1, 2) KVB_SCORE(1, 3)
  KVB_SCORE(2, 0) KVB_SCORE(2, 1) KVB_SCORE(2, 2) KVB_SCORE(2, 3)
  KVB_SCORE(3, 0) KVB_SCORE(3, 1) KVB_SCORE(3, 2) KVB_SCORE(3, 3)
#undef KVB_SCORE
  const uint32_t tl = t0 + 16u * g + (lane & 15u);  // token of this lane's scales
  const bool lane_tok_ok = full || (tl >= s0 && tl < e_max);
  if (!full) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t tok = t0 + 16u * g + uint32_t(j);
      if (!(tok >= s0 && tok < e_h)) sc[j] = neg_inf();
    }
  }
  float mx = sc[0];
#pragma unroll
  for (int j = 1; j < 16; ++j) mx = fmaxf(mx, sc[j]);
  mx = rows_max(mx);
  const float m_new = fmaxf(st.m, mx);

  // PV weight exponent: the largest |v_scale| of the tile sets 2^kexp so that
  // every w * v_scale * 2^kexp (w <= 1) is below 2^15, inside f16 range.
  const float vmax = wave_max(lane_tok_ok ? fabsf(t.vs) : 0.f);
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
  const float vsk = lane_tok_ok ? __builtin_amdgcn_ldexpf(t.vs, k_new) : 0.f;
  float p[16];
  float lsum = 0.f;
#define KVB_WEIGHT(j)                  \
  {                                    \
    const float w = exp_e(sc[j] - m_use); \
    lsum += w;                         \
    p[j] = w * bc<j>(vsk);             \
  }
  KVB_WEIGHT(0) KVB_WEIGHT(1) KVB_WEIGHT(2) KVB_WEIGHT(3)
  KVB_WEIGHT(4) KVB_WEIGHT(5) KVB_WEIGHT(6) KVB_WEIGHT(7)
  KVB_WEIGHT(8) KVB_WEIGHT(9) KVB_WEIGHT(10) KVB_WEIGHT(11)
  KVB_WEIGHT(12) KVB_WEIGHT(13) KVB_WEIGHT(14) KVB_WEIGHT(15)
#undef KVB_WEIGHT
  st.l += lsum;
  // ---- P as f16 hi + lo; B operand of K-step js holds tokens 16g + 8js + e.
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
  // ---- PV on MFMA: acc[mb][e] += O[d = 16mb + 4g + e][h]
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) {
    const uint4 w = t.v[mb];
    const f16x8 a0 = i8x8_to_f16(w.x, w.y);
    const f16x8 a1 = i8x8_to_f16(w.z, w.w);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bh[0], st.acc[mb], 0, 0, 0);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bl[0], st.acc[mb], 0, 0, 0);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bh[1], st.acc[mb], 0, 0, 0);
    st.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bl[1], st.acc[mb], 0, 0, 0);
  }
}

template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void split_tiled_kernel(
    SplitArgs a, const float* __restrict__ q, const int64_t* __restrict__ qpos,
    const int64_t* __restrict__ kpos, const uint32_t* __restrict__ table,
    const int8_t* __restrict__ kdata, const int8_t* __restrict__ vdata,
    const float* __restrict__ kscale, const float* __restrict__ vscale, float* __restrict__ scratch) {
  __shared__ float wm_s[NW][16];
  __shared__ float wl_s[NW][16];
  __shared__ float wacc_s[NW][16][D];

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane & 15u, g = lane >> 4;
  const uint32_t split = blockIdx.x;
  const uint32_t kv = blockIdx.y % a.kv_heads, hblock = blockIdx.y / a.kv_heads;
  const uint32_t head_rows = a.rows * a.group;
  const uint32_t hr = hblock * 16u + h;
  const bool hvalid = hr < head_rows;
  const uint32_t row = hvalid ? hr / a.group : 0u;
  const uint32_t head = kv * a.group + (hvalid ? hr % a.group : 0u);

  // Split interval [s0, s1) and its tiles [k_first, k_last] (64-token tiles in
  // absolute logical coordinates; boundary tiles are masked per token).
  const uint64_t s0_64 = uint64_t(a.begin) + uint64_t(split) * a.split_tokens;
  const uint32_t s0 = s0_64 < a.end ? uint32_t(s0_64) : a.end;
  const uint32_t s1 = uint64_t(s0) + a.split_tokens < a.end ? s0 + a.split_tokens : a.end;
  const uint32_t k_first = s0 / kTileTokens;
  const uint32_t k_last = s1 > s0 ? (s1 - 1u) / kTileTokens : k_first;

  WaveCtx c;
  c.kbase = kdata;
  c.vbase = vdata;
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
  auto tile_of = [&](uint32_t i) {  // i-th tile of this wave, clamped for harmless prefetch
    const uint32_t k = k_first + wave + i * NW;
    return k < k_last ? k : k_last;
  };

  // Start streaming this wave's first tile before anything else: the page
  // entries and the KV loads do not depend on the visibility search below.
  Tile<D> ta, tb;
  const bool first = s1 > s0 && k_first + wave <= k_last;
  Pages pb = {}, pc = {};
  if (first) {
    const Pages pa = fetch_pages(c, tile_of(0));
    pb = fetch_pages(c, tile_of(1));
    load_tile<D>(ta, c, tile_of(0), pa);
    pc = fetch_pages(c, tile_of(2));
  }

  // Visible end per head-row: tokens [s0, e_h) are visible to this lane's row
  // (k_positions are nondecreasing).  Common case: the last token of the split
  // is visible to every row of the block, so nothing is searched.
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
  // Row-of-16 reductions (every row of lanes holds the same 16 head-rows).
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

  // Q of this head-row, dims [g*D/4, (g+1)*D/4), scaled by 2^kq into f16 hi/lo.
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

  State<D> st;
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) st.acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = neg_inf();
  st.l = 0.f;
  st.kexp = 100;

  // Tiles holding visible tokens: [k_first, (e_max - 1) / 64]; the wave's
  // first tile (already in flight) is the first of its round-robin share.
  const uint32_t k_vis = e_max > s0 ? (e_max - 1u) / kTileTokens : 0u;
  const uint32_t k_count = e_max > s0 ? k_vis + 1u - k_first : 0u;
  const uint32_t nt = k_count > wave ? (k_count - wave + NW - 1u) / NW : 0u;
  auto is_full = [&](uint32_t k) {
    return k * kTileTokens >= s0 && (k + 1u) * kTileTokens <= e_min;
  };
  for (uint32_t i = 0; i < nt; i += 2) {
    // Invariant: ta holds (loads of) tile i; pb, pc are the pages of tiles i+1, i+2.
    if (i + 1 < nt) load_tile<D>(tb, c, tile_of(i + 1), pb);
    const Pages pd = fetch_pages(c, tile_of(i + 3));
    {
      const uint32_t k = tile_of(i);
      compute_tile<D>(st, ta, k, qh, ql, qlo, cq, is_full(k), s0, e_h, e_max, lane);
    }
    if (i + 1 >= nt) break;
    if (i + 2 < nt) load_tile<D>(ta, c, tile_of(i + 2), pc);
    const Pages pe = fetch_pages(c, tile_of(i + 4));
    {
      const uint32_t k = tile_of(i + 1);
      compute_tile<D>(st, tb, k, qh, ql, qlo, cq, is_full(k), s0, e_h, e_max, lane);
    }
    pb = pd;
    pc = pe;
  }

  // ---- combine the waves through LDS and write the split partial.
  const float l_h = rows_sum(st.l);
  if (g == 0) {
    wm_s[wave][h] = st.m;
    wl_s[wave][h] = l_h;
  }
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) {
    const f32x4 x = st.acc[mb];
    float4 y;
    y.x = __builtin_amdgcn_ldexpf(x[0], -st.kexp);
    y.y = __builtin_amdgcn_ldexpf(x[1], -st.kexp);
    y.z = __builtin_amdgcn_ldexpf(x[2], -st.kexp);
    y.w = __builtin_amdgcn_ldexpf(x[3], -st.kexp);
    *reinterpret_cast<float4*>(&wacc_s[wave][h][16 * mb + 4 * g]) = y;
  }
  __syncthreads();
  const uint32_t nvalid = head_rows - hblock * 16u < 16u ? head_rows - hblock * 16u : 16u;
  constexpr uint32_t W = D + 2;
  for (uint32_t idx = threadIdx.x; idx < nvalid * W; idx += 64u * NW) {
    const uint32_t hh = idx / W, col = idx % W;
    float mm = wm_s[0][hh];
#pragma unroll
    for (int w = 1; w < NW; ++w) mm = fmaxf(mm, wm_s[w][hh]);
    float val = mm;
    if (col > 0) {
      val = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = wm_s[w][hh];
        if (mw == neg_inf()) continue;
        const float f = exp_e(mw - mm);
        val = fmaf(f, col == 1 ? wl_s[w][hh] : wacc_s[w][hh][col - 2], val);
      }
    }
    const uint32_t hr2 = hblock * 16u + hh;
    const uint32_t row2 = hr2 / a.group, head2 = kv * a.group + hr2 % a.group;
    scratch[((size_t(row2) * a.q_heads + head2) * a.splits + split) * W + col] = val;
  }
}

#define KVB_TILED_ARGS                                                                           \
  a, a.q, a.q_positions, a.k_positions, a.page_table, static_cast<const int8_t*>(a.k),             \
      static_cast<const int8_t*>(a.v), a.k_scales, a.v_scales, a.scratch

// LDS holds one D-float numerator row per head-row and wave for the final
// combine; NW is capped so that stays within 32 KiB.
template <int D>
constexpr int kMaxWaves = 512 / D;

template <int D>
hipError_t launch_d(const SplitArgs& a, int nw, hipStream_t stream) {
  const uint32_t hblocks = (a.rows * a.group + 15u) / 16u;
  const dim3 grid(a.splits, a.kv_heads * hblocks);
  if (nw > kMaxWaves<D>) nw = kMaxWaves<D>;
  switch (nw) {
    case 1: hipLaunchKernelGGL((split_tiled_kernel<D, 1>), grid, dim3(64), 0, stream, KVB_TILED_ARGS); break;
    case 2: hipLaunchKernelGGL((split_tiled_kernel<D, 2>), grid, dim3(128), 0, stream, KVB_TILED_ARGS); break;
    case 4:
      if constexpr (kMaxWaves<D> >= 4)
        hipLaunchKernelGGL((split_tiled_kernel<D, 4>), grid, dim3(256), 0, stream, KVB_TILED_ARGS);
      break;
    default:
      if constexpr (kMaxWaves<D> >= 8)
        hipLaunchKernelGGL((split_tiled_kernel<D, 8>), grid, dim3(512), 0, stream, KVB_TILED_ARGS);
      break;
  }
  return hipGetLastError();
}

template <int D>
hipError_t preload_d() {
  hipFuncAttributes attr{};
  hipError_t e;
  if ((e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_tiled_kernel<D, 1>))) != hipSuccess) return e;
  if ((e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_tiled_kernel<D, 2>))) != hipSuccess) return e;
  if constexpr (kMaxWaves<D> >= 4)
    if ((e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_tiled_kernel<D, 4>))) != hipSuccess) return e;
  if constexpr (kMaxWaves<D> >= 8)
    if ((e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_tiled_kernel<D, 8>))) != hipSuccess) return e;
  return hipSuccess;
}

// Waves per work-group: enough tiles per wave to keep its double buffer busy.
// KVB_TILED_WAVES (1, 2, 4, 8) overrides the choice, for tuning sweeps.
int waves_for(const SplitArgs& a) {
  static const int forced = [] {
    const char* e = std::getenv("KVB_TILED_WAVES");
    return e ? std::atoi(e) : 0;
  }();
  if (forced == 1 || forced == 2 || forced == 4 || forced == 8) return forced;
  const uint32_t tiles = (a.split_tokens + kTileTokens - 1) / kTileTokens + 1u;
  if (tiles >= 32) return 4;
  if (tiles >= 12) return 2;
  return 1;
}

}  // namespace

hipError_t launch_split_tiled(const SplitArgs& a, hipStream_t stream) {
  const int nw = waves_for(a);
  switch (a.dim) {
    case 64: return launch_d<64>(a, nw, stream);
    case 128: return launch_d<128>(a, nw, stream);
    case 256: return launch_d<256>(a, nw, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t preload_tiled() {
  hipError_t e = preload_d<64>();
  if (e != hipSuccess) return e;
  if ((e = preload_d<128>()) != hipSuccess) return e;
  return preload_d<256>();
}

}  // namespace kvb
