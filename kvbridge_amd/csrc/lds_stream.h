// LDS streaming machinery shared by the LDS-staged split kernels: tile
// geometry, the XOR swizzles of the K and V tile images in LDS, inline LDS
// reads and counter waits, page-table lookup, and the LDS-DMA issue of K/V
// tiles (general page size, and the page-tile fast path where a 64-token
// tile lies inside one page and addresses are a per-lane constant plus a
// uniform offset).
#pragma once
#include <cstdint>
#include <type_traits>

#include "device_common.h"

namespace kvb {
namespace lds {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kTileTokens = 64;
typedef __attribute__((address_space(3))) void* lds_ptr;

// Cache policy of every K/V/scale DMA load: non-temporal (each byte is read
// once per call).  At the dense rows-8 / group-6 / dim-256 geometry the
// 1,024-token split kernel measured 43.25 against 43.9 us with cached loads.
constexpr int kDmaAux = 2;

template <int D>
struct Geo {
  static constexpr uint32_t kChunks = D / 16;                 // 16-byte chunks per K row
  static constexpr uint32_t kRowsPerLoad = 1024 / D;          // K rows per 1 KiB load
  static constexpr uint32_t kKBytes = 64 * D;
  static constexpr uint32_t kVBytes = D * 64;
  static constexpr uint32_t kBufBytes = kKBytes + kVBytes + 512;
  static constexpr uint32_t kLoadsPerTile = D / 16 + D / 16 + 2;  // K, V, k-scales, v-scales
};

// K chunk swizzle: row r = 16q + 4mb + i (q token group, i row in quad).
template <int D>
__device__ __forceinline__ uint32_t swz_k(uint32_t r) {
  if constexpr (D == 64) return ((r >> 4) & 3u) ^ (((r >> 1) & 1u) << 1);
  else if constexpr (D == 128) return (r & 3u) ^ (((r >> 4) & 1u) << 2) ^ ((r >> 5) & 1u);
  else return (r & 3u) | (((r >> 4) & 3u) << 2);
}
__device__ __forceinline__ uint32_t swz_v(uint32_t d) { return ((d >> 1) ^ (d >> 2)) & 3u; }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)(const_cast<void*>(p))));
}

template <uint32_t B, uint32_t E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<uint32_t, B>{});
    static_for<B + 1, E>(f);
  }
}

template <uint32_t OFF>
__device__ __forceinline__ uint4 ds_read16(uint32_t addr) {
  uint4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Values produced by the inline LDS reads are only valid after wait_lds();
// the compiler does not know that, so every such value is passed through an
// empty volatile asm placed after the wait, which orders all its uses after it.
template <class T>
__device__ __forceinline__ void lds_fence1(T& v) {
  if constexpr (sizeof(T) == 16) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    v4 x = __builtin_bit_cast(v4, v);
    asm volatile("" : "+v"(x));
    v = __builtin_bit_cast(T, x);
  } else {
    asm volatile("" : "+v"(v));
  }
}
template <class... T>
__device__ __forceinline__ void lds_fence(T&... v) {
  (lds_fence1(v), ...);
}
// Wait for every vector-memory operation of this wave.
template <uint32_t N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N == 0, "hand-counted waits go through wait_vm_keep");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// Hand-counted wait: retire all but the N most recent vector-memory
// operations, where N is what the KEEP most recent tile DMA groups of this
// wave are meant to hold, so that every older group has landed.  N is a
// count of emitted instructions, which the source cannot see: each group
// starts with dma_group_mark(), and check_vm_waits.py verifies on the
// device assembly, along every path, that such a wait leaves no operation of
// an older group in flight (the KEEP value travels in an assembler comment).
template <uint32_t N, uint32_t KEEP>
__device__ __forceinline__ void wait_vm_keep() {
  static_assert(N > 0 && N <= 63 && KEEP > 0, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) ; kvb-keep %1" ::"i"(N), "i"(KEEP) : "memory");
}
// Start of one tile's DMA group in the device assembly (an assembler
// comment, no instruction).
__device__ __forceinline__ void dma_group_mark() { asm volatile(";kvb-dma-group"); }

struct Ctx {
  const int8_t* __restrict__ k;
  const int8_t* __restrict__ v;
  const float* __restrict__ ks;
  const float* __restrict__ vs;
  const uint32_t* __restrict__ table;
  uint32_t kv, kv_heads, P, pages, lp_lo, lp_hi, lane;
  uint32_t ptab;  // lane j: page_table[lp_lo + j] (logical pages lp_lo .. lp_lo + 63)
};

struct Pages4 {
  uint32_t g[4];
};

// Physical pages of the tile's four 16-token groups.  Taken from the
// per-wave window of page-table entries with v_readlane (no memory access);
// a split spanning more than 64 pages falls back to scalar loads beyond the
// window.
__device__ __forceinline__ Pages4 tile_pages(const Ctx& c, uint32_t tile) {
  const uint32_t t0 = tile * kTileTokens;
  Pages4 p;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lp = clampu((t0 + 16u * i) / c.P, c.lp_lo, c.lp_hi);
    const uint32_t rel = lp - c.lp_lo;
    const uint32_t x = rel < 64u ? __builtin_amdgcn_readlane(c.ptab, rel) : c.table[lp];
    p.g[i] = x < c.pages ? x : c.pages - 1u;
  }
  return p;
}
__device__ __forceinline__ uint32_t pick4(const Pages4& p, uint32_t grp) {
  const uint32_t lo = (grp & 1u) ? p.g[1] : p.g[0];
  const uint32_t hi = (grp & 1u) ? p.g[3] : p.g[2];
  return (grp & 2u) ? hi : lo;
}

// Issue the D/8 + 2 LDS-DMA loads of one tile into buffer `buf`.
template <int D>
__device__ __forceinline__ void issue_tile(const Ctx& c, uint32_t tile, uint8_t* buf) {
  using G = Geo<D>;
  const Pages4 pg = tile_pages(c, tile);
  const uint32_t t0 = tile * kTileTokens;
  const uint32_t lane = c.lane;
  // K: load i covers token rows [i*R, (i+1)*R), lane -> (row, position).
#pragma unroll
  for (uint32_t i = 0; i < G::kChunks; ++i) {
    const uint32_t r = i * G::kRowsPerLoad + lane / G::kChunks;
    const uint32_t pos = lane % G::kChunks;
    const uint32_t chunk = pos ^ swz_k<D>(r);
    const uint32_t grp = r >> 4;
    const uint32_t slot = (t0 + 16u * grp) % c.P + (r & 15u);
    const uint32_t row = (pick4(pg, grp) * c.kv_heads + c.kv) * c.P + slot;
    const int8_t* src = c.k + size_t(row) * D + 16u * chunk;
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)(buf + 1024u * i), 16, 0, kDmaAux);
  }
  // V: load i covers dim rows [16i, 16i+16), 4 chunks (token groups) per row.
  uint8_t* vb = buf + G::kKBytes;
#pragma unroll
  for (uint32_t i = 0; i < D / 16; ++i) {
    const uint32_t d = 16u * i + (lane >> 2);
    const uint32_t grp = (lane & 3u) ^ swz_v(d);
    const uint32_t slab = pick4(pg, grp) * c.kv_heads + c.kv;
    const int8_t* src = c.v + (size_t(slab) * D + d) * c.P + (t0 + 16u * grp) % c.P;
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)(vb + 1024u * i), 16, 0, kDmaAux);
  }
  // Scales of token t0 + lane.
  {
    const uint32_t grp = lane >> 4;
    const uint32_t si = (pick4(pg, grp) * c.kv_heads + c.kv) * c.P + (t0 + 16u * grp) % c.P + (lane & 15u);
    uint8_t* sb = buf + G::kKBytes + G::kVBytes;
    __builtin_amdgcn_global_load_lds(c.ks + si, (lds_ptr)(sb), 4, 0, kDmaAux);
    __builtin_amdgcn_global_load_lds(c.vs + si, (lds_ptr)(sb + 256), 4, 0, kDmaAux);
  }
}

// ---- page-tile path (page_tokens a multiple of 64: a tile lies in one page).
// The DMA addresses are a per-lane constant (voffset, computed once) plus a
// per-tile uniform base (soffset), so issuing a tile costs no VALU work.
// Buffer descriptors also bound every access to its array.
constexpr int32_t kRsrcFlags = 0x00020000;  // raw 32-bit buffer, gfx9 dword3

struct PtCtx {
  __amdgpu_buffer_rsrc_t rk, rv, rks, rvs;
  uint32_t voff_k[8];   // K load i: per-lane byte offset inside the tile's K rows (D <= 128: i < 8)
  uint32_t voff_k2[8];  // K loads 8..15 (D == 256)
  uint32_t voff_v;      // V: per-lane byte offset inside the 16-row block
  uint32_t voff_s;      // scales: 4 * lane
};

template <int D>
__device__ __forceinline__ void pt_init(PtCtx& c, const int8_t* k, const int8_t* v, const float* ks, const float* vs,
                                        uint32_t kv_bytes, uint32_t scale_bytes, uint32_t P, uint32_t lane) {
  using G = Geo<D>;
  c.rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(k), 0, int(kv_bytes), kRsrcFlags);
  c.rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(v), 0, int(kv_bytes), kRsrcFlags);
  c.rks = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ks), 0, int(scale_bytes), kRsrcFlags);
  c.rvs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vs), 0, int(scale_bytes), kRsrcFlags);
#pragma unroll
  for (uint32_t i = 0; i < G::kChunks; ++i) {
    const uint32_t r = i * G::kRowsPerLoad + lane / G::kChunks;
    const uint32_t chunk = (lane % G::kChunks) ^ swz_k<D>(r);
    const uint32_t off = r * D + 16u * chunk;
    if (i < 8) c.voff_k[i] = off;
    else c.voff_k2[i - 8] = off;
  }
  const uint32_t d = lane >> 2;
  c.voff_v = d * P + 16u * ((lane & 3u) ^ swz_v(d));
  c.voff_s = 4u * lane;
}

template <int D>
__device__ __forceinline__ void pt_issue(const PtCtx& c, uint32_t slab, uint32_t slot0, uint32_t P, uint8_t* buf) {
  using G = Geo<D>;
  const uint32_t kbase = (slab * P + slot0) * D;  // bytes of the tile's first K row
#pragma unroll
  for (uint32_t i = 0; i < G::kChunks; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rk, (lds_ptr)(buf + 1024u * i), 16,
                                             i < 8 ? c.voff_k[i] : c.voff_k2[i - 8], kbase, 0, kDmaAux);
  const uint32_t vbase = slab * D * P + slot0;  // V row 0 of the tile
  uint8_t* vb = buf + G::kKBytes;
#pragma unroll
  for (uint32_t i = 0; i < D / 16; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rv, (lds_ptr)(vb + 1024u * i), 16, c.voff_v,
                                             vbase + 16u * i * P, 0, kDmaAux);
  const uint32_t sbase = (slab * P + slot0) * 4u;
  uint8_t* sb = buf + G::kKBytes + G::kVBytes;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rks, (lds_ptr)(sb), 4, c.voff_s, sbase, 0, kDmaAux);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rvs, (lds_ptr)(sb + 256), 4, c.voff_s, sbase, 0, kDmaAux);
}

// ---- one tile's DMA shared by WT waves: wave `part` issues the K and V
// loads i with i % WT == part, part 0 also the k-scales and part 1 the
// v-scales (WT == 1: one wave issues everything), so a wave holds the
// per-lane offsets of its own loads only and issuing costs each wave a
// WT-th of the instructions.
template <int D, uint32_t WT>
struct PtPart {
  static_assert(WT >= 1 && Geo<D>::kChunks % WT == 0 && (D / 16) % WT == 0, "whole shares");
  static constexpr uint32_t kK = Geo<D>::kChunks / WT;  // K loads of one wave
  static constexpr uint32_t kV = (D / 16) / WT;         // V loads of one wave
  __amdgpu_buffer_rsrc_t rk, rv, rks, rvs;
  uint32_t voff_k[kK];
  uint32_t voff_v, voff_s;
};

template <int D, uint32_t WT>
__device__ __forceinline__ void pt_part_init(PtPart<D, WT>& c, const int8_t* k, const int8_t* v, const float* ks,
                                             const float* vs, uint32_t kv_bytes, uint32_t scale_bytes, uint32_t P,
                                             uint32_t lane, uint32_t part) {
  using G = Geo<D>;
  c.rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(k), 0, int(kv_bytes), kRsrcFlags);
  c.rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(v), 0, int(kv_bytes), kRsrcFlags);
  c.rks = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ks), 0, int(scale_bytes), kRsrcFlags);
  c.rvs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vs), 0, int(scale_bytes), kRsrcFlags);
#pragma unroll
  for (uint32_t m = 0; m < PtPart<D, WT>::kK; ++m) {
    const uint32_t r = (part + WT * m) * G::kRowsPerLoad + lane / G::kChunks;
    c.voff_k[m] = r * D + 16u * ((lane % G::kChunks) ^ swz_k<D>(r));
  }
  const uint32_t d = lane >> 2;
  c.voff_v = d * P + 16u * ((lane & 3u) ^ swz_v(d));
  c.voff_s = 4u * lane;
}

// Page-tile path (a tile lies in one page): this wave's share of the tile
// whose first K row is row `slot0` of slab `slab`.
template <int D, uint32_t WT>
__device__ __forceinline__ void pt_part_issue(const PtPart<D, WT>& c, uint32_t slab, uint32_t slot0, uint32_t P,
                                              uint8_t* buf, uint32_t part) {
  using G = Geo<D>;
  const uint32_t kbase = (slab * P + slot0) * D;
#pragma unroll
  for (uint32_t m = 0; m < PtPart<D, WT>::kK; ++m)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rk, (lds_ptr)(buf + 1024u * (part + WT * m)), 16, c.voff_k[m], kbase,
                                             0, kDmaAux);
  const uint32_t vbase = slab * D * P + slot0;
  uint8_t* vb = buf + G::kKBytes;
#pragma unroll
  for (uint32_t m = 0; m < PtPart<D, WT>::kV; ++m) {
    const uint32_t i = part + WT * m;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rv, (lds_ptr)(vb + 1024u * i), 16, c.voff_v, vbase + 16u * i * P, 0, kDmaAux);
  }
  uint8_t* sb = buf + G::kKBytes + G::kVBytes;
  if (WT == 1u || part == 0u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rks, (lds_ptr)(sb), 4, c.voff_s, (slab * P + slot0) * 4u, 0, kDmaAux);
  if (WT == 1u || part == 1u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rvs, (lds_ptr)(sb + 256), 4, c.voff_s, (slab * P + slot0) * 4u, 0, kDmaAux);
}

// Any page size: this wave's share of tile `tile` (pages of its four
// 16-token groups from the page-table window).
template <int D, uint32_t WT>
__device__ __forceinline__ void part_issue(const Ctx& c, uint32_t tile, uint8_t* buf, uint32_t part) {
  using G = Geo<D>;
  const Pages4 pg = tile_pages(c, tile);
  const uint32_t t0 = tile * kTileTokens;
  const uint32_t lane = c.lane;
#pragma unroll
  for (uint32_t m = 0; m < PtPart<D, WT>::kK; ++m) {
    const uint32_t i = part + WT * m;
    const uint32_t r = i * G::kRowsPerLoad + lane / G::kChunks;
    const uint32_t chunk = (lane % G::kChunks) ^ swz_k<D>(r);
    const uint32_t grp = r >> 4;
    const uint32_t row = (pick4(pg, grp) * c.kv_heads + c.kv) * c.P + (t0 + 16u * grp) % c.P + (r & 15u);
    __builtin_amdgcn_global_load_lds(c.k + size_t(row) * D + 16u * chunk, (lds_ptr)(buf + 1024u * i), 16, 0, kDmaAux);
  }
  uint8_t* vb = buf + G::kKBytes;
#pragma unroll
  for (uint32_t m = 0; m < PtPart<D, WT>::kV; ++m) {
    const uint32_t i = part + WT * m;
    const uint32_t d = 16u * i + (lane >> 2);
    const uint32_t grp = (lane & 3u) ^ swz_v(d);
    const uint32_t slab = pick4(pg, grp) * c.kv_heads + c.kv;
    __builtin_amdgcn_global_load_lds(c.v + (size_t(slab) * D + d) * c.P + (t0 + 16u * grp) % c.P,
                                     (lds_ptr)(vb + 1024u * i), 16, 0, kDmaAux);
  }
  if (WT == 1u || part < 2u) {
    const uint32_t grp = lane >> 4;
    const uint32_t si = (pick4(pg, grp) * c.kv_heads + c.kv) * c.P + (t0 + 16u * grp) % c.P + (lane & 15u);
    uint8_t* sb = buf + G::kKBytes + G::kVBytes;
    if (WT == 1u || part == 0u) __builtin_amdgcn_global_load_lds(c.ks + si, (lds_ptr)(sb), 4, 0, kDmaAux);
    if (WT == 1u || part == 1u) __builtin_amdgcn_global_load_lds(c.vs + si, (lds_ptr)(sb + 256), 4, 0, kDmaAux);
  }
}

// Position of the next tile to issue: (logical page, slot of its first token),
// advanced without division; clamped at the split's last tile.
struct IssuePos {
  uint32_t k, lp, slot;
};

// Per-lane LDS byte offsets inside a tile buffer (tile-invariant).  The K
// swizzle depends only on lane bits, so M-block mb adds 4*mb*D; likewise V
// row block mb adds 1024*mb (both folded into ds_read immediates).
template <int D>
struct ReadOffsets {
  uint32_t k[D / 64];  // [chunk j] for M-block 0
  uint32_t v;          // M-block 0
  uint32_t sc;         // k-scales of tokens 16g .. 16g+15
};

template <int D>
__device__ __forceinline__ ReadOffsets<D> read_offsets(uint32_t lane) {
  using G = Geo<D>;
  ReadOffsets<D> o;
  const uint32_t m = lane & 15u, g = lane >> 4;
  const uint32_t r = 16u * (m >> 2) + (m & 3u);
#pragma unroll
  for (uint32_t j = 0; j < D / 64; ++j) {
    const uint32_t chunk = g * (G::kChunks / 4) + j;
    o.k[j] = r * D + 16u * (chunk ^ swz_k<D>(r));
  }
  o.v = G::kKBytes + m * 64u + 16u * (g ^ swz_v(m));
  o.sc = G::kKBytes + G::kVBytes + 64u * g;
  return o;
}


// ---- item streaming (two-pass kernels): an item is the K tile image or the
// V tile image of one 64-token tile, followed by both scale vectors, so every
// item is D/16 + 2 loads whatever its kind.
template <int D>
__device__ __forceinline__ void pt_issue_item(const PtCtx& c, bool is_v, uint32_t slab, uint32_t slot0, uint32_t P,
                                              uint8_t* buf) {
  using G = Geo<D>;
  if (!is_v) {
    const uint32_t kbase = (slab * P + slot0) * D;
#pragma unroll
    for (uint32_t i = 0; i < G::kChunks; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rk, (lds_ptr)(buf + 1024u * i), 16,
                                               i < 8 ? c.voff_k[i] : c.voff_k2[i - 8], kbase, 0, kDmaAux);
  } else {
    const uint32_t vbase = slab * D * P + slot0;
#pragma unroll
    for (uint32_t i = 0; i < D / 16; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rv, (lds_ptr)(buf + 1024u * i), 16, c.voff_v,
                                               vbase + 16u * i * P, 0, kDmaAux);
  }
  const uint32_t sbase = (slab * P + slot0) * 4u;
  uint8_t* sb = buf + G::kKBytes;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rks, (lds_ptr)(sb), 4, c.voff_s, sbase, 0, kDmaAux);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rvs, (lds_ptr)(sb + 256), 4, c.voff_s, sbase, 0, kDmaAux);
}

template <int D>
__device__ __forceinline__ void gen_issue_item(const Ctx& c, bool is_v, uint32_t tile, uint8_t* buf) {
  using G = Geo<D>;
  const Pages4 pg = tile_pages(c, tile);
  const uint32_t t0 = tile * kTileTokens;
  const uint32_t lane = c.lane;
  if (!is_v) {
#pragma unroll
    for (uint32_t i = 0; i < G::kChunks; ++i) {
      const uint32_t r = i * G::kRowsPerLoad + lane / G::kChunks;
      const uint32_t chunk = (lane % G::kChunks) ^ swz_k<D>(r);
      const uint32_t grp = r >> 4;
      const uint32_t slot = (t0 + 16u * grp) % c.P + (r & 15u);
      const uint32_t row = (pick4(pg, grp) * c.kv_heads + c.kv) * c.P + slot;
      __builtin_amdgcn_global_load_lds(c.k + size_t(row) * D + 16u * chunk, (lds_ptr)(buf + 1024u * i), 16, 0, kDmaAux);
    }
  } else {
#pragma unroll
    for (uint32_t i = 0; i < D / 16; ++i) {
      const uint32_t d = 16u * i + (lane >> 2);
      const uint32_t grp = (lane & 3u) ^ swz_v(d);
      const uint32_t slab = pick4(pg, grp) * c.kv_heads + c.kv;
      __builtin_amdgcn_global_load_lds(c.v + (size_t(slab) * D + d) * c.P + (t0 + 16u * grp) % c.P,
                                       (lds_ptr)(buf + 1024u * i), 16, 0, kDmaAux);
    }
  }
  const uint32_t grp = lane >> 4;
  const uint32_t si = (pick4(pg, grp) * c.kv_heads + c.kv) * c.P + (t0 + 16u * grp) % c.P + (lane & 15u);
  uint8_t* sb = buf + G::kKBytes;
  __builtin_amdgcn_global_load_lds(c.ks + si, (lds_ptr)(sb), 4, 0, kDmaAux);
  __builtin_amdgcn_global_load_lds(c.vs + si, (lds_ptr)(sb + 256), 4, 0, kDmaAux);
}

__device__ __forceinline__ uint32_t ds_read4(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
template <uint32_t OFF>
__device__ __forceinline__ u32x4_t ds_read16v(uint32_t addr) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <uint32_t OFF>
__device__ __forceinline__ uint32_t ds_read4o(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <uint32_t OFF>
__device__ __forceinline__ void ds_write16(uint32_t addr, u32x4_t v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(OFF) : "memory");
}
template <uint32_t OFF>
__device__ __forceinline__ void ds_write1(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b8 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(OFF) : "memory");
}

}  // namespace lds
}  // namespace kvb
