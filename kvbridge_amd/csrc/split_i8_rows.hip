// Int8-MFMA split partials for many head-rows per kv head, e.g. the
// reference's dense rows-8 / group-6 geometry (48 head-rows per kv head, dim
// 256; attention_shape.cpp:67-70).
//
// One work-group of four waves per (split, kv head) streams the split's KV
// tiles through a two-slot LDS ring (CT tiles per slot: the tile images of
// lds_stream.h), and wave w runs head-row block w (16 head-rows) over each
// tile, so the split's KV is read from HBM once for all its head-rows.  More
// than 64 head-rows (four blocks) stream the split again per group of four
// blocks.  The DMA runs one phase ahead of the compute:
//  - fewer blocks than waves (one round, e.g. 48 head-rows): the idle wave
//    issues every tile's DMA alone, phase p + 1 right after the barrier that
//    starts phase p (every wave is then done with its slot), so a busy memory
//    system's issue stalls never hold up a computing wave, and one barrier
//    per phase suffices;
//  - otherwise the waves share each tile's DMA and issue phase p + 2 after a
//    second barrier that ends phase p.
// The prologue's own loads (Q, positions) go out before the first DMA, so
// its waits do not include it.
//
// Per phase, wave-local and exact in integers as in the single-block int8
// kernel (split_i8.h):
//  - QK: v_mfma_i32_16x16x64_i8 with the raw INT8 K codes as A and digit dg
//    (hi, mid, lo) of the 23-bit integer 2^kq * q of the block's 16 head-rows
//    as B; the three digit products of a (token, head-row) land in one lane.
//  - phase maximum m_p per head-row, running maximum m = max(m, m_p); the
//    fp32 numerators and denominators so far are rescaled by 2^(m_old - m).
//  - PV: the weights 2^(s - m) * v_scale * 2^kp (below 2^21; kp from the
//    phase's largest v-scale) as three 7-bit digits form B in the token
//    order the QK result left in each lane (QK M-block mb takes tokens
//    16q + 4mb + r, so lane (h, g) holds tokens 16g .. 16g + 15, which are
//    its k-positions of PV), so nothing moves between lanes.  Each 16-dim
//    block's three int32 digit sums over the phase are folded into fp32 at
//    once (2^-kp).
// QK and PV are software-pipelined over their 16-row / 16-dim blocks: a
// block's LDS reads go out two blocks ahead (issued without a wait; the
// wait is a separate statement and the results are pinned after it), and a
// block's MFMAs are interleaved with the previous block's VALU work (scores,
// or the fold), so the matrix core, the VALU and the LDS work at once with
// one wave per SIMD.  Branches that would split those scheduling regions
// (masking) are taken once per phase.
// A wave owns whole head-rows and writes their partials from registers.
// Requires splits that start on a 64-token tile (host-checked).
#include <atomic>
#include <cstdio>
#include <type_traits>

#include "kernels.h"
#include "device_common.h"
#include "lds_stream.h"

namespace kvb {
namespace {

using namespace lds;
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlocks = 4;  // head-row blocks per round, one wave each
constexpr int kWaves = kBlocks;
constexpr float kLn2 = 0.6931471805599453f;

// LDS reads as one asm statement each: the reads and the wait for them, so
// the results exist only once the data is there (an asm read whose wait
// came later could have its destination copied by the compiler before the
// data lands), and the compiler sees no LDS load it would order after the
// in-flight DMA of the next phase.  MFMAs issued before a batch keep
// running while the wave waits for it.
template <uint32_t O0, uint32_t O1, uint32_t O2, uint32_t O3>
__device__ __forceinline__ void ds_read16x4(uint32_t a, u32x4_t& r0, u32x4_t& r1, u32x4_t& r2, u32x4_t& r3) {
  asm volatile(
      "ds_read_b128 %0, %4 offset:%5\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b128 %2, %4 offset:%7\n\t"
      "ds_read_b128 %3, %4 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(a), "i"(O0), "i"(O1), "i"(O2), "i"(O3)
      : "memory");
}
template <uint32_t O0, uint32_t O1>
__device__ __forceinline__ void ds_read16x2(uint32_t a, u32x4_t& r0, u32x4_t& r1) {
  asm volatile(
      "ds_read_b128 %0, %2 offset:%3\n\t"
      "ds_read_b128 %1, %2 offset:%4\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1)
      : "v"(a), "i"(O0), "i"(O1)
      : "memory");
}
template <uint32_t O0>
__device__ __forceinline__ uint32_t ds_read4_sync(uint32_t a) {
  uint32_t r;
  asm volatile("ds_read_b32 %0, %1 offset:%2\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(a), "i"(O0) : "memory");
  return r;
}

// K rows of one QK M-block over KS K-steps (one address per K-step, same
// immediate) plus the block's four k-scales, in one statement.
template <uint32_t OK, uint32_t OS>
__device__ __forceinline__ void ds_read_kblock(const uint32_t (&a)[4], uint32_t as, u32x4_t (&r)[4], u32x4_t& rs) {
  asm volatile(
      "ds_read_b128 %0, %5 offset:%10\n\t"
      "ds_read_b128 %1, %6 offset:%10\n\t"
      "ds_read_b128 %2, %7 offset:%10\n\t"
      "ds_read_b128 %3, %8 offset:%10\n\t"
      "ds_read_b128 %4, %9 offset:%11\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(rs)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(as), "i"(OK), "i"(OS)
      : "memory");
}
template <uint32_t OK, uint32_t OS>
__device__ __forceinline__ void ds_read_kblock(const uint32_t (&a)[2], uint32_t as, u32x4_t (&r)[2], u32x4_t& rs) {
  asm volatile(
      "ds_read_b128 %0, %3 offset:%6\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b128 %2, %5 offset:%7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(rs)
      : "v"(a[0]), "v"(a[1]), "v"(as), "i"(OK), "i"(OS)
      : "memory");
}

// LDS reads issued without a wait (the wait is a separate statement, and
// every use of the results comes after it, pinned there; the kernels'
// assembly is checked for early uses by check_lds_waits.py).
template <uint32_t O0, uint32_t O1>
__device__ __forceinline__ void ds_issue16x2(uint32_t a, u32x4_t& r0, u32x4_t& r1) {
  asm volatile(
      "ds_read_b128 %0, %2 offset:%3\n\t"
      "ds_read_b128 %1, %2 offset:%4"
      : "=&v"(r0), "=&v"(r1)
      : "v"(a), "i"(O0), "i"(O1)
      : "memory");
}
template <uint32_t O0, uint32_t O1, uint32_t O2, uint32_t O3>
__device__ __forceinline__ void ds_issue16x4(uint32_t a, u32x4_t& r0, u32x4_t& r1, u32x4_t& r2, u32x4_t& r3) {
  asm volatile(
      "ds_read_b128 %0, %4 offset:%5\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b128 %2, %4 offset:%7\n\t"
      "ds_read_b128 %3, %4 offset:%8"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(a), "i"(O0), "i"(O1), "i"(O2), "i"(O3)
      : "memory");
}
// ds_read_kblock without the wait.
template <uint32_t OK, uint32_t OS>
__device__ __forceinline__ void ds_issue_kblock(const uint32_t (&a)[4], uint32_t as, u32x4_t (&r)[4], u32x4_t& rs) {
  asm volatile(
      "ds_read_b128 %0, %5 offset:%10\n\t"
      "ds_read_b128 %1, %6 offset:%10\n\t"
      "ds_read_b128 %2, %7 offset:%10\n\t"
      "ds_read_b128 %3, %8 offset:%10\n\t"
      "ds_read_b128 %4, %9 offset:%11"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(rs)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(as), "i"(OK), "i"(OS)
      : "memory");
}
template <uint32_t OK, uint32_t OS>
__device__ __forceinline__ void ds_issue_kblock(const uint32_t (&a)[2], uint32_t as, u32x4_t (&r)[2], u32x4_t& rs) {
  asm volatile(
      "ds_read_b128 %0, %3 offset:%6\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b128 %2, %5 offset:%7"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(rs)
      : "v"(a[0]), "v"(a[1]), "v"(as), "i"(OK), "i"(OS)
      : "memory");
}
template <uint32_t O0>
__device__ __forceinline__ void ds_issue16x1(uint32_t a, u32x4_t& r0) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(r0) : "v"(a), "i"(O0) : "memory");
}
// s_barrier without the memory fences of __syncthreads (no wait for the
// wave's own loads before it); the asm keeps memory accesses on their side.
__device__ __forceinline__ void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }
template <uint32_t N>
__device__ __forceinline__ void wait_lgkm() { asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory"); }

// Pins a value at this point of the instruction stream: its producers stay
// before, its users after (keeps each block's VALU next to its MFMAs
// instead of letting the compiler sink it, which lengthens live ranges).
template <class T>
__device__ __forceinline__ void pin(T& v) {
  if constexpr (sizeof(T) == 16) {
    u32x4_t x = __builtin_bit_cast(u32x4_t, v);
    asm volatile("" : "+v"(x));
    v = __builtin_bit_cast(T, x);
  } else {
    asm volatile("" : "+v"(v));
  }
}

template <int D>
struct RowsGeo {
  static constexpr int kCT = D == 256 ? 2 : 4;  // tiles per phase (one LDS slot, about 66 KiB)
  static constexpr uint32_t kSlot = kCT * Geo<D>::kBufBytes;
};

template <int D, bool PT>
__global__ __launch_bounds__(64 * kWaves) void split_i8_rows_kernel(
    SplitArgs a, const float* __restrict__ q, const int64_t* __restrict__ qpos,
    const int64_t* __restrict__ kpos, const uint32_t* __restrict__ table,
    const int8_t* __restrict__ kdata, const int8_t* __restrict__ vdata,
    const float* __restrict__ kscale, const float* __restrict__ vscale, float* __restrict__ scratch, uint32_t spw) {
  using G = Geo<D>;
  constexpr int CT = RowsGeo<D>::kCT;
  constexpr uint32_t kSlot = RowsGeo<D>::kSlot;
  constexpr int KS = D / 64;  // K-steps of QK
  constexpr int MB = D / 16;  // 16-dim blocks of PV
  constexpr uint32_t W = D + 2;
  static_assert(CT <= kWaves, "every tile of a phase has an issuing wave");
  static_assert(G::kLoadsPerTile <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kSlot];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t n = lane & 15u, g = lane >> 4;
  const uint32_t kv = blockIdx.y;
  const uint32_t head_rows = a.rows * a.group, hblocks = (head_rows + 15u) / 16u;
  const uint32_t rounds = (hblocks + kBlocks - 1u) / kBlocks;

  // Splits [sp0, sp1) of this work-group, tokens [s0, s1).  With spw > 1 a
  // split is a whole number of phases (pps; host-checked) and every split's
  // partial is written at its last phase, so the partials are those of one
  // work-group per split.
  const uint32_t sp0 = blockIdx.x * spw;
  const uint32_t sp1 = sp0 + spw < a.splits ? sp0 + spw : a.splits;
  const uint32_t pps = a.split_tokens / (kTileTokens * CT);
  const uint64_t s0_64 = uint64_t(a.begin) + uint64_t(sp0) * a.split_tokens;
  const uint32_t s0 = s0_64 < a.end ? uint32_t(s0_64) : a.end;
  const uint64_t s1_64 = uint64_t(a.begin) + uint64_t(sp1) * a.split_tokens;
  const uint32_t s1 = s1_64 < a.end ? uint32_t(s1_64) : a.end;
  const uint32_t k_first = s0 / kTileTokens;
  const uint32_t ntiles = s1 > s0 ? (s1 - 1u) / kTileTokens + 1u - k_first : 0u;
  const uint32_t nphase = (ntiles + CT - 1u) / CT;

  // The DMA of each tile of a phase is shared by WT waves (wave w: tile
  // w / WT of the phase, share w % WT).
  constexpr uint32_t WT = kWaves / CT;
  using Part = PtPart<D, WT>;
  const uint32_t it_j = wave / WT, part = wave % WT;
  Ctx c;
  Part pc;
  if (ntiles > 0) {
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
    const uint32_t lp = c.lp_lo + lane;
    c.ptab = lp <= c.lp_hi ? table[lp] : 0u;
    if constexpr (PT) {
      const uint32_t kv_bytes = a.pages * a.kv_heads * a.page_tokens * uint32_t(D);
      const uint32_t sc_bytes = a.pages * a.kv_heads * a.page_tokens * 4u;
      pt_part_init<D, WT>(pc, kdata, vdata, kscale, vscale, kv_bytes, sc_bytes, a.page_tokens, lane, part);
    }
  }
  // When the blocks leave a wave idle (fewer blocks than waves: one round),
  // that wave issues every DMA of the split alone, so the issue stalls of a
  // busy memory system never hold up a computing wave; otherwise the waves
  // share each tile's DMA.
  const bool idle_dma = hblocks < uint32_t(kBlocks);
  const bool dma_wave = idle_dma && wave == uint32_t(kWaves - 1);
  using Part1 = PtPart<D, 1>;
  Part1 pc1;
  if constexpr (PT) {
    if (dma_wave && ntiles > 0) {
      const uint32_t kv_bytes = a.pages * a.kv_heads * a.page_tokens * uint32_t(D);
      const uint32_t sc_bytes = a.pages * a.kv_heads * a.page_tokens * 4u;
      pt_part_init<D, 1>(pc1, kdata, vdata, kscale, vscale, kv_bytes, sc_bytes, a.page_tokens, lane, 0u);
    }
  }
  // Tile p * CT + j of the split goes to slot p & 1, position j.
  auto issued = [&](uint32_t p) -> bool {
    return idle_dma ? dma_wave && p * CT < ntiles : p * CT + it_j < ntiles;
  };
  auto issue_tile_of = [&](auto wtc, const auto& ppc, uint32_t k, uint8_t* buf, uint32_t prt)
                           __attribute__((always_inline)) {
    constexpr uint32_t W2 = decltype(wtc)::value;
    dma_group_mark();
    if constexpr (PT) {
      const uint32_t lp = k * kTileTokens / a.page_tokens;
      const uint32_t rel = lp - c.lp_lo;
      uint32_t phys = rel < 64u ? __builtin_amdgcn_readlane(c.ptab, rel) : table[lp];
      phys = phys < a.pages ? phys : a.pages - 1u;
      pt_part_issue<D, W2>(ppc, phys * a.kv_heads + kv, k * kTileTokens - lp * a.page_tokens, a.page_tokens, buf,
                           prt);
    } else {
      part_issue<D, W2>(c, k, buf, prt);
    }
  };
  auto issue = [&](uint32_t p) {
    if (!issued(p)) return;
    if (idle_dma) {
      static_for<0, CT>([&](auto jc) __attribute__((always_inline)) {
        constexpr uint32_t j = decltype(jc)::value;
        if (p * CT + j < ntiles)
          issue_tile_of(std::integral_constant<uint32_t, 1>{}, pc1, k_first + p * CT + j,
                        smem + (p & 1u) * kSlot + j * G::kBufBytes, 0u);
      });
    } else {
      issue_tile_of(std::integral_constant<uint32_t, WT>{}, pc, k_first + p * CT + it_j,
                    smem + (p & 1u) * kSlot + it_j * G::kBufBytes, part);
    }
  };
  // Before phase p: this wave's loads of phase p done, those of phase p + 1
  // may stay in flight (shared issue: phase p + 1 went out at the end of
  // phase p - 1; the DMA wave issues phase p + 1 only after this wait).
  auto wait_next = [&](uint32_t p) __attribute__((always_inline)) {
    if (idle_dma || !issued(p + 1u)) {
      wait_vm<0>();
    } else if (WT == 1u) {
      wait_vm_keep<Part::kK + Part::kV + 2, 1>();
    } else if (part < 2u) {
      wait_vm_keep<Part::kK + Part::kV + 1, 1>();
    } else {
      wait_vm_keep<Part::kK + Part::kV, 1>();
    }
  };

  // Per-lane LDS offsets inside a tile image.  Row i of QK M-block mb is
  // token 16 * (i >> 2) + 4mb + (i & 3), so the QK result leaves tokens
  // 16g .. 16g + 15 of head-row h in lane (h, g) and the PV A operand of lane
  // (d, g) is V[d][16g .. 16g + 15], one 16-byte read.  K: lane (n, g) reads
  // row r = 16 * (n >> 2) + (n & 3) + 4mb, chunk 4s + g, at position
  // (4s + g) ^ swz_k(r) (swz_k(r) does not depend on mb).  V: dim row
  // d = 16mb + n, token group g at position g ^ swz_v(d) (swz_v(d) = swz_v(n)).
  const uint32_t lds_base = lds_addr(smem);
  uint32_t koff[KS];
  {
    const uint32_t r0 = 16u * (n >> 2) + (n & 3u);
#pragma unroll
    for (int s = 0; s < KS; ++s) koff[s] = r0 * D + 16u * ((4u * s + g) ^ swz_k<D>(r0));
  }
  const uint32_t voff = G::kKBytes + 64u * n + 16u * (g ^ swz_v(n));
  const uint32_t soff = G::kKBytes + G::kVBytes + 64u * g;  // k-scales of tokens 16g .. ; v-scales at +256
  const uint32_t vmoff = G::kKBytes + G::kVBytes + 256u + 4u * lane;

  for (uint32_t round = 0; round < rounds; ++round) {
    const uint32_t hblock = wave + kBlocks * round;
    const bool has = hblock < hblocks;  // wave-uniform
    // ---- block prologue: visibility, Q digits.  The prologue's own requests
    // (Q elements, the split's last key position, the block's query
    // positions) go out before the first two phases' DMA, so its waits do not
    // include the DMA.
    const uint32_t hr = hblock * 16u + n;
    const bool hvalid = hr < head_rows;
    const uint32_t row = hvalid ? hr / a.group : 0u;
    const uint32_t head = kv * a.group + (hvalid ? hr % a.group : 0u);
    uint32_t e_h = s0, e_min = s0, e_max = s0;
    i32x4 qd[3][KS];
    float cs = 0.f;
    // lane (h, g) holds dims 64s + 16g .. +15 of head-row h
    float qv[KS][16];
    int64_t klast = 0, qpos_l = INT64_MAX;  // lane i: query position of row r_lo + i
    const uint32_t r_lo = hblock * 16u / a.group;
    const uint32_t r_hi = (hblock * 16u + 15u < head_rows ? hblock * 16u + 15u : head_rows - 1u) / a.group;
    if (has) {
      if (hvalid) {
        const float* qp = q + (size_t(row) * a.q_heads + head) * D + 16u * g;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float4 x = reinterpret_cast<const float4*>(qp + 64 * s)[j];
            qv[s][4 * j] = x.x;
            qv[s][4 * j + 1] = x.y;
            qv[s][4 * j + 2] = x.z;
            qv[s][4 * j + 3] = x.w;
          }
      } else {
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int i = 0; i < 16; ++i) qv[s][i] = 0.f;
      }
      if (s1 > s0) {
        klast = kpos[s1 - 1u];
        if (lane <= r_hi - r_lo) qpos_l = qpos[r_lo + lane];  // at most 16 rows per block
      }
    }
    if (nphase > 0) issue(0);
    if (nphase > 1 && !idle_dma) issue(1);  // (the DMA wave issues phase p + 1 at the start of phase p)
    if (has) {
      if (s1 > s0) {
        if (__ballot(klast > qpos_l) == 0) {  // every row of the block sees the whole split
          e_h = s1;
        } else {
          for (uint32_t r = r_lo; r <= r_hi; ++r) {
            const uint64_t xb = uint64_t(qpos_l);
            const uint32_t xlo = __builtin_amdgcn_readlane(uint32_t(xb), r - r_lo);
            const uint32_t xhi = __builtin_amdgcn_readlane(uint32_t(xb >> 32), r - r_lo);
            const uint32_t e = visible_end(kpos, s0, s1, int64_t((uint64_t(xhi) << 32) | xlo), lane);
            if (row == r) e_h = e;
          }
        }
        if (!hvalid) e_h = s0;
      }
      uint32_t lo = hvalid ? e_h : 0xffffffffu, hi = e_h;
#define KVB_ROW_RED(N)                                                                                 \
  {                                                                                                    \
    const uint32_t o1 = uint32_t(__builtin_amdgcn_update_dpp(0, int(lo), 0x120 + N, 0xF, 0xF, false)); \
    const uint32_t o2 = uint32_t(__builtin_amdgcn_update_dpp(0, int(hi), 0x120 + N, 0xF, 0xF, false)); \
    lo = o1 < lo ? o1 : lo;                                                                            \
    hi = o2 > hi ? o2 : hi;                                                                            \
  }
      KVB_ROW_RED(8) KVB_ROW_RED(4) KVB_ROW_RED(2) KVB_ROW_RED(1)
#undef KVB_ROW_RED
      e_min = __builtin_amdgcn_readfirstlane(lo);
      e_max = __builtin_amdgcn_readfirstlane(hi);

      // Q digits (B of QK): digit dg of the 23-bit integer 2^kq * q in qd[dg].
      float amax = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(qv[s][i]));
      amax = rows_max(amax);
      int kq = 0;
      if (amax > 0.f) {
        kq = 22 - __builtin_amdgcn_frexp_expf(amax);  // |2^kq q| < 2^22: top digit in [-64, 64]
        kq = kq < -100 ? -100 : (kq > 100 ? 100 : kq);
      }
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        uint32_t w[3][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[0][i] = w[1][i] = w[2][i] = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          int qi = int(__builtin_rintf(__builtin_amdgcn_ldexpf(qv[s][i], kq)));  // |qi| <= 2^22
          if (a.scale < 0.f) qi = -qi;  // scores scale by |scale| (see cs)
          const int lo8 = __builtin_amdgcn_sbfe(qi, 0, 8);
          const int r1 = (qi - lo8) >> 8;
          const int mid8 = __builtin_amdgcn_sbfe(r1, 0, 8);
          const int hi8 = (r1 - mid8) >> 8;
          w[0][i / 4] |= (uint32_t(hi8) & 0xffu) << (8 * (i % 4));
          w[1][i / 4] |= (uint32_t(mid8) & 0xffu) << (8 * (i % 4));
          w[2][i / 4] |= (uint32_t(lo8) & 0xffu) << (8 * (i % 4));
        }
#pragma unroll
        for (int dg = 0; dg < 3; ++dg) qd[dg][s] = i32x4{int(w[dg][0]), int(w[dg][1]), int(w[dg][2]), int(w[dg][3])};
      }
      // Score factor in log2 units, > 0: the sign of the scale went into the
      // Q digits, and a zero factor becomes the smallest normal float (every
      // score then rounds to 0 in 2^(cs * y - mu) while masked y = -inf
      // stays -inf instead of 0 * inf).
      cs = __builtin_amdgcn_ldexpf(fabsf(a.scale), -kq) * kLog2e;
      cs = cs >= 1.17549435e-38f ? cs : 1.17549435e-38f;
    }
    const uint32_t nvis = has && e_max > s0 ? (e_max - 1u) / kTileTokens + 1u - k_first : 0u;  // tiles

    float m_run = neg_inf(), l_run = 0.f;  // per lane: head-row h's running max (log2) and partial sum
    f32x4 acc[MB];  // lane (h, g): dims 16mb + 4g + e
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // This block's partial of split `split` from the registers (lane (h, g):
    // dims 16mb + 4g + e), then a fresh state for the next split.
    auto write_partial = [&](uint32_t split) __attribute__((always_inline)) {
      if (!has) return;
      const float l_h = rows_sum(l_run);
      if (hvalid) {
        float* const dst = scratch + ((size_t(row) * a.q_heads + head) * a.splits + split) * W;
        if (g == 0) {
          dst[0] = m_run * kLn2;
          dst[1] = l_h;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[2 + 16 * mb + 4 * g + e] = acc[mb][e];
      }
      m_run = neg_inf();
      l_run = 0.f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // Splits of this work-group one after another (one split, or spw whole
    // splits of pps phases each); the DMA pipeline runs across them.
    const uint32_t ppsplit = spw > 1u ? pps : nphase;
    for (uint32_t sp = sp0; sp < sp1; ++sp) {
    const uint32_t p_lo = (sp - sp0) * ppsplit;
    const uint32_t p_hi = p_lo + ppsplit < nphase ? p_lo + ppsplit : nphase;
    for (uint32_t p = p_lo; p < p_hi; ++p) {
      wait_next(p);
      __syncthreads();  // phase p landed; every wave is done with phase p - 1 (slot (p + 1) & 1)
      if (idle_dma && p + 1u < nphase) issue(p + 1u);  // the DMA wave, while the others compute
      const uint32_t tp = p * CT;  // first tile of the phase (split-relative)
      if (tp < nvis) {
        // LDS addresses of the slot (tile j adds j * kBufBytes as an immediate).
        const uint32_t pb = lds_base + (p & 1u) * kSlot;
        uint32_t ka[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) ka[s] = pb + koff[s];
        const uint32_t va = pb + voff, sa = pb + soff, vma = pb + vmoff;

        // ---- QK: scores of the phase's tiles, lane (h, g): tokens 16g + 4mb + e,
        // as y = (integer dot) * k_scale; the score in log2 units is cs * y
        // (cs > 0, so maxima of y are maxima of scores).
        float sc[CT][16];
        float mx = neg_inf();
        // The phase's CT x 4 QK M-blocks (tile j = b / 4, block mb = b % 4) in
        // one software pipeline: block b's reads went out two blocks earlier
        // (three register sets), block b's MFMAs are interleaved with block
        // b - 1's scores.  Every tile runs (a tile past the visible range is
        // fully masked), so the pipeline has no branch.
        constexpr uint32_t NB = CT * 4u;
        constexpr uint32_t kRd = KS + 1u;  // LDS reads per block
        u32x4_t kr[3][KS], ksr[3];
        auto read_k = [&](auto bc) __attribute__((always_inline)) {
          constexpr uint32_t bb = decltype(bc)::value;
          constexpr uint32_t TB = (bb / 4u) * G::kBufBytes, mb = bb % 4u;
          ds_issue_kblock<TB + 4u * mb * D, TB + 16u * mb>(ka, sa, kr[bb % 3u], ksr[bb % 3u]);
        };
        i32x4 cq[2][3];
        u32x4_t ksc[2];  // k-scales of blocks b (set b & 1), copied before their registers are refilled
        // Masking per phase, outside the pipeline (a branch inside it would
        // split the scheduling regions that interleave MFMAs and VALU): a
        // phase whose tiles every head-row of the block sees in full runs
        // unmasked.
        uint32_t vis[CT];
#pragma unroll
        for (int j = 0; j < CT; ++j) {
          const uint32_t t0 = (k_first + tp + j) * kTileTokens;
          vis[j] = tp + j < nvis ? (e_h > t0 ? (e_h - t0 < kTileTokens ? e_h - t0 : kTileTokens) : 0u) : 0u;
        }
        const bool phase_full = tp + CT <= nvis && (k_first + tp + CT) * kTileTokens <= e_min;
        auto qk = [&](auto maskc) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(maskc)::value;
        auto scores = [&](auto bc) __attribute__((always_inline)) {
          constexpr uint32_t bb = decltype(bc)::value;
          constexpr uint32_t j = bb / 4u, mb = bb % 4u;
          const i32x4(&c)[3] = cq[bb & 1u];
          const u32x4_t ksm = ksc[bb & 1u];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int hi2 = c[0][e] * 256 + c[1][e];  // |.| < 2^29
            float s2 = fmaf(float(hi2), 256.f, float(c[2][e])) * __uint_as_float(ksm[e]);
            if constexpr (MASK) s2 = 16u * g + 4u * mb + e < vis[j] ? s2 : neg_inf();
            sc[j][4 * mb + e] = s2;
            mx = fmaxf(mx, s2);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) pin(sc[j][4 * mb + e]);
        };
        read_k(std::integral_constant<uint32_t, 0>{});
        read_k(std::integral_constant<uint32_t, 1>{});
        static_for<0, NB>([&](auto bc) __attribute__((always_inline)) {
          constexpr uint32_t bb = decltype(bc)::value;
          // block bb's reads done; block bb + 1's may still be in flight
          if constexpr (bb + 1 < NB) wait_lgkm<kRd>();
          else wait_lgkm<0>();
#pragma unroll
          for (int st = 0; st < KS; ++st) pin(kr[bb % 3u][st]);
          pin(ksr[bb % 3u]);
          ksc[bb & 1u] = ksr[bb % 3u];
          if constexpr (bb + 2 < NB) read_k(std::integral_constant<uint32_t, bb + 2>{});
          i32x4(&c)[3] = cq[bb & 1u];
#pragma unroll
          for (int dg = 0; dg < 3; ++dg) c[dg] = i32x4{0, 0, 0, 0};
#pragma unroll
          for (int st = 0; st < KS; ++st) {
            const u32x4_t& k4 = kr[bb % 3u][st];
            const i32x4 av = {int(k4[0]), int(k4[1]), int(k4[2]), int(k4[3])};
#pragma unroll
            for (int dg = 0; dg < 3; ++dg) c[dg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, qd[dg][st], c[dg], 0, 0, 0);
          }
          if constexpr (bb > 0) {
            scores(std::integral_constant<uint32_t, bb - 1>{});
#pragma unroll
            for (int i = 0; i < 3 * KS; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // then up to three VALU
            }
          }
        });
        scores(std::integral_constant<uint32_t, NB - 1>{});
        };
        if (phase_full) qk(std::false_type{});
        else qk(std::true_type{});
        pin(mx);

        // ---- v-scales of the phase, running maximum, weight exponent kp
        float vm = 0.f;
        static_for<0, CT>([&](auto jc) __attribute__((always_inline)) {
          constexpr uint32_t j = decltype(jc)::value;
          constexpr uint32_t TB = j * G::kBufBytes;
          if (tp + j >= nvis) return;
          const float v = __uint_as_float(ds_read4_sync<TB>(vma));
          const uint32_t t0 = (k_first + tp + j) * kTileTokens;
          vm = t0 + lane < e_max ? fmaxf(vm, fabsf(v)) : vm;
        });
        const float m_new = fmaxf(m_run, rows_max(mx) * cs);
        const float vmax = wave_max(vm);
        int kp = 0;
        if (vmax > 0.f) {
          kp = 21 - __builtin_amdgcn_frexp_expf(vmax * kVmaxMargin);
          kp = kp < -100 ? -100 : (kp > 100 ? 100 : kp);
        }
        const float f = m_run == neg_inf() ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb] *= f;  // exact where f == 1
        const float mu = (m_new == neg_inf() ? 0.f : m_new) - float(kp);  // 2^(s - mu) = w * 2^kp
        m_run = m_new;

        // ---- weights as three 7-bit digits (B of PV), k-position = token 16g + 4mb + e.
        // Slots past the block's last visible token (and every slot of a tile
        // past the visible range) get a zero v-scale, so stale LDS contents
        // cannot reach the digits; the masking is chosen per phase.
        i32x4 bd[CT][3];
        float lw = 0.f;
        const bool phase_vfull = tp + CT <= nvis && (k_first + tp + CT) * kTileTokens <= e_max;
        auto weights = [&](auto maskc) __attribute__((always_inline)) {
          constexpr bool MASK = decltype(maskc)::value;
          static_for<0, CT>([&](auto jc) __attribute__((always_inline)) {
            constexpr uint32_t j = decltype(jc)::value;
            constexpr uint32_t TB = j * G::kBufBytes;
            const uint32_t t0 = (k_first + tp + j) * kTileTokens;
            const uint32_t vlim = tp + j < nvis && e_max > t0 ? (e_max - t0 < kTileTokens ? e_max - t0 : kTileTokens) : 0u;
            u32x4_t vsr[4];  // v-scales of tokens 16g .. 16g + 15
            ds_read16x4<TB + 256u, TB + 272u, TB + 288u, TB + 304u>(sa, vsr[0], vsr[1], vsr[2], vsr[3]);
            uint32_t bw[3][4];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
              bw[0][mb] = bw[1][mb] = bw[2][mb] = 0u;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float w = __builtin_amdgcn_exp2f(fmaf(sc[j][4 * mb + e], cs, -mu));  // w * 2^kp
                lw += w;
                float vsl = __uint_as_float(vsr[mb][e]);
                if constexpr (MASK) vsl = 16u * g + 4u * mb + e < vlim ? vsl : 0.f;
                // p = w * v_scale rounded to an integer (0 <= p < 2^21) in one fma:
                // 1.5 * 2^23 + p lies in [2^23, 2^24), where the float's ulp is
                // 1, so its low 22 bits are p mod 2^22 (two's complement), and
                // bits 0-6, 7-13 and 14-21 are the three digits of p.
                const uint32_t pb = __float_as_uint(fmaf(w, vsl, 12582912.f));
                bw[0][mb] |= ((pb >> 14) & 0xffu) << (8 * e);
                bw[1][mb] |= ((pb >> 7) & 0x7fu) << (8 * e);
                bw[2][mb] |= (pb & 0x7fu) << (8 * e);
              }
            }
#pragma unroll
            for (int dg = 0; dg < 3; ++dg)
              bd[j][dg] = i32x4{int(bw[dg][0]), int(bw[dg][1]), int(bw[dg][2]), int(bw[dg][3])};
          });
        };
        if (phase_vfull) weights(std::false_type{});
        else weights(std::true_type{});
        const float inv = __builtin_amdgcn_ldexpf(1.f, -kp);
        l_run = fmaf(lw, inv, l_run * f);

        // ---- PV per 16-dim block: A = V[16mb + n][16g .. 16g + 15], one read per tile.
        // Software-pipelined: the reads of block mb + 2 go out while block
        // mb's MFMAs run (three register sets, so a set is refilled two
        // blocks after its MFMAs were issued), block mb's MFMAs are
        // interleaved with block mb - 1's fold into fp32.  Tiles past the
        // visible range have zero weight digits, so every tile runs without
        // a branch.
        u32x4_t vr[3][CT];
        auto read_v = [&](auto mc) __attribute__((always_inline)) {
          constexpr uint32_t mb = decltype(mc)::value;
          u32x4_t(&r)[CT] = vr[mb % 3u];
          if constexpr (CT == 2) {
            ds_issue16x2<1024u * mb, G::kBufBytes + 1024u * mb>(va, r[0], r[1]);
          } else {
            ds_issue16x4<1024u * mb, G::kBufBytes + 1024u * mb, 2u * G::kBufBytes + 1024u * mb,
                         3u * G::kBufBytes + 1024u * mb>(va, r[0], r[1], r[2], r[3]);
          }
        };
        read_v(std::integral_constant<uint32_t, 0>{});
        if constexpr (MB > 1) read_v(std::integral_constant<uint32_t, 1>{});
        i32x4 cv[2][3];
        auto fold = [&](auto mc) __attribute__((always_inline)) {
          constexpr uint32_t mb = decltype(mc)::value;
          const i32x4(&c)[3] = cv[mb & 1u];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int hi2 = c[0][e] * 128 + c[1][e];  // |.| < 2^29
            acc[mb][e] = fmaf(fmaf(float(hi2), 128.f, float(c[2][e])), inv, acc[mb][e]);
          }
        };
        static_for<0, MB>([&](auto mc) __attribute__((always_inline)) {
          constexpr uint32_t mb = decltype(mc)::value;
          // block mb's reads done; block mb + 1's may still be in flight
          if constexpr (mb + 1 < MB) wait_lgkm<CT>();
          else wait_lgkm<0>();
          u32x4_t(&r)[CT] = vr[mb % 3u];
#pragma unroll
          for (int j = 0; j < CT; ++j) pin(r[j]);
          if constexpr (mb + 2 < MB) read_v(std::integral_constant<uint32_t, mb + 2>{});
          i32x4(&c)[3] = cv[mb & 1u];
#pragma unroll
          for (int dg = 0; dg < 3; ++dg) c[dg] = i32x4{0, 0, 0, 0};
#pragma unroll
          for (int j = 0; j < CT; ++j) {
            const i32x4 av = {int(r[j][0]), int(r[j][1]), int(r[j][2]), int(r[j][3])};
#pragma unroll
            for (int dg = 0; dg < 3; ++dg) c[dg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bd[j][dg], c[dg], 0, 0, 0);
          }
          if constexpr (mb > 0) {
            fold(std::integral_constant<uint32_t, mb - 1>{});
            pin(acc[mb - 1]);
#pragma unroll
            for (int i = 0; i < 3 * CT; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // then up to four VALU
            }
          }
        });
        fold(std::integral_constant<uint32_t, MB - 1>{});
        pin(acc[MB - 1]);
      }
      if (!idle_dma) {
        __syncthreads();  // slot p & 1 is free
        if (p + 2u < nphase) issue(p + 2u);
      }
    }
    write_partial(sp);  // (an empty range leaves the empty partial)
    }
  }
}

// ---- Wave-specialized form: one round of at most three head-row blocks at
// dim 256 (the dense rows-8 / group-6 geometry, 48 head-rows).
//
// Eight waves per work-group: QK waves 0-2 (head-row block b = wave), the DMA
// wave 3, and PV waves 4-7.  The four-wave kernel above runs one wave per
// SIMD, and only three of them compute at 48 head-rows; a wave then stalls
// on every dependent MFMA -> VALU -> LDS step of its own.  Here each block's
// scores and weights run on a QK wave, and the PV products and fp32 folds of
// all blocks are spread over four PV waves (wave 4 + j takes dims 64j ..
// 64j + 63 of every block, whose V rows it reads once for all blocks), so
// every SIMD computes and each holds two waves that fill each other's
// stalls (waves w and w + 4 share a SIMD).  Step s (one 64-token tile; the
// split's tiles run through a four-slot ring of tile images):
//  - DMA: tile s landed (the wave's loads in flight are tiles s and s + 1),
//    barrier, then tile s + 2 goes into slot (s + 2) % 4 (two tiles of lead;
//    that slot held tile s - 2, whose last reader, PV step s - 1, is behind
//    the barrier);
//  - QK wave: scores of tile s, running maximum, the weights' three int8
//    digits in base 256 (B of PV; the two low ones balanced) into its
//    exchange slot s & 1 with the rescale factor f of each head-row and 2^-kp;
//  - PV waves: tile s - 1 from the other exchange slots, acc = acc * f +
//    (V . P) * 2^-kp per block.
// One barrier per step.  The arithmetic is the four-wave kernel's per
// 64-token step instead of per 128-token phase (running maximum, kp and the
// digit fold per tile), with the same integer weights p split into
// byte-aligned digits, so the partials agree with it to rounding.  The QK
// wave owns m and l of its block's head-rows and the PV waves the
// numerators; each writes its part of a split's partial after the split's
// last tile.
constexpr uint32_t kPcBlocks = 3;
constexpr uint32_t kPcWaves = 8;
constexpr uint32_t kPcSlots = 4;
constexpr float kPcHeadroom = 2.f;  // log2 units of maximum growth an epoch absorbs

template <int D, bool PT>
__global__ __launch_bounds__(64 * kPcWaves) void split_i8_rows_pc_kernel(
    SplitArgs a, const float* __restrict__ q, const int64_t* __restrict__ qpos,
    const int64_t* __restrict__ kpos, const uint32_t* __restrict__ table,
    const int8_t* __restrict__ kdata, const int8_t* __restrict__ vdata,
    const float* __restrict__ kscale, const float* __restrict__ vscale, float* __restrict__ scratch, uint32_t spw) {
  using G = Geo<D>;
  constexpr int KS = D / 64;  // K-steps of QK
  constexpr int MB = D / 16;  // 16-dim blocks of PV
  constexpr uint32_t W = D + 2;
  constexpr uint32_t kImg = G::kBufBytes;
  constexpr uint32_t kXBytes = 3u * 1024u;  // one block's weight digits of one tile: [digit][lane] x 16 bytes
  constexpr uint32_t kXBase = kPcSlots * kImg;
  static_assert(kXBase + kPcBlocks * 2u * kXBytes <= 160u * 1024u - 1024u, "LDS");
  __shared__ __attribute__((aligned(16))) uint8_t smem[kXBase + kPcBlocks * 2u * kXBytes];
  // [block][exchange slot]: a tile's epoch fold (f of head-rows 0-15, 2^-kp
  // of the epoch ending, flag) and a split's end (e of head-rows 0-15 at
  // 18-33, 2^-kp of its last epoch at 34)
  __shared__ float fx_s[kPcBlocks][2][36];
  __shared__ uint32_t nvis_s[kPcBlocks];
  __shared__ uint32_t rh_s[kPcBlocks * 16u];  // row * q_heads + head of each head-row (partial offsets)
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t n = lane & 15u, g = lane >> 4;
  const uint32_t kv = blockIdx.y;
  const uint32_t head_rows = a.rows * a.group, hblocks = (head_rows + 15u) / 16u;  // <= 3 (host-checked)
  const bool dma = wave == 3u;
  const bool qkw = wave < 3u;
  const uint32_t blk = wave;                // QK waves: their head-row block
  const bool has = qkw && blk < hblocks;    // wave-uniform

  // Splits [sp0, sp1) of this work-group, tokens [s0, s1) (as the four-wave
  // kernel; a split is a whole number of tiles).
  const uint32_t sp0 = blockIdx.x * spw;
  const uint32_t sp1 = sp0 + spw < a.splits ? sp0 + spw : a.splits;
  const uint32_t tps = a.split_tokens / kTileTokens;  // tiles per split
  const uint64_t s0_64 = uint64_t(a.begin) + uint64_t(sp0) * a.split_tokens;
  const uint32_t s0 = s0_64 < a.end ? uint32_t(s0_64) : a.end;
  const uint64_t s1_64 = uint64_t(a.begin) + uint64_t(sp1) * a.split_tokens;
  const uint32_t s1 = s1_64 < a.end ? uint32_t(s1_64) : a.end;
  const uint32_t k_first = s0 / kTileTokens;
  const uint32_t ntiles = s1 > s0 ? (s1 - 1u) / kTileTokens + 1u - k_first : 0u;

  // ---- DMA wave.
  Ctx c;
  PtCtx pc;
  if (dma && ntiles > 0) {
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
    const uint32_t lp = c.lp_lo + lane;
    c.ptab = lp <= c.lp_hi ? table[lp] : 0u;
    if constexpr (PT) {
      const uint32_t kv_bytes = a.pages * a.kv_heads * a.page_tokens * uint32_t(D);
      const uint32_t sc_bytes = a.pages * a.kv_heads * a.page_tokens * 4u;
      pt_init<D>(pc, kdata, vdata, kscale, vscale, kv_bytes, sc_bytes, a.page_tokens, lane);
    }
  }
  auto issue = [&](uint32_t t) __attribute__((always_inline)) {  // tile t of the range into slot t % 4
    uint8_t* const buf = smem + (t % kPcSlots) * kImg;
    const uint32_t k = k_first + t;
    dma_group_mark();
    if constexpr (PT) {
      const uint32_t lp = k * kTileTokens / a.page_tokens;
      const uint32_t rel = lp - c.lp_lo;
      uint32_t phys = rel < 64u ? __builtin_amdgcn_readlane(c.ptab, rel) : table[lp];
      phys = phys < a.pages ? phys : a.pages - 1u;
      pt_issue<D>(pc, phys * a.kv_heads + kv, k * kTileTokens - lp * a.page_tokens, a.page_tokens, buf);
    } else {
      part_issue<D, 1>(c, k, buf, 0u);
    }
  };

  // Per-lane LDS offsets inside a tile image (as the four-wave kernel).
  const uint32_t lds_base = lds_addr(smem);
  uint32_t koff[KS];
  {
    const uint32_t r0 = 16u * (n >> 2) + (n & 3u);
#pragma unroll
    for (int s = 0; s < KS; ++s) koff[s] = r0 * D + 16u * ((4u * s + g) ^ swz_k<D>(r0));
  }
  const uint32_t voff = G::kKBytes + 64u * n + 16u * (g ^ swz_v(n));
  const uint32_t soff = G::kKBytes + G::kVBytes + 64u * g;

  const uint32_t hr = blk * 16u + n;
  const bool hvalid = has && hr < head_rows;
  const uint32_t row = hvalid ? hr / a.group : 0u;
  const uint32_t head = kv * a.group + (hvalid ? hr % a.group : 0u);
  auto partial = [&](uint32_t sp) __attribute__((always_inline)) {
    return scratch + ((size_t(row) * a.q_heads + head) * a.splits + sp) * W;
  };

  // The three roles run their own step loops (ntiles + 1 barriers each), so
  // each role's registers live only in its own loop.
  if (dma) {
    // Tile s landed: the wave's loads are tiles s and s + 1, each exactly
    // kLoadsPerTile vector-memory instructions when the page-table window
    // covers the range (no table load inside an issue); else wait for all.
    // The emitted count per tile is checked on the device assembly
    // (check_vm_waits.py: the wait leaves only the newest tile in flight).
    static_assert(G::kLoadsPerTile == 34u, "the tile's DMA instruction count");
    const bool window = ntiles > 0u && c.lp_hi - c.lp_lo < 64u;
    // The page-table window comes from a vector load; consume it here, on
    // every path (the first issue needs it anyway), so that no wait the
    // compiler derives from it lands inside the step loop.
    asm volatile("" : "+v"(c.ptab));
    // The QK waves' own loads (Q, positions) go out first, chip-wide ahead
    // of the tiles, so their round trip does not queue behind the DMA (a
    // bare s_barrier: no wait for those loads).
    bare_barrier();
    if (ntiles > 0u) issue(0u);
    if (ntiles > 1u) issue(1u);
    // Tiles 0 and 1 both land before the first step, so tile 2 goes out
    // only after them: issuing it as soon as tile 0 has landed measured
    // slower (1,024-token splits at the dense geometry: 44.3 against 41.0 us
    // per call), the chip-wide start then having a third tile per work-group
    // in flight.
    wait_vm<0>();
    for (uint32_t s = 0; s <= ntiles; ++s) {
      if (s < ntiles) {
        if (s + 1u < ntiles && window) wait_vm_keep<G::kLoadsPerTile, 1>();
        else wait_vm<0>();
      }
      // Tile s visible to all; every wave is done with step s - 1.  A bare
      // s_barrier: this wave's only memory operations are the tile loads,
      // which the wait above covers, and __syncthreads's release fence
      // would add a wait for every load in flight (tile s + 1 too).
      bare_barrier();
      if (s + 2u < ntiles) issue(s + 2u);
    }
    return;
  }
  // Splits of this work-group past its last tile (a range that ends early,
  // or no tile at all) get empty partials.
  const uint32_t sp_e = ntiles > 0u ? sp0 + (ntiles - 1u) / tps + 1u : sp0;
  if (qkw) {
    // ---- QK waves: visibility and Q digits of the block.
    uint32_t e_h = s0, e_min = s0, e_max = s0, nvis = 0;
    float cs = 0.f;
    i32x4 qd[3][KS];
    if (!has) bare_barrier();  // the prologue barrier (see the DMA wave)
    if (has) {
      float qv[KS][16];
      int64_t klast = 0, qpos_l = INT64_MAX;  // lane i: query position of row r_lo + i
      const uint32_t r_lo = blk * 16u / a.group;
      const uint32_t r_hi = (blk * 16u + 15u < head_rows ? blk * 16u + 15u : head_rows - 1u) / a.group;
      if (hvalid) {
        const float* qp = q + (size_t(row) * a.q_heads + head) * D + 16u * g;
  #pragma unroll
        for (int s = 0; s < KS; ++s)
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float4 x = reinterpret_cast<const float4*>(qp + 64 * s)[j];
            qv[s][4 * j] = x.x;
            qv[s][4 * j + 1] = x.y;
            qv[s][4 * j + 2] = x.z;
            qv[s][4 * j + 3] = x.w;
          }
      } else {
  #pragma unroll
        for (int s = 0; s < KS; ++s)
  #pragma unroll
          for (int i = 0; i < 16; ++i) qv[s][i] = 0.f;
      }
      if (s1 > s0) {
        klast = kpos[s1 - 1u];
        if (lane <= r_hi - r_lo) qpos_l = qpos[r_lo + lane];  // at most 16 rows per block
      }
      bare_barrier();  // the loads above are out: the DMA wave may start
      asm volatile("" : "+v"(klast), "+v"(qpos_l));  // their uses (and waits) stay after the barrier
      if (s1 > s0) {
        if (__ballot(klast > qpos_l) == 0) {  // every row of the block sees the whole range
          e_h = s1;
        } else {
          for (uint32_t r = r_lo; r <= r_hi; ++r) {
            const uint64_t xb = uint64_t(qpos_l);
            const uint32_t xlo = __builtin_amdgcn_readlane(uint32_t(xb), r - r_lo);
            const uint32_t xhi = __builtin_amdgcn_readlane(uint32_t(xb >> 32), r - r_lo);
            const uint32_t e = visible_end(kpos, s0, s1, int64_t((uint64_t(xhi) << 32) | xlo), lane);
            if (row == r) e_h = e;
          }
        }
        if (!hvalid) e_h = s0;
      }
      uint32_t lo = hvalid ? e_h : 0xffffffffu, hi = e_h;
  #define KVB_ROW_RED(N)                                                                                 \
    {                                                                                                    \
      const uint32_t o1 = uint32_t(__builtin_amdgcn_update_dpp(0, int(lo), 0x120 + N, 0xF, 0xF, false)); \
      const uint32_t o2 = uint32_t(__builtin_amdgcn_update_dpp(0, int(hi), 0x120 + N, 0xF, 0xF, false)); \
      lo = o1 < lo ? o1 : lo;                                                                            \
      hi = o2 > hi ? o2 : hi;                                                                            \
    }
      KVB_ROW_RED(8) KVB_ROW_RED(4) KVB_ROW_RED(2) KVB_ROW_RED(1)
  #undef KVB_ROW_RED
      e_min = __builtin_amdgcn_readfirstlane(lo);
      e_max = __builtin_amdgcn_readfirstlane(hi);
      float amax = 0.f;
  #pragma unroll
      for (int s = 0; s < KS; ++s)
  #pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(qv[s][i]));
      amax = rows_max(amax);
      int kq = 0;
      if (amax > 0.f) {
        kq = 22 - __builtin_amdgcn_frexp_expf(amax);  // |2^kq q| < 2^22: top digit in [-64, 64]
        kq = kq < -100 ? -100 : (kq > 100 ? 100 : kq);
      }
  #pragma unroll
      for (int s = 0; s < KS; ++s) {
        uint32_t w[3][4];
  #pragma unroll
        for (int i = 0; i < 4; ++i) w[0][i] = w[1][i] = w[2][i] = 0u;
  #pragma unroll
        for (int i = 0; i < 16; ++i) {
          int qi = int(__builtin_rintf(__builtin_amdgcn_ldexpf(qv[s][i], kq)));  // |qi| <= 2^22
          if (a.scale < 0.f) qi = -qi;  // scores scale by |scale| (see cs)
          const int lo8 = __builtin_amdgcn_sbfe(qi, 0, 8);
          const int r1 = (qi - lo8) >> 8;
          const int mid8 = __builtin_amdgcn_sbfe(r1, 0, 8);
          const int hi8 = (r1 - mid8) >> 8;
          w[0][i / 4] |= (uint32_t(hi8) & 0xffu) << (8 * (i % 4));
          w[1][i / 4] |= (uint32_t(mid8) & 0xffu) << (8 * (i % 4));
          w[2][i / 4] |= (uint32_t(lo8) & 0xffu) << (8 * (i % 4));
        }
  #pragma unroll
        for (int dg = 0; dg < 3; ++dg) qd[dg][s] = i32x4{int(w[dg][0]), int(w[dg][1]), int(w[dg][2]), int(w[dg][3])};
      }
      cs = __builtin_amdgcn_ldexpf(fabsf(a.scale), -kq) * kLog2e;
      cs = cs >= 1.17549435e-38f ? cs : 1.17549435e-38f;
      nvis = e_max > s0 ? (e_max - 1u) / kTileTokens + 1u - k_first : 0u;
      if (lane == 0) nvis_s[blk] = nvis;
      if (g == 0) rh_s[hr] = row * a.q_heads + head;
    }

    float m_run = neg_inf(), l_run = 0.f;  // head-row h's running max (log2) and partial sum
    // Scale epochs: the weights of all tiles of an epoch use one reference R
    // per head-row (the running maximum at the epoch's first tile plus
    // kPcHeadroom) and one v-scale exponent kp, so the PV waves add the
    // epoch's int32 digit sums in the MFMA accumulators and fold them into
    // fp32 only when it ends.  A tile starts a new epoch when a head-row's
    // maximum passes its R, when its largest v-scale leaves [vlo, vcap) (a
    // quarter of the epoch's first, and the largest that keeps every weight
    // integer below 2^23 - 2^16), or after 1,024 tiles (the int32 range of
    // the digit sums).  l_run is in units of 2^(s - R).
    float R = neg_inf();
    int kp = 0;
    float vcap = 0.f, vlo = 0.f;
    uint32_t epoch_tiles = 0;
    bool epoch = false;
    // QK wave: tile t -> exchange slot t & 1.
    auto qk_tile = [&](uint32_t t) __attribute__((always_inline)) {
      const uint32_t pb = lds_base + (t % kPcSlots) * kImg;
      uint32_t ka[KS];
  #pragma unroll
      for (int s = 0; s < KS; ++s) ka[s] = pb + koff[s];
      const uint32_t sa = pb + soff;
      const uint32_t t0 = (k_first + t) * kTileTokens;
      float sc[16];
      float mx = neg_inf();
      constexpr uint32_t NB = 4u;        // QK M-blocks of a tile
      constexpr uint32_t kRd = KS + 1u;  // LDS reads per block
      u32x4_t kr[3][KS], ksr[3];
      auto read_k = [&](auto bc) __attribute__((always_inline)) {
        constexpr uint32_t mb = decltype(bc)::value;
        ds_issue_kblock<4u * mb * D, 16u * mb>(ka, sa, kr[mb % 3u], ksr[mb % 3u]);
      };
      i32x4 cq[2][3];
      u32x4_t ksc[2];
      const uint32_t vis = e_h > t0 ? (e_h - t0 < kTileTokens ? e_h - t0 : kTileTokens) : 0u;
      const bool full = t0 + kTileTokens <= e_min;
      auto qk = [&](auto maskc) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(maskc)::value;
        auto scores = [&](auto bc) __attribute__((always_inline)) {
          constexpr uint32_t mb = decltype(bc)::value;
          const i32x4(&cc)[3] = cq[mb & 1u];
          const u32x4_t ksm = ksc[mb & 1u];
  #pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int hi2 = cc[0][e] * 256 + cc[1][e];  // |.| < 2^29
            float s2 = fmaf(float(hi2), 256.f, float(cc[2][e])) * __uint_as_float(ksm[e]);
            if constexpr (MASK) s2 = 16u * g + 4u * mb + e < vis ? s2 : neg_inf();
            sc[4 * mb + e] = s2;
            mx = fmaxf(mx, s2);
          }
  #pragma unroll
          for (int e = 0; e < 4; ++e) pin(sc[4 * mb + e]);
        };
        read_k(std::integral_constant<uint32_t, 0>{});
        read_k(std::integral_constant<uint32_t, 1>{});
        static_for<0, NB>([&](auto bc) __attribute__((always_inline)) {
          constexpr uint32_t mb = decltype(bc)::value;
          if constexpr (mb + 1 < NB) wait_lgkm<kRd>();
          else wait_lgkm<0>();
  #pragma unroll
          for (int st = 0; st < KS; ++st) pin(kr[mb % 3u][st]);
          pin(ksr[mb % 3u]);
          ksc[mb & 1u] = ksr[mb % 3u];
          if constexpr (mb + 2 < NB) read_k(std::integral_constant<uint32_t, mb + 2>{});
          i32x4(&cc)[3] = cq[mb & 1u];
  #pragma unroll
          for (int dg = 0; dg < 3; ++dg) cc[dg] = i32x4{0, 0, 0, 0};
  #pragma unroll
          for (int st = 0; st < KS; ++st) {
            const u32x4_t& k4 = kr[mb % 3u][st];
            const i32x4 av = {int(k4[0]), int(k4[1]), int(k4[2]), int(k4[3])};
  #pragma unroll
            for (int dg = 0; dg < 3; ++dg)
              cc[dg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, qd[dg][st], cc[dg], 0, 0, 0);
          }
          if constexpr (mb > 0) {
            scores(std::integral_constant<uint32_t, mb - 1>{});
  #pragma unroll
            for (int i = 0; i < 3 * KS; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // then up to three VALU
            }
          }
        });
        scores(std::integral_constant<uint32_t, NB - 1>{});
      };
      if (full) qk(std::false_type{});
      else qk(std::true_type{});
      pin(mx);

      // v-scales of tokens 16g .. 16g + 15 (zero past the block's last
      // visible token, so stale LDS contents cannot reach the digits).
      const uint32_t vlim = e_max > t0 ? (e_max - t0 < kTileTokens ? e_max - t0 : kTileTokens) : 0u;
      float vsl[16];
      {
        u32x4_t vsr[4];
        ds_read16x4<256u, 272u, 288u, 304u>(sa, vsr[0], vsr[1], vsr[2], vsr[3]);
  #pragma unroll
        for (int i = 0; i < 16; ++i) vsl[i] = __uint_as_float(vsr[i / 4][i % 4]);
        if (t0 + kTileTokens > e_max) {
  #pragma unroll
          for (int i = 0; i < 16; ++i) vsl[i] = 16u * g + i < vlim ? vsl[i] : 0.f;
        }
      }
      float vloc = 0.f;
  #pragma unroll
      for (int i = 0; i < 16; ++i) vloc = fmaxf(vloc, fabsf(vsl[i]));

      // Weights as three base-256 int8 digits (k-position = token 16g + 4mb + e).
      i32x4 bd[3];
      float lw = 0.f;
      auto weights = [&](float mu) __attribute__((always_inline)) {  // 2^(s - mu) = w * 2^kp
        lw = 0.f;
        uint32_t bw[3][4];
  #pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          uint32_t x[4];
  #pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float w = __builtin_amdgcn_exp2f(fmaf(sc[4 * mb + e], cs, -mu));  // w * 2^kp
            lw += w;
            // p = w * v_scale rounded to an integer (0 <= p < 2^23 - 2^16): t =
            // 2^23 + 0x8080 + p lies in [2^23, 2^24), where the float's ulp is
            // 1, so its mantissa bits are q = p + 0x8080 and p = (q2 << 16) +
            // ((q1 - 128) << 8) + (q0 - 128) with q's bytes q2 (0 .. 127) and
            // q1, q0: the digits are byte 2 and bytes 1, 0 xor 0x80 (int8).
            x[e] = __float_as_uint(fmaf(w, vsl[4 * mb + e], 8421504.f));
          }
          // 4 x 3 byte transpose: digit k of the four tokens into one word.
          const uint32_t lo01 = __builtin_amdgcn_perm(x[1], x[0], 0x05010400u);  // x0.b0 x1.b0 x0.b1 x1.b1
          const uint32_t lo23 = __builtin_amdgcn_perm(x[3], x[2], 0x05010400u);
          const uint32_t hi01 = __builtin_amdgcn_perm(x[1], x[0], 0x0c0c0602u);  // x0.b2 x1.b2 0 0
          const uint32_t hi23 = __builtin_amdgcn_perm(x[3], x[2], 0x06020c0cu);  // 0 0 x2.b2 x3.b2
          bw[0][mb] = hi01 | hi23;
          bw[1][mb] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
          bw[2][mb] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
        }
  #pragma unroll
        for (int dg = 0; dg < 3; ++dg) bd[dg] = i32x4{int(bw[dg][0]), int(bw[dg][1]), int(bw[dg][2]), int(bw[dg][3])};
      };
      // The epoch's reference first (right unless this tile starts a new
      // epoch), so the weights need not wait for the cross-lane maxima.  A
      // split's first tile always starts one.
      if (epoch) weights((R == neg_inf() ? 0.f : R) - float(kp));

      // Running maximum and the tile's largest v-scale; a new epoch redoes
      // the weights.
      const float m_new = fmaxf(m_run, rows_max(mx) * cs);
      const float vmax = rows_max(vloc);
      float* const fx = fx_s[blk][t & 1u];
      const bool rise = __builtin_amdgcn_ballot_w64(m_new > R) != 0u;
      if (!epoch || rise || vmax >= vcap || vmax < vlo || epoch_tiles >= 1024u) {
        int kp_new = 100;  // no v-scale yet: any later one starts an epoch
        if (vmax > 0.f) {
          kp_new = 22 - __builtin_amdgcn_frexp_expf(vmax * kVmaxMargin);  // vmax * 2^kp < 2^22
          kp_new = kp_new < -100 ? -100 : (kp_new > 100 ? 100 : kp_new);
        }
        const float r_new = m_new == neg_inf() ? neg_inf() : m_new + kPcHeadroom;
        const float f = R == neg_inf() ? 0.f : __builtin_amdgcn_exp2f(R - r_new);  // <= 1
        l_run *= f;
        if (g == 0) fx[n] = f;
        if (lane == 0) {
          fx[16] = epoch ? __builtin_amdgcn_ldexpf(1.f, -kp) : 0.f;
          fx[17] = 1.f;
        }
        R = r_new;
        kp = kp_new;
        vcap = __builtin_amdgcn_ldexpf(0.9921875f, 23 - kp_new);
        vlo = 0.25f * vmax;
        epoch_tiles = 0;
        epoch = true;
        weights((R == neg_inf() ? 0.f : R) - float(kp));
      } else if (lane == 0) {
        fx[17] = 0.f;
      }
      ++epoch_tiles;
      m_run = m_new;
      l_run = fmaf(lw, __builtin_amdgcn_ldexpf(1.f, -kp), l_run);
      uint8_t* const xb = smem + kXBase + (blk * 2u + (t & 1u)) * kXBytes;
  #pragma unroll
      for (int dg = 0; dg < 3; ++dg) *reinterpret_cast<i32x4*>(xb + 1024u * dg + 16u * lane) = bd[dg];
    };

    // A split's end (after its tile t): the partial relative to the true
    // maximum, e = 2^(R - m) (1 .. 2^kPcHeadroom), also for the PV waves.
    auto write_ml = [&](uint32_t sp, uint32_t t) __attribute__((always_inline)) {
      const float e = m_run == neg_inf() ? 0.f : __builtin_amdgcn_exp2f(R - m_run);
      const float l_h = rows_sum(l_run) * e;
      if (hvalid && g == 0) {
        float* const dst = partial(sp);
        dst[0] = m_run * kLn2;
        dst[1] = l_h;
      }
      if (t != ~0u) {
        float* const fx = fx_s[blk][t & 1u];
        if (g == 0) fx[18 + n] = e;
        if (lane == 0) fx[34] = epoch ? __builtin_amdgcn_ldexpf(1.f, -kp) : 0.f;
      }
      m_run = neg_inf();
      l_run = 0.f;
      R = neg_inf();
      epoch = false;
      epoch_tiles = 0;
    };
    for (uint32_t s = 0; s <= ntiles; ++s) {
      __syncthreads();
      if (has && s < ntiles) {
        if (s < nvis) qk_tile(s);
        if (s % tps == tps - 1u || s + 1u == ntiles) write_ml(sp0 + s / tps, s);
      }
    }
    if (has)
      for (uint32_t sp = sp_e; sp < sp1; ++sp) write_ml(sp, ~0u);
    return;
  }
  // PV waves: wave 4 + j takes the 16-dim blocks 4j .. 4j + 3 of every
  // head-row block (the V rows it reads serve all three blocks), so the PV
  // work of the blocks is spread over all four SIMDs.
  const uint32_t pj = wave - 4u;
  bare_barrier();  // the prologue barrier (see the DMA wave)
  f32x4 acc[kPcBlocks][4];  // [block][m]: lane (h, g): dims 16 (4j + m) + 4g + e
  i32x4 cv[kPcBlocks][4][3];  // the current epoch's digit sums, digit 0 (top) .. 2
#pragma unroll
  for (uint32_t b = 0; b < kPcBlocks; ++b)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      acc[b][m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dg = 0; dg < 3; ++dg) cv[b][m][dg] = i32x4{0, 0, 0, 0};
    }
  // An epoch's digit sums into fp32: acc = (acc + (V . P) * 2^-kp) * f.
  auto fold = [&](auto bc, float f, float inv) __attribute__((always_inline)) {
    constexpr uint32_t b = decltype(bc)::value;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = fmaf(float(cv[b][m][0][e]), 65536.f, fmaf(float(cv[b][m][1][e]), 256.f, float(cv[b][m][2][e])));
        acc[b][m][e] = fmaf(x, inv, acc[b][m][e]) * f;
      }
#pragma unroll
      for (int dg = 0; dg < 3; ++dg) cv[b][m][dg] = i32x4{0, 0, 0, 0};
    }
  };
  auto pv_tile = [&](uint32_t t) __attribute__((always_inline)) {
    const uint32_t va = lds_base + (t % kPcSlots) * kImg + voff + 4096u * pj;
    const uint32_t xs = t & 1u;
    u32x4_t vr[4];
    ds_issue16x1<0u>(va, vr[0]);
    ds_issue16x1<1024u>(va, vr[1]);
    ds_issue16x1<2048u>(va, vr[2]);
    ds_issue16x1<3072u>(va, vr[3]);
    wait_lgkm<0>();
#pragma unroll
    for (int m = 0; m < 4; ++m) pin(vr[m]);
    static_for<0, kPcBlocks>([&](auto bc) __attribute__((always_inline)) {
      constexpr uint32_t b = decltype(bc)::value;
      if (b >= hblocks || t >= nvis_s[b]) return;  // a block this tile does not reach
      const float* const fx = fx_s[b][xs];
      // The tile starts a new epoch: fold the one that ends (none at a
      // split's first epoch, whose accumulators are still zero).
      if (fx[17] != 0.f && fx[16] != 0.f) fold(bc, fx[n], fx[16]);
      const uint8_t* const xb = smem + kXBase + (b * 2u + xs) * kXBytes;
      i32x4 bd[3];
#pragma unroll
      for (int dg = 0; dg < 3; ++dg) bd[dg] = *reinterpret_cast<const i32x4*>(xb + 1024u * dg + 16u * lane);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const i32x4 av = {int(vr[m][0]), int(vr[m][1]), int(vr[m][2]), int(vr[m][3])};
#pragma unroll
        for (int dg = 0; dg < 3; ++dg) cv[b][m][dg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bd[dg], cv[b][m][dg], 0, 0, 0);
      }
    });
  };

  // A split's end (after its tile t): fold the last epoch, scale to the true
  // maximum (e), write, restart.
  auto write_n = [&](uint32_t sp, uint32_t t) __attribute__((always_inline)) {
    static_for<0, kPcBlocks>([&](auto bc) __attribute__((always_inline)) {
      constexpr uint32_t b = decltype(bc)::value;
      const uint32_t hrb = b * 16u + n;
      if (b < hblocks && t != ~0u) {
        const float* const fx = fx_s[b][t & 1u];
        fold(bc, fx[18 + n], fx[34]);
      }
      if (b < hblocks && hrb < head_rows) {
        float* const dst = scratch + (size_t(rh_s[hrb]) * a.splits + sp) * W + 2 + 64u * pj;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[16 * m + 4 * g + e] = acc[b][m][e];
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[b][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    });
  };

  for (uint32_t s = 0; s <= ntiles; ++s) {
    __syncthreads();
    if (s > 0u) {
      const uint32_t t = s - 1u;
      pv_tile(t);
      if (t % tps == tps - 1u || t + 1u == ntiles) write_n(sp0 + t / tps, t);
    }
  }
  for (uint32_t sp = sp_e; sp < sp1; ++sp) write_n(sp, ~0u);
}

#define KVB_I8R_ARGS                                                                             \
  a, a.q, a.q_positions, a.k_positions, a.page_table, static_cast<const int8_t*>(a.k),             \
      static_cast<const int8_t*>(a.v), a.k_scales, a.v_scales, a.scratch, spw

// The wave-specialized kernel: dim 256 and one round of at most three
// head-row blocks (17 to 48 head-rows).
bool pc_shape(const SplitArgs& a) {
  const uint32_t hblocks = (a.rows * a.group + 15u) / 16u;
  return a.dim == 256 && hblocks <= kPcBlocks;
}

template <int D>
hipError_t launch_dim(const SplitArgs& a, hipStream_t stream) {
  // Short splits: several consecutive splits per work-group (one work-group
  // per CU where there are enough), when a split is a whole number of phases.
  uint32_t spw = 1u;
  if ((a.split_tokens / kTileTokens) % RowsGeo<D>::kCT == 0u) {
    const uint32_t per_cu = uint32_t((uint64_t(a.splits) * a.kv_heads) / device_cus());
    spw = per_cu > 1u ? per_cu : 1u;
  }
  const dim3 grid((a.splits + spw - 1u) / spw, a.kv_heads);
  const bool pt = a.page_tokens % kTileTokens == 0;
  if constexpr (D == 256) {
    if (pc_shape(a)) {
      if (pt)
        hipLaunchKernelGGL((split_i8_rows_pc_kernel<D, true>), grid, dim3(64 * kPcWaves), 0, stream, KVB_I8R_ARGS);
      else
        hipLaunchKernelGGL((split_i8_rows_pc_kernel<D, false>), grid, dim3(64 * kPcWaves), 0, stream, KVB_I8R_ARGS);
      return hipGetLastError();
    }
  }
  if (pt)
    hipLaunchKernelGGL((split_i8_rows_kernel<D, true>), grid, dim3(64 * kWaves), 0, stream, KVB_I8R_ARGS);
  else
    hipLaunchKernelGGL((split_i8_rows_kernel<D, false>), grid, dim3(64 * kWaves), 0, stream, KVB_I8R_ARGS);
  return hipGetLastError();
}

template <int D>
hipError_t preload_dim() {
  hipFuncAttributes attr{};
  hipError_t e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_i8_rows_kernel<D, true>));
  if (e == hipSuccess) e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_i8_rows_kernel<D, false>));
  if constexpr (D == 256) {
    if (e == hipSuccess) e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_i8_rows_pc_kernel<D, true>));
    if (e == hipSuccess) e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&split_i8_rows_pc_kernel<D, false>));
  }
  return e;
}

}  // namespace

// More than 8 head-rows (the single-block int8 kernel's limit), dim 128 or
// 256, one sequence, splits that start on a 64-token tile.
bool i8_rows_supported(const SplitArgs& a) {
  if (a.rows * a.group <= 8u || a.seq_starts != nullptr) return false;
  if (a.dim != 128 && a.dim != 256) return false;
  return a.begin % kTileTokens == 0 && a.split_tokens % kTileTokens == 0;
}

hipError_t launch_split_i8_rows(const SplitArgs& a, hipStream_t stream) {
  switch (a.dim) {
    case 128: return launch_dim<128>(a, stream);
    case 256: return launch_dim<256>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

const char* i8_rows_kernel_name(const SplitArgs& a) {
  static thread_local char buf[96];
  std::snprintf(buf, sizeof(buf), "%s<%u,%s>", pc_shape(a) ? "split_i8_rows_pc_kernel" : "split_i8_rows_kernel",
                a.dim, a.page_tokens % kTileTokens == 0 ? "true" : "false");
  return buf;
}

hipError_t preload_i8_rows() {
  const hipError_t e = preload_dim<128>();
  if (e != hipSuccess) return e;
  return preload_dim<256>();
}

// Compute units of the current device (cached per device; callers on
// several threads may fill an entry concurrently with the same value).
uint32_t device_cus() {
  static std::atomic<uint32_t> cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256u;
  uint32_t v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0u) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    v = uint32_t(n);
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace kvb
