// Host side of the integer-MFMA split kernel (split_i8.h): shape support,
// the (waves, ring slots) choice, and dispatch to the per-dim translation
// units split_i8_d64/_d128/_d256.hip (built in parallel).
#include <cstdio>
#include <cstdlib>

#include "kernels.h"

namespace kvb {

hipError_t launch_i8_d64(const SplitArgs& a, int cfg, hipStream_t stream);
hipError_t launch_i8_d128(const SplitArgs& a, int cfg, hipStream_t stream);
hipError_t launch_i8_d256(const SplitArgs& a, int cfg, hipStream_t stream);
hipError_t preload_i8_d64();
hipError_t preload_i8_d128();
hipError_t preload_i8_d256();

namespace {

constexpr uint32_t kTiles = 64;  // tokens per tile

// (waves, ring slots) per work-group as 10 * NW + NB.  A grid of at most
// two work-groups per CU of a 256-CU device: eight waves (two per SIMD,
// <= 256 registers each) where the state fits (head_rows <= 4, dim <= 128)
// and the split has >= 16 tiles.  Larger grids (batches) run several rounds
// of work-groups per CU, and smaller work-groups that share a CU hide each
// other's prologue and combine: four waves (two per SIMD) for <= 4
// head-rows, two waves for 8 head-rows (whose state takes one SIMD per
// wave).  Measured on MI355X (configs[2] / configs[3] batched calls,
// 2048-work-group grids): 118 / 216 us with these against 140 / 242 us with
// the single-sequence choice.  Large grids of short splits (<= 32 tiles)
// run one wave per work-group: the wave streams its split alone, so there is
// no wave combine, no work-group barrier and no idle wave per split, and
// eight such work-groups share a CU.  Measured: cfg2 through launch_attention
// (its 256-token splits, 2,048 work-groups) 47.7 -> 25.3 us for the split
// launch, configs[3] (64 chunks of 2,048 tokens, 8 head-rows) 203.5 -> 190.6
// us; configs[2] at 5,120-token splits (80 tiles) stays on four waves (91
// against 111 us).
// KVB_I8_CFG="NW,NB" overrides (tuning sweeps; unknown pairs fall back).
int i8_config(const SplitArgs& a) {
  static const int forced = [] {
    const char* e = std::getenv("KVB_I8_CFG");
    int nw = 0, nb = 0;
    char tail = 0;
    if (!e || std::sscanf(e, "%d,%d%c", &nw, &nb, &tail) != 2 || nw < 1 || nw > 9 || nb < 1 || nb > 9) return 0;
    return nw * 10 + nb;
  }();
  const uint32_t tiles = (a.split_tokens + kTiles - 1) / kTiles;
  const uint32_t hr = a.rows * a.group;
  const bool eight = hr <= 4 && a.dim <= 128;
  if (forced == 42 || forced == 22 || forced == 12 || ((forced == 82 || forced == 44) && eight) ||
      (forced == 14 && hr <= 4))
    return forced;
  const uint64_t groups = uint64_t(a.splits) * a.kv_heads * (a.seq_starts ? a.batch : 1u);
  if (groups > 512u) {
    if (tiles <= 32u) return 12;
    return hr <= 4 ? 42 : 22;
  }
  if (eight && tiles >= 16) return 82;
  return tiles >= 4 ? 42 : 22;
}

}  // namespace

// head_rows <= 8 (<= 4 at dim 256); page_tokens a power of two >= 16 (>= 64
// for batched calls); the small-page path addresses K/V with 32-bit offsets.
bool i8_supported(const SplitArgs& a) {
  const uint32_t hr = a.rows * a.group, P = a.page_tokens;
  if (hr > 8 || (a.dim == 256 && hr > 4)) return false;
  if (a.dim != 64 && a.dim != 128 && a.dim != 256) return false;
  if (P < 16 || (P & (P - 1u)) != 0) return false;
  if (a.seq_starts && P < kTiles) return false;  // batched calls: whole-tile pages only
  if (P < kTiles && uint64_t(a.pages) * a.kv_heads * P * a.dim >= (uint64_t(1) << 32)) return false;
  return true;
}

// The in-kernel merge of the single launch is worth it where it is short:
// the straight-line path (<= 32 splits, a thread per output, a wave per
// head-row) or at most two merge_rows passes with a thread per four columns;
// larger merges (e.g. 8 head-rows on two-wave work-groups) run faster as the
// stand-alone merge kernel, whose work-groups spread over every CU.  Grids
// of more than two work-groups per CU (batches) also run two launches: every
// work-group's ticket and the merges then sit between rounds of split work
// (configs[2]: 116 us for two launches against 121-123 us for one).
bool i8_fusable(const SplitArgs& a) {
  if (!i8_supported(a)) return false;
  if (uint64_t(a.splits) * a.kv_heads * (a.seq_starts ? a.batch : 1u) > 512u) return false;
  const uint32_t nw = uint32_t(i8_config(a)) / 10u, threads = 64u * nw;
  const uint32_t hr = a.rows * a.group, hs = hr <= 4 ? 4u : 8u;
  if (a.splits <= 32 && hr * a.dim <= threads && hr <= nw) return true;
  const uint32_t quads = hs * a.dim / 4u;
  if (quads > threads) return false;
  const uint32_t groups = threads / quads, per_pass = groups * (groups >= 4 ? 64u / groups : 16u);
  return (a.splits + per_pass - 1u) / per_pass <= 2u;
}

hipError_t launch_i8_fenced_d128(const SplitArgs& a, hipStream_t stream);

// Diagnostic single launch with formal release / acquire fences: only the
// eight-wave dim-128 page-tile configuration (cfg2's) has an instance.
bool i8_fenced_supported(const SplitArgs& a) {
  return a.dim == 128 && a.seq_starts == nullptr && a.page_tokens >= kTiles && i8_supported(a) && i8_fusable(a) &&
         i8_config(a) == 82;
}

hipError_t launch_split_i8_fenced(const SplitArgs& a, hipStream_t stream) {
  return i8_fenced_supported(a) ? launch_i8_fenced_d128(a, stream) : hipErrorInvalidValue;
}

hipError_t launch_split_i8(const SplitArgs& a, hipStream_t stream) {
  const int cfg = i8_config(a);
  switch (a.dim) {
    case 64: return launch_i8_d64(a, cfg, stream);
    case 128: return launch_i8_d128(a, cfg, stream);
    case 256: return launch_i8_d256(a, cfg, stream);
    default: return hipErrorInvalidValue;
  }
}

const char* i8_kernel_name(const SplitArgs& a) {
  static thread_local char buf[112];
  const int cfg = i8_config(a);
  std::snprintf(buf, sizeof(buf), "split_i8_kernel<%u,%d,%d,%s,%d,%s,%s,false>", a.dim, cfg / 10, cfg % 10,
                a.page_tokens >= kTiles ? "true" : "false", a.rows * a.group <= 4 ? 4 : 8,
                a.counters != nullptr ? "true" : "false", a.seq_starts != nullptr ? "true" : "false");
  return buf;
}

hipError_t preload_i8() {
  hipError_t e = preload_i8_d64();
  if (e == hipSuccess) e = preload_i8_d128();
  if (e == hipSuccess) e = preload_i8_d256();
  return e;
}

}  // namespace kvb
