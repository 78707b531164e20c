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

// (waves, ring slots) per work-group as 10 * NW + NB, by tiles per split:
// eight waves (two per SIMD, <= 256 registers each) where the state fits
// (head_rows <= 4, dim <= 128) and the split has >= 16 tiles.
// KVB_I8_CFG="NW,NB" overrides (tuning sweeps; unknown pairs fall back).
int i8_config(const SplitArgs& a) {
  static const int forced = [] {
    const char* e = std::getenv("KVB_I8_CFG");
    if (!e) return 0;
    return std::atoi(e) * 10 + std::atoi(e + 2);
  }();
  const uint32_t tiles = (a.split_tokens + kTiles - 1) / kTiles;
  const bool eight = a.rows * a.group <= 4 && a.dim <= 128;
  if (forced == 42 || forced == 22 || ((forced == 82 || forced == 44) && eight)) return forced;
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

bool i8_fusable(const SplitArgs& a) { return i8_supported(a); }

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
  std::snprintf(buf, sizeof(buf), "split_i8_kernel<%u,%d,%d,%s,%d,%s,%s>", a.dim, cfg / 10, cfg % 10,
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
