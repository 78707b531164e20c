// Integer-MFMA split kernel instances for head_dim 128 (kernel: split_i8.h).
#include "split_i8.h"

namespace kvb {

hipError_t launch_i8_d128(const SplitArgs& a, int cfg, hipStream_t stream) { return launch_dim<128>(a, cfg, stream); }

hipError_t preload_i8_d128() { return preload_dim<128>(); }

// Diagnostic: the single launch of the eight-wave page-tile configuration
// (cfg2's) with formal release / acquire fences around the ticket.
hipError_t launch_i8_fenced_d128(const SplitArgs& a, hipStream_t stream) {
  if (a.counters == nullptr || a.seq_starts != nullptr || a.page_tokens < kTileTokens || a.rows * a.group > 4)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL((split_i8_kernel<128, 8, 2, true, 4, true, false, true>), dim3(a.splits, a.kv_heads, 1u),
                     dim3(64 * 8), 0, stream, KVB_I8_ARGS);
  return hipGetLastError();
}

}  // namespace kvb
