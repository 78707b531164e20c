// Integer-MFMA split kernel instances for head_dim 64 (kernel: split_i8.h).
#include "split_i8.h"

namespace kvb {

hipError_t launch_i8_d64(const SplitArgs& a, int cfg, hipStream_t stream) { return launch_dim<64>(a, cfg, stream); }

hipError_t preload_i8_d64() { return preload_dim<64>(); }

}  // namespace kvb
