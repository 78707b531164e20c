// Integer-MFMA split kernel instances for head_dim 256 (kernel: split_i8.h).
#include "split_i8.h"

namespace kvb {

hipError_t launch_i8_d256(const SplitArgs& a, int cfg, hipStream_t stream) { return launch_dim<256>(a, cfg, stream); }

hipError_t preload_i8_d256() { return preload_dim<256>(); }

}  // namespace kvb
