// Integer-MFMA split kernel instances for head_dim 128 (kernel: split_i8.h).
#include "split_i8.h"

namespace kvb {

hipError_t launch_i8_d128(const SplitArgs& a, int cfg, hipStream_t stream) { return launch_dim<128>(a, cfg, stream); }

hipError_t preload_i8_d128() { return preload_dim<128>(); }

}  // namespace kvb
