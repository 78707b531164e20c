// HBM streaming-read probe (diagnostic, used by bench.py for context): reads
// `bytes` of device memory once and keeps the data live with a data-dependent
// store, so the measured time is what a single launch that only streams
// these bytes achieves on this device.  The structure is the best of the
// read patterns measured here: each work-group (8 waves) takes a contiguous
// run of 8 KiB items, each wave reads whole items (64 lanes x 8 x 16-byte
// non-temporal loads, one item in flight).  It plays the role of the
// reference's same-layout stream probe (data/att-bench-65536-v2-07.json:528-541).
#include "kernels.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr size_t kItem16 = 512;  // 16-byte chunks per 8 KiB item
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void read_probe_kernel(const u32x4* __restrict__ src, size_t items,
                                                              size_t per_group, size_t tail16,
                                                              uint32_t* __restrict__ sink) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const size_t i0 = size_t(blockIdx.x) * per_group;
  const size_t i1 = i0 + per_group < items ? i0 + per_group : items;
  uint32_t acc = 0;
  for (size_t it = i0 + wave; it < i1; it += kWaves) {
    const u32x4* p = src + it * kItem16 + lane;
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_nontemporal_load(p + 64 * j);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
  }
  if (blockIdx.x == 0) {  // bytes past the last whole item
    for (size_t k = threadIdx.x; k < tail16; k += kThreads) {
      const u32x4 v = __builtin_nontemporal_load(src + items * kItem16 + k);
      acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
  }
  // Data-dependent store keeps every load live; it practically never fires.
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t launch_read_probe(const void* src, size_t bytes, uint32_t* sink, uint32_t blocks,
                             hipStream_t stream) {
  const size_t items = bytes / (16 * kItem16);
  const size_t per_group = (items + blocks - 1) / blocks;
  const size_t tail16 = (bytes - items * 16 * kItem16) / 16;
  hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(kThreads), 0, stream, static_cast<const u32x4*>(src),
                     items, per_group, tail16, sink);
  return hipGetLastError();
}

}  // namespace kvb
