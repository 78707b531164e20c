// HBM streaming-read probe (diagnostic, used by bench.py for context): reads
// `bytes` of device memory once with 16-byte non-temporal loads spread over
// many waves and keeps them live with a data-dependent store, so the measured
// time is the achievable read bandwidth of this device for a pure stream.
// It plays the role of the reference's same-layout stream probe
// (data/att-bench-65536-v2-07.json:528-541), measured on MI355X.
#include "kernels.h"
#include "device_common.h"

namespace kvb {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void read_probe_kernel(const u32x4* __restrict__ src, size_t n16,
                                                              uint32_t* __restrict__ sink) {
  const size_t stride = size_t(gridDim.x) * kThreads;
  size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  // Data-dependent store keeps every load live; it practically never fires.
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t launch_read_probe(const void* src, size_t bytes, uint32_t* sink, uint32_t blocks,
                             hipStream_t stream) {
  hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(kThreads), 0, stream,
                     static_cast<const u32x4*>(src), bytes / 16, sink);
  return hipGetLastError();
}

}  // namespace kvb
