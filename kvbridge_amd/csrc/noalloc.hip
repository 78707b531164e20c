// kvb_decode_attention_noalloc: the single-launch decode call
// (kvb_decode_attention_fused) for callers that cannot allocate device memory
// (code under graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  Its scratch -- the split partials and the per-kv-head merge
// counters -- lives in `scratch`, a file-scope device array of fixed size;
// the caller passes only inputs and outputs.
//
// Host code never uses the array's name as a device address: the first call
// on each device (with that device current) looks its address up with
// hipGetSymbolAddress, and every call passes that pointer to the kernels.
// Layout: a fixed counter region of kCounterWords words (one per kv head of
// the largest single-launch grid: splits * kv_heads <= 512, so at most 512
// kv heads), then the partials.  The region does not depend on the call's
// kv_heads, so no call's partials ever land on another call's counter
// words.  The array is zero when the code object is loaded, and every
// completed single-launch call leaves the counter words it used zero again
// (the merging work-group resets them), which is the state the next call
// needs; partial words need no clearing.
// Every call on one device shares that device's array: calls that overlap on
// one device (two streams, two host threads) race.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>

#include "kernels.h"
#include "kvbridge_c.h"

namespace {

constexpr size_t kNoAllocBytes = size_t(8) << 20;       // 8 MiB per device
constexpr size_t kNoAllocWords = kNoAllocBytes / 4;
constexpr size_t kCounterWords = 512;  // = the single-launch grid limit (kv heads <= 512)
constexpr uint32_t kMaxDevices = 64;

static __device__ __align__(256) uint32_t scratch[kNoAllocWords];

std::mutex g_mutex;
void* g_ptr[kMaxDevices] = {};

// Device address of this device's array (looked up once per device).
hipError_t scratch_address(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || uint32_t(dev) >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_ptr[dev] = p;
  }
  *ptr = g_ptr[dev];
  return hipSuccess;
}

}  // namespace

extern "C" {

int kvb_decode_attention_noalloc(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens, float* m,
                                 float* l, float* n, void* out, int out_type, void* stream) {
  if (!sp || !ip)  // same status and message as the allocating entry point
    return kvb_decode_attention_fused(sp, ip, split_tokens, nullptr, nullptr, m, l, n, out, out_type, stream);
  size_t partials = 0;
  if (const int rc = kvb_scratch_elements_ex(sp, split_tokens, &partials); rc != KVB_OK) return rc;
  // The fixed counter region first, then the partials.  A call that is not
  // run as a single launch (more than 512 kv heads x splits) uses no counter,
  // so kCounterWords covers every counter a call can touch.
  if (partials > kNoAllocWords - kCounterWords)
    return kvb::set_error(KVB_EINVAL, "kvb_decode_attention_noalloc: the call needs " +
                                          std::to_string(partials * 4) + " bytes of partials, the static area holds " +
                                          std::to_string((kNoAllocWords - kCounterWords) * 4) +
                                          " (pass a buffer to kvb_decode_attention_fused instead)");
  void* base = nullptr;
  if (const hipError_t e = scratch_address(&base); e != hipSuccess)
    return kvb::set_error(KVB_ERUNTIME, std::string("no-alloc scratch lookup: ") + hipGetErrorString(e));
  uint32_t* counters = static_cast<uint32_t*>(base);
  float* partial_base = reinterpret_cast<float*>(counters + kCounterWords);
  return kvb_decode_attention_fused(sp, ip, split_tokens, partial_base, counters, m, l, n, out, out_type, stream);
}

}  // extern "C"
