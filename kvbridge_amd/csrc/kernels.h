// Internal launcher interface between the C ABI (capi.cpp) and the HIP
// translation units.  Shapes reaching these functions are already validated.
#pragma once
#include <hip/hip_runtime_api.h>
#include <cstdint>
#include <string>
#include "kvbridge/attention_common.h"

namespace kvb {

// Arguments common to both split kernels.  Token indices are logical; every
// physical offset fits 32 bits (attention_shape_error rejects larger KV).
struct SplitArgs {
  const float* q;
  const int64_t* q_positions;
  const int64_t* k_positions;
  const uint32_t* page_table;
  const void* k;
  const void* v;
  const float* k_scales;
  const float* v_scales;
  float* scratch;
  uint32_t rows, q_heads, kv_heads, group, dim, page_tokens, pages, begin, end;
  uint32_t split_tokens, splits;
  float scale;
  // Fused merge (kvb_decode_attention_fused): non-null counters make the
  // last work-group of each kv head merge that head's splits into m, l, n
  // (and out when out_type != 0).  counters[kv_heads] must be zero on entry
  // and are zero again when the kernel ends.
  uint32_t* counters;
  float* m;
  float* l;
  float* n;
  void* out;
  int out_type;
  // Batched call (kvb_decode_attention_batched): non-null seq_starts makes
  // grid.z the sequence index b, and every work-group first rebases these
  // arguments on sequence b (rebase_sequence, batch.h).  q, q_positions and
  // the outputs then hold `batch` consecutive blocks of rows * q_heads
  // row-heads, k_positions and page_table are concatenations indexed through
  // seq_starts / page_offsets, and `splits` is the partial stride of every
  // sequence (the split count of max_tokens).
  const uint32_t* seq_starts;    // [batch + 1] token offsets into k_positions
  const uint32_t* page_offsets;  // [batch] first page-table entry of each sequence
  uint32_t batch;
  uint32_t total_tokens;         // k_positions entries (device indices are clamped to it)
  uint32_t table_entries;        // page_table entries (likewise)
  uint32_t max_tokens;           // bound on every sequence's token count
};

// Sets the thread-local message kvb_last_error() returns; returns code.
int set_error(int code, const std::string& msg);

SplitArgs make_split_args(const kvbridge::Shape& s, const kvbridge::DeviceInput& in,
                          unsigned split_tokens, unsigned splits, float* scratch);

// Whether the tiled MFMA split kernels cover this shape and these buffers.
bool tiled_supported(const kvbridge::Shape& s, const kvbridge::DeviceInput& in);

hipError_t launch_split_lds(const SplitArgs& a, hipStream_t stream);  // LDS-DMA-staged tiles, f16 MFMA
hipError_t launch_split_i8(const SplitArgs& a, hipStream_t stream);   // register-staged tiles, int8 MFMA
bool i8_supported(const SplitArgs& a);  // head_rows <= 8 (<= 4 at dim 256), power-of-two pages
bool i8_fusable(const SplitArgs& a);    // the int8 kernel can run the fused merge
// Diagnostic: the fused launch with formal release / acquire fences around
// the merge ticket (eight-wave dim-128 page-tile configuration only).
bool i8_fenced_supported(const SplitArgs& a);
hipError_t launch_split_i8_fenced(const SplitArgs& a, hipStream_t stream);
// Int8-MFMA kernel for more than 8 head-rows over short tile-aligned splits
// (one work-group per split and kv head, the split's tiles held in LDS).
hipError_t launch_split_i8_rows(const SplitArgs& a, hipStream_t stream);
bool i8_rows_supported(const SplitArgs& a);  // dim 128/256, one sequence, splits of <= 8/4 whole tiles
const char* i8_rows_kernel_name(const SplitArgs& a);
// The MFMA split path used by the entry points: the int8-MFMA kernel where
// i8_supported, else the int8-MFMA rows kernel where i8_rows_supported, else
// the f16-MFMA LDS kernel.  KVB_SPLIT_IMPL=f16 forces the f16 kernels
// (comparisons).
hipError_t launch_split_fast(const SplitArgs& a, hipStream_t stream);
hipError_t launch_split_generic(const SplitArgs& a, bool int8, hipStream_t stream);
// Kernel instance a launch would run (diagnostics, profiles).
const char* lds_kernel_name(const SplitArgs& a);
const char* i8_kernel_name(const SplitArgs& a);
const char* split_kernel_name(const SplitArgs& a, bool tiled, bool int8);
uint32_t device_cus();  // compute units of the current device (cached per device)
// out_type: 0 none, 1 fp32, 2 fp16 (kvbridge_c.h KVB_OUT_*).
hipError_t launch_merge(uint32_t row_heads, uint32_t dim, uint32_t splits, const float* scratch,
                        float* m, float* l, float* n, void* out, int out_type,
                        hipStream_t stream);

// Paged INT8 KV append (append.hip): tokens rows of k_new / v_new
// ([token][kv_head][dim] at k_stride / v_stride elements per token, element
// type src_type: 1 fp32, 2 fp16, 3 bf16) quantized into physical slots
// slots[t] (page = slot / page_tokens) of the pool.
struct AppendArgs {
  const void* k_new;
  const void* v_new;
  const uint32_t* slots;
  int8_t* k;
  int8_t* v;
  float* k_scales;
  float* v_scales;
  uint32_t tokens, kv_heads, dim, page_tokens, pages;
  uint32_t k_stride, v_stride;
  int src_type;
};
hipError_t launch_append(const AppendArgs& a, hipStream_t stream);
hipError_t preload_append();

// Streaming HBM read probe (diagnostic).
hipError_t launch_read_probe(const void* src, size_t bytes, uint32_t* sink, uint32_t blocks,
                             hipStream_t stream);
// Paged read probe (diagnostic): a decode call's K, V and scale bytes read
// through its page table, no arithmetic (dim 64/128/256, page_tokens a
// multiple of 64, 16-byte aligned K and V).
hipError_t launch_paged_read_probe(const uint32_t* table, const void* k, const void* v, const float* ks,
                                   const float* vs, uint32_t kv_heads, uint32_t dim, uint32_t page_tokens,
                                   uint32_t pages, uint32_t begin, uint32_t end, uint32_t split_tokens,
                                   uint32_t splits, uint32_t* sink, hipStream_t stream);

hipError_t preload_lds();
hipError_t preload_i8();
hipError_t preload_i8_rows();
hipError_t preload_generic();
hipError_t preload_merge();

}  // namespace kvb
