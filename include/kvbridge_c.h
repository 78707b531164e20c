/* C ABI of the MI355X paged INT8-KV split-K decode-attention library
 * (libkvbridge_amd.so).  Plain C types only: device buffers are raw pointers,
 * the HIP stream is passed as void* (a hipStream_t, NULL = default stream).
 *
 * Every kvb_* entry point below replaces one function of the reference C++
 * API (cited per declaration) or is an additive extension (marked).  Calls
 * return KVB_OK or an error code; kvb_last_error() then holds the message of
 * the exception the reference would have thrown.  KVB_EINVAL corresponds to
 * std::invalid_argument (raised before anything is enqueued), KVB_ERUNTIME
 * to std::runtime_error (a HIP launch or setup failure).  Kernel execution is
 * asynchronous: device-side faults surface at the caller's synchronization.
 * The library allocates nothing; all buffers and the stream belong to the
 * caller.  No global state except the thread-local error message. */
#ifndef KVBRIDGE_C_H
#define KVBRIDGE_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { KVB_OK = 0, KVB_EINVAL = 1, KVB_ERUNTIME = 2 };
enum { KVB_OUT_NONE = 0, KVB_OUT_F32 = 1, KVB_OUT_F16 = 2 };
enum { KVB_KERNEL_TILED_MFMA = 1, KVB_KERNEL_GENERIC = 2 };

/* Mirrors kvbridge::Shape (reference include/kvbridge/attention_shape.h:9-13);
 * the bool becomes a uint32_t so the struct has one C layout. */
typedef struct kvb_shape {
  uint32_t rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, begin, end;
  float scale;
  uint32_t int8;
} kvb_shape;

/* Mirrors kvbridge::DeviceInput (reference include/kvbridge/attention_common.h:54-63). */
typedef struct kvb_device_input {
  const float* q;
  const int64_t* q_positions;
  const int64_t* k_positions;
  const uint32_t* page_table;
  const void* k;
  const void* v;
  const float* k_scales;
  const float* v_scales;
} kvb_device_input;

/* Message of the last failed kvb_* call on this thread ("" if none). */
const char* kvb_last_error(void);

/* kvbridge::kSplitTokens (reference attention_shape.h:7). */
uint32_t kvb_split_tokens(void);

/* kvbridge::attention_shape_error (reference src/attention_shape.cpp:20-46):
 * NULL when valid, else the first failed rule's message. */
const char* kvb_shape_error(const kvb_shape* s);
/* kvbridge::attention_shape_valid (reference src/attention_shape.cpp:48). */
int kvb_shape_valid(const kvb_shape* s);
/* kvbridge::split_count (reference src/attention_shape.cpp:52-55). */
int kvb_split_count(const kvb_shape* s, uint32_t* splits);
/* kvbridge::scratch_elements (reference src/attention_shape.cpp:56-59). */
int kvb_scratch_elements(const kvb_shape* s, size_t* elements);
/* kvbridge::output_scalar_elements (reference src/attention_shape.cpp:60-63). */
int kvb_output_scalar_elements(const kvb_shape* s, size_t* elements);
/* kvbridge::output_numerator_elements (reference src/attention_shape.cpp:64-66). */
int kvb_output_numerator_elements(const kvb_shape* s, size_t* elements);
/* kvbridge::attention_mma_supported (reference src/attention_shape.cpp:67-70). */
int kvb_mma_supported(const kvb_shape* s);

/* kvbridge::preload_attention_kernels / _reference_kernels / _mma_kernels
 * (reference include/kvbridge/attention_common.h:69-72, src/attention_shared.cu:376-387,
 * src/attention_mma.cu:13-31).  Return a hipError_t value (0 = success). */
int kvb_preload_attention_kernels(void);
int kvb_preload_attention_reference_kernels(void);
int kvb_preload_attention_mma_kernels(void);

/* kvbridge::launch_attention (reference include/kvbridge/attention_common.h:80-81,
 * src/attention_shared.cu:339-366): kSplitTokens-token split partials + merge. */
int kvb_launch_attention(const kvb_shape* s, const kvb_device_input* in, float* scratch,
                         float* m, float* l, float* n, void* stream);
/* kvbridge::launch_attention_mma (reference include/kvbridge/attention_common.h:90-91,
 * src/attention_mma.cu:33-45): same outputs; KVB_EINVAL unless kvb_mma_supported. */
int kvb_launch_attention_mma(const kvb_shape* s, const kvb_device_input* in, float* scratch,
                             float* m, float* l, float* n, void* stream);
/* kvbridge::merge_attention (reference include/kvbridge/attention_common.h:95-96,
 * src/attention_shared.cu:368-374): splits must equal kvb_split_count. */
int kvb_merge_attention(const kvb_shape* s, const float* scratch, uint32_t splits,
                        float* m, float* l, float* n, void* stream);

/* Extension: split count / scratch size for caller-chosen split_tokens. */
int kvb_split_count_ex(const kvb_shape* s, uint32_t split_tokens, uint32_t* splits);
int kvb_scratch_elements_ex(const kvb_shape* s, uint32_t split_tokens, size_t* elements);
/* Extension: split partials only, split_tokens tokens per split. */
int kvb_split_attention(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens,
                        float* scratch, void* stream);
/* Extension: LSE merge of `splits` partials, plus the normalized output
 * out[rh*dim+d] = l > 0 ? n/l : 0 in out_type (KVB_OUT_F32 / KVB_OUT_F16),
 * or no output for KVB_OUT_NONE (out may then be NULL). */
int kvb_merge_finalize(const kvb_shape* s, const float* scratch, uint32_t splits,
                       float* m, float* l, float* n, void* out, int out_type, void* stream);
/* Extension: kvb_split_attention then kvb_merge_finalize on one stream. */
int kvb_decode_attention(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens,
                         float* scratch, float* m, float* l, float* n, void* out, int out_type,
                         void* stream);
/* Extension (no counterpart in the reference library; for decode loops that
 * want one launch per call): kvb_decode_attention as a single kernel where
 * the int8-MFMA split kernel serves the shape and its in-kernel merge is
 * short (at most two 16-byte-load passes over the splits) -- the last
 * work-group to finish for each kv head merges that head's splits
 * (log-sum-exp) into m, l, n and out.  Otherwise it runs the two launches of
 * kvb_decode_attention.  `counters` holds kv_heads uint32 that must be zero
 * before the first call; every call leaves them zero (allocate and zero them
 * once, e.g. next to the scratch buffer).  Calls sharing `counters` must not
 * overlap in time (same rule as for scratch).  m, l, n, out equal those of
 * kvb_decode_attention up to fp32 summation order in the merge.  What the
 * single launch leaves in scratch is internal: where its merge takes the
 * short path (<= 32 splits) the partials are packed in a layout of their
 * own, not the rows kvb_split_attention writes. */
int kvb_decode_attention_fused(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens,
                               float* scratch, uint32_t* counters, float* m, float* l, float* n, void* out,
                               int out_type, void* stream);
/* Extension (no counterpart in the reference library, which serves one
 * sequence per call; for batched serving loops and the ragged-batch
 * workloads): a batch of independent decode sequences over one shared paged
 * KV pool, in one call.  Mirrors kvbridge::BatchShape / BatchInput
 * (include/kvbridge/attention_ext.h, which documents the layout): sequence b
 * attends to its tokens [0, T_b), T_b = seq_starts[b+1] - seq_starts[b], its
 * logical page p is physical page page_table[page_offsets[b] + p], and it runs
 * max(1, ceil(T_b / split_tokens)) splits.  seq_starts and page_offsets are
 * device arrays read by the kernels (graph-capturable with changing
 * lengths); every index is clamped to total_tokens / table_entries and T_b
 * to max_tokens. */
typedef struct kvb_batch_shape {
  uint32_t batch, rows, q_heads, kv_heads, dim, page_tokens, pages;
  uint32_t max_tokens, total_tokens, table_entries, split_tokens;
  float scale;
  uint32_t int8;
} kvb_batch_shape;

typedef struct kvb_batch_input {
  const float* q;
  const int64_t* q_positions;
  const uint32_t* seq_starts;
  const uint32_t* page_offsets;
  const int64_t* k_positions;
  const uint32_t* page_table;
  const void* k;
  const void* v;
  const float* k_scales;
  const float* v_scales;
} kvb_batch_input;

/* NULL when valid, else the first failed rule's message. */
const char* kvb_batch_shape_error(const kvb_batch_shape* s);
/* Partial stride per sequence (split count of max_tokens). */
int kvb_batch_split_count(const kvb_batch_shape* s, uint32_t* splits);
/* batch * rows * q_heads * kvb_batch_split_count * (dim + 2) floats. */
int kvb_batch_scratch_elements(const kvb_batch_shape* s, size_t* elements);
/* batch * rows * q_heads: elements of m and l (times dim: n and out). */
int kvb_batch_output_scalar_elements(const kvb_batch_shape* s, size_t* elements);
/* Split partials + log-sum-exp merge of every sequence into m, l, n and
 * out (KVB_OUT_*), in the batch's row-head order.  counters == NULL: two
 * launches (split, merge).  counters != NULL (batch * kv_heads uint32, zero
 * before the first call and left zero by every call): one launch where the
 * int8-MFMA kernel serves the shape and its in-kernel merge is short (as
 * for kvb_decode_attention_fused), the last work-group of each
 * (sequence, kv head) merging its splits; otherwise two launches.  The
 * single launch writes partials only for each sequence's own splits (the
 * rest of that sequence's scratch block is left as it was), in the internal
 * layout of kvb_decode_attention_fused. */
int kvb_decode_attention_batched(const kvb_batch_shape* s, const kvb_batch_input* in, float* scratch,
                                 uint32_t* counters, float* m, float* l, float* n, void* out, int out_type,
                                 void* stream);
/* Extension (diagnostic): name of the split kernel instance the batched call
 * would launch ("" if the arguments are invalid). */
const char* kvb_batch_kernel_name(const kvb_batch_shape* s, const kvb_batch_input* in, int fused);

/* Extension (no counterpart in the reference library, which ships no cache
 * writer; the write side of the layout in include/kvbridge/attention_common.h
 * and of the quantization the decode configs use): quantize the K and V rows
 * of `tokens` new tokens and store them into the paged pool.  New token t,
 * kv head h: its rows k_new[t * k_stride + h * dim + d] (likewise v_new) in
 * src_type (KVB_SRC_*) go to physical slot slots[t] (page = slot /
 * page_tokens), with per-(token, kv head) scale = absmax / 127 (1 when the
 * row is all zero) and code = clamp(rint(x / scale), -127, 127) in IEEE fp32
 * (round to nearest even): K token-major, V dim-major, scales into
 * k_scales / v_scales.  slots is a device array; ids >= pages * page_tokens
 * are skipped (padding).  Two tokens with the same slot race.  Asynchronous
 * on `stream`, allocates nothing. */
enum { KVB_SRC_F32 = 1, KVB_SRC_F16 = 2, KVB_SRC_BF16 = 3 };
typedef struct kvb_append_shape {
  uint32_t tokens, kv_heads, dim, page_tokens, pages;
  uint32_t k_stride, v_stride; /* elements between consecutive new tokens */
  uint32_t src_type;
} kvb_append_shape;

typedef struct kvb_append_io {
  const void* k_new;
  const void* v_new;
  const uint32_t* slots;
  int8_t* k;
  int8_t* v;
  float* k_scales;
  float* v_scales;
} kvb_append_io;

/* NULL when valid, else the first failed rule's message. */
const char* kvb_append_shape_error(const kvb_append_shape* s);
int kvb_append_kv(const kvb_append_shape* s, const kvb_append_io* io, void* stream);

/* Extension with no counterpart in the reference library, for callers that
 * cannot allocate device memory (code under hipGraph capture, tight serving
 * loops, harnesses that forbid hipMalloc): kvb_decode_attention_fused with its
 * scratch -- the split partials and the merge counters -- taken from a fixed
 * 8 MiB device array inside the library instead of caller buffers.  Same
 * kernels, results bitwise equal to kvb_decode_attention_fused.  The array
 * holds a fixed region of 512 counter words (the most a single launch uses)
 * and then the partials; a call whose kvb_scratch_elements_ex floats exceed
 * the remaining 8 MiB - 2 KiB is rejected with KVB_EINVAL.  The array is per
 * device and shared by every call on that device, which leaves the counters
 * zero and the partials as they were: calls that overlap on one device
 * (several streams or host threads) race.  Allocates nothing. */
int kvb_decode_attention_noalloc(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens, float* m,
                                 float* l, float* n, void* out, int out_type, void* stream);

/* Extension (diagnostic): which split kernel kvb_split_attention would run for
 * these arguments: KVB_KERNEL_TILED_MFMA or KVB_KERNEL_GENERIC; 0 if invalid. */
int kvb_selected_kernel(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens);
/* Extension (diagnostic): name of the kernel instance kvb_split_attention
 * (fused = 0) or kvb_decode_attention_fused (fused != 0) would launch, as
 * rocprofv3 reports it, e.g. "split_i8_kernel<128,8,2,true,4,false,false,false>"; "" if
 * the arguments are invalid.  Points to thread-local or static storage. */
const char* kvb_selected_kernel_name(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens,
                                     int fused);

/* Extension (diagnostic): kvb_decode_attention_fused with formal agent-scope
 * release / acquire fences around the merge ticket (a memory-model-formal
 * ordering of the partials; the default call gets the same ordering from
 * agent-scope atomic partial stores and loads, without the L2 write-back and
 * invalidate these fences add).  Same arguments and results, bitwise; only
 * the eight-wave dim-128 single launch (<= 4 head-rows per kv head, pages of
 * >= 64 tokens, splits of >= 16 tiles) has an instance, other calls return
 * KVB_EINVAL.  For measuring that ordering choice, not for production use. */
int kvb_decode_attention_fused_fenced(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens,
                                      float* scratch, uint32_t* counters, float* m, float* l, float* n, void* out,
                                      int out_type, void* stream);
/* Extension (diagnostic, no counterpart in the reference library): streams
 * `bytes` (a multiple of 16) of device memory with non-temporal 16-byte loads
 * over `blocks` work-groups of 512 threads (contiguous runs of 8 KiB items per
 * work-group), for measuring the device's
 * achievable HBM read bandwidth next to the attention kernels (the role of the
 * reference's stream probe, data/att-bench-65536-v2-07.json:528-541).  `sink`
 * needs `blocks` uint32 and is practically never written. */
int kvb_hbm_read_probe(const void* src, size_t bytes, uint32_t* sink, uint32_t blocks, void* stream);

/* Extension (diagnostic, no counterpart in the reference library): reads the
 * K, V and scale bytes a decode call with these arguments reads, through its
 * page table and with the decode kernels' work split (one work-group of 8
 * waves per split and kv head, 64-token tiles round-robin over the waves),
 * and computes nothing: the read floor of the paged access pattern next to
 * the attention kernels.  Needs int8 KV, dim 64/128/256, page_tokens 16, 32
 * or a multiple of 64, split_tokens and begin multiples of 64, 16-byte
 * aligned K/V.  `sink` needs splits * kv_heads uint32 and is practically
 * never written. */
int kvb_paged_read_probe(const kvb_shape* s, const kvb_device_input* in, uint32_t split_tokens, uint32_t* sink,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVBRIDGE_C_H */
