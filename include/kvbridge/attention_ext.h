#pragma once
// Additive extensions to the reference API (no counterpart in the reference's
// include/kvbridge): a caller-chosen split size, a fused merge + normalize
// step with fp16/fp32 output, and a single decode-attention call.  The
// reference entry points in attention_common.h are unchanged; these exist
// because the decode workloads ask for split counts other than
// end-begin / kSplitTokens and for a normalized fp16 output.
#include "kvbridge/attention_common.h"

namespace kvbridge {

// Output element type of the normalize step.
enum class OutputType : int { none = 0, f32 = 1, f16 = 2 };

// Splits over [begin, end) when each split covers split_tokens tokens
// (max(1, ceil((end - begin) / split_tokens))).  Validates the shape first;
// throws std::invalid_argument for an invalid shape, split_tokens == 0 or more
// than 65535 splits.
unsigned split_count(const Shape&, unsigned split_tokens);
size_t scratch_elements(const Shape&, unsigned split_tokens);

// Split partials only (same scratch layout as launch_attention, with
// split_count(s, split_tokens) splits).
void launch_split_attention(const Shape&, const DeviceInput&, unsigned split_tokens,
                            float* scratch, hipStream_t stream);

// LSE merge of `splits` partials into m/l/n, and when out_type != none also
// out[rh * dim + d] = l > 0 ? n / l : 0 as fp32 or fp16 (the normalized
// attention output; the zero row is the empty-row convention).
void merge_finalize_attention(const Shape&, const float* scratch, unsigned splits,
                              float* m, float* l, float* n, void* out,
                              OutputType out_type, hipStream_t stream);

// launch_split_attention followed by merge_finalize_attention on one stream.
void decode_attention(const Shape&, const DeviceInput&, unsigned split_tokens,
                      float* scratch, float* m, float* l, float* n, void* out,
                      OutputType out_type, hipStream_t stream);

// ---- batched ragged decode: many independent sequences over one paged pool.
// Sequence b has `rows` query rows (q_heads heads each, sharing its KV) that
// attend to its own tokens [0, T_b): T_b = seq_starts[b+1] - seq_starts[b],
// its key positions are k_positions[seq_starts[b] ..], and its logical page
// p is physical page page_table[page_offsets[b] + p] of the shared pool.
// Each sequence runs max(1, ceil(T_b / split_tokens)) splits; the partial
// stride per sequence is batch_split_count (the split count of max_tokens),
// and splits past a sequence's own count hold empty partials (two-launch
// path; the single launch leaves them untouched and packs its own partials
// in an internal layout of the same size).  The device
// metadata is read by the kernels (the call is graph-capturable with
// changing lengths); indices are clamped to total_tokens / table_entries and
// T_b to max_tokens, so a malformed batch cannot read out of bounds.
struct BatchShape {
  unsigned batch, rows, q_heads, kv_heads, dim, page_tokens, pages;
  unsigned max_tokens;     // bound on every T_b: sizes the grid and the scratch
  unsigned total_tokens;   // k_positions entries
  unsigned table_entries;  // page_table entries
  unsigned split_tokens;   // tokens per split
  float scale;
  bool int8;
};

struct BatchInput {
  const float* q;               // [batch][rows][q_heads][dim]
  const int64_t* q_positions;   // [batch][rows]
  const uint32_t* seq_starts;   // [batch + 1], nondecreasing
  const uint32_t* page_offsets; // [batch]
  const int64_t* k_positions;   // [total_tokens], nondecreasing within a sequence
  const uint32_t* page_table;   // [table_entries]
  const void* k;                // shared pool, layouts as DeviceInput
  const void* v;
  const float* k_scales;
  const float* v_scales;
};

// nullptr when valid, else the first failed rule (never throws).
const char* batch_shape_error(const BatchShape&) noexcept;
// Partial stride per sequence (split count of max_tokens); validates.
unsigned batch_split_count(const BatchShape&);
// batch * rows * q_heads * batch_split_count * (dim + 2) floats; validates.
size_t batch_scratch_elements(const BatchShape&);
// batch * rows * q_heads (m, l); times dim for n and out; validates.
size_t batch_output_scalar_elements(const BatchShape&);

// Split partials + LSE merge (+ normalized output) of every sequence.  With
// counters (batch * kv_heads uint32, zero before the first call and left
// zero) the int8-MFMA kernel serves the whole call in one launch where it
// supports the shape; with counters == nullptr, or otherwise, split and merge
// run as two launches.
void decode_attention_batched(const BatchShape&, const BatchInput&, float* scratch,
                              uint32_t* counters, float* m, float* l, float* n, void* out,
                              OutputType out_type, hipStream_t stream);

// ---- paged INT8 KV append: the write side of the cache layout.
// New token t, kv head h: the rows k_new / v_new[t * stride + h * dim + d]
// (fp32, fp16 or bf16) are quantized with scale = absmax / 127 (1 for an
// all-zero row) and code = clamp(rint(x / scale), -127, 127) in IEEE fp32,
// and stored at physical slot slots[t] (page = slot / page_tokens): K
// token-major, V dim-major, scales per (page, kv head, slot).  slots is a
// device array; ids >= pages * page_tokens are skipped.
enum class SourceType : int { f32 = 1, f16 = 2, bf16 = 3 };

struct AppendShape {
  unsigned tokens, kv_heads, dim, page_tokens, pages;
  unsigned k_stride, v_stride;  // elements between consecutive new tokens (>= kv_heads * dim)
  SourceType src_type;
};

// Throws std::invalid_argument for an invalid shape or null buffers,
// std::runtime_error for a launch failure.  Asynchronous on `stream`.
void append_kv(const AppendShape&, const void* k_new, const void* v_new, const uint32_t* slots, int8_t* k,
               int8_t* v, float* k_scales, float* v_scales, hipStream_t stream);

}  // namespace kvbridge
