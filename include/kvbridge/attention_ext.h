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

}  // namespace kvbridge
