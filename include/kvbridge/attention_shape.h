#pragma once
// Shape metadata for paged INT8-KV split-K decode attention, and the sizes the
// caller allocates from it. Host-only: nothing here includes HIP or touches a
// device. Mirrors the reference interface include/kvbridge/attention_shape.h:7-36
// (same names, argument meaning and throw behaviour) so callers drop in.
#include <cstddef>
#include <cstdint>

namespace kvbridge {

// Tokens per split used by the reference-compatible entry points
// (launch_attention / merge_attention).  Reference: attention_shape.h:7.
constexpr unsigned kSplitTokens = 256;

// Field order and types match the reference Shape (attention_shape.h:9-13):
// rows = query rows sharing one KV history, q_heads / kv_heads = GQA heads,
// dim = head dimension, page_tokens = slots per page, pages = page-table length
// (and physical pages allocated), tokens = logical backing length,
// [begin, end) = logical token interval attended, scale = finite score scale,
// int8 = INT8 KV (true) or fp32 KV (false).
struct Shape {
  uint32_t rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, begin, end;
  float scale;
  bool int8;
};

// Metadata validation.  Returns nullptr when the shape is valid, otherwise a
// static message for the first failed rule (rules are checked in a fixed
// order).  Never dereferences device pointers and never calls into HIP.
const char* attention_shape_error(const Shape&) noexcept;
bool attention_shape_valid(const Shape&) noexcept;
// Throws std::invalid_argument(attention_shape_error(s)) for invalid shapes.
void validate_shape(const Shape&);

// Allocation sizes in elements (not bytes).  Each validates first and throws
// std::invalid_argument on an invalid shape.  An empty [begin, end) still has
// one split, which produces m = -inf, l = 0, n = 0.
unsigned split_count(const Shape&);
size_t scratch_elements(const Shape&);           // floats of split partials
size_t output_scalar_elements(const Shape&);     // floats in each of m and l
size_t output_numerator_elements(const Shape&);  // floats in n (and in q)

// Geometry predicate of the dense multi-row entry point launch_attention_mma:
// INT8 KV, rows 8, 6 query heads per KV head, dim 256, 32-token pages and a
// page-aligned begin.  False for invalid shapes.  Reference: attention_shape.cpp:67-70.
bool attention_mma_supported(const Shape&) noexcept;

}  // namespace kvbridge
