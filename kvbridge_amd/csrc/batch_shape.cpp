// Validation and sizing of the batched decode call (host only, no HIP).
// The per-sequence shape rules are the reference's (src/attention_shape.cpp:20-46,
// applied to one sequence of max_tokens tokens); the batch adds its own
// bounds on the sequence count, the split count and the metadata sizes.
#include <limits>
#include <stdexcept>

#include "kvbridge/attention_ext.h"

namespace kvbridge {
namespace {

Shape sequence_shape(const BatchShape& b) {
  return Shape{b.rows, b.q_heads, b.kv_heads, b.dim, b.page_tokens, b.pages,
               b.max_tokens, 0, b.max_tokens, b.scale, b.int8};
}

uint64_t batch_splits(const BatchShape& b) {
  return b.max_tokens == 0 ? 1 : (uint64_t(b.max_tokens) + b.split_tokens - 1) / b.split_tokens;
}

void validate(const BatchShape& b) {
  if (const char* e = batch_shape_error(b)) throw std::invalid_argument(e);
}

}  // namespace

const char* batch_shape_error(const BatchShape& b) noexcept {
  if (b.batch == 0 || b.batch > 65535) return "batch must be in [1,65535]";
  if (const char* e = attention_shape_error(sequence_shape(b))) return e;
  if (b.split_tokens == 0) return "split_tokens must be positive";
  if (batch_splits(b) > 65535) return "split count exceeds 65535";
  if (b.total_tokens == 0 || b.table_entries == 0) return "total_tokens and table_entries must be positive";
  const uint64_t row_heads = uint64_t(b.batch) * b.rows * b.q_heads;
  if (row_heads > 0x7fffffffu) return "batch row/head product exceeds the grid limit";
  const uint64_t max_floats = std::numeric_limits<size_t>::max() / sizeof(float);
  if (row_heads * batch_splits(b) > max_floats / (uint64_t(b.dim) + 2)) return "scratch byte size exceeds size_t";
  return nullptr;
}

unsigned batch_split_count(const BatchShape& b) {
  validate(b);
  return unsigned(batch_splits(b));
}

size_t batch_scratch_elements(const BatchShape& b) {
  validate(b);
  return size_t(b.batch) * b.rows * b.q_heads * size_t(batch_splits(b)) * (size_t(b.dim) + 2);
}

size_t batch_output_scalar_elements(const BatchShape& b) {
  validate(b);
  return size_t(b.batch) * b.rows * b.q_heads;
}

}  // namespace kvbridge
