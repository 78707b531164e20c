// Shape validation and allocation sizes (host only, no HIP).
// Behaviour follows the reference src/attention_shape.cpp:9-70: the same rules
// in the same order (first failure wins), the same messages, the same sizing
// formulas and the same MMA geometry predicate, so the reference's own
// tests/shape_test.cpp passes against this file unchanged.
#include "kvbridge/attention_shape.h"

#include <cmath>
#include <limits>
#include <stdexcept>

namespace kvbridge {
namespace {

constexpr uint64_t kU32Max = std::numeric_limits<uint32_t>::max();
constexpr uint64_t kMaxSplits = 65535;       // grid-y bound kept from the reference API
constexpr uint64_t kMaxRowHeads = 0x7fffffffu;

// ceil((end - begin) / split_tokens), at least 1; requires begin <= end.
uint64_t splits_of(const Shape& s, uint64_t split_tokens) noexcept {
  const uint64_t len = uint64_t(s.end) - uint64_t(s.begin);
  return len == 0 ? 1 : (len + split_tokens - 1) / split_tokens;
}

// acc *= f, failing instead of exceeding `limit`.
bool scale_within(uint64_t& acc, uint64_t f, uint64_t limit) noexcept {
  if (f != 0 && acc > limit / f) return false;
  acc *= f;
  return true;
}

}  // namespace

const char* attention_shape_error(const Shape& s) noexcept {
  if (s.rows == 0 || s.q_heads == 0 || s.kv_heads == 0)
    return "rows and head counts must be positive";
  if (s.q_heads % s.kv_heads != 0) return "q_heads must be divisible by kv_heads";
  if (s.dim < 1 || s.dim > 256) return "dim must be in [1,256]";
  if (s.page_tokens == 0 || s.pages == 0 || s.tokens == 0)
    return "page_tokens, pages and tokens must be positive";
  if (!(s.begin <= s.end && s.end <= s.tokens)) return "require begin <= end <= tokens";
  if (uint64_t(s.tokens) > uint64_t(s.pages) * uint64_t(s.page_tokens))
    return "tokens exceed allocated page capacity";
  if (!std::isfinite(s.scale)) return "score scale must be finite";
  if (splits_of(s, kSplitTokens) > kMaxSplits) return "range exceeds CUDA grid-y split limit";
  if (uint64_t(s.rows) * uint64_t(s.q_heads) > kMaxRowHeads)
    return "row/head product exceeds CUDA grid-x limit";
  // Physical KV element count pages*kv_heads*page_tokens*dim must fit the
  // 32-bit offsets the kernels use.
  uint64_t kv_elems = s.pages;
  if (!scale_within(kv_elems, s.kv_heads, kU32Max) ||
      !scale_within(kv_elems, s.page_tokens, kU32Max) ||
      !scale_within(kv_elems, s.dim, kU32Max))
    return "physical KV extent exceeds 32-bit kernel offsets";
  const uint64_t max_floats = std::numeric_limits<size_t>::max() / sizeof(float);
  uint64_t partial_floats = uint64_t(s.rows) * uint64_t(s.q_heads);
  if (!scale_within(partial_floats, splits_of(s, kSplitTokens), max_floats) ||
      !scale_within(partial_floats, uint64_t(s.dim) + 2, max_floats))
    return "scratch byte size exceeds size_t";
  if (kv_elems > max_floats ||
      uint64_t(s.tokens) > std::numeric_limits<size_t>::max() / sizeof(int64_t) ||
      uint64_t(s.pages) > std::numeric_limits<size_t>::max() / sizeof(uint32_t))
    return "input byte size exceeds size_t";
  return nullptr;
}

bool attention_shape_valid(const Shape& s) noexcept { return attention_shape_error(s) == nullptr; }

void validate_shape(const Shape& s) {
  if (const char* why = attention_shape_error(s)) throw std::invalid_argument(why);
}

unsigned split_count(const Shape& s) {
  validate_shape(s);
  return unsigned(splits_of(s, kSplitTokens));
}

size_t scratch_elements(const Shape& s) {
  validate_shape(s);
  return size_t(s.rows) * s.q_heads * size_t(splits_of(s, kSplitTokens)) * (size_t(s.dim) + 2);
}

size_t output_scalar_elements(const Shape& s) {
  validate_shape(s);
  return size_t(s.rows) * s.q_heads;
}

size_t output_numerator_elements(const Shape& s) { return output_scalar_elements(s) * s.dim; }

bool attention_mma_supported(const Shape& s) noexcept {
  if (!attention_shape_valid(s)) return false;
  return s.int8 && s.rows == 8 && s.dim == 256 && s.page_tokens == 32 &&
         s.q_heads / s.kv_heads == 6 && s.begin % 32 == 0;
}

// ---- extension: caller-chosen split size -------------------------------

unsigned split_count(const Shape& s, unsigned split_tokens) {
  validate_shape(s);
  if (split_tokens == 0) throw std::invalid_argument("split_tokens must be positive");
  const uint64_t n = splits_of(s, split_tokens);
  if (n > kMaxSplits) throw std::invalid_argument("split count exceeds 65535");
  return unsigned(n);
}

size_t scratch_elements(const Shape& s, unsigned split_tokens) {
  const unsigned n = split_count(s, split_tokens);
  return size_t(s.rows) * s.q_heads * size_t(n) * (size_t(s.dim) + 2);
}

}  // namespace kvbridge
