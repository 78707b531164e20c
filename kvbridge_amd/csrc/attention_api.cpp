// C++ API (include/kvbridge/attention_common.h, attention_ext.h) as a thin
// layer over the extern "C" entry points.  Status codes become the
// reference's exception types: KVB_EINVAL -> std::invalid_argument,
// KVB_ERUNTIME -> std::runtime_error (reference src/attention_launch_checks.h:8-27).
#include <stdexcept>

#include "kvbridge/attention_ext.h"
#include "kvbridge_c.h"

namespace kvbridge {
namespace {

kvb_shape c_shape(const Shape& s) {
  return kvb_shape{s.rows, s.q_heads, s.kv_heads, s.dim, s.page_tokens, s.pages,
                   s.tokens, s.begin, s.end, s.scale, s.int8 ? 1u : 0u};
}

kvb_device_input c_input(const DeviceInput& in) {
  return kvb_device_input{in.q, in.q_positions, in.k_positions, in.page_table,
                          in.k, in.v, in.k_scales, in.v_scales};
}

void check(int rc) {
  if (rc == KVB_OK) return;
  if (rc == KVB_EINVAL) throw std::invalid_argument(kvb_last_error());
  throw std::runtime_error(kvb_last_error());
}

}  // namespace

hipError_t preload_attention_kernels() { return hipError_t(kvb_preload_attention_kernels()); }
hipError_t preload_attention_reference_kernels() {
  return hipError_t(kvb_preload_attention_reference_kernels());
}
hipError_t preload_attention_mma_kernels() { return hipError_t(kvb_preload_attention_mma_kernels()); }

void launch_attention(const Shape& s, const DeviceInput& in, float* scratch, float* m, float* l,
                      float* n, hipStream_t stream) {
  const kvb_shape cs = c_shape(s);
  const kvb_device_input ci = c_input(in);
  check(kvb_launch_attention(&cs, &ci, scratch, m, l, n, stream));
}

void launch_attention_mma(const Shape& s, const DeviceInput& in, float* scratch, float* m,
                          float* l, float* n, hipStream_t stream) {
  const kvb_shape cs = c_shape(s);
  const kvb_device_input ci = c_input(in);
  check(kvb_launch_attention_mma(&cs, &ci, scratch, m, l, n, stream));
}

void merge_attention(const Shape& s, const float* scratch, unsigned splits, float* m, float* l,
                     float* n, hipStream_t stream) {
  const kvb_shape cs = c_shape(s);
  check(kvb_merge_attention(&cs, scratch, splits, m, l, n, stream));
}

void launch_split_attention(const Shape& s, const DeviceInput& in, unsigned split_tokens,
                            float* scratch, hipStream_t stream) {
  const kvb_shape cs = c_shape(s);
  const kvb_device_input ci = c_input(in);
  check(kvb_split_attention(&cs, &ci, split_tokens, scratch, stream));
}

void merge_finalize_attention(const Shape& s, const float* scratch, unsigned splits, float* m,
                              float* l, float* n, void* out, OutputType out_type,
                              hipStream_t stream) {
  const kvb_shape cs = c_shape(s);
  check(kvb_merge_finalize(&cs, scratch, splits, m, l, n, out, int(out_type), stream));
}

void decode_attention(const Shape& s, const DeviceInput& in, unsigned split_tokens,
                      float* scratch, float* m, float* l, float* n, void* out,
                      OutputType out_type, hipStream_t stream) {
  const kvb_shape cs = c_shape(s);
  const kvb_device_input ci = c_input(in);
  check(kvb_decode_attention(&cs, &ci, split_tokens, scratch, m, l, n, out, int(out_type), stream));
}

void decode_attention_batched(const BatchShape& b, const BatchInput& in, float* scratch, uint32_t* counters,
                              float* m, float* l, float* n, void* out, OutputType out_type, hipStream_t stream) {
  const kvb_batch_shape cs{b.batch,      b.rows,         b.q_heads,      b.kv_heads,     b.dim,
                           b.page_tokens, b.pages,        b.max_tokens,   b.total_tokens, b.table_entries,
                           b.split_tokens, b.scale,       b.int8 ? 1u : 0u};
  const kvb_batch_input ci{in.q,          in.q_positions, in.seq_starts, in.page_offsets, in.k_positions,
                           in.page_table, in.k,           in.v,          in.k_scales,     in.v_scales};
  check(kvb_decode_attention_batched(&cs, &ci, scratch, counters, m, l, n, out, int(out_type), stream));
}

void append_kv(const AppendShape& a, const void* k_new, const void* v_new, const uint32_t* slots, int8_t* k,
               int8_t* v, float* k_scales, float* v_scales, hipStream_t stream) {
  const kvb_append_shape cs{a.tokens,   a.kv_heads, a.dim,      a.page_tokens,
                            a.pages,    a.k_stride, a.v_stride, uint32_t(a.src_type)};
  const kvb_append_io io{k_new, v_new, slots, k, v, k_scales, v_scales};
  check(kvb_append_kv(&cs, &io, stream));
}

}  // namespace kvbridge
