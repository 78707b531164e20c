#pragma once
// Public device API of the MI355X (gfx950) paged INT8-KV split-K decode
// attention library.  Same entry points, argument meaning and error behaviour
// as the reference include/kvbridge/attention_common.h:54-96, with HIP types in
// place of CUDA ones.  Every function here is a thin C++ wrapper over the
// extern "C" layer in include/kvbridge_c.h: it converts status codes back into
// the reference's exception types.
//
// Device memory formats (caller-owned; the library never allocates):
//   q           float[rows * q_heads * dim]      row-major fp32
//   q_positions int64[rows]                      absolute position per query row
//   k_positions int64[tokens]                    absolute position per logical token,
//                                                nondecreasing in logical order
//   page_table  uint32[pages]                    logical page -> physical page (< pages)
//   k           int8[((page * kv_heads + kv) * page_tokens + slot) * dim + d]   token-major
//   v           int8[((page * kv_heads + kv) * dim + d) * page_tokens + slot]   dim-major
//   k_scales    float[(page * kv_heads + kv) * page_tokens + slot]
//   v_scales    float[same index as k_scales]
// (fp32 KV, int8 == false: k and v hold float in the same layouts, scales unused.)
//
// A key token t is visible to query row r when begin <= t < end and
// k_positions[t] <= q_positions[r].  Logical token t lives in physical page
// page_table[t / page_tokens] at slot t % page_tokens.
//
// Split partials (floats):
//   scratch[((row * q_heads + head) * splits + split) * (dim + 2) + col]
//   col 0 = split max score, col 1 = sum of exp(score - max) (v-scale free),
//   col 2 + d = sum of exp(score - max) * v_scale * v_code[d].
// merge_attention combines them into m[rh], l[rh], n[rh * dim + d] with
// rh = row * q_heads + head.  The normalized output is n / l where l > 0; an
// empty or fully masked row-head has m = -inf, l = 0, n = 0.
#include <hip/hip_runtime_api.h>
#include <cstddef>
#include <cstdint>
#include "kvbridge/attention_shape.h"

namespace kvbridge {

struct DeviceInput {
  const float* q;
  const int64_t* q_positions;
  const int64_t* k_positions;
  const uint32_t* page_table;
  const void* k;            // int8[] (or float[] when Shape::int8 is false)
  const void* v;
  const float* k_scales;    // ignored for fp32 KV
  const float* v_scales;
};

// Eager kernel-object load on the current device.  Return the first HIP error.
// Reference: attention_common.h:69-72.
hipError_t preload_attention_kernels();
hipError_t preload_attention_reference_kernels();
hipError_t preload_attention_mma_kernels();

// Split partials over kSplitTokens-token splits plus the LSE merge, for any
// valid Shape (int8 or fp32 KV).  Invalid metadata, null or misaligned
// buffers throw std::invalid_argument before anything is enqueued; launch
// failures throw std::runtime_error.  Asynchronous on `stream`.
// Reference: attention_common.h:80-81.
void launch_attention(const Shape&, const DeviceInput&, float* scratch,
                      float* m, float* l, float* n, hipStream_t stream);

// Same outputs for the dense multi-row geometry (attention_mma_supported);
// throws std::invalid_argument for any other shape, with no fallback.
// Reference: attention_common.h:90-91.
void launch_attention_mma(const Shape&, const DeviceInput&, float* scratch,
                          float* m, float* l, float* n, hipStream_t stream);

// LSE merge of kSplitTokens-token split partials; splits must equal
// split_count(shape).  Reference: attention_common.h:95-96.
void merge_attention(const Shape&, const float* scratch, unsigned splits,
                     float* m, float* l, float* n, hipStream_t stream);

}  // namespace kvbridge
