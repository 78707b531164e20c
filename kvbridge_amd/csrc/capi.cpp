// extern "C" boundary (include/kvbridge_c.h): validation, kernel selection
// and launches.  Errors never cross the C ABI as exceptions: each entry point
// returns a status code and leaves the message in a thread-local string.
//
// Validation order and messages follow the reference:
//   validate_outputs / validate_launch  src/attention_launch_checks.h:8-23
//   split-count check of merge          src/attention_shared.cu:371
//   MMA geometry gate                   src/attention_mma.cu:36-38
//   launch error mapping (check_cuda)   src/attention_launch_checks.h:24-27
#include "kvbridge_c.h"

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <stdexcept>
#include <string>

#include "kernels.h"
#include "kvbridge/attention_ext.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* msg) {
  g_error = msg;
  return code;
}

kvbridge::Shape to_shape(const kvb_shape& s) {
  return kvbridge::Shape{s.rows, s.q_heads, s.kv_heads, s.dim, s.page_tokens, s.pages,
                         s.tokens, s.begin, s.end, s.scale, s.int8 != 0};
}

kvbridge::DeviceInput to_input(const kvb_device_input& in) {
  return kvbridge::DeviceInput{in.q, in.q_positions, in.k_positions, in.page_table,
                               in.k, in.v, in.k_scales, in.v_scales};
}

// Returns nullptr when the outputs are acceptable, else the reference message.
const char* outputs_error(const kvbridge::Shape& s, const void* scratch, const void* m,
                          const void* l, const void* n) {
  if (const char* e = kvbridge::attention_shape_error(s)) return e;
  if (!scratch || !m || !l || !n) return "scratch, m, l and n must be non-null device buffers";
  return nullptr;
}

const char* launch_error(const kvbridge::Shape& s, const kvbridge::DeviceInput& in,
                         const void* scratch) {
  if (const char* e = kvbridge::attention_shape_error(s)) return e;
  if (!scratch) return "scratch, m, l and n must be non-null device buffers";
  if (!in.q || !in.q_positions || !in.k_positions || !in.page_table || !in.k || !in.v ||
      (s.int8 && (!in.k_scales || !in.v_scales)))
    return "attention input device buffers must be non-null";
  if (s.int8 && s.dim % 4 == 0 && s.page_tokens % 4 == 0 &&
      ((reinterpret_cast<uintptr_t>(in.k) % 4) || (reinterpret_cast<uintptr_t>(in.v) % 4)))
    return "vectorized INT8 K/V buffers must be 4-byte aligned";
  return nullptr;
}

int hip_status(hipError_t e, const char* op) {
  if (e == hipSuccess) return KVB_OK;
  g_error = std::string(op) + ": " + hipGetErrorString(e);
  return KVB_ERUNTIME;
}

// Split partials for a validated shape with `splits` splits of split_tokens.
int run_split(const kvbridge::Shape& s, const kvbridge::DeviceInput& in, unsigned split_tokens,
              unsigned splits, float* scratch, hipStream_t stream, const char* op) {
  const kvb::SplitArgs a = kvb::make_split_args(s, in, split_tokens, splits, scratch);
  const hipError_t e = kvb::tiled_supported(s, in) ? kvb::launch_split_fast(a, stream)
                                                   : kvb::launch_split_generic(a, s.int8, stream);
  return hip_status(e, op);
}

int run_merge(const kvbridge::Shape& s, const float* scratch, unsigned splits, float* m,
              float* l, float* n, void* out, int out_type, hipStream_t stream, const char* op) {
  const hipError_t e = kvb::launch_merge(s.rows * s.q_heads, s.dim, splits, scratch, m, l, n,
                                         out, out_type, stream);
  return hip_status(e, op);
}

template <class F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const std::invalid_argument& e) {
    return fail(KVB_EINVAL, e.what());
  } catch (const std::exception& e) {
    return fail(KVB_ERUNTIME, e.what());
  } catch (...) {
    return fail(KVB_ERUNTIME, "unknown error");
  }
}

kvbridge::BatchShape to_batch_shape(const kvb_batch_shape& b) {
  return kvbridge::BatchShape{b.batch,      b.rows,         b.q_heads,       b.kv_heads,     b.dim,
                              b.page_tokens, b.pages,        b.max_tokens,    b.total_tokens, b.table_entries,
                              b.split_tokens, b.scale,       b.int8 != 0};
}

// One sequence of max_tokens tokens: the shape the per-sequence kernels see.
kvbridge::Shape batch_sequence_shape(const kvbridge::BatchShape& b) {
  return kvbridge::Shape{b.rows, b.q_heads, b.kv_heads, b.dim, b.page_tokens, b.pages,
                         b.max_tokens, 0, b.max_tokens, b.scale, b.int8};
}

kvbridge::DeviceInput batch_device_input(const kvb_batch_input& in) {
  return kvbridge::DeviceInput{in.q, in.q_positions, in.k_positions, in.page_table,
                               in.k, in.v, in.k_scales, in.v_scales};
}

const char* batch_launch_error(const kvbridge::BatchShape& b, const kvb_batch_input& in, const void* scratch,
                               const void* m, const void* l, const void* n) {
  if (const char* e = kvbridge::batch_shape_error(b)) return e;
  if (!scratch || !m || !l || !n) return "scratch, m, l and n must be non-null device buffers";
  if (!in.q || !in.q_positions || !in.seq_starts || !in.page_offsets || !in.k_positions || !in.page_table ||
      !in.k || !in.v || (b.int8 && (!in.k_scales || !in.v_scales)))
    return "attention input device buffers must be non-null";
  if (b.int8 && b.dim % 4 == 0 && b.page_tokens % 4 == 0 &&
      ((reinterpret_cast<uintptr_t>(in.k) % 4) || (reinterpret_cast<uintptr_t>(in.v) % 4)))
    return "vectorized INT8 K/V buffers must be 4-byte aligned";
  return nullptr;
}

kvb::SplitArgs batch_split_args(const kvbridge::BatchShape& b, const kvb_batch_input& in, float* scratch) {
  const kvbridge::Shape s = batch_sequence_shape(b);
  kvb::SplitArgs a = kvb::make_split_args(s, batch_device_input(in), b.split_tokens,
                                          kvbridge::batch_split_count(b), scratch);
  a.seq_starts = in.seq_starts;
  a.page_offsets = in.page_offsets;
  a.batch = b.batch;
  a.total_tokens = b.total_tokens;
  a.table_entries = b.table_entries;
  a.max_tokens = b.max_tokens;
  return a;
}

// The batched split kernel: int8 MFMA where it applies, else the generic one.
bool batch_uses_i8(const kvbridge::BatchShape& b, const kvb_batch_input& in, const kvb::SplitArgs& a) {
  return kvb::tiled_supported(batch_sequence_shape(b), batch_device_input(in)) && kvb::i8_supported(a);
}

}  // namespace

namespace kvb {

int set_error(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

SplitArgs make_split_args(const kvbridge::Shape& s, const kvbridge::DeviceInput& in,
                          unsigned split_tokens, unsigned splits, float* scratch) {
  SplitArgs a{};
  a.q = in.q;
  a.q_positions = in.q_positions;
  a.k_positions = in.k_positions;
  a.page_table = in.page_table;
  a.k = in.k;
  a.v = in.v;
  a.k_scales = in.k_scales;
  a.v_scales = in.v_scales;
  a.scratch = scratch;
  a.rows = s.rows;
  a.q_heads = s.q_heads;
  a.kv_heads = s.kv_heads;
  a.group = s.q_heads / s.kv_heads;
  a.dim = s.dim;
  a.page_tokens = s.page_tokens;
  a.pages = s.pages;
  a.begin = s.begin;
  a.end = s.end;
  a.split_tokens = split_tokens;
  a.splits = splits;
  a.scale = s.scale;
  return a;
}

static bool force_f16() {
  static const bool f = [] {
    const char* e = std::getenv("KVB_SPLIT_IMPL");
    return e && std::string(e) == "f16";
  }();
  return f;
}

hipError_t launch_split_fast(const SplitArgs& a, hipStream_t stream) {
  if (!force_f16() && i8_supported(a)) return launch_split_i8(a, stream);
  if (!force_f16() && i8_rows_supported(a)) return launch_split_i8_rows(a, stream);
  return launch_split_lds(a, stream);
}

const char* split_kernel_name(const SplitArgs& a, bool tiled, bool int8) {
  if (!tiled) {
    if (a.seq_starts) return int8 ? "split_generic_kernel<true, true>" : "split_generic_kernel<false, true>";
    return int8 ? "split_generic_kernel<true, false>" : "split_generic_kernel<false, false>";
  }
  if (!force_f16() && i8_supported(a)) return i8_kernel_name(a);
  if (!force_f16() && i8_rows_supported(a)) return i8_rows_kernel_name(a);
  return lds_kernel_name(a);
}

bool tiled_supported(const kvbridge::Shape& s, const kvbridge::DeviceInput& in) {
  if (!s.int8) return false;
  if (s.dim != 64 && s.dim != 128 && s.dim != 256) return false;
  if (s.page_tokens % 16 != 0) return false;
  const uint64_t head_rows = uint64_t(s.rows) * (s.q_heads / s.kv_heads);
  if (uint64_t(s.kv_heads) * ((head_rows + 15) / 16) > 65535) return false;  // grid.y
  const auto al = [](const void* p, uintptr_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  return al(in.k, 16) && al(in.v, 16) && al(in.q, 16) && al(in.k_scales, 4) && al(in.v_scales, 4);
}

}  // namespace kvb

extern "C" {

const char* kvb_last_error(void) { return g_error.c_str(); }

uint32_t kvb_split_tokens(void) { return kvbridge::kSplitTokens; }

const char* kvb_shape_error(const kvb_shape* s) {
  if (!s) return "shape pointer must be non-null";
  return kvbridge::attention_shape_error(to_shape(*s));
}

int kvb_shape_valid(const kvb_shape* s) {
  return s && kvbridge::attention_shape_valid(to_shape(*s)) ? 1 : 0;
}

int kvb_split_count(const kvb_shape* s, uint32_t* splits) {
  return guarded([&]() -> int {
    if (!s || !splits) return fail(KVB_EINVAL, "null argument");
    *splits = kvbridge::split_count(to_shape(*s));
    return KVB_OK;
  });
}

int kvb_scratch_elements(const kvb_shape* s, size_t* elements) {
  return guarded([&]() -> int {
    if (!s || !elements) return fail(KVB_EINVAL, "null argument");
    *elements = kvbridge::scratch_elements(to_shape(*s));
    return KVB_OK;
  });
}

int kvb_output_scalar_elements(const kvb_shape* s, size_t* elements) {
  return guarded([&]() -> int {
    if (!s || !elements) return fail(KVB_EINVAL, "null argument");
    *elements = kvbridge::output_scalar_elements(to_shape(*s));
    return KVB_OK;
  });
}

int kvb_output_numerator_elements(const kvb_shape* s, size_t* elements) {
  return guarded([&]() -> int {
    if (!s || !elements) return fail(KVB_EINVAL, "null argument");
    *elements = kvbridge::output_numerator_elements(to_shape(*s));
    return KVB_OK;
  });
}

int kvb_mma_supported(const kvb_shape* s) {
  return s && kvbridge::attention_mma_supported(to_shape(*s)) ? 1 : 0;
}

int kvb_preload_attention_reference_kernels(void) {
  hipError_t e = kvb::preload_generic();
  if (e == hipSuccess) e = kvb::preload_i8();
  if (e == hipSuccess) e = kvb::preload_i8_rows();
  if (e == hipSuccess) e = kvb::preload_lds();
  if (e == hipSuccess) e = kvb::preload_merge();
  if (e == hipSuccess) e = kvb::preload_append();
  return int(e);
}

int kvb_preload_attention_mma_kernels(void) {
  // The dense multi-row geometry runs on the tiled MFMA kernel; any gfx950
  // device qualifies.  Checks that a device is current and the code object
  // holds the kernels for it.
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return int(e);
  e = kvb::preload_lds();
  if (e == hipSuccess) e = kvb::preload_i8_rows();
  if (e == hipSuccess) e = kvb::preload_merge();
  return int(e);
}

int kvb_preload_attention_kernels(void) {
  const int e = kvb_preload_attention_reference_kernels();
  return e != 0 ? e : kvb_preload_attention_mma_kernels();
}

int kvb_launch_attention(const kvb_shape* sp, const kvb_device_input* ip, float* scratch,
                         float* m, float* l, float* n, void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip) return fail(KVB_EINVAL, "shape and input descriptors must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    const kvbridge::DeviceInput in = to_input(*ip);
    if (const char* e = outputs_error(s, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (const char* e = launch_error(s, in, scratch)) return fail(KVB_EINVAL, e);
    const unsigned splits = kvbridge::split_count(s);
    const auto st = static_cast<hipStream_t>(stream);
    // Launch-failure messages name the reference's launches
    // (src/attention_shared.cu:354-365): its shared-group kernel serves
    // group <= 8, its legacy per-head kernel larger groups.
    const bool legacy = s.q_heads / s.kv_heads > 8u;
    int rc = run_split(s, in, kvbridge::kSplitTokens, splits, scratch, st,
                       legacy ? "reference legacy split launch" : "reference split launch");
    if (rc != KVB_OK) return rc;
    return run_merge(s, scratch, splits, m, l, n, nullptr, KVB_OUT_NONE, st, "reference merge launch");
  });
}

int kvb_launch_attention_mma(const kvb_shape* sp, const kvb_device_input* ip, float* scratch,
                             float* m, float* l, float* n, void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip) return fail(KVB_EINVAL, "shape and input descriptors must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    const kvbridge::DeviceInput in = to_input(*ip);
    if (const char* e = outputs_error(s, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (const char* e = launch_error(s, in, scratch)) return fail(KVB_EINVAL, e);
    if (!kvbridge::attention_mma_supported(s))
      return fail(KVB_EINVAL,
                  "launch_attention_mma requires int8 KV, rows8/group6/dim256/page32 and a page-aligned begin");
    // Current-device check before the launch (src/attention_mma.cu:39).
    int device = 0;
    if (const int rc = hip_status(hipGetDevice(&device), "MMA current-context preparation"); rc != KVB_OK)
      return rc;
    // The geometry always qualifies for the tiled MFMA kernel; buffers that
    // are 4- but not 16-byte aligned take the generic kernel (same results).
    const unsigned splits = kvbridge::split_count(s);
    const auto st = static_cast<hipStream_t>(stream);
    int rc = run_split(s, in, kvbridge::kSplitTokens, splits, scratch, st, "MMA split launch");
    if (rc != KVB_OK) return rc;
    return run_merge(s, scratch, splits, m, l, n, nullptr, KVB_OUT_NONE, st, "attention merge launch");
  });
}

int kvb_merge_attention(const kvb_shape* sp, const float* scratch, uint32_t splits, float* m,
                        float* l, float* n, void* stream) {
  return guarded([&]() -> int {
    if (!sp) return fail(KVB_EINVAL, "shape descriptor must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    if (const char* e = outputs_error(s, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (splits != kvbridge::split_count(s))
      return fail(KVB_EINVAL, "merge split count does not match shape");
    return run_merge(s, scratch, splits, m, l, n, nullptr, KVB_OUT_NONE,
                     static_cast<hipStream_t>(stream), "attention merge launch");
  });
}

int kvb_split_count_ex(const kvb_shape* s, uint32_t split_tokens, uint32_t* splits) {
  return guarded([&]() -> int {
    if (!s || !splits) return fail(KVB_EINVAL, "null argument");
    *splits = kvbridge::split_count(to_shape(*s), split_tokens);
    return KVB_OK;
  });
}

int kvb_scratch_elements_ex(const kvb_shape* s, uint32_t split_tokens, size_t* elements) {
  return guarded([&]() -> int {
    if (!s || !elements) return fail(KVB_EINVAL, "null argument");
    *elements = kvbridge::scratch_elements(to_shape(*s), split_tokens);
    return KVB_OK;
  });
}

int kvb_split_attention(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens,
                        float* scratch, void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip) return fail(KVB_EINVAL, "shape and input descriptors must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    const kvbridge::DeviceInput in = to_input(*ip);
    if (const char* e = launch_error(s, in, scratch)) return fail(KVB_EINVAL, e);
    const unsigned splits = kvbridge::split_count(s, split_tokens);
    return run_split(s, in, split_tokens, splits, scratch, static_cast<hipStream_t>(stream),
                     "split launch");
  });
}

int kvb_merge_finalize(const kvb_shape* sp, const float* scratch, uint32_t splits, float* m,
                       float* l, float* n, void* out, int out_type, void* stream) {
  return guarded([&]() -> int {
    if (!sp) return fail(KVB_EINVAL, "shape descriptor must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    if (const char* e = outputs_error(s, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (splits == 0 || splits > 65535) return fail(KVB_EINVAL, "split count must be in [1,65535]");
    if (out_type != KVB_OUT_NONE && out_type != KVB_OUT_F32 && out_type != KVB_OUT_F16)
      return fail(KVB_EINVAL, "unknown output type");
    if (out_type != KVB_OUT_NONE && !out) return fail(KVB_EINVAL, "output buffer must be non-null");
    return run_merge(s, scratch, splits, m, l, n, out, out_type, static_cast<hipStream_t>(stream),
                     "attention merge launch");
  });
}

int kvb_decode_attention(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens,
                         float* scratch, float* m, float* l, float* n, void* out, int out_type,
                         void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip) return fail(KVB_EINVAL, "shape and input descriptors must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    const kvbridge::DeviceInput in = to_input(*ip);
    if (const char* e = outputs_error(s, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (const char* e = launch_error(s, in, scratch)) return fail(KVB_EINVAL, e);
    if (out_type != KVB_OUT_NONE && out_type != KVB_OUT_F32 && out_type != KVB_OUT_F16)
      return fail(KVB_EINVAL, "unknown output type");
    if (out_type != KVB_OUT_NONE && !out) return fail(KVB_EINVAL, "output buffer must be non-null");
    const unsigned splits = kvbridge::split_count(s, split_tokens);
    const auto st = static_cast<hipStream_t>(stream);
    int rc = run_split(s, in, split_tokens, splits, scratch, st, "split launch");
    if (rc != KVB_OK) return rc;
    return run_merge(s, scratch, splits, m, l, n, out, out_type, st, "attention merge launch");
  });
}

int kvb_decode_attention_fused(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens,
                               float* scratch, uint32_t* counters, float* m, float* l, float* n, void* out,
                               int out_type, void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip) return fail(KVB_EINVAL, "shape and input descriptors must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    const kvbridge::DeviceInput in = to_input(*ip);
    if (const char* e = outputs_error(s, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (const char* e = launch_error(s, in, scratch)) return fail(KVB_EINVAL, e);
    if (!counters) return fail(KVB_EINVAL, "counters must be a non-null device buffer");
    if (out_type != KVB_OUT_NONE && out_type != KVB_OUT_F32 && out_type != KVB_OUT_F16)
      return fail(KVB_EINVAL, "unknown output type");
    if (out_type != KVB_OUT_NONE && !out) return fail(KVB_EINVAL, "output buffer must be non-null");
    const unsigned splits = kvbridge::split_count(s, split_tokens);
    const auto st = static_cast<hipStream_t>(stream);
    kvb::SplitArgs a = kvb::make_split_args(s, in, split_tokens, splits, scratch);
    if (kvb::tiled_supported(s, in) && kvb::i8_fusable(a)) {
      a.counters = counters;
      a.m = m;
      a.l = l;
      a.n = n;
      a.out = out;
      a.out_type = out_type;
      return hip_status(kvb::launch_split_i8(a, st), "fused decode launch");
    }
    int rc = run_split(s, in, split_tokens, splits, scratch, st, "split launch");
    if (rc != KVB_OK) return rc;
    return run_merge(s, scratch, splits, m, l, n, out, out_type, st, "attention merge launch");
  });
}

int kvb_decode_attention_fused_fenced(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens,
                                      float* scratch, uint32_t* counters, float* m, float* l, float* n, void* out,
                                      int out_type, void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip) return fail(KVB_EINVAL, "shape and input descriptors must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    const kvbridge::DeviceInput in = to_input(*ip);
    if (const char* e = outputs_error(s, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (const char* e = launch_error(s, in, scratch)) return fail(KVB_EINVAL, e);
    if (!counters) return fail(KVB_EINVAL, "counters must be a non-null device buffer");
    if (out_type != KVB_OUT_NONE && out_type != KVB_OUT_F32 && out_type != KVB_OUT_F16)
      return fail(KVB_EINVAL, "unknown output type");
    if (out_type != KVB_OUT_NONE && !out) return fail(KVB_EINVAL, "output buffer must be non-null");
    const unsigned splits = kvbridge::split_count(s, split_tokens);
    kvb::SplitArgs a = kvb::make_split_args(s, in, split_tokens, splits, scratch);
    a.counters = counters;
    a.m = m;
    a.l = l;
    a.n = n;
    a.out = out;
    a.out_type = out_type;
    if (!kvb::tiled_supported(s, in) || !kvb::i8_fenced_supported(a))
      return fail(KVB_EINVAL,
                  "the fenced diagnostic call covers only the eight-wave dim-128 single launch "
                  "(<= 4 head-rows per kv head, pages of >= 64 tokens, splits of >= 16 tiles)");
    return hip_status(kvb::launch_split_i8_fenced(a, static_cast<hipStream_t>(stream)), "fenced decode launch");
  });
}

int kvb_hbm_read_probe(const void* src, size_t bytes, uint32_t* sink, uint32_t blocks, void* stream) {
  if (!src || !sink || bytes % 16 != 0 || blocks == 0)
    return fail(KVB_EINVAL, "probe needs non-null 16-byte-multiple source, a sink and blocks > 0");
  return hip_status(kvb::launch_read_probe(src, bytes, sink, blocks, static_cast<hipStream_t>(stream)),
                    "read probe launch");
}

int kvb_paged_read_probe(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens, uint32_t* sink,
                         void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip || !sink) return fail(KVB_EINVAL, "shape, input and sink must be non-null");
    const kvbridge::Shape s = to_shape(*sp);
    const kvbridge::DeviceInput in = to_input(*ip);
    if (const char* e = launch_error(s, in, sink)) return fail(KVB_EINVAL, e);
    const auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (!s.int8 || (s.dim != 64 && s.dim != 128 && s.dim != 256) || (s.page_tokens % 64 != 0 && s.page_tokens != 16 && s.page_tokens != 32) || split_tokens % 64 != 0 ||
        s.begin % 64 != 0 || !al16(in.k) || !al16(in.v))
      return fail(KVB_EINVAL,
                  "paged probe needs int8 KV, dim 64/128/256, pages of 16, 32 or a multiple of 64 tokens, "
                  "64-token-aligned splits and begin, "
                  "16-byte aligned K/V");
    const unsigned splits = kvbridge::split_count(s, split_tokens);
    return hip_status(kvb::launch_paged_read_probe(in.page_table, in.k, in.v, in.k_scales, in.v_scales, s.kv_heads,
                                                   s.dim, s.page_tokens, s.pages, s.begin, s.end, split_tokens,
                                                   splits, sink, static_cast<hipStream_t>(stream)),
                      "paged read probe launch");
  });
}

int kvb_selected_kernel(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens) {
  if (!sp || !ip || split_tokens == 0) return 0;
  const kvbridge::Shape s = to_shape(*sp);
  if (!kvbridge::attention_shape_valid(s)) return 0;
  return kvb::tiled_supported(s, to_input(*ip)) ? KVB_KERNEL_TILED_MFMA : KVB_KERNEL_GENERIC;
}

const char* kvb_selected_kernel_name(const kvb_shape* sp, const kvb_device_input* ip, uint32_t split_tokens,
                                     int fused) {
  if (!sp || !ip || split_tokens == 0) return "";
  const kvbridge::Shape s = to_shape(*sp);
  if (!kvbridge::attention_shape_valid(s)) return "";
  const kvbridge::DeviceInput in = to_input(*ip);
  unsigned splits = 0;
  try {
    splits = kvbridge::split_count(s, split_tokens);
  } catch (...) {
    return "";
  }
  kvb::SplitArgs a = kvb::make_split_args(s, in, split_tokens, splits, nullptr);
  static uint32_t dummy_counter;  // only its non-nullness is read
  if (fused && kvb::tiled_supported(s, in) && kvb::i8_fusable(a)) a.counters = &dummy_counter;
  return kvb::split_kernel_name(a, kvb::tiled_supported(s, in), s.int8);
}

const char* kvb_batch_shape_error(const kvb_batch_shape* s) {
  if (!s) return "shape pointer must be non-null";
  return kvbridge::batch_shape_error(to_batch_shape(*s));
}

int kvb_batch_split_count(const kvb_batch_shape* s, uint32_t* splits) {
  return guarded([&]() -> int {
    if (!s || !splits) return fail(KVB_EINVAL, "shape and output pointers must be non-null");
    *splits = kvbridge::batch_split_count(to_batch_shape(*s));
    return KVB_OK;
  });
}

int kvb_batch_scratch_elements(const kvb_batch_shape* s, size_t* elements) {
  return guarded([&]() -> int {
    if (!s || !elements) return fail(KVB_EINVAL, "shape and output pointers must be non-null");
    *elements = kvbridge::batch_scratch_elements(to_batch_shape(*s));
    return KVB_OK;
  });
}

int kvb_batch_output_scalar_elements(const kvb_batch_shape* s, size_t* elements) {
  return guarded([&]() -> int {
    if (!s || !elements) return fail(KVB_EINVAL, "shape and output pointers must be non-null");
    *elements = kvbridge::batch_output_scalar_elements(to_batch_shape(*s));
    return KVB_OK;
  });
}

int kvb_decode_attention_batched(const kvb_batch_shape* sp, const kvb_batch_input* ip, float* scratch,
                                 uint32_t* counters, float* m, float* l, float* n, void* out, int out_type,
                                 void* stream) {
  return guarded([&]() -> int {
    if (!sp || !ip) return fail(KVB_EINVAL, "shape and input descriptors must be non-null");
    const kvbridge::BatchShape b = to_batch_shape(*sp);
    if (const char* e = batch_launch_error(b, *ip, scratch, m, l, n)) return fail(KVB_EINVAL, e);
    if (out_type != KVB_OUT_NONE && out_type != KVB_OUT_F32 && out_type != KVB_OUT_F16)
      return fail(KVB_EINVAL, "unknown output type");
    if (out_type != KVB_OUT_NONE && !out) return fail(KVB_EINVAL, "output buffer must be non-null");
    const auto st = static_cast<hipStream_t>(stream);
    kvb::SplitArgs a = batch_split_args(b, *ip, scratch);
    const bool i8 = batch_uses_i8(b, *ip, a);
    if (i8 && counters && kvb::i8_fusable(a)) {
      a.counters = counters;
      a.m = m;
      a.l = l;
      a.n = n;
      a.out = out;
      a.out_type = out_type;
      return hip_status(kvb::launch_split_i8(a, st), "fused batched decode launch");
    }
    const hipError_t e = i8 ? kvb::launch_split_i8(a, st) : kvb::launch_split_generic(a, b.int8, st);
    if (const int rc = hip_status(e, "batched split launch"); rc != KVB_OK) return rc;
    const uint32_t row_heads = b.batch * b.rows * b.q_heads;
    return hip_status(kvb::launch_merge(row_heads, b.dim, a.splits, scratch, m, l, n, out, out_type, st),
                      "batched merge launch");
  });
}

const char* kvb_batch_kernel_name(const kvb_batch_shape* sp, const kvb_batch_input* ip, int fused) {
  if (!sp || !ip) return "";
  const kvbridge::BatchShape b = to_batch_shape(*sp);
  if (kvbridge::batch_shape_error(b)) return "";
  kvb::SplitArgs a = batch_split_args(b, *ip, nullptr);
  const bool i8 = batch_uses_i8(b, *ip, a);
  static uint32_t dummy_counter;  // only its non-nullness is read
  if (fused && i8 && kvb::i8_fusable(a)) a.counters = &dummy_counter;
  return kvb::split_kernel_name(a, i8, b.int8);
}

const char* kvb_append_shape_error(const kvb_append_shape* s) {
  if (!s) return "shape pointer must be non-null";
  if (s->kv_heads == 0 || s->page_tokens == 0 || s->pages == 0)
    return "kv_heads, page_tokens and pages must be positive";
  if (s->dim < 1 || s->dim > 256) return "dim must be in [1,256]";
  const uint64_t extent = uint64_t(s->pages) * s->kv_heads * s->page_tokens * s->dim;
  if (extent > 0xffffffffull) return "physical KV extent exceeds 32-bit kernel offsets";
  if (s->src_type != KVB_SRC_F32 && s->src_type != KVB_SRC_F16 && s->src_type != KVB_SRC_BF16)
    return "unknown source element type";
  if (uint64_t(s->k_stride) < uint64_t(s->kv_heads) * s->dim || uint64_t(s->v_stride) < uint64_t(s->kv_heads) * s->dim)
    return "token stride must cover kv_heads * dim elements";
  return nullptr;
}

int kvb_append_kv(const kvb_append_shape* s, const kvb_append_io* io, void* stream) {
  return guarded([&]() -> int {
    if (!s || !io) return fail(KVB_EINVAL, "shape and buffer descriptors must be non-null");
    if (const char* e = kvb_append_shape_error(s)) return fail(KVB_EINVAL, e);
    if (s->tokens == 0) return KVB_OK;
    if (!io->k_new || !io->v_new || !io->slots || !io->k || !io->v || !io->k_scales || !io->v_scales)
      return fail(KVB_EINVAL, "append buffers must be non-null");
    const uintptr_t el = s->src_type == KVB_SRC_F32 ? 4 : 2;
    if (reinterpret_cast<uintptr_t>(io->k_new) % el || reinterpret_cast<uintptr_t>(io->v_new) % el)
      return fail(KVB_EINVAL, "source rows must be aligned to their element size");
    kvb::AppendArgs a{};
    a.k_new = io->k_new;
    a.v_new = io->v_new;
    a.slots = io->slots;
    a.k = io->k;
    a.v = io->v;
    a.k_scales = io->k_scales;
    a.v_scales = io->v_scales;
    a.tokens = s->tokens;
    a.kv_heads = s->kv_heads;
    a.dim = s->dim;
    a.page_tokens = s->page_tokens;
    a.pages = s->pages;
    a.k_stride = s->k_stride;
    a.v_stride = s->v_stride;
    a.src_type = int(s->src_type);
    return hip_status(kvb::launch_append(a, static_cast<hipStream_t>(stream)), "kv append launch");
  });
}

}  // extern "C"
