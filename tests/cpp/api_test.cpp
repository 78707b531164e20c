// Host-only check of the C++ face of libkvbridge_amd.so: the reference API
// names and signatures (include/kvbridge/attention_shape.h,
// attention_common.h) with the reference exception types
// (src/attention_launch_checks.h:8-23).  Makes no device call: every launch
// below is rejected on the host before anything is enqueued.
#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "kvbridge/attention_ext.h"

static int failures = 0;
static void expect(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s\n", what);
    ++failures;
  }
}

template <class F>
static std::string invalid_message(F&& f) {
  try {
    f();
  } catch (const std::invalid_argument& e) {
    return e.what();
  } catch (...) {
    return "<other exception>";
  }
  return "<no exception>";
}

int main() {
  const kvbridge::Shape base{8, 24, 4, 256, 32, 2048, 65536, 0, 65536, .0625f, true};
  expect(kvbridge::kSplitTokens == 256, "kSplitTokens");
  expect(kvbridge::attention_shape_valid(base), "valid base");
  expect(kvbridge::split_count(base) == 256, "split_count");
  expect(kvbridge::scratch_elements(base) == size_t(192) * 256 * 258, "scratch_elements");
  expect(kvbridge::split_count(base, 2048) == 32, "explicit split_count");
  kvbridge::Shape bad = base;
  bad.scale = NAN;
  expect(kvbridge::attention_shape_error(bad) != nullptr, "NaN scale rejected");
  expect(invalid_message([&] { kvbridge::validate_shape(bad); }) != "<no exception>", "validate_shape throws");
  expect(invalid_message([&] { (void)kvbridge::scratch_elements(bad); }) != "<no exception>",
         "scratch_elements throws invalid_argument");

  kvbridge::DeviceInput none{};
  float* fake = reinterpret_cast<float*>(0x1000);
  expect(invalid_message([&] { kvbridge::launch_attention(base, none, nullptr, fake, fake, fake, nullptr); }) ==
             "scratch, m, l and n must be non-null device buffers",
         "null outputs message");
  expect(invalid_message([&] { kvbridge::launch_attention(base, none, fake, fake, fake, fake, nullptr); }) ==
             "attention input device buffers must be non-null",
         "null inputs message");
  kvbridge::Shape one_row = base;
  one_row.rows = 1;
  kvbridge::DeviceInput some{fake,
                             reinterpret_cast<const int64_t*>(0x2000),
                             reinterpret_cast<const int64_t*>(0x2000),
                             reinterpret_cast<const uint32_t*>(0x2000),
                             reinterpret_cast<const void*>(0x2000),
                             reinterpret_cast<const void*>(0x2000),
                             fake,
                             fake};
  expect(invalid_message([&] { kvbridge::launch_attention_mma(one_row, some, fake, fake, fake, fake, nullptr); }) ==
             "launch_attention_mma requires int8 KV, rows8/group6/dim256/page32 and a page-aligned begin",
         "mma geometry message");
  expect(invalid_message([&] { kvbridge::merge_attention(base, fake, 255, fake, fake, fake, nullptr); }) !=
             "<no exception>",
         "merge split-count mismatch");
  // batched extension: sizing and host-side rejections
  const kvbridge::BatchShape bs{4, 1, 64, 8, 128, 64, 8192, 131072, 4 * 131072, 8192, 2048, 0.0883883f, true};
  expect(kvbridge::batch_shape_error(bs) == nullptr, "valid batch shape");
  expect(kvbridge::batch_split_count(bs) == 64, "batch split count");
  expect(kvbridge::batch_scratch_elements(bs) == size_t(4) * 64 * 64 * 130, "batch scratch elements");
  expect(kvbridge::batch_output_scalar_elements(bs) == 256, "batch output elements");
  kvbridge::BatchShape bad_batch = bs;
  bad_batch.batch = 0;
  expect(invalid_message([&] { (void)kvbridge::batch_split_count(bad_batch); }) == "batch must be in [1,65535]",
         "batch count message");
  kvbridge::BatchInput bnone{};
  expect(invalid_message([&] {
           kvbridge::decode_attention_batched(bs, bnone, fake, nullptr, fake, fake, fake, nullptr,
                                              kvbridge::OutputType::none, nullptr);
         }) == "attention input device buffers must be non-null",
         "batched null inputs message");
  // append extension: host-side rejections
  const kvbridge::AppendShape as{4, 8, 128, 64, 10, 1024, 1024, kvbridge::SourceType::f16};
  expect(invalid_message([&] {
           kvbridge::append_kv(as, fake, fake, nullptr, nullptr, nullptr, fake, fake, nullptr);
         }) == "append buffers must be non-null",
         "append null buffers message");
  kvbridge::AppendShape as_bad = as;
  as_bad.dim = 0;
  expect(invalid_message([&] { kvbridge::append_kv(as_bad, fake, fake, nullptr, nullptr, nullptr, fake, fake, nullptr); }) ==
             "dim must be in [1,256]",
         "append dim message");
  if (failures) return 1;
  std::printf("PASS C++ API host checks\n");
  return 0;
}
