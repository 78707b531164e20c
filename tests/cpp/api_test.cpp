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
  if (failures) return 1;
  std::printf("PASS C++ API host checks\n");
  return 0;
}
