// Check of the C++ face of libkvbridge_amd.so: the reference API names and
// signatures (include/kvbridge/attention_shape.h, attention_common.h) with
// the reference exception types (src/attention_launch_checks.h:8-23).
// Without arguments it makes no device call: every launch below is rejected
// on the host before anything is enqueued.  With --gpu it also calls the
// three preload entry points (reference src/attention_shared.cu:376-387,
// src/attention_mma.cu:13-31), which must return hipSuccess, and runs
// launch_attention on a one-token cache, whose result is known exactly:
// softmax over one visible token gives l = 1 and n = v_code * v_scale.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

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

int main(int argc, char** argv) {
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
  if (argc > 1 && std::strcmp(argv[1], "--gpu") == 0) {
    expect(kvbridge::preload_attention_reference_kernels() == hipSuccess, "preload_attention_reference_kernels");
    expect(kvbridge::preload_attention_mma_kernels() == hipSuccess, "preload_attention_mma_kernels");
    expect(kvbridge::preload_attention_kernels() == hipSuccess, "preload_attention_kernels");
    // One token, one kv head, two query heads, dim 64, page 16: softmax over
    // the single visible token is exactly 1, so l = 1 and n[d] = v[d] * vs.
    const kvbridge::Shape one{1, 2, 1, 64, 16, 1, 1, 0, 1, 0.125f, true};
    std::vector<float> hq(2 * 64, 0.5f);
    const int64_t qpos = 0, kpos = 0;
    const uint32_t table = 0;
    std::vector<int8_t> hk(16 * 64, 3), hv(64 * 16, 0);
    for (int d = 0; d < 64; ++d) hv[d * 16] = int8_t(d - 32);  // slot 0 of dim-major V
    std::vector<float> hks(16, 0.25f), hvs(16, 0.5f);
    float *q, *ks, *vs, *sc, *m, *l, *n;
    int64_t *qp, *kp;
    uint32_t* tb;
    int8_t *k, *v;
    bool ok = hipMalloc(&q, hq.size() * 4) == hipSuccess && hipMalloc(&ks, 64) == hipSuccess &&
              hipMalloc(&vs, 64) == hipSuccess && hipMalloc(&qp, 8) == hipSuccess && hipMalloc(&kp, 8) == hipSuccess &&
              hipMalloc(&tb, 4) == hipSuccess && hipMalloc(&k, hk.size()) == hipSuccess &&
              hipMalloc(&v, hv.size()) == hipSuccess && hipMalloc(&sc, kvbridge::scratch_elements(one) * 4) == hipSuccess &&
              hipMalloc(&m, 8) == hipSuccess && hipMalloc(&l, 8) == hipSuccess && hipMalloc(&n, 2 * 64 * 4) == hipSuccess;
    expect(ok, "device allocations");
    if (!ok) return 1;
    const auto h2d = [](void* dst, const void* src, size_t bytes) {
      return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) == hipSuccess;
    };
    expect(h2d(q, hq.data(), hq.size() * 4) && h2d(ks, hks.data(), 64) && h2d(vs, hvs.data(), 64) &&
               h2d(qp, &qpos, 8) && h2d(kp, &kpos, 8) && h2d(tb, &table, 4) && h2d(k, hk.data(), hk.size()) &&
               h2d(v, hv.data(), hv.size()),
           "uploads");
    const kvbridge::DeviceInput in{q, qp, kp, tb, k, v, ks, vs};
    try {
      kvbridge::launch_attention(one, in, sc, m, l, n, nullptr);
    } catch (const std::exception& e) {
      std::fprintf(stderr, "launch_attention threw: %s\n", e.what());
      ++failures;
    }
    expect(hipDeviceSynchronize() == hipSuccess, "device synchronize");
    float hm[2], hl[2], hn[128];
    expect(hipMemcpy(hm, m, 8, hipMemcpyDeviceToHost) == hipSuccess &&
               hipMemcpy(hl, l, 8, hipMemcpyDeviceToHost) == hipSuccess &&
               hipMemcpy(hn, n, sizeof(hn), hipMemcpyDeviceToHost) == hipSuccess,
           "downloads");
    const float score = 0.125f * 64 * 0.5f * 3 * 0.25f;  // scale * sum_d q * k_code * k_scale
    for (int h = 0; h < 2; ++h) {
      expect(std::fabs(hm[h] - score) <= 1e-5f * score, "m is the single token's score");
      expect(hl[h] == 1.0f, "l = 1");
      for (int d = 0; d < 64; ++d) expect(hn[h * 64 + d] == float(d - 32) * 0.5f, "n = v_code * v_scale");
    }
    for (void* p : {(void*)q, (void*)ks, (void*)vs, (void*)qp, (void*)kp, (void*)tb, (void*)k, (void*)v, (void*)sc,
                    (void*)m, (void*)l, (void*)n})
      hipFree(p);
    if (failures) return 1;
    std::printf("PASS C++ API device checks\n");
  }
  return 0;
}
