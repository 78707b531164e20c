// Host-only check of the C ABI (include/kvbridge_c.h), meant to run under
// AddressSanitizer + UndefinedBehaviorSanitizer (tests/cpp/Makefile
// capi_reject_asan).  No call below reaches the device: every launch is
// rejected on the host before anything is enqueued (the reference's
// invalid_argument path, src/attention_launch_checks.h:8-23), and the shape,
// batch and append rules run over a deterministic sweep of boundary values
// (zero, one, powers of two and their neighbours, 2^31 - 1, 2^32 - 1), which
// exercises every overflow check of the sizing code.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>

#include "kvbridge_c.h"

static int failures = 0;
static long checks = 0;
static void expect(bool ok, const char* what) {
  ++checks;
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s\n", what);
    ++failures;
  }
}

// An error status must come with a message (kvb_last_error).
static void expect_einval(int rc, const char* what) {
  expect(rc == KVB_EINVAL, what);
  const char* e = kvb_last_error();
  expect(e != nullptr && e[0] != '\0', "error message set");
}

static const uint32_t kEdge[] = {0u,      1u,      2u,         3u,          7u,          8u,          16u,
                                 31u,     32u,     63u,        64u,         255u,        256u,        257u,
                                 65535u,  65536u,  0x7fffffffu, 0x80000000u, 0xfffffffeu, 0xffffffffu};
static const size_t kNumEdge = sizeof(kEdge) / sizeof(kEdge[0]);

struct Lcg {
  uint64_t s;
  uint32_t next() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return uint32_t(s >> 33);
  }
  uint32_t edge() { return kEdge[next() % kNumEdge]; }
  uint32_t pick(uint32_t base) {  // half the time a boundary value, else near the base
    return (next() & 1u) ? edge() : base + next() % 3u;
  }
};

static void sweep_shapes() {
  const kvb_shape base = {1, 32, 8, 128, 64, 1024, 65536, 0, 65536, 0.0883883f, 1};
  expect(kvb_shape_valid(&base) == 1, "cfg2 shape valid");
  uint32_t splits = 0;
  expect(kvb_split_count_ex(&base, 2048, &splits) == KVB_OK && splits == 32, "cfg2 splits");
  const float scales[] = {0.f, -1.f, 1e-30f, 3e38f, std::numeric_limits<float>::infinity(),
                          std::numeric_limits<float>::quiet_NaN()};
  Lcg r{0x4B564252ull};
  long valid = 0;
  for (int it = 0; it < 200000; ++it) {
    kvb_shape s = base;
    switch (r.next() % 4) {  // perturb a few fields at a time
      case 0: s.rows = r.pick(1); s.q_heads = r.pick(32); break;
      case 1: s.kv_heads = r.pick(8); s.dim = r.pick(128); s.page_tokens = r.pick(64); break;
      case 2: s.pages = r.pick(1024); s.tokens = r.pick(65536); break;
      default: s.begin = r.pick(0); s.end = r.pick(65536); break;
    }
    if (r.next() % 8 == 0) s.scale = scales[r.next() % 6];
    if (r.next() % 8 == 0) s.int8 = r.next() % 3;
    const char* err = kvb_shape_error(&s);
    const int ok = kvb_shape_valid(&s);
    expect((err == nullptr) == (ok == 1), "shape_error and shape_valid agree");
    valid += ok;
    size_t n1 = 0, n2 = 0, n3 = 0, n4 = 0;
    const int a = kvb_split_count(&s, &splits), b = kvb_scratch_elements(&s, &n1);
    const int c = kvb_output_scalar_elements(&s, &n2), d = kvb_output_numerator_elements(&s, &n3);
    expect((a == KVB_OK) == (ok == 1) && (b == KVB_OK) == (ok == 1), "sizing rejects exactly the invalid shapes");
    expect((c == KVB_OK) == (ok == 1) && (d == KVB_OK) == (ok == 1), "output sizes reject exactly the invalid shapes");
    if (ok) {
      expect(splits >= 1 && splits <= 65535, "split count in the grid range");
      expect(n2 == size_t(s.rows) * s.q_heads && n3 == n2 * s.dim, "output element counts");
      expect(n1 == n2 * splits * (s.dim + 2), "scratch element count");
    }
    (void)kvb_mma_supported(&s);
    const uint32_t st = r.edge();
    const int e = kvb_split_count_ex(&s, st, &splits), f = kvb_scratch_elements_ex(&s, st, &n4);
    expect((e == KVB_OK) == (f == KVB_OK), "explicit split sizing agrees");
    if (e == KVB_OK) expect(st > 0 && splits >= 1 && n4 == n2 * splits * (s.dim + 2), "explicit scratch count");
  }
  expect(valid > 1000, "the sweep reaches valid shapes");
  // null descriptors and outputs
  expect(kvb_shape_error(nullptr) != nullptr && kvb_shape_valid(nullptr) == 0, "null shape");
  expect_einval(kvb_split_count(nullptr, &splits), "split_count null shape");
  expect_einval(kvb_split_count(&base, nullptr), "split_count null output");
  size_t n = 0;
  expect_einval(kvb_scratch_elements(&base, nullptr), "scratch_elements null output");
  expect_einval(kvb_scratch_elements_ex(nullptr, 2048, &n), "scratch_elements_ex null shape");
}

static void sweep_batches() {
  const kvb_batch_shape base = {4, 1, 64, 8, 128, 64, 8192, 131072, 4 * 131072, 8192, 2048, 0.0883883f, 1};
  expect(kvb_batch_shape_error(&base) == nullptr, "cfg4 batch valid");
  Lcg r{0x4B564253ull};
  long valid = 0;
  for (int it = 0; it < 100000; ++it) {
    kvb_batch_shape s = base;
    switch (r.next() % 4) {
      case 0: s.batch = r.pick(4); s.rows = r.pick(1); break;
      case 1: s.q_heads = r.pick(64); s.kv_heads = r.pick(8); s.dim = r.pick(128); break;
      case 2: s.page_tokens = r.pick(64); s.pages = r.pick(8192); s.table_entries = r.pick(8192); break;
      default: s.max_tokens = r.pick(131072); s.total_tokens = r.pick(4 * 131072); s.split_tokens = r.pick(2048); break;
    }
    const bool ok = kvb_batch_shape_error(&s) == nullptr;
    valid += ok;
    uint32_t splits = 0;
    size_t n1 = 0, n2 = 0;
    const int a = kvb_batch_split_count(&s, &splits), b = kvb_batch_scratch_elements(&s, &n1),
              c = kvb_batch_output_scalar_elements(&s, &n2);
    expect((a == KVB_OK) == ok && (b == KVB_OK) == ok && (c == KVB_OK) == ok, "batch sizing rejects exactly the invalid shapes");
    if (ok) expect(n2 == size_t(s.batch) * s.rows * s.q_heads && n1 == n2 * splits * (s.dim + 2), "batch sizes");
  }
  expect(valid > 1000, "the batch sweep reaches valid shapes");
  expect(kvb_batch_shape_error(nullptr) != nullptr, "null batch shape");
}

static void sweep_appends() {
  const kvb_append_shape base = {4096, 8, 128, 64, 1024, 1024, 1024, KVB_SRC_F16};
  expect(kvb_append_shape_error(&base) == nullptr, "append shape valid");
  Lcg r{0x4B564254ull};
  for (int it = 0; it < 100000; ++it) {
    kvb_append_shape s = base;
    switch (r.next() % 3) {
      case 0: s.tokens = r.pick(4096); s.kv_heads = r.pick(8); break;
      case 1: s.dim = r.pick(128); s.page_tokens = r.pick(64); s.pages = r.pick(1024); break;
      default: s.k_stride = r.pick(1024); s.v_stride = r.pick(1024); s.src_type = r.next() % 5; break;
    }
    (void)kvb_append_shape_error(&s);
  }
  expect(kvb_append_shape_error(nullptr) != nullptr, "null append shape");
  kvb_append_io io;
  std::memset(&io, 0, sizeof(io));
  expect_einval(kvb_append_kv(&base, &io, nullptr), "append null buffers");
  expect_einval(kvb_append_kv(nullptr, &io, nullptr), "append null shape");
  expect_einval(kvb_append_kv(&base, nullptr, nullptr), "append null io");
}

static void launches_rejected() {
  // Fake device addresses: never dereferenced, every call fails its host checks first.
  float* f = reinterpret_cast<float*>(0x10000);
  uint32_t* u = reinterpret_cast<uint32_t*>(0x10000);
  const int64_t* p64 = reinterpret_cast<const int64_t*>(0x10000);
  const kvb_shape s = {1, 8, 2, 64, 16, 32, 512, 0, 512, 0.125f, 1};
  const kvb_device_input none = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  const kvb_device_input fake = {f, p64, p64, u, f, f, f, f};
  const kvb_device_input misaligned = {f, p64, p64, u, reinterpret_cast<const void*>(0x10002), f, f, f};
  kvb_shape bad = s;
  bad.rows = 0;
  const kvb_shape* const bad_shapes[] = {&bad, nullptr};
  for (const kvb_shape* sp : bad_shapes) {
    expect_einval(kvb_launch_attention(sp, &fake, f, f, f, f, nullptr), "launch_attention bad shape");
    expect_einval(kvb_launch_attention_mma(sp, &fake, f, f, f, f, nullptr), "launch_attention_mma bad shape");
    expect_einval(kvb_merge_attention(sp, f, 4, f, f, f, nullptr), "merge bad shape");
    expect_einval(kvb_split_attention(sp, &fake, 128, f, nullptr), "split bad shape");
    expect_einval(kvb_merge_finalize(sp, f, 4, f, f, f, f, KVB_OUT_F32, nullptr), "merge_finalize bad shape");
    expect_einval(kvb_decode_attention(sp, &fake, 128, f, f, f, f, f, KVB_OUT_F32, nullptr), "decode bad shape");
    expect_einval(kvb_decode_attention_fused(sp, &fake, 128, f, u, f, f, f, f, KVB_OUT_F32, nullptr),
                  "fused bad shape");
    expect_einval(kvb_decode_attention_noalloc(sp, &fake, 128, f, f, f, f, KVB_OUT_F32, nullptr), "noalloc bad shape");
    expect_einval(kvb_decode_attention_fused_fenced(sp, &fake, 128, f, u, f, f, f, f, KVB_OUT_F32, nullptr),
                  "fenced bad shape");
    expect_einval(kvb_paged_read_probe(sp, &fake, 128, u, nullptr), "paged probe bad shape");
    expect(kvb_selected_kernel(sp, &fake, 128) == 0, "selected_kernel of an invalid shape");
  }
  expect_einval(kvb_launch_attention(&s, &none, f, f, f, f, nullptr), "null inputs");
  expect_einval(kvb_launch_attention(&s, nullptr, f, f, f, f, nullptr), "null input descriptor");
  expect_einval(kvb_launch_attention(&s, &fake, nullptr, f, f, f, nullptr), "null scratch");
  expect_einval(kvb_launch_attention(&s, &misaligned, f, f, f, f, nullptr), "misaligned K");
  expect(std::strstr(kvb_last_error(), "aligned") != nullptr, "alignment message");
  expect_einval(kvb_launch_attention_mma(&s, &fake, f, f, f, f, nullptr), "mma geometry");
  expect(std::strstr(kvb_last_error(), "launch_attention_mma requires") != nullptr, "mma geometry message");
  expect_einval(kvb_merge_attention(&s, f, 3, f, f, f, nullptr), "merge split-count mismatch");
  expect_einval(kvb_merge_attention(&s, nullptr, 4, f, f, f, nullptr), "merge null scratch");
  expect_einval(kvb_merge_finalize(&s, f, 0, f, f, f, f, KVB_OUT_F32, nullptr), "merge_finalize zero splits");
  expect_einval(kvb_merge_finalize(&s, f, 4, f, f, f, f, 7, nullptr), "merge_finalize unknown output type");
  expect_einval(kvb_merge_finalize(&s, f, 4, f, f, f, nullptr, KVB_OUT_F16, nullptr), "merge_finalize null output");
  expect_einval(kvb_split_attention(&s, &fake, 0, f, nullptr), "split zero split size");
  expect_einval(kvb_decode_attention(&s, &fake, 128, f, f, f, f, f, 9, nullptr), "decode unknown output type");
  expect_einval(kvb_decode_attention_fused(&s, &fake, 128, f, nullptr, f, f, f, f, KVB_OUT_F32, nullptr),
                "fused null counters");
  expect_einval(kvb_decode_attention_fused(&s, &misaligned, 128, f, u, f, f, f, f, KVB_OUT_F32, nullptr),
                "fused misaligned K");
  // The fenced diagnostic call has an instance only for the eight-wave dim-128 launch.
  expect_einval(kvb_decode_attention_fused_fenced(&s, &fake, 128, f, u, f, f, f, f, KVB_OUT_F32, nullptr),
                "fenced unsupported shape");
  expect(std::strstr(kvb_last_error(), "fenced diagnostic") != nullptr, "fenced shape message");
  // The static area of the no-alloc call cannot hold 64 q heads x 4,096 splits.
  const kvb_shape big = {1, 64, 8, 128, 64, 16384, 1u << 20, 0, 1u << 20, 0.0883883f, 1};
  expect_einval(kvb_decode_attention_noalloc(&big, &fake, 256, f, f, f, f, KVB_OUT_F16, nullptr), "noalloc too big");
  expect(std::strstr(kvb_last_error(), "static area") != nullptr, "noalloc size message");
  expect_einval(kvb_hbm_read_probe(f, 17, u, 4, nullptr), "probe byte count");
  expect_einval(kvb_hbm_read_probe(nullptr, 16, u, 4, nullptr), "probe null source");
  expect_einval(kvb_paged_read_probe(&s, &fake, 100, u, nullptr), "paged probe split size");
  // batched call
  const kvb_batch_shape bs = {4, 1, 64, 8, 128, 64, 8192, 131072, 4 * 131072, 8192, 2048, 0.0883883f, 1};
  const kvb_batch_input bnone = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  expect_einval(kvb_decode_attention_batched(&bs, &bnone, f, nullptr, f, f, f, nullptr, KVB_OUT_NONE, nullptr),
                "batched null inputs");
  expect_einval(kvb_decode_attention_batched(nullptr, &bnone, f, nullptr, f, f, f, nullptr, KVB_OUT_NONE, nullptr),
                "batched null shape");
  kvb_batch_shape bbad = bs;
  bbad.batch = 0;
  expect(kvb_batch_kernel_name(&bbad, &bnone, 1) != nullptr, "batch kernel name of an invalid shape");
}

int main() {
  expect(kvb_split_tokens() == 256, "kSplitTokens");
  sweep_shapes();
  sweep_batches();
  sweep_appends();
  launches_rejected();
  if (failures) {
    std::fprintf(stderr, "%d of %ld checks failed\n", failures, checks);
    return 1;
  }
  std::printf("PASS C ABI host checks (%ld checks)\n", checks);
  return 0;
}
