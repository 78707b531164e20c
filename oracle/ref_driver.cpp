// TEST INFRASTRUCTURE ONLY.  C entry point around the reference's own FP64
// oracle, compiled from the reference sources where they lie
// (examples/attention_reference.h, src/attention_shape.cpp) by oracle/Makefile
// into oracle/_ref/libkvbridge_ref.so.  Used to pin the repository's C
// restatement and as the "reference" CPU baseline.  Nothing from the
// reference is copied here; the header is included at build time.
#include <cstdint>
#include <cstring>
#include <vector>

#include "attention_reference.h"

extern "C" {

// Same field layout as kvb_shape.
struct ref_shape {
  uint32_t rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, begin, end;
  float scale;
  uint32_t int8;
};

// Runs kvbridge_example::reference on caller arrays (INT8 KV only, like the
// reference oracle).  Returns 0 on success, 1 if the reference rejected the
// shape.  out: rows*q_heads*dim doubles; visible: rows*q_heads bytes.
int ref_fp64_oracle(const ref_shape* rs, const float* q, const int64_t* qpos, const int64_t* kpos,
                    const uint32_t* table, const int8_t* k, const int8_t* v, const float* ks,
                    const float* vs, double* out, uint8_t* visible) {
  try {
    kvbridge_example::Fixture f;
    f.shape = kvbridge::Shape{rs->rows, rs->q_heads, rs->kv_heads, rs->dim, rs->page_tokens,
                              rs->pages, rs->tokens, rs->begin, rs->end, rs->scale, rs->int8 != 0};
    const auto& s = f.shape;
    const size_t slots = size_t(s.pages) * s.kv_heads * s.page_tokens;
    f.q.assign(q, q + size_t(s.rows) * s.q_heads * s.dim);
    f.qpos.assign(qpos, qpos + s.rows);
    f.kpos.assign(kpos, kpos + s.tokens);
    f.table.assign(table, table + s.pages);
    f.k.assign(k, k + slots * s.dim);
    f.v.assign(v, v + slots * s.dim);
    f.ks.assign(ks, ks + slots);
    f.vs.assign(vs, vs + slots);
    const auto o = kvbridge_example::reference(f);
    std::memcpy(out, o.normalized.data(), o.normalized.size() * sizeof(double));
    for (size_t i = 0; i < o.visible.size(); ++i) visible[i] = o.visible[i] ? 1 : 0;
    return 0;
  } catch (...) {
    return 1;
  }
}

// The reference fixture generator (make_fixture) for tokens / permute.
// Arrays sized for shape {8,24,4,256,32,ceil(tokens/32),tokens,...}.
void ref_make_fixture(unsigned tokens, int permute, float* q, int64_t* qpos, int64_t* kpos,
                      uint32_t* table, int8_t* k, int8_t* v, float* ks, float* vs) {
  const auto f = kvbridge_example::make_fixture(tokens, permute != 0);
  std::memcpy(q, f.q.data(), f.q.size() * sizeof(float));
  std::memcpy(qpos, f.qpos.data(), f.qpos.size() * sizeof(int64_t));
  std::memcpy(kpos, f.kpos.data(), f.kpos.size() * sizeof(int64_t));
  std::memcpy(table, f.table.data(), f.table.size() * sizeof(uint32_t));
  std::memcpy(k, f.k.data(), f.k.size());
  std::memcpy(v, f.v.data(), f.v.size());
  std::memcpy(ks, f.ks.data(), f.ks.size() * sizeof(float));
  std::memcpy(vs, f.vs.data(), f.vs.size() * sizeof(float));
}

}  // extern "C"
