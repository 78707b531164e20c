/* TEST INFRASTRUCTURE ONLY: CPU oracle (see attention_oracle.c).  Not part of
 * the product; the product path must never load or call it. */
#ifndef KVB_ATTENTION_ORACLE_H
#define KVB_ATTENTION_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order and meaning as kvb_shape / kvbridge::Shape. */
typedef struct oracle_shape {
  uint32_t rows, q_heads, kv_heads, dim, page_tokens, pages, tokens, begin, end;
  float scale;
  uint32_t int8;
} oracle_shape;

/* FP64 normalized output out[rh*dim+d] and visible[rh] (reference
 * examples/attention_reference.h:53-90).  k/v are int8 codes (int8 != 0) or
 * float values; threads > 1 splits row-heads over pthreads. */
void oracle_fp64(const oracle_shape* s, const float* q, const int64_t* qpos, const int64_t* kpos,
                 const uint32_t* table, const void* k, const void* v, const float* ks,
                 const float* vs, double* out, uint8_t* visible, int threads);

/* fp32 split partials in the library's scratch layout. */
void oracle_split_fp32(const oracle_shape* s, const float* q, const int64_t* qpos,
                       const int64_t* kpos, const uint32_t* table, const void* k, const void* v,
                       const float* ks, const float* vs, uint32_t split_tokens, uint32_t splits,
                       float* scratch, int threads);

/* fp32 LSE merge into m, l, n. */
void oracle_merge_fp32(const oracle_shape* s, const float* scratch, uint32_t splits, float* m,
                       float* l, float* n);

/* Closed-form fixture of the reference (examples/attention_reference.h:19-48). */
void oracle_fixture(uint32_t tokens, int permute, float* q, int64_t* qpos, int64_t* kpos,
                    uint32_t* table, int8_t* k, int8_t* v, float* ks, float* vs);

#ifdef __cplusplus
}
#endif

#endif
