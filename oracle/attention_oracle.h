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

/* Quantizing append into the paged pool (the write side of the cache layout;
 * the quantization BASELINE's configs describe): for new token t and kv head
 * h, the fp32 rows k_new / v_new[t * stride + h * dim + d] get scale =
 * absmax / 127 (1 for an all-zero row) and codes clamp(rint(x / scale),
 * -127, 127) in fp32 round-to-nearest-even, stored at physical slot
 * slots[t] (page = slot / page_tokens): K token-major, V dim-major, scales
 * per (page, kv, slot).  Ids >= pages * page_tokens are skipped. */
void oracle_append_int8(uint32_t tokens, uint32_t kv_heads, uint32_t dim, uint32_t page_tokens, uint32_t pages,
                        const float* k_new, const float* v_new, uint32_t k_stride, uint32_t v_stride,
                        const uint32_t* slots, int8_t* k, int8_t* v, float* ks, float* vs);

/* Planted mistakes for the tests that show the oracle's checks have teeth.
 * Process-global; 0 restores the faithful oracle. */
enum {
  ORACLE_FAULT_NONE = 0,
  ORACLE_FAULT_KSCALE_DROPPED = 1,   /* k-scale not applied to the dot        */
  ORACLE_FAULT_VSCALE_DROPPED = 2,   /* v-scale not applied to V              */
  ORACLE_FAULT_SCALE_DROPPED = 3,    /* score scale not applied               */
  ORACLE_FAULT_MASK_STRICT = 4,      /* kpos < qpos instead of kpos <= qpos   */
  ORACLE_FAULT_TABLE_IGNORED = 5,    /* logical page used as physical page    */
  ORACLE_FAULT_V_TOKEN_MAJOR = 6,    /* V read token-major (transposed)       */
  ORACLE_FAULT_GQA_MODULO = 7,       /* kv head = h % kv_heads                */
  ORACLE_FAULT_SPLIT_IGNORES_BEGIN = 8, /* splits start at 0, not at begin    */
  ORACLE_FAULT_MERGE_NO_SKIP = 9,    /* merge does not skip l <= 0 splits     */
  ORACLE_FAULT_QUANT_ROUND_AWAY = 10, /* append rounds halves away from zero  */
  ORACLE_FAULT_QUANT_SCALE_128 = 11,  /* append uses absmax / 128             */
  ORACLE_FAULT_QUANT_V_TOKEN_MAJOR = 12 /* append stores V token-major        */
};
void oracle_set_fault(int code);

#ifdef __cplusplus
}
#endif

#endif
