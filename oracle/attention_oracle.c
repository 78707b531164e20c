/* TEST INFRASTRUCTURE ONLY.  CPU oracle for paged INT8-KV split-K decode
 * attention.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the
 * timed CPU baseline -- never as the product path.
 *
 * Restates, in plain C:
 *   oracle_fp64         examples/attention_reference.h:53-90 (scalar FP64
 *                       direct softmax; "the CPU reference path")
 *   oracle_split_fp32   src/attention_shared.cu:42-209 semantics (per split:
 *                       fp32 dots with the k-scale folded into K, split max,
 *                       expf weights, v-scale folded into the weights)
 *   oracle_merge_fp32   src/attention_shared.cu:295-335 (LSE merge, splits
 *                       with l <= 0 skipped)
 *   oracle_fixture      examples/attention_reference.h:19-48 (closed-form
 *                       patterned fixture)
 *   oracle_append_int8  the per-(token, kv head) symmetric int8 quantization
 *                       BASELINE.json's configs describe (the reference ships
 *                       no cache writer), stored in the reference's layout
 *                       (include/kvbridge/attention_common.h:11-46)
 * Pinned by tests/test_oracle.py against the reference's own known-answer
 * tests (tests/reference_test.cpp), golden vectors produced by the
 * reference's FP64 oracle built from source (tests/golden), and closed forms.
 *
 * oracle_set_fault() plants one known mistake (a dropped term, a wrong index
 * or comparison) so the tests can show that their checks catch it; 0 (the
 * default) is the faithful oracle. */
#include "attention_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static int g_fault = ORACLE_FAULT_NONE;
void oracle_set_fault(int code) { g_fault = code; }

static int visible_pos(int64_t kpos, int64_t qpos) {
  return g_fault == ORACLE_FAULT_MASK_STRICT ? kpos < qpos : kpos <= qpos;
}

static double kv_at(const oracle_shape* s, const void* base, size_t i) {
  if (s->int8) return (double)((const int8_t*)base)[i];
  return (double)((const float*)base)[i];
}

/* Index of (physical page, kv head, slot) in the scale arrays; K row = this * dim. */
static size_t page_of(const oracle_shape* s, const uint32_t* table, uint32_t t) {
  return g_fault == ORACLE_FAULT_TABLE_IGNORED ? t / s->page_tokens : table[t / s->page_tokens];
}

static size_t slot_index(const oracle_shape* s, const uint32_t* table, uint32_t t, uint32_t kv) {
  const size_t page = page_of(s, table, t);
  return (page * s->kv_heads + kv) * s->page_tokens + t % s->page_tokens;
}

/* V element (d) of logical token t: V is dim-major inside a page. */
static size_t v_index(const oracle_shape* s, const uint32_t* table, uint32_t t, uint32_t kv, uint32_t d) {
  const size_t page = page_of(s, table, t);
  if (g_fault == ORACLE_FAULT_V_TOKEN_MAJOR)
    return ((page * s->kv_heads + kv) * s->page_tokens + t % s->page_tokens) * s->dim + d;
  return ((page * s->kv_heads + kv) * s->dim + d) * s->page_tokens + t % s->page_tokens;
}

typedef struct {
  const oracle_shape* s;
  const float *q, *ks, *vs;
  const int64_t *qpos, *kpos;
  const uint32_t* table;
  const void *k, *v;
  double* out;
  uint8_t* visible;
  uint32_t rh_begin, rh_end;
} fp64_job;

static uint32_t kv_of(const oracle_shape* s, uint32_t h) {
  if (g_fault == ORACLE_FAULT_GQA_MODULO) return h % s->kv_heads;
  return h / (s->q_heads / s->kv_heads);
}

static double kscale_of(const oracle_shape* s, const float* ks, size_t si) {
  if (!s->int8 || g_fault == ORACLE_FAULT_KSCALE_DROPPED) return 1.0;
  return (double)ks[si];
}

static double vscale_of(const oracle_shape* s, const float* vs, size_t si) {
  if (!s->int8 || g_fault == ORACLE_FAULT_VSCALE_DROPPED) return 1.0;
  return (double)vs[si];
}

static double score_scale(const oracle_shape* s) {
  return g_fault == ORACLE_FAULT_SCALE_DROPPED ? 1.0 : (double)s->scale;
}

static void fp64_rows(const fp64_job* j) {
  const oracle_shape* s = j->s;
  const uint32_t n = s->end - s->begin;
  double* logits = (double*)malloc(sizeof(double) * (n ? n : 1));
  for (uint32_t rh = j->rh_begin; rh < j->rh_end; ++rh) {
    const uint32_t r = rh / s->q_heads, h = rh % s->q_heads, kv = kv_of(s, h);
    const float* q = j->q + (size_t)rh * s->dim;
    double* o = j->out + (size_t)rh * s->dim;
    double mx = -INFINITY;
    int any = 0;
    for (uint32_t d = 0; d < s->dim; ++d) o[d] = 0.0;
    for (uint32_t t = s->begin; t < s->end; ++t) {
      double lg = -INFINITY;
      if (visible_pos(j->kpos[t], j->qpos[r])) {
        const size_t si = slot_index(s, j->table, t, kv);
        const double ks = kscale_of(s, j->ks, si);
        double dot = 0.0;
        for (uint32_t d = 0; d < s->dim; ++d) dot += (double)q[d] * kv_at(s, j->k, si * s->dim + d) * ks;
        lg = dot * score_scale(s);
        any = 1;
      }
      logits[t - s->begin] = lg;
      if (lg > mx) mx = lg;
    }
    j->visible[rh] = (uint8_t)any;
    if (!any) continue;
    double den = 0.0;
    for (uint32_t t = s->begin; t < s->end; ++t) {
      const double w = exp(logits[t - s->begin] - mx);
      if (w == 0.0) continue;
      den += w;
      const size_t si = slot_index(s, j->table, t, kv);
      const double vs = vscale_of(s, j->vs, si);
      for (uint32_t d = 0; d < s->dim; ++d) o[d] += w * kv_at(s, j->v, v_index(s, j->table, t, kv, d)) * vs;
    }
    for (uint32_t d = 0; d < s->dim; ++d) o[d] /= den;
  }
  free(logits);
}

static void* fp64_thread(void* p) {
  fp64_rows((const fp64_job*)p);
  return NULL;
}

void oracle_fp64(const oracle_shape* s, const float* q, const int64_t* qpos, const int64_t* kpos,
                 const uint32_t* table, const void* k, const void* v, const float* ks,
                 const float* vs, double* out, uint8_t* visible, int threads) {
  const uint32_t total = s->rows * s->q_heads;
  if (threads < 1) threads = 1;
  if ((uint32_t)threads > total) threads = (int)total;
  fp64_job* jobs = (fp64_job*)calloc((size_t)threads, sizeof(fp64_job));
  pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  for (int i = 0; i < threads; ++i) {
    fp64_job j = {s, q, ks, vs, qpos, kpos, table, k, v, out, visible,
                  (uint32_t)((uint64_t)total * i / threads), (uint32_t)((uint64_t)total * (i + 1) / threads)};
    jobs[i] = j;
  }
  if (threads == 1) {
    fp64_rows(&jobs[0]);
  } else {
    for (int i = 0; i < threads; ++i) pthread_create(&tids[i], NULL, fp64_thread, &jobs[i]);
    for (int i = 0; i < threads; ++i) pthread_join(tids[i], NULL);
  }
  free(jobs);
  free(tids);
}

/* ---- fp32 split-K partials + LSE merge -------------------------------- */

typedef struct {
  const oracle_shape* s;
  const float *q, *ks, *vs;
  const int64_t *qpos, *kpos;
  const uint32_t* table;
  const void *k, *v;
  uint32_t split_tokens, splits;
  float* scratch;
  uint32_t unit_begin, unit_end; /* units = (row*q_heads + head) * splits + split */
} split_job;

static void split_units(const split_job* j) {
  const oracle_shape* s = j->s;
  const uint32_t stride = s->dim + 2;
  float* w = (float*)malloc(sizeof(float) * (j->split_tokens ? j->split_tokens : 1));
  for (uint32_t u = j->unit_begin; u < j->unit_end; ++u) {
    const uint32_t rh = u / j->splits, split = u % j->splits;
    const uint32_t r = rh / s->q_heads, h = rh % s->q_heads, kv = kv_of(s, h);
    const float* q = j->q + (size_t)rh * s->dim;
    float* part = j->scratch + (size_t)u * stride;
    const uint64_t start64 = (g_fault == ORACLE_FAULT_SPLIT_IGNORES_BEGIN ? 0u : (uint64_t)s->begin) +
                             (uint64_t)split * j->split_tokens;
    const uint32_t start = start64 < s->end ? (uint32_t)start64 : s->end;
    const uint32_t count = (uint64_t)s->end - start < j->split_tokens ? s->end - start : j->split_tokens;
    float mx = -INFINITY;
    for (uint32_t i = 0; i < count; ++i) {
      const uint32_t t = start + i;
      float sc = -INFINITY;
      if (visible_pos(j->kpos[t], j->qpos[r])) {
        const size_t si = slot_index(s, j->table, t, kv);
        const float kscale = (float)kscale_of(s, j->ks, si);
        float dot = 0.0f;
        for (uint32_t d = 0; d < s->dim; ++d) {
          const float kf = s->int8 ? (float)((const int8_t*)j->k)[si * s->dim + d] * kscale
                                   : ((const float*)j->k)[si * s->dim + d];
          dot = fmaf(q[d], kf, dot);
        }
        sc = dot * (float)score_scale(s);
      }
      w[i] = sc;
      if (sc > mx) mx = sc;
    }
    float den = 0.0f;
    for (uint32_t d = 0; d < s->dim; ++d) part[2 + d] = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
      const float wt = mx == -INFINITY ? 0.0f : expf(w[i] - mx);
      den += wt;
      if (wt == 0.0f) continue;
      const uint32_t t = start + i;
      const size_t si = slot_index(s, j->table, t, kv);
      const float wsc = wt * (float)vscale_of(s, j->vs, si);
      for (uint32_t d = 0; d < s->dim; ++d) {
        const size_t vi = v_index(s, j->table, t, kv, d);
        const float vf = s->int8 ? (float)((const int8_t*)j->v)[vi] : ((const float*)j->v)[vi];
        part[2 + d] = fmaf(wsc, vf, part[2 + d]);
      }
    }
    part[0] = mx;
    part[1] = den;
  }
  free(w);
}

static void* split_thread(void* p) {
  split_units((const split_job*)p);
  return NULL;
}

void oracle_split_fp32(const oracle_shape* s, const float* q, const int64_t* qpos,
                       const int64_t* kpos, const uint32_t* table, const void* k, const void* v,
                       const float* ks, const float* vs, uint32_t split_tokens, uint32_t splits,
                       float* scratch, int threads) {
  const uint32_t total = s->rows * s->q_heads * splits;
  if (threads < 1) threads = 1;
  if ((uint32_t)threads > total) threads = (int)total;
  split_job* jobs = (split_job*)calloc((size_t)threads, sizeof(split_job));
  pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  for (int i = 0; i < threads; ++i) {
    split_job j = {s, q, ks, vs, qpos, kpos, table, k, v, split_tokens, splits, scratch,
                   (uint32_t)((uint64_t)total * i / threads), (uint32_t)((uint64_t)total * (i + 1) / threads)};
    jobs[i] = j;
  }
  if (threads == 1) {
    split_units(&jobs[0]);
  } else {
    for (int i = 0; i < threads; ++i) pthread_create(&tids[i], NULL, split_thread, &jobs[i]);
    for (int i = 0; i < threads; ++i) pthread_join(tids[i], NULL);
  }
  free(jobs);
  free(tids);
}

void oracle_merge_fp32(const oracle_shape* s, const float* scratch, uint32_t splits, float* m,
                       float* l, float* n) {
  const uint32_t stride = s->dim + 2;
  for (uint32_t rh = 0; rh < s->rows * s->q_heads; ++rh) {
    const float* base = scratch + (size_t)rh * splits * stride;
    float mx = -INFINITY;
    for (uint32_t j = 0; j < splits; ++j)
      if (base[(size_t)j * stride] > mx) mx = base[(size_t)j * stride];
    float den = 0.0f;
    for (uint32_t d = 0; d < s->dim; ++d) n[(size_t)rh * s->dim + d] = 0.0f;
    for (uint32_t j = 0; j < splits; ++j) {
      const float* p = base + (size_t)j * stride;
      if (!(p[1] > 0.0f) && g_fault != ORACLE_FAULT_MERGE_NO_SKIP) continue;
      const float f = expf(p[0] - mx);
      den += f * p[1];
      for (uint32_t d = 0; d < s->dim; ++d)
        n[(size_t)rh * s->dim + d] = fmaf(f, p[2 + d], n[(size_t)rh * s->dim + d]);
    }
    m[rh] = mx;
    l[rh] = den;
  }
}

/* ---- closed-form fixture ----------------------------------------------
 * Shape {8, 24, 4, 256, 32, ceil(tokens/32), tokens, 0, tokens, 1/16, int8}.
 * Arrays must be sized by the caller from that shape. */
void oracle_fixture(uint32_t tokens, int permute, float* q, int64_t* qpos, int64_t* kpos,
                    uint32_t* table, int8_t* k, int8_t* v, float* ks, float* vs) {
  const uint32_t rows = 8, q_heads = 24, kv_heads = 4, dim = 256, P = 32;
  const uint32_t pages = (tokens + P - 1) / P;
  const size_t slots = (size_t)pages * kv_heads * P;
  for (uint32_t p = 0; p < pages; ++p) table[p] = permute ? pages - 1 - p : p;
  for (size_t i = 0; i < (size_t)rows * q_heads * dim; ++i)
    q[i] = (float)((int)((i * 7) % 257) - 128) / 1024.0f;
  for (uint32_t r = 0; r < rows; ++r) qpos[r] = (int64_t)tokens - rows + r;
  memset(k, 0, slots * dim);
  memset(v, 0, slots * dim);
  for (size_t i = 0; i < slots; ++i) {
    ks[i] = 1.0f;
    vs[i] = 1.0f;
  }
  for (uint32_t t = 0; t < tokens; ++t) {
    kpos[t] = t;
    const uint32_t page = table[t / P], slot = t % P;
    for (uint32_t h = 0; h < kv_heads; ++h) {
      const size_t si = ((size_t)page * kv_heads + h) * P + slot;
      ks[si] = (float)((t + h) % 7 + 1) / 512.0f;
      vs[si] = (float)((t * 3 + h) % 5 + 1) / 512.0f;
      for (uint32_t d = 0; d < dim; ++d) {
        k[si * dim + d] = (int8_t)((int)((t * 17 + h * 11 + d * 3) % 256) - 128);
        v[(((size_t)page * kv_heads + h) * dim + d) * P + slot] =
            (int8_t)((int)((t * 7 + h * 13 + d * 5) % 256) - 128);
      }
    }
  }
}

/* scale = absmax / 127 (1 for an all-zero row), code = clamp(rint(x / scale),
 * -127, 127), in fp32 with IEEE maxNum / minNum (fmaxf / fminf) for the max
 * and the clamp: NaN elements are left out of the absmax, an infinite element
 * makes the scale infinite, and a NaN quotient clamps to -127. */
static void quantize_row(const float* x, uint32_t dim, int8_t* code, float* scale) {
  float amax = 0.0f;
  for (uint32_t d = 0; d < dim; ++d) amax = fmaxf(amax, fabsf(x[d]));
  const float div = g_fault == ORACLE_FAULT_QUANT_SCALE_128 ? 128.0f : 127.0f;
  const float sc = amax == 0.0f ? 1.0f : amax / div;
  for (uint32_t d = 0; d < dim; ++d) {
    const float q = x[d] / sc;
    const float r = g_fault == ORACLE_FAULT_QUANT_ROUND_AWAY ? roundf(q) : rintf(q);
    code[d] = (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
  }
  *scale = sc;
}

void oracle_append_int8(uint32_t tokens, uint32_t kv_heads, uint32_t dim, uint32_t page_tokens, uint32_t pages,
                        const float* k_new, const float* v_new, uint32_t k_stride, uint32_t v_stride,
                        const uint32_t* slots, int8_t* k, int8_t* v, float* ks, float* vs) {
  int8_t code[256];
  for (uint32_t t = 0; t < tokens; ++t) {
    const uint32_t id = slots[t];
    if ((uint64_t)id >= (uint64_t)pages * page_tokens) continue;
    const size_t page = id / page_tokens, slot = id % page_tokens;
    for (uint32_t h = 0; h < kv_heads; ++h) {
      const size_t row = (page * kv_heads + h) * page_tokens + slot;
      float sc;
      quantize_row(k_new + (size_t)t * k_stride + (size_t)h * dim, dim, code, &sc);
      memcpy(k + row * dim, code, dim);
      ks[row] = sc;
      quantize_row(v_new + (size_t)t * v_stride + (size_t)h * dim, dim, code, &sc);
      for (uint32_t d = 0; d < dim; ++d) {
        const size_t vi = g_fault == ORACLE_FAULT_QUANT_V_TOKEN_MAJOR ? row * dim + d
                                                                       : ((page * kv_heads + h) * dim + d) * page_tokens + slot;
        v[vi] = code[d];
      }
      vs[row] = sc;
    }
  }
}
