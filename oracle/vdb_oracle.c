/*
 * vdb_oracle.c -- CPU restatement of vdb's nearest-neighbour hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see vdb_oracle.h): the oracle the HIP backend is compared
 * against, never part of the product.  Citations are path:line in the reference
 * (KoduruChandrasekhar/HNSW-Vector-DB).  Built with -ffp-contract=off: the only fused
 * multiply-adds are the explicit fmaf() calls that stand for the reference's
 * _mm*_fmadd_ps intrinsics.
 */
#include "vdb_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* Hot loops get ISA clones; each lane of an emulated SIMD register is computed
 * independently with the same fmaf/add/sub, so every clone gives identical bits. */
#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define OR_HOT __attribute__((target_clones("avx512f", "fma", "default")))
#else
#define OR_HOT
#endif

/* ------------------------------------------------------------------ distances */

/* GCC's _mm512_reduce_add_ps tree (avx512fintrin.h __MM512_REDUCE_OP): upper 256 bits
 * plus lower, upper 128 plus lower, lanes {0,1}+{2,3}, then lane 0 + lane 1. */
static inline float reduce16(const float v[16]) {
  float t3[8], t6[4];
  for (int i = 0; i < 8; ++i) t3[i] = v[8 + i] + v[i];
  for (int i = 0; i < 4; ++i) t6[i] = t3[4 + i] + t3[i];
  float t80 = t6[0] + t6[2];
  float t81 = t6[1] + t6[3];
  return t80 + t81;
}

/* HorizontalSum of an 8-lane register (src/distance/avx2.cc:11-16): low 128 + high 128,
 * then two _mm_hadd_ps: (s0 + s1) + (s2 + s3). */
static inline float hsum8(const float v[8]) {
  float s[4];
  for (int i = 0; i < 4; ++i) s[i] = v[i] + v[4 + i];
  return (s[0] + s[1]) + (s[2] + s[3]);
}

/* l2_sq_scalar (src/distance/scalar.cc:8-15): one accumulator, no fusion. */
static float l2_scalar(const float* a, const float* b, size_t d) {
  float s = 0.f;
  for (size_t i = 0; i < d; ++i) {
    float t = a[i] - b[i];
    s += t * t;
  }
  return s;
}

/* dot_scalar (scalar.cc:17-21). */
static float dot_scalar(const float* a, const float* b, size_t d) {
  float s = 0.f;
  for (size_t i = 0; i < d; ++i) s += a[i] * b[i];
  return s;
}

/* l2_sq_avx512 (src/distance/avx512.cc:19-33): two 16-lane FMA accumulators over 32-float
 * steps, a 16-float tail into the first, then add and reduce. */
OR_HOT float l2_avx512(const float* a, const float* b, size_t d) {
  float acc0[16] = {0}, acc1[16] = {0};
  size_t i = 0;
  for (; i + 32 <= d; i += 32) {
    for (int l = 0; l < 16; ++l) {
      float d0 = a[i + l] - b[i + l];
      acc0[l] = fmaf(d0, d0, acc0[l]);
    }
    for (int l = 0; l < 16; ++l) {
      float d1 = a[i + 16 + l] - b[i + 16 + l];
      acc1[l] = fmaf(d1, d1, acc1[l]);
    }
  }
  if (i < d) {
    for (int l = 0; l < 16; ++l) {
      float d0 = a[i + l] - b[i + l];
      acc0[l] = fmaf(d0, d0, acc0[l]);
    }
  }
  float s[16];
  for (int l = 0; l < 16; ++l) s[l] = acc0[l] + acc1[l];
  return reduce16(s);
}

/* dot_avx512 (avx512.cc:35-44). */
OR_HOT float dot_avx512(const float* a, const float* b, size_t d) {
  float acc0[16] = {0}, acc1[16] = {0};
  size_t i = 0;
  for (; i + 32 <= d; i += 32) {
    for (int l = 0; l < 16; ++l) acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
    for (int l = 0; l < 16; ++l) acc1[l] = fmaf(a[i + 16 + l], b[i + 16 + l], acc1[l]);
  }
  if (i < d)
    for (int l = 0; l < 16; ++l) acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
  float s[16];
  for (int l = 0; l < 16; ++l) s[l] = acc0[l] + acc1[l];
  return reduce16(s);
}

/* l2_sq_avx2 (src/distance/avx2.cc:26-35): per 16 floats, lanes 0-7 into acc0 and
 * 8-15 into acc1. */
OR_HOT float l2_avx2(const float* a, const float* b, size_t d) {
  float acc0[8] = {0}, acc1[8] = {0};
  for (size_t i = 0; i < d; i += 16) {
    for (int l = 0; l < 8; ++l) {
      float d0 = a[i + l] - b[i + l];
      acc0[l] = fmaf(d0, d0, acc0[l]);
    }
    for (int l = 0; l < 8; ++l) {
      float d1 = a[i + 8 + l] - b[i + 8 + l];
      acc1[l] = fmaf(d1, d1, acc1[l]);
    }
  }
  float s[8];
  for (int l = 0; l < 8; ++l) s[l] = acc0[l] + acc1[l];
  return hsum8(s);
}

/* dot_avx2 (avx2.cc:37-44). */
OR_HOT float dot_avx2(const float* a, const float* b, size_t d) {
  float acc0[8] = {0}, acc1[8] = {0};
  for (size_t i = 0; i < d; i += 16) {
    for (int l = 0; l < 8; ++l) acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
    for (int l = 0; l < 8; ++l) acc1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], acc1[l]);
  }
  float s[8];
  for (int l = 0; l < 8; ++l) s[l] = acc0[l] + acc1[l];
  return hsum8(s);
}

float or_l2(int kset, const float* a, const float* b, size_t d) {
  switch (kset) {
    case OR_KSET_AVX512: return l2_avx512(a, b, d);
    case OR_KSET_AVX2: return l2_avx2(a, b, d);
    default: return l2_scalar(a, b, d);
  }
}

float or_dot(int kset, const float* a, const float* b, size_t d) {
  switch (kset) {
    case OR_KSET_AVX512: return dot_avx512(a, b, d);
    case OR_KSET_AVX2: return dot_avx2(a, b, d);
    default: return dot_scalar(a, b, d);
  }
}

/* MetricDistance (src/distance/cpu_features.cc:71-73): L2 -> squared L2, IP and cosine ->
 * minus the dot product (ip_dist_* = -dot_*, scalar.cc:23, avx512.cc:46). */
float or_metric_dist(int kset, int metric, const float* a, const float* b, size_t d) {
  return metric == OR_METRIC_L2 ? or_l2(kset, a, b, d) : -or_dot(kset, a, b, d);
}

/* sq8_l2_scalar (scalar.cc:25-34): decode vmin + c * scale in two roundings. */
static float sq8_l2_scalar(const float* q, const uint8_t* c, const float* vmin,
                           const float* scale, size_t d) {
  float s = 0.f;
  for (size_t i = 0; i < d; ++i) {
    float x = vmin[i] + (float)c[i] * scale[i];
    float t = q[i] - x;
    s += t * t;
  }
  return s;
}

/* sq8_ip_scalar (scalar.cc:36-41). */
static float sq8_ip_scalar(const float* q, const uint8_t* c, const float* vmin,
                           const float* scale, size_t d) {
  float s = 0.f;
  for (size_t i = 0; i < d; ++i) s += q[i] * (vmin[i] + (float)c[i] * scale[i]);
  return -s;
}

/* sq8_l2_avx512 (avx512.cc:48-56): Decode16 = fma(c, scale, vmin) (:11-15), one
 * accumulator, reduce. */
OR_HOT float sq8_l2_avx512(const float* q, const uint8_t* c, const float* vmin,
                                  const float* scale, size_t d) {
  float acc[16] = {0};
  for (size_t i = 0; i < d; i += 16) {
    for (int l = 0; l < 16; ++l) {
      float x = fmaf((float)c[i + l], scale[i + l], vmin[i + l]);
      float diff = q[i + l] - x;
      acc[l] = fmaf(diff, diff, acc[l]);
    }
  }
  return reduce16(acc);
}

/* sq8_ip_avx512 (avx512.cc:58-64). */
OR_HOT float sq8_ip_avx512(const float* q, const uint8_t* c, const float* vmin,
                                  const float* scale, size_t d) {
  float acc[16] = {0};
  for (size_t i = 0; i < d; i += 16) {
    for (int l = 0; l < 16; ++l) {
      float x = fmaf((float)c[i + l], scale[i + l], vmin[i + l]);
      acc[l] = fmaf(q[i + l], x, acc[l]);
    }
  }
  return -reduce16(acc);
}

/* sq8_l2_avx2 (avx2.cc:48-61): Decode8 on each half of 16 code bytes. */
OR_HOT float sq8_l2_avx2(const float* q, const uint8_t* c, const float* vmin,
                                const float* scale, size_t d) {
  float acc0[8] = {0}, acc1[8] = {0};
  for (size_t i = 0; i < d; i += 16) {
    for (int l = 0; l < 8; ++l) {
      float x0 = fmaf((float)c[i + l], scale[i + l], vmin[i + l]);
      float d0 = q[i + l] - x0;
      acc0[l] = fmaf(d0, d0, acc0[l]);
    }
    for (int l = 0; l < 8; ++l) {
      float x1 = fmaf((float)c[i + 8 + l], scale[i + 8 + l], vmin[i + 8 + l]);
      float d1 = q[i + 8 + l] - x1;
      acc1[l] = fmaf(d1, d1, acc1[l]);
    }
  }
  float s[8];
  for (int l = 0; l < 8; ++l) s[l] = acc0[l] + acc1[l];
  return hsum8(s);
}

/* sq8_ip_avx2 (avx2.cc:63-74). */
OR_HOT float sq8_ip_avx2(const float* q, const uint8_t* c, const float* vmin,
                                const float* scale, size_t d) {
  float acc0[8] = {0}, acc1[8] = {0};
  for (size_t i = 0; i < d; i += 16) {
    for (int l = 0; l < 8; ++l) {
      float x0 = fmaf((float)c[i + l], scale[i + l], vmin[i + l]);
      acc0[l] = fmaf(q[i + l], x0, acc0[l]);
    }
    for (int l = 0; l < 8; ++l) {
      float x1 = fmaf((float)c[i + 8 + l], scale[i + 8 + l], vmin[i + 8 + l]);
      acc1[l] = fmaf(q[i + 8 + l], x1, acc1[l]);
    }
  }
  float s[8];
  for (int l = 0; l < 8; ++l) s[l] = acc0[l] + acc1[l];
  return -hsum8(s);
}

float or_sq8_l2(int kset, const float* q, const uint8_t* c, const float* vmin,
                const float* scale, size_t d) {
  switch (kset) {
    case OR_KSET_AVX512: return sq8_l2_avx512(q, c, vmin, scale, d);
    case OR_KSET_AVX2: return sq8_l2_avx2(q, c, vmin, scale, d);
    default: return sq8_l2_scalar(q, c, vmin, scale, d);
  }
}

float or_sq8_ip(int kset, const float* q, const uint8_t* c, const float* vmin,
                const float* scale, size_t d) {
  switch (kset) {
    case OR_KSET_AVX512: return sq8_ip_avx512(q, c, vmin, scale, d);
    case OR_KSET_AVX2: return sq8_ip_avx2(q, c, vmin, scale, d);
    default: return sq8_ip_scalar(q, c, vmin, scale, d);
  }
}

/* MetricSq8Distance (cpu_features.cc:75-78). */
float or_metric_sq8(int kset, int metric, const float* q, const uint8_t* c,
                    const float* vmin, const float* scale, size_t d) {
  return metric == OR_METRIC_L2 ? or_sq8_l2(kset, q, c, vmin, scale, d)
                                : or_sq8_ip(kset, q, c, vmin, scale, d);
}

/* L2SqAny (scalar.cc:43-60): four accumulators over groups of four, tail into s0. */
float or_l2sq_any(const float* a, const float* b, size_t d) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  size_t i = 0;
  for (; i + 4 <= d; i += 4) {
    float t0 = a[i] - b[i], t1 = a[i + 1] - b[i + 1];
    float t2 = a[i + 2] - b[i + 2], t3 = a[i + 3] - b[i + 3];
    s0 += t0 * t0;
    s1 += t1 * t1;
    s2 += t2 * t2;
    s3 += t3 * t3;
  }
  for (; i < d; ++i) {
    float t = a[i] - b[i];
    s0 += t * t;
  }
  return (s0 + s1) + (s2 + s3);
}

/* DotAny (scalar.cc:62-73). */
float or_dot_any(const float* a, const float* b, size_t d) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  size_t i = 0;
  for (; i + 4 <= d; i += 4) {
    s0 += a[i] * b[i];
    s1 += a[i + 1] * b[i + 1];
    s2 += a[i + 2] * b[i + 2];
    s3 += a[i + 3] * b[i + 3];
  }
  for (; i < d; ++i) s0 += a[i] * b[i];
  return (s0 + s1) + (s2 + s3);
}

/* ------------------------------------------------------------------ top-k */

typedef struct {
  float d;
  uint32_t id;
} nb_t;

/* Neighbor::operator< (include/vdb/types.h:23-25): distance, then id. */
static inline int nb_lt(nb_t a, nb_t b) { return a.d < b.d || (a.d == b.d && a.id < b.id); }

static int nb_cmp(const void* pa, const void* pb) {
  nb_t a = *(const nb_t*)pa, b = *(const nb_t*)pb;
  return nb_lt(a, b) ? -1 : (nb_lt(b, a) ? 1 : 0);
}

/* TopK (src/util/topk.h:13-54): a max-heap of the k smallest (dist, id) pairs. */
typedef struct {
  nb_t* h;
  size_t n, k;
} topk_t;

static void topk_init(topk_t* t, size_t k) {
  t->h = (nb_t*)malloc(sizeof(nb_t) * (k + 1));
  t->n = 0;
  t->k = k;
}
static void topk_free(topk_t* t) { free(t->h); }
static inline float topk_threshold(const topk_t* t) {
  return (t->n >= t->k && t->k > 0) ? t->h[0].d : INFINITY;
}

static void topk_push(topk_t* t, float d, uint32_t id) {
  if (t->k == 0) return;
  nb_t x = {d, id};
  if (t->n < t->k) {
    size_t i = t->n++;
    t->h[i] = x;
    while (i > 0) {
      size_t p = (i - 1) / 2;
      if (!nb_lt(t->h[p], t->h[i])) break;
      nb_t tmp = t->h[p];
      t->h[p] = t->h[i];
      t->h[i] = tmp;
      i = p;
    }
  } else if (nb_lt(x, t->h[0])) {
    t->h[0] = x;
    size_t i = 0;
    for (;;) {
      size_t l = 2 * i + 1, r = l + 1, m = i;
      if (l < t->n && nb_lt(t->h[m], t->h[l])) m = l;
      if (r < t->n && nb_lt(t->h[m], t->h[r])) m = r;
      if (m == i) break;
      nb_t tmp = t->h[m];
      t->h[m] = t->h[i];
      t->h[i] = tmp;
      i = m;
    }
  }
}

/* sorted_into (topk.h:44-47): ascending (dist, id). */
static size_t topk_sorted(topk_t* t, nb_t* out) {
  memcpy(out, t->h, sizeof(nb_t) * t->n);
  qsort(out, t->n, sizeof(nb_t), nb_cmp);
  return t->n;
}

size_t or_topk(const float* dist, const uint32_t* id, size_t n, size_t k, float* out_d,
               uint32_t* out_id) {
  topk_t t;
  topk_init(&t, k);
  for (size_t i = 0; i < n; ++i) topk_push(&t, dist[i], id[i]);
  nb_t* s = (nb_t*)malloc(sizeof(nb_t) * (t.n + 1));
  size_t m = topk_sorted(&t, s);
  for (size_t i = 0; i < m; ++i) {
    out_d[i] = s[i].d;
    out_id[i] = s[i].id;
  }
  free(s);
  topk_free(&t);
  return m;
}

static inline int row_allowed(const uint64_t* w, size_t r) {
  return w == NULL || ((w[r >> 6] >> (r & 63)) & 1u);
}

static void write_padded(const nb_t* s, size_t m, size_t k, float* od, uint32_t* oi) {
  for (size_t i = 0; i < k; ++i) {
    od[i] = i < m ? s[i].d : INFINITY;
    oi[i] = i < m ? s[i].id : UINT32_MAX;
  }
}

/* ------------------------------------------------------------------ threads */

typedef void (*or_task_fn)(void* ctx, size_t begin, size_t end);
typedef struct {
  or_task_fn fn;
  void* ctx;
  size_t b, e;
} or_job_t;

static void* or_job_main(void* p) {
  or_job_t* j = (or_job_t*)p;
  if (j->b < j->e) j->fn(j->ctx, j->b, j->e);
  return NULL;
}

static void or_parallel(size_t n, int nthreads, or_task_fn fn, void* ctx) {
  if (nthreads <= 1 || n < 2) {
    fn(ctx, 0, n);
    return;
  }
  if ((size_t)nthreads > n) nthreads = (int)n;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  or_job_t* jobs = (or_job_t*)malloc(sizeof(or_job_t) * (size_t)nthreads);
  size_t chunk = (n + (size_t)nthreads - 1) / (size_t)nthreads;
  for (int t = 0; t < nthreads; ++t) {
    size_t b = (size_t)t * chunk, e = b + chunk < n ? b + chunk : n;
    jobs[t] = (or_job_t){fn, ctx, b < n ? b : n, e};
    pthread_create(&th[t], NULL, or_job_main, &jobs[t]);
  }
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(jobs);
  free(th);
}

/* ------------------------------------------------------------------ flat search */

typedef struct {
  int kset, metric;
  const float* base;
  size_t rows, pd;
  const float* queries;
  size_t k;
  const uint64_t* allow;
  float* out_d;
  uint32_t* out_id;
} flat_ctx_t;

/* FlatSearch without a pool (src/index/flat_index.cc:11-36): rows in order, skip the
 * ones the filter rejects, push every distance into TopK(k), return sorted. */
static void flat_task(void* p, size_t b, size_t e) {
  flat_ctx_t* c = (flat_ctx_t*)p;
  topk_t t;
  topk_init(&t, c->k);
  nb_t* s = (nb_t*)malloc(sizeof(nb_t) * (c->k + 1));
  for (size_t qi = b; qi < e; ++qi) {
    const float* q = c->queries + qi * c->pd;
    t.n = 0;
    if (c->k > 0) {
      for (size_t r = 0; r < c->rows; ++r) {
        if (!row_allowed(c->allow, r)) continue;
        topk_push(&t, or_metric_dist(c->kset, c->metric, q, c->base + r * c->pd, c->pd),
                  (uint32_t)r);
      }
    }
    size_t m = topk_sorted(&t, s);
    write_padded(s, m, c->k, c->out_d + qi * c->k, c->out_id + qi * c->k);
  }
  free(s);
  topk_free(&t);
}

void or_flat_search_batch(int kset, int metric, const float* base, size_t rows, size_t pd,
                          const float* queries, size_t nq, size_t k,
                          const uint64_t* allow_words, float* out_d, uint32_t* out_id,
                          int nthreads) {
  flat_ctx_t c = {kset, metric, base, rows, pd, queries, k, allow_words, out_d, out_id};
  or_parallel(nq, nthreads, flat_task, &c);
}

/* ------------------------------------------------------------------ rerank */

/* Rerank (src/index/index.cc:89-95): exact distance for every candidate, TopK(k). */
size_t or_rerank(int kset, int metric, const float* base, size_t pd, const float* q,
                 const uint32_t* cand_ids, size_t ncand, size_t k, float* out_d,
                 uint32_t* out_id) {
  topk_t t;
  topk_init(&t, k);
  for (size_t i = 0; i < ncand; ++i)
    topk_push(&t, or_metric_dist(kset, metric, q, base + (size_t)cand_ids[i] * pd, pd),
              cand_ids[i]);
  nb_t* s = (nb_t*)malloc(sizeof(nb_t) * (t.n + 1));
  size_t m = topk_sorted(&t, s);
  for (size_t i = 0; i < m; ++i) {
    out_d[i] = s[i].d;
    out_id[i] = s[i].id;
  }
  free(s);
  topk_free(&t);
  return m;
}

/* ------------------------------------------------------------------ SQ8 */

/* Sq8Quantizer::train (src/index/quant/sq8.cc:9-26): per real dimension min and max
 * with std::min/std::max (the first of equal values is kept); padding dims get 0. */
void or_sq8_train(const float* base, size_t rows, size_t dim, size_t pd, float* vmin,
                  float* scale) {
  for (size_t i = 0; i < pd; ++i) vmin[i] = scale[i] = 0.f;
  if (rows == 0) return;
  float* vmax = (float*)malloc(sizeof(float) * (dim + 1));
  for (size_t i = 0; i < dim; ++i) {
    vmax[i] = -INFINITY;
    vmin[i] = INFINITY;
  }
  for (size_t r = 0; r < rows; ++r) {
    const float* x = base + r * pd;
    for (size_t i = 0; i < dim; ++i) {
      vmin[i] = (x[i] < vmin[i]) ? x[i] : vmin[i]; /* std::min(vmin, x) */
      vmax[i] = (vmax[i] < x[i]) ? x[i] : vmax[i]; /* std::max(vmax, x) */
    }
  }
  for (size_t i = 0; i < dim; ++i) scale[i] = (vmax[i] - vmin[i]) / 255.f;
  free(vmax);
}

/* Sq8Quantizer::encode (sq8.cc:28-37): IEEE divide, nearbyint (round half to even in the
 * default mode), clamp to [0, 255]; padding dims and scale <= 0 give 0. */
void or_sq8_encode(const float* x, size_t dim, size_t pd, const float* vmin,
                   const float* scale, uint8_t* code) {
  for (size_t i = 0; i < pd; ++i) {
    if (i >= dim || scale[i] <= 0.f) {
      code[i] = 0;
      continue;
    }
    float c = nearbyintf((x[i] - vmin[i]) / scale[i]);
    float cl = c < 0.f ? 0.f : (255.f < c ? 255.f : c); /* std::clamp(c, 0, 255) */
    code[i] = (uint8_t)cl;
  }
}

void or_sq8_encode_rows(const float* base, size_t rows, size_t dim, size_t pd,
                        const float* vmin, const float* scale, uint8_t* codes) {
  for (size_t r = 0; r < rows; ++r)
    or_sq8_encode(base + r * pd, dim, pd, vmin, scale, codes + r * pd);
}

/* Sq8Quantizer::decode (sq8.cc:39-41). */
void or_sq8_decode(const uint8_t* code, size_t pd, const float* vmin, const float* scale,
                   float* x) {
  for (size_t i = 0; i < pd; ++i) x[i] = vmin[i] + (float)code[i] * scale[i];
}

typedef struct {
  int kset, metric;
  const float* base;
  const uint8_t* codes;
  size_t rows, pd;
  const float *vmin, *scale, *queries;
  size_t k, depth;
  const uint64_t* allow;
  float* out_d;
  uint32_t* out_id;
} sq8_ctx_t;

/* Exhaustive SQ8 scan into TopK(max(depth, k)) with MetricSq8Distance, then Rerank with
 * MetricDistance over the sorted candidates (the composition HnswSq8Index::search makes,
 * src/index/hnsw/hnsw_index.cc:82-100, with the graph replaced by a full scan). */
static void sq8_task(void* p, size_t b, size_t e) {
  sq8_ctx_t* c = (sq8_ctx_t*)p;
  size_t cap = c->depth > c->k ? c->depth : c->k;
  topk_t t;
  topk_init(&t, cap);
  nb_t* s = (nb_t*)malloc(sizeof(nb_t) * (cap + 1));
  uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * (cap + 1));
  float* rd = (float*)malloc(sizeof(float) * (c->k + 1));
  uint32_t* ri = (uint32_t*)malloc(sizeof(uint32_t) * (c->k + 1));
  for (size_t qi = b; qi < e; ++qi) {
    const float* q = c->queries + qi * c->pd;
    t.n = 0;
    if (c->k > 0) {
      for (size_t r = 0; r < c->rows; ++r) {
        if (!row_allowed(c->allow, r)) continue;
        topk_push(&t,
                  or_metric_sq8(c->kset, c->metric, q, c->codes + r * c->pd, c->vmin,
                                c->scale, c->pd),
                  (uint32_t)r);
      }
    }
    size_t m = topk_sorted(&t, s);
    float* od = c->out_d + qi * c->k;
    uint32_t* oi = c->out_id + qi * c->k;
    if (c->depth == 0) {
      write_padded(s, m < c->k ? m : c->k, c->k, od, oi);
      continue;
    }
    for (size_t i = 0; i < m; ++i) ids[i] = s[i].id;
    size_t n2 = or_rerank(c->kset, c->metric, c->base, c->pd, q, ids, m, c->k, rd, ri);
    for (size_t i = 0; i < c->k; ++i) {
      od[i] = i < n2 ? rd[i] : INFINITY;
      oi[i] = i < n2 ? ri[i] : UINT32_MAX;
    }
  }
  free(ri);
  free(rd);
  free(ids);
  free(s);
  topk_free(&t);
}

void or_sq8_search_batch(int kset, int metric, const float* base, const uint8_t* codes,
                         size_t rows, size_t pd, const float* vmin, const float* scale,
                         const float* queries, size_t nq, size_t k, size_t depth,
                         const uint64_t* allow_words, float* out_d, uint32_t* out_id,
                         int nthreads) {
  sq8_ctx_t c = {kset, metric, base, codes, rows, pd, vmin, scale, queries, k, depth,
                 allow_words, out_d, out_id};
  or_parallel(nq, nthreads, sq8_task, &c);
}

/* ------------------------------------------------------------------ PQ */

#define OR_KSUB 256

/* ProductQuantizer::encode (src/index/quant/pq.cc:43-57): per subspace the first
 * centroid with the smallest L2SqAny (strict <). */
void or_pq_encode(const float* centroids, size_t m, size_t dsub, const float* x,
                  uint8_t* code) {
  for (size_t j = 0; j < m; ++j) {
    const float* xs = x + j * dsub;
    float best = INFINITY;
    size_t arg = 0;
    for (size_t c = 0; c < OR_KSUB; ++c) {
      float d = or_l2sq_any(xs, centroids + (j * OR_KSUB + c) * dsub, dsub);
      if (d < best) {
        best = d;
        arg = c;
      }
    }
    code[j] = (uint8_t)arg;
  }
}

/* ProductQuantizer::compute_table (pq.cc:63-73): L2 -> L2SqAny, otherwise -DotAny. */
void or_pq_compute_table(const float* centroids, size_t m, size_t dsub, const float* q,
                         int metric, float* table) {
  for (size_t j = 0; j < m; ++j) {
    const float* qs = q + j * dsub;
    float* t = table + j * OR_KSUB;
    for (size_t c = 0; c < OR_KSUB; ++c) {
      const float* cen = centroids + (j * OR_KSUB + c) * dsub;
      t[c] = metric == OR_METRIC_L2 ? or_l2sq_any(qs, cen, dsub) : -or_dot_any(qs, cen, dsub);
    }
  }
}

/* ProductQuantizer::adc (src/index/quant/pq.h:36-46): four accumulators over j mod 4. */
float or_pq_adc(const float* table, size_t m, const uint8_t* code) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  size_t j = 0;
  for (; j + 4 <= m; j += 4) {
    s0 += table[(j + 0) * OR_KSUB + code[j + 0]];
    s1 += table[(j + 1) * OR_KSUB + code[j + 1]];
    s2 += table[(j + 2) * OR_KSUB + code[j + 2]];
    s3 += table[(j + 3) * OR_KSUB + code[j + 3]];
  }
  for (; j < m; ++j) s0 += table[j * OR_KSUB + code[j]];
  return (s0 + s1) + (s2 + s3);
}

/* ------------------------------------------------------------------ assignment */

typedef struct {
  int kset;
  const float* data;
  size_t d, stride;
  const float* cen;
  size_t k;
  uint32_t* assign;
  float* dist;
} assign_ctx_t;

/* AssignNearest (src/index/quant/kmeans.cc:23-55): PickL2 (:16-19) uses the SIMD kernel
 * when d and stride are multiples of 16, else L2SqAny; the first centroid with the
 * smallest distance wins (strict <).  The 8-point blocking does not change results. */
static void assign_task(void* p, size_t b, size_t e) {
  assign_ctx_t* c = (assign_ctx_t*)p;
  int simd = (c->d % 16 == 0) && (c->stride % 16 == 0);
  for (size_t i = b; i < e; ++i) {
    const float* x = c->data + i * c->stride;
    float best = INFINITY;
    uint32_t arg = 0;
    for (size_t j = 0; j < c->k; ++j) {
      const float* cr = c->cen + j * c->d;
      float dd = simd ? or_l2(c->kset, x, cr, c->d) : or_l2sq_any(x, cr, c->d);
      if (dd < best) {
        best = dd;
        arg = (uint32_t)j;
      }
    }
    c->assign[i] = arg;
    if (c->dist) c->dist[i] = best;
  }
}

void or_assign_nearest(int kset, const float* data, size_t n, size_t d, size_t stride,
                       const float* centroids, size_t k, uint32_t* assign, float* dist,
                       int nthreads) {
  assign_ctx_t c = {kset, data, d, stride, centroids, k, assign, dist};
  or_parallel(n, nthreads, assign_task, &c);
}

/* ------------------------------------------------------------------ IVF-PQ */

/* IvfPqIndex::precompute_tables (src/index/quant/ivf_pq.cc:152-167):
 * term2[l][j][c] = DotAny(C, C) + 2 * DotAny(coarse_l,j, C). */
void or_ivfpq_term2(const float* coarse, size_t nlist, size_t pd, const float* pq_centroids,
                    size_t m, size_t dsub, float* term2) {
  float* norms = (float*)malloc(sizeof(float) * m * OR_KSUB);
  for (size_t j = 0; j < m; ++j)
    for (size_t c = 0; c < OR_KSUB; ++c) {
      const float* cc = pq_centroids + (j * OR_KSUB + c) * dsub;
      norms[j * OR_KSUB + c] = or_dot_any(cc, cc, dsub);
    }
  for (size_t l = 0; l < nlist; ++l) {
    const float* cl = coarse + l * pd;
    float* t = term2 + l * m * OR_KSUB;
    for (size_t j = 0; j < m; ++j)
      for (size_t c = 0; c < OR_KSUB; ++c)
        t[j * OR_KSUB + c] =
            norms[j * OR_KSUB + c] +
            2.f * or_dot_any(cl + j * dsub, pq_centroids + (j * OR_KSUB + c) * dsub, dsub);
  }
  free(norms);
}

typedef struct {
  int kset, metric;
  const float* base;
  size_t dim, pd;
  const float* coarse;
  size_t nlist;
  const float* pqc;
  size_t m;
  const uint64_t* off;
  const uint32_t* ids;
  const uint8_t* codes;
  const float* term2;
  const float* queries;
  size_t k, nprobe;
  int rerank;
  const uint64_t* allow;
  float* out_d;
  uint32_t* out_id;
  uint64_t* dc;
} ivf_ctx_t;

/* IvfPqIndex::search (ivf_pq.cc:169-222) with FinishSearch (:28-36) and RerankDepth
 * (:16-19). */
static void ivf_task(void* p, size_t b, size_t e) {
  ivf_ctx_t* c = (ivf_ctx_t*)p;
  const size_t m = c->m, dsub = c->dim / m, ts = m * OR_KSUB;
  size_t depth = c->rerank < 0 ? (10 * c->k > 100 ? 10 * c->k : 100) : (size_t)c->rerank;
  size_t cap = depth > c->k ? depth : c->k;
  nb_t* cd = (nb_t*)malloc(sizeof(nb_t) * c->nlist);
  float* table = (float*)malloc(sizeof(float) * ts);
  float* qtab = (float*)malloc(sizeof(float) * ts);
  float* resid = (float*)malloc(sizeof(float) * c->dim);
  nb_t* s = (nb_t*)malloc(sizeof(nb_t) * (cap + 1));
  uint32_t* cand = (uint32_t*)malloc(sizeof(uint32_t) * (cap + 1));
  float* rd = (float*)malloc(sizeof(float) * (c->k + 1));
  uint32_t* ri = (uint32_t*)malloc(sizeof(uint32_t) * (c->k + 1));
  topk_t t;
  topk_init(&t, cap);
  const int l2 = c->metric == OR_METRIC_L2;
  const int pre = l2 && c->term2 != NULL;
  for (size_t qi = b; qi < e; ++qi) {
    const float* q = c->queries + qi * c->pd;
    float* od = c->out_d + qi * c->k;
    uint32_t* oi = c->out_id + qi * c->k;
    uint64_t dc = c->nlist;
    if (c->nlist == 0 || c->k == 0) {
      write_padded(s, 0, c->k, od, oi);
      if (c->dc) c->dc[qi] = 0;
      continue;
    }
    for (size_t l = 0; l < c->nlist; ++l)
      cd[l] = (nb_t){or_metric_dist(c->kset, c->metric, q, c->coarse + l * c->pd, c->pd),
                     (uint32_t)l};
    size_t nprobe = c->nprobe < 1 ? 1 : (c->nprobe > c->nlist ? c->nlist : c->nprobe);
    /* partial_sort by Neighbor order == the nprobe smallest (dist, list id), ascending */
    qsort(cd, c->nlist, sizeof(nb_t), nb_cmp);
    t.n = 0;
    if (!l2) or_pq_compute_table(c->pqc, m, dsub, q, c->metric, table);
    if (pre) {
      or_pq_compute_table(c->pqc, m, dsub, q, OR_METRIC_IP, qtab);
      for (size_t i = 0; i < ts; ++i) qtab[i] *= 2.f;
    }
    for (size_t pi = 0; pi < nprobe; ++pi) {
      const size_t l = cd[pi].id;
      const float* cen = c->coarse + l * c->pd;
      float offset = 0;
      if (pre) {
        offset = cd[pi].d;
        const float* t2 = c->term2 + l * ts;
        for (size_t i = 0; i < ts; ++i) table[i] = t2[i] + qtab[i];
      } else if (l2) {
        for (size_t j = 0; j < c->dim; ++j) resid[j] = q[j] - cen[j];
        or_pq_compute_table(c->pqc, m, dsub, resid, OR_METRIC_L2, table);
      } else {
        offset = -or_dot_any(q, cen, c->dim);
      }
      for (uint64_t r = c->off[l]; r < c->off[l + 1]; ++r) {
        uint32_t id = c->ids[r];
        if (!row_allowed(c->allow, id)) continue;
        topk_push(&t, offset + or_pq_adc(table, m, c->codes + r * m), id);
      }
      dc += c->off[l + 1] - c->off[l];
    }
    size_t n = topk_sorted(&t, s);
    if (depth == 0) {
      write_padded(s, n < c->k ? n : c->k, c->k, od, oi);
    } else {
      for (size_t i = 0; i < n; ++i) cand[i] = s[i].id;
      size_t n2 = or_rerank(c->kset, c->metric, c->base, c->pd, q, cand, n, c->k, rd, ri);
      dc += n;
      for (size_t i = 0; i < c->k; ++i) {
        od[i] = i < n2 ? rd[i] : INFINITY;
        oi[i] = i < n2 ? ri[i] : UINT32_MAX;
      }
    }
    if (c->dc) c->dc[qi] = dc;
  }
  topk_free(&t);
  free(ri);
  free(rd);
  free(cand);
  free(s);
  free(resid);
  free(qtab);
  free(table);
  free(cd);
}

void or_ivfpq_search_batch(int kset, int metric, const float* base, size_t dim, size_t pd,
                           const float* coarse, size_t nlist, const float* pq_centroids,
                           size_t m, const uint64_t* list_off, const uint32_t* list_ids,
                           const uint8_t* list_codes, const float* term2,
                           const float* queries, size_t nq, size_t k, size_t nprobe,
                           int rerank, const uint64_t* allow_words, float* out_d,
                           uint32_t* out_id, uint64_t* dist_comps, int nthreads) {
  ivf_ctx_t c = {kset,  metric, base,    dim,    pd,     coarse,  nlist,       pq_centroids,
                 m,     list_off, list_ids, list_codes, term2, queries, k,     nprobe,
                 rerank, allow_words, out_d, out_id, dist_comps};
  or_parallel(nq, nthreads, ivf_task, &c);
}

/* ------------------------------------------------------------------ query prep */

/* NormalizeVector (src/util/dataset.cc:33-41): fp64 sum of squares, float(1/sqrt),
 * then an fp32 multiply per element. */
int or_normalize(float* v, size_t dim) {
  double norm = 0;
  for (size_t i = 0; i < dim; ++i) norm += (double)v[i] * v[i];
  if (!(norm > 0) || !isfinite(norm)) return 0;
  float inv = (float)(1.0 / sqrt(norm));
  for (size_t i = 0; i < dim; ++i) v[i] *= inv;
  return 1;
}

/* ------------------------------------------------------------------ merge */

typedef struct {
  float d;
  uint32_t part, row;
} cand_t;

static int cand_cmp(const void* pa, const void* pb) {
  const cand_t* a = (const cand_t*)pa;
  const cand_t* b = (const cand_t*)pb;
  if (a->d < b->d) return -1;
  if (b->d < a->d) return 1;
  if (a->part != b->part) return a->part < b->part ? -1 : 1;
  if (a->row != b->row) return a->row < b->row ? -1 : 1;
  return 0;
}

/* CollectionImpl::Search merge (src/engine/collection_impl.cc:1076-1112): all parts'
 * hits sorted by (dist, part, row), the first occurrence of each external id kept,
 * stop at k. */
size_t or_merge_parts(size_t nparts, size_t k, const float* part_d, const uint32_t* part_row,
                      const uint64_t* ext, const uint64_t* part_off, float* out_d,
                      uint64_t* out_ext) {
  cand_t* all = (cand_t*)malloc(sizeof(cand_t) * (nparts * k + 1));
  size_t n = 0;
  for (size_t p = 0; p < nparts; ++p)
    for (size_t i = 0; i < k; ++i) {
      uint32_t r = part_row[p * k + i];
      if (r == UINT32_MAX) continue;
      all[n++] = (cand_t){part_d[p * k + i], (uint32_t)p, r};
    }
  qsort(all, n, sizeof(cand_t), cand_cmp);
  size_t out = 0;
  for (size_t i = 0; i < n && out < k; ++i) {
    uint64_t e = ext[part_off[all[i].part] + all[i].row];
    int seen = 0;
    for (size_t j = 0; j < out; ++j)
      if (out_ext[j] == e) {
        seen = 1;
        break;
      }
    if (seen) continue;
    out_d[out] = all[i].d;
    out_ext[out] = e;
    ++out;
  }
  free(all);
  return out;
}

/* SearchDiskSegment's choice for one segment (src/engine/planner.cc:53-108): no filter ->
 * the index (0); matches == 0 -> empty (1); the Auto cost model (:70-80: exact when matches
 * <= prefilter_threshold, or <= 10 * max(ef, k) / selectivity, or the index is flat) ->
 * prefilter_exact (2) or filtered_index (3) with nprobe raised to ceil(nprobe / selectivity)
 * under Auto (:92-99); post_filter (5).  Selectivity = matches / live rows, floored at 1e-9. */
int or_plan_segment(int has_filter, size_t rows, size_t deleted, size_t matches, int index_flat,
                    int strategy, size_t ef, size_t k, size_t nprobe,
                    size_t prefilter_threshold, size_t* nprobe_out) {
  *nprobe_out = nprobe;
  if (!has_filter) return 0;
  const size_t live = rows - (deleted < rows ? deleted : rows);
  const double sel = live == 0 ? 0.0 : (double)matches / (double)live;
  const double s = sel > 1e-9 ? sel : 1e-9;
  int strat = strategy;
  if (strat == 0) {
    const double graph_cost = 10.0 * (double)(ef > k ? ef : k) / s;
    strat = (matches <= prefilter_threshold || (double)matches <= graph_cost || index_flat) ? 1 : 2;
  }
  if (matches == 0) return 1;
  if (strat == 1) return 2;
  if (strat == 2) {
    if (strategy == 0) {
      const size_t boosted = (size_t)ceil((double)nprobe / s);
      *nprobe_out = boosted > nprobe ? boosted : nprobe;
    }
    return 3;
  }
  return 5;
}

/* ------------------------------------------------------------------ crc32c */

/* CRC32C with the reflected Castagnoli polynomial 0x82F63B78 (src/util/crc32c.cc:14),
 * bitwise: Extend(crc, data) continues a previous Value(). */
uint32_t or_crc32c(uint32_t crc, const void* data, size_t n) {
  const uint8_t* p = (const uint8_t*)data;
  uint32_t c = ~crc;
  for (size_t i = 0; i < n; ++i) {
    c ^= p[i];
    for (int b = 0; b < 8; ++b) c = (c >> 1) ^ (0x82F63B78u & (0u - (c & 1u)));
  }
  return ~c;
}

/* ------------------------------------------------------------------ HNSW-SQ8 search */

/* A VDBHSQ81 file's parts (HnswSq8Index::save, src/index/hnsw/hnsw_index.cc:108-115): u64
 * rows, the Sq8Quantizer (sq8.cc:43-63), rows x pd codes, then the graph (HnswGraph::serialize,
 * hnsw_graph.h:352-366). */
typedef struct {
  uint64_t cap, size;
  uint32_t M, M0;
  int max_level;
  uint32_t ep;
  uint8_t* level;
  uint32_t* links0; /* cap x (1 + M0): [count][links] */
  uint64_t* up_at;  /* per node: offset of its layer-1 list in up */
  uint32_t* up;     /* per node with level > 0: level x (1 + M) */
  size_t pd;
  const float* vmin;
  const float* scale;
  const uint8_t* codes;
  float* vbuf;
} or_hnsw_t;

static int rd_take(const uint8_t** p, size_t* left, void* dst, size_t n) {
  if (*left < n) return 0;
  if (dst != NULL) memcpy(dst, *p, n);
  *p += n;
  *left -= n;
  return 1;
}

static void or_hnsw_free(or_hnsw_t* g) {
  free(g->level);
  free(g->links0);
  free(g->up_at);
  free(g->up);
  free(g->vbuf);
}

/* Parses the file (LoadIndex's footer check, index.cc:47-56, then HnswSq8Index::load,
 * hnsw_index.cc:117-129, and HnswGraph::Deserialize, hnsw_graph.h:368-413, without its
 * validation: the files here are written by the reference). */
static int or_hnsw_parse(const uint8_t* f, size_t len, size_t rows, size_t pd, or_hnsw_t* g) {
  memset(g, 0, sizeof(*g));
  if (len < 12 || memcmp(f, "VDBHSQ81", 8) != 0) return -1;
  const uint8_t* p = f + 8;
  size_t left = len - 12;
  uint64_t n = 0, cap = 0, sz = 0, seed = 0;
  uint32_t qd = 0, qp = 0, m = 0, efc = 0, maxl = 0, ep = 0;
  if (!rd_take(&p, &left, &n, 8) || n != rows || !rd_take(&p, &left, &qd, 4) ||
      !rd_take(&p, &left, &qp, 4) || qp != pd)
    return -1;
  g->pd = pd;
  g->vbuf = (float*)malloc(sizeof(float) * 2 * pd + 4);
  if (!rd_take(&p, &left, g->vbuf, 4 * pd) || !rd_take(&p, &left, g->vbuf + pd, 4 * pd)) return -1;
  g->vmin = g->vbuf;
  g->scale = g->vbuf + pd;
  g->codes = p;
  if (!rd_take(&p, &left, NULL, rows * pd)) return -1;
  if (!rd_take(&p, &left, &cap, 8) || !rd_take(&p, &left, &sz, 8) || !rd_take(&p, &left, &m, 4) ||
      !rd_take(&p, &left, &efc, 4) || !rd_take(&p, &left, &seed, 8) ||
      !rd_take(&p, &left, &maxl, 4) || !rd_take(&p, &left, &ep, 4) || cap != rows || m < 2)
    return -1;
  g->cap = cap;
  g->size = sz;
  g->M = m;
  g->M0 = 2 * m;
  g->max_level = (int)maxl;
  g->ep = ep;
  g->level = (uint8_t*)malloc(cap + 1);
  g->links0 = (uint32_t*)malloc(sizeof(uint32_t) * (cap * (1 + g->M0) + 1));
  g->up_at = (uint64_t*)calloc(cap + 1, sizeof(uint64_t));
  if (!rd_take(&p, &left, g->level, cap) ||
      !rd_take(&p, &left, g->links0, sizeof(uint32_t) * cap * (1 + g->M0)))
    return -1;
  uint64_t tot = 0;
  for (uint64_t i = 0; i < cap; ++i) {
    g->up_at[i] = tot;
    tot += (uint64_t)g->level[i] * (1 + m);
  }
  g->up = (uint32_t*)malloc(sizeof(uint32_t) * (tot + 1));
  if (!rd_take(&p, &left, g->up, sizeof(uint32_t) * tot)) return -1;
  return 0;
}

/* links_at (hnsw_graph.h:425-428). */
static const uint32_t* or_links(const or_hnsw_t* g, uint32_t id, int layer) {
  if (layer == 0) return g->links0 + (size_t)id * (1 + g->M0);
  return g->up + g->up_at[id] + (size_t)(layer - 1) * (1 + g->M);
}

/* Binary heaps of (dist, id): max-heap (the results, worst on top) when max_heap, else
 * min-heap (the candidates, closest on top); std::push_heap / pop_heap with Neighbor's
 * order (types.h:23-26).  Only the top is ever read, and the order is total, so any heap
 * holds the same top. */
static inline int heap_before(nb_t a, nb_t b, int max_heap) {
  return max_heap ? nb_lt(b, a) : nb_lt(a, b);
}
static void heap_push(nb_t* h, size_t* n, nb_t x, int max_heap) {
  size_t i = (*n)++;
  h[i] = x;
  while (i > 0) {
    size_t p = (i - 1) / 2;
    if (!heap_before(h[i], h[p], max_heap)) break;
    nb_t t = h[p];
    h[p] = h[i];
    h[i] = t;
    i = p;
  }
}
static void heap_pop(nb_t* h, size_t* n, int max_heap) {
  h[0] = h[--(*n)];
  size_t i = 0;
  for (;;) {
    size_t l = 2 * i + 1, r = l + 1, b = i;
    if (l < *n && heap_before(h[l], h[b], max_heap)) b = l;
    if (r < *n && heap_before(h[r], h[b], max_heap)) b = r;
    if (b == i) break;
    nb_t t = h[b];
    h[b] = h[i];
    h[i] = t;
    i = b;
  }
}

typedef struct {
  int kset, metric;
  const or_hnsw_t* g;
  const float* base;
  const float* queries;
  size_t k, ef;
  int rerank;
  const uint64_t* allow;
  float* out_d;
  uint32_t* out_id;
  uint64_t* dc;
} hnsw_ctx_t;

static inline float or_hnsw_dist(const hnsw_ctx_t* c, const float* q, uint32_t id) {
  const or_hnsw_t* g = c->g;
  return or_metric_sq8(c->kset, c->metric, q, g->codes + (size_t)id * g->pd, g->vmin, g->scale,
                       g->pd);
}

/* HnswGraph::search (hnsw_graph.h:301-324) with the greedy descent (:467-496) and the layer-0
 * beam search_layer<false, kFiltered> (:501-548).  Writes up to kk results ascending into
 * out and returns their count; *dc counts distance computations as the reference does. */
static size_t or_hnsw_walk(const hnsw_ctx_t* c, const float* q, size_t kk, size_t ef,
                           uint8_t* seen, nb_t* res, nb_t* cand, nb_t* out, uint64_t* dc) {
  const or_hnsw_t* g = c->g;
  if (g->max_level < 0 || kk == 0) return 0;
  uint64_t n_dc = 1;
  uint32_t cur = g->ep;
  float curd = or_hnsw_dist(c, q, cur);
  for (int l = g->max_level; l > 0; --l) {
    for (int changed = 1; changed;) {
      changed = 0;
      const uint32_t* ll = or_links(g, cur, l);
      const uint32_t cnt = ll[0];
      const uint32_t* nb = ll + 1;
      for (uint32_t j = 0; j < cnt; ++j) {
        float d = or_hnsw_dist(c, q, nb[j]);
        ++n_dc;
        if (d < curd) {
          curd = d;
          cur = nb[j];
          changed = 1;
        }
      }
    }
  }
  if (ef < kk) ef = kk;
  const int filtered = c->allow != NULL;
  size_t nr = 0, nc = 0;
  memset(seen, 0, g->cap);
  seen[cur] = 1;
  float lower = INFINITY;
  nb_t e0 = {curd, cur};
  if (!filtered || row_allowed(c->allow, cur)) {
    heap_push(res, &nr, e0, 1);
    lower = curd;
  }
  heap_push(cand, &nc, e0, 0);
  while (nc > 0) {
    const nb_t top = cand[0];
    if (top.d > lower && (!filtered || nr >= ef)) break;
    heap_pop(cand, &nc, 0);
    const uint32_t* ll = or_links(g, top.id, 0);
    const uint32_t cnt = ll[0];
    for (uint32_t j = 0; j < cnt; ++j) {
      const uint32_t e = ll[1 + j];
      if (seen[e]) continue;
      seen[e] = 1;
      const float de = or_hnsw_dist(c, q, e);
      ++n_dc;
      if (nr < ef || de < lower) {
        nb_t x = {de, e};
        heap_push(cand, &nc, x, 0);
        if (!filtered || row_allowed(c->allow, e)) {
          heap_push(res, &nr, x, 1);
          if (nr > ef) heap_pop(res, &nr, 1);
          lower = res[0].d;
        }
      }
    }
  }
  while (nr > kk) heap_pop(res, &nr, 1);
  memcpy(out, res, sizeof(nb_t) * nr);
  qsort(out, nr, sizeof(nb_t), nb_cmp);
  *dc += n_dc;
  return nr;
}

static void hnsw_task(void* p, size_t b, size_t e) {
  hnsw_ctx_t* c = (hnsw_ctx_t*)p;
  const or_hnsw_t* g = c->g;
  /* depth and ef of HnswSq8Index::search (hnsw_index.cc:88-89) */
  const size_t depth = c->rerank < 0 ? (c->ef > c->k ? c->ef : c->k) : (size_t)c->rerank;
  size_t ef = c->ef > c->k ? c->ef : c->k;
  if (depth > ef) ef = depth;
  const size_t kk = depth > c->k ? depth : c->k;
  uint8_t* seen = (uint8_t*)malloc(g->cap + 1);
  /* the candidate heap holds at most every node once, the results ef + 1 */
  nb_t* cand = (nb_t*)malloc(sizeof(nb_t) * (g->cap + 1));
  nb_t* res = (nb_t*)malloc(sizeof(nb_t) * (ef + 2));
  nb_t* out = (nb_t*)malloc(sizeof(nb_t) * (ef + 2));
  uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * (ef + 2));
  float* rd = (float*)malloc(sizeof(float) * (c->k + 1));
  uint32_t* ri = (uint32_t*)malloc(sizeof(uint32_t) * (c->k + 1));
  for (size_t qi = b; qi < e; ++qi) {
    const float* q = c->queries + qi * g->pd;
    float* od = c->out_d + qi * c->k;
    uint32_t* oi = c->out_id + qi * c->k;
    uint64_t dc = 0;
    if (c->k == 0) {
      if (c->dc) c->dc[qi] = 0;
      continue;
    }
    if (depth == 0) {
      size_t m = or_hnsw_walk(c, q, c->k, ef, seen, res, cand, out, &dc);
      write_padded(out, m, c->k, od, oi);
    } else {
      size_t m = or_hnsw_walk(c, q, kk, ef, seen, res, cand, out, &dc);
      for (size_t i = 0; i < m; ++i) ids[i] = out[i].id;
      /* Rerank (index.cc:89-95): exact distances of every candidate, TopK(k) */
      size_t n2 = or_rerank(c->kset, c->metric, c->base, g->pd, q, ids, m, c->k, rd, ri);
      dc += m;
      for (size_t i = 0; i < c->k; ++i) {
        od[i] = i < n2 ? rd[i] : INFINITY;
        oi[i] = i < n2 ? ri[i] : UINT32_MAX;
      }
    }
    if (c->dc) c->dc[qi] = dc;
  }
  free(ri);
  free(rd);
  free(ids);
  free(out);
  free(res);
  free(cand);
  free(seen);
}

int or_hnsw_sq8_search_file(int kset, int metric, const uint8_t* file, size_t len,
                            const float* base, size_t rows, size_t pd, const float* queries,
                            size_t nq, size_t k, size_t ef, int rerank,
                            const uint64_t* allow_words, float* out_d, uint32_t* out_id,
                            uint64_t* dist_comps, int nthreads) {
  or_hnsw_t g;
  if (or_hnsw_parse(file, len, rows, pd, &g) != 0) {
    or_hnsw_free(&g);
    return -1;
  }
  hnsw_ctx_t c = {kset, metric, &g, base, queries, k, ef, rerank, allow_words, out_d, out_id,
                  dist_comps};
  or_parallel(nq, nthreads, hnsw_task, &c);
  or_hnsw_free(&g);
  return 0;
}

/* ------------------------------------------------------------------ PQ-flat search */

typedef struct {
  int kset, metric;
  const float* base;
  size_t rows, pd;
  const float* cen;
  size_t m, dsub;
  const uint8_t* codes;
  const float* queries;
  size_t k;
  int rerank;
  const uint64_t* allow;
  float* out_d;
  uint32_t* out_id;
  uint64_t* dc;
} pqflat_ctx_t;

/* PqFlatIndex::search (src/index/quant/ivf_pq.cc:59-79): compute_table, ADC of every allowed
 * row into TopK(max(depth, k)), FinishSearch (:28-36) with RerankDepth (:16-19). */
static void pqflat_task(void* p, size_t b, size_t e) {
  pqflat_ctx_t* c = (pqflat_ctx_t*)p;
  const size_t depth = c->rerank < 0 ? (10 * c->k > 100 ? 10 * c->k : 100) : (size_t)c->rerank;
  const size_t cap = depth > c->k ? depth : c->k;
  float* table = (float*)malloc(sizeof(float) * c->m * OR_KSUB);
  topk_t t;
  topk_init(&t, cap);
  nb_t* s = (nb_t*)malloc(sizeof(nb_t) * (cap + 1));
  uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * (cap + 1));
  float* rd = (float*)malloc(sizeof(float) * (c->k + 1));
  uint32_t* ri = (uint32_t*)malloc(sizeof(uint32_t) * (c->k + 1));
  for (size_t qi = b; qi < e; ++qi) {
    const float* q = c->queries + qi * c->pd;
    float* od = c->out_d + qi * c->k;
    uint32_t* oi = c->out_id + qi * c->k;
    if (c->rows == 0 || c->k == 0) {
      write_padded(s, 0, c->k, od, oi);
      if (c->dc) c->dc[qi] = 0;
      continue;
    }
    or_pq_compute_table(c->cen, c->m, c->dsub, q, c->metric == OR_METRIC_L2 ? 0 : 1, table);
    t.n = 0;
    for (size_t r = 0; r < c->rows; ++r) {
      if (!row_allowed(c->allow, r)) continue;
      topk_push(&t, or_pq_adc(table, c->m, c->codes + r * c->m), (uint32_t)r);
    }
    size_t m = topk_sorted(&t, s);
    uint64_t dc = c->rows;
    if (depth == 0) {
      write_padded(s, m < c->k ? m : c->k, c->k, od, oi);
    } else {
      for (size_t i = 0; i < m; ++i) ids[i] = s[i].id;
      size_t n2 = or_rerank(c->kset, c->metric, c->base, c->pd, q, ids, m, c->k, rd, ri);
      dc += m;
      for (size_t i = 0; i < c->k; ++i) {
        od[i] = i < n2 ? rd[i] : INFINITY;
        oi[i] = i < n2 ? ri[i] : UINT32_MAX;
      }
    }
    if (c->dc) c->dc[qi] = dc;
  }
  free(ri);
  free(rd);
  free(ids);
  free(s);
  topk_free(&t);
  free(table);
}

void or_pqflat_search_batch(int kset, int metric, const float* base, size_t rows, size_t pd,
                            const float* pq_centroids, size_t m, size_t dsub,
                            const uint8_t* codes, const float* queries, size_t nq, size_t k,
                            int rerank, const uint64_t* allow_words, float* out_d,
                            uint32_t* out_id, uint64_t* dist_comps, int nthreads) {
  pqflat_ctx_t c = {kset, metric, base, rows, pd, pq_centroids, m, dsub, codes, queries, k,
                    rerank, allow_words, out_d, out_id, dist_comps};
  or_parallel(nq, nthreads, pqflat_task, &c);
}
