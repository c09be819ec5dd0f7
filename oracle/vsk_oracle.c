/*
 * vsk_oracle.c -- CPU restatement of VectorStoreKit's search hot path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU-baseline timing).  The
 * shipped HIP library never links or calls it.  Build: oracle/Makefile
 * (gcc -O3 -ffp-contract=off; no -ffast-math, so the fp32 order written
 * here is the order executed).
 *
 * Reference paths below are relative to Sources/VectorStoreKit/ of
 * gifton/VectorStoreKit.
 */
#include "vsk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* threading: a static split of [0, n) over nthreads pthreads                 */
/* ------------------------------------------------------------------------ */
typedef void (*range_fn)(void *ctx, int64_t lo, int64_t hi);
typedef struct {
  range_fn fn;
  void *ctx;
  int64_t lo, hi;
} range_job;

static void *range_trampoline(void *p) {
  range_job *j = (range_job *)p;
  j->fn(j->ctx, j->lo, j->hi);
  return NULL;
}

int32_t vsko_num_threads(void) {
  long c = sysconf(_SC_NPROCESSORS_ONLN);
  return c > 0 ? (int32_t)c : 1;
}

static void parallel_for(int64_t n, int32_t nthreads, range_fn fn, void *ctx) {
  if (nthreads <= 0) nthreads = vsko_num_threads();
  if (nthreads > n) nthreads = (int32_t)(n > 0 ? n : 1);
  if (nthreads <= 1) {
    fn(ctx, 0, n);
    return;
  }
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * nthreads);
  range_job *jobs = (range_job *)malloc(sizeof(range_job) * nthreads);
  for (int32_t t = 0; t < nthreads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].lo = n * t / nthreads;
    jobs[t].hi = n * (t + 1) / nthreads;
    pthread_create(&th[t], NULL, range_trampoline, &jobs[t]);
  }
  for (int32_t t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
}

/* ------------------------------------------------------------------------ */
/* distances                                                                  */
/* ------------------------------------------------------------------------ */

/* sum (a_i - b_i)^2, i ascending, no FMA.
 * Indexes/IVFIndex.swift:542-549 (computeDistance, before its sqrt);
 * Quantization/ProductQuantizer.swift:362-369 (euclideanDistanceSquared). */
float vsko_l2sq(const float *a, const float *b, int32_t d) {
  float s = 0.0f;
  for (int32_t i = 0; i < d; ++i) {
    float diff = a[i] - b[i];
    s += diff * diff;
  }
  return s;
}

/* sum a_i * b_i, i ascending (vDSP_dotpr in
 * Acceleration/AccelerateOptimizer.swift:301-307,371-377; the order inside
 * vDSP is not published, sequential order is this restatement's choice). */
float vsko_dot(const float *a, const float *b, int32_t d) {
  float s = 0.0f;
  for (int32_t i = 0; i < d; ++i) s += a[i] * b[i];
  return s;
}

/* sum |a_i - b_i|  (Acceleration/AccelerateOptimizer.swift:322-360:
 * vDSP_vsub, vDSP_vabs, vDSP_sve). */
float vsko_l1(const float *a, const float *b, int32_t d) {
  float s = 0.0f;
  for (int32_t i = 0; i < d; ++i) s += fabsf(a[i] - b[i]);
  return s;
}

/* Acceleration/AccelerateOptimizer.swift:251-383 (euclidean: sqrt of the
 * sum of squares; cosine: 1 - dot/(|q||x| + 1e-8) with magnitudes from
 * vDSP_svesq + sqrt; dotProduct: -dot; manhattan: sum |q-x|) and
 * Acceleration/Metal/Shaders/DistanceShaders.metal:815-845 (normalized
 * cosine: 1 - dot). */
float vsko_distance(const float *q, const float *x, int32_t d,
                    int32_t metric) {
  switch (metric) {
  case VSKO_L2SQ:
    return vsko_l2sq(q, x, d);
  case VSKO_L2:
    return sqrtf(vsko_l2sq(q, x, d));
  case VSKO_COSINE: {
    float qn = sqrtf(vsko_dot(q, q, d));
    float xn = sqrtf(vsko_dot(x, x, d));
    float dp = vsko_dot(q, x, d);
    return 1.0f - dp / (qn * xn + 1e-8f);
  }
  case VSKO_COSINE_NORMALIZED:
    return 1.0f - vsko_dot(q, x, d);
  case VSKO_DOT:
    return -vsko_dot(q, x, d);
  case VSKO_L1:
    return vsko_l1(q, x, d);
  case VSKO_HAMMING: {
    /* Core/Distance/UnifiedDistanceComputation.swift:249-261: count += 1
     * where a[i] != b[i] (fp32 counter) */
    float c = 0.0f;
    for (int32_t i = 0; i < d; ++i)
      if (q[i] != x[i]) c += 1.0f;
    return c;
  }
  default:
    return NAN;
  }
}

/* AccelerateOptimizer.scalarQuantize (Acceleration/AccelerateOptimizer.swift:
 * 387-430), the CPU path of MetalAccelerationEngine.quantizeVectors(scheme:
 * .scalar(bits:)): min and max of the vector (vDSP_minv / vDSP_maxv),
 * scale = Float(1 << bits - 1) / range (Swift's << binds tighter than -, so
 * 2^bits - 1), or 1 when range == 0; code = UInt8(min(max((v - min) *
 * scale, 0), 255)), the conversion truncating toward zero. */
void vsko_scalar_quantize_u8(const float *x, int64_t n, int32_t d, int32_t bits,
                             uint8_t *codes, float *scale, float *minv) {
  const float levels = (float)((1 << bits) - 1);
  for (int64_t r = 0; r < n; ++r) {
    const float *xr = x + r * d;
    float mn = xr[0], mx = xr[0];
    for (int32_t i = 1; i < d; ++i) {
      if (xr[i] < mn) mn = xr[i];
      if (xr[i] > mx) mx = xr[i];
    }
    const float range = mx - mn;
    const float s = range > 0.0f ? levels / range : 1.0f;
    for (int32_t i = 0; i < d; ++i) {
      float t = (xr[i] - mn) * s;
      if (t < 0.0f) t = 0.0f;
      if (t > 255.0f) t = 255.0f;
      codes[r * d + i] = (uint8_t)t;
    }
    if (scale) scale[r] = s;
    if (minv) minv[r] = mn;
  }
}

/* HNSWIndex's DistanceComputer.distance (Indexes/HNSWIndex.swift:1920-1959).
 * Swift's SIMD.sum() on floating point adds the lanes in index order starting
 * from -0.0 (the standard library's generic implementation); reduce(0)
 * starts from +0.0.
 *   euclidean: sqrt(((v1 - v2) * (v1 - v2)).sum())
 *   cosine:    1 - (v1 * v2).sum() / (sqrt((v1*v1).sum()) * sqrt((v2*v2).sum()))
 *   manhattan: reduce(0) { sum + abs(diff[i]) }
 * VSKO_L2SQ is the euclidean sum before its sqrt. */
float vsko_hnsw_distance(const float *q, const float *x, int32_t d, int32_t metric) {
  if (metric == VSKO_L1) {
    float s = 0.0f;
    for (int32_t i = 0; i < d; ++i) s += fabsf(q[i] - x[i]);
    return s;
  }
  if (metric == VSKO_COSINE_NOEPS) {
    float dot = -0.0f, qq = -0.0f, xx = -0.0f;
    for (int32_t i = 0; i < d; ++i) dot += q[i] * x[i];
    for (int32_t i = 0; i < d; ++i) qq += q[i] * q[i];
    for (int32_t i = 0; i < d; ++i) xx += x[i] * x[i];
    const float m1 = sqrtf(qq), m2 = sqrtf(xx);
    return 1.0f - dot / (m1 * m2);
  }
  float s = -0.0f;
  for (int32_t i = 0; i < d; ++i) {
    const float t = q[i] - x[i];
    s += t * t;
  }
  return metric == VSKO_L2SQ ? s : sqrtf(s);
}

/* query i against rows[offsets[i] .. offsets[i+1]) of x */
void vsko_hnsw_distances(const float *q, int64_t nq, const float *x, int32_t d,
                         const int64_t *offsets, const int32_t *rows, int32_t metric,
                         float *out) {
  for (int64_t i = 0; i < nq; ++i)
    for (int64_t j = offsets[i]; j < offsets[i + 1]; ++j)
      out[j] = vsko_hnsw_distance(q + i * d, x + (int64_t)rows[j] * d, d, metric);
}

/* normalizeVectors (Acceleration/Metal/Shaders/DistanceShaders.metal:
 * 403-429): magnitude = sum of x_i * x_i in index order, then
 * sqrt(magnitude) + 1e-8, then every component divided by it (a division,
 * not a multiply by the reciprocal). */
void vsko_normalize(const float *x, int64_t n, int32_t d, float *out) {
  for (int64_t r = 0; r < n; ++r) {
    const float *xr = x + r * d;
    float m = 0.0f;
    for (int32_t i = 0; i < d; ++i) {
      float v = xr[i];
      m += v * v;
    }
    m = sqrtf(m) + 1e-8f;
    for (int32_t i = 0; i < d; ++i) out[r * d + i] = xr[i] / m;
  }
}

/* matrixMultiply's CPU loop (Acceleration/Metal/MetalMatrixCompute.swift:
 * 791-806): result[i][j] starts at 0 and adds a[i][t] * b[t][j] for t in
 * order (a product, then a sum).  a is m x k, b is k x n, c is m x n, all
 * row-major. */
void vsko_matmul(const float *a, int64_t m, int32_t k, const float *b, int64_t n, float *c) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float s = 0.0f;
      for (int32_t t = 0; t < k; ++t) s += a[i * k + t] * b[(int64_t)t * n + j];
      c[i * n + j] = s;
    }
}

/* 16 independent accumulators: what a SIMD library loop does.  Used only by
 * the CPU-baseline timing (fast != 0), never by parity checks. */
static float dot16(const float *a, const float *b, int32_t d) {
  float acc[16] = {0};
  int32_t i = 0;
  for (; i + 16 <= d; i += 16)
    for (int j = 0; j < 16; ++j) acc[j] += a[i + j] * b[i + j];
  float s = 0.0f;
  for (int j = 0; j < 16; ++j) s += acc[j];
  for (; i < d; ++i) s += a[i] * b[i];
  return s;
}
static float l2sq16(const float *a, const float *b, int32_t d) {
  float acc[16] = {0};
  int32_t i = 0;
  for (; i + 16 <= d; i += 16)
    for (int j = 0; j < 16; ++j) {
      float t = a[i + j] - b[i + j];
      acc[j] += t * t;
    }
  float s = 0.0f;
  for (int j = 0; j < 16; ++j) s += acc[j];
  for (; i < d; ++i) {
    float t = a[i] - b[i];
    s += t * t;
  }
  return s;
}
static float l116(const float *a, const float *b, int32_t d) {
  float acc[16] = {0};
  int32_t i = 0;
  for (; i + 16 <= d; i += 16)
    for (int j = 0; j < 16; ++j) acc[j] += fabsf(a[i + j] - b[i + j]);
  float s = 0.0f;
  for (int j = 0; j < 16; ++j) s += acc[j];
  for (; i < d; ++i) s += fabsf(a[i] - b[i]);
  return s;
}
static float distance_fast(const float *q, const float *x, int32_t d,
                           int32_t metric, float qnorm) {
  switch (metric) {
  case VSKO_L2SQ:
    return l2sq16(q, x, d);
  case VSKO_L2:
    return sqrtf(l2sq16(q, x, d));
  case VSKO_COSINE: {
    float xn = sqrtf(dot16(x, x, d));
    return 1.0f - dot16(q, x, d) / (qnorm * xn + 1e-8f);
  }
  case VSKO_COSINE_NORMALIZED:
    return 1.0f - dot16(q, x, d);
  case VSKO_DOT:
    return -dot16(q, x, d);
  case VSKO_L1:
    return l116(q, x, d);
  case VSKO_HAMMING:
    return vsko_distance(q, x, d, VSKO_HAMMING);
  default:
    return NAN;
  }
}

typedef struct {
  const float *q, *x;
  int64_t n;
  int32_t d, metric;
  float *out;
} dist_ctx;
static void dist_range(void *p, int64_t lo, int64_t hi) {
  dist_ctx *c = (dist_ctx *)p;
  for (int64_t i = lo; i < hi; ++i)
    for (int64_t j = 0; j < c->n; ++j)
      c->out[i * c->n + j] =
          vsko_distance(c->q + i * c->d, c->x + j * c->d, c->d, c->metric);
}
void vsko_distances(const float *q, int64_t nq, const float *x, int64_t n,
                    int32_t d, int32_t metric, float *out, int32_t nthreads) {
  dist_ctx c = {q, x, n, d, metric, out};
  parallel_for(nq, nthreads, dist_range, &c);
}

/* ------------------------------------------------------------------------ */
/* top-k: k smallest by (value, tie) ascending                                */
/* ------------------------------------------------------------------------ */
typedef struct {
  float v;
  int64_t t; /* tie key */
} pair_t;

static int pair_less(pair_t a, pair_t b) {
  return a.v < b.v || (a.v == b.v && a.t < b.t);
}

/* max-heap of size k on (v, t): root = current worst kept element */
static void heap_sift_down(pair_t *h, int32_t n, int32_t i) {
  for (;;) {
    int32_t l = 2 * i + 1, r = l + 1, m = i;
    if (l < n && pair_less(h[m], h[l])) m = l;
    if (r < n && pair_less(h[m], h[r])) m = r;
    if (m == i) return;
    pair_t t = h[i];
    h[i] = h[m];
    h[m] = t;
    i = m;
  }
}
static void heap_sift_up(pair_t *h, int32_t i) {
  while (i > 0) {
    int32_t p = (i - 1) / 2;
    if (!pair_less(h[p], h[i])) return;
    pair_t t = h[i];
    h[i] = h[p];
    h[p] = t;
    i = p;
  }
}
typedef struct {
  pair_t *h;
  int32_t n, k;
} topk_t;
static void topk_push(topk_t *s, float v, int64_t t) {
  pair_t p = {v, t};
  if (s->n < s->k) {
    s->h[s->n] = p;
    heap_sift_up(s->h, s->n);
    s->n++;
  } else if (s->k > 0 && pair_less(p, s->h[0])) {
    s->h[0] = p;
    heap_sift_down(s->h, s->n, 0);
  }
}
static int pair_cmp(const void *a, const void *b) {
  pair_t x = *(const pair_t *)a, y = *(const pair_t *)b;
  if (pair_less(x, y)) return -1;
  if (pair_less(y, x)) return 1;
  return 0;
}
/* sorted ascending into out; slots past the kept count get (inf, -1) */
static void topk_finish(topk_t *s, float *out_v, int64_t *out_t) {
  qsort(s->h, (size_t)s->n, sizeof(pair_t), pair_cmp);
  for (int32_t i = 0; i < s->k; ++i) {
    if (i < s->n) {
      out_v[i] = s->h[i].v;
      out_t[i] = s->h[i].t;
    } else {
      out_v[i] = INFINITY;
      out_t[i] = -1;
    }
  }
}

/* The selection the reference's stable sort + prefix(k) performs
 * (Indexes/IVFIndex.swift:175-176), with ties broken by index; it does NOT
 * reproduce AccelerateOptimizer.selectTopK's k>=10 heap branch
 * (Acceleration/AccelerateOptimizer.swift:136-148), which keeps a min-heap
 * and so returns the wrong elements. */
void vsko_topk(const float *dist, int64_t n, int32_t k, float *out_dist,
               int64_t *out_idx) {
  topk_t s = {(pair_t *)malloc(sizeof(pair_t) * (k > 0 ? k : 1)), 0, k};
  for (int64_t i = 0; i < n; ++i) topk_push(&s, dist[i], i);
  topk_finish(&s, out_dist, out_idx);
  free(s.h);
}

/* ------------------------------------------------------------------------ */
/* flat exact search                                                          */
/* ------------------------------------------------------------------------ */
typedef struct {
  const float *q, *x;
  int64_t n;
  int32_t d, k, metric, fast;
  float *od;
  int64_t *oi;
} flat_ctx;

/* per query: distance to every row (Acceleration/AccelerateOptimizer.swift:
 * 96-121 batchComputeDistances -> computeDistances), then the k smallest. */
static void flat_range(void *p, int64_t lo, int64_t hi) {
  flat_ctx *c = (flat_ctx *)p;
  topk_t s = {(pair_t *)malloc(sizeof(pair_t) * (c->k > 0 ? c->k : 1)), 0,
              c->k};
  for (int64_t i = lo; i < hi; ++i) {
    const float *qi = c->q + i * c->d;
    float qn = sqrtf(dot16(qi, qi, c->d));
    s.n = 0;
    for (int64_t j = 0; j < c->n; ++j) {
      const float *xj = c->x + j * c->d;
      float v = c->fast ? distance_fast(qi, xj, c->d, c->metric, qn)
                        : vsko_distance(qi, xj, c->d, c->metric);
      topk_push(&s, v, j);
    }
    topk_finish(&s, c->od + i * c->k, c->oi + i * c->k);
  }
  free(s.h);
}
/* ---- the exact path vectorised across rows ------------------------------
 * Each SIMD lane holds one row's running sum, taken in dimension order with
 * no FMA, so every lane computes exactly what vsko_distance computes for its
 * row; only the rows are processed side by side.  Rows are first copied into
 * blocks of RB rows stored dimension-major (xt[(b*d + i)*RB + r] = row
 * b*RB + r, dimension i; rows past n are zero and never reported). */
#define RB 16
#define QG 4
typedef float vrow __attribute__((vector_size(RB * 4), aligned(64)));
typedef int32_t vrowi __attribute__((vector_size(RB * 4), aligned(64)));

typedef struct {
  const float *x;
  int64_t n;
  int32_t d;
  float *xt;
  float *xnorm; /* sqrtf(sum x^2) per row, COSINE only */
} xt_ctx;
static void xt_range(void *p, int64_t lo, int64_t hi) {
  xt_ctx *c = (xt_ctx *)p;
  const int32_t d = c->d;
  for (int64_t b = lo; b < hi; ++b) {
    float *blk = c->xt + b * (int64_t)d * RB;
    for (int32_t r = 0; r < RB; ++r) {
      const int64_t row = b * RB + r;
      const float *xr = row < c->n ? c->x + row * d : NULL;
      for (int32_t i = 0; i < d; ++i) blk[(int64_t)i * RB + r] = xr ? xr[i] : 0.0f;
    }
    if (c->xnorm) {
      vrow a = {0};
      for (int32_t i = 0; i < d; ++i) {
        vrow v = *(const vrow *)(blk + (int64_t)i * RB);
        a += v * v;
      }
      for (int32_t r = 0; r < RB && b * RB + r < c->n; ++r) c->xnorm[b * RB + r] = sqrtf(a[r]);
    }
  }
}

/* acc[g][r] = the metric's running sum for query g and row r of one block.
 * A block's RB = 16 lanes are two 8-lane halves (AVX2 registers), so the
 * 4 x 2 accumulators stay in registers. */
typedef float v8f __attribute__((vector_size(32)));
typedef int32_t v8i __attribute__((vector_size(32)));
#define V8_STEP(OP)                                                             \
  for (int32_t i = 0; i < d; ++i) {                                             \
    const v8f xl = *(const v8f *)(blk + (int64_t)i * RB);                       \
    const v8f xh = *(const v8f *)(blk + (int64_t)i * RB + 8);                   \
    const float s0 = q0[i], s1 = q1[i], s2 = q2[i], s3 = q3[i];                 \
    OP(a0l, a0h, s0);                                                           \
    OP(a1l, a1h, s1);                                                           \
    OP(a2l, a2h, s2);                                                           \
    OP(a3l, a3h, s3);                                                           \
  }
#define OP_L2(al, ah, sc)                                                       \
  {                                                                             \
    v8f tl = sc - xl, th = sc - xh;                                             \
    al += tl * tl;                                                              \
    ah += th * th;                                                              \
  }
#define OP_L1(al, ah, sc)                                                       \
  {                                                                             \
    v8f tl = sc - xl, th = sc - xh;                                             \
    al += (v8f)((v8i)tl & absmask);                                             \
    ah += (v8f)((v8i)th & absmask);                                             \
  }
#define OP_DOT(al, ah, sc)                                                      \
  {                                                                             \
    al += sc * xl;                                                              \
    ah += sc * xh;                                                              \
  }
static void block_sums(const float *blk, int32_t d, const float *const *qs, int32_t metric,
                       vrow acc[QG]) {
  v8f a0l = {0}, a0h = {0}, a1l = {0}, a1h = {0}, a2l = {0}, a2h = {0}, a3l = {0}, a3h = {0};
  const float *q0 = qs[0], *q1 = qs[1], *q2 = qs[2], *q3 = qs[3];
  const v8i absmask = (v8i){0} + 0x7fffffff;
  switch (metric) {
  case VSKO_L2SQ:
  case VSKO_L2:
    V8_STEP(OP_L2);
    break;
  case VSKO_L1:
    V8_STEP(OP_L1);
    break;
  default: /* the dot-product metrics */
    V8_STEP(OP_DOT);
  }
  for (int r = 0; r < 8; ++r) {
    acc[0][r] = a0l[r], acc[0][r + 8] = a0h[r];
    acc[1][r] = a1l[r], acc[1][r + 8] = a1h[r];
    acc[2][r] = a2l[r], acc[2][r + 8] = a2h[r];
    acc[3][r] = a3l[r], acc[3][r + 8] = a3h[r];
  }
}

typedef struct {
  const float *q, *xt, *xnorm;
  int64_t n;
  int32_t d, k, metric;
  float *od;
  int64_t *oi;
} flatv_ctx;

/* vsko_distance's final step on a lane's sum (same operations, same order) */
static float finish_sum(float s, int32_t metric, float qn, float xn) {
  switch (metric) {
  case VSKO_L2:
    return sqrtf(s);
  case VSKO_COSINE:
    return 1.0f - s / (qn * xn + 1e-8f);
  case VSKO_COSINE_NORMALIZED:
    return 1.0f - s;
  case VSKO_DOT:
    return -s;
  default: /* L2SQ, L1 */
    return s;
  }
}

static void flatv_range(void *p, int64_t lo, int64_t hi) {
  flatv_ctx *c = (flatv_ctx *)p;
  const int64_t m = hi - lo;
  if (m <= 0) return;
  const int32_t d = c->d, k = c->k;
  topk_t *heaps = (topk_t *)malloc(sizeof(topk_t) * (size_t)m);
  pair_t *store = (pair_t *)malloc(sizeof(pair_t) * (size_t)m * (k > 0 ? k : 1));
  float *qn = (float *)malloc(sizeof(float) * (size_t)m);
  for (int64_t i = 0; i < m; ++i) {
    heaps[i].h = store + i * (k > 0 ? k : 1);
    heaps[i].n = 0;
    heaps[i].k = k;
    const float *qi = c->q + (lo + i) * d;
    qn[i] = c->metric == VSKO_COSINE ? sqrtf(vsko_dot(qi, qi, d)) : 0.0f;
  }
  const int64_t nblocks = (c->n + RB - 1) / RB;
  vrow acc[QG];
  for (int64_t b = 0; b < nblocks; ++b) {
    const float *blk = c->xt + b * (int64_t)d * RB;
    const int32_t rows = (int32_t)(c->n - b * RB < RB ? c->n - b * RB : RB);
    for (int64_t g0 = 0; g0 < m; g0 += QG) {
      const float *qs[QG];
      const int32_t ng = (int32_t)(m - g0 < QG ? m - g0 : QG);
      for (int32_t g = 0; g < QG; ++g) qs[g] = c->q + (lo + g0 + (g < ng ? g : 0)) * d;
      block_sums(blk, d, qs, c->metric, acc);
      for (int32_t g = 0; g < ng; ++g)
        for (int32_t r = 0; r < rows; ++r) {
          const int64_t row = b * RB + r;
          const float xn = c->xnorm ? c->xnorm[row] : 0.0f;
          topk_push(&heaps[g0 + g], finish_sum(acc[g][r], c->metric, qn[g0 + g], xn), row);
        }
    }
  }
  for (int64_t i = 0; i < m; ++i)
    topk_finish(&heaps[i], c->od + (lo + i) * k, c->oi + (lo + i) * k);
  free(qn);
  free(store);
  free(heaps);
}

/* A database in the row-vectorised layout (and its row norms), made once
 * and searched many times, as a CPU index keeps its rows resident. */
struct vsko_flatdb {
  int64_t n;
  int32_t d;
  float *xt, *xnorm;
};

vsko_flatdb *vsko_flat_prepare(const float *x, int64_t n, int32_t d, int32_t nthreads) {
  if (n <= 0 || d <= 0) return NULL;
  vsko_flatdb *db = (vsko_flatdb *)malloc(sizeof(vsko_flatdb));
  const int64_t nblocks = (n + RB - 1) / RB;
  db->n = n;
  db->d = d;
  db->xt = (float *)aligned_alloc(64, sizeof(float) * (size_t)nblocks * d * RB);
  db->xnorm = (float *)malloc(sizeof(float) * (size_t)n);
  xt_ctx tc = {x, n, d, db->xt, db->xnorm};
  parallel_for(nblocks, nthreads, xt_range, &tc);
  return db;
}

void vsko_flat_free(vsko_flatdb *db) {
  if (!db) return;
  free(db->xt);
  free(db->xnorm);
  free(db);
}

/* the exact flat search over a prepared database (not the hamming metric) */
void vsko_flat_search(const vsko_flatdb *db, const float *q, int64_t nq, int32_t k,
                      int32_t metric, float *out_dist, int64_t *out_ids, int32_t nthreads) {
  flatv_ctx c = {q, db->xt, metric == VSKO_COSINE ? db->xnorm : NULL, db->n, db->d, k,
                 metric, out_dist, out_ids};
  parallel_for(nq, nthreads, flatv_range, &c);
}

void vsko_search_flat(const float *q, int64_t nq, const float *x, int64_t n,
                      int32_t d, int32_t k, int32_t metric, float *out_dist,
                      int64_t *out_ids, int32_t nthreads, int32_t fast) {
  if (fast || metric == VSKO_HAMMING || n <= 0 || d <= 0) {
    flat_ctx c = {q, x, n, d, k, metric, fast, out_dist, out_ids};
    parallel_for(nq, nthreads, flat_range, &c);
    return;
  }
  vsko_flatdb *db = vsko_flat_prepare(x, n, d, nthreads);
  vsko_flat_search(db, q, nq, k, metric, out_dist, out_ids, nthreads);
  vsko_flat_free(db);
}

/* ------------------------------------------------------------------------ */
/* IVF-Flat                                                                   */
/* ------------------------------------------------------------------------ */
typedef struct {
  const float *x, *c;
  int32_t nlist, d;
  int32_t *out;
} assign_ctx;
/* Indexes/IVFIndex.swift:514-527 findNearestCentroid: distance =
 * sqrt(sum diff^2) (:542-549), strict '<' so the first minimum wins. */
static void assign_range(void *p, int64_t lo, int64_t hi) {
  assign_ctx *a = (assign_ctx *)p;
  for (int64_t i = lo; i < hi; ++i) {
    float best = INFINITY;
    int32_t bi = 0;
    for (int32_t c = 0; c < a->nlist; ++c) {
      float v = sqrtf(vsko_l2sq(a->x + i * a->d, a->c + (int64_t)c * a->d,
                                a->d));
      if (v < best) {
        best = v;
        bi = c;
      }
    }
    a->out[i] = bi;
  }
}
void vsko_ivf_assign(const float *x, int64_t n, const float *centroids,
                     int32_t nlist, int32_t d, int32_t *out_list,
                     int32_t nthreads) {
  assign_ctx a = {x, centroids, nlist, d, out_list};
  parallel_for(n, nthreads, assign_range, &a);
}

/* Indexes/IVFIndex.swift:529-540 findNearestCentroids: sqrt-L2 to every
 * centroid, stable sort ascending, first `count` indices. */
static void probe_one(const float *q, const float *centroids, int32_t nlist,
                      int32_t d, int32_t nprobe, int32_t *out, pair_t *buf) {
  topk_t s = {buf, 0, nprobe};
  for (int32_t c = 0; c < nlist; ++c)
    topk_push(&s, sqrtf(vsko_l2sq(q, centroids + (int64_t)c * d, d)), c);
  qsort(s.h, (size_t)s.n, sizeof(pair_t), pair_cmp);
  for (int32_t i = 0; i < nprobe; ++i)
    out[i] = i < s.n ? (int32_t)s.h[i].t : -1;
}
typedef struct {
  const float *q, *c;
  int32_t nlist, d, nprobe;
  int32_t *out;
} probe_ctx;
static void probe_range(void *p, int64_t lo, int64_t hi) {
  probe_ctx *a = (probe_ctx *)p;
  pair_t *buf = (pair_t *)malloc(sizeof(pair_t) * (a->nprobe + 1));
  for (int64_t i = lo; i < hi; ++i)
    probe_one(a->q + i * a->d, a->c, a->nlist, a->d, a->nprobe,
              a->out + i * a->nprobe, buf);
  free(buf);
}
void vsko_ivf_probe(const float *q, int64_t nq, const float *centroids,
                    int32_t nlist, int32_t d, int32_t nprobe,
                    int32_t *out_lists, int32_t nthreads) {
  probe_ctx a = {q, centroids, nlist, d, nprobe, out_lists};
  parallel_for(nq, nthreads, probe_range, &a);
}

typedef struct {
  const float *q, *x, *c;
  const int64_t *ids;
  const int64_t *list_start; /* [nlist+1] offsets into rows_by_list */
  const int64_t *rows_by_list;
  int32_t d, nlist, nprobe, k, squared;
  float *od;
  int64_t *oi;
} ivf_ctx;

/* Indexes/IVFIndex.swift:124-176: probe (:147-148), concatenate the probed
 * lists in probe order (:151-157), exact sqrt-L2 per candidate (:167-172),
 * stable sort + prefix(k) (:175-176).  The tie key is the position in the
 * concatenation, which is what a stable sort keeps. */
static void ivf_range(void *p, int64_t lo, int64_t hi) {
  ivf_ctx *a = (ivf_ctx *)p;
  int32_t *probes = (int32_t *)malloc(sizeof(int32_t) * a->nprobe);
  pair_t *pbuf = (pair_t *)malloc(sizeof(pair_t) * (a->nprobe + 1));
  pair_t *kbuf = (pair_t *)malloc(sizeof(pair_t) * (a->k > 0 ? a->k : 1));
  int64_t *pos_row = NULL;
  int64_t cap = 0;
  for (int64_t i = lo; i < hi; ++i) {
    const float *qi = a->q + i * a->d;
    probe_one(qi, a->c, a->nlist, a->d, a->nprobe, probes, pbuf);
    topk_t s = {kbuf, 0, a->k};
    int64_t pos = 0;
    for (int32_t pi = 0; pi < a->nprobe; ++pi) {
      int32_t l = probes[pi];
      if (l < 0) continue;
      int64_t b = a->list_start[l], e = a->list_start[l + 1];
      if (pos + (e - b) > cap) {
        cap = (pos + (e - b)) * 2;
        pos_row = (int64_t *)realloc(pos_row, sizeof(int64_t) * cap);
      }
      for (int64_t r = b; r < e; ++r) {
        int64_t row = a->rows_by_list[r];
        float s2 = vsko_l2sq(qi, a->x + row * a->d, a->d);
        float v = a->squared ? s2 : sqrtf(s2);
        pos_row[pos] = row;
        topk_push(&s, v, pos);
        ++pos;
      }
    }
    topk_finish(&s, a->od + i * a->k, a->oi + i * a->k);
    for (int32_t j = 0; j < a->k; ++j) {
      int64_t ps = a->oi[i * a->k + j];
      a->oi[i * a->k + j] = ps >= 0 ? a->ids[pos_row[ps]] : -1;
    }
  }
  free(pos_row);
  free(kbuf);
  free(pbuf);
  free(probes);
}

void vsko_ivf_search(const float *q, int64_t nq, const float *x,
                     const int64_t *ids, const int32_t *list_of, int64_t n,
                     int32_t d, const float *centroids, int32_t nlist,
                     int32_t nprobe, int32_t k, int32_t squared,
                     float *out_dist, int64_t *out_ids, int32_t nthreads) {
  /* inverted lists keep insertion order (Indexes/IVFIndex.swift:80-122
   * appends to invertedLists[nearest]) */
  int64_t *start = (int64_t *)calloc((size_t)nlist + 1, sizeof(int64_t));
  int64_t *rows = (int64_t *)malloc(sizeof(int64_t) * (n > 0 ? n : 1));
  for (int64_t i = 0; i < n; ++i) start[list_of[i] + 1]++;
  for (int32_t l = 0; l < nlist; ++l) start[l + 1] += start[l];
  int64_t *fill = (int64_t *)malloc(sizeof(int64_t) * (nlist + 1));
  memcpy(fill, start, sizeof(int64_t) * (nlist + 1));
  for (int64_t i = 0; i < n; ++i) rows[fill[list_of[i]]++] = i;
  free(fill);
  ivf_ctx a = {q, x,      centroids, ids, start,    rows,   d,
               nlist, nprobe, k,      squared ? 1 : 0, out_dist, out_ids};
  parallel_for(nq, nthreads, ivf_range, &a);
  free(rows);
  free(start);
}

/* ------------------------------------------------------------------------ */
/* scalar quantization, int8                                                  */
/* ------------------------------------------------------------------------ */

/* Quantization/ScalarQuantizer.swift:389-418 (min/max over the values) and
 * :420-451 (.int8: scale = 255/(max-min), offset = -min*scale - 128).  The
 * reference uses the global min/max; per_dim applies the same formulas per
 * column.  A zero range would give an infinite scale in the reference; here
 * scale = 1 is used so every value maps to -128. */
static void sq8_params(float mn, float mx, float *s, float *o) {
  float range = mx - mn;
  float scale = range > 0.0f ? 255.0f / range : 1.0f;
  *s = scale;
  *o = -mn * scale - 128.0f;
}
void vsko_sq8_train(const float *x, int64_t n, int32_t d, int32_t per_dim,
                    float *scale, float *offset) {
  if (per_dim) {
    for (int32_t j = 0; j < d; ++j) {
      float mn = INFINITY, mx = -INFINITY;
      for (int64_t i = 0; i < n; ++i) {
        float v = x[i * d + j];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
      }
      sq8_params(mn, mx, &scale[j], &offset[j]);
    }
  } else {
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < n * d; ++i) {
      if (x[i] < mn) mn = x[i];
      if (x[i] > mx) mx = x[i];
    }
    sq8_params(mn, mx, &scale[0], &offset[0]);
  }
}

/* Quantization/ScalarQuantizer.swift:251-270 quantizeToInt8:
 * vDSP_vsmsa (t = x*scale + offset) then vDSP_vfix8 (conversion toward
 * zero).  Out-of-range values are clamped to [-128, 127] here (vDSP_vfix8's
 * out-of-range behaviour is not published). */
static int8_t sq8_code(float v, float s, float o) {
  float t = v * s;
  t = t + o;
  if (!(t > -128.0f)) return -128; /* also NaN */
  if (t >= 127.0f) return 127;
  return (int8_t)(int32_t)t; /* C conversion truncates toward zero */
}
void vsko_sq8_encode(const float *x, int64_t n, int32_t d, int32_t per_dim,
                     const float *scale, const float *offset, int8_t *codes) {
  for (int64_t i = 0; i < n; ++i)
    for (int32_t j = 0; j < d; ++j) {
      float s = per_dim ? scale[j] : scale[0];
      float o = per_dim ? offset[j] : offset[0];
      codes[i * d + j] = sq8_code(x[i * d + j], s, o);
    }
}
/* Quantization/ScalarQuantizer.swift:568-580 dequantizeFromInt8:
 * (code - offset) / scale */
void vsko_sq8_decode(const int8_t *codes, int64_t n, int32_t d,
                     int32_t per_dim, const float *scale, const float *offset,
                     float *out) {
  for (int64_t i = 0; i < n; ++i)
    for (int32_t j = 0; j < d; ++j) {
      float s = per_dim ? scale[j] : scale[0];
      float o = per_dim ? offset[j] : offset[0];
      out[i * d + j] = ((float)codes[i * d + j] - o) / s;
    }
}
/* exact integer dot of two code vectors (the int32-accumulated score the
 * scan ranks by; the reference has no int8 distance, so this is the
 * documented build rule: distance = -score). */
int32_t vsko_sq8_dot(const int8_t *a, const int8_t *b, int32_t d) {
  int32_t s = 0;
  for (int32_t i = 0; i < d; ++i) s += (int32_t)a[i] * (int32_t)b[i];
  return s;
}
typedef struct {
  const int8_t *q, *x;
  int64_t n;
  int32_t d, k;
  int32_t *os;
  int64_t *oi;
} sq8_ctx;
/* top-k on integer keys (distance = -score as int64, tie = row): the same
 * max-heap as pair_t, exact for any score */
typedef struct {
  int64_t v, t;
} ipair_t;
static int ipair_less(ipair_t a, ipair_t b) { return a.v < b.v || (a.v == b.v && a.t < b.t); }
static void iheap_push(ipair_t *h, int32_t *n, int32_t k, ipair_t p) {
  if (*n < k) {
    int32_t i = (*n)++;
    h[i] = p;
    while (i > 0) {
      int32_t up = (i - 1) / 2;
      if (!ipair_less(h[up], h[i])) break;
      ipair_t t = h[i];
      h[i] = h[up];
      h[up] = t;
      i = up;
    }
  } else if (k > 0 && ipair_less(p, h[0])) {
    h[0] = p;
    for (int32_t i = 0;;) {
      int32_t l = 2 * i + 1, r = l + 1, m = i;
      if (l < *n && ipair_less(h[m], h[l])) m = l;
      if (r < *n && ipair_less(h[m], h[r])) m = r;
      if (m == i) break;
      ipair_t t = h[i];
      h[i] = h[m];
      h[m] = t;
      i = m;
    }
  }
}
static int ipair_cmp(const void *a, const void *b) {
  ipair_t x = *(const ipair_t *)a, y = *(const ipair_t *)b;
  return ipair_less(x, y) ? -1 : (ipair_less(y, x) ? 1 : 0);
}

static void sq8_range(void *p, int64_t lo, int64_t hi) {
  sq8_ctx *c = (sq8_ctx *)p;
  ipair_t *h = (ipair_t *)malloc(sizeof(ipair_t) * (c->k > 0 ? c->k : 1));
  for (int64_t i = lo; i < hi; ++i) {
    int32_t m = 0;
    for (int64_t j = 0; j < c->n; ++j) {
      ipair_t e = {-(int64_t)vsko_sq8_dot(c->q + i * c->d, c->x + j * c->d, c->d), j};
      iheap_push(h, &m, c->k, e);
    }
    qsort(h, (size_t)m, sizeof(ipair_t), ipair_cmp);
    for (int32_t t = 0; t < c->k; ++t) {
      c->os[i * c->k + t] = t < m ? (int32_t)(-h[t].v) : INT32_MIN;
      c->oi[i * c->k + t] = t < m ? h[t].t : -1;
    }
  }
  free(h);
}
/* Keys are the int64 negated scores, so the order is exact for any d (an
 * int32 score itself holds |score| <= 128 * 128 * d for d < 131072). */
void vsko_sq8_search(const int8_t *qcodes, int64_t nq, const int8_t *codes,
                     int64_t n, int32_t d, int32_t k, int32_t *out_score,
                     int64_t *out_ids, int32_t nthreads) {
  sq8_ctx c = {qcodes, codes, n, d, k, out_score, out_ids};
  parallel_for(nq, nthreads, sq8_range, &c);
}

/* ------------------------------------------------------------------------ */
/* product quantization                                                       */
/* ------------------------------------------------------------------------ */

/* Quantization/ProductQuantizer.swift:209-233 precomputeDistanceTables:
 * table[m][c] = euclideanDistanceSquared(q segment m, codeword c)
 * (:362-369, sequential, no FMA). */
void vsko_pq_lut(const float *q, const float *codebooks, int32_t M,
                 int32_t ksub, int32_t dsub, float *lut) {
  for (int32_t m = 0; m < M; ++m)
    for (int32_t c = 0; c < ksub; ++c)
      lut[m * ksub + c] = vsko_l2sq(
          q + m * dsub, codebooks + ((int64_t)m * ksub + c) * dsub, dsub);
}

/* Quantization/ProductQuantizerCodebook.swift:12-30 Codebook.encode:
 * argmin over codewords of the squared distance, strict '<'. */
typedef struct {
  const float *x, *cb;
  int32_t M, ksub, dsub;
  uint8_t *codes;
} pqenc_ctx;
static void pqenc_range(void *p, int64_t lo, int64_t hi) {
  pqenc_ctx *a = (pqenc_ctx *)p;
  int32_t d = a->M * a->dsub;
  for (int64_t i = lo; i < hi; ++i)
    for (int32_t m = 0; m < a->M; ++m) {
      float best = INFINITY;
      int32_t bc = 0;
      for (int32_t c = 0; c < a->ksub; ++c) {
        float v = vsko_l2sq(a->x + i * d + m * a->dsub,
                            a->cb + ((int64_t)m * a->ksub + c) * a->dsub,
                            a->dsub);
        if (v < best) {
          best = v;
          bc = c;
        }
      }
      a->codes[i * a->M + m] = (uint8_t)bc;
    }
}
void vsko_pq_encode(const float *x, int64_t n, const float *codebooks,
                    int32_t M, int32_t ksub, int32_t dsub, uint8_t *codes,
                    int32_t nthreads) {
  pqenc_ctx a = {x, codebooks, M, ksub, dsub, codes};
  parallel_for(n, nthreads, pqenc_range, &a);
}
/* Quantization/ProductQuantizerCodebook.swift:32-34 decode (codeword copy) */
void vsko_pq_decode(const uint8_t *codes, int64_t n, const float *codebooks,
                    int32_t M, int32_t ksub, int32_t dsub, float *out) {
  for (int64_t i = 0; i < n; ++i)
    for (int32_t m = 0; m < M; ++m)
      memcpy(out + i * M * dsub + m * dsub,
             codebooks + ((int64_t)m * ksub + codes[i * M + m]) * dsub,
             sizeof(float) * dsub);
}

/* Quantization/ProductQuantizerTypes.swift:14-20 DistanceTables.computeDistance
 * before its sqrt: sum over segments in ascending order, starting at 0. */
float vsko_pq_adc_sum(const float *lut, const uint8_t *code, int32_t M,
                      int32_t ksub) {
  float s = 0.0f;
  for (int32_t m = 0; m < M; ++m) s += lut[m * ksub + code[m]];
  return s;
}
void vsko_pq_adc_scan(const float *lut, const uint8_t *codes, int64_t n,
                      int32_t M, int32_t ksub, float *out_sum) {
  for (int64_t i = 0; i < n; ++i)
    out_sum[i] = vsko_pq_adc_sum(lut, codes + i * M, M, ksub);
}

typedef struct {
  const float *q, *cb, *x;
  const uint8_t *codes;
  int64_t n;
  int32_t M, ksub, dsub, k_adc, k, rerank;
  float *od;
  int64_t *oi;
} pqs_ctx;
static void pqs_range(void *p, int64_t lo, int64_t hi) {
  pqs_ctx *a = (pqs_ctx *)p;
  int32_t d = a->M * a->dsub;
  float *lut = (float *)malloc(sizeof(float) * a->M * a->ksub);
  pair_t *buf = (pair_t *)malloc(sizeof(pair_t) * (a->k_adc > 0 ? a->k_adc : 1));
  pair_t *buf2 = (pair_t *)malloc(sizeof(pair_t) * (a->k > 0 ? a->k : 1));
  float *cd = (float *)malloc(sizeof(float) * (a->k_adc > 0 ? a->k_adc : 1));
  int64_t *ci = (int64_t *)malloc(sizeof(int64_t) * (a->k_adc > 0 ? a->k_adc : 1));
  for (int64_t i = lo; i < hi; ++i) {
    const float *qi = a->q + i * d;
    vsko_pq_lut(qi, a->cb, a->M, a->ksub, a->dsub, lut);
    topk_t s = {buf, 0, a->k_adc};
    for (int64_t j = 0; j < a->n; ++j)
      topk_push(&s, vsko_pq_adc_sum(lut, a->codes + j * a->M, a->M, a->ksub),
                j);
    topk_finish(&s, cd, ci);
    if (a->x && a->rerank >= 0) {
      topk_t s2 = {buf2, 0, a->k};
      for (int32_t t = 0; t < a->k_adc; ++t)
        if (ci[t] >= 0)
          topk_push(&s2, vsko_distance(qi, a->x + ci[t] * d, d, a->rerank),
                    ci[t]);
      topk_finish(&s2, a->od + i * a->k, a->oi + i * a->k);
    } else {
      for (int32_t t = 0; t < a->k; ++t) {
        a->od[i * a->k + t] =
            t < a->k_adc && ci[t] >= 0 ? sqrtf(cd[t]) : INFINITY;
        a->oi[i * a->k + t] = t < a->k_adc ? ci[t] : -1;
      }
    }
  }
  free(ci);
  free(cd);
  free(buf2);
  free(buf);
  free(lut);
}
void vsko_pq_search(const float *q, int64_t nq, const float *codebooks,
                    const uint8_t *codes, int64_t n, int32_t M, int32_t ksub,
                    int32_t dsub, int32_t k_adc, int32_t k, const float *x,
                    int32_t rerank_metric, float *out_dist, int64_t *out_ids,
                    int32_t nthreads) {
  pqs_ctx a = {q,    codebooks, x,     codes, n,        M,       ksub,
               dsub, k_adc,     k,     rerank_metric, out_dist, out_ids};
  parallel_for(nq, nthreads, pqs_range, &a);
}

/* ------------------------------------------------------------------------ */
/* k-means (used only to make test fixtures: PQ codebooks)                    */
/* ------------------------------------------------------------------------ */
static uint64_t splitmix64(uint64_t *s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
typedef struct {
  const float *x, *c;
  int32_t d, k;
  int32_t *assign;
} km_ctx;
static void km_assign_range(void *p, int64_t lo, int64_t hi) {
  km_ctx *a = (km_ctx *)p;
  for (int64_t i = lo; i < hi; ++i) {
    float best = INFINITY;
    int32_t bi = 0;
    for (int32_t c = 0; c < a->k; ++c) {
      float v = vsko_l2sq(a->x + i * a->d, a->c + (int64_t)c * a->d, a->d);
      if (v < best) {
        best = v;
        bi = c;
      }
    }
    a->assign[i] = bi;
  }
}
/* Clustering/KMeansClustering.swift:48-113 (Lloyd loop), :271-295
 * (assignment with strict '<'), :342-380 (mean update).  Initialisation
 * here is a seeded sample of k distinct rows, not k-means++. */
void vsko_kmeans(const float *x, int64_t n, int32_t d, int32_t k,
                 int32_t iters, uint64_t seed, float *centroids,
                 int32_t nthreads) {
  int64_t *perm = (int64_t *)malloc(sizeof(int64_t) * n);
  for (int64_t i = 0; i < n; ++i) perm[i] = i;
  uint64_t st = seed;
  for (int64_t i = 0; i < k && i < n; ++i) {
    int64_t j = i + (int64_t)(splitmix64(&st) % (uint64_t)(n - i));
    int64_t t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
  for (int32_t c = 0; c < k; ++c)
    memcpy(centroids + (int64_t)c * d, x + perm[c % n] * d,
           sizeof(float) * d);
  free(perm);
  int32_t *assign = (int32_t *)malloc(sizeof(int32_t) * n);
  double *sum = (double *)malloc(sizeof(double) * (size_t)k * d);
  int64_t *cnt = (int64_t *)malloc(sizeof(int64_t) * k);
  for (int32_t it = 0; it < iters; ++it) {
    km_ctx a = {x, centroids, d, k, assign};
    parallel_for(n, nthreads, km_assign_range, &a);
    memset(sum, 0, sizeof(double) * (size_t)k * d);
    memset(cnt, 0, sizeof(int64_t) * k);
    for (int64_t i = 0; i < n; ++i) {
      cnt[assign[i]]++;
      for (int32_t j = 0; j < d; ++j)
        sum[(int64_t)assign[i] * d + j] += x[i * d + j];
    }
    for (int32_t c = 0; c < k; ++c)
      if (cnt[c] > 0)
        for (int32_t j = 0; j < d; ++j)
          centroids[(int64_t)c * d + j] =
              (float)(sum[(int64_t)c * d + j] / (double)cnt[c]);
  }
  free(cnt);
  free(sum);
  free(assign);
}

/* ------------------------------------------------------------------------ */
/* KMeansClustering.cluster restated (Clustering/KMeansClustering.swift)      */
/* ------------------------------------------------------------------------ */

/* SeedableRNG.next (Clustering/KMeansClustering.swift:480-491): a 64-bit
 * LCG, state = state * 2862933555777941757 + 3037000493, returns state. */
static uint64_t swift_lcg(uint64_t *s) {
  *s = *s * 2862933555777941757ull + 3037000493ull;
  return *s;
}
/* Swift stdlib RandomNumberGenerator.next(upperBound:) for UInt64: Lemire's
 * nearly-divisionless method (arXiv:1805.10941), which Int.random(in: 0..<n,
 * using:) calls with upperBound n. */
uint64_t vsko_swift_bounded(uint64_t *state, uint64_t bound) {
  uint64_t r = swift_lcg(state);
  unsigned __int128 m = (unsigned __int128)r * bound;
  if ((uint64_t)m < bound) {
    uint64_t t = (0 - bound) % bound;
    while ((uint64_t)m < t) {
      r = swift_lcg(state);
      m = (unsigned __int128)r * bound;
    }
  }
  return (uint64_t)(m >> 64);
}

/* initializeRandom (Clustering/KMeansClustering.swift:197-207): the first k
 * of vectors.indices.shuffled(using: SeedableRNG(seed)).  Swift's
 * MutableCollection.shuffle(using:) is Fisher-Yates from the front: step i
 * swaps element i with element i + Int.random(in: 0..<(n - i)); element i
 * is final after step i, so k steps give the prefix. */
void vsko_kmeans_init_random(int64_t n, int32_t k, uint64_t seed,
                             int64_t *rows) {
  int64_t *perm = (int64_t *)malloc(sizeof(int64_t) * n);
  for (int64_t i = 0; i < n; ++i) perm[i] = i;
  uint64_t st = seed;
  for (int64_t i = 0; i < k && i < n - 1; ++i) {
    int64_t j = i + (int64_t)vsko_swift_bounded(&st, (uint64_t)(n - i));
    int64_t t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
  for (int32_t c = 0; c < k; ++c) rows[c] = perm[c];
  free(perm);
}

/* euclideanDistance (Clustering/KMeansClustering.swift:421-428):
 * sqrt of the sequential, unfused sum of squared differences */
static float km_l2(const float *a, const float *b, int32_t d) {
  return sqrtf(vsko_l2sq(a, b, d));
}

typedef struct {
  const float *x, *c;
  int32_t d, k;
  int32_t *assign;
  float *dist;
} kmc_ctx;
/* assignWithCPU (:271-295): strict '<' over the centroids in order, the
 * first minimum wins; minDistance starts at +inf with index 0 */
static void kmc_assign_range(void *p, int64_t lo, int64_t hi) {
  kmc_ctx *a = (kmc_ctx *)p;
  for (int64_t i = lo; i < hi; ++i) {
    float best = INFINITY;
    int32_t bi = 0;
    for (int32_t c = 0; c < a->k; ++c) {
      float v = km_l2(a->x + i * a->d, a->c + (int64_t)c * a->d, a->d);
      if (v < best) {
        best = v;
        bi = c;
      }
    }
    a->assign[i] = bi;
    a->dist[i] = best;
  }
}

/* k-means++ seeding (initializeKMeansPlusPlus, :209-259) with the D^2
 * weighting the method defines: the reference's weights D^2 / sum(D) (:237)
 * do not sum to one, and are not reproduced.  First row:
 * Int.random(in: 0..<n) on SeedableRNG(seed) (:214-218).  Pick r + 1: D(x)
 * = min over picked rows of the sqrt-L2 (computeMinDistances, :401-419),
 * weight = floor(D^2 / max D^2 * 2^32) (an exact integer, so the total does
 * not depend on a summation order), u = Int.random(in: 0..<total) drawn
 * from the same SeedableRNG stream, and the pick is the first row whose
 * running weight sum exceeds u.  (The reference reseeds every pick with
 * seed + picks so far, :241; an LCG's first output is affine in its seed, so
 * those draws are correlated from pick to pick, and one stream serves all
 * picks here.)  Returns -1 when every weight is zero (degenerateData,
 * :235-237), else 0. */
static uint64_t kpp_fixed(float dm, float maxw) {
  if (!(maxw > 0.0f)) return 0;
  const float w = dm * dm;
  return (uint64_t)((double)w / (double)maxw * 4294967296.0);
}
typedef struct {
  const float *x, *c;
  int32_t d;
  float *D;
} kpp_ctx;
static void kpp_update_range(void *p, int64_t lo, int64_t hi) {
  kpp_ctx *a = (kpp_ctx *)p;
  for (int64_t i = lo; i < hi; ++i) {
    const float dist = km_l2(a->x + i * a->d, a->c, a->d);
    if (dist < a->D[i]) a->D[i] = dist;
  }
}
int32_t vsko_kmeans_init_plusplus(const float *x, int64_t n, int32_t d,
                                  int32_t k, uint64_t seed, int64_t *rows,
                                  int32_t nthreads) {
  float *D = (float *)malloc(sizeof(float) * n);
  for (int64_t i = 0; i < n; ++i) D[i] = INFINITY;
  uint64_t st = seed;
  rows[0] = (int64_t)vsko_swift_bounded(&st, (uint64_t)n);
  int32_t rc = 0;
  for (int32_t r = 0; r + 1 < k; ++r) {
    kpp_ctx a = {x, x + rows[r] * d, d, D};
    parallel_for(n, nthreads, kpp_update_range, &a);
    float maxw = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
      const float w = D[i] * D[i];
      if (w > maxw) maxw = w;
    }
    uint64_t total = 0;
    for (int64_t i = 0; i < n; ++i) total += kpp_fixed(D[i], maxw);
    if (total == 0) {
      rc = -1;
      break;
    }
    const uint64_t u = vsko_swift_bounded(&st, total);
    uint64_t cum = 0;
    int64_t pick = -1;
    for (int64_t i = 0; i < n; ++i) {
      const uint64_t f = kpp_fixed(D[i], maxw);
      if (f > 0 && u < cum + f) {
        pick = i;
        break;
      }
      cum += f;
    }
    rows[r + 1] = pick;
  }
  free(D);
  return rc;
}

/* KMeansClustering.cluster (:48-113) with the update step of :342-380.
 * Per iteration: assignment; fp32 sums in row order
 * (newCentroids[a][j] += x[i][j] * w, counts[a] += w, w = 1 without
 * weights); means by fp32 division; inertia = the fp32 sum of the assigned
 * distances in row order; converged = |inertia - previous| < tol (previous
 * starts at +inf).  An empty cluster takes row Int.random(in: 0..<n) of a
 * SeedableRNG seeded with seed + 0x9E3779B97F4A7C15, drawn in ascending
 * cluster order (the reference draws it from the unseeded system generator,
 * :374, which no run can reproduce).  init_method: 0 initializeRandom with
 * seed, 1 init = k x d starting centroids (.custom), 2 k-means++ as above
 * (returns -1 on degenerate data).  Outputs the
 * centroids after the last update, the assignments and inertia of the last
 * assignment step, the iteration count and the converged flag, as
 * ClusteringResult (:9-29). */
int32_t vsko_kmeans_cluster(const float *x, int64_t n, int32_t d, int32_t k,
                            int32_t init_method, const float *init,
                            const float *weights, int32_t max_iter, float tol,
                            uint64_t seed, float *centroids, int32_t *assign,
                            int32_t *iters_out, int32_t *converged_out,
                            float *inertia_out, int32_t nthreads) {
  float *cur = (float *)malloc(sizeof(float) * (size_t)k * d);
  if (init_method == 1) {
    memcpy(cur, init, sizeof(float) * (size_t)k * d);
  } else {
    int64_t *rows = (int64_t *)malloc(sizeof(int64_t) * k);
    if (init_method == 2) {
      if (vsko_kmeans_init_plusplus(x, n, d, k, seed, rows, nthreads) != 0) {
        free(rows);
        free(cur);
        return -1;
      }
    } else {
      vsko_kmeans_init_random(n, k, seed, rows);
    }
    for (int32_t c = 0; c < k; ++c)
      memcpy(cur + (int64_t)c * d, x + rows[c] * d, sizeof(float) * d);
    free(rows);
  }
  int32_t *a = (int32_t *)calloc((size_t)n, sizeof(int32_t));
  float *dist = (float *)malloc(sizeof(float) * n);
  float *sums = (float *)malloc(sizeof(float) * (size_t)k * d);
  float *cnt = (float *)malloc(sizeof(float) * k);
  uint64_t empty_rng = seed + 0x9E3779B97F4A7C15ull;
  float prev = INFINITY, inertia = INFINITY;
  int32_t it = 0, conv = 0;
  while (it < max_iter && !conv) {
    kmc_ctx ac = {x, cur, d, k, a, dist};
    parallel_for(n, nthreads, kmc_assign_range, &ac);
    memset(sums, 0, sizeof(float) * (size_t)k * d);
    memset(cnt, 0, sizeof(float) * k);
    for (int64_t i = 0; i < n; ++i) {
      const float w = weights ? weights[i] : 1.0f;
      float *s = sums + (int64_t)a[i] * d;
      for (int32_t j = 0; j < d; ++j) s[j] += x[i * d + j] * w;
      cnt[a[i]] += w;
    }
    for (int32_t c = 0; c < k; ++c) {
      float *s = sums + (int64_t)c * d;
      if (cnt[c] > 0) {
        for (int32_t j = 0; j < d; ++j) s[j] /= cnt[c];
      } else {
        int64_t r = (int64_t)vsko_swift_bounded(&empty_rng, (uint64_t)n);
        memcpy(s, x + r * d, sizeof(float) * d);
      }
    }
    inertia = 0.0f;
    for (int64_t i = 0; i < n; ++i) inertia += dist[i];
    conv = fabsf(inertia - prev) < tol;
    memcpy(cur, sums, sizeof(float) * (size_t)k * d);
    prev = inertia;
    ++it;
  }
  memcpy(centroids, cur, sizeof(float) * (size_t)k * d);
  if (assign) memcpy(assign, a, sizeof(int32_t) * n);
  *iters_out = it;
  *converged_out = conv;
  *inertia_out = it > 0 ? prev : INFINITY;
  free(cnt);
  free(sums);
  free(dist);
  free(a);
  free(cur);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* binary quantization and Hamming search                                     */
/* ------------------------------------------------------------------------ */

/* Acceleration/AccelerateOptimizer.swift:447-481 (binaryQuantize): bytes
 * zeroed, then bit i%8 of byte i/8 set where x_i > 0. */
void vsko_binary_encode(const float *x, int64_t n, int32_t d, uint8_t *codes) {
  const int32_t nb = (d + 7) / 8;
  for (int64_t r = 0; r < n; ++r) {
    uint8_t *c = codes + r * nb;
    memset(c, 0, (size_t)nb);
    for (int32_t i = 0; i < d; ++i)
      if (x[r * d + i] > 0.0f) c[i / 8] |= (uint8_t)(1u << (i % 8));
  }
}

/* Acceleration/Metal/Shaders/QuantizationShaders.metal:285-305
 * (binaryHammingDistance): popcount of the xor, summed */
int32_t vsko_bin_hamming(const uint8_t *a, const uint8_t *b, int32_t nbytes) {
  int32_t s = 0;
  for (int32_t i = 0; i < nbytes; ++i) s += __builtin_popcount((unsigned)(a[i] ^ b[i]));
  return s;
}

typedef struct {
  const uint8_t *q, *x;
  int64_t n;
  int32_t d, k;
  int32_t *od;
  int64_t *oi;
} bins_ctx;
/* per query: every distance, a histogram over 0..d, then the rows of the
 * smallest distances in ascending row order (the (distance, id) order) */
static void bins_range(void *p, int64_t lo, int64_t hi) {
  bins_ctx *a = (bins_ctx *)p;
  const int32_t nb = (a->d + 7) / 8;
  int32_t *dist = (int32_t *)malloc(sizeof(int32_t) * a->n);
  int64_t *hist = (int64_t *)malloc(sizeof(int64_t) * (a->d + 1));
  for (int64_t qi = lo; qi < hi; ++qi) {
    memset(hist, 0, sizeof(int64_t) * (a->d + 1));
    for (int64_t r = 0; r < a->n; ++r) {
      dist[r] = vsko_bin_hamming(a->q + qi * nb, a->x + r * nb, nb);
      hist[dist[r]]++;
    }
    int32_t *od = a->od + qi * a->k;
    int64_t *oi = a->oi + qi * a->k;
    int32_t got = 0;
    for (int32_t dv = 0; dv <= a->d && got < a->k; ++dv) {
      if (!hist[dv]) continue;
      for (int64_t r = 0; r < a->n && got < a->k; ++r)
        if (dist[r] == dv) {
          od[got] = dv;
          oi[got] = r;
          ++got;
        }
    }
    for (; got < a->k; ++got) {
      od[got] = 0x7FFFFFFF;
      oi[got] = -1;
    }
  }
  free(hist);
  free(dist);
}
void vsko_bin_search(const uint8_t *qcodes, int64_t nq, const uint8_t *codes,
                     int64_t n, int32_t d, int32_t k, int32_t *out_dist,
                     int64_t *out_ids, int32_t nthreads) {
  bins_ctx a = {qcodes, codes, n, d, k, out_dist, out_ids};
  parallel_for(nq, nthreads, bins_range, &a);
}
