/* Drives every oracle function on small, ragged inputs (odd dimensions, k
 * above n, one row, threads on) so that a host build with AddressSanitizer
 * and UndefinedBehaviorSanitizer sees their memory accesses and arithmetic.
 * Built and run by tests/test_oracle_sanitize.py; exits nonzero on a
 * sanitizer report (halt_on_error) or a failed self-check. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vsk_oracle.h"

static uint64_t st = 0x9E3779B97F4A7C15ull;
static float rnd(void) {
  st = st * 6364136223846793005ull + 1442695040888963407ull;
  return (float)((double)(st >> 11) / 9007199254740992.0 * 2.0 - 1.0);
}
static float *vec(int64_t m) {
  float *p = (float *)malloc(sizeof(float) * (size_t)(m ? m : 1));
  for (int64_t i = 0; i < m; ++i) p[i] = rnd();
  return p;
}
#define CHECK(c)                                              \
  do {                                                        \
    if (!(c)) {                                               \
      fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
      return 1;                                               \
    }                                                         \
  } while (0)

int main(void) {
  const int32_t dims[] = {1, 3, 37, 64};
  for (int di = 0; di < 4; ++di) {
    const int32_t d = dims[di];
    const int64_t n = 53, nq = 5;
    const int32_t k = 60;  /* k > n: padded results */
    float *x = vec(n * d), *q = vec(nq * d);
    float *dist = (float *)malloc(sizeof(float) * nq * k);
    int64_t *ids = (int64_t *)malloc(sizeof(int64_t) * nq * k);
    for (int32_t m = 0; m <= 5; ++m) {  /* every flat metric */
      vsko_search_flat(q, nq, x, n, d, k, m, dist, ids, 3, 0);
      CHECK(ids[k - 1] == -1);
    }
    vsko_flatdb *db = vsko_flat_prepare(x, n, d, 2);
    vsko_flat_search(db, q, nq, k, 0, dist, ids, 2);
    vsko_flat_free(db);
    float *all = (float *)malloc(sizeof(float) * nq * n);
    vsko_distances(q, nq, x, n, d, 1, all, 2);
    vsko_topk(all, n, 7, dist, ids);
    float *nx = (float *)malloc(sizeof(float) * n * d);
    vsko_normalize(x, n, d, nx);
    const int32_t hm[4] = {0, 1, 5, 7};  /* the HNSW metrics */
    for (int32_t m = 0; m < 4; ++m) (void)vsko_hnsw_distance(q, x, d, hm[m]);
    /* IVF */
    const int32_t nlist = 7;
    int32_t *lists = (int32_t *)malloc(sizeof(int32_t) * n);
    vsko_ivf_assign(x, n, q, (int32_t)nq, d, lists, 2);
    int32_t *probes = (int32_t *)malloc(sizeof(int32_t) * nq * nlist);
    float *cent = vec((int64_t)nlist * d);
    vsko_ivf_probe(q, nq, cent, nlist, d, nlist, probes, 2);
    int64_t *rid = (int64_t *)malloc(sizeof(int64_t) * n);
    for (int64_t i = 0; i < n; ++i) rid[i] = 1000 + i;
    vsko_ivf_assign(x, n, cent, nlist, d, lists, 2);
    vsko_ivf_search(q, nq, x, rid, lists, n, d, cent, nlist, 3, k, 0, dist, ids, 2);
    /* SQ8 */
    float sc[64], of[64];
    int8_t *codes = (int8_t *)malloc((size_t)n * d), *qc = (int8_t *)malloc((size_t)nq * d);
    vsko_sq8_train(x, n, d, 1, sc, of);
    vsko_sq8_encode(x, n, d, 1, sc, of, codes);
    vsko_sq8_encode(q, nq, d, 1, sc, of, qc);
    float *dec = (float *)malloc(sizeof(float) * n * d);
    vsko_sq8_decode(codes, n, d, 1, sc, of, dec);
    int32_t *score = (int32_t *)malloc(sizeof(int32_t) * nq * k);
    vsko_sq8_search(qc, nq, codes, n, d, k, score, ids, 2);
    uint8_t *u8 = (uint8_t *)malloc((size_t)n * d);
    float mn[64], scale[64];
    vsko_scalar_quantize_u8(x, n, d, 8, u8, mn, scale);
    /* binary */
    const int32_t nb = (d + 7) / 8;
    uint8_t *bc = (uint8_t *)malloc((size_t)n * nb), *bq = (uint8_t *)malloc((size_t)nq * nb);
    vsko_binary_encode(x, n, d, bc);
    vsko_binary_encode(q, nq, d, bq);
    int32_t *hd = (int32_t *)malloc(sizeof(int32_t) * nq * k);
    vsko_bin_search(bq, nq, bc, n, d, k, hd, ids, 2);
    /* PQ (segments of 1 dim for odd d) */
    const int32_t M = d % 2 ? d : d / 2, dsub = d / M, ksub = 16;
    float *cb = vec((int64_t)M * ksub * dsub);
    uint8_t *pc = (uint8_t *)malloc((size_t)n * M);
    vsko_pq_encode(x, n, cb, M, ksub, dsub, pc, 2);
    float *lut = (float *)malloc(sizeof(float) * M * ksub);
    vsko_pq_lut(q, cb, M, ksub, dsub, lut);
    float *sums = (float *)malloc(sizeof(float) * n);
    vsko_pq_adc_scan(lut, pc, n, M, ksub, sums);
    CHECK(sums[0] == vsko_pq_adc_sum(lut, pc, M, ksub));
    vsko_pq_decode(pc, n, cb, M, ksub, dsub, dec);
    vsko_pq_search(q, nq, cb, pc, n, M, ksub, dsub, 20, 10, x, 5, dist, ids, 2);
    vsko_pq_search(q, nq, cb, pc, n, M, ksub, dsub, 20, 10, NULL, -1, dist, ids, 2);
    /* k-means */
    float *cen = (float *)malloc(sizeof(float) * 5 * d);
    int32_t *asg = (int32_t *)malloc(sizeof(int32_t) * n);
    int32_t it = 0, conv = 0;
    float inertia = 0.f;
    for (int32_t init = 0; init <= 2; init += 2)
      (void)vsko_kmeans_cluster(x, n, d, 5, init, NULL, NULL, 6, 1e-4f, 7, cen, asg, &it, &conv,
                                &inertia, 2);
    vsko_kmeans(x, n, d, 5, 3, 11, cen, 2);
    int64_t rows[5];
    vsko_kmeans_init_random(n, 5, 3, rows);
    free(x); free(q); free(dist); free(ids); free(all); free(nx); free(lists); free(probes);
    free(cent); free(rid); free(codes); free(qc); free(dec); free(score); free(u8); free(bc);
    free(bq); free(hd); free(cb); free(pc); free(lut); free(sums); free(cen); free(asg);
  }
  printf("oracle sanitize ok\n");
  return 0;
}
