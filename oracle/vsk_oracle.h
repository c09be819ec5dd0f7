/*
 * vsk_oracle.h -- CPU restatement of VectorStoreKit's search hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code.  It is used by tests/ (as the parity checker), by
 * __graft_entry__.smoke() (as the checker of one small GPU call) and by
 * bench.py's cpu_baseline leg (timed on the host, never as the GPU result).
 *
 * All arithmetic is plain fp32 in the reference's order (sequential, index
 * ascending, no FMA contraction: built with -ffp-contract=off), int32 for
 * int8 codes.  Every function names the reference file:line it restates
 * (paths relative to Sources/VectorStoreKit/ of gifton/VectorStoreKit).
 *
 * Ordering rule used everywhere: ascending (distance, tie key) where the tie
 * key is the row id for flat/SQ/PQ search, the centroid index for IVF
 * probing and the position in the probe-ordered candidate concatenation for
 * IVF search.  That is what the reference's stable `sort` + `prefix(k)`
 * produces (Indexes/IVFIndex.swift:175-176, :538-539).
 */
#ifndef VSK_ORACLE_H
#define VSK_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* metric codes (same values as the VSK_METRIC_* codes of the C ABI) */
enum {
  VSKO_L2SQ = 0,              /* sum (q-x)^2                                 */
  VSKO_L2 = 1,                /* sqrt(sum (q-x)^2)                           */
  VSKO_COSINE = 2,            /* 1 - q.x / (|q||x| + 1e-8)                   */
  VSKO_COSINE_NORMALIZED = 3, /* 1 - q.x (unit-norm inputs)                  */
  VSKO_DOT = 4,               /* -q.x                                        */
  VSKO_L1 = 5,                /* sum |q-x|                                   */
  VSKO_HAMMING = 6,           /* count of q_i != x_i                         */
  VSKO_COSINE_NOEPS = 7       /* 1 - q.x / (|q||x|), HNSW's cosine           */
};

/* ---- distances ---------------------------------------------------------- */
float vsko_l2sq(const float *a, const float *b, int32_t d);
float vsko_dot(const float *a, const float *b, int32_t d);
float vsko_l1(const float *a, const float *b, int32_t d);
float vsko_distance(const float *q, const float *x, int32_t d, int32_t metric);
/* quantizeVectors(.scalar(bits)) on the CPU path: per-vector min/max,
 * uint8 codes truncated; scale/minv per vector (either may be NULL) */
void vsko_scalar_quantize_u8(const float *x, int64_t n, int32_t d, int32_t bits,
                             uint8_t *codes, float *scale, float *minv);
/* HNSWIndex DistanceComputer.distance (L2, L2SQ, L1, COSINE_NOEPS) and its
 * batched form over CSR neighbour lists */
float vsko_hnsw_distance(const float *q, const float *x, int32_t d, int32_t metric);
void vsko_hnsw_distances(const float *q, int64_t nq, const float *x, int32_t d,
                         const int64_t *offsets, const int32_t *rows, int32_t metric,
                         float *out);
/* normalizeVectors: out = x / (sqrt(sum x^2) + 1e-8) per row */
void vsko_normalize(const float *x, int64_t n, int32_t d, float *out);
/* matrixMultiply: c (m x n) = a (m x k) . b (k x n), sequential sums */
void vsko_matmul(const float *a, int64_t m, int32_t k, const float *b, int64_t n, float *c);
/* out[i*n + j] = distance(q_i, x_j) */
void vsko_distances(const float *q, int64_t nq, const float *x, int64_t n,
                    int32_t d, int32_t metric, float *out, int32_t nthreads);

/* ---- exact flat k-NN ---------------------------------------------------- */
/* fast != 0 uses a 16-accumulator dot/L2 (timing only; different fp order). */
void vsko_search_flat(const float *q, int64_t nq, const float *x, int64_t n,
                      int32_t d, int32_t k, int32_t metric, float *out_dist,
                      int64_t *out_ids, int32_t nthreads, int32_t fast);
/* The same exact search over a database prepared once (rows re-laid out
 * 16 to a SIMD group, row norms): what a resident CPU index does.  Not for
 * the hamming metric. */
typedef struct vsko_flatdb vsko_flatdb;
vsko_flatdb *vsko_flat_prepare(const float *x, int64_t n, int32_t d, int32_t nthreads);
void vsko_flat_free(vsko_flatdb *db);
void vsko_flat_search(const vsko_flatdb *db, const float *q, int64_t nq, int32_t k,
                      int32_t metric, float *out_dist, int64_t *out_ids, int32_t nthreads);
/* k smallest of dist[0..n) by (dist, index); missing slots get (inf, -1). */
void vsko_topk(const float *dist, int64_t n, int32_t k, float *out_dist,
               int64_t *out_idx);

/* ---- IVF-Flat ----------------------------------------------------------- */
void vsko_ivf_assign(const float *x, int64_t n, const float *centroids,
                     int32_t nlist, int32_t d, int32_t *out_list,
                     int32_t nthreads);
void vsko_ivf_probe(const float *q, int64_t nq, const float *centroids,
                    int32_t nlist, int32_t d, int32_t nprobe,
                    int32_t *out_lists, int32_t nthreads);
/* list_of[i] = inverted list of row i (rows keep insertion order inside a
 * list); ids[i] = user id of row i.  Output distances are L2 (sqrt), or the
 * squared sum when squared != 0 (ranked on that sum). */
void vsko_ivf_search(const float *q, int64_t nq, const float *x,
                     const int64_t *ids, const int32_t *list_of, int64_t n,
                     int32_t d, const float *centroids, int32_t nlist,
                     int32_t nprobe, int32_t k, int32_t squared,
                     float *out_dist, int64_t *out_ids, int32_t nthreads);

/* ---- scalar quantization (int8) ----------------------------------------- */
/* per_dim != 0: scale[d], offset[d] from per-column min/max;
 * per_dim == 0: scale[0], offset[0] from the global min/max. */
void vsko_sq8_train(const float *x, int64_t n, int32_t d, int32_t per_dim,
                    float *scale, float *offset);
void vsko_sq8_encode(const float *x, int64_t n, int32_t d, int32_t per_dim,
                     const float *scale, const float *offset, int8_t *codes);
void vsko_sq8_decode(const int8_t *codes, int64_t n, int32_t d,
                     int32_t per_dim, const float *scale, const float *offset,
                     float *out);
int32_t vsko_sq8_dot(const int8_t *a, const int8_t *b, int32_t d);
/* top-k by (-score, id); out_score = score (int32) */
void vsko_sq8_search(const int8_t *qcodes, int64_t nq, const int8_t *codes,
                     int64_t n, int32_t d, int32_t k, int32_t *out_score,
                     int64_t *out_ids, int32_t nthreads);

/* ---- product quantization ----------------------------------------------- */
/* codebooks: [M][ksub][dsub] fp32; lut: [M][ksub] */
void vsko_pq_lut(const float *q, const float *codebooks, int32_t M,
                 int32_t ksub, int32_t dsub, float *lut);
void vsko_pq_encode(const float *x, int64_t n, const float *codebooks,
                    int32_t M, int32_t ksub, int32_t dsub, uint8_t *codes,
                    int32_t nthreads);
void vsko_pq_decode(const uint8_t *codes, int64_t n, const float *codebooks,
                    int32_t M, int32_t ksub, int32_t dsub, float *out);
float vsko_pq_adc_sum(const float *lut, const uint8_t *code, int32_t M,
                      int32_t ksub);
/* ADC top-k_adc by (sum, id).  If x != NULL and rerank_metric >= 0 the
 * k_adc candidates are re-scored with the exact metric on x and the top k
 * by (exact, id) are returned; otherwise the first k ADC results are
 * returned with distance sqrt(sum). */
void vsko_pq_search(const float *q, int64_t nq, const float *codebooks,
                    const uint8_t *codes, int64_t n, int32_t M, int32_t ksub,
                    int32_t dsub, int32_t k_adc, int32_t k, const float *x,
                    int32_t rerank_metric, float *out_dist, int64_t *out_ids,
                    int32_t nthreads);
/* ADC sums only: out_sum[i] = sum_m lut[m][codes[i][m]] */
void vsko_pq_adc_scan(const float *lut, const uint8_t *codes, int64_t n,
                      int32_t M, int32_t ksub, float *out_sum);

/* ---- k-means (fixture generation only) ---------------------------------- */
/* Lloyd iterations from the first k rows of a seeded permutation; strict '<'
 * assignment, empty clusters keep their previous centre. */
void vsko_kmeans(const float *x, int64_t n, int32_t d, int32_t k,
                 int32_t iters, uint64_t seed, float *centroids,
                 int32_t nthreads);

/* ---- binary quantization ------------------------------------------------ */
/* AccelerateOptimizer.binaryQuantize: codes n x ceil(d/8) bytes, bit i =
 * x_i > 0 at byte i/8, bit i%8 */
void vsko_binary_encode(const float *x, int64_t n, int32_t d, uint8_t *codes);
/* binaryHammingDistance: popcount(a xor b) over nbytes */
int32_t vsko_bin_hamming(const uint8_t *a, const uint8_t *b, int32_t nbytes);
/* top k by (Hamming distance, row id); missing: INT32_MAX and -1 */
void vsko_bin_search(const uint8_t *qcodes, int64_t nq, const uint8_t *codes,
                     int64_t n, int32_t d, int32_t k, int32_t *out_dist,
                     int64_t *out_ids, int32_t nthreads);

/* ---- KMeansClustering.cluster (Clustering/KMeansClustering.swift:48-113) */
/* Int.random(in: 0..<bound, using: &SeedableRNG): Swift's Lemire bounded
 * draw on the reference's LCG; state is advanced in place */
uint64_t vsko_swift_bounded(uint64_t *state, uint64_t bound);
/* initializeRandom: rows[k] = the first k of (0..<n).shuffled(seed) */
void vsko_kmeans_init_random(int64_t n, int32_t k, uint64_t seed,
                             int64_t *rows);
/* k-means++ rows[k] with exact fixed-point D^2 weights; -1 = degenerate */
int32_t vsko_kmeans_init_plusplus(const float *x, int64_t n, int32_t d,
                                  int32_t k, uint64_t seed, int64_t *rows,
                                  int32_t nthreads);
/* Lloyd loop as the reference runs it (fp32 row-order sums, fp32 means,
 * fp32 sequential inertia, |inertia - previous| < tol); init_method 0
 * random, 1 custom (init = k x d), 2 k-means++; weights may be NULL; assign
 * may be NULL.  Returns -1 on degenerate data (k-means++), else 0. */
int32_t vsko_kmeans_cluster(const float *x, int64_t n, int32_t d, int32_t k,
                            int32_t init_method, const float *init,
                            const float *weights, int32_t max_iter, float tol,
                            uint64_t seed, float *centroids, int32_t *assign,
                            int32_t *iters_out, int32_t *converged_out,
                            float *inertia_out, int32_t nthreads);

int32_t vsko_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
