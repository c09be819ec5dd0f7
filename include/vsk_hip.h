/*
 * vsk_hip.h -- C ABI of the MI355X (gfx950) search hot path of
 * VectorStoreKit: flat k-NN (L2, L2^2, cosine, dot, Manhattan) with fused
 * top-k, IVF-Flat (coarse probe + inverted-list scan), int8 scalar-quantized
 * scan and product-quantized ADC scan with exact re-rank.
 *
 * Reference paths are relative to Sources/VectorStoreKit/ of
 * gifton/VectorStoreKit.  Each entry point names the reference interface it
 * replaces.
 *
 * Conventions
 *  - Every function returns vsk_status (0 = OK, negative = error);
 *    vsk_last_error(ctx) returns the message of the last failure on ctx.
 *  - Pointer arguments may point to host memory or to device memory of the
 *    context's GPU (hipMalloc / torch tensors); the library inspects each
 *    pointer and stages host buffers through device memory itself.
 *  - One context owns one HIP stream.  Calls on one context are serialised
 *    by the caller (the reference makes every engine/index an actor); calls
 *    on distinct contexts may run concurrently.  Every call returns after
 *    its results are in the caller's buffers.
 *  - Results are ordered ascending by (distance, tie key); the tie key is
 *    the row id (flat, SQ, PQ), the centroid index (IVF probe) or the
 *    position of the row in the probe-ordered candidate list (IVF search),
 *    which is the order the reference's stable sort + prefix(k) produces
 *    (Indexes/IVFIndex.swift:175-176).  Missing results (k larger than the
 *    number of candidates) are reported as distance +inf and id -1.
 *  - Row ids are int64 in the outputs; a database handle holds at most
 *    2^31 - 1 rows.
 */
#ifndef VSK_HIP_H
#define VSK_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t vsk_status;

/* Status codes.  They map 1:1 onto the reference's Swift errors:
 * MetalComputeError (Acceleration/Metal/MetalErrors.swift:10-39),
 * AcceleratorError (API/Strategies/AcceleratorStrategies.swift:504-510),
 * IVFError (Indexes/IVFIndex.swift:619-623) and QuantizationError
 * (Quantization/ProductQuantizerTypes.swift:33-39). */
#define VSK_OK 0
#define VSK_ERR_DEVICE_NOT_AVAILABLE (-1) /* .deviceNotAvailable / .noDevice  */
#define VSK_ERR_INVALID_ARGUMENT (-2)     /* .invalidInputData / .invalidParameter */
#define VSK_ERR_EMPTY_INPUT (-3)          /* .emptyInput                      */
#define VSK_ERR_DIMENSION_MISMATCH (-4)   /* .dimensionMismatch               */
#define VSK_ERR_OUT_OF_MEMORY (-5)        /* .bufferAllocationFailed / .deviceOutOfMemory */
#define VSK_ERR_EXECUTION_FAILED (-6)     /* .commandBufferExecutionFailed    */
#define VSK_ERR_NOT_TRAINED (-7)          /* IVFError/QuantizationError.notTrained */
#define VSK_ERR_UNSUPPORTED (-8)          /* .unsupportedOperation            */
#define VSK_ERR_INVALID_BUFFER_SIZE (-9)  /* .invalidBufferSize (k or size over a limit) */
#define VSK_ERR_IO (-10)                  /* index file unreadable, unwritable or malformed */

/* Distance metrics: DistanceMetric raw values "euclidean", "cosine",
 * "dotProduct", "manhattan", "hamming" (Core/SearchTypes.swift:105-112; the
 * five UnifiedDistanceComputation evaluates, Core/Distance/
 * UnifiedDistanceComputation.swift:171-186,249-261) plus the
 * squared-L2 and pre-normalised cosine forms the reference's kernels use
 * (Acceleration/Metal/Shaders/DistanceShaders.metal:620-654, 815-845). */
#define VSK_METRIC_L2SQ 0              /* sum (q-x)^2                        */
#define VSK_METRIC_L2 1                /* sqrt(sum (q-x)^2)     "euclidean"  */
#define VSK_METRIC_COSINE 2            /* 1 - q.x/(|q||x|+1e-8) "cosine"     */
#define VSK_METRIC_COSINE_NORMALIZED 3 /* 1 - q.x (unit-norm rows/queries)  */
#define VSK_METRIC_DOT 4               /* -q.x                  "dotProduct" */
#define VSK_METRIC_L1 5                /* sum |q-x|             "manhattan"  */
#define VSK_METRIC_HAMMING 6           /* count of q_i != x_i   "hamming"    */
#define VSK_METRIC_COSINE_NOEPS 7      /* 1 - q.x/(|q||x|), HNSW's cosine
                                          (vsk_hnsw_distances only)          */

#define VSK_MAX_K 1024 /* largest k of any top-k call */

/* vsk_db_upload_f32 flags */
#define VSK_DB_NORMALIZE 1 /* L2-normalise each row on the device, x/(|x|+1e-8)
                              (normalizeVectors, DistanceShaders.metal:403-429) */

typedef struct vsk_ctx vsk_ctx;
typedef struct vsk_db vsk_db;
typedef struct vsk_ivf vsk_ivf;
typedef struct vsk_sq8 vsk_sq8;
typedef struct vsk_pq vsk_pq;
typedef struct vsk_bin vsk_bin;

/* Device description; backs ComputeAccelerator.capabilities()
 * (Core/Protocols.swift:11-20). */
typedef struct {
  char name[96];
  char arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t device;
  int32_t compute_units;
  int32_t wavefront_size;
  int32_t lds_bytes_per_block;
  int64_t global_mem_bytes;
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width_bits;
} vsk_caps;

/* Per-kernel timing collected with HIP events on the context's stream.
 * work = items the launches processed: (query, row) pairs for the scans. */
typedef struct {
  char name[64];
  int64_t launches;
  double total_ms;
  double work;
} vsk_kernel_stat;

/* ---- context --------------------------------------------------------------
 * Replaces ComputeAccelerator.initialize() -> DeviceType
 * (Core/Protocols.swift:18; Metal: API/Strategies/AcceleratorStrategies.swift:
 * 20-214) and the MetalAccelerationEngine initialiser
 * (Acceleration/MetalAccelerationEngine.swift:40-70). */
vsk_status vsk_create(int32_t device, vsk_ctx **out);
vsk_status vsk_destroy(vsk_ctx *ctx);
/* ComputeAccelerator.capabilities() (Core/Protocols.swift:19) */
vsk_status vsk_device_info(vsk_ctx *ctx, vsk_caps *caps);
const char *vsk_last_error(const vsk_ctx *ctx);
/* HIP stream the context launches on (a hipStream_t), for interop. */
void *vsk_stream(vsk_ctx *ctx);
/* Wall time of the last API call's device work, from HIP events; replaces
 * MetalProfiler.recordOperation (Acceleration/Metal/MetalProfiler.swift:
 * 74-110). */
float vsk_last_kernel_ms(const vsk_ctx *ctx);
/* How often the last API call on ctx waited on the host for its stream
 * (the call's final synchronisation included).  A search is queued whole
 * and waits once; more waits mean a rare path ran (a query whose top-k
 * candidates overflowed, or that failed the screen's bound) or a buffer
 * grew.  A diagnostic with no counterpart in the reference. */
int32_t vsk_last_sync_count(const vsk_ctx *ctx);
/* Which queries of the last vsk_search_flat call on ctx the exact screen
 * redid: tier 1 = screened again keeping 1024 candidates, tier 2 = the
 * exact scan over every row (queries whose bound test failed; see
 * flat_screen.hip).  *count receives their number; the first min(cap,
 * count) query indices, ascending, go to out (out may be NULL if cap is 0).
 * Complements MetalProfiler's per-operation records
 * (Acceleration/Metal/MetalProfiler.swift:74-110). */
vsk_status vsk_last_screen_redo(const vsk_ctx *ctx, int32_t tier, int64_t *out,
                                int64_t cap, int64_t *count);
/* Measured ceilings of this GPU, for the rooflines' "fraction of the
 * measured peak" next to the datasheet one: dense bf16 and int8 matrix-core
 * rates (register-resident 16x16x32 bf16 and 16x16x64 int8 MFMAs, 32 and 16
 * independent accumulators per wave, 8 waves per CU), HBM copy bandwidth
 * (2 GiB, bytes read plus written) and HBM read bandwidth.  Takes about half a second
 * and 4 GiB of device memory.  No counterpart in the reference: it serves
 * the benchmark, which reports each kernel against re-measured peaks
 * beside the datasheet ones. */
typedef struct {
  double bf16_tflops;
  double int8_tops;
  double hbm_gbs;
  double hbm_read_gbs;
} vsk_peaks;
vsk_status vsk_measure_peaks(vsk_ctx *ctx, vsk_peaks *out);
/* ---- configuration ----------------------------------------------------------
 * HIPAccelerationConfiguration, the HIP counterpart of MetalComputeConfiguration
 * (Config/Acceleration/MetalComputeConfiguration.swift:8-46) and of the
 * store's DistanceComputeBackend choice (Config/Core/StoreConfiguration.swift:
 * 145-166).  A context starts from the environment (VSK_FLAT_KERNEL,
 * VSK_MAX_TILE_BYTES); vsk_configure replaces those settings for later
 * calls on ctx.  VSK_IVF_COMPACT=0, read at creation only, makes the
 * screened IVF list scan keep every candidate's word instead of those under
 * each query's bound (same results; for comparison and tests). */
#define VSK_KERNEL_AUTO 0   /* the bf16 screen where it is exact and pays, else exact scans */
#define VSK_KERNEL_EXACT 1  /* no screen: the exact scans alone (flat, IVF, PQ LUT, argmin) */
#define VSK_KERNEL_SCREEN 2 /* the screen at every size (where the metric allows it) */
#define VSK_KERNEL_BF16X3 3 /* flat search on the bf16x3 kernel (tolerance path) */
#define VSK_KERNEL_FP32 4   /* flat search on the fp32 MFMA kernel (tolerance path) */
typedef struct {
  int32_t kernel;           /* VSK_KERNEL_* */
  int32_t enable_profiling; /* per-kernel event timing (MetalComputeConfiguration.enableProfiling) */
  int64_t max_tile_bytes;   /* largest working buffer of a query batch; 0 = 2 GiB of
                               candidate keys.  Searches split their queries into
                               batches under it, as MetalDistanceCompute chunks queries
                               under its buffer limit (Acceleration/Metal/
                               MetalDistanceCompute.swift:371-380,450-473) */
} vsk_config;
vsk_status vsk_configure(vsk_ctx *ctx, const vsk_config *cfg);
vsk_status vsk_get_config(const vsk_ctx *ctx, vsk_config *cfg);
/* Per-kernel event timing (off by default). */
vsk_status vsk_profile_enable(vsk_ctx *ctx, int32_t on);
/* Restricts the timing to the timers named in names (comma-separated;
 * NULL or "" times every kernel again), so that a run can time its main
 * kernel with two events a launch and nothing else.  While a restriction
 * holds, work counts that live on the device (candidate totals, fallback
 * counts) are not read back: those stats report 0 work.  A profiling
 * control of this library with no counterpart in the reference. */
vsk_status vsk_profile_only(vsk_ctx *ctx, const char *names);
vsk_status vsk_profile_reset(vsk_ctx *ctx);
int32_t vsk_profile_count(const vsk_ctx *ctx);
vsk_status vsk_profile_get(const vsk_ctx *ctx, int32_t i, vsk_kernel_stat *out);

/* ---- flat database -------------------------------------------------------
 * Replaces the per-call candidate upload of
 * MetalAccelerationEngine.batchComputeDistancesGPU
 * (Acceleration/MetalAccelerationEngine.swift:393-405): rows are uploaded
 * once and stay resident in HBM.  x: n x d fp32 row-major. */
vsk_status vsk_db_upload_f32(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                             int32_t flags, vsk_db **out);
vsk_status vsk_db_free(vsk_ctx *ctx, vsk_db *db);
vsk_status vsk_db_info(const vsk_db *db, int64_t *n, int32_t *d);
/* Copy rows [row0, row0+count) back (after VSK_DB_NORMALIZE: normalised). */
vsk_status vsk_db_read_f32(vsk_ctx *ctx, const vsk_db *db, int64_t row0,
                           int64_t count, float *out);

/* ---- flat search ---------------------------------------------------------
 * MetalAccelerationEngine.batchComputeDistances(queries:candidates:metric:
 * topK:) (Acceleration/MetalAccelerationEngine.swift:139-204) with the top-k
 * fused on the device and ids returned (the reference returns distances
 * only, after a CPU sort of the full matrix, :457-477).  Also the exact
 * path of VectorIndex.search (Core/Protocols.swift:116-121).
 * Every metric returns the reference CPU path's fp32 distances (sums in
 * dimension order, its own formulas) and its (distance, row) order bit for
 * bit, for every k <= VSK_MAX_K; only VSK_KERNEL_BF16X3 / _FP32
 * (vsk_configure) trade that for a tolerance-path kernel.
 * q: nq x d fp32; out_dist: nq x k fp32; out_ids: nq x k int64. */
vsk_status vsk_search_flat(vsk_ctx *ctx, const vsk_db *db, const float *q,
                           int64_t nq, int32_t k, int32_t metric,
                           float *out_dist, int64_t *out_ids);
/* vsk_search_flat over the rows a filter keeps: row r is a candidate when
 * r < allow_bits and bit r of allow is set (bit r % 32 of allow[r / 32]);
 * rows past allow_bits are excluded.  The results are those of a search of
 * the kept rows alone, with the original row ids (ties still go to the lower
 * row).  Backs VectorIndex.search(query:k:strategy:filter:)
 * (Core/Protocols.swift:116-121) for a flat index: the reference applies
 * the filter to the candidates before it ranks them (Indexes/IVFIndex.swift:
 * 161-176 for IVF).  allow = NULL with allow_bits = 0 is vsk_search_flat. */
vsk_status vsk_search_flat_filtered(vsk_ctx *ctx, const vsk_db *db, const float *q,
                                    int64_t nq, int32_t k, int32_t metric,
                                    const uint32_t *allow, int64_t allow_bits,
                                    float *out_dist, int64_t *out_ids);
/* Full distance matrix out[i*n + j] = dist(q_i, x_j): computeDistances
 * (:76-136, nq = 1) and batchComputeDistances(topK: nil) (:139-204). */
vsk_status vsk_distances(vsk_ctx *ctx, const vsk_db *db, const float *q,
                         int64_t nq, int32_t metric, float *out);
/* MetalAccelerationEngine.matrixMultiply(matrixA:matrixB:)
 * (Acceleration/MetalAccelerationEngine.swift:209-229): c (m x n) =
 * a (m x k) . b (k x n), row-major fp32.  Every entry is summed over the k
 * products in order from 0, a product and then a sum (no FMA), as the
 * reference's CPU loop adds it (Acceleration/Metal/MetalMatrixCompute.swift:
 * 791-806).  Pointers may be host or device memory. */
vsk_status vsk_matrix_multiply(vsk_ctx *ctx, const float *a, int64_t m, int32_t k,
                               const float *b, int64_t n, float *c);

/* ---- IVF-Flat ------------------------------------------------------------
 * IVFIndex (Indexes/IVFIndex.swift).  The coarse centroids come from
 * training (IVFIndex.train, :397-446); vsk_ivf_create takes them as given. */
vsk_status vsk_ivf_create(vsk_ctx *ctx, const float *centroids, int32_t nlist,
                          int32_t d, vsk_ivf **out);
vsk_status vsk_ivf_free(vsk_ctx *ctx, vsk_ivf *ivf);
/* One-call build: vsk_ivf_create with the trained centroids, then
 * vsk_ivf_add of n rows x (n x d fp32; ids may be NULL; n may be 0) --
 * IVFIndex.train (:397-446, centroids given) followed by insert (:80-122).
 * On failure nothing is returned and *out is NULL. */
vsk_status vsk_ivf_build(vsk_ctx *ctx, const float *centroids, int32_t nlist,
                         const float *x, const int64_t *ids, int64_t n,
                         int32_t d, vsk_ivf **out);
/* IVFIndex.insert (:80-122): each row goes to its nearest centroid
 * (findNearestCentroid, :514-527, strict '<'), appended in call order.
 * ids may be NULL (then ids are the running row count). */
vsk_status vsk_ivf_add(vsk_ctx *ctx, vsk_ivf *ivf, const float *x,
                       const int64_t *ids, int64_t n);
/* findNearestCentroid for each row (:514-527): out_list[n] */
vsk_status vsk_ivf_assign(vsk_ctx *ctx, const vsk_ivf *ivf, const float *x,
                          int64_t n, int32_t *out_list);
/* findNearestCentroids (:529-540): out_lists[nq x nprobe] */
vsk_status vsk_ivf_probe(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                         int64_t nq, int32_t nprobe, int32_t *out_lists);
/* IVFIndex.search (:124-202): probe nprobe lists, exact L2 over their
 * union, top k.  nprobe >= nlist is the .exact strategy (:551-554).
 * metric: VSK_METRIC_L2 (the reference's computeDistance, :542-549, sqrt of
 * the sum) or VSK_METRIC_L2SQ (the sum itself); other metrics return
 * VSK_ERR_UNSUPPORTED, as IVFIndex ranks by euclidean distance only.  The
 * probe always ranks centroids by sqrt-L2 (:529-540). */
vsk_status vsk_ivf_search(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                          int64_t nq, int32_t nprobe, int32_t k,
                          int32_t metric, float *out_dist, int64_t *out_ids);
/* IVFIndex.search with a filter (:124-202): the probed lists' rows are
 * filtered first (applyFilter, :161-165), then ranked, so a query gets the
 * k nearest rows that pass among its probed candidates, at any selectivity.
 * The filter is a bitmap over the stored rows' ids: a row with id i is a
 * candidate when 0 <= i < allow_bits and bit i % 32 of allow[i / 32] is
 * set (rows added with ids = NULL have ids 0, 1, 2, ... in insertion
 * order).  The probes are the unfiltered ones (the reference probes before
 * it filters).  allow = NULL with allow_bits = 0 is vsk_ivf_search. */
vsk_status vsk_ivf_search_filtered(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                                   int64_t nq, int32_t nprobe, int32_t k, int32_t metric,
                                   const uint32_t *allow, int64_t allow_bits, float *out_dist,
                                   int64_t *out_ids);
/* IVFIndex.delete(id:) (:210-220): every stored row whose id is one of
 * ids[0 .. n) leaves its inverted list; the rows after it in the list keep
 * their order, so later searches rank exactly as the reference's lists do
 * after remove(at:).  *removed (may be NULL) receives the number of rows
 * removed.  Codes made by vsk_ivf_encode_* stay valid for the rows kept. */
vsk_status vsk_ivf_remove(vsk_ctx *ctx, vsk_ivf *ivf, const int64_t *ids, int64_t n,
                          int64_t *removed);
/* getVectorsFromList for every list at once (:487-490): ids (total, may be
 * NULL) receives the stored rows' ids in list order and offsets (nlist + 1,
 * may be NULL) where each list starts; list l holds ids[offsets[l] ..
 * offsets[l+1]). */
vsk_status vsk_ivf_list_ids(vsk_ctx *ctx, const vsk_ivf *ivf, int64_t *ids, int64_t *offsets);
/* sizes[nlist] = rows per inverted list; total = sum */
vsk_status vsk_ivf_list_sizes(vsk_ctx *ctx, const vsk_ivf *ivf,
                              int64_t *sizes);
/* ---- IVF-SQ8 and IVF-PQ ----------------------------------------------------
 * IVFConfiguration declares quantized lists (Config/Indexes/IVFConfiguration.
 * swift:13,18-21) that IVFIndex never implements.  Here an IVF index can
 * carry codes of its stored rows in the same list order, and a search
 * probes lists exactly as vsk_ivf_search (IVFIndex.search, Indexes/
 * IVFIndex.swift:149-202) but scores the probed lists' codes:
 *  - SQ8: score = sum_j qcode_j * code_j, the vsk_sq8_search score
 *    (codes from vsk_sq8_encode with the given parameters, ScalarQuantizer.
 *    quantizeToInt8, Quantization/ScalarQuantizer.swift:251-270);
 *  - PQ: the ADC sum of vsk_pq_search (DistanceTables.computeDistance,
 *    Quantization/ProductQuantizerTypes.swift:14-20), codes from
 *    vsk_pq_encode; returned as its square root.
 * Candidates are ordered as the stable sort of IVFIndex.search orders them:
 * by score (descending) or ADC sum (ascending), ties in probe order then
 * list order.  Codes are made from the rows the index holds at the call;
 * rows added later make the search fail with VSK_ERR_NOT_TRAINED until
 * the index is encoded again. */
vsk_status vsk_ivf_encode_sq8(vsk_ctx *ctx, vsk_ivf *ivf, int32_t per_dim,
                              const float *scale, const float *offset);
vsk_status vsk_ivf_encode_pq(vsk_ctx *ctx, vsk_ivf *ivf, const vsk_pq *pq);
/* q: nq x d fp32 (probing); qcodes: nq x d int8 (vsk_sq8_encode of q with
 * the same parameters).  out_score nq x k (INT32_MIN / -1 where missing). */
vsk_status vsk_ivf_search_sq8(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                              const int8_t *qcodes, int64_t nq, int32_t nprobe, int32_t k,
                              int32_t *out_score, int64_t *out_ids);
/* pq: the quantizer the codes were made with.  out_dist nq x k = sqrt of
 * the ADC sum (+inf / -1 where missing). */
vsk_status vsk_ivf_search_pq(vsk_ctx *ctx, const vsk_ivf *ivf, const vsk_pq *pq,
                             const float *q, int64_t nq, int32_t nprobe, int32_t k,
                             float *out_dist, int64_t *out_ids);

/* ---- IVF index file ----------------------------------------------------------
 * IVFIndex persistence keeps only the configuration and centroids
 * (export(format:), Indexes/IVFIndex.swift:297-328: the lists are dropped).
 * This file holds the whole index, little-endian:
 *   "VSKIVF02"; int32 nlist, d; int64 total, next_id;
 *   int32 code_kind, code_stride, pq_M, pq_ksub, sq8_per_dim, pq_dsub
 *   (code_kind 0 = none, 1 = SQ8, 2 = PQ; 17 / 18 = SQ8 / PQ codes only,
 *   without the rows section); int64 meta_bytes;
 *   float centroids[nlist][d]; int64 list_off[nlist + 1]; int64 ids[total];
 *   float rows[total][d] (list order); uint8 codes[total][code_stride];
 *   float quantizer[] (SQ8: scale then offset, d each when per-dimension,
 *   else 1 each; PQ: the codebooks, pq_M x pq_ksub x pq_dsub);
 *   uint8 meta[meta_bytes] (vsk_ivf_set_meta);
 *   uint64 FNV-1a of every byte before it.
 * Stale codes (rows added after the last encode) are not written.  Loading
 * bounds every header size (d <= 65536, nlist <= 2^24, total < 2^31, meta
 * <= 1 GiB), requires the file length the header implies, checks the list
 * offsets, that every PQ code is below pq_ksub, and the checksum
 * (VSK_ERR_IO otherwise). */
vsk_status vsk_ivf_save(vsk_ctx *ctx, const vsk_ivf *ivf, const char *path);
vsk_status vsk_ivf_load(vsk_ctx *ctx, const char *path, vsk_ivf **out);
/* Caller bytes kept with the index and its file (e.g. the encoded
 * IVFConfiguration, which IVFIndex's export keeps, :297-303).  get: *n =
 * the stored size; the first min(cap, *n) bytes go to out. */
vsk_status vsk_ivf_set_meta(vsk_ctx *ctx, vsk_ivf *ivf, const void *bytes, int64_t n);
vsk_status vsk_ivf_get_meta(vsk_ctx *ctx, const vsk_ivf *ivf, void *out, int64_t cap,
                            int64_t *n);
/* getCentroids() (:483): out nlist x d */
vsk_status vsk_ivf_centroids(vsk_ctx *ctx, const vsk_ivf *ivf, float *out);
/* The SQ8 parameters the index's codes were made with (scale and offset: d
 * floats each when *per_dim, else 1); VSK_ERR_NOT_TRAINED without current
 * SQ8 codes.  vsk_ivf_search_pq likewise refuses a quantizer whose
 * codebooks differ from the ones the codes were made with
 * (VSK_ERR_DIMENSION_MISMATCH). */
vsk_status vsk_ivf_sq8_params(vsk_ctx *ctx, const vsk_ivf *ivf, int32_t *per_dim,
                              float *scale, float *offset);
/* A quantized index that keeps only its codes: IVFConfiguration's
 * quantization (Config/Indexes/IVFConfiguration.swift:13,18-21) is there to
 * shrink the index, which the reference declares but never builds.  After
 * vsk_ivf_encode_sq8 / _pq, the fp32 rows (total x d x 4 bytes) and their
 * screen plane are freed; ids, lists, codes and the quantizer stay.  Then
 * vsk_ivf_search_sq8 / _pq answer exactly as before, vsk_ivf_add encodes the
 * new rows with the stored quantizer (their codes are what vsk_sq8_encode /
 * vsk_pq_encode give), vsk_ivf_remove and vsk_ivf_save / load keep codes
 * only, and the calls that read rows (vsk_ivf_search, _filtered,
 * vsk_ivf_encode_*) return VSK_ERR_UNSUPPORTED.  VSK_ERR_NOT_TRAINED
 * without current codes. */
vsk_status vsk_ivf_drop_rows(vsk_ctx *ctx, vsk_ivf *ivf);
/* *codes_only (may be NULL): 1 after vsk_ivf_drop_rows; *device_bytes (may
 * be NULL): the device memory the index holds (centroids and their planes,
 * rows, ids, list offsets, codes, the list screen's plane). */
vsk_status vsk_ivf_storage(vsk_ctx *ctx, const vsk_ivf *ivf, int32_t *codes_only,
                           int64_t *device_bytes);
/* nlist, d, total rows and code kind (0 none, 1 SQ8, 2 PQ) of an index */
vsk_status vsk_ivf_info(vsk_ctx *ctx, const vsk_ivf *ivf, int32_t *nlist, int32_t *d,
                        int64_t *total, int32_t *code_kind);


/* ---- int8 scalar quantization ---------------------------------------------
 * ScalarQuantizer (Quantization/ScalarQuantizer.swift).  per_dim = 0 is the
 * reference's global min/max (:389-451); per_dim = 1 applies the same
 * formulas per dimension.  scale/offset: d floats (per_dim) or 1. */
vsk_status vsk_sq8_train(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                         int32_t per_dim, float *scale, float *offset);
/* quantizeToInt8 (:251-270): code = clamp(trunc(x*scale + offset)) */
vsk_status vsk_sq8_encode(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                          int32_t per_dim, const float *scale,
                          const float *offset, int8_t *codes);
/* dequantizeFromInt8 (:568-580): x = (code - offset) / scale, n x d fp32 */
vsk_status vsk_sq8_decode(vsk_ctx *ctx, const int8_t *codes, int64_t n, int32_t d,
                          int32_t per_dim, const float *scale, const float *offset,
                          float *out);
/* quantizeVectors(vectors:scheme: .scalar(bits:)) of MetalAccelerationEngine
 * (Acceleration/MetalAccelerationEngine.swift:234-262) as its CPU path
 * computes it (AccelerateOptimizer.scalarQuantize, Acceleration/
 * AccelerateOptimizer.swift:387-430): per vector, scale = (2^bits - 1) /
 * (max - min) (1 when max == min) and code_i = UInt8(clamp((x_i - min) *
 * scale, 0, 255)), truncated toward zero.  codes: n x d uint8; scale, minv:
 * n floats each (may be NULL; the reference keeps them for dequantisation). */
vsk_status vsk_scalar_quantize_u8(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                                  int32_t bits, uint8_t *codes, float *scale, float *minv);
/* Resident database of n x d int8 codes (QuantizedVectorStore, :68-81).
 * Codes of up to 512 bytes are held only in a tiled layout (16-row blocks
 * in the matrix cores' operand order, rows padded to 64-byte k-steps),
 * which every scan reads; wider codes stay row-major.  The upload holds
 * both for the moment it converts. */
vsk_status vsk_sq8_upload(vsk_ctx *ctx, const int8_t *codes, int64_t n,
                          int32_t d, vsk_sq8 **out);
vsk_status vsk_sq8_free(vsk_ctx *ctx, vsk_sq8 *db);
/* Top k by score = sum_j qcode_j * code_j (int32, exact), i.e. ascending
 * distance -score.  out_score: nq x k int32 (INT32_MIN where missing). */
vsk_status vsk_sq8_search(vsk_ctx *ctx, const vsk_sq8 *db,
                          const int8_t *qcodes, int64_t nq, int32_t k,
                          int32_t *out_score, int64_t *out_ids);

/* No counterpart in the reference: vsk_sq8_search without any device
 * allocation, for callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * vsk_sq8_search, bit for bit, but qcodes, out_score and out_ids must be
 * device memory, and the working buffers (candidate keys, thresholds,
 * counters, padded query codes) live in one static 64 MiB device array per
 * GPU, held until the process ends.  Queries run in batches that fit it; a
 * (k, d) whose single query does not fit returns
 * VSK_ERR_INVALID_BUFFER_SIZE.  Every call on one GPU shares that array:
 * calls that overlap on one GPU (several contexts or threads) race.  The
 * call waits for the context's own stream before it returns (as every call
 * does), so it cannot be captured into a HIP graph. */
vsk_status vsk_sq8_search_noalloc(vsk_ctx *ctx, const vsk_sq8 *db,
                                  const int8_t *qcodes, int64_t nq, int32_t k,
                                  int32_t *out_score, int64_t *out_ids);

/* ---- product quantization -------------------------------------------------
 * ProductQuantizer (Quantization/ProductQuantizer.swift): M segments of
 * dsub dims, ksub codewords each (ksub <= 256, codes uint8).
 * codebooks: M x ksub x dsub fp32. */
vsk_status vsk_pq_create(vsk_ctx *ctx, const float *codebooks, int32_t M,
                         int32_t ksub, int32_t dsub, vsk_pq **out);
vsk_status vsk_pq_free(vsk_ctx *ctx, vsk_pq *pq);
/* One-call upload of a trained 8-bit quantizer (ksub = 256, the
 * configuration ProductQuantizationConfig fixes with codeSize 8,
 * Config/Quantization/ProductQuantizationConfig.swift:17-49) and n x M
 * resident codes (n may be 0): vsk_pq_create + vsk_pq_add_codes.  On failure
 * nothing is returned and *out is NULL. */
vsk_status vsk_pq_upload(vsk_ctx *ctx, const float *codebooks,
                         const uint8_t *codes, int64_t n, int32_t M,
                         int32_t dsub, vsk_pq **out);
/* encode (:68-112) via Codebook.encode (ProductQuantizerCodebook.swift:12-30):
 * codes n x M uint8 */
vsk_status vsk_pq_encode(vsk_ctx *ctx, const vsk_pq *pq, const float *x,
                         int64_t n, uint8_t *codes);
/* decode (:142-160, without the optional norm correction of :162-180, whose
 * norm these codes do not carry): out n x (M * dsub) fp32, each segment's
 * codeword */
vsk_status vsk_pq_decode(vsk_ctx *ctx, const vsk_pq *pq, const uint8_t *codes,
                         int64_t n, float *out);
/* Append n x M codes to the resident code database. */
vsk_status vsk_pq_add_codes(vsk_ctx *ctx, vsk_pq *pq, const uint8_t *codes,
                            int64_t n);
/* precomputeDistanceTables (:209-233): lut nq x M x ksub fp32 */
vsk_status vsk_pq_lut(vsk_ctx *ctx, const vsk_pq *pq, const float *q,
                      int64_t nq, float *lut);
/* ADC scan (DistanceTables.computeDistance, ProductQuantizerTypes.swift:
 * 14-20) over all resident codes -> top k_adc by ADC sum, then, when
 * rerank_db != NULL and rerank_metric >= 0, exact re-rank of those
 * candidates with rerank_metric on rerank_db's rows -> top k.  Without
 * re-rank the first k ADC results are returned as sqrt(sum). */
vsk_status vsk_pq_search(vsk_ctx *ctx, const vsk_pq *pq, const float *q,
                         int64_t nq, int32_t k_adc, int32_t k,
                         int32_t rerank_metric, const vsk_db *rerank_db,
                         float *out_dist, int64_t *out_ids);

/* ---- binary quantization ---------------------------------------------------
 * quantizeVectors(scheme: .binary) (Acceleration/MetalAccelerationEngine.swift:
 * 234-262) -> AccelerateOptimizer.binaryQuantize
 * (Acceleration/AccelerateOptimizer.swift:447-481): bit i of a code is
 * x_i > 0, stored in byte i/8 at bit i%8 (the Metal binaryQuantize,
 * Acceleration/Metal/Shaders/QuantizationShaders.metal:232-260, writes the
 * same bits as little-endian 32-bit words).  codes: n x ceil(d/8) bytes. */
vsk_status vsk_binary_encode(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                             uint8_t *codes);
/* Resident binary codes: n x ceil(d/8) bytes, d bits each. */
vsk_status vsk_bin_upload(vsk_ctx *ctx, const uint8_t *codes, int64_t n,
                          int32_t d, vsk_bin **out);
vsk_status vsk_bin_free(vsk_ctx *ctx, vsk_bin *bin);
/* Top k by Hamming distance popcount(q xor x) (binaryHammingDistance,
 * QuantizationShaders.metal:285-305), ties by row id.  qcodes: nq x
 * ceil(d/8) bytes; out_dist: nq x k int32 (INT32_MAX where missing). */
vsk_status vsk_bin_search(vsk_ctx *ctx, const vsk_bin *bin, const uint8_t *qcodes,
                          int64_t nq, int32_t k, int32_t *out_dist,
                          int64_t *out_ids);
/* binaryHammingDistance for every (query, row): out nq x n float, as the
 * Metal kernel writes it. */
vsk_status vsk_bin_distances(vsk_ctx *ctx, const vsk_bin *bin,
                             const uint8_t *qcodes, int64_t nq, float *out);

/* ---- HNSW neighbour distances ---------------------------------------------
 * The distance evaluations of HNSWIndex's graph walk (greedySearchLayer /
 * searchLayer0, Indexes/HNSWIndex.swift:1035-1221), batched over many
 * concurrent searches: for query i, the rows rows[offsets[i] ..
 * offsets[i+1]) of db (the nodes' vectors; a CSR list of its frontier's
 * neighbours) get out[j] = DistanceComputer.distance(q_i, x_rows[j])
 * (:1920-1959): VSK_METRIC_L2 sqrt of SIMD.sum() of the squared differences,
 * VSK_METRIC_COSINE_NOEPS 1 - dot/(|q||x|) (no epsilon), VSK_METRIC_L1 the
 * sum of |q_i - x_i|; VSK_METRIC_L2SQ the sum without the sqrt.  Sums run in
 * dimension order without FMA (SIMD.sum() from -0, reduce(0) from +0), so
 * the distances equal the reference's bit for bit.  DistanceComputer falls
 * back to euclidean for the other metrics; other codes return
 * VSK_ERR_UNSUPPORTED.  offsets: nq + 1 non-decreasing int64 starting at 0;
 * rows: offsets[nq] int32 row indices of db (an index outside it returns
 * VSK_ERR_INVALID_ARGUMENT); out: offsets[nq] floats. */
vsk_status vsk_hnsw_distances(vsk_ctx *ctx, const vsk_db *db, const float *q, int64_t nq,
                              const int64_t *offsets, const int32_t *rows, int32_t metric,
                              float *out);

/* ---- k-means -------------------------------------------------------------
 * KMeansClustering.cluster (Clustering/KMeansClustering.swift:48-113), the
 * trainer behind IVFIndex.train (Indexes/IVFIndex.swift:397-446) and
 * ProductQuantizer's codebooks (Quantization/ProductQuantizer.swift:270-324).
 * Each iteration assigns every row to its nearest centroid (sqrt-L2 summed in
 * dimension order, strict '<', :271-295), replaces each centroid by the fp32
 * mean of its rows summed in row order (x * weight, counts += weight,
 * :342-380), and stops when |inertia - previous| < tolerance, inertia being
 * the fp32 sum of the assigned distances in row order (:97-98).  An empty
 * cluster takes row Int.random(in: 0..<n) of SeedableRNG(seed +
 * 0x9E3779B97F4A7C15) (:374 draws it unseeded). */
#define VSK_KMEANS_INIT_RANDOM 0    /* .random: first k of shuffled rows (:197-207) */
#define VSK_KMEANS_INIT_CUSTOM 1    /* .custom(centroids) (:189-193)              */
#define VSK_KMEANS_INIT_PLUSPLUS 2  /* .kMeansPlusPlus (:209-259), D^2 sampling     */

/* ClusteringResult (:9-29) without the arrays */
typedef struct {
  int32_t iterations;
  int32_t converged;
  float inertia; /* +inf when no iteration ran */
} vsk_kmeans_result;

/* x: n x d rows; weights: n or NULL; init_centroids: k x d for
 * VSK_KMEANS_INIT_CUSTOM (else ignored); out_centroids: k x d;
 * out_assign: n or NULL (the last assignment step; zeros when max_iter = 0).
 * Errors as ClusteringError (:453-478): n = 0 -> VSK_ERR_EMPTY_INPUT,
 * k outside 1..n -> VSK_ERR_INVALID_ARGUMENT, degenerate data for
 * k-means++ -> VSK_ERR_INVALID_ARGUMENT. */
vsk_status vsk_kmeans(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                      int32_t k, const float *weights, int32_t init_method,
                      const float *init_centroids, uint64_t seed,
                      int32_t max_iter, float tolerance, float *out_centroids,
                      int32_t *out_assign, vsk_kmeans_result *result);

#ifdef __cplusplus
}
#endif
#endif /* VSK_HIP_H */
