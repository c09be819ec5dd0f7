// flat.hpp -- the flat scan kernels' launch interface, shared by the flat
// search, IVF probing/assignment and the PQ re-rank.
#pragma once

#include "vsk_api.hpp"

namespace vsk {

// internal metric: sqrt(sum (q-x)^2) summed in dimension order without FMA
// (bit-identical to a sequential fp32 loop; VALU kernel)
constexpr int32_t METRIC_L2_EXACT = 100;
// the same for L2^2, normalised cosine (1 - dot) and dot (-dot)
constexpr int32_t METRIC_L2SQ_EXACT = 101;
constexpr int32_t METRIC_CN_EXACT = 102;
constexpr int32_t METRIC_DOT_EXACT = 103;
// the reference's cosine 1 - q.x/(|q||x| + 1e-8): the dot product summed in
// dimension order, with the norms of seq_norms (a.qaux, a.xaux)
constexpr int32_t METRIC_COS_EXACT = 104;
// the exact VALU metric that computes a public metric as the CPU reference
// does (-1 if none)
inline int32_t exact_metric(int32_t metric) {
  switch (metric) {
  case VSK_METRIC_L2SQ: return METRIC_L2SQ_EXACT;
  case VSK_METRIC_L2: return METRIC_L2_EXACT;
  case VSK_METRIC_COSINE_NORMALIZED: return METRIC_CN_EXACT;
  case VSK_METRIC_DOT: return METRIC_DOT_EXACT;
  case VSK_METRIC_COSINE: return METRIC_COS_EXACT;
  case VSK_METRIC_L1: return VSK_METRIC_L1;
  case VSK_METRIC_HAMMING: return VSK_METRIC_HAMMING;
  default: return -1;
  }
}

// The 32-bit candidate word that selections skip: the word of a NaN distance
// and of a candidate a search's row filter excludes.
constexpr uint32_t kWordNone = 0xFFFFFFFFu;

enum { MODE_DENSE = 0, MODE_FILTER = 1, MODE_MATRIX = 2, MODE_ARGMIN = 3,
       // the screen only: per (query, row split) the smallest key and the
       // second smallest distance (a.cand[q * a.ldm + split] and
       // a.mat[q * a.ldm + split])
       MODE_TOP2 = 4 };

struct FlatArgs {
  const float *X;
  int64_t ldx;
  const float *Q;
  int64_t ldq;
  const float *xaux;  // |x|^2 (L2), |x| (cosine), else null
  const float *qaux;  // same for queries
  int32_t kdim;       // padded dimension (multiple of 4)
  int32_t nq;
  int64_t r0, r1;
  int64_t rows_per_split;
  int32_t metric;
  const uint64_t *thresh;
  const uint8_t *active;
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
  float *mat;  // MODE_MATRIX output, row-major nq x ldm
  int64_t ldm;
  int32_t splits_per_xcd;  // bf16x3 kernel: row splits owned by each XCD
  // screen kernel: > 0 selects the split-major order, XCD x taking query
  // tiles x*Q .. x*Q+Q-1 (Q = this value) over every row split in turn
  int32_t qtiles_per_xcd;
  // screen kernel, filter mode: candidate slots each workgroup reserves per
  // query (0: append through per-candidate atomics)
  int32_t sub;
  // screen kernel, filter mode: segmented lists (segment = row split, at
  // q*cap + split*sub) with their key counts here (nq x nseg), else null
  int32_t *seg_n;
  // MODE_ARGMIN: the winning distance per query (optional)
  float *amin;
};

// bf16 of an fp32 value, round to nearest even (NaN stays NaN)
__device__ inline uint16_t bf16_rn(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFF) ? 0x40 : 0));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// float not below a non-negative double (the error bounds round up)
__device__ inline float f_up(double v) {
  float f = (float)v;
  if ((double)f < v) f = __uint_as_float(__float_as_uint(f) + 1u);
  return f;
}
// the largest float at or below v >= 0
__device__ inline float f_down(double v) {
  float f = (float)v;
  if ((double)f > v) f = __uint_as_float(__float_as_uint(f) - 1u);
  return f;
}

// The screen's error bound eps for a query with |bf16(q)| = qh and
// |q - bf16(q)| = qr against rows whose maxima of |bf16(x)| and |x - bf16(x)|
// are xh and xr, over d dimensions (the derivation heads flat_screen.hip):
// every screened distance lies within eps of the reference's fp32 one.
// With the query as two bf16 planes (q = qh' + ql' + r), qh is |qh'| + |ql'|,
// qr is |r| and the screen sums nprod = 2d exact products instead of d.
// Cosine with the reference's epsilon (1 - q.x/(|q||x| + 1e-8)): xh and xr
// are then the maxima over the rows of |bf16(x)| / |x| and |x - bf16(x)| /
// |x| (|x| the fp32 norm the screen divides by, rows of norm 0 excluded:
// both forms give exactly 1 there) and qnorm the query's fp32 norm.  The dot
// product's error is then at most |x| (qh xr + qr xh + qr xr + 2(d-1)u qh xh)
// and its quotient by |q||x| + 1e-8 at most that over |q| (times 1 + (d+8)u
// for the norms' roundings); the reference's own sums, norms, quotient and
// subtraction err by at most (2.1 d + 11) u and the screen's fp32 norms and
// last operations by (1.1 d + 9) u.  A zero query gives 1 for every row in
// both forms (no error); a query of tiny or non-finite norm gets no bound
// (it fails the check and is redone exactly).
__device__ inline double screen_eps_of(double qh, double qr, double xh, double xr, int32_t d,
                                       int32_t metric, int32_t nprod = 0, double qnorm = 0.0) {
  const double u = 0x1p-24;
  const double qn = qh + qr, xn = xh + xr, dd = (double)d;
  const double np = nprod > 0 ? (double)nprod : dd;
  if (metric == VSK_METRIC_COSINE) {
    if (qh == 0.0 && qr == 0.0) return 4.0 * u;
    if (!(qnorm >= 0x1p-60) || !(qnorm <= 0x1p60)) return __builtin_inf();
    const double x = qh * xr + qr * xh + qr * xr + 2.0 * (np - 1.0) * u * qh * xh;
    return (x / qnorm * (1.0 + (dd + 8.0) * u) + (3.2 * dd + 20.0) * u + 0x1p-80) * 1.01;
  }
  const double e_dot =
      qh * xr + qr * xh + qr * xr + 2.0 * (np - 1.0) * u * qh * xh + np * 0x1p-126;
  const double e_ref = 1.01 * dd * u * qn * xn;
  double eps;
  if (metric == VSK_METRIC_DOT)
    eps = e_dot + e_ref;
  else if (metric == VSK_METRIC_COSINE_NORMALIZED)
    eps = e_dot + e_ref + 2.02 * u * (1.0 + qn * xn + e_dot);
  else
    // (the last term: the filter pass accumulates dot - |x|^2/2 from
    // -|x|^2/2, so its partial sums carry |x|^2/2 more: 2 np u |x|^2/2 more
    // on the dot, twice that on the distance, plus a rounding of each)
    eps = 2.0 * e_dot + (2.0 * dd + 8.0) * u * (qn + xn) * (qn + xn) * 1.05 +
          (2.0 * np + 4.0) * u * xn * xn * 1.01;
  return eps * 1.0001;
}

// Screened keys a within the margin of the k-th.  With A_k the k-th
// smallest screened distance, a row whose a exceeds A_k + 2 eps (for sqrt-L2
// ranking (A_k + eps)(1 + 2^-20) + eps, so that the square root's rounding
// cannot tie it) has an exact distance strictly above k rows' and cannot be
// in the top k: only the keys at or below that limit need their exact
// distances.  One workgroup per query over 32-bit screened words: word i of
// query q is words[wseg[q] + i], i < cnt[q] (wseg a multiple of 4), keyed
// (word, i).  The keys within the margin go to out[q * cap ...], unordered,
// their number to nout[q]; ok[q] = nout[q] <= cap and bad[q] its negation.
struct MarginArgs {
  int64_t nq = 0;
  int32_t k = 0;
  const uint32_t *words = nullptr;
  // query q's words: at wseg[q], cnt[q] of them; or, wseg and cnt null, at
  // q * wstride (a multiple of 4), wn of them
  const int64_t *wseg = nullptr, *cnt = nullptr;
  int64_t wstride = 0, wn = 0;
  const float *qnh = nullptr, *qnr = nullptr;  // per query |qh|, |q - qh|
  double xh = 0, xr = 0;
  int32_t d = 0, metric = 0;
  int32_t nprod = 0;  // products the screen summed (0: d; 2d with a query lo plane)
  uint64_t *out = nullptr;
  int32_t cap = 0;
  int32_t *nout = nullptr;
  uint8_t *ok = nullptr, *bad = nullptr;
  unsigned long long *nbad = nullptr;  // optional: += the queries over cap
};
void launch_screen_margin(vsk_ctx *ctx, const MarginArgs &a);

// A screen's whole tail for a query in one workgroup: the margin gather of
// m (at most m.cap <= 1024 keys, kept in LDS), their exact distances -- the
// reference's sequential fp32 sum of (q - x)^2 over ld columns, its square
// root unless squared -- and the top m.k of those, sorted, into best_out.
// A query with more than m.cap keys in its margin has the exact key of
// every candidate written to all (at seg_off[q], or q * all_n with all_n
// candidates) and selected from there instead.  Rows: with list_off, a
// candidate's position maps to its probe slot (pos_base, probes: np a
// query) and row as in the IVF candidate segments; without, the position
// is the row.  m.out, m.nout, m.ok and m.bad are not used.
struct ScreenTailArgs {
  MarginArgs m;
  const float *rows = nullptr, *Q = nullptr;
  int32_t ld = 0, squared = 0;
  const int64_t *list_off = nullptr, *pos_base = nullptr;
  const int32_t *probes = nullptr;
  int32_t np = 0;
  uint64_t *all = nullptr;
  const int64_t *seg_off = nullptr;
  int64_t all_n = 0;
  uint64_t *best_out = nullptr;
  // compact candidates (the IVF list scan under a per-query bound, list_off
  // set, np <= 256): probe slot p's kept candidates are the first
  // pcnt[q * np + p] words from its base, m.words[wseg[q] + pos_base], and
  // at the same places of prow their rows' offsets in the list (the
  // candidate's position is the base plus that offset); a slot whose list
  // is empty has none.  Null: every candidate's word at its position.
  const int32_t *pcnt = nullptr;
  const uint32_t *prow = nullptr;
  // only the queries with active[q] (all when null)
  const uint8_t *active = nullptr;
};
void launch_screen_tail(vsk_ctx *ctx, const ScreenTailArgs &a, const char *name);

// Exact top k per query of 32-bit words keyed (word, index), sorted
// ascending into best_out[q * k ...] (NONE past the words): query q's words
// are words[wseg[q] + i], i < cnt[q] (wseg a multiple of 4); only queries
// with active[q] (all when null).  The keys are those of a scan writing
// (word << 32) | position.
struct WordSelectArgs {
  int64_t nq = 0;
  int32_t k = 0;
  const uint32_t *words = nullptr;
  const int64_t *wseg = nullptr, *cnt = nullptr;
  uint64_t *best_out = nullptr;
  const uint8_t *active = nullptr;
};
void launch_select_words(vsk_ctx *ctx, const WordSelectArgs &a, const char *name);

// bf16 hi/lo operand planes of the bf16x3 kernel
struct SplitPtrs {
  const uint16_t *xh, *xl;  // row planes, stride ldxb
  const uint16_t *qh, *ql;  // query planes, stride ldqb
  int64_t ldxb, ldqb;
  int32_t kb;               // padded dimension (multiple of 64)
};
// hi = bf16(x) and (lo non-null) lo = bf16(x - hi) of an (n x ld) fp32
// matrix, ldb columns; nhi/nres (optional): per-row |hi| and |x - hi|,
// rounded up, with their maxima over the rows atomically max-ed (as float
// bits) into maxbits[0..1] when maxbits is given
void split_bf16(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
                uint16_t *hi, uint16_t *lo, int32_t ldb, float *nhi = nullptr,
                float *nres = nullptr, uint32_t *maxbits = nullptr);
// bf16 MFMA scan: passes 3 = hi/lo split products (fp32-level accuracy),
// passes 1 = hi products only (the screen; no matrix mode, no COSINE)
void launch_flat_bf16x3(vsk_ctx *ctx, FlatArgs a, const SplitPtrs &s, int mode,
                        int passes = 3);
// the screen's one-pass kernel on 256 x 256 tiles (dense or filter mode;
// L2^2, L2, normalised cosine, dot)
// (filter mode with a.seg_n: *nseg and *stride receive the segment layout)
void launch_flat_screen(vsk_ctx *ctx, FlatArgs a, const SplitPtrs &s, int mode,
                        int32_t *nseg = nullptr, int64_t *stride = nullptr);

// launch one scan over rows [a.r0, a.r1) of a.X for the a.nq queries of a.Q
// (mode MODE_*; argmin output only for MODE_ARGMIN).  a.rows_per_split is
// chosen here.
void launch_flat(vsk_ctx *ctx, FlatArgs a, int mode, int32_t *argmin);

// top-k of queries dq (device, stride db->ld) over a resident database;
// best: nq*k keys.  Returns true when the keys hold the final distances
// (the screen path: exact fp32, sqrt applied for L2), false when they hold
// the kernel's distances (squared for L2).
struct ScreenDeferred;
bool flat_topk_device(vsk_ctx *ctx, const vsk_db *db, const float *dq,
                      int64_t nq, int32_t k, int32_t metric, uint64_t *best,
                      ScreenDeferred *defer = nullptr);
// progressive top-k on the bf16 kernel with the given passes (3: fp32-level
// distances; 1: the screen's hi products) or, for L1, the exact VALU kernel;
// qnh/qnr (optional): per-query |hi| and |q - hi| of the split;
// max_growth: the progressive scan's chunk growth limit (0: none)
void approx_topk(vsk_ctx *ctx, const vsk_db *db, const float *dq, int64_t nq,
                 int32_t k, int32_t metric, uint64_t *best, int passes,
                 float *qnh = nullptr, float *qnr = nullptr,
                 int64_t max_growth = 0);
// the bf16 planes of the database (built once, with the maxima of |hi| and
// |x - hi| over its rows) and of a query batch (lo plane when qlo; per-query
// |hi| into qnh and |q - hi| into qnr when given)
SplitPtrs make_split(vsk_ctx *ctx, const vsk_db *db, const float *dq,
                     int64_t nq, bool qlo, float *qnh, float *qnr);
// |x|^2 (L2 metrics) or |x| (cosine) of the rows / of a query batch; for
// METRIC_COS_EXACT the reference's sequential norms (ensure_seq_norms makes
// the rows' first)
const float *x_aux(const vsk_db *db, int32_t metric);
void ensure_seq_norms(vsk_ctx *ctx, const vsk_db *db);
float *q_aux(vsk_ctx *ctx, const float *dq, int64_t nq, int32_t d, int32_t ld,
             int32_t metric);
// bf16 planes and norms of a query batch for screen_argmin: hi plane
// (stride ldb = roundup(d, 64)), |hi|, |q - hi| and |q|^2 per query
// the screen's bound check over each query's kc kept screen keys (see
// flat_screen.hip): ok[q] when the kept keys hold the exact top k, and
// nvalid[q] = how many kept keys lie within the bound's margin of the k-th
struct CheckArgs {
  const uint64_t *best;  // nq x kc screen keys, ascending, NONE last
  int64_t nq;
  int32_t k, kc, d, metric;
  const float *qnh, *qnr;  // per query |qh|, |q - qh|
  double xh, xr;           // maxima over the rows of |xh|, |x - xh| (cosine: relative)
  const float *qn = nullptr;  // cosine: per query |q| (fp32, as the screen divides)
  uint8_t *ok;
  int32_t *nvalid;
  int32_t *fails;
  bool test;  // false: count the valid keys only
};
void launch_screen_check(vsk_ctx *ctx, const CheckArgs &ca);

struct ArgminQueries {
  const uint16_t *qh = nullptr;
  const float *qnh = nullptr, *qnr = nullptr, *qsq = nullptr;
  int32_t ldb = 0;
  // a second plane ql = bf16(q - qh) when the screen takes the query as two
  // planes (then qnh = |qh| + |ql|, qnr = |q - qh - ql|, nprod = 2d)
  const uint16_t *ql = nullptr;
  int32_t nprod = 0;
};
ArgminQueries argmin_queries(vsk_ctx *ctx, const float *dq, int64_t nq, int32_t d,
                             int32_t ld, const char *slot);
// whether the screen serves an argmin of nq queries over n rows of d dims
bool screen_argmin_applies(vsk_ctx *ctx, int64_t nq, int64_t n, int32_t d);
// exact nearest row of each query (sqrt-L2 summed in dimension order, the
// first minimum under strict '<'): argmin[q] and its distance dist[q].  X:
// n x ld rows with |x|^2 in xsq; dq: the queries (stride ld) with their
// planes qp.  A bf16 screen keeps each query's smallest and second smallest
// approximate distance; a query whose two are apart by more than the
// screen's error bound takes the first (its exact distance recomputed), the
// rest are redone by the exact VALU scan.
void screen_argmin(vsk_ctx *ctx, const float *X, const float *xsq, int64_t n,
                   int32_t d, int32_t ld, const float *dq, int64_t nq,
                   const ArgminQueries &qp, int32_t *argmin, float *dist);

// exact top-k through the screen (flat_screen.hip): a one-pass bf16 scan
// keeps screen_keep(k) candidates per query, a proven error bound shows they
// hold the exact top-k, and an fp32 rescore in the CPU reference's summation
// order ranks them (a query failing the bound is redone by the exact VALU
// scan); best: final keys (exact distances)
bool screen_applies(int32_t metric, int32_t k);
// cosine through the screen needs the rows' relative residual maxima (made
// here once per database); false when a row's norm is too small or not
// finite for the bound (cosine then takes the exact scan)
bool cosine_screen_ok(vsk_ctx *ctx, const vsk_db *db);
int32_t screen_keep(int32_t k);
// With defer, screen_topk queues every batch without waiting for the bound
// check: each batch's count of failing queries goes to pinned memory with
// the stream, and screen_finish, called after the caller's synchronisation,
// redoes the failing queries (rare) -- true when it redid any (best then
// holds their new keys).
struct ScreenDeferred {
  struct Batch {
    int64_t b0, nb;
  };
  std::vector<Batch> batches;
  int32_t *fails_host = nullptr;  // pinned, one count per batch
  uint8_t *ok = nullptr;          // device, per query
  int32_t kc = 0;
  bool active = false;
};
void screen_topk(vsk_ctx *ctx, const vsk_db *db, const float *dq, int64_t nq,
                 int32_t k, int32_t metric, uint64_t *best,
                 ScreenDeferred *defer = nullptr);
bool screen_finish(vsk_ctx *ctx, const vsk_db *db, const float *dq, int32_t k,
                   int32_t metric, uint64_t *best, ScreenDeferred &defer);

// out[s * len ...] = the keys of in[s * len ...] sorted ascending, for
// each of nseg segments of len keys (at most 2^31 - 1 keys in all)
void segmented_sort_u64(vsk_ctx *ctx, const uint64_t *in, uint64_t *out, int64_t nseg,
                        int64_t len);

// a PQ quantizer's shape for other translation units: returns d
int32_t pq_shape(const vsk_pq *pq, int32_t *M, int32_t *ksub);
bool pq_shape_matches(const vsk_pq *pq, int32_t d, int32_t M, int32_t ksub);
// the quantizer's codebooks on the host (M x ksub x dsub) and its dsub
const std::vector<float> &pq_host_codebooks(const vsk_pq *pq, int32_t *dsub);

}  // namespace vsk
