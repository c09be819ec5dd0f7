// flat_screen.hip -- exact flat top-k for L2^2, L2, cosine (the reference's
// epsilon form), normalised cosine and dot: a one-pass bf16 MFMA screen, a
// proven bound on its error, and an fp32 rescore of the survivors in the CPU
// reference's own summation order.
//
// Bound.  With qh = bf16(q), xh = bf16(x) and the exact residuals
// dq = q - qh, dx = x - xh, Cauchy-Schwarz gives
//   |q.x - qh.xh| <= |qh||dx| + |dq||xh| + |dq||dx|.
// Each product qh_i xh_i is exact in fp32 (8-bit significands), and any fp32
// summation of d of them, in any order and with round-to-nearest or
// truncation, errs by at most 2(d-1)u sum|qh_i xh_i| <= 2(d-1)u |qh||xh|,
// u = 2^-24.  Taking the maxima of |xh| and |dx| over the rows bounds every
// pair of one query: eps_dot(q).  (The filter pass on L2 and L2^2 starts
// its sums at -|x|^2/2 instead of 0: that adds 2 d u |x|^2/2 to the sum's
// error, which screen_eps_of adds for those metrics.)  The screen's distance
// a(x) of each metric
// is then within eps(q) of the distance d(x) the rescore computes; eps adds
// the error of the reference's sequential fp32 sum and of the metric's last
// operations (norms and the final subtraction for L2^2, 1 - s for cosine).
//
// Claim: if A_kc - eps > A_k + eps, where A_j is the j-th smallest a over
// all rows and the screen kept the kc rows of smallest a, those kc rows hold
// the exact top-k.  Any other row y has d(y) >= a(y) - eps >= A_kc - eps,
// while the k rows with a <= A_k have d <= A_k + eps: y is strictly beaten
// by k rows.  For L2 the ranking distance is sqrt(d), and the test asks for
// a relative gap of 2^-20 so that rounding of the square root cannot tie
// them.  A query failing the test (rows closer to each other than the
// bound: none of config 2's queries, but planted near-duplicates do it) is
// screened again keeping 1024 candidates, and one failing that too is redone
// by the exact VALU scan, which evaluates the reference's formula for every
// row.  The epsilon cosine's bound is relative to the norms (screen_eps_of).
//
// Kept rows above that limit are beaten the same way, so only the rows of
// a within 2 eps of A_k are rescored.
//
// The rescore sums in dimension order without FMA, exactly as the CPU
// reference (Indexes/IVFIndex.swift:542-549 and
// Acceleration/AccelerateOptimizer.swift:251-383 restated sequentially), so
// the returned distances are bit-identical to it and the order is (distance,
// row id) over exact fp32 distances.
#include <cstring>
#include <vector>

#include "flat.hpp"

namespace vsk {

bool screen_applies(int32_t metric, int32_t k) {
  if (metric != VSK_METRIC_L2SQ && metric != VSK_METRIC_L2 &&
      metric != VSK_METRIC_COSINE_NORMALIZED && metric != VSK_METRIC_DOT &&
      metric != VSK_METRIC_COSINE)
    return false;
  return k <= VSK_MAX_K;
}

// per row (one wave): |bf16(x)| and |x - bf16(x)| (sums of squares in
// double, square roots rounded up) over the fp32 norm |x| the screen
// divides by, their maxima over the rows with |x| > 0 as float bits
// (atomic max, ratios rounded up) in rel[0..1]; rel[2] = 1 when a row with
// a nonzero component has a norm below 2^-60 or not finite
__global__ __launch_bounds__(256) void k_cos_rel(const float *x, int64_t n, int32_t d,
                                                 int32_t ld, const float *norm, uint32_t *rel) {
  const int lane = threadIdx.x & 63;
  uint32_t mh = 0, mr = 0, bad = 0;
  for (int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < n; r += (int64_t)gridDim.x * 4) {
    double sh = 0.0, sr = 0.0;
    for (int32_t c = lane; c < d; c += 64) {
      const float v = x[r * ld + c];
      const float hv = __uint_as_float((uint32_t)bf16_rn(v) << 16);
      const float rv = v - hv;  // exact
      sh += (double)hv * (double)hv;
      sr += (double)rv * (double)rv;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      sh += __shfl_xor(sh, o);
      sr += __shfl_xor(sr, o);
    }
    const double nx = (double)norm[r];
    if (sh == 0.0 && sr == 0.0) continue;  // a zero row: exactly 1 either way
    if (!(nx >= 0x1p-60) || !(nx <= 0x1p60)) {
      bad = 1;
      continue;
    }
    const float a = f_up(sqrt(sh) / nx * (1.0 + 1e-12));
    const float b = f_up(sqrt(sr) / nx * (1.0 + 1e-12));
    mh = __float_as_uint(a) > mh ? __float_as_uint(a) : mh;
    mr = __float_as_uint(b) > mr ? __float_as_uint(b) : mr;
  }
  if (lane == 0) {
    if (mh | mr) {
      atomicMax(&rel[0], mh);
      atomicMax(&rel[1], mr);
    }
    if (bad) atomicMax(&rel[2], 1u);
  }
}

bool cosine_screen_ok(vsk_ctx *ctx, const vsk_db *db) {
  if (db->cos_state == 0) {
    uint32_t *rel = static_cast<uint32_t *>(ctx->scratch_ptr("screen.cosrel", 16));
    fill_i32(ctx, reinterpret_cast<int32_t *>(rel), 4, 0);
    int64_t g = ceil_div(db->n, 4);
    if (g > 16384) g = 16384;
    k_cos_rel<<<(unsigned)g, 256, 0, ctx->stream>>>(db->x.as<float>(), db->n, db->d, db->ld,
                                                    db->norm.as<float>(), rel);
    check_launch("cos_rel");
    uint32_t h[3];
    VSK_HIP(hipMemcpyAsync(h, rel, sizeof(h), hipMemcpyDeviceToHost, ctx->stream));
    stream_sync(ctx);
    std::memcpy(&db->cos_rel_hi, &h[0], sizeof(float));
    std::memcpy(&db->cos_rel_res, &h[1], sizeof(float));
    db->cos_state = h[2] ? -1 : 1;
  }
  return db->cos_state > 0;
}

// candidates kept per query: on config 2 (k = 100) some 200-250 rows fall
// within the bound's margin of the k-th, so 3k + 64 makes the second,
// wider screen rare
int32_t screen_keep(int32_t k) {
  // 3k + 64, at least 256, at most the selection's VSK_MAX_K: above k = 320
  // the margin narrows (k = VSK_MAX_K keeps none, so only a database of at
  // most VSK_MAX_K rows passes the check; the others go to the exact scan)
  const int32_t kc = 3 * k + 64;
  return kc < 256 ? 256 : (kc > VSK_MAX_K ? VSK_MAX_K : kc);
}

// Exact distance of each screened candidate, summed in dimension order
// without FMA as the CPU reference does.  A block is 4 waves; a wave owns 64
// candidates of one query (uniform query loads).  Per 64-dim block the wave
// gathers its 64 rows with 256-byte segments (16 lanes per row) into its own
// LDS tile, then every lane continues the sequential sum of its row from
// there: coalesced reads, bit-exact sums.  The 16 segment loads of a block
// are unconditional (a missing candidate reads row 0, a segment past the
// row's end is clamped into it; neither is summed), so all of them are in
// flight at once, and the next block's loads run while this one is summed.
// out[q][c] = key(distance, row) for the first nvalid[q] candidates, NONE
// for the rest.
constexpr int RS_W = 64;       // dims per gathered block
constexpr int RS_LD = RS_W + 4;  // LDS row stride (floats): conflict-free
typedef float rs_f4 __attribute__((ext_vector_type(4)));

template <int METRIC>
__global__ __launch_bounds__(256) void k_rescore(const float *X, int64_t ldx,
                                                 const float *Q, int64_t ldq,
                                                 int32_t d, const uint64_t *cand,
                                                 int32_t kc, const int32_t *nvalid,
                                                 uint64_t *out) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float tile[4][64 * RS_LD];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t q = blockIdx.x;
  const int32_t c = blockIdx.y * 256 + threadIdx.x;
  const uint64_t key = c < nvalid[q] ? cand[q * kc + c] : VSK_KEY_NONE;
  const bool valid = key != VSK_KEY_NONE;
  const uint32_t row = (uint32_t)key;
  if (!__builtin_amdgcn_ballot_w64(valid)) return;  // wave past the candidates
  const float *qq = Q + q * ldq;
  float *t = tile[w];
  const int seg = lane & 15, sub = lane >> 4;  // 16 lanes per row segment
  // the rows this lane gathers: candidates sub, sub + 4, ..., sub + 60
  const uint32_t my_row = valid ? row : 0u;
  const float *src[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    src[i] = X + (int64_t)__shfl(my_row, sub + 4 * i) * ldx;
  const int32_t cmax = (int32_t)ldx - 4;  // a segment past the row end is clamped
  rs_f4 buf[16];
  {
    const int32_t col = 4 * seg < cmax ? 4 * seg : cmax;
#pragma unroll
    for (int i = 0; i < 16; ++i) buf[i] = *reinterpret_cast<const rs_f4 *>(src[i] + col);
  }
  float s = 0.f, sq = 0.f, sx = 0.f;  // (cosine: the two norms' sums)
  for (int32_t j0 = 0; j0 < d; j0 += RS_W) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      *reinterpret_cast<rs_f4 *>(t + (sub + 4 * i) * RS_LD + 4 * seg) = buf[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {
      // the next block (the last one reloads itself: no condition on the
      // loads)
      const int32_t jnext = j0 + RS_W < d ? j0 + RS_W : j0;
      const int32_t col = jnext + 4 * seg < cmax ? jnext + 4 * seg : cmax;
#pragma unroll
      for (int i = 0; i < 16; ++i) buf[i] = *reinterpret_cast<const rs_f4 *>(src[i] + col);
    }
    const int32_t jn = d - j0 < RS_W ? d - j0 : RS_W;
    const float *xr = t + lane * RS_LD;
    for (int32_t j = 0; j < jn; ++j) {
      const float qv = qq[j0 + j], xv = xr[j];
      if constexpr (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2) {
        const float tt = qv - xv;
        s = s + tt * tt;
      } else {
        s = s + qv * xv;
        if constexpr (METRIC == VSK_METRIC_COSINE) {
          sq = sq + qv * qv;
          sx = sx + xv * xv;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  if (c >= kc) return;
  if (!valid) {
    out[q * kc + c] = VSK_KEY_NONE;
    return;
  }
  float dist;
  if constexpr (METRIC == VSK_METRIC_L2SQ) dist = s;
  else if constexpr (METRIC == VSK_METRIC_L2) dist = sqrtf(s);
  else if constexpr (METRIC == VSK_METRIC_COSINE_NORMALIZED) dist = 1.0f - s;
  else if constexpr (METRIC == VSK_METRIC_COSINE)
    dist = 1.0f - s / (sqrtf(sq) * sqrtf(sx) + 1e-8f);  // the reference's formula
  else dist = -s;
  out[q * kc + c] = vsk_key(dist, row);
}

// the screen's error bound eps(q) for the metric (see the file comment)
__device__ double screen_eps(const CheckArgs &a, int64_t q) {
  return screen_eps_of(a.qnh[q], a.qnr[q], a.xh, a.xr, a.d, a.metric, 0,
                       a.qn ? (double)a.qn[q] : 0.0);
}

__global__ void k_screen_check(CheckArgs a) {
  const int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (q >= a.nq) return;
  const uint64_t *b = a.best + q * a.kc;
  int32_t lo = 0, hi = a.kc;  // first NONE (keys ascending, NONE last)
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (b[mid] == VSK_KEY_NONE) hi = mid;
    else lo = mid + 1;
  }
  a.nvalid[q] = lo;
  if (!a.test) return;
  bool good = true;
  if (lo >= a.k) {
    // a kept row y with a(y) - eps > A_k + eps (relative gap 2^-20 for
    // sqrt) is strictly beaten by k rows: only rows below lim are rescored,
    // and rows past the kept ones can be ignored when A_kc > lim
    const double ak = vsk_ord2f((uint32_t)(b[a.k - 1] >> 32));
    const double eps = screen_eps(a, q);
    double lim = ak + 2.0 * eps;
    if (a.metric == VSK_METRIC_L2) lim = (ak + eps) * (1.0 + 0x1p-20) + eps;
    int32_t l2 = a.k, h2 = lo;  // first kept key above lim
    while (l2 < h2) {
      const int32_t mid = (l2 + h2) >> 1;
      if ((double)vsk_ord2f((uint32_t)(b[mid] >> 32)) > lim) h2 = mid;
      else l2 = mid + 1;
    }
    a.nvalid[q] = l2;
    if (lo == a.kc) good = l2 < a.kc;  // rows beyond the kept ones exist
  }
  a.ok[q] = good ? 1 : 0;
  if (!good) atomicAdd(a.fails, 1);
}

void launch_screen_check(vsk_ctx *ctx, const CheckArgs &ca) {
  KernelTimer t(ctx, "screen_check");
  k_screen_check<<<(unsigned)ceil_div(ca.nq, 256), 256, 0, ctx->stream>>>(ca);
  check_launch("screen_check");
}

__global__ void k_gather_rows(const float *src, int64_t ld, const int32_t *idx,
                              int64_t m, float *dst) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < m * ld;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / ld, c = i - r * ld;
    dst[i] = src[(int64_t)idx[r] * ld + c];
  }
}

__global__ void k_scatter_keys(const uint64_t *src, int64_t m, int32_t k,
                               const int32_t *idx, uint64_t *dst) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < m * k;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / k, c = i - r * k;
    dst[(int64_t)idx[r] * k + c] = src[i];
  }
}

static unsigned grid_for(int64_t n) {
  int64_t g = ceil_div(n, 256);
  return (unsigned)(g < 1 ? 1 : (g > 16384 ? 16384 : g));
}

static void rescore(vsk_ctx *ctx, const vsk_db *db, const float *dq, int64_t nq,
                    const uint64_t *cand, int32_t kc, const int32_t *nvalid,
                    int32_t metric, uint64_t *out) {
  dim3 grid((unsigned)nq, (unsigned)ceil_div(kc, 256));
  KernelTimer t(ctx, "screen_rescore", (double)nq * kc);
  const float *X = db->x.as<float>();
  switch (metric) {
  case VSK_METRIC_L2SQ:
    k_rescore<VSK_METRIC_L2SQ><<<grid, 256, 0, ctx->stream>>>(X, db->ld, dq, db->ld,
                                                              db->d, cand, kc, nvalid, out);
    break;
  case VSK_METRIC_L2:
    k_rescore<VSK_METRIC_L2><<<grid, 256, 0, ctx->stream>>>(X, db->ld, dq, db->ld,
                                                            db->d, cand, kc, nvalid, out);
    break;
  case VSK_METRIC_COSINE_NORMALIZED:
    k_rescore<VSK_METRIC_COSINE_NORMALIZED><<<grid, 256, 0, ctx->stream>>>(
        X, db->ld, dq, db->ld, db->d, cand, kc, nvalid, out);
    break;
  case VSK_METRIC_COSINE:
    k_rescore<VSK_METRIC_COSINE><<<grid, 256, 0, ctx->stream>>>(X, db->ld, dq, db->ld, db->d,
                                                                cand, kc, nvalid, out);
    break;
  default:
    k_rescore<VSK_METRIC_DOT><<<grid, 256, 0, ctx->stream>>>(X, db->ld, dq, db->ld,
                                                             db->d, cand, kc, nvalid, out);
  }
  check_launch("screen_rescore");
}

// exact top-k of nb queries from their kc screened candidates: rescore,
// then select k by (exact distance, row)
static void rescore_select(vsk_ctx *ctx, const vsk_db *db, const float *dq,
                           int64_t nb, int32_t k, int32_t kc, int32_t metric,
                           const uint64_t *cand, const int32_t *nvalid,
                           uint64_t *best) {
  uint64_t *resc = static_cast<uint64_t *>(
      ctx->scratch_ptr("screen.resc", sizeof(uint64_t) * (size_t)nb * kc));
  rescore(ctx, db, dq, nb, cand, kc, nvalid, metric, resc);
  SelectArgs sa;
  sa.nq = nb;
  sa.k = k;
  sa.cand = resc;
  sa.cap = kc;
  sa.counts = nvalid;
  sa.best_out = best;
  launch_select(ctx, sa, "screen_select");
}

// one screen tier over nb queries keeping kc candidates each: screen,
// bound test, exact rescore and select into best (nb x k; rows of failing
// queries are written too but must be redone).  Returns the failing query
// indices.
// With fail_host (pinned), the tier does not wait for the check: ok_out
// (nb bytes of device memory) keeps each query's result and the failing
// count goes to *fail_host with the stream; the caller redoes the failing
// queries after its synchronisation (screen_finish).
static std::vector<int32_t> screen_tier(vsk_ctx *ctx, const vsk_db *db,
                                        const float *qbat, int64_t nb, int32_t k,
                                        int32_t kc, int32_t metric,
                                        uint64_t *best, const char *tag,
                                        uint8_t *ok_out = nullptr,
                                        int32_t *fail_host = nullptr) {
  uint64_t *cand = static_cast<uint64_t *>(ctx->scratch_ptr(
      std::string("screen.cand") + tag, sizeof(uint64_t) * (size_t)nb * kc));
  float *qn = static_cast<float *>(ctx->scratch_ptr(
      std::string("screen.qnorm") + tag, sizeof(float) * 2 * (size_t)nb));
  approx_topk(ctx, db, qbat, nb, kc, metric, cand, 1, qn, qn + nb, 8);

  uint8_t *ok = ok_out ? ok_out
                      : static_cast<uint8_t *>(
                            ctx->scratch_ptr(std::string("screen.ok") + tag, (size_t)nb));
  int32_t *nvalid = static_cast<int32_t *>(ctx->scratch_ptr(
      std::string("screen.nvalid") + tag, sizeof(int32_t) * (size_t)nb));
  int32_t *fails = static_cast<int32_t *>(
      ctx->scratch_ptr(std::string("screen.fails") + tag, sizeof(int32_t)));
  fill_i32(ctx, fails, 1, 0);
  CheckArgs ca;
  ca.best = cand;
  ca.nq = nb;
  ca.k = k;
  ca.kc = kc;
  ca.d = db->d;
  ca.metric = metric;
  ca.qnh = qn;
  ca.qnr = qn + nb;
  ca.xh = db->split_max_hi;
  ca.xr = db->split_max_res;
  if (metric == VSK_METRIC_COSINE) {
    // relative maxima and the queries' fp32 norms (those the screen divided by)
    ca.xh = db->cos_rel_hi;
    ca.xr = db->cos_rel_res;
    float *qnorm = static_cast<float *>(ctx->scratch_ptr(
        std::string("screen.qn") + tag, sizeof(float) * (size_t)nb));
    row_norms(ctx, qbat, nb, db->d, db->ld, nullptr, qnorm);
    ca.qn = qnorm;
  }
  ca.ok = ok;
  ca.nvalid = nvalid;
  ca.fails = fails;
  ca.test = true;
  {
    KernelTimer t(ctx, "screen_check");
    k_screen_check<<<grid_for(nb), 256, 0, ctx->stream>>>(ca);
    check_launch("screen_check");
  }
  rescore_select(ctx, db, qbat, nb, k, kc, metric, cand, nvalid, best);

  if (fail_host) {
    VSK_HIP(hipMemcpyAsync(fail_host, fails, sizeof(int32_t), hipMemcpyDeviceToHost,
                           ctx->stream));
    return {};
  }
  int32_t nfail = 0;
  VSK_HIP(hipMemcpyAsync(&nfail, fails, sizeof(int32_t), hipMemcpyDeviceToHost,
                         ctx->stream));
  stream_sync(ctx);
  std::vector<int32_t> idx;
  if (nfail == 0) return idx;
  std::vector<uint8_t> hok((size_t)nb);
  VSK_HIP(hipMemcpyAsync(hok.data(), ok, (size_t)nb, hipMemcpyDeviceToHost,
                         ctx->stream));
  stream_sync(ctx);
  for (int64_t i = 0; i < nb; ++i)
    if (!hok[(size_t)i]) idx.push_back((int32_t)i);
  return idx;
}

// queries idx of qbat, gathered; results scattered back into best (stride k).
// gidx[i] is the call-wide index of query i of qbat (recorded per tier).
static void redo_queries(vsk_ctx *ctx, const vsk_db *db, const float *qbat,
                         const std::vector<int32_t> &idx, int32_t k,
                         int32_t metric, uint64_t *best, bool exact_scan,
                         const std::vector<int64_t> &gidx) {
  const int64_t m = (int64_t)idx.size();
  std::vector<int64_t> sub((size_t)m);
  for (int64_t i = 0; i < m; ++i) sub[(size_t)i] = gidx[(size_t)idx[(size_t)i]];
  auto &rec = ctx->screen_redo[exact_scan ? 1 : 0];
  rec.insert(rec.end(), sub.begin(), sub.end());
  // profiled as one "launch" whose work counter is the number of queries
  KernelTimer tf(ctx, exact_scan ? "screen_fallback" : "screen_retry", (double)m);
  const char *tag = exact_scan ? ".x" : ".r";
  int32_t *didx = static_cast<int32_t *>(ctx->scratch_ptr(
      std::string("screen.fidx") + tag, sizeof(int32_t) * (size_t)m));
  VSK_HIP(hipMemcpyAsync(didx, idx.data(), sizeof(int32_t) * (size_t)m,
                         hipMemcpyHostToDevice, ctx->stream));
  float *q2 = static_cast<float *>(ctx->scratch_ptr(
      std::string("screen.fq") + tag, sizeof(float) * (size_t)m * db->ld));
  k_gather_rows<<<grid_for(m * db->ld), 256, 0, ctx->stream>>>(qbat, db->ld, didx,
                                                               m, q2);
  check_launch("screen_gather");
  uint64_t *best2 = static_cast<uint64_t *>(ctx->scratch_ptr(
      std::string("screen.fbest") + tag, sizeof(uint64_t) * (size_t)m * k));
  if (exact_scan) {
    // the reference's formula over every row: no cancellation, no bound
    approx_topk(ctx, db, q2, m, k, exact_metric(metric), best2, 3);
  } else {
    // a wider screen (the candidate count within the margin is some 2-3 k
    // on real data); queries failing it too take the exact scan
    std::vector<int32_t> again =
        screen_tier(ctx, db, q2, m, k, VSK_MAX_K, metric, best2, ".r");
    if (!again.empty())
      redo_queries(ctx, db, q2, again, k, metric, best2, true, sub);
  }
  k_scatter_keys<<<grid_for(m * k), 256, 0, ctx->stream>>>(best2, m, k, didx, best);
  check_launch("screen_scatter");
}

// ---------------------------------------------------------------------------
// exact argmin through the screen (k-means and IVF assignment)
// ---------------------------------------------------------------------------
// The bound of the file comment with k = 1: the screen's smallest
// distance a1 (row w) and second smallest a2 over all rows; if
// a2 > (a1 + eps)(1 + 2^-20) + eps, every other row y has
// d(y) >= a(y) - eps >= a2 - eps > (a1 + eps)(1 + 2^-20) >= d(w)(1 + 2^-20),
// so w is the unique exact minimum even after the square roots are rounded.
// One thread per query merges the row splits' pairs, tests the bound and
// recomputes the winner's exact distance in dimension order (no FMA);
// queries failing the test are listed for the exact VALU scan.
// One wave per 64 queries.  Each lane merges its query's split pairs and
// tests the bound; then, per 64-dim block, the wave gathers the 64 query
// rows and the 64 winners' rows in 256-byte segments (16 lanes per row) into
// LDS and every lane continues its own sequential sum from there (no FMA),
// so the winners' exact distances come from coalesced reads.
__global__ __launch_bounds__(64) void k_argmin_finish(
    const uint64_t *k1, const float *a2, int32_t nsplit, int64_t nq, const float *qnh,
    const float *qnr, const uint32_t *maxbits, int32_t d, const float *X, int64_t ld,
    const float *Q, int32_t *argmin, float *dist, int64_t qoff, int32_t *fail_idx,
    uint64_t *fail_thr, int32_t *nfail) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float tq[64 * RS_LD];
  __shared__ __attribute__((aligned(16))) float tx[64 * RS_LD];
  const int lane = threadIdx.x;
  const int64_t qb = (int64_t)blockIdx.x * 64;
  const int64_t q = qb + lane;
  const bool live = q < nq;
  uint64_t k = VSK_KEY_NONE;
  float m2 = __int_as_float(0x7f800000);
  if (live) {
    for (int32_t sp = 0; sp < nsplit; ++sp) {
      const uint64_t ko = k1[q * nsplit + sp];
      const float mo = a2[q * nsplit + sp];
      const uint64_t hi = ko < k ? k : ko;
      k = ko < k ? ko : k;
      const float hd = hi == VSK_KEY_NONE ? __int_as_float(0x7f800000)
                                          : vsk_ord2f((uint32_t)(hi >> 32));
      m2 = fminf(fminf(m2, mo), hd);
    }
  }
  bool good = live && k != VSK_KEY_NONE;
  double lim = 0.0;
  if (good) {
    CheckArgs ca{};
    ca.d = d;
    ca.metric = VSK_METRIC_L2SQ;
    ca.qnh = qnh;
    ca.qnr = qnr;
    ca.xh = (double)__uint_as_float(maxbits[0]);
    ca.xr = (double)__uint_as_float(maxbits[1]);
    // plus the screen's packing of positions into the distances' low bits
    const double qn = (double)qnh[q] + qnr[q], xn = ca.xh + ca.xr;
    const double eps = screen_eps(ca, q) + 0x1p-16 * (qn + xn) * (qn + xn);
    const double a1 = vsk_ord2f((uint32_t)(k >> 32));
    lim = (a1 + eps) * (1.0 + 0x1p-20) + eps;
    good = (double)m2 > lim;
  }
  if (live && !good) {
    // the rows that can still win have screened distance <= lim: the
    // threshold of the collecting pass (+inf when nothing was screened)
    float f = (float)lim;
    if ((double)f < lim) f = __uint_as_float(__float_as_uint(f) + 1u);
    const int32_t pos = atomicAdd(nfail, 1);
    fail_idx[pos] = (int32_t)(qoff + q);
    fail_thr[pos] = k == VSK_KEY_NONE ? VSK_KEY_NONE : vsk_key(f, 0xFFFFFFFFu);
  }
  if (!__builtin_amdgcn_ballot_w64(good)) return;
  // the exact distance of each decided query's winner
  const uint32_t row = good ? (uint32_t)k : 0u;
  const int64_t myq = live ? q : qb;  // lanes past nq gather the block's first query
  const int seg = lane & 15, sub = lane >> 4;
  const float *qsrc[16], *xsrc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    qsrc[i] = Q + (int64_t)__shfl((int)myq - (int)qb, sub + 4 * i) * ld + qb * ld;
    xsrc[i] = X + (int64_t)__shfl(row, sub + 4 * i) * ld;
  }
  const int32_t cmax = (int32_t)ld - 4;  // a segment past the row end is clamped
  float s = 0.f;
  for (int32_t j0 = 0; j0 < d; j0 += RS_W) {
    const int32_t col = j0 + 4 * seg < cmax ? j0 + 4 * seg : cmax;
    rs_f4 bq[16], bx[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      bq[i] = *reinterpret_cast<const rs_f4 *>(qsrc[i] + col);
      bx[i] = *reinterpret_cast<const rs_f4 *>(xsrc[i] + col);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      *reinterpret_cast<rs_f4 *>(tq + (sub + 4 * i) * RS_LD + 4 * seg) = bq[i];
      *reinterpret_cast<rs_f4 *>(tx + (sub + 4 * i) * RS_LD + 4 * seg) = bx[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int32_t jn = d - j0 < RS_W ? d - j0 : RS_W;
    const float *qr = tq + lane * RS_LD, *xr = tx + lane * RS_LD;
    for (int32_t j = 0; j < jn; ++j) {
      const float t = qr[j] - xr[j];
      s = s + t * t;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  if (good) {
    argmin[q] = (int32_t)row;
    dist[q] = sqrtf(s);
  }
}

// gathers the undecided queries: their fp32 rows, hi-plane rows and |q|^2
__global__ void k_gather_argmin_queries(const float *Q, int64_t ld, const uint16_t *qh,
                                        int32_t ldb, const float *qsq, const int32_t *idx,
                                        int64_t m, float *Q2, uint16_t *qh2, float *qsq2) {
  const int64_t i = blockIdx.x;
  if (i >= m) return;
  const int64_t src = idx[i];
  for (int64_t c = threadIdx.x; c < ld; c += blockDim.x) Q2[i * ld + c] = Q[src * ld + c];
  for (int64_t c = threadIdx.x; c < ldb; c += blockDim.x) qh2[i * ldb + c] = qh[src * ldb + c];
  if (threadIdx.x == 0) qsq2[i] = qsq[src];
}

// The collected candidates of each undecided query: one wave per query, a
// lane per slot; lanes holding a candidate compute its exact distance in
// dimension order (no FMA) and the wave keeps the smallest (distance, row).
// A query whose candidates overflowed (count > cap) or that had none is
// listed for the exact scan.  cap <= 64.
__global__ __launch_bounds__(64) void k_argmin_collect(
    const uint64_t *cand, int32_t cap, const int32_t *counts, int64_t m, const float *X,
    int64_t ld, const float *Q, int32_t d, const int32_t *idx, int32_t *argmin, float *dist,
    int32_t *redo, int32_t *nredo) {
#pragma clang fp contract(off)
  const int64_t i = blockIdx.x;
  const int lane = threadIdx.x;
  if (i >= m) return;
  const uint64_t key = lane < cap ? cand[i * cap + lane] : VSK_KEY_NONE;
  uint64_t best = VSK_KEY_NONE;
  if (key != VSK_KEY_NONE) {
    const uint32_t row = (uint32_t)key;
    const float *qq = Q + i * ld, *xx = X + (int64_t)row * ld;
    float s = 0.f;
    for (int32_t j = 0; j < d; ++j) {
      const float t = qq[j] - xx[j];
      s = s + t * t;
    }
    best = vsk_key(sqrtf(s), row);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)best, o), hi = __shfl_xor((uint32_t)(best >> 32), o);
    const uint64_t v = ((uint64_t)hi << 32) | lo;
    best = v < best ? v : best;
  }
  if (lane != 0) return;
  if (counts[i] > cap || best == VSK_KEY_NONE) {
    redo[atomicAdd(nredo, 1)] = (int32_t)i;
    return;
  }
  argmin[idx[i]] = (int32_t)(uint32_t)best;
  dist[idx[i]] = vsk_ord2f((uint32_t)(best >> 32));
}

// out[i] = map[idx[i]]
__global__ void k_map_index(const int32_t *idx, const int32_t *map, int64_t m, int32_t *out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < m;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = map[idx[i]];
}

__global__ void k_scatter_argmin(const int32_t *src_a, const float *src_d, int64_t m,
                                 const int32_t *idx, int32_t *argmin, float *dist) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < m;
       i += (int64_t)gridDim.x * blockDim.x) {
    argmin[idx[i]] = src_a[i];
    dist[idx[i]] = src_d[i];
  }
}

ArgminQueries argmin_queries(vsk_ctx *ctx, const float *dq, int64_t nq, int32_t d,
                             int32_t ld, const char *slot) {
  ArgminQueries qp;
  qp.ldb = (d + 63) & ~63;
  const std::string sl(slot);
  uint16_t *qh = static_cast<uint16_t *>(
      ctx->scratch_ptr(sl + ".qh", sizeof(uint16_t) * (size_t)nq * qp.ldb));
  float *nrm = static_cast<float *>(ctx->scratch_ptr(sl + ".qn", sizeof(float) * 3 * (size_t)nq));
  split_bf16(ctx, dq, nq, d, ld, qh, nullptr, qp.ldb, nrm, nrm + nq, nullptr);
  row_norms(ctx, dq, nq, d, ld, nrm + 2 * nq, nullptr);
  qp.qh = qh;
  qp.qnh = nrm;
  qp.qnr = nrm + nq;
  qp.qsq = nrm + 2 * nq;
  return qp;
}

bool screen_argmin_applies(vsk_ctx *ctx, int64_t nq, int64_t n, int32_t d) {
  if (ctx->flat_no_screen || ctx->flat_fp32 || ctx->exact_only) return false;
  if (n >= 0x7FFFFFFFll || d < 32) return false;  // narrow rows: the padding to 64 dims costs
  // small problems take the exact scan alone (the screen's fixed launches)
  return ctx->flat_force_screen || (double)nq * (double)n * d >= (double)(1ll << 30);
}

void screen_argmin(vsk_ctx *ctx, const float *X, const float *xsq, int64_t n,
                   int32_t d, int32_t ld, const float *dq, int64_t nq,
                   const ArgminQueries &qp, int32_t *argmin, float *dist) {
  KernelTimer tm(ctx, "screen_argmin", (double)nq * (double)n);
  const int32_t ldb = qp.ldb;
  // the rows' hi plane and the maxima of |hi| and |x - hi| over them
  uint16_t *xh = static_cast<uint16_t *>(
      ctx->scratch_ptr("sam.xh", sizeof(uint16_t) * (size_t)n * ldb));
  uint32_t *maxbits = static_cast<uint32_t *>(ctx->scratch_ptr("sam.max", 2 * sizeof(uint32_t)));
  fill_i32(ctx, reinterpret_cast<int32_t *>(maxbits), 2, 0);
  split_bf16(ctx, X, n, d, ld, xh, nullptr, ldb, nullptr, nullptr, maxbits);
  SplitPtrs sp;
  sp.xh = xh;
  sp.xl = nullptr;
  sp.qh = qp.qh;
  sp.ql = nullptr;
  sp.ldxb = ldb;
  sp.ldqb = ldb;
  sp.kb = ldb;
  const int64_t qb_max = (int64_t)1 << 22;  // queries per launch
  const int64_t qcap = nq < qb_max ? nq : qb_max;
  // the most row splits launch_flat_screen picks for this shape (a multiple
  // of 8, at most 8 rounds of workgroups and one tile per split)
  // (fewer queries allow more splits: the bound is taken at the last,
  // smallest batch)
  const int64_t nlast = nq - ((nq - 1) / qb_max) * qb_max;
  const int64_t tiles = ceil_div(n, 256);
  int64_t top = 8 * ceil_div(8 * (int64_t)ctx->cu_count, 8 * ceil_div(nlast, 256));
  if (top > 8 * ceil_div(tiles, 8)) top = 8 * ceil_div(tiles, 8);
  if (top < 8) top = 8;
  uint64_t *k1 = static_cast<uint64_t *>(
      ctx->scratch_ptr("sam.k1", sizeof(uint64_t) * (size_t)qcap * top));
  float *a2 = static_cast<float *>(
      ctx->scratch_ptr("sam.a2", sizeof(float) * (size_t)qcap * top));
  int32_t *fidx = static_cast<int32_t *>(
      ctx->scratch_ptr("sam.fidx", sizeof(int32_t) * (size_t)(nq + 1)));
  int32_t *nfail = fidx + nq;
  uint64_t *fthr = static_cast<uint64_t *>(
      ctx->scratch_ptr("sam.fthr", sizeof(uint64_t) * (size_t)nq));
  fill_i32(ctx, nfail, 1, 0);
  for (int64_t b0 = 0; b0 < nq; b0 += qb_max) {
    const int64_t nb = nq - b0 < qb_max ? nq - b0 : qb_max;
    FlatArgs a{};
    a.X = X;
    a.ldx = ld;
    a.Q = dq + b0 * ld;
    a.ldq = ld;
    a.xaux = xsq;
    a.qaux = qp.qsq + b0;
    a.kdim = ld;
    a.nq = (int32_t)nb;
    a.r0 = 0;
    a.r1 = n;
    a.metric = VSK_METRIC_L2SQ;
    a.cand = k1;
    a.mat = a2;
    SplitPtrs sb = sp;
    sb.qh = qp.qh + b0 * ldb;
    // splits without rows write nothing: their pairs must read as empty
    fill_u64(ctx, k1, nb * top, VSK_KEY_NONE);
    fill_i32(ctx, reinterpret_cast<int32_t *>(a2), nb * top, 0x7f800000);
    int32_t nsplit = 0;
    launch_flat_screen(ctx, a, sb, MODE_TOP2, &nsplit, nullptr);
    if (nsplit < 1 || nsplit > top)
      fail(VSK_ERR_EXECUTION_FAILED, "argmin screen: unexpected split count");
    k_argmin_finish<<<(unsigned)ceil_div(nb, 64), 64, 0, ctx->stream>>>(
        k1, a2, nsplit, nb, qp.qnh + b0, qp.qnr + b0, maxbits, d, X, ld, dq + b0 * ld,
        argmin + b0, dist + b0, b0, fidx, fthr, nfail);
    check_launch("screen_argmin_finish");
  }
  int32_t hf = 0;
  VSK_HIP(hipMemcpyAsync(&hf, nfail, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
  stream_sync(ctx);
  if (hf == 0) return;
  // Undecided queries (near ties).  A second screen pass over them keeps
  // every row whose screened distance is within their limit (at most
  // kCollect per query, kCollect / 8 per row split), those rows' exact
  // distances are computed in dimension order and the smallest key wins.  A query with more candidates than that is redone by the exact
  // VALU scan over every row.
  constexpr int32_t kCollect = 64;
  const int64_t m = hf;
  KernelTimer tf(ctx, "screen_argmin_collect", (double)m);
  float *q2 = static_cast<float *>(ctx->scratch_ptr("sam.fq", sizeof(float) * (size_t)m * ld));
  uint16_t *qh2 = static_cast<uint16_t *>(
      ctx->scratch_ptr("sam.fqh", sizeof(uint16_t) * (size_t)m * ldb));
  float *qsq2 = static_cast<float *>(ctx->scratch_ptr("sam.fqsq", sizeof(float) * (size_t)m));
  k_gather_argmin_queries<<<(unsigned)m, 128, 0, ctx->stream>>>(dq, ld, qp.qh, ldb, qp.qsq,
                                                                 fidx, m, q2, qh2, qsq2);
  check_launch("screen_argmin_gather");
  uint64_t *cand = static_cast<uint64_t *>(
      ctx->scratch_ptr("sam.cand", sizeof(uint64_t) * (size_t)m * kCollect));
  int32_t *cnt = static_cast<int32_t *>(
      ctx->scratch_ptr("sam.ccnt", sizeof(int32_t) * (size_t)m));
  int32_t *redo = static_cast<int32_t *>(
      ctx->scratch_ptr("sam.redo", sizeof(int32_t) * ((size_t)m + 1)));
  int32_t *nredo = redo + m;
  // slots no workgroup reserves are never written: they must read as empty
  fill_u64(ctx, cand, m * kCollect, VSK_KEY_NONE);
  fill_i32(ctx, cnt, m, 0);
  fill_i32(ctx, nredo, 1, 0);
  for (int64_t r0 = 0; r0 < m; r0 += qb_max) {
    const int64_t mb = m - r0 < qb_max ? m - r0 : qb_max;
    FlatArgs a{};
    a.X = X;
    a.ldx = ld;
    a.Q = q2 + r0 * ld;
    a.ldq = ld;
    a.xaux = xsq;
    a.qaux = qsq2 + r0;
    a.kdim = ld;
    a.nq = (int32_t)mb;
    a.r0 = 0;
    a.r1 = n;
    a.metric = VSK_METRIC_L2SQ;
    a.thresh = fthr + r0;
    a.cand = cand + r0 * kCollect;
    a.cap = kCollect;
    a.counts = cnt + r0;
    SplitPtrs sb = sp;
    sb.qh = qh2 + r0 * ldb;
    launch_flat_screen(ctx, a, sb, MODE_FILTER, nullptr, nullptr);
  }
  k_argmin_collect<<<(unsigned)m, 64, 0, ctx->stream>>>(cand, kCollect, cnt, m, X, ld, q2, d,
                                                        fidx, argmin, dist, redo, nredo);
  check_launch("screen_argmin_collect");
  int32_t hr = 0;
  VSK_HIP(hipMemcpyAsync(&hr, nredo, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
  stream_sync(ctx);
  if (hr == 0) return;
  // overflowing candidate lists: the exact VALU argmin over every row
  KernelTimer tv(ctx, "screen_argmin_fallback", (double)hr);
  const int64_t mr = hr;
  float *q3 = static_cast<float *>(ctx->scratch_ptr("sam.rq", sizeof(float) * (size_t)mr * ld));
  k_gather_rows<<<grid_for(mr * ld), 256, 0, ctx->stream>>>(q2, ld, redo, mr, q3);
  check_launch("screen_argmin_gather");
  int32_t *ridx = static_cast<int32_t *>(
      ctx->scratch_ptr("sam.ridx", sizeof(int32_t) * (size_t)mr));
  k_map_index<<<grid_for(mr), 256, 0, ctx->stream>>>(redo, fidx, mr, ridx);
  check_launch("screen_argmin_map");
  int32_t *a_out = static_cast<int32_t *>(
      ctx->scratch_ptr("sam.fa", (sizeof(int32_t) + sizeof(float)) * (size_t)mr));
  float *d_out = reinterpret_cast<float *>(a_out + mr);
  const int64_t chunk = 1 << 24;
  for (int64_t r = 0; r < mr; r += chunk) {
    const int64_t mm = mr - r < chunk ? mr - r : chunk;
    FlatArgs a{};
    a.X = X;
    a.ldx = ld;
    a.Q = q3 + r * ld;
    a.ldq = ld;
    a.kdim = ld;
    a.nq = (int32_t)mm;
    a.r0 = 0;
    a.r1 = n;
    a.metric = METRIC_L2_EXACT;
    a.amin = d_out + r;
    launch_flat(ctx, a, MODE_ARGMIN, a_out + r);
  }
  k_scatter_argmin<<<grid_for(mr), 256, 0, ctx->stream>>>(a_out, d_out, mr, ridx, argmin,
                                                          dist);
  check_launch("screen_argmin_scatter");
}

void screen_topk(vsk_ctx *ctx, const vsk_db *db, const float *dq, int64_t nq,
                 int32_t k, int32_t metric, uint64_t *best, ScreenDeferred *defer) {
  const int32_t kc = screen_keep(k);
  const int64_t qb = query_batch(ctx, nq, screen_cap(kc));
  if (defer) {
    // every batch enqueued; the failing counts come back with the call's
    // synchronisation (pinned slots taken before any work is queued)
    const int64_t nbat = ceil_div(nq, qb);
    defer->fails_host = static_cast<int32_t *>(ctx->pinned_ptr(sizeof(int32_t) * nbat));
    defer->ok = static_cast<uint8_t *>(ctx->scratch_ptr("screen.okall", (size_t)nq));
    defer->batches.clear();
    defer->active = true;
    defer->kc = kc;
    for (int64_t b0 = 0, i = 0; b0 < nq; b0 += qb, ++i) {
      const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
      screen_tier(ctx, db, dq + b0 * db->ld, nb, k, kc, metric, best + b0 * k, "",
                  defer->ok + b0, defer->fails_host + i);
      defer->batches.push_back({b0, nb});
    }
    return;
  }
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    const float *qbat = dq + b0 * db->ld;
    std::vector<int32_t> fail =
        screen_tier(ctx, db, qbat, nb, k, kc, metric, best + b0 * k, "");
    if (fail.empty()) continue;
    std::vector<int64_t> gidx((size_t)nb);
    for (int64_t i = 0; i < nb; ++i) gidx[(size_t)i] = b0 + i;
    redo_queries(ctx, db, qbat, fail, k, metric, best + b0 * k,
                 kc >= VSK_MAX_K, gidx);
  }
  for (auto &rec : ctx->screen_redo) std::sort(rec.begin(), rec.end());
}

bool screen_finish(vsk_ctx *ctx, const vsk_db *db, const float *dq, int32_t k,
                   int32_t metric, uint64_t *best, ScreenDeferred &defer) {
  bool any = false;
  if (!defer.active) return false;
  for (size_t i = 0; i < defer.batches.size(); ++i) {
    if (defer.fails_host[i] <= 0) continue;
    const int64_t b0 = defer.batches[i].b0, nb = defer.batches[i].nb;
    std::vector<uint8_t> hok((size_t)nb);
    VSK_HIP(hipMemcpyAsync(hok.data(), defer.ok + b0, (size_t)nb, hipMemcpyDeviceToHost,
                           ctx->stream));
    stream_sync(ctx);
    std::vector<int32_t> idx;
    for (int64_t j = 0; j < nb; ++j)
      if (!hok[(size_t)j]) idx.push_back((int32_t)j);
    if (idx.empty()) continue;
    std::vector<int64_t> gidx((size_t)nb);
    for (int64_t j = 0; j < nb; ++j) gidx[(size_t)j] = b0 + j;
    redo_queries(ctx, db, dq + b0 * db->ld, idx, k, metric, best + b0 * k,
                 defer.kc >= VSK_MAX_K, gidx);
    any = true;
  }
  defer.active = false;
  for (auto &rec : ctx->screen_redo) std::sort(rec.begin(), rec.end());
  return any;
}

}  // namespace vsk
