// hnsw.hip -- batched neighbour-distance evaluation for HNSW graph walks.
//
// Reference: HNSWIndex's greedySearchLayer / searchLayer0
// (Indexes/HNSWIndex.swift:1035-1221) visit a node, then score each unvisited
// neighbour with DistanceComputer.distance (:1920-1959), one call at a time:
//   euclidean  sqrt((v1 - v2) * (v1 - v2)).sum()
//   cosine     1 - dot / (|v1| |v2|), dot = (v1 * v2).sum(), |v| =
//              sqrt((v * v).sum()) -- no epsilon
//   manhattan  reduce(0) { sum + |v1_i - v2_i| }
// SIMD.sum() on floating point adds the lanes in index order starting from
// -0.0; reduce(0) starts from +0.0.  Every sum here is taken in that order
// with no FMA, so the distances are bit-identical to the reference's.
//
// Here many searches advance together: the caller hands over, for each query,
// the list of neighbour rows of its current frontier (CSR: offsets[nq + 1],
// rows[offsets[nq]]) and gets every distance back in one launch.  One lane per
// (query, row) pair; each wave gathers its 64 rows in 256-byte segments (16
// lanes per row) into LDS, 64 dimensions at a time, so the row reads stay
// coalesced although the rows are scattered, and every lane continues its own
// sequential sums from there.  The query element is read by all lanes of the
// query at one address (a broadcast from the cache).
#include <algorithm>

#include "vsk_api.hpp"

namespace vsk {

constexpr int HN_W = 64;          // dims per gathered block
constexpr int HN_LD = HN_W + 4;   // LDS row stride (floats): conflict-free
typedef float hn_f4 __attribute__((ext_vector_type(4)));

struct HnswArgs {
  const float *X;
  int64_t ldx, n;
  const float *Q;
  int64_t ldq, nq;
  int32_t d;
  const int64_t *offsets;  // nq + 1
  const int32_t *rows;     // offsets[nq]
  int64_t pairs;
  float *out;
  int32_t *bad;  // set to 1 when a row index is out of range
};

template <int METRIC>
__global__ __launch_bounds__(256) void k_hnsw_dist(HnswArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float tile[4][64 * HN_LD];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool live = p < a.pairs;
  if (!__builtin_amdgcn_ballot_w64(live)) return;  // wave past the last pair
  // the pair's query: the last q with offsets[q] <= p
  int64_t qi = 0;
  int32_t row = 0;
  bool valid = false;
  if (live) {
    int64_t lo = 0, hi = a.nq;  // invariant: offsets[lo] <= p < offsets[hi]
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if (a.offsets[mid] <= p) lo = mid;
      else hi = mid;
    }
    qi = lo;
    row = a.rows[p];
    valid = row >= 0 && (int64_t)row < a.n;
    if (!valid) atomicOr(a.bad, 1);
  }
  const float *qq = a.Q + qi * a.ldq;
  float *t = tile[w];
  const int seg = lane & 15, sub = lane >> 4;  // 16 lanes per row segment
  const int32_t my_row = valid ? row : 0;
  const float *src[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) src[i] = a.X + (int64_t)__shfl(my_row, sub + 4 * i) * a.ldx;
  const int32_t cmax = (int32_t)a.ldx - 4;  // a segment past the row end is clamped
  hn_f4 buf[16];
  {
    const int32_t col = 4 * seg < cmax ? 4 * seg : cmax;
#pragma unroll
    for (int i = 0; i < 16; ++i) buf[i] = *reinterpret_cast<const hn_f4 *>(src[i] + col);
  }
  // euclidean and cosine: SIMD.sum() from -0; manhattan: reduce(0) from +0
  float s = METRIC == VSK_METRIC_L1 ? 0.0f : -0.0f;
  float sqq = -0.0f, sxx = -0.0f;  // cosine: the two magnitudes' sums
  for (int32_t j0 = 0; j0 < a.d; j0 += HN_W) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      *reinterpret_cast<hn_f4 *>(t + (sub + 4 * i) * HN_LD + 4 * seg) = buf[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {
      const int32_t jnext = j0 + HN_W < a.d ? j0 + HN_W : j0;
      const int32_t col = jnext + 4 * seg < cmax ? jnext + 4 * seg : cmax;
#pragma unroll
      for (int i = 0; i < 16; ++i) buf[i] = *reinterpret_cast<const hn_f4 *>(src[i] + col);
    }
    const int32_t jn = a.d - j0 < HN_W ? a.d - j0 : HN_W;
    const float *xr = t + lane * HN_LD;
    for (int32_t j = 0; j < jn; ++j) {
      const float qv = qq[j0 + j], xv = xr[j];
      if constexpr (METRIC == VSK_METRIC_L1) {
        s = s + fabsf(qv - xv);
      } else if constexpr (METRIC == VSK_METRIC_COSINE_NOEPS) {
        s = s + qv * xv;
        sqq = sqq + qv * qv;
        sxx = sxx + xv * xv;
      } else {
        const float tt = qv - xv;
        s = s + tt * tt;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  if (!live) return;
  float dist;
  if (!valid) {
    dist = __int_as_float(0x7fc00000);
  } else if constexpr (METRIC == VSK_METRIC_L2) {
    dist = sqrtf(s);
  } else if constexpr (METRIC == VSK_METRIC_COSINE_NOEPS) {
    const float m1 = sqrtf(sqq), m2 = sqrtf(sxx);
    const float den = m1 * m2;
    dist = 1.0f - s / den;
  } else {
    dist = s;  // L2SQ, L1
  }
  a.out[p] = dist;
}

}  // namespace vsk

using namespace vsk;

extern "C" {

vsk_status vsk_hnsw_distances(vsk_ctx *ctx, const vsk_db *db, const float *q, int64_t nq,
                              const int64_t *offsets, const int32_t *rows, int32_t metric,
                              float *out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(db, VSK_ERR_INVALID_ARGUMENT, "db is null");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(q && offsets, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(metric == VSK_METRIC_L2 || metric == VSK_METRIC_L2SQ || metric == VSK_METRIC_L1 ||
                  metric == VSK_METRIC_COSINE_NOEPS,
              VSK_ERR_UNSUPPORTED,
              "HNSW distances: euclidean, squared euclidean, manhattan or cosine without "
              "epsilon");
  // the offsets decide the launch: read them on the host (nq + 1 values)
  std::vector<int64_t> hoff((size_t)nq + 1);
  if (is_device_ptr(offsets)) {
    VSK_HIP(hipMemcpyAsync(hoff.data(), offsets, sizeof(int64_t) * hoff.size(),
                           hipMemcpyDeviceToHost, ctx->stream));
    stream_sync(ctx);
  } else {
    std::copy(offsets, offsets + nq + 1, hoff.begin());
  }
  VSK_REQUIRE(hoff[0] == 0, VSK_ERR_INVALID_ARGUMENT, "offsets[0] must be 0");
  for (int64_t i = 0; i < nq; ++i)
    VSK_REQUIRE(hoff[(size_t)i + 1] >= hoff[(size_t)i], VSK_ERR_INVALID_ARGUMENT,
                "offsets must be non-decreasing");
  const int64_t pairs = hoff[(size_t)nq];
  if (pairs == 0) return VSK_OK;
  VSK_REQUIRE(rows && out, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(pairs <= 0x7FFFFFFFll * 128, VSK_ERR_INVALID_BUFFER_SIZE, "too many pairs");
  CallScope cs(ctx);
  const float *dq = rows_to_device_padded(ctx, q, nq, db->d, db->ld, "hnsw.q");
  const int64_t *doff = static_cast<const int64_t *>(
      input_to_device(ctx, hoff.data(), sizeof(int64_t) * hoff.size(), "hnsw.off"));
  const int32_t *drows = static_cast<const int32_t *>(
      input_to_device(ctx, rows, sizeof(int32_t) * (size_t)pairs, "hnsw.rows"));
  OutputStage od(ctx, out, sizeof(float) * (size_t)pairs, "hnsw.out");
  int32_t *bad = static_cast<int32_t *>(ctx->scratch_ptr("hnsw.bad", sizeof(int32_t)));
  fill_i32(ctx, bad, 1, 0);
  HnswArgs a{};
  a.X = db->x.as<float>();
  a.ldx = db->ld;
  a.n = db->n;
  a.Q = dq;
  a.ldq = db->ld;
  a.nq = nq;
  a.d = db->d;
  a.offsets = doff;
  a.rows = drows;
  a.pairs = pairs;
  a.out = od.ptr<float>();
  a.bad = bad;
  const unsigned grid = (unsigned)ceil_div(pairs, 256);
  {
    KernelTimer t(ctx, "hnsw_distances", (double)pairs);
    switch (metric) {
    case VSK_METRIC_L2:
      k_hnsw_dist<VSK_METRIC_L2><<<grid, 256, 0, ctx->stream>>>(a);
      break;
    case VSK_METRIC_L2SQ:
      k_hnsw_dist<VSK_METRIC_L2SQ><<<grid, 256, 0, ctx->stream>>>(a);
      break;
    case VSK_METRIC_L1:
      k_hnsw_dist<VSK_METRIC_L1><<<grid, 256, 0, ctx->stream>>>(a);
      break;
    default:
      k_hnsw_dist<VSK_METRIC_COSINE_NOEPS><<<grid, 256, 0, ctx->stream>>>(a);
    }
    check_launch("hnsw_distances");
  }
  od.copy_back();
  int32_t hbad = 0;
  VSK_HIP(hipMemcpyAsync(&hbad, bad, sizeof(int32_t), hipMemcpyDeviceToHost, ctx->stream));
  cs.finish();
  VSK_REQUIRE(hbad == 0, VSK_ERR_INVALID_ARGUMENT, "a row index is outside the database");
  VSK_API_END(ctx);
}

}  // extern "C"
