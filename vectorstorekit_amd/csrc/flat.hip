// flat.hip -- flat (brute-force) k-NN: query x row distances on fp32 MFMA
// (L2^2 / L2 / cosine / normalised cosine / dot) or on the VALU (Manhattan),
// fused with the filter/append stage of the progressive top-k, so no
// query x row distance matrix is written to HBM.
//
// Reference: the batched distance kernels batchEuclideanDistance /
// batchCosineDistance / batchManhattanDistance / batchDotProduct
// (Acceleration/Metal/Shaders/DistanceShaders.metal:248-379, one thread per
// (query, row) pair) and their host side
// MetalAccelerationEngine.batchComputeDistancesGPU
// (Acceleration/MetalAccelerationEngine.swift:377-478), which reads back the
// full matrix and sorts each row on the CPU.
//
// MFMA kernel: a workgroup owns 64 queries and a contiguous slice of rows,
// walks the slice in tiles of 128 rows; each of its 4 waves computes a
// 32-row x 64-query block as 2x4 v_mfma_f32_16x16x4f32 tiles, with both
// operands staged through LDS in 32-dim stages.  Distances follow from the
// dot product and precomputed norms:
//   L2^2 = |q|^2 + |x|^2 - 2 q.x       cosine = 1 - q.x / (|q||x| + 1e-8)
//   normalised cosine = 1 - q.x        dot = -q.x
#include <cstring>

#include "flat.hpp"

namespace vsk {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int FB_N = 128;  // rows per tile
constexpr int FB_Q = 64;   // queries per workgroup
constexpr int FB_K = 32;   // dims per LDS stage
constexpr int FS = FB_K + 2;  // LDS row stride (floats): conflict-free MFMA reads

// the metric is a template parameter: the epilogue has no runtime switch
template <int METRIC>
__device__ inline float metric_from_dot(float dot, float qa, float xa) {
  if constexpr (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2)
    return fmaxf(qa + xa - 2.0f * dot, 0.0f);
  else if constexpr (METRIC == VSK_METRIC_COSINE)
    return 1.0f - dot / (qa * xa + 1e-8f);
  else if constexpr (METRIC == VSK_METRIC_COSINE_NORMALIZED)
    return 1.0f - dot;
  else
    return -dot;
}

// one (query, row, distance) result of a tile
template <int MODE, int METRIC>
__device__ inline void emit(const FlatArgs &a, int64_t qi, int64_t row,
                            float dist, uint64_t th) {
  if constexpr (MODE == MODE_MATRIX) {
    a.mat[qi * a.ldm + row] = METRIC == VSK_METRIC_L2 ? sqrtf(dist) : dist;
  } else {
    uint64_t key = vsk_key(dist, (uint32_t)row);
    if constexpr (MODE == MODE_DENSE) {
      a.cand[qi * a.cap + (row - a.r0)] = key;
    } else if (key <= th) {
      int slot = atomicAdd(&a.counts[qi], 1);
      if (slot < a.cap) a.cand[qi * a.cap + slot] = key;
    }
  }
}

template <int MODE, int METRIC>
__global__ __launch_bounds__(256) void k_flat_mfma(FlatArgs a) {
  __shared__ float xs[FB_N * FS];
  __shared__ float qs[FB_Q * FS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t q0 = (int64_t)blockIdx.x * FB_Q;
  const int64_t s0 = a.r0 + (int64_t)blockIdx.y * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;

  // the 4 queries this lane's accumulators belong to
  int64_t qi[4];
  bool qok[4];
  uint64_t th[4];
  float qa[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    qi[j] = q0 + j * 16 + (lane & 15);
    qok[j] = qi[j] < a.nq && (!a.active || a.active[qi[j]]);
    th[j] = (MODE == MODE_FILTER && qok[j]) ? a.thresh[qi[j]] : 0;
    qa[j] = (a.qaux && qi[j] < a.nq) ? a.qaux[qi[j]] : 0.f;
  }
  // global->LDS copy assignment: 8 threads per 32-float row segment
  const int crow = tid >> 3, ccol = (tid & 7) * 4;

  for (int64_t t0 = s0; t0 < s1; t0 += FB_N) {
    f4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    f4 xr[4], qr[2];
    auto gload = [&](int k0) {
      const bool kin = k0 + ccol < a.kdim;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        int64_t grow = t0 + u * 32 + crow;
        xr[u] = (kin && grow < s1)
                    ? *reinterpret_cast<const f4 *>(a.X + grow * a.ldx + k0 +
                                                    ccol)
                    : f4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        int64_t gq = q0 + u * 32 + crow;
        qr[u] = (kin && gq < a.nq)
                    ? *reinterpret_cast<const f4 *>(a.Q + gq * a.ldq + k0 +
                                                    ccol)
                    : f4{0.f, 0.f, 0.f, 0.f};
      }
    };
    gload(0);
    for (int k0 = 0; k0 < a.kdim; k0 += FB_K) {
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float *p = xs + (u * 32 + crow) * FS + ccol;
        p[0] = xr[u].x;
        p[1] = xr[u].y;
        p[2] = xr[u].z;
        p[3] = xr[u].w;
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float *p = qs + (u * 32 + crow) * FS + ccol;
        p[0] = qr[u].x;
        p[1] = qr[u].y;
        p[2] = qr[u].z;
        p[3] = qr[u].w;
      }
      __syncthreads();
      if (k0 + FB_K < a.kdim) gload(k0 + FB_K);
#pragma unroll
      for (int kk = 0; kk < FB_K; kk += 4) {
        float af[2], bf[4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          af[i] = xs[(w * 32 + i * 16 + (lane & 15)) * FS + kk + (lane >> 4)];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bf[j] = qs[(j * 16 + (lane & 15)) * FS + kk + (lane >> 4)];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j],
                                                             acc[i][j], 0, 0,
                                                             0);
      }
    }
    // epilogue: D[row = 4*(lane/16) + r][query = lane%16] of each tile
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = t0 + w * 32 + i * 16 + 4 * (lane >> 4) + r;
        if (row >= s1) continue;
        const float xa = a.xaux ? a.xaux[row] : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!qok[j]) continue;
          float dist = metric_from_dot<METRIC>(acc[i][j][r], qa[j], xa);
          emit<MODE, METRIC>(a, qi[j], row, dist, th[j]);
        }
      }
    }
  }
}

// Exact VALU distances, every term added in dimension order:
//  OP_L1    sum |q-x|   (the order of the reference's per-candidate vDSP
//           loop, Acceleration/AccelerateOptimizer.swift:322-360)
//  OP_L2SEQ sqrt(sum (q-x)^2) with separate multiply and add (no FMA), as
//           IVFIndex.computeDistance (Indexes/IVFIndex.swift:542-549)
// so the distances are bit-identical to a sequential fp32 loop.  Thread
// (tid) owns rows (tid%32)+32u, u<4, and queries (tid/32)+8v, v<8.
// MODE_ARGMIN keeps, per query, the smallest (distance, row) key over all
// rows, i.e. the first minimum under strict '<' (findNearestCentroid,
// Indexes/IVFIndex.swift:514-527), and writes the row index to argmin[q]
// (and its distance to a.amin[q] when a.amin is set).
constexpr int LS = FB_K + 1;  // odd stride: conflict-free column reads
// sequential (dimension-order, no FMA) terms and final transforms of the
// exact VALU kernel, one per metric of the CPU reference
//  OP_COSSEQ 1 - (sum q x)/(|q| |x| + 1e-8) with the norms the reference
//           computes (AccelerateOptimizer.swift:285-320, sums sequential)
enum { OP_L1 = 0, OP_L2SEQ = 1, OP_L2SQSEQ = 2, OP_CNSEQ = 3, OP_DOTSEQ = 4, OP_HAM = 5,
       OP_COSSEQ = 6 };

__device__ inline uint64_t shfl_xor_u64(uint64_t v, int m) {
  uint32_t lo = __shfl_xor((uint32_t)v, m);
  uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

template <int OP>
__device__ inline float valu_term(float q, float x) {
#pragma clang fp contract(off)
  if constexpr (OP == OP_L1) {
    return fabsf(q - x);
  } else if constexpr (OP == OP_HAM) {
    // hammingDistance: count += 1 where the components differ
    // (Core/Distance/UnifiedDistanceComputation.swift:249-261; NaN differs)
    return q != x ? 1.0f : 0.0f;
  } else if constexpr (OP == OP_L2SEQ || OP == OP_L2SQSEQ) {
    float t = q - x;
    return t * t;
  } else {
    return q * x;
  }
}

template <int OP>
__device__ inline float valu_final(float s) {
  if constexpr (OP == OP_L2SEQ) return sqrtf(s);
  else if constexpr (OP == OP_CNSEQ) return 1.0f - s;
  else if constexpr (OP == OP_DOTSEQ) return -s;
  else return s;
}

template <int MODE, int OP, int U, int V>
__global__ __launch_bounds__(256) void k_flat_valu(FlatArgs a, int32_t *argmin) {
#pragma clang fp contract(off)
  // a tile of 32 U rows x 8 V queries; thread (rsub, qsub) owns rows
  // rsub + 32 u and queries qsub + 8 v
  static_assert(V % 4 == 0, "queries are staged 32 at a time");
  __shared__ float xs[32 * U * LS];
  __shared__ float qs[8 * V * LS];
  const int tid = threadIdx.x;
  const int64_t q0 = (int64_t)blockIdx.x * (8 * V);
  const int64_t s0 = a.r0 + (int64_t)blockIdx.y * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;
  const int rsub = tid & 31, qsub = tid >> 5;
  int64_t qi[V];
  bool qok[V];
  uint64_t th[V];
  uint64_t best[V];
  float qn[V];  // OP_COSSEQ: the queries' norms
#pragma unroll
  for (int v = 0; v < V; ++v) {
    qi[v] = q0 + qsub + 8 * v;
    qok[v] = qi[v] < a.nq && (!a.active || a.active[qi[v]]);
    qn[v] = (OP == OP_COSSEQ && qi[v] < a.nq) ? a.qaux[qi[v]] : 0.f;
    th[v] = (MODE == MODE_FILTER && qok[v]) ? a.thresh[qi[v]] : 0;
    best[v] = VSK_KEY_NONE;
  }
  const int crow = tid >> 3, ccol = (tid & 7) * 4;
  for (int64_t t0 = s0; t0 < s1; t0 += 32 * U) {
    float acc[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < V; ++v) acc[u][v] = 0.f;
    for (int k0 = 0; k0 < a.kdim; k0 += FB_K) {
      const bool kin = k0 + ccol < a.kdim;
      __syncthreads();
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int64_t grow = t0 + u * 32 + crow;
        f4 v = (kin && grow < s1)
                   ? *reinterpret_cast<const f4 *>(a.X + grow * a.ldx + k0 +
                                                   ccol)
                   : f4{0.f, 0.f, 0.f, 0.f};
        float *p = xs + (u * 32 + crow) * LS + ccol;
        p[0] = v.x;
        p[1] = v.y;
        p[2] = v.z;
        p[3] = v.w;
      }
#pragma unroll
      for (int u = 0; u < V / 4; ++u) {
        int64_t gq = q0 + u * 32 + crow;
        f4 v = (kin && gq < a.nq)
                   ? *reinterpret_cast<const f4 *>(a.Q + gq * a.ldq + k0 +
                                                   ccol)
                   : f4{0.f, 0.f, 0.f, 0.f};
        float *p = qs + (u * 32 + crow) * LS + ccol;
        p[0] = v.x;
        p[1] = v.y;
        p[2] = v.z;
        p[3] = v.w;
      }
      __syncthreads();
      const int kend = a.kdim - k0 < FB_K ? a.kdim - k0 : FB_K;
      for (int kk = 0; kk < kend; ++kk) {
        float xv[U], qv[V];
#pragma unroll
        for (int u = 0; u < U; ++u) xv[u] = xs[(rsub + 32 * u) * LS + kk];
#pragma unroll
        for (int v = 0; v < V; ++v) qv[v] = qs[(qsub + 8 * v) * LS + kk];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int v = 0; v < V; ++v) acc[u][v] += valu_term<OP>(qv[v], xv[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = t0 + rsub + 32 * u;
      if (row >= s1) continue;
      const float xn = OP == OP_COSSEQ ? a.xaux[row] : 0.f;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (!qok[v]) continue;
        const float dist = OP == OP_COSSEQ ? 1.0f - acc[u][v] / (qn[v] * xn + 1e-8f)
                                           : valu_final<OP>(acc[u][v]);
        if constexpr (MODE == MODE_ARGMIN) {
          uint64_t key = vsk_key(dist, (uint32_t)row);
          best[v] = key < best[v] ? key : best[v];
        } else {
          // the keys/matrix carry the final distance already
          emit<MODE, VSK_METRIC_L1>(a, qi[v], row, dist, th[v]);
        }
      }
    }
  }
  if constexpr (MODE == MODE_ARGMIN) {
    // the 32 lanes with equal qsub hold disjoint rows of the same queries
#pragma unroll
    for (int v = 0; v < V; ++v) {
      uint64_t b = best[v];
#pragma unroll
      for (int m = 16; m > 0; m >>= 1) {
        uint64_t o = shfl_xor_u64(b, m);
        b = o < b ? o : b;
      }
      if (rsub == 0 && qok[v]) {
        argmin[qi[v]] = (int32_t)(uint32_t)b;
        if (a.amin) a.amin[qi[v]] = vsk_ord2f((uint32_t)(b >> 32));
      }
    }
  }
}

template <int METRIC>
static void launch_mfma(vsk_ctx *ctx, dim3 grid, const FlatArgs &a, int mode) {
  if (mode == MODE_DENSE)
    k_flat_mfma<MODE_DENSE, METRIC><<<grid, 256, 0, ctx->stream>>>(a);
  else if (mode == MODE_FILTER)
    k_flat_mfma<MODE_FILTER, METRIC><<<grid, 256, 0, ctx->stream>>>(a);
  else
    k_flat_mfma<MODE_MATRIX, METRIC><<<grid, 256, 0, ctx->stream>>>(a);
}

template <int OP, int U, int V>
static void launch_valu(vsk_ctx *ctx, dim3 grid, const FlatArgs &a, int mode,
                        int32_t *argmin) {
  if (mode == MODE_DENSE)
    k_flat_valu<MODE_DENSE, OP, U, V><<<grid, 256, 0, ctx->stream>>>(a, argmin);
  else if (mode == MODE_FILTER)
    k_flat_valu<MODE_FILTER, OP, U, V><<<grid, 256, 0, ctx->stream>>>(a, argmin);
  else if (mode == MODE_MATRIX)
    k_flat_valu<MODE_MATRIX, OP, U, V><<<grid, 256, 0, ctx->stream>>>(a, argmin);
  else
    k_flat_valu<MODE_ARGMIN, OP, U, V><<<grid, 256, 0, ctx->stream>>>(a, argmin);
}

// the exact VALU scan in tiles of 128 rows x 64 queries, or, when those
// leave fewer than 4 workgroups per CU, 64 rows x 32 queries (a quarter of
// the work per thread: small problems are latency-bound)
template <int OP>
static void launch_valu_sized(vsk_ctx *ctx, FlatArgs a, int mode, int32_t *argmin,
                              bool small) {
  const int64_t rows = a.r1 - a.r0;
  const int64_t tq = small ? 32 : FB_Q, tn = small ? 64 : FB_N;
  const int64_t qt = ceil_div(a.nq, tq);
  int64_t splits = mode == MODE_ARGMIN ? 1 : ceil_div(4096, qt);
  const int64_t max_splits = ceil_div(rows, tn);
  if (splits > max_splits) splits = max_splits;
  if (splits > 65535) splits = 65535;
  if (splits < 1) splits = 1;
  a.rows_per_split = ceil_div(ceil_div(rows, splits), tn) * tn;
  splits = ceil_div(rows, a.rows_per_split);
  if (qt > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "too many queries");
  const dim3 grid((unsigned)qt, (unsigned)splits);
  if (small)
    launch_valu<OP, 2, 4>(ctx, grid, a, mode, argmin);
  else
    launch_valu<OP, 4, 8>(ctx, grid, a, mode, argmin);
}

// grid: query tiles x row splits, enough workgroups to fill 256 CUs (argmin
// keeps every row of a query in one workgroup)
void launch_flat(vsk_ctx *ctx, FlatArgs a, int mode, int32_t *argmin) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  const int64_t qt = ceil_div(a.nq, FB_Q);
  int64_t splits = mode == MODE_ARGMIN ? 1 : ceil_div(4096, qt);
  const int64_t max_splits = ceil_div(rows, FB_N);
  if (splits > max_splits) splits = max_splits;
  if (splits > 65535) splits = 65535;
  if (splits < 1) splits = 1;
  a.rows_per_split = ceil_div(ceil_div(rows, splits), FB_N) * FB_N;
  splits = ceil_div(rows, a.rows_per_split);
  if (qt > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "too many queries");
  dim3 grid((unsigned)qt, (unsigned)splits);
  const bool valu = a.metric == VSK_METRIC_L1 || a.metric == VSK_METRIC_HAMMING ||
                    a.metric >= METRIC_L2_EXACT;
  static const char *names[2][4] = {
      {"flat_mfma_dense", "flat_mfma_filter", "flat_mfma_matrix", "flat_mfma_argmin"},
      {"flat_valu_dense", "flat_valu_filter", "flat_valu_matrix", "flat_valu_argmin"}};
  const char *name = names[valu ? 1 : 0][mode];
  KernelTimer t(ctx, name, (double)a.nq * (double)rows);
  if (valu) {
    const bool small = mode != MODE_ARGMIN && qt * splits < 4 * (int64_t)ctx->cu_count;
    switch (a.metric) {
    case VSK_METRIC_L1: launch_valu_sized<OP_L1>(ctx, a, mode, argmin, small); break;
    case VSK_METRIC_HAMMING: launch_valu_sized<OP_HAM>(ctx, a, mode, argmin, small); break;
    case METRIC_L2_EXACT: launch_valu_sized<OP_L2SEQ>(ctx, a, mode, argmin, small); break;
    case METRIC_L2SQ_EXACT: launch_valu_sized<OP_L2SQSEQ>(ctx, a, mode, argmin, small); break;
    case METRIC_CN_EXACT: launch_valu_sized<OP_CNSEQ>(ctx, a, mode, argmin, small); break;
    case METRIC_DOT_EXACT: launch_valu_sized<OP_DOTSEQ>(ctx, a, mode, argmin, small); break;
    case METRIC_COS_EXACT: launch_valu_sized<OP_COSSEQ>(ctx, a, mode, argmin, small); break;
    default: fail(VSK_ERR_INVALID_ARGUMENT, "no exact kernel for this metric");
    }
  } else {
    if (mode == MODE_ARGMIN)
      fail(VSK_ERR_UNSUPPORTED, "argmin needs an exact VALU metric");
    switch (a.metric) {
    case VSK_METRIC_L2SQ: launch_mfma<VSK_METRIC_L2SQ>(ctx, grid, a, mode); break;
    case VSK_METRIC_L2: launch_mfma<VSK_METRIC_L2>(ctx, grid, a, mode); break;
    case VSK_METRIC_COSINE: launch_mfma<VSK_METRIC_COSINE>(ctx, grid, a, mode); break;
    case VSK_METRIC_COSINE_NORMALIZED:
      launch_mfma<VSK_METRIC_COSINE_NORMALIZED>(ctx, grid, a, mode);
      break;
    default: launch_mfma<VSK_METRIC_DOT>(ctx, grid, a, mode); break;
    }
  }
  check_launch(name);
}

const float *x_aux(const vsk_db *db, int32_t metric) {
  if (metric == VSK_METRIC_L2SQ || metric == VSK_METRIC_L2)
    return db->sqnorm.as<float>();
  if (metric == VSK_METRIC_COSINE) return db->norm.as<float>();
  if (metric == METRIC_COS_EXACT) {
    if (!db->seqnorm.p) fail(VSK_ERR_EXECUTION_FAILED, "exact cosine norms not made");
    return db->seqnorm.as<float>();
  }
  return nullptr;
}

void ensure_seq_norms(vsk_ctx *ctx, const vsk_db *db) {
  if (db->seqnorm.p) return;
  db->seqnorm.reserve(sizeof(float) * (size_t)db->n);
  seq_norms(ctx, db->x.as<float>(), db->n, db->d, db->ld, db->seqnorm.as<float>());
}

float *q_aux(vsk_ctx *ctx, const float *dq, int64_t nq, int32_t d, int32_t ld,
             int32_t metric) {
  if (metric != VSK_METRIC_L2SQ && metric != VSK_METRIC_L2 &&
      metric != VSK_METRIC_COSINE && metric != METRIC_COS_EXACT)
    return nullptr;
  float *aux = static_cast<float *>(ctx->scratch_ptr("flat.qaux", 4 * nq));
  if (metric == METRIC_COS_EXACT)
    seq_norms(ctx, dq, nq, d, ld, aux);
  else if (metric == VSK_METRIC_COSINE)
    row_norms(ctx, dq, nq, d, ld, nullptr, aux);
  else
    row_norms(ctx, dq, nq, d, ld, aux, nullptr);
  return aux;
}

static bool use_bf16x3(const vsk_ctx *ctx, int32_t metric) {
  return !ctx->flat_fp32 && metric != VSK_METRIC_L1 && metric != VSK_METRIC_HAMMING &&
         metric < METRIC_L2_EXACT;
}

SplitPtrs make_split(vsk_ctx *ctx, const vsk_db *db, const float *dq,
                     int64_t nq, bool qlo, float *qnh, float *qnr) {
  // whole 64-dimension stages of the screen (zero padding)
  const int32_t ldb = (db->d + 63) & ~63;
  if (!db->split.p) {
    // the hi plane (all the screen reads) and the maxima of its bound
    db->split.reserve(sizeof(uint16_t) * (size_t)db->n * ldb);
    db->ldb = ldb;
    uint32_t *mb =
        static_cast<uint32_t *>(ctx->scratch_ptr("flat.splitmax", 2 * sizeof(uint32_t)));
    fill_i32(ctx, reinterpret_cast<int32_t *>(mb), 2, 0);
    split_bf16(ctx, db->x.as<float>(), db->n, db->d, db->ld, db->split.as<uint16_t>(), nullptr,
               ldb, nullptr, nullptr, mb);
    uint32_t hb[2];
    VSK_HIP(hipMemcpyAsync(hb, mb, sizeof(hb), hipMemcpyDeviceToHost, ctx->stream));
    stream_sync(ctx);
    std::memcpy(&db->split_max_hi, &hb[0], sizeof(float));
    std::memcpy(&db->split_max_res, &hb[1], sizeof(float));
  }
  if (qlo && !db->split_lo.p) {
    // the lo plane only for the bf16x3 kernel (hi is written again, the
    // same values)
    db->split_lo.reserve(sizeof(uint16_t) * (size_t)db->n * ldb);
    split_bf16(ctx, db->x.as<float>(), db->n, db->d, db->ld, db->split.as<uint16_t>(),
               db->split_lo.as<uint16_t>(), ldb, nullptr, nullptr, nullptr);
  }
  uint16_t *qs = static_cast<uint16_t *>(ctx->scratch_ptr(
      "flat.qsplit", sizeof(uint16_t) * (qlo ? 2 : 1) * (size_t)nq * ldb));
  split_bf16(ctx, dq, nq, db->d, db->ld, qs, qlo ? qs + (size_t)nq * ldb : nullptr,
             ldb, qnh, qnr, nullptr);
  SplitPtrs s;
  s.xh = db->split.as<uint16_t>();
  s.xl = db->split_lo.as<uint16_t>();  // (null until a bf16x3 call made it)
  s.qh = qs;
  s.ql = qlo ? qs + (size_t)nq * ldb : nullptr;
  s.ldxb = ldb;
  s.ldqb = ldb;
  s.kb = ldb;
  return s;
}

// top-k over a resident database for queries already on the device
bool flat_topk_device(vsk_ctx *ctx, const vsk_db *db, const float *dq,
                      int64_t nq, int32_t k, int32_t metric, uint64_t *best,
                      ScreenDeferred *defer) {
  // a small problem (at most 2^28 query x row x dimension terms, some 20 us
  // of exact VALU work) is cheaper by the exact sequential scan alone than
  // by the screen's fixed chain of launches and its check read-back
  const bool screen = !ctx->flat_no_screen && screen_applies(metric, k);
  if (screen && !ctx->flat_force_screen &&
      (ctx->exact_only || (double)nq * (double)db->n * (double)db->d <= 268435456.0)) {
    approx_topk(ctx, db, dq, nq, k, exact_metric(metric), best, 3);
    return true;
  }
  if (screen && (metric != VSK_METRIC_COSINE || cosine_screen_ok(ctx, db))) {
    screen_topk(ctx, db, dq, nq, k, metric, best, defer);
    return true;
  }
  if (screen) {
    // cosine over rows whose norms the screen's bound cannot cover: the
    // exact scan
    approx_topk(ctx, db, dq, nq, k, exact_metric(metric), best, 3);
    return true;
  }
  approx_topk(ctx, db, dq, nq, k, metric, best, 3);
  return false;
}

void approx_topk(vsk_ctx *ctx, const vsk_db *db, const float *dq, int64_t nq,
                 int32_t k, int32_t metric, uint64_t *best, int passes,
                 float *qnh, float *qnr, int64_t max_growth) {
  const int64_t cap = passes == 1 ? screen_cap(k) : default_cap(k);
  const int64_t qb = query_batch(ctx, nq, cap);
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    const float *qbat = dq + b0 * db->ld;
    if (metric == METRIC_COS_EXACT) ensure_seq_norms(ctx, db);
    float *qa = q_aux(ctx, qbat, nb, db->d, db->ld, metric);
    FlatArgs base{};
    base.X = db->x.as<float>();
    base.ldx = db->ld;
    base.Q = qbat;
    base.ldq = db->ld;
    base.xaux = x_aux(db, metric);
    base.qaux = qa;
    base.kdim = db->ld;
    base.nq = (int32_t)nb;
    base.metric = metric;
    const bool x3 = use_bf16x3(ctx, metric);
    SplitPtrs sp{};
    if (x3)
      sp = make_split(ctx, db, qbat, nb, passes == 3, qnh ? qnh + b0 : nullptr,
                      qnr ? qnr + b0 : nullptr);
    ScanFn scan = [&](const ScanRequest &r) {
      FlatArgs a = base;
      a.r0 = r.r0;
      a.r1 = r.r1;
      a.thresh = r.thresh;
      a.active = r.active;
      a.cand = r.cand;
      a.cap = r.cap;
      a.counts = r.counts;
      if (x3 && passes == 1) {
        a.seg_n = r.dense ? nullptr : r.seg_n;
        launch_flat_screen(ctx, a, sp, r.dense ? MODE_DENSE : MODE_FILTER, r.seg_nseg,
                           r.seg_stride);
      }
      else if (x3)
        launch_flat_bf16x3(ctx, a, sp, r.dense ? MODE_DENSE : MODE_FILTER, passes);
      else
        launch_flat(ctx, a, r.dense ? MODE_DENSE : MODE_FILTER, nullptr);
    };
    progressive_topk(ctx, nb, db->n, k, cap, scan, best + b0 * k,
                     "flat_select", max_growth);
  }
}

// a row filter's rows as a database of their own: row t = rows[t] of db,
// with its norms (the same values, so the filtered search ranks as the
// whole database does)
__global__ void k_gather_db_rows(const float *X, const float *sq, const float *nrm, int32_t ld,
                                 const int32_t *rows, int64_t m, float *out, float *osq,
                                 float *onrm) {
  const int lane = threadIdx.x & 63;
  for (int64_t t = blockIdx.x * 4 + (threadIdx.x >> 6); t < m; t += (int64_t)gridDim.x * 4) {
    const int64_t r = rows[t];
    for (int j = lane; j < ld; j += 64) out[t * ld + j] = X[r * ld + j];
    if (lane == 0) {
      osq[t] = sq[r];
      onrm[t] = nrm[r];
    }
  }
}

}  // namespace vsk

using namespace vsk;

extern "C" {

static vsk_status search_flat_filtered_body(vsk_ctx *ctx, const vsk_db *db, const float *q,
                                    int64_t nq, int32_t k, int32_t metric,
                                    const uint32_t *allow, int64_t allow_bits,
                                    float *out_dist, int64_t *out_ids) {
  if (!allow && allow_bits == 0)
    return vsk_search_flat(ctx, db, q, nq, k, metric, out_dist, out_ids);
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(db, VSK_ERR_INVALID_ARGUMENT, "db is null");
  VSK_REQUIRE(metric_valid(metric), VSK_ERR_INVALID_ARGUMENT, "unknown metric");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(q && out_dist && out_ids, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(k >= 1, VSK_ERR_INVALID_ARGUMENT, "k must be >= 1");
  VSK_REQUIRE(k <= VSK_MAX_K, VSK_ERR_INVALID_BUFFER_SIZE, "k exceeds VSK_MAX_K");
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE, "too many queries");
  VSK_REQUIRE(allow && allow_bits >= 0, VSK_ERR_INVALID_ARGUMENT,
              "row filter: null bitmap or negative size");
  CallScope cs(ctx);
  for (auto &rec : ctx->screen_redo) rec.clear();
  // the rows the filter keeps, ascending (so ties still go to the lower row)
  const int64_t nbits = allow_bits < db->n ? allow_bits : db->n;
  std::vector<uint32_t> bits((size_t)ceil_div(nbits, 32));
  if (!bits.empty()) {
    VSK_HIP(hipMemcpyAsync(bits.data(), allow, sizeof(uint32_t) * bits.size(), hipMemcpyDefault,
                           ctx->stream));
    stream_sync(ctx);
  }
  std::vector<int32_t> rows;
  for (int64_t r = 0; r < nbits; ++r)
    if ((bits[(size_t)(r >> 5)] >> (r & 31)) & 1u) rows.push_back((int32_t)r);
  const int64_t m = (int64_t)rows.size();
  OutputStage od(ctx, out_dist, sizeof(float) * (size_t)nq * k, "out.dist");
  OutputStage oi(ctx, out_ids, sizeof(int64_t) * (size_t)nq * k, "out.ids");
  uint64_t *best = static_cast<uint64_t *>(
      ctx->scratch_ptr("flat.best", sizeof(uint64_t) * (size_t)nq * k));
  vsk_db sub;  // (freed after the call's synchronisation below)
  bool final_keys = true;
  int64_t *id_map = nullptr;
  if (m == 0) {
    fill_u64(ctx, best, nq * (int64_t)k, VSK_KEY_NONE);  // nothing passes
  } else {
    sub.n = m;
    sub.d = db->d;
    sub.ld = db->ld;
    sub.x.reserve(sizeof(float) * (size_t)m * db->ld);
    sub.sqnorm.reserve(sizeof(float) * (size_t)m);
    sub.norm.reserve(sizeof(float) * (size_t)m);
    int32_t *drows = static_cast<int32_t *>(
        ctx->scratch_ptr("flat.frows", sizeof(int32_t) * (size_t)m));
    id_map = static_cast<int64_t *>(ctx->scratch_ptr("flat.fmap", sizeof(int64_t) * (size_t)m));
    std::vector<int64_t> map(rows.begin(), rows.end());
    VSK_HIP(hipMemcpyAsync(drows, rows.data(), sizeof(int32_t) * (size_t)m,
                           hipMemcpyHostToDevice, ctx->stream));
    VSK_HIP(hipMemcpyAsync(id_map, map.data(), sizeof(int64_t) * (size_t)m,
                           hipMemcpyHostToDevice, ctx->stream));
    {
      KernelTimer t(ctx, "flat_filter_gather");
      const int64_t g = ceil_div(m, 4);
      k_gather_db_rows<<<(unsigned)(g < 65535 * 16 ? g : 65535 * 16), 256, 0, ctx->stream>>>(
          db->x.as<float>(), db->sqnorm.as<float>(), db->norm.as<float>(), db->ld, drows, m,
          sub.x.as<float>(), sub.sqnorm.as<float>(), sub.norm.as<float>());
      check_launch("flat_filter_gather");
    }
    const float *dq = rows_to_device_padded(ctx, q, nq, db->d, db->ld, "flat.q");
    final_keys = flat_topk_device(ctx, &sub, dq, nq, k, metric, best);
    // (the host vectors above must outlive their copies)
    stream_sync(ctx);
  }
  decode_keys(ctx, best, nq * (int64_t)k, metric == VSK_METRIC_L2 && !final_keys, id_map,
              od.ptr<float>(), oi.ptr<int64_t>());
  od.copy_back();
  oi.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

// top-k overflow is checked at the call's end (topk_call)
vsk_status vsk_search_flat_filtered(vsk_ctx *ctx, const vsk_db *db, const float *q,
                                    int64_t nq, int32_t k, int32_t metric,
                                    const uint32_t *allow, int64_t allow_bits,
                                    float *out_dist, int64_t *out_ids) {
  return topk_call(ctx, [&] { return search_flat_filtered_body(ctx, db, q, nq, k, metric, allow, allow_bits, out_dist, out_ids); });
}

static vsk_status search_flat_body(vsk_ctx *ctx, const vsk_db *db, const float *q,
                           int64_t nq, int32_t k, int32_t metric,
                           float *out_dist, int64_t *out_ids) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(db, VSK_ERR_INVALID_ARGUMENT, "db is null");
  VSK_REQUIRE(metric_valid(metric), VSK_ERR_INVALID_ARGUMENT,
              "unknown metric");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(q && out_dist && out_ids, VSK_ERR_INVALID_ARGUMENT,
              "null buffer");
  VSK_REQUIRE(k >= 1, VSK_ERR_INVALID_ARGUMENT, "k must be >= 1");
  VSK_REQUIRE(k <= VSK_MAX_K, VSK_ERR_INVALID_BUFFER_SIZE,
              "k exceeds VSK_MAX_K");
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "too many queries");
  CallScope cs(ctx);
  for (auto &rec : ctx->screen_redo) rec.clear();
  const float *dq = rows_to_device_padded(ctx, q, nq, db->d, db->ld, "flat.q");
  uint64_t *best = static_cast<uint64_t *>(
      ctx->scratch_ptr("flat.best", sizeof(uint64_t) * (size_t)nq * k));
  // the screen's bound check is read with the call's synchronisation
  ScreenDeferred defer;
  const bool final_keys = flat_topk_device(ctx, db, dq, nq, k, metric, best, &defer);
  OutputStage od(ctx, out_dist, sizeof(float) * (size_t)nq * k, "out.dist");
  OutputStage oi(ctx, out_ids, sizeof(int64_t) * (size_t)nq * k, "out.ids");
  decode_keys(ctx, best, nq * (int64_t)k, metric == VSK_METRIC_L2 && !final_keys,
              nullptr, od.ptr<float>(), oi.ptr<int64_t>());
  od.copy_back();
  oi.copy_back();
  cs.finish();
  // queries that failed the bound (near ties) are redone now and the
  // results written again; an overflowed top-k reruns the whole call
  if (!ctx->topk_overflowed && screen_finish(ctx, db, dq, k, metric, best, defer)) {
    decode_keys(ctx, best, nq * (int64_t)k, false, nullptr, od.ptr<float>(),
                oi.ptr<int64_t>());
    od.copy_back();
    oi.copy_back();
    cs.finish();
  }
  VSK_API_END(ctx);
}

// top-k overflow is checked at the call's end (topk_call)
vsk_status vsk_search_flat(vsk_ctx *ctx, const vsk_db *db, const float *q,
                           int64_t nq, int32_t k, int32_t metric,
                           float *out_dist, int64_t *out_ids) {
  return topk_call(ctx, [&] { return search_flat_body(ctx, db, q, nq, k, metric, out_dist, out_ids); });
}

vsk_status vsk_distances(vsk_ctx *ctx, const vsk_db *db, const float *q,
                         int64_t nq, int32_t metric, float *out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(db, VSK_ERR_INVALID_ARGUMENT, "db is null");
  VSK_REQUIRE(metric_valid(metric), VSK_ERR_INVALID_ARGUMENT,
              "unknown metric");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(q && out, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "too many queries");
  CallScope cs(ctx);
  const float *dq = rows_to_device_padded(ctx, q, nq, db->d, db->ld, "flat.q");
  OutputStage om(ctx, out, sizeof(float) * (size_t)nq * db->n, "out.matrix");
  FlatArgs a{};
  a.X = db->x.as<float>();
  a.ldx = db->ld;
  a.Q = dq;
  a.ldq = db->ld;
  a.xaux = x_aux(db, metric);
  a.qaux = q_aux(ctx, dq, nq, db->d, db->ld, metric);
  a.kdim = db->ld;
  a.nq = (int32_t)nq;
  a.r0 = 0;
  a.r1 = db->n;
  a.metric = metric;
  a.mat = om.ptr<float>();
  a.ldm = db->n;
  // Every metric of the reference's CPU path is evaluated as it evaluates
  // it, on the exact VALU kernel: L2 and L2^2 sum (q - x)^2 in dimension
  // order (the norm expansion |q|^2 + |x|^2 - 2 q.x of an MFMA path cancels
  // for close pairs: a duplicate row would get sqrt of the rounding error,
  // not 0); cosine, normalised cosine and dot sum q.x in dimension order,
  // cosine with the sequential norms.  The matrix is then the reference's
  // bit for bit, and exactly symmetric when the rows are the queries.
  if (exact_metric(metric) >= 0) {
    a.metric = exact_metric(metric);
    a.xaux = nullptr;
    a.qaux = nullptr;
    if (metric == VSK_METRIC_COSINE) {
      ensure_seq_norms(ctx, db);
      a.xaux = x_aux(db, METRIC_COS_EXACT);
      a.qaux = q_aux(ctx, dq, nq, db->d, db->ld, METRIC_COS_EXACT);
    }
  }
  if (use_bf16x3(ctx, a.metric))
    launch_flat_bf16x3(ctx, a, make_split(ctx, db, dq, nq, true, nullptr, nullptr),
                       MODE_MATRIX);
  else
    launch_flat(ctx, a, MODE_MATRIX, nullptr);
  om.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

}  // extern "C"
