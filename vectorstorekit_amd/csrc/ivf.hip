// ivf.hip -- IVF-Flat: coarse probing, insertion into CSR inverted lists and
// the list-major inverted-list scan.
//
// Reference: IVFIndex (Indexes/IVFIndex.swift): insert (:80-122) appends a
// row to the list of its nearest centroid (findNearestCentroid, :514-527);
// search (:124-202) ranks the centroids by sqrt-L2 (findNearestCentroids,
// :529-540), concatenates the nprobe lists in probe order (:151-157),
// computes the exact sqrt-L2 of every candidate (:167-172) and keeps the
// first k after a stable sort (:175-176).
//
// Layout in HBM: the centroids as a resident flat database; the lists as
// CSR -- rows sorted by list (insertion order inside a list), their user
// ids, and list offsets.
//
// Search pipeline (all on the stream):
//  1. probe: exact sequential-L2 (VALU, bit-identical to the reference's
//     loop) of every (query, centroid) pair + top-nprobe selection with ties
//     broken by centroid index;
//  2. per query, the candidate count and each probe's position base (the
//     offset of its list in the probe-ordered concatenation);
//  3. the (query, probe) pairs are grouped by list, so each list is read
//     from HBM once per group of up to QG queries rather than once per
//     query; a thread owns one list row and keeps QG sequential-L2
//     accumulators; every distance is written as a (distance, position) key
//     into its query's candidate segment;
//  4. per-query selection over the segment -> k smallest (distance,
//     position), i.e. the stable-sort prefix; positions map back to ids.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <numeric>

#include "flat.hpp"

// largest dimension and list count an index (and its file) may have
constexpr int32_t kMaxDim = 65536, kMaxLists = 1 << 24;

struct vsk_ivf {
  int32_t nlist = 0, d = 0, ld = 0;
  vsk_db centroids;
  vsk::DevBuf rows;     // total x ld fp32, grouped by list
  vsk::DevBuf ids;      // total int64
  vsk::DevBuf list_off; // nlist+1 int64 (device copy of off)
  std::vector<int64_t> off;  // nlist+1
  int64_t total = 0;
  int64_t next_id = 0;
  // codes of the stored rows, same list-grouped order (vsk_ivf_encode_*):
  // kind 1 = SQ8 (d int8), 2 = PQ (M uint8); rows of cstride bytes, zero
  // padded; valid while ctotal == total
  vsk::DevBuf codes;
  int32_t ckind = 0, cstride = 0, cM = 0, cksub = 0;
  int64_t ctotal = -1;
  // the quantizer the codes were made with: SQ8 scale then offset (d values
  // each when cper_dim, else 1), or the PQ codebooks (cM x cksub x cdsub)
  std::vector<float> cparams;
  int32_t cper_dim = 0, cdsub = 0;
  // codes only (vsk_ivf_drop_rows): the fp32 rows are gone, the codes stay
  // current (inserts are encoded with the stored quantizer)
  bool codes_only = false;
  // caller bytes stored with the index file (e.g. the index configuration)
  std::vector<uint8_t> meta;
  // the bf16 screen of the list scan: the stored rows as a bf16 plane of
  // xldb columns, |x|^2 per row and the maxima of |bf16(x)| and
  // |x - bf16(x)| over the rows, valid while xversion == version (version
  // counts the changes of the stored rows)
  int64_t version = 0;
  mutable int64_t xversion = -1;
  mutable vsk::DevBuf xplane, xsq;
  mutable int32_t xldb = 0;
  mutable double xh_max = 0, xr_max = 0;
  // per list the largest distance of its rows from its centroid (for the
  // list scan's per-query bound), valid with the plane
  mutable vsk::DevBuf xrad;
};

namespace vsk {

typedef float f4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------
__global__ void k_scatter_rows(const float *src, const int64_t *src_ids,
                               int64_t id_base, const int64_t *dest, int64_t n,
                               int32_t ld, float *dst, int64_t *dst_ids) {
  // one wave per row
  const int lane = threadIdx.x & 63;
  for (int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < n;
       r += (int64_t)gridDim.x * 4) {
    const int64_t t = dest[r];
    for (int j = lane; j < ld; j += 64) dst[t * ld + j] = src[r * ld + j];
    if (lane == 0) dst_ids[t] = src_ids ? src_ids[r] : id_base + r;
  }
}

// keys (dist, centroid) of the top-nprobe -> centroid indices
__global__ void k_keys_to_tie(const uint64_t *keys, int64_t total,
                              int32_t *out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = keys[i] == VSK_KEY_NONE ? -1 : (int32_t)(uint32_t)keys[i];
}

// per query: candidate count and the position base of each probe (the
// exclusive prefix of its probes' list sizes); one wave per query, 64
// probes at a time with a shuffle scan
// With keys, the probes are first taken from the probe's ranked keys
// (NONE: -1) and written out.  With lcnt, the blocks also clear the nlist
// per-list pair counters for the first batch's grouping.
// With bound.qlim (and keys), each query's bound on the screened words the
// list scan keeps.  The rows of a list whose centroid lies at distance d
// from the query are within d + R of it (R: the list's radius, the largest
// distance of its rows from the centroid), so the smallest V for which the
// lists with d + R <= V hold k rows bounds the k-th distance.  d, R and the
// exact distances are fp32 sums, each within 2^-16 of the real distance
// relatively, so V (1 + 2^-10) bounds the k-th exact one, and a candidate whose
// screened squared distance is above that squared (times 1 + 2^-10) plus
// 2 eps -- eps the screen's bound -- is farther than k others: it cannot be
// among the k nearest.  From the first 64 probes; none that hold k rows
// (or a bound that is not finite): every candidate is kept.
struct ProbeBound {
  uint32_t *qlim = nullptr;
  const float *rad = nullptr;   // per list R
  int32_t k = 0;
  const float *qnh = nullptr, *qnr = nullptr;  // the queries' plane norms
  double xh = 0, xr = 0;
  int32_t d = 0, metric = 0, nprod = 0;
};
__global__ __launch_bounds__(256) void k_probe_bases(int32_t *probes, const uint64_t *keys,
                                                     int64_t nq, int32_t np,
                                                     const int64_t *list_off,
                                                     int64_t *pos_base, int64_t *cnt,
                                                     int32_t *lcnt, int32_t nlist,
                                                     ProbeBound bound = ProbeBound{}) {
  if (lcnt)
    for (int64_t l = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; l < nlist;
         l += (int64_t)gridDim.x * blockDim.x)
      lcnt[l] = 0;
  const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (q >= nq) return;
  int64_t carry = 0;
  for (int p0 = 0; p0 < np; p0 += 64) {
    const int p = p0 + lane;
    int64_t sz = 0;
    if (p < np) {
      int32_t l;
      if (keys) {
        const uint64_t key = keys[q * np + p];
        l = key == VSK_KEY_NONE ? -1 : (int32_t)(uint32_t)key;
        probes[q * np + p] = l;
      } else {
        l = probes[q * np + p];
      }
      if (l >= 0) sz = list_off[l + 1] - list_off[l];
    }
    int64_t incl = sz;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    if (p < np) pos_base[q * np + p] = carry + incl - sz;
    carry += __shfl(incl, 63);
    if (bound.qlim && keys && p0 == 0) {
      float v = __int_as_float(0x7f800000);  // this probe's d + R
      if (p < np && sz > 0) {
        const uint64_t key = keys[q * np + p];
        const int32_t l = (int32_t)(uint32_t)key;
        v = vsk_ord2f((uint32_t)(key >> 32)) + bound.rad[l];
        if (!(v < __int_as_float(0x7f800000))) v = __int_as_float(0x7f800000);
      }
      // the rows of the probes whose d + R is at most this one's (each
      // probe's value and size read out of its lane into scalars)
      const int32_t sz32 = (int32_t)min<int64_t>(sz, 0x7FFFFFFF);
      const int npl = np < 64 ? np : 64;
      int64_t rows = 0;
      for (int i = 0; i < npl; ++i) {
        const float vi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
        const int32_t si = __builtin_amdgcn_readlane(sz32, i);
        if (vi <= v) rows += si;
      }
      float V = rows >= bound.k ? v : __int_as_float(0x7f800000);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) V = fminf(V, __shfl_xor(V, o));
      if (lane == 0) {
        uint32_t lim = kWordNone - 1u;  // every candidate
        if (V < __int_as_float(0x7f800000)) {
          const double u = (double)V * (1.0 + 0x1p-10);
          const double eps = screen_eps_of(bound.qnh[q], bound.qnr[q], bound.xh, bound.xr,
                                           bound.d, bound.metric, bound.nprod);
          const double w = u * u * (1.0 + 0x1p-10) + 2.0 * eps;
          if (w < 0x1p127) lim = vsk_f2ord(f_down(w));
        }
        bound.qlim[q] = lim;
      }
    }
  }
  if (lane == 0) cnt[q] = carry;
}

// pair (q, p) -> its slot in the list-grouped pair array: its list's
// first slot plus its rank there
// (lcnt, read by the offsets before this launch, is cleared here for the
// next batch)
__global__ void k_group_pairs(const int32_t *probes, int64_t npairs, const int64_t *lstart,
                              const int32_t *rank, int32_t *pairs, int32_t *lcnt,
                              int32_t nlist) {
  for (int64_t l = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; l < nlist;
       l += (int64_t)gridDim.x * blockDim.x)
    lcnt[l] = 0;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < npairs;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t l = probes[i];
    if (l < 0) continue;
    pairs[lstart[l] + rank[i]] = (int32_t)i;  // i = q * np + p
  }
}

// exclusive prefix over a block of 1024 threads of NV values per thread,
// continuing the running totals carry[0..NV) (shared memory)
template <int NV>
__device__ void block_scan_1024(const int64_t (&v)[NV], int64_t (&out)[NV],
                                int64_t (*wsum)[NV], int64_t *carry) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int64_t incl[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    incl[j] = v[j];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t u = __shfl_up(incl[j], o);
      if (lane >= o) incl[j] += u;
    }
  }
  if (lane == 63)
#pragma unroll
    for (int j = 0; j < NV; ++j) wsum[w][j] = incl[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    int64_t before = carry[j];
    for (int i = 0; i < w; ++i) before += wsum[i][j];
    out[j] = before + incl[j] - v[j];
  }
  __syncthreads();
  if (t == 1023)
#pragma unroll
    for (int j = 0; j < NV; ++j) carry[j] = out[j] + v[j];
  __syncthreads();
}

// seg[i] = cnt[0] + ... + cnt[i-1] for i = 0..m (one block of 1024, each
// thread a run of consecutive counts, one block scan of the runs' sums);
// with wseg, the same over the counts rounded up to multiples of 4
__device__ void seg_offsets(const int64_t *cnt, int64_t m, int64_t *seg, int64_t *wseg) {
  __shared__ int64_t wsum[16][2];
  __shared__ int64_t carry[2];
  if (threadIdx.x < 2) carry[threadIdx.x] = 0;
  __syncthreads();
  const int64_t run = (m + 1023) / 1024;
  const int64_t i0 = threadIdx.x * run, i1 = i0 + run < m ? i0 + run : m;
  int64_t v[2] = {0, 0};
  // runs of up to 16 are read into registers at once (a loop that waits
  // for each load took most of the launch)
  constexpr int RUN = 16;
  int64_t cr[RUN];
  if (run <= RUN) {
#pragma unroll
    for (int u = 0; u < RUN; ++u) cr[u] = i0 + u < i1 ? cnt[i0 + u] : 0;
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
      v[0] += cr[u];
      v[1] += (cr[u] + 3) & ~3ll;
    }
  } else {
    for (int64_t i = i0; i < i1; ++i) {
      const int64_t c = cnt[i];
      v[0] += c;
      v[1] += (c + 3) & ~3ll;
    }
  }
  int64_t o[2];
  block_scan_1024<2>(v, o, wsum, carry);
  if (run <= RUN) {
#pragma unroll
    for (int u = 0; u < RUN; ++u)
      if (i0 + u < i1) {
        seg[i0 + u] = o[0];
        if (wseg) wseg[i0 + u] = o[1];
        o[0] += cr[u];
        o[1] += (cr[u] + 3) & ~3ll;
      }
  } else {
    for (int64_t i = i0; i < i1; ++i) {
      const int64_t c = cnt[i];
      seg[i] = o[0];
      if (wseg) wseg[i] = o[1];
      o[0] += c;
      o[1] += (c + 3) & ~3ll;
    }
  }
  if (threadIdx.x == 0) {
    seg[m] = carry[0];
    if (wseg) wseg[m] = carry[1];
  }
}

// pairs per list, and each pair's rank among its list's pairs
__global__ void k_list_pair_counts(const int32_t *probes, int64_t npairs, int32_t *lcnt,
                                   int32_t *rank) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < npairs;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t l = probes[i];
    if (l >= 0) rank[i] = atomicAdd(&lcnt[l], 1);
  }
}

// The same with the counting in LDS: workgroup b takes pairs [b per,
// (b + 1) per), ranks them within its share of each list by LDS atomics,
// takes its base in each list it touches with one device atomic, and adds
// it.  Device atomics drop from one a pair to one a (workgroup, list).
// Dynamic LDS: nlist counters.
__global__ __launch_bounds__(1024) void k_list_pair_counts_lds(const int32_t *probes,
                                                               int64_t npairs, int64_t per,
                                                               int32_t *lcnt, int32_t *rank,
                                                               int32_t nlist) {
  extern __shared__ int32_t s_cnt[];
  for (int l = threadIdx.x; l < nlist; l += blockDim.x) s_cnt[l] = 0;
  __syncthreads();
  const int64_t i0 = blockIdx.x * per, i1 = i0 + per < npairs ? i0 + per : npairs;
  // eight pairs a thread at a time, their loads issued together
  constexpr int U = 8;
  for (int64_t b = i0 + threadIdx.x; b < i1; b += U * (int64_t)blockDim.x) {
    int32_t l[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = b + u * (int64_t)blockDim.x;
      l[u] = i < i1 ? probes[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (l[u] >= 0) rank[b + u * (int64_t)blockDim.x] = atomicAdd(&s_cnt[l[u]], 1);
  }
  __syncthreads();
  for (int l = threadIdx.x; l < nlist; l += blockDim.x) {
    const int32_t c = s_cnt[l];
    if (c > 0) s_cnt[l] = atomicAdd(&lcnt[l], c);
  }
  __syncthreads();
  for (int64_t b = i0 + threadIdx.x; b < i1; b += U * (int64_t)blockDim.x) {
    int32_t l[U], r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = b + u * (int64_t)blockDim.x;
      l[u] = i < i1 ? probes[i] : -1;
      r[u] = l[u] >= 0 ? rank[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (l[u] >= 0) rank[b + u * (int64_t)blockDim.x] = r[u] + s_cnt[l[u]];
  }
}

// per list: its first pair slot (lstart)
// and its first group (gstart; ceil(pairs / G) groups for a list holding
// rows, none for an empty one); totals at [nlist].  One block of 1024,
// each thread a run of consecutive lists.
__device__ inline int64_t list_groups(const int32_t *lcnt, const int64_t *list_off, int64_t l,
                                      int32_t G) {
  const int64_t c = lcnt[l];
  return c > 0 && list_off[l + 1] > list_off[l] ? (c + G - 1) / G : 0;
}
__device__ void list_offsets(const int32_t *lcnt, const int64_t *list_off, int32_t nlist,
                             int32_t G, int64_t *lstart, int64_t *gstart, int4 *groups) {
  __shared__ int64_t wsum[16][2];
  __shared__ int64_t carry[2];
  if (threadIdx.x < 2) carry[threadIdx.x] = 0;
  __syncthreads();
  const int64_t run = (nlist + 1023) / 1024;
  const int64_t l0 = threadIdx.x * run, l1 = l0 + run < nlist ? l0 + run : nlist;
  int64_t v[2] = {0, 0};
  // the list's groups: (list, first pair slot, pairs, 0), up to G pairs
  auto emit = [&](int64_t l, int32_t c, int64_t ng, int64_t (&o)[2]) {
    for (int64_t j = 0; j < ng; ++j)
      groups[o[1] + j] = int4{(int)l, (int)(o[0] + j * G), (int)min<int64_t>(G, c - j * G), 0};
    lstart[l] = o[0];
    gstart[l] = o[1];
    o[0] += c;
    o[1] += ng;
  };
  // runs of up to 8 lists are read into registers at once
  constexpr int RUN = 8;
  int32_t cr[RUN];
  int64_t gr[RUN];
  int64_t o[2];
  if (run <= RUN) {
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
      cr[u] = l0 + u < l1 ? lcnt[l0 + u] : 0;
      gr[u] = l0 + u < l1 ? list_groups(lcnt, list_off, l0 + u, G) : 0;
    }
#pragma unroll
    for (int u = 0; u < RUN; ++u) {
      v[0] += cr[u];
      v[1] += gr[u];
    }
    block_scan_1024<2>(v, o, wsum, carry);
#pragma unroll
    for (int u = 0; u < RUN; ++u)
      if (l0 + u < l1) emit(l0 + u, cr[u], gr[u], o);
  } else {
    for (int64_t l = l0; l < l1; ++l) {
      v[0] += lcnt[l];
      v[1] += list_groups(lcnt, list_off, l, G);
    }
    block_scan_1024<2>(v, o, wsum, carry);
    for (int64_t l = l0; l < l1; ++l) emit(l, lcnt[l], list_groups(lcnt, list_off, l, G), o);
  }
  if (threadIdx.x == 0) {
    lstart[nlist] = carry[0];
    gstart[nlist] = carry[1];
  }
}

// block 0: the batch's segment offsets (seg_offsets); block 1 (when there
// are lists to group): the lists' pair and group offsets and the groups
__global__ __launch_bounds__(1024) void k_batch_offsets(const int64_t *cnt, int64_t m,
                                                        int64_t *seg, int64_t *wseg,
                                                        const int32_t *lcnt,
                                                        const int64_t *list_off, int32_t nlist,
                                                        int32_t G, int64_t *lstart,
                                                        int64_t *gstart, int4 *groups) {
  if (blockIdx.x == 0) seg_offsets(cnt, m, seg, wseg);
  else list_offsets(lcnt, list_off, nlist, G, lstart, gstart, groups);
}


struct ListScanArgs {
  const float *rows;     // list rows, ld stride
  const int64_t *list_off;
  const float *Q;        // queries (batch), ld stride
  int32_t ld;
  int32_t np;            // probes per query
  const int32_t *probes; // [nq][np]
  const int32_t *pairs;  // pair ids (q*np+p) grouped by list
  const int4 *groups;    // (list, pair_begin, pair_count, 0)
  const int64_t *ngroups;   // groups made (the grid is an upper bound)
  const int64_t *pos_base;  // [nq][np]
  // each candidate's distance as its order-preserving 32-bit word (the
  // high half of its (distance, position) key) at words[wseg[q] + position]
  const int64_t *wseg;      // [nq+1] word segment offsets (multiples of 4)
  uint32_t *words;
  int32_t squared;          // 1: key on sum (q-x)^2, 0: on its sqrt
  // coded scans
  const uint8_t *codes;     // list-grouped codes, cstride bytes per row
  int32_t cstride;
  const int8_t *qc;         // SQ8: query codes, cstride bytes each (batch)
  const float *lut;         // PQ: [nq][M][ksub] (batch)
  int32_t M, ksub;
};

// the QG query slots of a group: query index, candidate-segment base and
// position base of each (slots past the group's count repeat its first)
#define VSK_GROUP_SLOTS(QG)                                        \
  if (blockIdx.x >= *a.ngroups) return;                            \
  const int4 g = a.groups[blockIdx.x];                             \
  const int32_t l = g.x;                                           \
  const int npair = g.z;                                           \
  const int64_t v0 = a.list_off[l], v1 = a.list_off[l + 1];        \
  int32_t qidx[QG];                                                \
  int64_t obase[QG], tbase[QG];                                    \
  _Pragma("unroll") for (int j = 0; j < QG; ++j) {                 \
    const int32_t pid = a.pairs[g.y + (j < npair ? j : 0)];        \
    qidx[j] = pid / a.np;                                          \
    obase[j] = a.wseg[qidx[j]] + a.pos_base[pid];                  \
    tbase[j] = a.pos_base[pid];                                    \
  }

// IVF-SQ8 list scan: score = sum_j qcode_j * code_j (exact int32, four
// products per v_dot4), keyed as distance -score.  Query codes of the group
// in LDS, one row per thread, 16-byte code loads.
template <int QG>
__global__ __launch_bounds__(256) void k_list_scan_sq8(ListScanArgs a) {
  extern __shared__ int32_t qw[];  // QG x cstride bytes
  VSK_GROUP_SLOTS(QG)
  const int cw = a.cstride / 4;
  for (int i = threadIdx.x; i < QG * cw; i += blockDim.x) {
    const int j = i / cw, c = i - j * cw;
    qw[i] = reinterpret_cast<const int32_t *>(a.qc + (int64_t)qidx[j] * a.cstride)[c];
  }
  __syncthreads();
  for (int64_t v = v0 + threadIdx.x; v < v1; v += blockDim.x) {
    const int4 *x = reinterpret_cast<const int4 *>(a.codes + v * a.cstride);
    int32_t acc[QG];
#pragma unroll
    for (int j = 0; j < QG; ++j) acc[j] = 0;
    for (int c = 0; c < cw / 4; ++c) {
      const int4 xv = x[c];
#pragma unroll
      for (int j = 0; j < QG; ++j) {
        const int4 qv = reinterpret_cast<const int4 *>(qw + j * cw)[c];
        acc[j] = __builtin_amdgcn_sdot4(qv.x, xv.x, acc[j], false);
        acc[j] = __builtin_amdgcn_sdot4(qv.y, xv.y, acc[j], false);
        acc[j] = __builtin_amdgcn_sdot4(qv.z, xv.z, acc[j], false);
        acc[j] = __builtin_amdgcn_sdot4(qv.w, xv.w, acc[j], false);
      }
    }
    const int64_t i = v - v0;
#pragma unroll
    for (int j = 0; j < QG; ++j)
      if (j < npair) a.words[obase[j] + i] = (uint32_t)(-acc[j]) ^ 0x80000000u;
  }
}

// one workgroup per group: up to QG queries probing the same list
template <int QG>
__global__ __launch_bounds__(256) void k_list_scan(ListScanArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float qs[];  // QG x ld
  if (blockIdx.x >= *a.ngroups) return;
  const int4 g = a.groups[blockIdx.x];
  const int32_t l = g.x;
  const int npair = g.z;
  const int64_t v0 = a.list_off[l], v1 = a.list_off[l + 1];
  int32_t qidx[QG];
  int64_t obase[QG], tbase[QG];
#pragma unroll
  for (int j = 0; j < QG; ++j) {
    int32_t pid = a.pairs[g.y + (j < npair ? j : 0)];
    int32_t q = pid / a.np;
    qidx[j] = q;
    obase[j] = a.wseg[q] + a.pos_base[pid];
    tbase[j] = a.pos_base[pid];
  }
  for (int i = threadIdx.x; i < QG * a.ld; i += blockDim.x) {
    int j = i / a.ld, c = i - j * a.ld;
    int32_t pid = a.pairs[g.y + (j < npair ? j : 0)];
    qs[i] = a.Q[(int64_t)(pid / a.np) * a.ld + c];
  }
  __syncthreads();
  for (int64_t v = v0 + threadIdx.x; v < v1; v += blockDim.x) {
    const float *x = a.rows + v * a.ld;
    float acc[QG];
#pragma unroll
    for (int j = 0; j < QG; ++j) acc[j] = 0.f;
    for (int c = 0; c < a.ld; c += 4) {
      const f4 xv = *reinterpret_cast<const f4 *>(x + c);
#pragma unroll
      for (int j = 0; j < QG; ++j) {
        const f4 qv = *reinterpret_cast<const f4 *>(qs + j * a.ld + c);
        float t;
        t = qv.x - xv.x;
        acc[j] = acc[j] + t * t;
        t = qv.y - xv.y;
        acc[j] = acc[j] + t * t;
        t = qv.z - xv.z;
        acc[j] = acc[j] + t * t;
        t = qv.w - xv.w;
        acc[j] = acc[j] + t * t;
      }
    }
    const int64_t i = v - v0;
#pragma unroll
    for (int j = 0; j < QG; ++j)
      if (j < npair)
        a.words[obase[j] + i] = vsk_f2ord(a.squared ? acc[j] : sqrtf(acc[j]));
  }
  (void)qidx;
}

// IVF-PQ list scan: ADC sum = sum over segments m, in order, of
// lut[q][m][code_m] (fp32, each addition rounded: DistanceTables.
// computeDistance, Quantization/ProductQuantizerTypes.swift:14-20), keyed
// (sum, position).  One workgroup per query: its tables stay in LDS while it
// walks its probed lists (a table is 4 M ksub bytes, a probed list's codes
// a few KB, so keeping the table and streaming the codes moves the least).
__global__ __launch_bounds__(256) void k_list_scan_pq_q(ListScanArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float tl[];  // M x ksub
  const int64_t q = blockIdx.x;
  const int tsz = a.M * a.ksub;
  for (int i = threadIdx.x; i < tsz; i += blockDim.x) tl[i] = a.lut[q * tsz + i];
  __syncthreads();
  const int64_t seg = a.wseg[q];
  for (int p = 0; p < a.np; ++p) {
    const int32_t l = a.probes[q * a.np + p];
    if (l < 0) continue;
    const int64_t v0 = a.list_off[l], v1 = a.list_off[l + 1];
    const int64_t tb = a.pos_base[q * a.np + p];
    for (int64_t v = v0 + threadIdx.x; v < v1; v += blockDim.x) {
      const uint32_t *x = reinterpret_cast<const uint32_t *>(a.codes + v * a.cstride);
      float acc = 0.f;
      for (int m0 = 0; m0 < a.M; m0 += 4) {
        const uint32_t w = x[m0 >> 2];
        const int mm = a.M - m0 < 4 ? a.M - m0 : 4;
        for (int t = 0; t < mm; ++t)
          acc = acc + tl[(m0 + t) * a.ksub + (int)((w >> (8 * t)) & 0xFFu)];
      }
      a.words[seg + tb + (v - v0)] = vsk_f2ord(acc);
    }
  }
}

// A search's row filter in list order: bit v of lmask is set when stored row
// v may be a candidate, i.e. its id i has 0 <= i < allow_bits and bit i of
// the caller's bitmap allow (ids the bitmap does not reach are excluded).
// Each wave writes the two words of its 64 rows.
__global__ __launch_bounds__(256) void k_allow_list_bits(const int64_t *ids, int64_t total,
                                                         const uint32_t *allow,
                                                         int64_t allow_bits, uint32_t *lmask) {
  const int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  bool ok = false;
  if (v < total) {
    const int64_t id = ids[v];
    ok = id >= 0 && id < allow_bits && ((allow[id >> 5] >> (id & 31)) & 1u);
  }
  const uint64_t b = __ballot(ok);
  const int64_t w0 = v - (threadIdx.x & 63);  // the wave's first row
  if ((threadIdx.x & 63) == 0 && w0 < total) {
    lmask[w0 >> 5] = (uint32_t)b;
    lmask[(w0 >> 5) + 1] = (uint32_t)(b >> 32);
  }
}

// Candidates the filter excludes leave their query's ranking: the word at
// each excluded position becomes kWordNone, which every selection skips
// (and which the screens' margins never reach).  One workgroup per query
// walks its probes' lists; the positions are those the list scans write.
__global__ __launch_bounds__(256) void k_mask_words(const int32_t *probes, int32_t np,
                                                    const int64_t *pos_base,
                                                    const int64_t *list_off, const int64_t *wseg,
                                                    const uint32_t *lmask, uint32_t *words,
                                                    int64_t nq) {
  const int64_t q = blockIdx.x;
  if (q >= nq) return;
  uint32_t *W = words + wseg[q];
  for (int p = 0; p < np; ++p) {
    const int32_t l = probes[q * np + p];
    if (l < 0) continue;
    const int64_t v0 = list_off[l], v1 = list_off[l + 1];
    const int64_t tb = pos_base[q * np + p];
    for (int64_t v = v0 + threadIdx.x; v < v1; v += blockDim.x)
      if (!((lmask[v >> 5] >> (v & 31)) & 1u)) W[tb + (v - v0)] = kWordNone;
  }
}

// row removal: dst row t = src row idx[t] (ld floats, one wave a row), its
// id, and (codes non-null) its cstride code bytes (a multiple of 4)
__global__ void k_gather_stored(const float *src, const int64_t *src_ids, const uint8_t *codes,
                                int32_t cstride, const int64_t *idx, int64_t n, int32_t ld,
                                float *dst, int64_t *dst_ids, uint8_t *dst_codes) {
  const int lane = threadIdx.x & 63;
  for (int64_t t = blockIdx.x * 4 + (threadIdx.x >> 6); t < n; t += (int64_t)gridDim.x * 4) {
    const int64_t s = idx[t];
    if (src)  // (a codes-only index has no rows)
      for (int j = lane; j < ld; j += 64) dst[t * ld + j] = src[s * ld + j];
    if (codes) {
      const uint32_t *cs = reinterpret_cast<const uint32_t *>(codes + s * cstride);
      uint32_t *cd = reinterpret_cast<uint32_t *>(dst_codes + t * cstride);
      for (int j = lane; j < cstride / 4; j += 64) cd[j] = cs[j];
    }
    if (lane == 0) dst_ids[t] = src_ids[s];
  }
}

// code rows to their list positions (a codes-only index's insert): row r
// of src (w bytes at src_stride; null: left as is) goes to dest[r] of dst
// (cstride bytes a row, zero padded beforehand), its id with it (src_ids
// null: id_base + r).  One wave per row, byte copies (w is a few hundred
// bytes at most).
__global__ void k_scatter_codes(const uint8_t *src, int32_t src_stride, int32_t w,
                                const int64_t *src_ids, int64_t id_base, const int64_t *dest,
                                int64_t n, int32_t cstride, uint8_t *dst, int64_t *dst_ids) {
  const int lane = threadIdx.x & 63;
  for (int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < n; r += (int64_t)gridDim.x * 4) {
    const int64_t t = dest[r];
    if (src)
      for (int j = lane; j < w; j += 64) dst[t * cstride + j] = src[r * src_stride + j];
    if (lane == 0) dst_ids[t] = src_ids ? src_ids[r] : id_base + r;
  }
}

// best keys (dist, position) -> (dist, user id)
__global__ void k_ivf_decode(const uint64_t *best, int64_t nq, int32_t k,
                             const int32_t *probes, int32_t np,
                             const int64_t *pos_base, const int64_t *list_off,
                             const int64_t *ids, void *out_dist,
                             int64_t *out_ids, int32_t kind) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= nq * k) return;
  const int64_t q = i / k;
  const uint64_t key = best[i];
  float *of = static_cast<float *>(out_dist);
  int32_t *os = static_cast<int32_t *>(out_dist);
  if (key == VSK_KEY_NONE) {
    if (kind == 1)
      os[i] = INT32_MIN;
    else
      of[i] = __int_as_float(0x7f800000);
    out_ids[i] = -1;
    return;
  }
  const int64_t pos = (uint32_t)key;
  const int64_t *pb = pos_base + q * np;
  int p = np - 1;
  while (p > 0 && (pb[p] > pos || probes[q * np + p] < 0)) --p;
  const int32_t l = probes[q * np + p];
  const int64_t row = list_off[l] + (pos - pb[p]);
  const uint32_t hi = (uint32_t)(key >> 32);
  if (kind == 1)
    os[i] = -(int32_t)(hi ^ 0x80000000u);  // the score
  else if (kind == 2)
    of[i] = sqrtf(vsk_ord2f(hi));  // ADC sum -> its square root
  else
    of[i] = vsk_ord2f(hi);
  out_ids[i] = ids[row];
}

// ---------------------------------------------------------------------------
// The list scan through the bf16 matrix cores (IVF-Flat, L2 and L2^2).  The
// flat screen's argument carries over: with bf16 planes of the rows and the
// queries, every (query, candidate) pair gets a screened distance a within
// eps(q) of the exact one (flat_screen.hip); the kc smallest screened keys
// per query are kept, the bound check proves they hold the exact top k (or
// the query's whole candidate set is rescored), and only the kept keys
// within the margin get their exact distances -- the reference's sequential
// fp32 sums -- with their (distance, position) keys unchanged in form.
// ---------------------------------------------------------------------------
typedef __bf16 bf8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

// one workgroup per group of up to 128 queries probing one list, two
// halves of 4 waves with 64 queries each (the second half reads the rows
// the first just read, from cache).  A is the half's query fragments (4
// tiles of 16 queries x KS k-steps of 32 dims, held in registers for the
// whole list), B a 16-row block of the list's plane, so lane l of a product
// holds query 4 (l / 16) + r of the tile against row l % 16 of the block:
// 16 lanes write 16 consecutive values of one query.  Wave w of a half
// takes the list's blocks w, w + 4, ...  Each screened
// distance goes, as its order-preserving 32-bit word, to its candidate
// position in the query's word segment, out[wseg[q] + position].
//
// DENSE: the same over one block of rows for every query -- the probe's
// screen over the centroids: workgroup b takes rows 256 (b % nchunks) ..
// (at most 256, below nrows) for queries 128 (b / nchunks) .. (below nq),
// writing out[q * wstride + row].
struct DenseScreen {
  int64_t nq, nrows, wstride;
  int32_t nchunks;
};
// CMP: only the candidates whose word is at most the query's bound qlim[q]
// are kept, compactly: a pair's first pcnt[pair] words from the start of
// its place in the query's word segment, with their rows' offsets in the
// list at the same places of prow (the order is that of the workgroup's
// atomics; the tail's keys carry the positions)
struct ScreenKeep {
  const uint32_t *qlim = nullptr;
  int32_t *pcnt = nullptr;
  uint32_t *prow = nullptr;
};
constexpr int kScreenQ = 128;  // queries per screen workgroup: 2 halves of 4 waves
template <int KS, bool DENSE, int PL, bool CMP = false>
__global__ __launch_bounds__(512) void k_list_screen(
    const uint16_t *xplane, const float *xsq, int32_t ldb, const int64_t *list_off,
    const uint16_t *qplane, const uint16_t *qlo, const float *qsq, const int32_t *pairs,
    const int4 *groups,
    const int64_t *ngroups, int32_t np, const int64_t *pos_base, const int64_t *wseg,
    uint32_t *out, DenseScreen ds, ScreenKeep keep = ScreenKeep{}) {
  static_assert(!(CMP && DENSE), "the probe's screen keeps every word");
  if (!DENSE && blockIdx.x >= *ngroups) return;
  __shared__ int64_t s_out[kScreenQ];  // value address of the list's first row (-1: none)
  __shared__ float s_qa[kScreenQ];     // |q|^2
  // CMP: per slot, the query's bound, the pair and its kept count
  __shared__ uint32_t s_lim[CMP ? kScreenQ : 1];
  __shared__ int32_t s_pid[CMP ? kScreenQ : 1], s_n[CMP ? kScreenQ : 1];
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3, half = threadIdx.x >> 8;
  int64_t v0, v1, q0 = 0;
  int npair;
  int4 g{};
  if constexpr (DENSE) {
    v0 = 256 * (int64_t)(blockIdx.x % ds.nchunks);
    v1 = v0 + 256 < ds.nrows ? v0 + 256 : ds.nrows;
    q0 = kScreenQ * (int64_t)(blockIdx.x / ds.nchunks);
    npair = ds.nq - q0 < kScreenQ ? (int)(ds.nq - q0) : kScreenQ;
  } else {
    g = groups[blockIdx.x];
    v0 = list_off[g.x];
    v1 = list_off[g.x + 1];
    npair = g.z;
  }
  // the query of slot j (slots past npair repeat the first)
  auto query = [&](int j) -> int64_t {
    if constexpr (DENSE) return q0 + (j < npair ? j : 0);
    return pairs[g.y + (j < npair ? j : 0)] / np;
  };
  if (threadIdx.x < kScreenQ) {
    const int j = threadIdx.x;
    const int64_t q = query(j);
    if constexpr (DENSE) {
      s_out[j] = j < npair ? q * ds.wstride + v0 : -1;
    } else {
      const int32_t pid = pairs[g.y + (j < npair ? j : 0)];
      s_out[j] = j < npair ? wseg[q] + pos_base[pid] : -1;
      if constexpr (CMP) {
        s_lim[j] = keep.qlim[q];
        s_pid[j] = pid;
        s_n[j] = 0;
      }
    }
    s_qa[j] = qsq[q];
  }
  const int kc = 8 * (lane >> 4);  // this lane's 8 dims of a k-step
  // ALLQ (the query planes in LDS, the list scan): each of the 8 waves
  // takes every query tile of the group for its row blocks (a row block
  // loaded once a workgroup, half as many a wave); otherwise each half's 4
  // waves take its 64 queries, slots 64 half + 16 t
  constexpr bool ALLQ = PL == 2 && !DENSE;
  constexpr int TPW = ALLQ ? 8 : 4;  // query tiles a wave
  const int hbase = ALLQ ? 0 : 64 * half;
  const int ntile = npair - hbase <= 0 ? 0 : (npair - hbase + 15) >> 4;
  const int wrow = ALLQ ? (int)(threadIdx.x >> 6) : w;  // the wave's first row block
  constexpr int RSTEP = ALLQ ? 128 : 64;
  // one plane: the half's query fragments in registers; two planes: both
  // planes of the group's queries in LDS (the registers of both would halve
  // the waves a SIMD holds), rows padded by 16 bytes so that the 16 lanes
  // reading one fragment (16 queries, one column) touch distinct banks
  bf8v qf[PL == 1 ? 4 : 1][PL == 1 ? KS : 1];
  if constexpr (PL == 1) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = hbase + 16 * t + (lane & 15);
      const int64_t q = query(j);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[t][ks] = *reinterpret_cast<const bf8v *>(qplane + q * ldb + 32 * ks + kc);
    }
  }
  constexpr int QLP = PL == 2 ? 32 * KS + 8 : 8;  // row pitch in bf16
  __shared__ __attribute__((aligned(16))) uint16_t s_qh[PL == 2 ? kScreenQ * QLP : 8];
  __shared__ __attribute__((aligned(16))) uint16_t s_ql[PL == 2 ? kScreenQ * QLP : 8];
  if constexpr (PL == 2) {
    constexpr int CH = 4 * KS;  // 16-byte chunks a row
    // the rows of the group's query tiles (slots past them are never read)
    const int nrow = (npair + 15) & ~15;
    for (int e = threadIdx.x; e < nrow * CH; e += 512) {
      const int j = e / CH, c = e - j * CH;
      const int64_t qo = query(j) * ldb + 8 * c;
      *reinterpret_cast<bf8v *>(s_qh + j * QLP + 8 * c) =
          *reinterpret_cast<const bf8v *>(qplane + qo);
      *reinterpret_cast<bf8v *>(s_ql + j * QLP + 8 * c) =
          *reinterpret_cast<const bf8v *>(qlo + qo);
    }
  }
  __syncthreads();
  if (!CMP && ntile == 0) return;  // (after the block's only barrier)
  for (int64_t b = v0 + 16 * wrow; ntile > 0 && b < v1; b += RSTEP) {
    const int64_t row = b + (lane & 15);
    const bool live = row < v1;
    bf8v xf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      xf[ks] = live ? *reinterpret_cast<const bf8v *>(xplane + row * ldb + 32 * ks + kc)
                    : bf8v{};
    const float xa = live ? xsq[row] : 0.f;
    const int64_t i = row - v0;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      if (t >= ntile) break;  // uniform
      f4v acc = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if constexpr (PL == 1) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[t][ks], xf[ks], acc, 0, 0, 0);
        } else {
          const int off = (hbase + 16 * t + (lane & 15)) * QLP + 32 * ks + kc;
          const bf8v hi = *reinterpret_cast<const bf8v *>(s_qh + off);
          const bf8v lo = *reinterpret_cast<const bf8v *>(s_ql + off);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, xf[ks], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, xf[ks], acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = hbase + 16 * t + 4 * (lane >> 4) + r;
        const int64_t o = s_out[j];
        const uint32_t word = vsk_f2ord(fmaxf(s_qa[j] + xa - 2.0f * acc[r], 0.0f));
        if constexpr (CMP) {
          if (live && o >= 0 && word <= s_lim[j]) {
            const int slot = atomicAdd(&s_n[j], 1);  // < the list's rows
            out[o + slot] = word;
            keep.prow[o + slot] = (uint32_t)i;
          }
        } else {
          if (live && o >= 0) out[o + i] = word;
        }
      }
    }
  }
  if constexpr (CMP) {
    __syncthreads();
    if (threadIdx.x < npair) keep.pcnt[s_pid[threadIdx.x]] = s_n[threadIdx.x];
  }
}

// exact keys for screened ones: key (a, position) -> (the reference's
// sequential fp32 distance, position), the same sum as k_list_scan (and,
// sqrt taken, as the exact centroid scan).  Query q's keys are the first
// cnt[q] of in[q*in_stride ...], written to out[q*in_stride ...]; or (cnt
// null) every position of the query's candidates gets its exact key in
// place, at in[seg_off[q] + position] (or in[q*all_n + position], all_n
// positions each, without seg_off); only queries with active[q].  One wave
// per query, a key per lane; each lane loads 64 floats of its row and of
// the query ahead of their sequential sum.  With list_off, a position maps
// to its probe slot -- the last one whose base is at or below it, which
// holds at least one row past the base -- and so to the row; without, the
// position is the row.
struct RescoreArgs {
  const float *rows;
  int32_t ld;
  const int64_t *list_off;
  const float *Q;
  const int32_t *probes;
  int32_t np;
  const int64_t *pos_base;
  uint64_t *in;
  int64_t in_stride;
  const int32_t *cnt;
  const int64_t *seg_off;
  int64_t all_n;
  uint64_t *out;
  const uint8_t *active;
  int64_t nq;
  int32_t squared;
  // every-candidate mode (cnt null): a candidate whose screened word, at
  // words[wseg[q] + position], is kWordNone (excluded by the row filter)
  // gets the NONE key (words null: none are excluded)
  const uint32_t *words;
  const int64_t *wseg;
};
__global__ __launch_bounds__(256) void k_list_rescore(RescoreArgs a) {
#pragma clang fp contract(off)
  const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (q >= a.nq || !a.active[q]) return;
  const int32_t ld = a.ld;
  const uint64_t *src = a.cnt ? a.in + q * a.in_stride : nullptr;
  uint64_t *dst = a.cnt ? a.out + q * a.in_stride
                        : a.in + (a.seg_off ? a.seg_off[q] : q * a.all_n);
  const int64_t n = a.cnt ? (int64_t)a.cnt[q]
                          : (a.seg_off ? a.seg_off[q + 1] - a.seg_off[q] : a.all_n);
  const float *qq = a.Q + q * ld;
  const int64_t *pb = a.list_off ? a.pos_base + q * a.np : nullptr;
  const int32_t *pr = a.list_off ? a.probes + q * a.np : nullptr;
  const uint32_t *W = !src && a.words ? a.words + a.wseg[q] : nullptr;
  for (int64_t i = lane; i < n; i += 64) {
    const int64_t p = src ? (int64_t)(uint32_t)src[i] : i;
    if (W && W[p] == kWordNone) {
      dst[i] = VSK_KEY_NONE;
      continue;
    }
    int64_t row = p;
    if (a.list_off) {
      int lo = 0, hi = a.np;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pb[mid] <= p) lo = mid;
        else hi = mid;
      }
      row = a.list_off[pr[lo]] + (p - pb[lo]);
    }
    const float *x = a.rows + row * ld;
    float acc = 0.f;
    for (int c0 = 0; c0 < ld; c0 += 64) {
      const int m = ld - c0 < 64 ? (ld - c0) >> 2 : 16;  // ld is a multiple of 4
      f4 xv[16], qv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < m) {
          xv[u] = *reinterpret_cast<const f4 *>(x + c0 + 4 * u);
          qv[u] = *reinterpret_cast<const f4 *>(qq + c0 + 4 * u);
        }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < m) {
          float t;
          t = qv[u].x - xv[u].x;
          acc = acc + t * t;
          t = qv[u].y - xv[u].y;
          acc = acc + t * t;
          t = qv[u].z - xv[u].z;
          acc = acc + t * t;
          t = qv[u].w - xv[u].w;
          acc = acc + t * t;
        }
    }
    dst[i] = vsk_key(a.squared ? acc : sqrtf(acc), (uint32_t)p);
  }
}

static unsigned grid1(int64_t n, int threads = 256) {
  int64_t g = ceil_div(n, threads);
  return (unsigned)(g < 65535 * 16 ? (g > 0 ? g : 1) : 65535 * 16);
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
static FlatArgs centroid_args(const vsk_ivf *ivf, const float *dq, int64_t nq) {
  FlatArgs a{};
  a.X = ivf->centroids.x.as<float>();
  a.ldx = ivf->ld;
  a.Q = dq;
  a.ldq = ivf->ld;
  a.kdim = ivf->ld;
  a.nq = (int32_t)nq;
  a.r0 = 0;
  a.r1 = ivf->nlist;
  a.metric = METRIC_L2_EXACT;
  return a;
}

// nearest centroid of every row (strict '<', first minimum): the bf16
// screen with exact recomputation for large problems, else the exact VALU
// scan
static void ivf_assign_device(vsk_ctx *ctx, const vsk_ivf *ivf, const float *dx,
                              int64_t n, int32_t *out) {
  if (screen_argmin_applies(ctx, n, ivf->nlist, ivf->d)) {
    const ArgminQueries qp = argmin_queries(ctx, dx, n, ivf->d, ivf->ld, "ivf.aq");
    float *dist = static_cast<float *>(ctx->scratch_ptr("ivf.adist", sizeof(float) * (size_t)n));
    screen_argmin(ctx, ivf->centroids.x.as<float>(), ivf->centroids.sqnorm.as<float>(),
                  ivf->nlist, ivf->d, ivf->ld, dx, n, qp, out, dist);
    return;
  }
  const int64_t chunk = 1 << 24;  // rows per launch (grid.x bound)
  for (int64_t r = 0; r < n; r += chunk) {
    int64_t m = n - r < chunk ? n - r : chunk;
    FlatArgs a = centroid_args(ivf, dx + r * ivf->ld, m);
    launch_flat(ctx, a, MODE_ARGMIN, out + r);
  }
}

static void ivf_probe_exact(vsk_ctx *ctx, const vsk_ivf *ivf, const float *dq,
                            int64_t nq, int32_t np, uint64_t *keys);
static ArgminQueries screen_queries(vsk_ctx *ctx, const float *dq, int64_t nq, int32_t d,
                                    int32_t ld);
static void probe_screen(vsk_ctx *ctx, const vsk_ivf *ivf, const float *dq, int64_t nq,
                         int32_t np, const ArgminQueries &qp, uint64_t *keys);

// whether the probe goes through the bf16 screen over the centroids: at
// most 256 dims, enough work (forced by VSK_FLAT_KERNEL=screen, off by
// =exact / =bf16x3 / =fp32)
static bool probe_screen_applies(vsk_ctx *ctx, const vsk_ivf *ivf, int64_t nq, int32_t np) {
  if (ctx->flat_no_screen || ctx->flat_fp32 || ctx->exact_only) return false;
  if (ivf->d > 256 || np > VSK_MAX_K) return false;
  return ctx->flat_force_screen ||
         (double)nq * (double)ivf->nlist * (double)ivf->d >= (double)(1ll << 30);
}

// top-nprobe centroids per query (ties by centroid index); qp: the
// queries' bf16 planes when the caller has them.  With keys_out, the
// ranked (distance, centroid) keys are left there and probes is not
// written (the search turns them into ids itself).
static void ivf_probe_device(vsk_ctx *ctx, const vsk_ivf *ivf, const float *dq,
                             int64_t nq, int32_t np, int32_t *probes,
                             const ArgminQueries *qp = nullptr,
                             uint64_t **keys_out = nullptr) {
  uint64_t *keys = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.probe_keys", sizeof(uint64_t) * nq * np));
  if (probe_screen_applies(ctx, ivf, nq, np)) {
    if (qp) {
      probe_screen(ctx, ivf, dq, nq, np, *qp, keys);
    } else {
      const ArgminQueries own = screen_queries(ctx, dq, nq, ivf->d, ivf->ld);
      probe_screen(ctx, ivf, dq, nq, np, own, keys);
    }
  } else {
    ivf_probe_exact(ctx, ivf, dq, nq, np, keys);
  }
  if (keys_out) {
    *keys_out = keys;
    return;
  }
  KernelTimer t(ctx, "ivf_probe_ids");
  k_keys_to_tie<<<grid1(nq * np), 256, 0, ctx->stream>>>(keys, nq * np, probes);
  check_launch("ivf_probe_ids");
}

// the exact VALU scan over every centroid, one dense chunk per query batch
static void ivf_probe_exact(vsk_ctx *ctx, const vsk_ivf *ivf, const float *dq,
                            int64_t nq, int32_t np, uint64_t *keys) {
  const int64_t cap = ivf->nlist;  // one dense chunk
  const int64_t qb = query_batch(ctx, nq, cap);
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    FlatArgs base = centroid_args(ivf, dq + b0 * ivf->ld, nb);
    ScanFn scan = [&](const ScanRequest &r) {
      FlatArgs a = base;
      a.r0 = r.r0;
      a.r1 = r.r1;
      a.thresh = r.thresh;
      a.active = r.active;
      a.cand = r.cand;
      a.cap = r.cap;
      a.counts = r.counts;
      launch_flat(ctx, a, r.dense ? MODE_DENSE : MODE_FILTER, nullptr);
    };
    progressive_topk(ctx, nb, ivf->nlist, np, cap, scan, keys + b0 * np,
                     "ivf_probe_select");
  }
}

// every centroid of each query ranked by (exact sqrt-L2, centroid): the
// exact VALU scan's dense keys, sorted per query (batches of at most 2^26
// keys), written as the probe list probes[nq][nlist]
static void ivf_rank_all(vsk_ctx *ctx, const vsk_ivf *ivf, const float *dq, int64_t nq,
                         int32_t *probes) {
  const int64_t nl = ivf->nlist;
  const int64_t qb = std::max<int64_t>(1, std::min<int64_t>(nq, tile_keys(ctx, 1ll << 26, 16) / nl));
  uint64_t *k0 = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.rank0", sizeof(uint64_t) * (size_t)(qb * nl)));
  uint64_t *k1 = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.rank1", sizeof(uint64_t) * (size_t)(qb * nl)));
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    FlatArgs a = centroid_args(ivf, dq + b0 * ivf->ld, nb);
    a.cand = k0;
    a.cap = nl;
    launch_flat(ctx, a, MODE_DENSE, nullptr);
    segmented_sort_u64(ctx, k0, k1, nb, nl);
    KernelTimer t(ctx, "ivf_probe_ids");
    k_keys_to_tie<<<grid1(nb * nl), 256, 0, ctx->stream>>>(k1, nb * nl, probes + b0 * nl);
    check_launch("ivf_probe_ids");
  }
}

// the queries as two bf16 planes for the screens: hi = bf16(q), lo =
// bf16(q - hi) (ldb columns, zero padded), |hi| + |lo| and |q - hi - lo|
// (sums of squares in double, square roots rounded up), one wave per query
__global__ __launch_bounds__(256) void k_query_planes2(const float *Q, int64_t nq, int32_t d,
                                                       int32_t ld, int32_t ldb, uint16_t *hi,
                                                       uint16_t *lo, float *nh, float *nr,
                                                       float *nh1, float *nr1) {
#pragma clang fp contract(off)
  const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (q >= nq) return;
  double sh = 0.0, sl = 0.0, sr = 0.0, s1 = 0.0;
  for (int c = lane; c < ldb; c += 64) {
    const float v = c < d ? Q[q * ld + c] : 0.f;
    const uint16_t h = bf16_rn(v);
    const float hv = __uint_as_float((uint32_t)h << 16);
    const float rv = v - hv;  // exact
    const uint16_t l = bf16_rn(rv);
    const float lv = __uint_as_float((uint32_t)l << 16);
    const float r2 = rv - lv;  // exact
    hi[q * ldb + c] = h;
    lo[q * ldb + c] = l;
    sh += (double)hv * (double)hv;
    sl += (double)lv * (double)lv;
    sr += (double)r2 * (double)r2;
    s1 += (double)rv * (double)rv;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    sh += __shfl_xor(sh, o);
    sl += __shfl_xor(sl, o);
    sr += __shfl_xor(sr, o);
    s1 += __shfl_xor(s1, o);
  }
  if (lane == 0) {
    nh[q] = f_up((sqrt(sh) + sqrt(sl)) * (1.0 + 1e-12));
    nr[q] = f_up(sqrt(sr) * (1.0 + 1e-12));
    nh1[q] = f_up(sqrt(sh) * (1.0 + 1e-12));
    nr1[q] = f_up(sqrt(s1) * (1.0 + 1e-12));
  }
}

// The screens' query planes.  one: the hi plane with |hi| and |q - hi|;
// two (d <= 128, the lo plane's fragments fit the list screen's LDS):
// the same hi plane and a lo plane, with |hi| + |lo| and |q - hi - lo|.  The
// list scan's rescore reads about half the rows with two planes (the
// bound's query term shrinks 2^8-fold); the probe, whose margin holds few
// centroids beyond the nprobe, keeps one plane and its cheaper screen.
// |q|^2 for both.
struct ScreenQueries {
  ArgminQueries one, two;
};
static ScreenQueries screen_queries2(vsk_ctx *ctx, const float *dq, int64_t nq, int32_t d,
                                     int32_t ld) {
  ScreenQueries sq;
  if (d > 128) {
    sq.one = sq.two = argmin_queries(ctx, dq, nq, d, ld, "ivf.sq");
    return sq;
  }
  ArgminQueries qp;
  qp.ldb = (d + 63) & ~63;
  uint16_t *qh = static_cast<uint16_t *>(
      ctx->scratch_ptr("ivf.sq2.planes", sizeof(uint16_t) * 2 * (size_t)nq * qp.ldb));
  float *nrm = static_cast<float *>(ctx->scratch_ptr("ivf.sq2.norms", sizeof(float) * 5 * (size_t)nq));
  {
    KernelTimer t(ctx, "query_planes");
    k_query_planes2<<<(unsigned)ceil_div(nq, 4), 256, 0, ctx->stream>>>(
        dq, nq, d, ld, qp.ldb, qh, qh + (size_t)nq * qp.ldb, nrm, nrm + nq, nrm + 3 * nq,
        nrm + 4 * nq);
    check_launch("query_planes");
  }
  row_norms(ctx, dq, nq, d, ld, nrm + 2 * nq, nullptr);
  qp.qh = qh;
  qp.qsq = nrm + 2 * nq;
  sq.one = qp;
  sq.one.qnh = nrm + 3 * nq;
  sq.one.qnr = nrm + 4 * nq;
  sq.two = qp;
  sq.two.ql = qh + (size_t)nq * qp.ldb;
  sq.two.qnh = nrm;
  sq.two.qnr = nrm + nq;
  sq.two.nprod = 2 * d;
  return sq;
}
static ArgminQueries screen_queries(vsk_ctx *ctx, const float *dq, int64_t nq, int32_t d,
                                    int32_t ld) {
  return screen_queries2(ctx, dq, nq, d, ld).one;
}

// whether the list scan of kind 0 goes through the bf16 screen: L2 / L2^2,
// at most 256 dims (the query fragments stay in registers), k whose kept
// candidates fit a selection, and enough work to pay for the extra
// launches (forced by VSK_FLAT_KERNEL=screen, off by =exact / =bf16x3)
static bool list_screen_applies(vsk_ctx *ctx, const vsk_ivf *ivf, int32_t metric, int32_t k,
                                double ncand) {
  if (ctx->flat_no_screen || ctx->flat_fp32 || ctx->exact_only) return false;
  if (metric != VSK_METRIC_L2 && metric != VSK_METRIC_L2SQ) return false;
  if (ivf->d > 256) return false;
  return ctx->flat_force_screen || ncand * ivf->d >= (double)(1ll << 30);
}

// candidates a query can have with np probes: the sizes of the np largest
// lists summed (every row when every list is probed)
static int64_t probe_bound(const vsk_ivf *ivf, int32_t np) {
  if (np >= ivf->nlist) return ivf->total;
  std::vector<int64_t> sz(ivf->nlist);
  for (int32_t l = 0; l < ivf->nlist; ++l) sz[l] = ivf->off[l + 1] - ivf->off[l];
  std::nth_element(sz.begin(), sz.begin() + np, sz.end(), std::greater<int64_t>());
  int64_t s = 0;
  for (int32_t i = 0; i < np; ++i) s += sz[i];
  return s;
}

// the stored rows' bf16 plane (roundup(d, 64) columns), |x|^2 per row and
// the maxima of |bf16(x)| and |x - bf16(x)|, rebuilt after the rows change
// per list l, the largest fp32 distance of its rows from its centroid c_l
// (0 for an empty list; infinite when a row gives NaN): one workgroup a
// list, a wave a row at a time with the dimensions over its lanes.  The sum
// is a tree, not the reference's sequential order: any order lies within
// (d + 2) u of the real distance, which the bound's slack covers.
__global__ __launch_bounds__(256) void k_list_radius(const float *rows, int32_t ld, int32_t d,
                                                    const int64_t *list_off, const float *cent,
                                                    int32_t cld, float *rad) {
  const int64_t l = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const float *c = cent + l * cld;
  float m = 0.f;
  for (int64_t r = list_off[l] + wv; r < list_off[l + 1]; r += 4) {
    const float *x = rows + r * ld;
    float acc = 0.f;
    for (int j = lane; j < d; j += 64) {
      const float t = x[j] - c[j];
      acc = __builtin_fmaf(t, t, acc);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    m = acc == acc ? fmaxf(m, sqrtf(acc)) : __int_as_float(0x7f800000);
  }
  __shared__ float s_m[4];
  if (lane == 0) s_m[wv] = m;
  __syncthreads();
  if (threadIdx.x == 0) rad[l] = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
}

static void list_screen_plane(vsk_ctx *ctx, const vsk_ivf *ivf) {
  if (ivf->xversion == ivf->version) return;
  const int32_t ldb = (ivf->d + 63) & ~63;
  const int64_t n = std::max<int64_t>(ivf->total, 1);
  ivf->xplane.reserve(sizeof(uint16_t) * (size_t)n * ldb);
  ivf->xsq.reserve(sizeof(float) * (size_t)n);
  uint32_t *mb = static_cast<uint32_t *>(ctx->scratch_ptr("ivf.planemax", 2 * sizeof(uint32_t)));
  fill_i32(ctx, reinterpret_cast<int32_t *>(mb), 2, 0);
  split_bf16(ctx, ivf->rows.as<float>(), ivf->total, ivf->d, ivf->ld,
             ivf->xplane.as<uint16_t>(), nullptr, ldb, nullptr, nullptr, mb);
  row_norms(ctx, ivf->rows.as<float>(), ivf->total, ivf->d, ivf->ld, ivf->xsq.as<float>(),
            nullptr);
  ivf->xrad.reserve(sizeof(float) * (size_t)std::max<int32_t>(ivf->nlist, 1));
  if (ivf->nlist > 0) {
    KernelTimer t(ctx, "ivf_list_radius");
    k_list_radius<<<(unsigned)ivf->nlist, 256, 0, ctx->stream>>>(
        ivf->rows.as<float>(), ivf->ld, ivf->d, ivf->list_off.as<int64_t>(),
        ivf->centroids.x.as<float>(), ivf->centroids.ld, ivf->xrad.as<float>());
    check_launch("ivf_list_radius");
  }
  uint32_t hb[2];
  VSK_HIP(hipMemcpyAsync(hb, mb, sizeof(hb), hipMemcpyDeviceToHost, ctx->stream));
  stream_sync(ctx);
  ivf->xh_max = __builtin_bit_cast(float, hb[0]);
  ivf->xr_max = __builtin_bit_cast(float, hb[1]);
  ivf->xldb = ldb;
  ivf->xversion = ivf->version;
}

static void require_ivf(const vsk_ivf *ivf) {
  VSK_REQUIRE(ivf, VSK_ERR_INVALID_ARGUMENT, "ivf is null");
}

// the calls that read the fp32 rows
static void require_rows(const vsk_ivf *ivf) {
  VSK_REQUIRE(!ivf->codes_only, VSK_ERR_UNSUPPORTED,
              "the index holds codes only (vsk_ivf_drop_rows): search it with "
              "vsk_ivf_search_sq8 / vsk_ivf_search_pq");
}

// codes of n rows x (n x d, dense, host or device) with the index's stored
// quantizer, n x w bytes dense into out (w = d for SQ8, M for PQ)
static void encode_with_stored(vsk_ctx *ctx, const vsk_ivf *ivf, const float *x, int64_t n,
                               uint8_t *out) {
  vsk_status st = VSK_OK;
  if (ivf->ckind == 1) {
    const size_t ns = ivf->cper_dim ? (size_t)ivf->d : 1;
    st = vsk_sq8_encode(ctx, x, n, ivf->d, ivf->cper_dim, ivf->cparams.data(),
                        ivf->cparams.data() + ns, reinterpret_cast<int8_t *>(out));
  } else {
    vsk_pq *pq = nullptr;
    st = vsk_pq_create(ctx, ivf->cparams.data(), ivf->cM, ivf->cksub, ivf->cdsub, &pq);
    if (st == VSK_OK) {
      st = vsk_pq_encode(ctx, pq, x, n, out);
      vsk_pq_free(ctx, pq);
    }
  }
  if (st != VSK_OK) fail(st, "encoding the inserted rows with the index's quantizer failed");
}

}  // namespace vsk

using namespace vsk;

extern "C" {

vsk_status vsk_ivf_create(vsk_ctx *ctx, const float *centroids, int32_t nlist,
                          int32_t d, vsk_ivf **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(centroids, VSK_ERR_NOT_TRAINED, "no centroids (index not trained)");
  VSK_REQUIRE(nlist > 0, VSK_ERR_NOT_TRAINED, "nlist must be positive");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(d <= kMaxDim && nlist <= kMaxLists, VSK_ERR_INVALID_BUFFER_SIZE,
              "at most 65536 dimensions and 2^24 lists");
  std::unique_ptr<vsk_ivf> ivf(new vsk_ivf());
  ivf->nlist = nlist;
  ivf->d = d;
  ivf->ld = padded_ld(d);
  CallScope cs(ctx);
  vsk_db &c = ivf->centroids;
  c.n = nlist;
  c.d = d;
  c.ld = ivf->ld;
  c.x.reserve(sizeof(float) * (size_t)nlist * c.ld);
  const float *src = rows_to_device_padded(ctx, centroids, nlist, d, c.ld,
                                           "ivf.centroids_in");
  VSK_HIP(hipMemcpyAsync(c.x.p, src, sizeof(float) * (size_t)nlist * c.ld,
                         hipMemcpyDeviceToDevice, ctx->stream));
  c.sqnorm.reserve(sizeof(float) * nlist);
  c.norm.reserve(sizeof(float) * nlist);
  row_norms(ctx, c.x.as<float>(), nlist, d, c.ld, c.sqnorm.as<float>(),
            c.norm.as<float>());
  ivf->off.assign(nlist + 1, 0);
  ivf->list_off.reserve(sizeof(int64_t) * (nlist + 1));
  VSK_HIP(hipMemcpyAsync(ivf->list_off.p, ivf->off.data(),
                         sizeof(int64_t) * (nlist + 1), hipMemcpyHostToDevice,
                         ctx->stream));
  cs.finish();
  *out = ivf.release();
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_build(vsk_ctx *ctx, const float *centroids, int32_t nlist,
                         const float *x, const int64_t *ids, int64_t n,
                         int32_t d, vsk_ivf **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(n >= 0, VSK_ERR_INVALID_ARGUMENT, "row count is negative");
  vsk_ivf *ivf = nullptr;
  vsk_status st = vsk_ivf_create(ctx, centroids, nlist, d, &ivf);
  if (st != VSK_OK) return st;
  if (n > 0) {
    st = vsk_ivf_add(ctx, ivf, x, ids, n);
    if (st != VSK_OK) {
      // keep the add's message: free does not touch the error state
      vsk_ivf_free(ctx, ivf);
      return st;
    }
  }
  *out = ivf;
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_free(vsk_ctx *ctx, vsk_ivf *ivf) {
  if (ctx) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
  }
  delete ivf;
  return VSK_OK;
}

vsk_status vsk_ivf_assign(vsk_ctx *ctx, const vsk_ivf *ivf, const float *x,
                          int64_t n, int32_t *out_list) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no rows");
  VSK_REQUIRE(x && out_list, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  CallScope cs(ctx);
  const float *dx = rows_to_device_padded(ctx, x, n, ivf->d, ivf->ld, "ivf.x");
  OutputStage o(ctx, out_list, sizeof(int32_t) * n, "out.assign");
  ivf_assign_device(ctx, ivf, dx, n, o.ptr<int32_t>());
  o.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_add(vsk_ctx *ctx, vsk_ivf *ivf, const float *x,
                       const int64_t *ids, int64_t n) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no rows");
  VSK_REQUIRE(x, VSK_ERR_INVALID_ARGUMENT, "x is null");
  VSK_REQUIRE(ivf->total + n <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "an IVF index holds at most 2^31-1 rows");
  CallScope cs(ctx);
  const int32_t ld = ivf->ld, nlist = ivf->nlist;
  const float *dx = rows_to_device_padded(ctx, x, n, ivf->d, ld, "ivf.x");
  const int64_t *did = ids ? static_cast<const int64_t *>(input_to_device(
                                 ctx, ids, sizeof(int64_t) * n, "ivf.ids_in"))
                           : nullptr;
  int32_t *assign =
      static_cast<int32_t *>(ctx->scratch_ptr("ivf.assign", 4 * n));
  ivf_assign_device(ctx, ivf, dx, n, assign);
  std::vector<int32_t> h_assign(n);
  VSK_HIP(hipMemcpyAsync(h_assign.data(), assign, 4 * n, hipMemcpyDeviceToHost,
                         ctx->stream));
  stream_sync(ctx);

  // new CSR: old lists keep their order, new rows follow in call order
  std::vector<int64_t> add(nlist, 0);
  for (int64_t i = 0; i < n; ++i) add[h_assign[i]]++;
  std::vector<int64_t> noff(nlist + 1, 0);
  for (int32_t l = 0; l < nlist; ++l)
    noff[l + 1] = noff[l] + (ivf->off[l + 1] - ivf->off[l]) + add[l];
  const int64_t total = ivf->total + n;
  std::vector<int64_t> dest_old(ivf->total), dest_new(n);
  for (int32_t l = 0; l < nlist; ++l)
    for (int64_t r = ivf->off[l]; r < ivf->off[l + 1]; ++r)
      dest_old[r] = noff[l] + (r - ivf->off[l]);
  std::vector<int64_t> cursor(nlist);
  for (int32_t l = 0; l < nlist; ++l)
    cursor[l] = noff[l] + (ivf->off[l + 1] - ivf->off[l]);
  for (int64_t i = 0; i < n; ++i) dest_new[i] = cursor[h_assign[i]]++;

  int64_t *ddest = static_cast<int64_t *>(
      ctx->scratch_ptr("ivf.dest", sizeof(int64_t) * std::max(ivf->total, n)));
  if (ivf->codes_only) {
    // the new rows' codes with the index's own quantizer, then old and new
    // codes (and ids) to their places in the new list order
    const int32_t w = ivf->ckind == 1 ? ivf->d : ivf->cM;
    uint8_t *fresh = static_cast<uint8_t *>(ctx->scratch_ptr("ivf.newcodes", (size_t)n * w));
    encode_with_stored(ctx, ivf, x, n, fresh);
    DevBuf codes2, ids2;
    codes2.reserve((size_t)total * ivf->cstride + 16);
    fill_i32(ctx, codes2.as<int32_t>(), ((int64_t)total * ivf->cstride + 16) / 4, 0);
    ids2.reserve(sizeof(int64_t) * total);
    if (ivf->total > 0) {
      VSK_HIP(hipMemcpyAsync(ddest, dest_old.data(), 8 * ivf->total, hipMemcpyHostToDevice,
                             ctx->stream));
      k_scatter_codes<<<grid1(ivf->total, 4), 256, 0, ctx->stream>>>(
          ivf->codes.as<uint8_t>(), ivf->cstride, ivf->cstride, ivf->ids.as<int64_t>(), 0,
          ddest, ivf->total, ivf->cstride, codes2.as<uint8_t>(), ids2.as<int64_t>());
      check_launch("ivf_scatter_old_codes");
      stream_sync(ctx);
    }
    VSK_HIP(hipMemcpyAsync(ddest, dest_new.data(), 8 * n, hipMemcpyHostToDevice, ctx->stream));
    k_scatter_codes<<<grid1(n, 4), 256, 0, ctx->stream>>>(
        fresh, w, w, did, ivf->next_id, ddest, n, ivf->cstride, codes2.as<uint8_t>(),
        ids2.as<int64_t>());
    check_launch("ivf_scatter_new_codes");
    VSK_HIP(hipMemcpyAsync(ivf->list_off.p, noff.data(), sizeof(int64_t) * (nlist + 1),
                           hipMemcpyHostToDevice, ctx->stream));
    stream_sync(ctx);
    std::swap(ivf->codes.p, codes2.p);
    std::swap(ivf->codes.bytes, codes2.bytes);
    std::swap(ivf->ids.p, ids2.p);
    std::swap(ivf->ids.bytes, ids2.bytes);
    ++ivf->version;
    ivf->off = noff;
    ivf->total = total;
    ivf->ctotal = total;
    ivf->next_id += n;
    cs.finish();
    return VSK_OK;
  }
  auto rows2 = std::make_unique<DevBuf>();
  auto ids2 = std::make_unique<DevBuf>();
  rows2->reserve(sizeof(float) * (size_t)total * ld);
  ids2->reserve(sizeof(int64_t) * total);
  if (ivf->total > 0) {
    VSK_HIP(hipMemcpyAsync(ddest, dest_old.data(), 8 * ivf->total,
                           hipMemcpyHostToDevice, ctx->stream));
    k_scatter_rows<<<grid1(ivf->total, 4), 256, 0, ctx->stream>>>(
        ivf->rows.as<float>(), ivf->ids.as<int64_t>(), 0, ddest, ivf->total,
        ld, rows2->as<float>(), ids2->as<int64_t>());
    check_launch("ivf_scatter_old");
    stream_sync(ctx);
  }
  VSK_HIP(hipMemcpyAsync(ddest, dest_new.data(), 8 * n, hipMemcpyHostToDevice,
                         ctx->stream));
  k_scatter_rows<<<grid1(n, 4), 256, 0, ctx->stream>>>(
      dx, did, ivf->next_id, ddest, n, ld, rows2->as<float>(),
      ids2->as<int64_t>());
  check_launch("ivf_scatter_new");
  VSK_HIP(hipMemcpyAsync(ivf->list_off.p, noff.data(),
                         sizeof(int64_t) * (nlist + 1), hipMemcpyHostToDevice,
                         ctx->stream));
  stream_sync(ctx);
  std::swap(ivf->rows.p, rows2->p);
  std::swap(ivf->rows.bytes, rows2->bytes);
  ++ivf->version;
  std::swap(ivf->ids.p, ids2->p);
  std::swap(ivf->ids.bytes, ids2->bytes);
  ivf->off = noff;
  ivf->total = total;
  ivf->next_id += n;
  cs.finish();
  VSK_API_END(ctx);
}

static vsk_status ivf_probe_body(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                         int64_t nq, int32_t nprobe, int32_t *out_lists) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(q && out_lists, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(nprobe >= 1 && nprobe <= VSK_MAX_K, VSK_ERR_INVALID_ARGUMENT,
              "nprobe must be in [1, VSK_MAX_K]");
  CallScope cs(ctx);
  const float *dq = rows_to_device_padded(ctx, q, nq, ivf->d, ivf->ld, "ivf.q");
  OutputStage o(ctx, out_lists, sizeof(int32_t) * nq * nprobe, "out.probes");
  ivf_probe_device(ctx, ivf, dq, nq, nprobe, o.ptr<int32_t>());
  o.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

// top-k overflow is checked at the call's end (topk_call)
vsk_status vsk_ivf_probe(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                         int64_t nq, int32_t nprobe, int32_t *out_lists) {
  return topk_call(ctx, [&] { return ivf_probe_body(ctx, ivf, q, nq, nprobe, out_lists); });
}

vsk_status vsk_ivf_list_sizes(vsk_ctx *ctx, const vsk_ivf *ivf,
                              int64_t *sizes) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(sizes, VSK_ERR_INVALID_ARGUMENT, "sizes is null");
  for (int32_t l = 0; l < ivf->nlist; ++l)
    sizes[l] = ivf->off[l + 1] - ivf->off[l];
  VSK_API_END(ctx);
}

}  // extern "C"

// the pair and group arrays of a batch (sized for the largest batch)
struct ListGroups {
  int32_t *lcnt;            // pairs per list
  int64_t *lstart, *gstart;  // nlist + 1 each
  int32_t *rank;            // each pair's rank in its list
  int32_t *pairs;
  int4 *groups;
};

// the batch's pairs grouped by list, up to G a group (the group count in
// gstart[nlist]), and its candidate segment offsets: counts and ranks, the
// offsets of both in one launch, then the scatter (pairs null: the offsets
// only)
static void batch_groups(vsk_ctx *ctx, const vsk_ivf *ivf, const int32_t *probes,
                         int64_t npairs, const int64_t *cnt, int64_t nb, int64_t *dseg,
                         int64_t *wseg, int G, const ListGroups &lg) {
  const int32_t nlist = ivf->nlist;
  const bool lists = lg.pairs != nullptr;
  if (lists) {
    // (lcnt starts cleared: by the probe bases for the first batch, by the
    // previous batch's scatter after it)
    KernelTimer t(ctx, "ivf_pair_counts");
    if ((int64_t)nlist * 4 <= 64 * 1024 && npairs >= 8192) {
      // about 16 workgroups, each with at least 4,096 pairs
      const int64_t per = std::max<int64_t>(4096, ceil_div(ceil_div(npairs, 16), 1024) * 1024);
      k_list_pair_counts_lds<<<(unsigned)ceil_div(npairs, per), 1024, sizeof(int32_t) * nlist,
                               ctx->stream>>>(probes, npairs, per, lg.lcnt, lg.rank, nlist);
    } else {
      k_list_pair_counts<<<grid1(npairs), 256, 0, ctx->stream>>>(probes, npairs, lg.lcnt,
                                                                  lg.rank);
    }
    check_launch("ivf_list_pair_counts");
  }
  {
    KernelTimer t(ctx, "ivf_batch_offsets");
    k_batch_offsets<<<lists ? 2 : 1, 1024, 0, ctx->stream>>>(
        cnt, nb, dseg, wseg, lg.lcnt, ivf->list_off.as<int64_t>(), nlist, G, lg.lstart,
        lg.gstart, lg.groups);
    check_launch("ivf_batch_offsets");
  }
  if (lists) {
    KernelTimer t(ctx, "ivf_group_pairs");
    k_group_pairs<<<grid1(npairs), 256, 0, ctx->stream>>>(probes, npairs, lg.lstart, lg.rank,
                                                          lg.pairs, lg.lcnt, nlist);
    check_launch("ivf_group_pairs");
  }
}

// the row filter over a batch's candidate words (k_mask_words)
static void mask_words(vsk_ctx *ctx, const int32_t *probes, int32_t np, const int64_t *pos_base,
                       const vsk_ivf *ivf, const int64_t *wseg, const uint32_t *lmask,
                       uint32_t *words, int64_t nb) {
  KernelTimer t(ctx, "ivf_mask_words");
  k_mask_words<<<(unsigned)nb, 256, 0, ctx->stream>>>(
      probes, np, pos_base, ivf->list_off.as<int64_t>(), wseg, lmask, words, nb);
  check_launch("ivf_mask_words");
}

// one query batch of the screened list scan: the screened distance of
// every candidate (a 32-bit word at its position in the query's word
// segment, wseg), the keys within the margin of the k-th screened distance
// (at most cap per query), their exact distances and the top k of those --
// or, for a query with more than cap keys in the margin, the top k of
// every candidate's exact distance (in its segment of cand, seg_off) --
// into best[b0 * k ...].  Up to k = 256 one launch after the screen does
// all of that per query (k_screen_tail); above, the margin, rescore and
// selections are launches of their own, the fallback's finding no active
// query when none overflows.  No read-back either way.
static void list_screen_batch(vsk_ctx *ctx, const vsk_ivf *ivf, const ArgminQueries &qp,
                              const float *dq, int64_t b0, int64_t nb, int32_t np, int32_t k,
                              int32_t metric, const int32_t *probes, const int64_t *pos_base,
                              const int64_t *cnt, const int64_t *dseg, const int64_t *wseg,
                              const ListGroups &lg, uint32_t *words, uint64_t *cand,
                              uint64_t *best, const uint32_t *lmask,
                              const ScreenKeep *keep) {
  const int32_t ld = ivf->ld, ldb = ivf->xldb, nlist = ivf->nlist;
  const int64_t npairs = nb * np;
  const int32_t *bprobes = probes + b0 * np;
  const int64_t *bpos = pos_base + b0 * np;
  {
    KernelTimer t(ctx, "ivf_list_screen");
    t.device_work(dseg + nb);
    const unsigned gmax =
        (unsigned)(std::min<int64_t>(nlist, npairs) + ceil_div(npairs, kScreenQ));
    // (compact: the batch's bounds, the pair counts and row offsets)
    ScreenKeep kb;
    if (keep) kb = ScreenKeep{keep->qlim + b0, keep->pcnt, keep->prow};
#define VSK_LS1(KS, PL, CMP)                                                                \
  k_list_screen<KS, false, PL, CMP><<<gmax, 512, 0, ctx->stream>>>(                        \
      ivf->xplane.as<uint16_t>(), ivf->xsq.as<float>(), ldb, ivf->list_off.as<int64_t>(),   \
      qp.qh + b0 * qp.ldb, qp.ql ? qp.ql + b0 * qp.ldb : nullptr, qp.qsq + b0, lg.pairs,    \
      lg.groups, lg.gstart + nlist, np, bpos, wseg, words, DenseScreen{}, kb)
#define VSK_LS(KS, PL)         \
  do {                         \
    if (keep)                  \
      VSK_LS1(KS, PL, true);   \
    else                       \
      VSK_LS1(KS, PL, false);  \
  } while (0)
    switch (ldb / 32) {
    case 2: if (qp.ql) VSK_LS(2, 2); else VSK_LS(2, 1); break;
    case 4: if (qp.ql) VSK_LS(4, 2); else VSK_LS(4, 1); break;
    case 6: VSK_LS(6, 1); break;
    default: VSK_LS(8, 1); break;
    }
#undef VSK_LS
#undef VSK_LS1
    check_launch("ivf_list_screen");
  }
  if (lmask) mask_words(ctx, bprobes, np, bpos, ivf, wseg, lmask, words, nb);
  const int32_t sq = metric == VSK_METRIC_L2SQ ? 1 : 0;
  const float *rows = ivf->rows.as<float>();
  const int64_t *loff = ivf->list_off.as<int64_t>();
  // the overflowing queries' count as the fallback's work (profiling)
  int64_t *nbad =
      ctx->count_work() ? static_cast<int64_t *>(ctx->scratch_ptr("ivf.nbad", 8)) : nullptr;
  if (nbad) fill_i32(ctx, reinterpret_cast<int32_t *>(nbad), 2, 0);
  MarginArgs ma;
  ma.nq = nb;
  ma.k = k;
  ma.words = words;
  ma.wseg = wseg;
  ma.cnt = cnt + b0;
  ma.qnh = qp.qnh + b0;
  ma.qnr = qp.qnr + b0;
  ma.xh = ivf->xh_max;
  ma.xr = ivf->xr_max;
  ma.d = ivf->d;
  ma.nprod = qp.nprod;
  ma.metric = metric;
  ma.nbad = reinterpret_cast<unsigned long long *>(nbad);
  if (k <= 256) {
    // the margin, its exact rescore and the selection in one launch
    ScreenTailArgs ta;
    ta.m = ma;
    ta.m.cap = 1024;
    ta.rows = rows;
    ta.Q = dq + b0 * ld;
    ta.ld = ld;
    ta.squared = sq;
    ta.list_off = loff;
    ta.pos_base = bpos;
    ta.probes = bprobes;
    ta.np = np;
    ta.all = cand;
    ta.seg_off = dseg;
    ta.best_out = best + b0 * k;
    if (keep) {
      ta.pcnt = keep->pcnt;
      ta.prow = keep->prow;
    }
    KernelTimer t(ctx, "ivf_screen_tail");
    if (nbad) t.device_work(nbad);
    launch_screen_tail(ctx, ta, "screen_tail");
    return;
  }
  const int32_t cap = 4 * k;
  uint64_t *kept = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.kept", sizeof(uint64_t) * nb * cap));
  uint64_t *exact = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.kexact", sizeof(uint64_t) * nb * cap));
  uint8_t *ok = static_cast<uint8_t *>(ctx->scratch_ptr("ivf.ok", 2 * (size_t)nb));
  uint8_t *bad = ok + nb;
  int32_t *nout = static_cast<int32_t *>(ctx->scratch_ptr("ivf.nout", 4 * (size_t)nb + 8));
  ma.out = kept;
  ma.cap = cap;
  ma.nout = nout;
  ma.ok = ok;
  ma.bad = bad;
  launch_screen_margin(ctx, ma);
  RescoreArgs ra{};
  ra.rows = rows;
  ra.ld = ld;
  ra.list_off = loff;
  ra.Q = dq + b0 * ld;
  ra.probes = bprobes;
  ra.np = np;
  ra.pos_base = bpos;
  ra.nq = nb;
  ra.squared = sq;
  {
    KernelTimer t(ctx, "ivf_screen_rescore");
    RescoreArgs r = ra;
    r.in = kept;
    r.in_stride = cap;
    r.cnt = nout;
    r.out = exact;
    r.active = ok;
    k_list_rescore<<<(unsigned)ceil_div(nb, 4), 256, 0, ctx->stream>>>(r);
    check_launch("ivf_screen_rescore");
  }
  {
    SelectArgs sa;
    sa.nq = nb;
    sa.k = k;
    sa.cand = exact;
    sa.cap = cap;
    sa.counts = nout;
    sa.active = ok;
    sa.regs = cap <= 8192;
    sa.small = cap <= 1024;
    sa.best_out = best + b0 * k;
    launch_select(ctx, sa, "ivf_select");
  }
  // queries with more than cap keys in the margin: every candidate exact
  {
    KernelTimer t(ctx, "ivf_screen_redo");
    if (nbad) t.device_work(nbad);
    RescoreArgs r = ra;
    r.in = cand;
    r.seg_off = dseg;
    r.active = bad;
    r.words = words;
    r.wseg = wseg;
    k_list_rescore<<<(unsigned)ceil_div(nb, 4), 256, 0, ctx->stream>>>(r);
    check_launch("ivf_screen_redo");
  }
  SelectArgs sa;
  sa.nq = nb;
  sa.k = k;
  sa.cand = cand;
  sa.seg_off = dseg;
  sa.active = bad;
  sa.best_out = best + b0 * k;
  launch_select(ctx, sa, "ivf_select");
}

namespace vsk {

// The probe through the bf16 screen: the screened distance of every (query,
// centroid) as a 32-bit word, the keys within the margin of the np-th
// screened distance, their exact sqrt-L2 (dimension order, the exact
// scan's own sum) keyed (distance, centroid) and the top np of those; a
// query with more than cap keys in the margin has every centroid's exact
// key ranked instead.  No read-back.
static void probe_screen(vsk_ctx *ctx, const vsk_ivf *ivf, const float *dq, int64_t nq,
                         int32_t np, const ArgminQueries &qp, uint64_t *keys) {
  const vsk_db *cdb = &ivf->centroids;
  make_split(ctx, cdb, dq, 0, false, nullptr, nullptr);  // the centroids' planes
  const int32_t nlist = ivf->nlist, ld = ivf->ld, ldb = cdb->ldb;
  const int64_t wstride = ceil_div(nlist, 4) * 4;
  // batches whose words and fallback keys stay under 1 GiB
  const int64_t qb =
      std::max<int64_t>(1, std::min<int64_t>(nq, tile_keys(ctx, 1ll << 27, 12) / wstride));
  const int32_t cap = std::max<int32_t>(1024, 4 * np);
  uint32_t *words = static_cast<uint32_t *>(
      ctx->scratch_ptr("ivf.pwords", sizeof(uint32_t) * qb * wstride));
  uint64_t *all = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.pall", sizeof(uint64_t) * qb * nlist));
  uint64_t *kept = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.pkept", sizeof(uint64_t) * qb * cap));
  uint64_t *exact = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.pexact", sizeof(uint64_t) * qb * cap));
  uint8_t *ok = static_cast<uint8_t *>(ctx->scratch_ptr("ivf.pok", 2 * (size_t)qb));
  uint8_t *bad = ok + qb;
  int32_t *nout = static_cast<int32_t *>(ctx->scratch_ptr("ivf.pnout", 4 * (size_t)qb));
  // the overflowing queries' count as the fallback's work (profiling)
  int64_t *nbad =
      ctx->count_work() ? static_cast<int64_t *>(ctx->scratch_ptr("ivf.pnbad", 8)) : nullptr;
  const int32_t nchunks = (int32_t)ceil_div(nlist, 256);
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    {
      KernelTimer t(ctx, "ivf_probe_screen", (double)nb * nlist);
      const unsigned grid = (unsigned)(nchunks * ceil_div(nb, kScreenQ));
      const DenseScreen ds{nb, nlist, wstride, nchunks};
#define VSK_PS(KS, PL)                                                                        \
  k_list_screen<KS, true, PL><<<grid, 512, 0, ctx->stream>>>(                                \
      cdb->split.as<uint16_t>(), cdb->sqnorm.as<float>(), ldb, nullptr, qp.qh + b0 * qp.ldb, \
      qp.ql ? qp.ql + b0 * qp.ldb : nullptr, qp.qsq + b0, nullptr, nullptr, nullptr, 0,      \
      nullptr, nullptr, words, ds)
      switch (ldb / 32) {
      case 2: if (qp.ql) VSK_PS(2, 2); else VSK_PS(2, 1); break;
      case 4: if (qp.ql) VSK_PS(4, 2); else VSK_PS(4, 1); break;
      case 6: VSK_PS(6, 1); break;
      default: VSK_PS(8, 1); break;
      }
#undef VSK_PS
      check_launch("ivf_probe_screen");
    }
    MarginArgs ma;
    ma.nq = nb;
    ma.k = np;
    ma.words = words;
    ma.wstride = wstride;
    ma.wn = nlist;
    ma.qnh = qp.qnh + b0;
    ma.qnr = qp.qnr + b0;
    ma.xh = cdb->split_max_hi;
    ma.xr = cdb->split_max_res;
    ma.d = ivf->d;
    ma.nprod = qp.nprod;
    ma.metric = VSK_METRIC_L2;
    if (nbad) fill_i32(ctx, reinterpret_cast<int32_t *>(nbad), 2, 0);
    ma.nbad = reinterpret_cast<unsigned long long *>(nbad);
    if (np <= 256) {
      // the margin, its exact rescore and the selection in one launch
      ScreenTailArgs ta;
      ta.m = ma;
      ta.m.cap = 1024;
      ta.rows = cdb->x.as<float>();
      ta.Q = dq + b0 * ld;
      ta.ld = ld;
      ta.squared = 0;
      ta.all = all;
      ta.all_n = nlist;
      ta.best_out = keys + b0 * np;
      KernelTimer t(ctx, "ivf_probe_tail");
      if (nbad) t.device_work(nbad);
      launch_screen_tail(ctx, ta, "probe_tail");
      continue;
    }
    ma.out = kept;
    ma.cap = cap;
    ma.nout = nout;
    ma.ok = ok;
    ma.bad = bad;
    launch_screen_margin(ctx, ma);
    RescoreArgs ra{};
    ra.rows = cdb->x.as<float>();
    ra.ld = ld;
    ra.Q = dq + b0 * ld;
    ra.nq = nb;
    {
      KernelTimer t(ctx, "ivf_probe_rescore");
      RescoreArgs r = ra;
      r.in = kept;
      r.in_stride = cap;
      r.cnt = nout;
      r.out = exact;
      r.active = ok;
      k_list_rescore<<<(unsigned)ceil_div(nb, 4), 256, 0, ctx->stream>>>(r);
      check_launch("ivf_probe_rescore");
    }
    SelectArgs sa;
    sa.nq = nb;
    sa.k = np;
    sa.cand = exact;
    sa.cap = cap;
    sa.counts = nout;
    sa.active = ok;
    sa.regs = cap <= 8192;
    sa.small = cap <= 1024;
    sa.best_out = keys + b0 * np;
    launch_select(ctx, sa, "ivf_probe_select");
    // queries with more than cap keys in the margin: every centroid exact
    {
      KernelTimer t(ctx, "ivf_probe_redo");
      if (nbad) t.device_work(nbad);
      RescoreArgs r = ra;
      r.in = all;
      r.all_n = nlist;
      r.active = bad;
      k_list_rescore<<<(unsigned)ceil_div(nb, 4), 256, 0, ctx->stream>>>(r);
      check_launch("ivf_probe_redo");
    }
    SelectArgs sb;
    sb.nq = nb;
    sb.k = np;
    sb.cand = all;
    sb.cap = nlist;
    sb.active = bad;
    sb.regs = true;
    sb.best_out = keys + b0 * np;
    launch_select(ctx, sb, "ivf_probe_select");
  }
}

}  // namespace vsk

// kind 0: the rows (metric L2 / L2SQ); 1: SQ8 codes, qextra = nq x d int8
// query codes; 2: PQ codes, qextra = the vsk_pq whose tables score them
// allow (may be null): the row filter, a bitmap over the stored rows' ids
// of allow_bits bits (k_allow_list_bits)
static vsk_status ivf_search_any(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                                 const void *qextra, int64_t nq, int32_t nprobe, int32_t k,
                                 int32_t metric, int32_t kind, void *out_dist,
                                 int64_t *out_ids, const uint32_t *allow = nullptr,
                                 int64_t allow_bits = 0) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  if (kind == 0) require_rows(ivf);
  if (kind == 0)
    VSK_REQUIRE(metric == VSK_METRIC_L2 || metric == VSK_METRIC_L2SQ,
                VSK_ERR_UNSUPPORTED,
                "IVF search ranks by euclidean distance (VSK_METRIC_L2 or "
                "VSK_METRIC_L2SQ)");
  if (kind != 0) {
    VSK_REQUIRE(ivf->ckind == kind, VSK_ERR_NOT_TRAINED,
                kind == 1 ? "the index holds no SQ8 codes (vsk_ivf_encode_sq8)"
                          : "the index holds no PQ codes (vsk_ivf_encode_pq)");
    VSK_REQUIRE(ivf->ctotal == ivf->total, VSK_ERR_NOT_TRAINED,
                "rows were added after the codes were made: encode again");
    VSK_REQUIRE(qextra, VSK_ERR_INVALID_ARGUMENT,
                kind == 1 ? "query codes are null" : "pq is null");
  }
  if (kind == 2) {
    const vsk_pq *pq = static_cast<const vsk_pq *>(qextra);
    int32_t dsub = 0;
    VSK_REQUIRE(pq_shape_matches(pq, ivf->d, ivf->cM, ivf->cksub) &&
                    pq_host_codebooks(pq, &dsub) == ivf->cparams,
                VSK_ERR_DIMENSION_MISMATCH,
                "pq does not match the codebook the codes were made with");
  }
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(q && out_dist && out_ids, VSK_ERR_INVALID_ARGUMENT,
              "null buffer");
  VSK_REQUIRE(k >= 1, VSK_ERR_INVALID_ARGUMENT, "k must be >= 1");
  VSK_REQUIRE(k <= VSK_MAX_K, VSK_ERR_INVALID_BUFFER_SIZE,
              "k exceeds VSK_MAX_K");
  VSK_REQUIRE(nprobe >= 1, VSK_ERR_INVALID_ARGUMENT, "nprobe must be >= 1");
  VSK_REQUIRE(allow_bits >= 0 && (allow || allow_bits == 0), VSK_ERR_INVALID_ARGUMENT,
              "row filter: null bitmap or negative size");
  const int32_t np = nprobe < ivf->nlist ? nprobe : ivf->nlist;  // .exact
  VSK_REQUIRE(np <= VSK_MAX_K || np == ivf->nlist, VSK_ERR_INVALID_ARGUMENT,
              "nprobe must be <= VSK_MAX_K or cover every list");
  float *dlut = nullptr;
  if (kind == 2) {
    // the tables first: that call syncs the stream itself
    dlut = static_cast<float *>(ctx->scratch_ptr(
        "ivf.lut", sizeof(float) * (size_t)nq * ivf->cM * ivf->cksub));
    const vsk_status st = vsk_pq_lut(ctx, static_cast<const vsk_pq *>(qextra), q, nq, dlut);
    if (st != VSK_OK) return st;
  }
  CallScope cs(ctx);
  const int32_t ld = ivf->ld;
  const float *dq = rows_to_device_padded(ctx, q, nq, ivf->d, ld, "ivf.q");
  int8_t *dqc = nullptr;
  if (kind == 1) {
    // query codes at the code stride, zero padded
    const int8_t *src = static_cast<const int8_t *>(
        input_to_device(ctx, qextra, (size_t)nq * ivf->d, "ivf.qc_in"));
    dqc = static_cast<int8_t *>(
        ctx->scratch_ptr("ivf.qc", (size_t)nq * ivf->cstride));
    fill_i32(ctx, reinterpret_cast<int32_t *>(dqc), nq * (ivf->cstride / 4), 0);
    VSK_HIP(hipMemcpy2DAsync(dqc, ivf->cstride, src, ivf->d, ivf->d, nq,
                             hipMemcpyDeviceToDevice, ctx->stream));
  }
  OutputStage od(ctx, out_dist, sizeof(float) * nq * k, "out.dist");
  OutputStage oi(ctx, out_ids, sizeof(int64_t) * nq * k, "out.ids");
  // the row filter in list order (one bit per stored row)
  uint32_t *lmask = nullptr;
  if (allow && ivf->total > 0) {
    const uint32_t *dallow = static_cast<const uint32_t *>(input_to_device(
        ctx, allow, sizeof(uint32_t) * (size_t)ceil_div(allow_bits, 32), "ivf.allow"));
    const int64_t blocks = ceil_div(ivf->total, 256);
    lmask = static_cast<uint32_t *>(
        ctx->scratch_ptr("ivf.lmask", sizeof(uint32_t) * (size_t)(8 * blocks)));
    KernelTimer t(ctx, "ivf_allow_bits");
    k_allow_list_bits<<<(unsigned)blocks, 256, 0, ctx->stream>>>(
        ivf->ids.as<int64_t>(), ivf->total, dallow, allow_bits, lmask);
    check_launch("ivf_allow_bits");
  }

  // the bf16 screen of the list scan (kind 0) and of the probe share the
  // queries' bf16 planes
  const double per_query = ivf->nlist > 0 ? (double)ivf->total * np / ivf->nlist : 0.0;
  const bool screen =
      kind == 0 && list_screen_applies(ctx, ivf, metric, k, (double)nq * per_query);
  const bool exact_all = np == ivf->nlist && np > VSK_MAX_K;
  ScreenQueries sqp;
  if (screen || (!exact_all && probe_screen_applies(ctx, ivf, nq, np)))
    sqp = screen_queries2(ctx, dq, nq, ivf->d, ld);

  // 1. probes (ranked keys, turned into ids by the probe bases below)
  int32_t *probes = static_cast<int32_t *>(
      ctx->scratch_ptr("ivf.probes", sizeof(int32_t) * nq * np));
  uint64_t *pkeys = nullptr;
  if (exact_all) {
    // .exact with more lists than a selection holds: every list, ranked by
    // (exact distance, centroid) as findNearestCentroids sorts them, so
    // that candidates tied on distance keep the reference's order
    ivf_rank_all(ctx, ivf, dq, nq, probes);
  } else {
    ivf_probe_device(ctx, ivf, dq, nq, np, probes, sqp.one.qh ? &sqp.one : nullptr, &pkeys);
  }
  // 2. candidate counts and probe position bases
  int64_t *pos_base = static_cast<int64_t *>(
      ctx->scratch_ptr("ivf.pos_base", sizeof(int64_t) * nq * np));
  int64_t *cnt =
      static_cast<int64_t *>(ctx->scratch_ptr("ivf.cnt", sizeof(int64_t) * nq));

  // queries per group: their rows, codes or tables fit 64 KiB of LDS
  const int64_t per_q = kind == 0 ? (int64_t)ld * 4
                        : kind == 1 ? (int64_t)ivf->cstride
                                    : (int64_t)ivf->cM * ivf->cksub * 4;
  const int QG = per_q * 16 <= 64 * 1024 ? 16
                 : per_q * 8 <= 64 * 1024 ? 8
                 : per_q * 4 <= 64 * 1024 ? 4
                                           : 1;
  VSK_REQUIRE(per_q * QG <= 64 * 1024, VSK_ERR_UNSUPPORTED,
              kind == 2 ? "PQ tables too large for the IVF list scan (M x ksub > 16384)"
                        : "dimension too large for the IVF list scan");
  // candidates per query: at most the np largest lists; query batches
  // whose bound fits 2^27 keys (one query at least).  Everything below runs
  // on the stream without a read-back: segment offsets, pairs and groups
  // are made on the device, and grids take their upper bounds.
  const int64_t ubound = probe_bound(ivf, np);
  // (pair ids q * np + p are 32-bit)
  const int64_t qb = std::max<int64_t>(
      1, std::min<int64_t>({nq, tile_keys(ctx, 1ll << 27, 12) / std::max<int64_t>(ubound, 1),
                            (int64_t)INT32_MAX / np}));
  // the screen's groups are up to kScreenQ queries
  const int G = screen ? kScreenQ : QG;
  if (screen) list_screen_plane(ctx, ivf);
  // the per-list pair counters of the grouping, cleared by the probe bases
  int32_t *lcnt = kind != 2 ? static_cast<int32_t *>(
                                  ctx->scratch_ptr("ivf.lcnt", sizeof(int32_t) * ivf->nlist))
                            : nullptr;
  // the screened list scan keeps only the candidates under each query's
  // bound, from the probe's exact centroid distances (not with a row
  // filter, whose excluded rows may be the ones that make the bound)
  const bool compact =
      screen && !lmask && pkeys && np <= 256 && k <= 256 && !ctx->ivf_no_compact;
  ProbeBound pbd;
  if (compact) {
    pbd.qlim = static_cast<uint32_t *>(ctx->scratch_ptr("ivf.qlim", sizeof(uint32_t) * nq));
    pbd.rad = ivf->xrad.as<float>();
    pbd.k = k;
    pbd.qnh = sqp.two.qnh;
    pbd.qnr = sqp.two.qnr;
    pbd.xh = ivf->xh_max;
    pbd.xr = ivf->xr_max;
    pbd.d = ivf->d;
    pbd.metric = metric;
    pbd.nprod = sqp.two.nprod;
  }
  {
    KernelTimer t(ctx, "ivf_probe_bases");
    k_probe_bases<<<(unsigned)ceil_div(nq, 4), 256, 0, ctx->stream>>>(
        probes, pkeys, nq, np, ivf->list_off.as<int64_t>(), pos_base, cnt, lcnt, ivf->nlist,
        pbd);
    check_launch("ivf_probe_bases");
  }
  const int64_t nbmax = qb, npmax = nbmax * np;
  const int32_t nlist = ivf->nlist;
  const int64_t gmax = std::min<int64_t>(nlist, npmax) + ceil_div(npmax, G);
  uint64_t *best = static_cast<uint64_t *>(
      ctx->scratch_ptr("ivf.best", sizeof(uint64_t) * nq * k));
  int64_t *dseg = static_cast<int64_t *>(
      ctx->scratch_ptr("ivf.seg", sizeof(int64_t) * 2 * (nbmax + 1)));
  int64_t *wseg = dseg + (nbmax + 1);
  int64_t *loffs = static_cast<int64_t *>(
      ctx->scratch_ptr("ivf.loffs", sizeof(int64_t) * 3 * (nlist + 1)));
  int64_t *lstart = loffs, *gstart = loffs + 2 * (nlist + 1);
  int32_t *rank = static_cast<int32_t *>(
      ctx->scratch_ptr("ivf.rank", sizeof(int32_t) * (npmax + 1)));
  const ListGroups lg{lcnt, lstart, gstart, rank, nullptr, nullptr};
  int32_t *dpairs = static_cast<int32_t *>(
      ctx->scratch_ptr("ivf.pairs", sizeof(int32_t) * (npmax + 1)));
  int4 *dgroups = static_cast<int4 *>(ctx->scratch_ptr("ivf.groups", sizeof(int4) * (gmax + 1)));
  ListGroups lgp = lg;
  lgp.pairs = dpairs;
  lgp.groups = dgroups;
  // (the screen's 32-bit words, each query's padded to a multiple of 4,
  // share this memory)
  uint64_t *cand = static_cast<uint64_t *>(ctx->scratch_ptr(
      "ivf.cand", std::max(sizeof(uint64_t) * (nbmax * ubound + 1),
                           sizeof(uint32_t) * (nbmax * (ubound + 3) + 4))));
  const int64_t *loff = ivf->list_off.as<int64_t>();
  // the screen's words in memory of their own: the fused tail of one query
  // writes exact keys into cand while other queries' words are still read
  uint32_t *swords = screen ? static_cast<uint32_t *>(ctx->scratch_ptr(
                                  "ivf.words", sizeof(uint32_t) * (nbmax * (ubound + 3) + 4)))
                            : nullptr;
  ScreenKeep keep;
  if (compact) {
    keep.qlim = pbd.qlim;
    keep.pcnt = static_cast<int32_t *>(
        ctx->scratch_ptr("ivf.pcnt", sizeof(int32_t) * (npmax + 1)));
    keep.prow = static_cast<uint32_t *>(ctx->scratch_ptr(
        "ivf.prow", sizeof(uint32_t) * (nbmax * (ubound + 3) + 4)));
  }

  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    const int64_t npairs = nb * np;
    const int64_t ng = std::min<int64_t>(nlist, npairs) + ceil_div(npairs, G);
    // 3. segment offsets; pairs grouped by list, groups of up to G pairs
    {
      ListGroups g = lgp;
      if (kind == 2) g.pairs = nullptr;  // the PQ scan walks each query's probes itself
      batch_groups(ctx, ivf, probes + b0 * np, npairs, cnt + b0, nb, dseg, wseg, G, g);
    }
    if (screen) {
      list_screen_batch(ctx, ivf, sqp.two, dq, b0, nb, np, k, metric, probes, pos_base, cnt,
                        dseg, wseg, lgp, swords, cand, best, lmask, compact ? &keep : nullptr);
      continue;
    }
    const int64_t *ngroups = gstart + nlist;
    ListScanArgs la;
    la.rows = ivf->rows.as<float>();
    la.list_off = loff;
    la.Q = dq + b0 * ld;
    la.ld = ld;
    la.np = np;
    la.probes = probes + b0 * np;
    la.pairs = dpairs;
    la.groups = dgroups;
    la.ngroups = ngroups;
    la.pos_base = pos_base + b0 * np;
    la.wseg = wseg;
    la.words = reinterpret_cast<uint32_t *>(cand);
    la.squared = metric == VSK_METRIC_L2SQ ? 1 : 0;
    la.codes = ivf->codes.as<uint8_t>();
    la.cstride = ivf->cstride;
    la.qc = dqc ? dqc + b0 * ivf->cstride : nullptr;
    la.lut = dlut ? dlut + b0 * ivf->cM * ivf->cksub : nullptr;
    la.M = ivf->cM;
    la.ksub = ivf->cksub;
    {
      const size_t lds = (size_t)(per_q * QG);
      const unsigned g = (unsigned)ng;
      static const char *names[3] = {"ivf_list_scan", "ivf_sq8_list_scan", "ivf_pq_list_scan"};
      KernelTimer t(ctx, names[kind]);
      t.device_work(dseg + nb);
#define VSK_SCAN_QG(K)                                                  \
  if (QG == 16) K<16><<<g, 256, lds, ctx->stream>>>(la);               \
  else if (QG == 8) K<8><<<g, 256, lds, ctx->stream>>>(la);            \
  else if (QG == 4) K<4><<<g, 256, lds, ctx->stream>>>(la);            \
  else K<1><<<g, 256, lds, ctx->stream>>>(la);
      if (kind == 0) {
        VSK_SCAN_QG(k_list_scan)
      } else if (kind == 1) {
        VSK_SCAN_QG(k_list_scan_sq8)
      } else {
        k_list_scan_pq_q<<<(unsigned)nb, 256, (size_t)per_q, ctx->stream>>>(la);
      }
#undef VSK_SCAN_QG
      check_launch(names[kind]);
    }
    if (lmask)
      mask_words(ctx, la.probes, np, la.pos_base, ivf, wseg, lmask, la.words, nb);
    // 4. selection per query segment
    WordSelectArgs sa;
    sa.nq = nb;
    sa.k = k;
    sa.words = la.words;
    sa.wseg = wseg;
    sa.cnt = cnt + b0;
    sa.best_out = best + b0 * k;
    launch_select_words(ctx, sa, "ivf_select");
  }
  {
    KernelTimer t(ctx, "ivf_decode");
    k_ivf_decode<<<grid1(nq * k), 256, 0, ctx->stream>>>(
        best, nq, k, probes, np, pos_base, ivf->list_off.as<int64_t>(),
        ivf->ids.as<int64_t>(), od.ptr<float>(), oi.ptr<int64_t>(), kind);
    check_launch("ivf_decode");
  }
  od.copy_back();
  oi.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

// the rows of the index, contiguous (total x d fp32), into dst
static void ivf_rows_dense(vsk_ctx *ctx, const vsk_ivf *ivf, float *dst) {
  VSK_HIP(hipMemcpy2DAsync(dst, sizeof(float) * ivf->d, ivf->rows.p, sizeof(float) * ivf->ld,
                           sizeof(float) * ivf->d, ivf->total, hipMemcpyDeviceToDevice,
                           ctx->stream));
}

// codes (total x w bytes, dense) -> the index's code store at stride
// round_up(w, align), zero padded
static void ivf_store_codes(vsk_ctx *ctx, vsk_ivf *ivf, const void *dense, int32_t w,
                            int32_t align, int32_t kind) {
  const int32_t stride = (w + align - 1) / align * align;
  auto buf = std::make_unique<DevBuf>();
  buf->reserve((size_t)ivf->total * stride + 16);
  fill_i32(ctx, buf->as<int32_t>(), ((int64_t)ivf->total * stride + 16) / 4, 0);
  VSK_HIP(hipMemcpy2DAsync(buf->p, stride, dense, w, w, ivf->total, hipMemcpyDeviceToDevice,
                           ctx->stream));
  stream_sync(ctx);
  std::swap(ivf->codes.p, buf->p);
  std::swap(ivf->codes.bytes, buf->bytes);
  ivf->ckind = kind;
  ivf->cstride = stride;
  ivf->ctotal = ivf->total;
}

extern "C" {

vsk_status vsk_ivf_search(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                          int64_t nq, int32_t nprobe, int32_t k, int32_t metric,
                          float *out_dist, int64_t *out_ids) {
  return topk_call(ctx, [&] { return ivf_search_any(ctx, ivf, q, nullptr, nq, nprobe, k, metric, 0, out_dist, out_ids); });
}

vsk_status vsk_ivf_search_filtered(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                                   int64_t nq, int32_t nprobe, int32_t k, int32_t metric,
                                   const uint32_t *allow, int64_t allow_bits, float *out_dist,
                                   int64_t *out_ids) {
  if (!allow && allow_bits == 0)
    return topk_call(ctx, [&] { return ivf_search_any(ctx, ivf, q, nullptr, nq, nprobe, k, metric, 0, out_dist, out_ids); });
  return topk_call(ctx, [&] { return ivf_search_any(ctx, ivf, q, nullptr, nq, nprobe, k, metric, 0, out_dist, out_ids,
                        allow, allow_bits); });
}

vsk_status vsk_ivf_search_sq8(vsk_ctx *ctx, const vsk_ivf *ivf, const float *q,
                              const int8_t *qcodes, int64_t nq, int32_t nprobe, int32_t k,
                              int32_t *out_score, int64_t *out_ids) {
  return topk_call(ctx, [&] { return ivf_search_any(ctx, ivf, q, qcodes, nq, nprobe, k, -1, 1, out_score, out_ids); });
}

vsk_status vsk_ivf_search_pq(vsk_ctx *ctx, const vsk_ivf *ivf, const vsk_pq *pq,
                             const float *q, int64_t nq, int32_t nprobe, int32_t k,
                             float *out_dist, int64_t *out_ids) {
  return topk_call(ctx, [&] { return ivf_search_any(ctx, ivf, q, pq, nq, nprobe, k, -1, 2, out_dist, out_ids); });
}

vsk_status vsk_ivf_remove(vsk_ctx *ctx, vsk_ivf *ivf, const int64_t *ids, int64_t n,
                          int64_t *removed) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(n >= 0 && (ids || n == 0), VSK_ERR_INVALID_ARGUMENT, "null ids");
  if (removed) *removed = 0;
  if (n > 0 && ivf->total > 0) {
    CallScope cs(ctx);
    std::vector<int64_t> want((size_t)n), hids((size_t)ivf->total);
    VSK_HIP(hipMemcpyAsync(want.data(), ids, sizeof(int64_t) * (size_t)n, hipMemcpyDefault,
                           ctx->stream));
    VSK_HIP(hipMemcpyAsync(hids.data(), ivf->ids.p, sizeof(int64_t) * hids.size(),
                           hipMemcpyDeviceToHost, ctx->stream));
    stream_sync(ctx);
    std::sort(want.begin(), want.end());
    // the rows kept, list by list in their order
    std::vector<int64_t> keep, off((size_t)ivf->nlist + 1);
    keep.reserve(hids.size());
    for (int32_t l = 0; l < ivf->nlist; ++l) {
      off[(size_t)l] = (int64_t)keep.size();
      for (int64_t v = ivf->off[(size_t)l]; v < ivf->off[(size_t)l + 1]; ++v)
        if (!std::binary_search(want.begin(), want.end(), hids[(size_t)v])) keep.push_back(v);
    }
    off[(size_t)ivf->nlist] = (int64_t)keep.size();
    const int64_t m = (int64_t)keep.size(), gone = ivf->total - m;
    if (gone > 0) {
      const bool codes = ivf->ckind != 0 && ivf->ctotal == ivf->total;
      DevBuf rows, nids, ncodes, didx, doff;
      if (!ivf->codes_only) rows.reserve(sizeof(float) * (size_t)m * ivf->ld);
      nids.reserve(sizeof(int64_t) * (size_t)m);
      if (codes) {
        ncodes.reserve((size_t)m * ivf->cstride + 16);
        fill_i32(ctx, ncodes.as<int32_t>(), ((int64_t)m * ivf->cstride + 16) / 4, 0);
      }
      didx.reserve(sizeof(int64_t) * (size_t)m);
      doff.reserve(sizeof(int64_t) * off.size());
      VSK_HIP(hipMemcpyAsync(didx.p, keep.data(), sizeof(int64_t) * (size_t)m,
                             hipMemcpyHostToDevice, ctx->stream));
      VSK_HIP(hipMemcpyAsync(doff.p, off.data(), sizeof(int64_t) * off.size(),
                             hipMemcpyHostToDevice, ctx->stream));
      if (m > 0) {
        k_gather_stored<<<grid1(m, 4), 256, 0, ctx->stream>>>(
            ivf->codes_only ? nullptr : ivf->rows.as<float>(), ivf->ids.as<int64_t>(),
            codes ? ivf->codes.as<uint8_t>() : nullptr, ivf->cstride, didx.as<int64_t>(), m,
            ivf->ld, rows.as<float>(), nids.as<int64_t>(), ncodes.as<uint8_t>());
        check_launch("ivf_remove_gather");
      }
      stream_sync(ctx);
      std::swap(ivf->rows.p, rows.p);
      std::swap(ivf->rows.bytes, rows.bytes);
      std::swap(ivf->ids.p, nids.p);
      std::swap(ivf->ids.bytes, nids.bytes);
      std::swap(ivf->list_off.p, doff.p);
      std::swap(ivf->list_off.bytes, doff.bytes);
      if (codes) {
        std::swap(ivf->codes.p, ncodes.p);
        std::swap(ivf->codes.bytes, ncodes.bytes);
      }
      ivf->off.swap(off);
      ivf->total = m;
      // codes made before later inserts stay stale (the count must not
      // come to match again)
      ivf->ctotal = codes ? m : -1;
      ++ivf->version;
    }
    cs.finish();
    if (removed) *removed = gone;
  }
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_list_ids(vsk_ctx *ctx, const vsk_ivf *ivf, int64_t *ids, int64_t *offsets) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  if (offsets) std::memcpy(offsets, ivf->off.data(), sizeof(int64_t) * ivf->off.size());
  if (ids && ivf->total > 0) {
    CallScope cs(ctx);
    VSK_HIP(hipMemcpyAsync(ids, ivf->ids.p, sizeof(int64_t) * (size_t)ivf->total,
                           hipMemcpyDefault, ctx->stream));
    cs.finish();
  }
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_drop_rows(vsk_ctx *ctx, vsk_ivf *ivf) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(ivf->ckind != 0 && ivf->ctotal == ivf->total, VSK_ERR_NOT_TRAINED,
              "the index holds no current codes (vsk_ivf_encode_sq8 / vsk_ivf_encode_pq)");
  if (!ivf->codes_only) {
    stream_sync(ctx);  // (nothing queued may still read the rows)
    ivf->rows.release();
    ivf->xplane.release();
    ivf->xsq.release();
    ivf->xversion = -1;
    ivf->codes_only = true;
  }
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_storage(vsk_ctx *ctx, const vsk_ivf *ivf, int32_t *codes_only,
                           int64_t *device_bytes) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  if (codes_only) *codes_only = ivf->codes_only ? 1 : 0;
  if (device_bytes)
    *device_bytes = (int64_t)(ivf->centroids.x.bytes + ivf->centroids.sqnorm.bytes +
                              ivf->centroids.norm.bytes + ivf->centroids.split.bytes +
                              ivf->centroids.split_lo.bytes + ivf->centroids.seqnorm.bytes +
                              ivf->rows.bytes + ivf->ids.bytes + ivf->list_off.bytes +
                              ivf->codes.bytes + ivf->xplane.bytes + ivf->xsq.bytes);
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_encode_sq8(vsk_ctx *ctx, vsk_ivf *ivf, int32_t per_dim,
                              const float *scale, const float *offset) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  require_rows(ivf);
  VSK_REQUIRE(ivf->total > 0, VSK_ERR_EMPTY_INPUT, "the index holds no rows");
  VSK_REQUIRE(scale && offset, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  DevBuf dense, codes;
  dense.reserve(sizeof(float) * (size_t)ivf->total * ivf->d);
  codes.reserve((size_t)ivf->total * ivf->d);
  ivf_rows_dense(ctx, ivf, dense.as<float>());
  const vsk_status st = vsk_sq8_encode(ctx, dense.as<float>(), ivf->total, ivf->d, per_dim,
                                       scale, offset, codes.as<int8_t>());
  if (st != VSK_OK) return st;
  ivf_store_codes(ctx, ivf, codes.p, ivf->d, 16, 1);
  ivf->cM = ivf->cksub = ivf->cdsub = 0;
  // keep the parameters: they identify the codes and travel with the file
  const size_t ns = per_dim ? (size_t)ivf->d : 1;
  ivf->cparams.assign(2 * ns, 0.f);
  VSK_HIP(hipMemcpy(ivf->cparams.data(), scale, sizeof(float) * ns, hipMemcpyDefault));
  VSK_HIP(hipMemcpy(ivf->cparams.data() + ns, offset, sizeof(float) * ns, hipMemcpyDefault));
  ivf->cper_dim = per_dim ? 1 : 0;
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_encode_pq(vsk_ctx *ctx, vsk_ivf *ivf, const vsk_pq *pq) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  require_rows(ivf);
  VSK_REQUIRE(ivf->total > 0, VSK_ERR_EMPTY_INPUT, "the index holds no rows");
  VSK_REQUIRE(pq, VSK_ERR_INVALID_ARGUMENT, "pq is null");
  int32_t M = 0, ksub = 0;
  VSK_REQUIRE(pq_shape(pq, &M, &ksub) == ivf->d, VSK_ERR_DIMENSION_MISMATCH,
              "pq dimension differs from the index's");
  DevBuf dense, codes;
  dense.reserve(sizeof(float) * (size_t)ivf->total * ivf->d);
  codes.reserve((size_t)ivf->total * M);
  ivf_rows_dense(ctx, ivf, dense.as<float>());
  const vsk_status st = vsk_pq_encode(ctx, pq, dense.as<float>(), ivf->total, codes.as<uint8_t>());
  if (st != VSK_OK) return st;
  ivf_store_codes(ctx, ivf, codes.p, M, 4, 2);
  ivf->cM = M;
  ivf->cksub = ksub;
  ivf->cparams = pq_host_codebooks(pq, &ivf->cdsub);
  ivf->cper_dim = 0;
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_centroids(vsk_ctx *ctx, const vsk_ivf *ivf, float *out) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  CallScope cs(ctx);
  copy_rows(ctx, out, sizeof(float) * ivf->d, ivf->centroids.x.p, sizeof(float) * ivf->ld,
            sizeof(float) * ivf->d, ivf->nlist);
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_sq8_params(vsk_ctx *ctx, const vsk_ivf *ivf, int32_t *per_dim,
                              float *scale, float *offset) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(ivf->ckind == 1 && ivf->ctotal == ivf->total, VSK_ERR_NOT_TRAINED,
              "the index holds no current SQ8 codes");
  const size_t ns = ivf->cper_dim ? (size_t)ivf->d : 1;
  if (per_dim) *per_dim = ivf->cper_dim;
  if (scale) memcpy(scale, ivf->cparams.data(), sizeof(float) * ns);
  if (offset) memcpy(offset, ivf->cparams.data() + ns, sizeof(float) * ns);
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_set_meta(vsk_ctx *ctx, vsk_ivf *ivf, const void *bytes, int64_t n) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(n >= 0 && n <= (int64_t(1) << 30), VSK_ERR_INVALID_BUFFER_SIZE,
              "metadata is limited to 1 GiB");
  VSK_REQUIRE(n == 0 || bytes, VSK_ERR_INVALID_ARGUMENT, "bytes is null");
  const uint8_t *b = static_cast<const uint8_t *>(bytes);
  ivf->meta.assign(b, b + n);
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_get_meta(vsk_ctx *ctx, const vsk_ivf *ivf, void *out, int64_t cap,
                            int64_t *n) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(n, VSK_ERR_INVALID_ARGUMENT, "n is null");
  VSK_REQUIRE(cap >= 0 && (cap == 0 || out), VSK_ERR_INVALID_ARGUMENT, "bad output buffer");
  *n = (int64_t)ivf->meta.size();
  const size_t m = (size_t)std::min<int64_t>(cap, *n);
  if (m) memcpy(out, ivf->meta.data(), m);
  VSK_API_END(ctx);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// index file (layout in the header's comment on vsk_ivf_save)
// ---------------------------------------------------------------------------
namespace vsk {
namespace {

constexpr char kIvfMagic[8] = {'V', 'S', 'K', 'I', 'V', 'F', '0', '2'};
constexpr int64_t kHeaderBytes = 8 + 8 + 16 + 16 + 8 + 8;  // magic .. meta size
constexpr int64_t kMaxMeta = int64_t(1) << 30;
constexpr size_t kIoChunk = 64u << 20;  // host staging per transfer

struct Fnv1a {
  uint64_t h = 0xcbf29ce484222325ull;
  void add(const void *p, size_t n) {
    const uint8_t *b = static_cast<const uint8_t *>(p);
    for (size_t i = 0; i < n; ++i) {
      h ^= b[i];
      h *= 0x100000001b3ull;
    }
  }
};

struct FileCloser {
  void operator()(FILE *f) const { fclose(f); }
};
using File = std::unique_ptr<FILE, FileCloser>;

void put(FILE *f, Fnv1a &h, const void *p, size_t n) {
  if (n && fwrite(p, 1, n, f) != n) fail(VSK_ERR_IO, "index file: write failed");
  h.add(p, n);
}

void get(FILE *f, Fnv1a &h, void *p, size_t n) {
  if (n && fread(p, 1, n, f) != n) fail(VSK_ERR_IO, "index file: truncated");
  h.add(p, n);
}

// rows x w bytes at a device pitch -> file, through host chunks
void put_rows(vsk_ctx *ctx, FILE *f, Fnv1a &h, const void *dev, int64_t rows, size_t pitch,
              size_t w) {
  if (rows == 0) return;
  const int64_t per = std::max<int64_t>(1, (int64_t)(kIoChunk / w));
  std::vector<uint8_t> buf((size_t)std::min(per, rows) * w);
  for (int64_t r = 0; r < rows; r += per) {
    const int64_t cnt = std::min(per, rows - r);
    VSK_HIP(hipMemcpy2DAsync(buf.data(), w, static_cast<const uint8_t *>(dev) + r * pitch,
                             pitch, w, cnt, hipMemcpyDeviceToHost, ctx->stream));
    stream_sync(ctx);
    put(f, h, buf.data(), (size_t)cnt * w);
  }
}

// file -> rows x w bytes at a device pitch; check(chunk, rows) may reject a
// chunk before it is uploaded
void get_rows(vsk_ctx *ctx, FILE *f, Fnv1a &h, void *dev, int64_t rows, size_t pitch,
              size_t w, const std::function<bool(const uint8_t *, int64_t)> &check = nullptr) {
  if (rows == 0) return;
  const int64_t per = std::max<int64_t>(1, (int64_t)(kIoChunk / w));
  std::vector<uint8_t> buf((size_t)std::min(per, rows) * w);
  for (int64_t r = 0; r < rows; r += per) {
    const int64_t cnt = std::min(per, rows - r);
    get(f, h, buf.data(), (size_t)cnt * w);
    if (check && !check(buf.data(), cnt)) fail(VSK_ERR_IO, "index file: bad code values");
    VSK_HIP(hipMemcpy2DAsync(static_cast<uint8_t *>(dev) + r * pitch, pitch, buf.data(), w, w,
                             cnt, hipMemcpyHostToDevice, ctx->stream));
    stream_sync(ctx);
  }
}

struct IvfDeleter {
  vsk_ctx *ctx;
  void operator()(vsk_ivf *p) const { vsk_ivf_free(ctx, p); }
};

}  // namespace
}  // namespace vsk

extern "C" {

vsk_status vsk_ivf_save(vsk_ctx *ctx, const vsk_ivf *ivf, const char *path) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  VSK_REQUIRE(path, VSK_ERR_INVALID_ARGUMENT, "path is null");
  stream_sync(ctx);
  File f(fopen(path, "wb"));
  VSK_REQUIRE(f, VSK_ERR_IO, std::string("cannot open for writing: ") + path);
  Fnv1a h;
  const bool coded = ivf->ckind != 0 && ivf->ctotal == ivf->total;
  // a codes-only index (no rows section) marks its code kind with 16
  const int32_t hdr32[8] = {ivf->nlist,
                            ivf->d,
                            coded ? ivf->ckind | (ivf->codes_only ? 16 : 0) : 0,
                            coded ? ivf->cstride : 0,
                            coded ? ivf->cM : 0,
                            coded ? ivf->cksub : 0,
                            coded ? ivf->cper_dim : 0,
                            coded ? ivf->cdsub : 0};
  const int64_t hdr64[2] = {ivf->total, ivf->next_id};
  const int64_t meta_n = (int64_t)ivf->meta.size();
  put(f.get(), h, kIvfMagic, 8);
  put(f.get(), h, &hdr32[0], 8);
  put(f.get(), h, hdr64, 16);
  put(f.get(), h, &hdr32[2], 24);
  put(f.get(), h, &meta_n, 8);
  const size_t ldb = sizeof(float) * ivf->ld, db = sizeof(float) * ivf->d;
  put_rows(ctx, f.get(), h, ivf->centroids.x.p, ivf->nlist, ldb, db);
  put(f.get(), h, ivf->off.data(), sizeof(int64_t) * (ivf->nlist + 1));
  put_rows(ctx, f.get(), h, ivf->ids.p, ivf->total, 8, 8);
  if (!ivf->codes_only) put_rows(ctx, f.get(), h, ivf->rows.p, ivf->total, ldb, db);
  if (coded) {
    put_rows(ctx, f.get(), h, ivf->codes.p, ivf->total, ivf->cstride, ivf->cstride);
    put(f.get(), h, ivf->cparams.data(), sizeof(float) * ivf->cparams.size());
  }
  put(f.get(), h, ivf->meta.data(), ivf->meta.size());
  const uint64_t sum = h.h;
  VSK_REQUIRE(fwrite(&sum, 8, 1, f.get()) == 1 && fflush(f.get()) == 0, VSK_ERR_IO,
              "index file: write failed");
  VSK_REQUIRE(fclose(f.release()) == 0, VSK_ERR_IO, "index file: close failed");
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_load(vsk_ctx *ctx, const char *path, vsk_ivf **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(path, VSK_ERR_INVALID_ARGUMENT, "path is null");
  File f(fopen(path, "rb"));
  VSK_REQUIRE(f, VSK_ERR_IO, std::string("cannot open: ") + path);
  Fnv1a h;
  char magic[8];
  get(f.get(), h, magic, 8);
  VSK_REQUIRE(memcmp(magic, kIvfMagic, 8) == 0, VSK_ERR_IO, "not an IVF index file (VSKIVF02)");
  int32_t nd[2], ck[6];
  int64_t tn[2], meta_n = 0;
  get(f.get(), h, nd, 8);
  get(f.get(), h, tn, 16);
  get(f.get(), h, ck, 24);
  get(f.get(), h, &meta_n, 8);
  const int32_t nlist = nd[0], d = nd[1];
  const int64_t total = tn[0], next_id = tn[1];
  // every size is bounded before any arithmetic on it
  VSK_REQUIRE(nlist > 0 && nlist <= kMaxLists && d > 0 && d <= kMaxDim && total >= 0 &&
                  total <= 0x7FFFFFFFll && next_id >= 0 && meta_n >= 0 && meta_n <= kMaxMeta,
              VSK_ERR_IO, "index file: bad header");
  int64_t nparams = 0;  // floats of quantizer parameters
  bool kind_ok = false;
  // code kind 17 / 18: SQ8 / PQ codes without the rows (vsk_ivf_drop_rows)
  const bool codes_only = ck[0] == 17 || ck[0] == 18;
  if (codes_only) ck[0] -= 16;
  if (ck[0] == 0) kind_ok = ck[1] == 0 && ck[2] == 0 && ck[3] == 0 && ck[4] == 0 && ck[5] == 0;
  if (ck[0] == 1) {
    kind_ok = ck[1] == (d + 15) / 16 * 16 && ck[2] == 0 && ck[3] == 0 &&
              (ck[4] == 0 || ck[4] == 1) && ck[5] == 0;
    nparams = 2 * (ck[4] ? (int64_t)d : 1);
  }
  if (ck[0] == 2) {
    kind_ok = ck[2] > 0 && d % ck[2] == 0 && ck[3] >= 1 && ck[3] <= 256 &&
              ck[1] == (ck[2] + 3) / 4 * 4 && ck[4] == 0 && ck[5] == d / ck[2];
    nparams = kind_ok ? (int64_t)ck[2] * ck[3] * ck[5] : 0;
  }
  VSK_REQUIRE(kind_ok, VSK_ERR_IO, "index file: bad code header");
  // the file's length must be exactly what the header describes (bounded
  // sizes: no product below can overflow int64)
  const int64_t body = kHeaderBytes + 4ll * nlist * d + 8ll * (nlist + 1) + 8 * total +
                       (codes_only ? 0 : 4 * total * d) + (int64_t)ck[1] * total +
                       4 * nparams + meta_n + 8;
  VSK_REQUIRE(fseek(f.get(), 0, SEEK_END) == 0 && ftell(f.get()) == body &&
                  fseek(f.get(), kHeaderBytes, SEEK_SET) == 0,
              VSK_ERR_IO, "index file: length does not match its header");
  std::vector<float> cent((size_t)nlist * d);
  get(f.get(), h, cent.data(), 4 * cent.size());
  std::vector<int64_t> off((size_t)nlist + 1);
  get(f.get(), h, off.data(), 8 * off.size());
  bool off_ok = off[0] == 0 && off[nlist] == total;
  for (int32_t l = 0; l < nlist && off_ok; ++l) off_ok = off[l] <= off[l + 1];
  VSK_REQUIRE(off_ok, VSK_ERR_IO, "index file: bad list offsets");
  vsk_ivf *raw = nullptr;
  const vsk_status st = vsk_ivf_create(ctx, cent.data(), nlist, d, &raw);
  if (st != VSK_OK) return st;
  std::unique_ptr<vsk_ivf, IvfDeleter> ivf(raw, IvfDeleter{ctx});
  const int32_t ld = ivf->ld;
  ivf->ids.reserve(sizeof(int64_t) * (size_t)std::max<int64_t>(total, 1));
  get_rows(ctx, f.get(), h, ivf->ids.p, total, 8, 8);
  if (!codes_only) {
    ivf->rows.reserve(sizeof(float) * (size_t)std::max<int64_t>(total, 1) * ld);
    fill_i32(ctx, ivf->rows.as<int32_t>(), std::max<int64_t>(total, 1) * ld, 0);
    get_rows(ctx, f.get(), h, ivf->rows.p, total, sizeof(float) * ld, sizeof(float) * d);
  }
  ++ivf->version;
  if (ck[0] != 0) {
    ivf->codes.reserve((size_t)total * ck[1] + 16);
    fill_i32(ctx, ivf->codes.as<int32_t>(), ((int64_t)total * ck[1] + 16) / 4, 0);
    // PQ codes index the ksub-entry tables: every code byte must be < ksub
    // and the row padding zero
    const int32_t stride = ck[1], M = ck[2], ksub = ck[3];
    auto pq_ok = [&](const uint8_t *b, int64_t rows) {
      for (int64_t r = 0; r < rows; ++r)
        for (int32_t j = 0; j < stride; ++j) {
          const uint8_t c = b[r * stride + j];
          if (j < M ? c >= ksub : c != 0) return false;
        }
      return true;
    };
    get_rows(ctx, f.get(), h, ivf->codes.p, total, stride, stride,
             ck[0] == 2 ? std::function<bool(const uint8_t *, int64_t)>(pq_ok) : nullptr);
    ivf->cparams.resize((size_t)nparams);
    get(f.get(), h, ivf->cparams.data(), sizeof(float) * ivf->cparams.size());
  }
  ivf->meta.resize((size_t)meta_n);
  get(f.get(), h, ivf->meta.data(), ivf->meta.size());
  uint64_t sum = 0;
  VSK_REQUIRE(fread(&sum, 8, 1, f.get()) == 1 && sum == h.h, VSK_ERR_IO,
              "index file: checksum mismatch");
  VSK_HIP(hipMemcpyAsync(ivf->list_off.p, off.data(), sizeof(int64_t) * (nlist + 1),
                         hipMemcpyHostToDevice, ctx->stream));
  stream_sync(ctx);
  ivf->off = off;
  ivf->total = total;
  ivf->next_id = next_id;
  ivf->ckind = ck[0];
  ivf->cstride = ck[1];
  ivf->cM = ck[2];
  ivf->cksub = ck[3];
  ivf->cper_dim = ck[4];
  ivf->cdsub = ck[5];
  ivf->ctotal = ck[0] ? total : -1;
  ivf->codes_only = codes_only;
  *out = ivf.release();
  VSK_API_END(ctx);
}

vsk_status vsk_ivf_info(vsk_ctx *ctx, const vsk_ivf *ivf, int32_t *nlist, int32_t *d,
                        int64_t *total, int32_t *code_kind) {
  VSK_API_BEGIN(ctx);
  require_ivf(ivf);
  if (nlist) *nlist = ivf->nlist;
  if (d) *d = ivf->d;
  if (total) *total = ivf->total;
  if (code_kind) *code_kind = ivf->ctotal == ivf->total ? ivf->ckind : 0;
  VSK_API_END(ctx);
}

}  // extern "C"
