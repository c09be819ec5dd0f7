// kmeans.hip -- k-means on the GPU as KMeansClustering.cluster runs it
// (Clustering/KMeansClustering.swift:48-113): the trainer of IVF coarse
// centroids (Indexes/IVFIndex.swift:397-446) and of PQ codebooks
// (Quantization/ProductQuantizer.swift:270-324).
//
// One Lloyd iteration is
//   assignment  each row's nearest centroid under the sequential sqrt-L2 of
//               :421-428 (strict '<', :271-295) and its distance: the bf16
//               screen with a proven bound and an exact recomputation of the
//               winner (flat_screen.hip, screen_argmin) when the problem is
//               large, else the exact VALU argmin scan (flat.hip);
//   inertia     distances.reduce(0, +) (:97): one wave adds the distances in
//               row order, so the fp32 rounding is the reference's;
//   grouping    a stable LSD radix pass per 4-bit digit of the cluster id
//               lists the rows of every cluster in row order;
//   update      one wave per (cluster, 64 columns) adds its rows' values in
//               that order, x * weight then +=, and divides by the fp32
//               count (:342-380), so every centroid is bit-identical to the
//               reference's sequential loop.
// Empty clusters are refilled on the device from a seeded draw (the
// reference's draw, :374, is unseeded).  The inertia is summed on a second
// stream while the next iteration already runs; the host reads it back
// (pinned memory) and tests convergence (|inertia - previous| < tolerance,
// :98).  An iteration started past convergence writes only the other halves
// of the double-buffered centroids, assignments and distances, and is
// dropped.
//
// k-means++ (:209-259) picks each next centroid with probability
// proportional to D(x)^2, D the distance to the nearest chosen centroid.  The
// reference's weights are D^2 / sum(D) (:237), which is not a distribution,
// and its cumulative fp32 sum is sequential over all rows per pick.  Here the
// weights are D^2 as 32-bit fixed point of D^2 / max D^2 (exact integer
// sums, so any summation order gives the same draw) and the draw is
// Int.random(in: 0..<total) from one SeedableRNG(seed) stream that also drew
// the first row.  (The reference reseeds each pick with seed + picks so far,
// :241; an LCG's first output is affine in its seed, which correlates those
// draws from pick to pick.)  All k picks run on the device.
#include <unordered_map>
#include <vector>

#include "flat.hpp"

namespace vsk {

// ---------------------------------------------------------------------------
// SeedableRNG (:480-491) and Swift's bounded draw (RandomNumberGenerator.
// next(upperBound:), Lemire's nearly-divisionless method, arXiv:1805.10941)
// ---------------------------------------------------------------------------
__host__ __device__ inline uint64_t swift_lcg(uint64_t &s) {
  s = s * 2862933555777941757ull + 3037000493ull;
  return s;
}
__host__ __device__ inline uint64_t mul_hi64(uint64_t a, uint64_t b) {
#ifdef __HIP_DEVICE_COMPILE__
  return __umul64hi(a, b);
#else
  return (uint64_t)(((unsigned __int128)a * b) >> 64);
#endif
}
__host__ __device__ inline uint64_t swift_bounded(uint64_t &s, uint64_t bound) {
  uint64_t r = swift_lcg(s);
  uint64_t lo = r * bound;
  if (lo < bound) {
    const uint64_t t = (0 - bound) % bound;
    while (lo < t) {
      r = swift_lcg(s);
      lo = r * bound;
    }
  }
  return mul_hi64(r, bound);
}

// ---------------------------------------------------------------------------
// inertia: the fp32 sum of n values in index order, by one wave.  The wave
// copies blocks of 4096 values into LDS with coalesced loads (the next
// block's loads in flight meanwhile), and lane 0 adds each block in order
// from 16-byte LDS reads: the adds form one dependent chain with no
// cross-lane moves in it.  v must be 16-byte aligned.
// ---------------------------------------------------------------------------
constexpr int SS_BLOCK = 4096;  // values per LDS block (16 KB)
typedef float ss_f4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(64) void k_seq_sum(const float *v, int64_t n,
                                                float *out) {
  __shared__ ss_f4 buf[SS_BLOCK / 4];
  const int lane = threadIdx.x;
  const int64_t nb = n / SS_BLOCK;  // whole blocks
  const ss_f4 *src = reinterpret_cast<const ss_f4 *>(v);
  ss_f4 r[SS_BLOCK / 256];
  if (nb > 0) {
#pragma unroll
    for (int u = 0; u < SS_BLOCK / 256; ++u) r[u] = src[u * 64 + lane];
  }
  float s = 0.f;
  for (int64_t b = 0; b < nb; ++b) {
#pragma unroll
    for (int u = 0; u < SS_BLOCK / 256; ++u) buf[u * 64 + lane] = r[u];
    __syncthreads();
    if (b + 1 < nb) {
      const ss_f4 *nx = src + (b + 1) * (SS_BLOCK / 4);
#pragma unroll
      for (int u = 0; u < SS_BLOCK / 256; ++u) r[u] = nx[u * 64 + lane];
    }
    if (lane == 0) {
      for (int i = 0; i < SS_BLOCK / 4; ++i) {
        const ss_f4 t = buf[i];
        s = s + t.x;
        s = s + t.y;
        s = s + t.z;
        s = s + t.w;
      }
    }
    __syncthreads();
  }
  if (lane == 0) {
    for (int64_t i = nb * SS_BLOCK; i < n; ++i) s = s + v[i];
    out[0] = s;
  }
}

// ---------------------------------------------------------------------------
// grouping: stable LSD radix sort of (cluster, row) by cluster, 4-bit digits.
// A block owns GR_B consecutive rows, GR_PER consecutive ones per thread, so
// the order inside a digit is thread order then row order: the row order.
// ---------------------------------------------------------------------------
constexpr int GR_T = 256, GR_PER = 8, GR_B = GR_T * GR_PER;

// cnt[g][t] = rows of thread t in this block with digit g
__device__ inline void grp_count(const int32_t *keys, int64_t n, int shift,
                                 int32_t (*cnt)[GR_T]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int g = 0; g < 16; ++g) cnt[g][t] = 0;
  const int64_t r0 = (int64_t)blockIdx.x * GR_B + (int64_t)t * GR_PER;
#pragma unroll
  for (int j = 0; j < GR_PER; ++j) {
    const int64_t r = r0 + j;
    if (r < n) cnt[(keys[r] >> shift) & 15][t] += 1;
  }
}

// hist[g * nb + b] = rows of block b with digit g
__global__ __launch_bounds__(GR_T) void k_grp_hist(const int32_t *keys, int64_t n,
                                                   int shift, int32_t *hist) {
  __shared__ int32_t cnt[16][GR_T];
  grp_count(keys, n, shift, cnt);
  __syncthreads();
  // thread t sums 16 entries of digit t/16; the 16 threads of a digit share
  // one wave quarter and reduce by shuffles
  const int t = threadIdx.x, g = t >> 4, part = t & 15;
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += cnt[g][part * 16 + i];
#pragma unroll
  for (int m = 8; m > 0; m >>= 1) s += __shfl_xor(s, m, 16);
  if (part == 0) hist[(int64_t)g * gridDim.x + blockIdx.x] = s;
}

// in-place exclusive scan of m int32 values by one block of 1024 threads
__global__ __launch_bounds__(1024) void k_scan_excl(int32_t *h, int64_t m) {
  __shared__ int32_t wsum[16];
  __shared__ int32_t carry_s;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (t == 0) carry_s = 0;
  __syncthreads();
  for (int64_t base = 0; base < m; base += 1024) {
    const int64_t i = base + t;
    const int32_t v = i < m ? h[i] : 0;
    int32_t incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t u = __shfl_up(incl, o);
      if (lane >= o) incl += u;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    int32_t before = carry_s;
    for (int j = 0; j < w; ++j) before += wsum[j];
    if (i < m) h[i] = before + incl - v;
    __syncthreads();
    if (t == 1023) carry_s = before + incl;
    __syncthreads();
  }
}

// scatter rows to hist-scanned positions, stable within the block
__global__ __launch_bounds__(GR_T) void k_grp_scatter(
    const int32_t *keys, const int32_t *vals, int64_t n, int shift,
    const int32_t *hist, int32_t *keys_out, int32_t *vals_out) {
  __shared__ int32_t cnt[16][GR_T];
  __shared__ int32_t wtot[16][GR_T / 64];
  grp_count(keys, n, shift, cnt);
  __syncthreads();
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  // exclusive prefix of cnt[g][.] over the threads, plus the block's base
  int32_t incl[16];
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    int32_t x = cnt[g][t];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t u = __shfl_up(x, o);
      if (lane >= o) x += u;
    }
    incl[g] = x;
    if (lane == 63) wtot[g][w] = x;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    int32_t before = hist[(int64_t)g * gridDim.x + blockIdx.x];
    for (int j = 0; j < w; ++j) before += wtot[g][j];
    cnt[g][t] = before + incl[g] - cnt[g][t];  // this thread's next slot
  }
  // (each thread reads and writes only its own column of cnt)
  const int64_t r0 = (int64_t)blockIdx.x * GR_B + (int64_t)t * GR_PER;
#pragma unroll
  for (int j = 0; j < GR_PER; ++j) {
    const int64_t r = r0 + j;
    if (r < n) {
      const int32_t key = keys[r];
      const int g = (key >> shift) & 15;
      const int32_t pos = cnt[g][t];
      cnt[g][t] = pos + 1;
      keys_out[pos] = key;
      vals_out[pos] = vals ? vals[r] : (int32_t)r;
    }
  }
}

__global__ void k_count_clusters(const int32_t *assign, int64_t n, int32_t *counts) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    atomicAdd(&counts[assign[i]], 1);
}

// ---------------------------------------------------------------------------
// update: one wave per (cluster c = blockIdx.x, columns 64 * blockIdx.y ..).
// The members' row numbers are read 64 at a time; rows are loaded 16 ahead
// of the sequential adds.  cent[c][j] = sum / count for j < d, 0 in the
// padding; cntf[c] = the fp32 count (or weight sum) the reference divides
// by.  A cluster whose count is not > 0 keeps zeros (the host refills it).
// ---------------------------------------------------------------------------
constexpr int MU = 16;
__global__ __launch_bounds__(64) void k_cluster_means(
    const float *x, int64_t ld, int32_t d, const int32_t *order,
    const int32_t *off, const int32_t *counts, const float *weights,
    float *cent, float *cntf) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x;
  const int64_t c = blockIdx.x;
  const int64_t col = (int64_t)blockIdx.y * 64 + lane;
  const bool colok = col < ld;
  const int32_t m = counts[c], o = off[c];
  float s = 0.f, cw = 0.f;
  for (int32_t p0 = 0; p0 < m; p0 += 64) {
    const int32_t idx = p0 + lane < m ? order[o + p0 + lane] : 0;
    const float wl = weights ? weights[idx] : 1.f;
    const int32_t mm = m - p0 < 64 ? m - p0 : 64;
    for (int32_t j = 0; j < mm; j += MU) {
      float v[MU];
      float wv[MU];
#pragma unroll
      for (int u = 0; u < MU; ++u) {
        // rows past mm load row idx of lane 0's slot (in bounds), unused
        const int32_t row = __builtin_amdgcn_readlane(idx, (j + u) & 63);
        v[u] = colok ? x[(int64_t)row * ld + col] : 0.f;
        wv[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), (j + u) & 63));
      }
#pragma unroll
      for (int u = 0; u < MU; ++u) {
        if (j + u < mm) {
          if (weights) {
            s = s + v[u] * wv[u];
            cw = cw + wv[u];
          } else {
            s = s + v[u];
          }
        }
      }
    }
  }
  // fp32 count += 1 saturates at 2^24 (2^24 + 1 rounds back to it)
  const float cnt = weights ? cw : (m > (1 << 24) ? 16777216.f : (float)m);
  if (colok) cent[c * ld + col] = (col < d && cnt > 0.f) ? s / cnt : 0.f;
  if (blockIdx.y == 0 && lane == 0) cntf[c] = cnt;
}

// empty clusters (fp32 count not > 0) in ascending order each take row
// Int.random(in: 0..<n) of the SeedableRNG stream whose state is *rng: one
// wave, every lane draws the same sequence, the lanes copy the row
__global__ __launch_bounds__(64) void k_refill_empty(const float *cntf, int32_t k,
                                                     const float *x, int64_t ld, int32_t d,
                                                     int64_t n, uint64_t *rng, float *cent) {
  const int lane = threadIdx.x;
  uint64_t st = *rng;
  for (int32_t c0 = 0; c0 < k; c0 += 64) {
    const int32_t c = c0 + lane;
    const bool empty = c < k && !(cntf[c] > 0.f);
    uint64_t mask = __builtin_amdgcn_ballot_w64(empty);
    while (mask) {
      const int b = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int64_t r = (int64_t)swift_bounded(st, (uint64_t)n);
      const float *src = x + r * ld;
      float *dst = cent + (int64_t)(c0 + b) * ld;
      for (int32_t j = lane; j < d; j += 64) dst[j] = src[j];
    }
  }
  if (lane == 0) *rng = st;
}

__global__ void k_gather_rows_i64(const float *src, int64_t ld, const int64_t *rows,
                                  int64_t m, float *dst) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < m * ld;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / ld, c = i - r * ld;
    dst[i] = src[rows[r] * ld + c];
  }
}

// ---------------------------------------------------------------------------
// k-means++ on the device
// ---------------------------------------------------------------------------
constexpr int KP_T = 256;

constexpr int KPU_C = 32;     // columns of one staged chunk in k_kpp_update
constexpr int KP_SLOTS = 64;  // max slots per pick (a power of two, one wave's lanes)
constexpr int KPU_GRID = 4096;  // waves of k_kpp_update at most (16 per CU)

// cc[a] = |x_c - x_{chosen[a]}| for the picks a < r, c = chosen[r]: one
// wave per a, lanes over the coordinates.  Only the triangle test of
// k_kpp_update reads it, so any summation order with a small relative error
// serves (this one's is under (d / 64 + 11) 2^-25).
__global__ __launch_bounds__(256) void k_kpp_cc(const float *x, int64_t ld, int32_t d,
                                                const int64_t *chosen, int r, float *cc) {
#pragma clang fp contract(off)
  const int64_t c = chosen[r];
  if (c < 0) return;
  const int a = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (a >= r) return;  // wave-uniform
  const float *xc = x + c * ld, *xa = x + chosen[a] * ld;
  float s = 0.f;
  for (int32_t j = lane; j < d; j += 64) {
    const float t = xc[j] - xa[j];
    s = s + t * t;
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) s = s + __shfl_xor(s, m);
  if (lane == 0) cc[a] = sqrtf(s);
}

// D[i] = min(D[i], |x_i - x_c|) with c = chosen[r] (sequential sqrt-L2, as
// computeMinDistances, :401-419), near[i] = the pick that set D[i]; the max
// over rows of D^2 lands in maxbits[(r + 1) * KP_SLOTS + s] for the KP_SLOTS
// slots s (non-negative floats order as their bits; spread so the atomics
// do not queue on one address).
//
// One wave per block strides over groups of 64 rows.  A row is skipped
// (not read) when its nearest pick a has |x_c - x_a| >= 2 D skipm,
// skipm = 1 + (d + 4) 2^-22.  The exact distance is >= |x_c - x_a| -
// |x_i - x_a|, and (d + 4) 2^-22 exceeds the relative errors of the three
// computed distances taken together (a sequential one: under (d + 4) 2^-25;
// k_kpp_cc's: under (d / 64 + 11) 2^-25, counted twice), so the computed
// distance would be >= D and D[i] would not change.  The test is only taken
// for 2^-60 <= D <= 2^60, where no sum under- or overflows enough to break
// the relative bounds.  The rows that do need the distance queue in LDS;
// each full batch of 64 is staged through LDS in 128-byte column chunks
// (coalesced) and every lane sums its own row in coordinate order.
__global__ __launch_bounds__(64) void k_kpp_update(const float *__restrict__ x, int64_t ld,
                                                   int32_t d, int64_t n,
                                                   const int64_t *__restrict__ chosen, int r,
                                                   const float *__restrict__ cc, float skipm,
                                                   float *__restrict__ D,
                                                   int32_t *__restrict__ near,
                                                   uint32_t *__restrict__ maxbits) {
#pragma clang fp contract(off)
  __shared__ float tile[64 * (KPU_C + 1)];
  __shared__ int64_t l_row[128];
  __shared__ float l_dm[128];
  const int64_t c = chosen[r];
  if (c < 0) return;  // an earlier pick found degenerate data
  const int lane = threadIdx.x;
  const float *__restrict__ xc = x + c * ld;
  uint32_t b = 0;  // max D^2 bits seen by this lane
  // the distances of the first m <= 64 queued rows
  auto run = [&](int m) {
    float s = 0.f;
    for (int32_t j0 = 0; j0 < d; j0 += KPU_C) {
      const int cw = d - j0 < KPU_C ? d - j0 : KPU_C;
      __syncthreads();  // the previous chunk has been read
#pragma unroll
      for (int t = 0; t < KPU_C; ++t) {
        const int rr = t * (64 / KPU_C) + lane / KPU_C, col = lane % KPU_C;
        if (rr < m && col < cw)
          tile[rr * (KPU_C + 1) + col] = x[l_row[rr] * ld + j0 + col];
      }
      __syncthreads();
      if (lane < m)
        for (int jj = 0; jj < cw; ++jj) {
          const float t = tile[lane * (KPU_C + 1) + jj] - xc[j0 + jj];
          s = s + t * t;
        }
    }
    if (lane < m) {
      float dm = l_dm[lane];
      const float dist = sqrtf(s);
      if (dist < dm) {
        dm = dist;
        const int64_t i = l_row[lane];
        D[i] = dm;
        near[i] = r;
      }
      const uint32_t bw = __float_as_uint(dm * dm);
      b = bw > b ? bw : b;
    }
  };
  int cnt = 0;  // queued rows (wave-uniform)
  for (int64_t row0 = (int64_t)blockIdx.x * 64; row0 < n; row0 += (int64_t)gridDim.x * 64) {
    const int64_t i = row0 + lane;
    bool need = false;
    float dm = 0.f;
    if (i < n) {
      dm = D[i];
      const int32_t a = near[i];
      need = !(a >= 0 && dm >= 0x1p-60f && dm <= 0x1p60f && cc[a] >= 2.0f * dm * skipm);
      if (!need) {
        const uint32_t bw = __float_as_uint(dm * dm);
        b = bw > b ? bw : b;
      }
    }
    const uint64_t mask = __ballot(need);
    if (need) {
      const int pos = cnt + (int)__builtin_amdgcn_mbcnt_hi(
                                (uint32_t)(mask >> 32),
                                __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
      l_row[pos] = i;
      l_dm[pos] = dm;
    }
    cnt += __popcll(mask);
    if (cnt >= 64) {
      __syncthreads();
      run(64);
      __syncthreads();
      if (lane < cnt - 64) {
        l_row[lane] = l_row[64 + lane];
        l_dm[lane] = l_dm[64 + lane];
      }
      cnt -= 64;
    }
  }
  if (cnt > 0) {
    __syncthreads();
    run(cnt);
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint32_t o = __shfl_xor(b, m);
    b = o > b ? o : b;
  }
  if (lane == 0) atomicMax(&maxbits[(r + 1) * KP_SLOTS + blockIdx.x % KP_SLOTS], b);
}

// the max of pick r + 1's KP_SLOTS slots, through LDS to the whole block
__device__ inline float kpp_maxw(const uint32_t *maxbits, int r, uint32_t *sm) {
  if (threadIdx.x < 64) {
    uint32_t b = maxbits[(r + 1) * KP_SLOTS + threadIdx.x];
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
      const uint32_t o = __shfl_xor(b, m);
      b = o > b ? o : b;
    }
    if (threadIdx.x == 0) *sm = b;
  }
  __syncthreads();
  return __uint_as_float(*sm);
}

// the 32-bit fixed-point weight of D^2 (exact: one correctly rounded
// division, an exact scaling, truncation)
__device__ inline uint64_t kpp_fixed(float dm, float maxw) {
  if (!(maxw > 0.f)) return 0;
  const float w = dm * dm;
  return (uint64_t)((double)w / (double)maxw * 4294967296.0);
}

// bsum[b] = sum of the fixed weights of block b's rows
__global__ __launch_bounds__(KP_T) void k_kpp_blocksum(const float *D, int64_t n,
                                                       const uint32_t *maxbits,
                                                       const int64_t *chosen, int r,
                                                       uint64_t *bsum) {
  __shared__ uint64_t ws[KP_T / 64];
  __shared__ uint32_t s_mx;
  if (chosen[r] < 0) return;
  const float maxw = kpp_maxw(maxbits, r, &s_mx);
  const int64_t i = blockIdx.x * (int64_t)KP_T + threadIdx.x;
  uint64_t f = i < n ? kpp_fixed(D[i], maxw) : 0;
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint64_t lo = __shfl_xor((uint32_t)f, m), hi = __shfl_xor((uint32_t)(f >> 32), m);
    f += (hi << 32) | lo;
  }
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = f;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t s = 0;
    for (int j = 0; j < KP_T / 64; ++j) s += ws[j];
    bsum[blockIdx.x] = s;
  }
}

__device__ inline uint64_t shfl_up_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_up((uint32_t)v, o), hi = __shfl_up((uint32_t)(v >> 32), o);
  return ((uint64_t)hi << 32) | lo;
}

// exclusive prefix over a 1024-thread block of one uint64 per thread;
// *total receives the block's sum
__device__ uint64_t block_excl_u64(uint64_t v, uint64_t *wsum, uint64_t *total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  uint64_t incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t u = shfl_up_u64(incl, o);
    if (lane >= o) incl += u;
  }
  __syncthreads();
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  uint64_t before = 0, all = 0;
  for (int j = 0; j < (int)(blockDim.x >> 6); ++j) {
    if (j < w) before += wsum[j];
    all += wsum[j];
  }
  *total = all;
  return before + incl - v;
}

// pick r + 1: u = Int.random(in: 0..<total) from the SeedableRNG stream
// whose state is *rng; the chosen row is the first whose inclusive
// fixed-weight prefix exceeds u.  One block of 1024 threads.  total = 0
// (every row on a chosen centroid) is the reference's degenerateData
// (:235-237): chosen[r + 1] = -1.
__global__ __launch_bounds__(1024) void k_kpp_pick(const uint64_t *bsum, int64_t nb,
                                                   const float *D, int64_t n,
                                                   const uint32_t *maxbits,
                                                   uint64_t *rng, int r,
                                                   int64_t *chosen) {
  __shared__ uint64_t wsum[16];
  __shared__ uint64_t s_u, s_base;
  __shared__ int64_t s_blk, s_row;
  const int t = threadIdx.x;
  if (chosen[r] < 0) {
    if (t == 0) chosen[r + 1] = -1;
    return;
  }
  // the total
  uint64_t part = 0;
  for (int64_t b = t; b < nb; b += 1024) part += bsum[b];
  uint64_t total;
  (void)block_excl_u64(part, wsum, &total);
  if (total == 0) {
    if (t == 0) chosen[r + 1] = -1;
    return;
  }
  if (t == 0) {
    uint64_t st = *rng;
    s_u = swift_bounded(st, total);
    *rng = st;
    s_blk = -1;
    s_row = -1;
  }
  __syncthreads();
  const uint64_t u = s_u;
  // the block holding u
  uint64_t carry = 0;
  for (int64_t b0 = 0; b0 < nb; b0 += 1024) {
    const int64_t b = b0 + t;
    const uint64_t v = b < nb ? bsum[b] : 0;
    uint64_t tile;
    const uint64_t ex = carry + block_excl_u64(v, wsum, &tile);
    if (b < nb && v > 0 && ex <= u && u < ex + v) {
      s_blk = b;
      s_base = ex;
    }
    carry += tile;
    __syncthreads();
    if (s_blk >= 0) break;
  }
  // the row inside it (a block is always found: the blocks' sums partition
  // [0, total); the test keeps a broken invariant from reading out of range)
  const int64_t blk = s_blk;
  if (blk < 0) {
    if (t == 0) chosen[r + 1] = -1;
    return;
  }
  __shared__ uint32_t s_mx;
  const float maxw = kpp_maxw(maxbits, r, &s_mx);
  const int64_t i = blk * KP_T + t;
  const uint64_t f = (t < KP_T && i < n) ? kpp_fixed(D[i], maxw) : 0;
  uint64_t tot2;
  const uint64_t ex = s_base + block_excl_u64(f, wsum, &tot2);
  if (t < KP_T && i < n && f > 0 && ex <= u && u < ex + f) s_row = i;
  __syncthreads();
  if (t == 0) chosen[r + 1] = s_row;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static unsigned grid1d(int64_t n, int threads) {
  int64_t g = ceil_div(n, threads);
  return (unsigned)(g < 1 ? 1 : (g > 65535 * 32 ? 65535 * 32 : g));
}

// nearest centroid and its distance for each of the n rows of dx: the bf16
// screen with exact recomputation (qp.qh set) or the exact VALU scan
static void kmeans_assign(vsk_ctx *ctx, const float *cent, int32_t k, int32_t d,
                          int32_t ld, const float *dx, int64_t n, const ArgminQueries &qp,
                          int32_t *assign, float *dist) {
  if (qp.qh) {
    float *csq = static_cast<float *>(ctx->scratch_ptr("km.csq", sizeof(float) * (size_t)k));
    row_norms(ctx, cent, k, d, ld, csq, nullptr);
    screen_argmin(ctx, cent, csq, k, d, ld, dx, n, qp, assign, dist);
    return;
  }
  const int64_t chunk = 1 << 24;  // rows per launch (grid.x bound)
  for (int64_t r = 0; r < n; r += chunk) {
    const int64_t m = n - r < chunk ? n - r : chunk;
    FlatArgs a{};
    a.X = cent;
    a.ldx = ld;
    a.Q = dx + r * ld;
    a.ldq = ld;
    a.kdim = ld;
    a.nq = (int32_t)m;
    a.r0 = 0;
    a.r1 = k;
    a.metric = METRIC_L2_EXACT;
    a.amin = dist + r;
    launch_flat(ctx, a, MODE_ARGMIN, assign + r);
  }
}

// order[...] = the rows grouped by cluster, each cluster's rows ascending;
// off[c] = first position of cluster c, counts[c] = its rows
static void group_rows(vsk_ctx *ctx, const int32_t *assign, int64_t n, int32_t k,
                       int32_t *counts, int32_t *off, const int32_t **order) {
  KernelTimer tm(ctx, "kmeans_group", (double)n);
  fill_i32(ctx, counts, k, 0);
  k_count_clusters<<<grid1d(n, 256), 256, 0, ctx->stream>>>(assign, n, counts);
  check_launch("kmeans_count");
  VSK_HIP(hipMemcpyAsync(off, counts, sizeof(int32_t) * k, hipMemcpyDeviceToDevice,
                         ctx->stream));
  k_scan_excl<<<1, 1024, 0, ctx->stream>>>(off, k);
  check_launch("kmeans_scan");
  const int64_t nb = ceil_div(n, GR_B);
  int32_t *hist = static_cast<int32_t *>(
      ctx->scratch_ptr("km.hist", sizeof(int32_t) * 16 * (size_t)nb));
  int32_t *buf = static_cast<int32_t *>(
      ctx->scratch_ptr("km.radix", sizeof(int32_t) * 4 * (size_t)n));
  int32_t *ka = buf, *va = buf + n, *kb = buf + 2 * n, *vb = buf + 3 * n;
  const int32_t *kin = assign, *vin = nullptr;
  int shift = 0;
  do {
    k_grp_hist<<<(unsigned)nb, GR_T, 0, ctx->stream>>>(kin, n, shift, hist);
    check_launch("kmeans_radix_hist");
    k_scan_excl<<<1, 1024, 0, ctx->stream>>>(hist, 16 * nb);
    check_launch("kmeans_radix_scan");
    k_grp_scatter<<<(unsigned)nb, GR_T, 0, ctx->stream>>>(kin, vin, n, shift, hist,
                                                          ka, va);
    check_launch("kmeans_radix_scatter");
    kin = ka;
    vin = va;
    std::swap(ka, kb);
    std::swap(va, vb);
    shift += 4;
  } while (shift < 31 && ((k - 1) >> shift) > 0);
  *order = vin;
}

// the k starting rows of initializeRandom (:197-207): Fisher-Yates from the
// front on SeedableRNG(seed); positions touched are kept in a map
static std::vector<int64_t> init_random_rows(int64_t n, int32_t k, uint64_t seed) {
  std::unordered_map<int64_t, int64_t> perm;
  auto at = [&](int64_t i) {
    auto it = perm.find(i);
    return it == perm.end() ? i : it->second;
  };
  std::vector<int64_t> rows((size_t)k);
  uint64_t st = seed;
  for (int64_t i = 0; i < k; ++i) {
    if (i < n - 1) {
      const int64_t j = i + (int64_t)swift_bounded(st, (uint64_t)(n - i));
      const int64_t vi = at(i), vj = at(j);
      perm[i] = vj;
      perm[j] = vi;
    }
    rows[(size_t)i] = at(i);
  }
  return rows;
}

// k-means++ starting rows (see the file comment); false on degenerate data
static bool init_plusplus(vsk_ctx *ctx, const float *dx, int64_t n, int32_t d,
                          int32_t ld, int32_t k, uint64_t seed, int64_t *chosen) {
  KernelTimer tm(ctx, "kmeans_plusplus", (double)n * k);
  float *D = static_cast<float *>(ctx->scratch_ptr("km.kppD", sizeof(float) * (size_t)n));
  fill_i32(ctx, reinterpret_cast<int32_t *>(D), n, 0x7F800000);  // +inf
  int32_t *near = static_cast<int32_t *>(
      ctx->scratch_ptr("km.kppnear", sizeof(int32_t) * (size_t)n));
  fill_i32(ctx, near, n, -1);
  float *cc = static_cast<float *>(ctx->scratch_ptr("km.kppcc", sizeof(float) * (size_t)k));
  const float skipm = 1.0f + (float)(d + 4) * 0x1p-22f;
  uint32_t *maxbits = static_cast<uint32_t *>(
      ctx->scratch_ptr("km.kppmax", sizeof(uint32_t) * (size_t)(k + 1) * KP_SLOTS));
  fill_i32(ctx, reinterpret_cast<int32_t *>(maxbits), (int64_t)(k + 1) * KP_SLOTS, 0);
  const int64_t nb = ceil_div(n, KP_T);
  uint64_t *bsum = static_cast<uint64_t *>(
      ctx->scratch_ptr("km.kppbsum", sizeof(uint64_t) * (size_t)nb));
  // [first row, stream state after drawing it]
  uint64_t st = seed;
  const int64_t first = (int64_t)swift_bounded(st, (uint64_t)n);
  const uint64_t init[2] = {(uint64_t)first, st};
  uint64_t *rng = static_cast<uint64_t *>(ctx->scratch_ptr("km.kpprng", sizeof(uint64_t)));
  VSK_HIP(hipMemcpyAsync(chosen, &init[0], sizeof(int64_t), hipMemcpyHostToDevice,
                         ctx->stream));
  VSK_HIP(hipMemcpyAsync(rng, &init[1], sizeof(uint64_t), hipMemcpyHostToDevice,
                         ctx->stream));
  for (int r = 0; r + 1 < k; ++r) {
    if (r > 0)
      k_kpp_cc<<<(unsigned)ceil_div(r, 4), 256, 0, ctx->stream>>>(dx, ld, d, chosen, r, cc);
    k_kpp_update<<<(unsigned)std::min<int64_t>(ceil_div(n, 64), KPU_GRID), 64, 0,
                   ctx->stream>>>(
        dx, ld, d, n, chosen, r, cc, skipm, D, near, maxbits);
    k_kpp_blocksum<<<(unsigned)nb, KP_T, 0, ctx->stream>>>(D, n, maxbits, chosen, r,
                                                           bsum);
    k_kpp_pick<<<1, 1024, 0, ctx->stream>>>(bsum, nb, D, n, maxbits, rng, r, chosen);
  }
  check_launch("kmeans_plusplus");
  std::vector<int64_t> h((size_t)k);
  VSK_HIP(hipMemcpyAsync(h.data(), chosen, sizeof(int64_t) * k, hipMemcpyDeviceToHost,
                         ctx->stream));
  stream_sync(ctx);
  for (int64_t v : h)
    if (v < 0 || v >= n) return false;
  return true;
}

}  // namespace vsk

using namespace vsk;

vsk_status vsk_kmeans(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                      int32_t k, const float *weights, int32_t init_method,
                      const float *init_centroids, uint64_t seed,
                      int32_t max_iter, float tolerance, float *out_centroids,
                      int32_t *out_assign, vsk_kmeans_result *result) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "cannot cluster an empty dataset");
  VSK_REQUIRE(x && out_centroids && result, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(k > 0 && (int64_t)k <= n, VSK_ERR_INVALID_ARGUMENT,
              "invalid number of clusters: must be between 1 and the row count");
  VSK_REQUIRE(n <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "k-means takes at most 2^31-1 rows");
  VSK_REQUIRE(init_method == VSK_KMEANS_INIT_RANDOM ||
                  init_method == VSK_KMEANS_INIT_CUSTOM ||
                  init_method == VSK_KMEANS_INIT_PLUSPLUS,
              VSK_ERR_INVALID_ARGUMENT, "unknown initialisation method");
  VSK_REQUIRE(init_method != VSK_KMEANS_INIT_CUSTOM || init_centroids,
              VSK_ERR_INVALID_ARGUMENT, "custom initialisation needs k x d centroids");
  VSK_REQUIRE(max_iter >= 0, VSK_ERR_INVALID_ARGUMENT, "negative iteration limit");
  CallScope cs(ctx);
  const int32_t ld = padded_ld(d);
  const float *dx = rows_to_device_padded(ctx, x, n, d, ld, "km.x");
  const float *dw = weights ? static_cast<const float *>(input_to_device(
                                  ctx, weights, sizeof(float) * n, "km.w"))
                            : nullptr;
  float *cbuf = static_cast<float *>(
      ctx->scratch_ptr("km.cent", sizeof(float) * 2 * (size_t)k * ld));
  float *cur0 = cbuf;
  // starting centroids
  if (init_method == VSK_KMEANS_INIT_CUSTOM) {
    if (ld != d) fill_i32(ctx, reinterpret_cast<int32_t *>(cur0), (int64_t)k * ld, 0);
    copy_rows(ctx, cur0, sizeof(float) * ld, init_centroids, sizeof(float) * d,
              sizeof(float) * d, k);
  } else {
    int64_t *rows = static_cast<int64_t *>(
        ctx->scratch_ptr("km.rows", sizeof(int64_t) * (size_t)k));
    if (init_method == VSK_KMEANS_INIT_RANDOM) {
      std::vector<int64_t> h = init_random_rows(n, k, seed);
      VSK_HIP(hipMemcpyAsync(rows, h.data(), sizeof(int64_t) * k, hipMemcpyHostToDevice,
                             ctx->stream));
      stream_sync(ctx);  // h goes out of scope
    } else {
      VSK_REQUIRE(init_plusplus(ctx, dx, n, d, ld, k, seed, rows),
                  VSK_ERR_INVALID_ARGUMENT,
                  "data is degenerate (all points are identical)");
    }
    k_gather_rows_i64<<<grid1d((int64_t)k * ld, 256), 256, 0, ctx->stream>>>(
        dx, ld, rows, k, cur0);
    check_launch("kmeans_gather");
  }
  // assignments and distances double-buffered: iteration i + 1 runs while
  // iteration i's inertia is summed on the auxiliary stream
  int32_t *assign2 = static_cast<int32_t *>(
      ctx->scratch_ptr("km.assign", sizeof(int32_t) * 2 * (size_t)n));
  float *dist2 = static_cast<float *>(
      ctx->scratch_ptr("km.dist", sizeof(float) * 2 * (size_t)n));
  int32_t *counts = static_cast<int32_t *>(
      ctx->scratch_ptr("km.counts", sizeof(int32_t) * 2 * (size_t)k));
  int32_t *off = counts + k;
  float *cntf = static_cast<float *>(ctx->scratch_ptr("km.cntf", sizeof(float) * (size_t)k));
  float *dinert = static_cast<float *>(ctx->scratch_ptr("km.inertia", 2 * sizeof(float)));
  uint64_t *rng = static_cast<uint64_t *>(ctx->scratch_ptr("km.rng", sizeof(uint64_t)));
  fill_u64(ctx, rng, 1, seed + 0x9E3779B97F4A7C15ull);
  float *h_inert = static_cast<float *>(ctx->pinned_ptr(2 * sizeof(float)));
  hipStream_t aux = ctx->aux_stream();
  hipEvent_t ev_assigned[2] = {ctx->take_event(), ctx->take_event()};
  hipEvent_t ev_summed[2] = {ctx->take_event(), ctx->take_event()};
  // the rows' bf16 planes for the screened assignment, made once
  ArgminQueries qp;
  if (max_iter > 0 && screen_argmin_applies(ctx, n, k, d))
    qp = argmin_queries(ctx, dx, n, d, ld, "km.q");
  // one Lloyd iteration i: centroids cbuf[i & 1] -> cbuf[(i + 1) & 1]
  auto enqueue = [&](int32_t i) {
    const float *cur = cbuf + (size_t)(i & 1) * k * ld;
    float *nxt = cbuf + (size_t)((i + 1) & 1) * k * ld;
    int32_t *assign = assign2 + (size_t)(i & 1) * n;
    float *dist = dist2 + (size_t)(i & 1) * n;
    kmeans_assign(ctx, cur, k, d, ld, dx, n, qp, assign, dist);
    VSK_HIP(hipEventRecord(ev_assigned[i & 1], ctx->stream));
    VSK_HIP(hipStreamWaitEvent(aux, ev_assigned[i & 1], 0));
    {
      KernelTimer tm(ctx, "kmeans_inertia", (double)n, aux);
      k_seq_sum<<<1, 64, 0, aux>>>(dist, n, dinert + (i & 1));
      check_launch("kmeans_inertia");
    }
    VSK_HIP(hipMemcpyAsync(h_inert + (i & 1), dinert + (i & 1), sizeof(float),
                           hipMemcpyDeviceToHost, aux));
    VSK_HIP(hipEventRecord(ev_summed[i & 1], aux));
    const int32_t *order = nullptr;
    group_rows(ctx, assign, n, k, counts, off, &order);
    {
      KernelTimer tm(ctx, "kmeans_means", (double)n * d);
      dim3 grid((unsigned)k, (unsigned)ceil_div(ld, 64));
      k_cluster_means<<<grid, 64, 0, ctx->stream>>>(dx, ld, d, order, off, counts, dw, nxt,
                                                    cntf);
      check_launch("kmeans_means");
    }
    k_refill_empty<<<1, 64, 0, ctx->stream>>>(cntf, k, dx, ld, d, n, rng, nxt);
    check_launch("kmeans_refill");
  };
  float prev = INFINITY;
  int32_t it = 0;
  bool conv = false;
  if (max_iter > 0) enqueue(0);
  while (it < max_iter && !conv) {
    // the next iteration goes in before this one's inertia is known; if
    // this one converged, its results (other buffers) are discarded
    if (it + 1 < max_iter) enqueue(it + 1);
    VSK_HIP(hipEventSynchronize(ev_summed[it & 1]));
    const float inertia = h_inert[it & 1];
    conv = fabsf(inertia - prev) < tolerance;
    prev = inertia;
    ++it;
  }
  for (hipEvent_t e : {ev_assigned[0], ev_assigned[1], ev_summed[0], ev_summed[1]})
    ctx->event_pool.push_back(e);
  const float *cur = cbuf + (size_t)(it & 1) * k * ld;
  const int32_t *assign = assign2 + (size_t)((it + 1) & 1) * n;  // iteration it - 1
  if (it == 0) fill_i32(ctx, assign2 + n, n, 0);
  copy_rows(ctx, out_centroids, sizeof(float) * d, cur, sizeof(float) * ld,
            sizeof(float) * d, k);
  if (out_assign)
    VSK_HIP(hipMemcpyAsync(out_assign, assign, sizeof(int32_t) * n,
                           is_device_ptr(out_assign) ? hipMemcpyDeviceToDevice
                                                     : hipMemcpyDeviceToHost,
                           ctx->stream));
  cs.finish();
  result->iterations = it;
  result->converged = conv ? 1 : 0;
  result->inertia = it > 0 ? prev : INFINITY;
  VSK_API_END(ctx);
}
