// select.hip -- exact k-smallest selection over composite (distance, tie)
// keys, one workgroup per query, and the progressive chunked driver that
// keeps the full query x row distance matrix out of HBM.
//
// The reference selects on the CPU after reading back the whole distance
// matrix (Acceleration/MetalAccelerationEngine.swift:457-477) with a stable
// sort + prefix(k) (Indexes/IVFIndex.swift:175-176).  Here every distance
// carries its tie key in the low 32 bits, so all keys of a query are
// distinct and "the k smallest keys" is exactly the stable-sort prefix.
//
// Selection is a most-significant-digit radix select over the bits below
// the highest one where the query's smallest and largest keys differ: 8-bit
// digits (the last one narrower), each a 256-bin LDS histogram of the keys
// that still match the resolved prefix; it stops early as soon as the bucket
// holding the k-th key is taken whole.  The <= k winners are gathered into LDS and
// bitonic-sorted (at most 1024 of them).
#include <type_traits>

#include "flat.hpp"

namespace vsk {

constexpr int SEL_THREADS = 256;

// element i of a query's keys: the previous list, then the candidates --
// 64-bit keys, or (W32) 32-bit distances keyed by their index in the list
template <bool W32>
__device__ inline uint64_t sel_elem(const uint64_t *P, int64_t np, const uint64_t *C,
                                    const uint32_t *C32, int64_t i) {
  if constexpr (W32) return ((uint64_t)C32[i] << 32) | (uint32_t)i;
  return i < np ? P[i] : C[i - np];
}

// ascending bitonic sort of sel[0..m) in LDS by the whole block (sel holds
// the next power of two; the padding is NONE); ends with a barrier
__device__ void block_sort(uint64_t *sel, int m) {
  const int tid = threadIdx.x;
  int P2 = 1;
  while (P2 < m) P2 <<= 1;
  for (int i = m + tid; i < P2; i += SEL_THREADS) sel[i] = VSK_KEY_NONE;
  __syncthreads();
  for (int size = 2; size <= P2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < (P2 >> 1); i += SEL_THREADS) {
        int lo = 2 * i - (i & (stride - 1));
        int hi = lo + stride;
        bool up = (lo & size) == 0;
        uint64_t x = sel[lo], y = sel[hi];
        if ((x > y) == up) {
          sel[lo] = y;
          sel[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// block-wide shared state of a threshold search
struct SelShared {
  uint32_t hist[256 + 32];
  int bucket, take_all;
  uint32_t before, bcount;
  uint64_t lo[SEL_THREADS / 64], hi[SEL_THREADS / 64];
};

// Most-significant-digit radix search over one query's keys, which
// each_key(f) hands to f (every thread its share; NONE skipped): T_out is a
// key with exactly the k smallest keys at or below it, or take_all when
// there are at most k keys; hi_out the largest key.  Called by every
// thread of the block.
template <class EachKey>
__device__ void radix_threshold(EachKey &&each_key, int32_t k, SelShared &sh, uint64_t &T_out,
                                bool &take_all_out, uint64_t &hi_out) {
  const int tid = threadIdx.x, lane = tid & 63;
  // smallest and largest key: the digits start at the highest bit where
  // they differ (the distances of one query share their leading bits, and a
  // histogram of a digit every key agrees on is a pass spent on one bin)
  uint64_t lo = VSK_KEY_NONE, hi = 0;
  each_key([&](uint64_t key) {
    if (key == VSK_KEY_NONE) return;
    lo = key < lo ? key : lo;
    hi = key > hi ? key : hi;
  });
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t l2 = __shfl_xor(lo, o), h2 = __shfl_xor(hi, o);
    lo = l2 < lo ? l2 : lo;
    hi = h2 > hi ? h2 : hi;
  }
  if (lane == 0) {
    sh.lo[tid >> 6] = lo;
    sh.hi[tid >> 6] = hi;
  }
  __syncthreads();
  lo = sh.lo[0];
  hi = sh.hi[0];
#pragma unroll
  for (int wv = 1; wv < SEL_THREADS / 64; ++wv) {
    lo = sh.lo[wv] < lo ? sh.lo[wv] : lo;
    hi = sh.hi[wv] > hi ? sh.hi[wv] : hi;
  }

  uint64_t prefix = 0, mask = 0, T = VSK_KEY_NONE;
  int64_t need = k;
  bool take_all = false;
  // top: the highest undecided bit (inclusive); bits above it are common
  int top = 63;
  if (lo != VSK_KEY_NONE && lo != hi) {
    top = 63 - __builtin_clzll(lo ^ hi);
    mask = top == 63 ? 0 : ~((2ull << top) - 1);
    prefix = lo & mask;
  }
  bool first = true;

  while (top >= 0) {
    const int width = top + 1 >= 8 ? 8 : top + 1;
    const int shift = top + 1 - width;
    const uint32_t dmask = (1u << width) - 1;
    for (int i = tid; i < 256 + 32; i += SEL_THREADS) sh.hist[i] = 0;
    __syncthreads();
    // without branches: a key outside the prefix counts into one of 32
    // spare bins (distinct banks across a half-wave)
    const uint32_t spare = 256u + (uint32_t)(lane & 31);
    each_key([&](uint64_t key) {
      const bool in = key != VSK_KEY_NONE && (key & mask) == prefix;
      atomicAdd(&sh.hist[in ? (uint32_t)(key >> shift) & dmask : spare], 1u);
    });
    __syncthreads();
    if (tid < 64) {
      uint32_t h0 = sh.hist[4 * lane], h1 = sh.hist[4 * lane + 1],
               h2 = sh.hist[4 * lane + 2], h3 = sh.hist[4 * lane + 3];
      uint32_t s = h0 + h1 + h2 + h3;
      uint32_t incl = s;
      for (int o = 1; o < 64; o <<= 1) {
        uint32_t v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
      }
      uint32_t all = __shfl(incl, 63);
      uint32_t excl = incl - s;
      if (first && all <= (uint32_t)k) {
        if (lane == 0) sh.take_all = 1;
      } else {
        if (lane == 0) sh.take_all = 0;
        bool here = excl < (uint64_t)need && (uint64_t)need <= incl;
        if (here) {
          uint32_t hs[4] = {h0, h1, h2, h3};
          uint32_t before = excl;
          int j = 0;
          while (before + hs[j] < (uint64_t)need) {
            before += hs[j];
            ++j;
          }
          sh.bucket = 4 * lane + j;
          sh.before = before;
          sh.bcount = hs[j];
        }
      }
    }
    __syncthreads();
    if (sh.take_all) {
      take_all = true;
      break;
    }
    first = false;
    const uint32_t b = (uint32_t)sh.bucket;
    need -= sh.before;
    prefix |= (uint64_t)b << shift;
    mask |= (uint64_t)dmask << shift;
    const bool full = (uint64_t)sh.bcount == (uint64_t)need;
    __syncthreads();  // everyone has read the sh_* values
    if (full || shift == 0) {
      T = prefix | ~mask;
      break;
    }
    top = shift - 1;
  }

  T_out = T;
  take_all_out = take_all;
  hi_out = hi;
}

// in-register bitonic sort of R 64-bit keys a lane across the wave (key e
// at lane e / R, register e % R), ascending
template <int R>
__device__ void wave_sort_u64(uint64_t (&v)[R]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64 * R; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      if (j < R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r & j) continue;
          const bool asc = ((lane * R + r) & size) == 0;
          const uint64_t a = v[r], b = v[r + j];
          const bool sw = (a > b) == asc;
          v[r] = sw ? b : a;
          v[r + j] = sw ? a : b;
        }
      } else {
        const int lj = j / R;
        const bool lower = (lane & lj) == 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const bool asc = ((lane * R + r) & size) == 0;
          const uint64_t p = __shfl_xor(v[r], lj);
          const uint64_t mn = v[r] < p ? v[r] : p, mx = v[r] < p ? p : v[r];
          v[r] = lower == asc ? mn : mx;
        }
      }
    }
  }
}

// REG: keys per thread held in registers when a query's list fits (REG x
// SEL_THREADS keys): every pass then reads registers, not the list again.
// The registers cost occupancy, so only callers whose lists are a few
// thousand keys (IVF candidate segments, a dense chunk as small as the IVF
// probe's centroids) take it.
// W32: the candidates are a.cand32 (no previous list).  FAST: the short
// cut below for k <= 128 (its registers would slow the radix search of the
// other instances).  SEGB: a segmented list is read SEGB segments a wave
// at a time, one key a lane from each, every load issued before the first
// is used: with few queries a launch (a workgroup or two a CU) each pass
// otherwise waits on the memory latency once per segment.  The loads' registers
// cost occupancy, which launches of many queries need more.
template <int REG, bool W32, bool FAST = false, int SEGB = 0>
__global__ __launch_bounds__(SEL_THREADS) void k_select(SelectArgs a) {
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  if (a.active && !a.active[q]) return;

  const int32_t k = a.k;
  const uint64_t *P = a.prev ? a.prev + q * (int64_t)k : nullptr;
  const int64_t np = P ? k : 0;
  int64_t base = a.seg_off ? a.seg_off[q] : q * a.cap;
  int64_t cnt = a.counts ? (int64_t)a.counts[q]
                         : (a.seg_off ? a.seg_off[q + 1] - base : a.cap);
  bool overflow = false;
  if (a.counts && !a.seg_off && cnt > a.cap) {
    overflow = true;
    cnt = a.cap;
  }
  if (overflow) {
    if (tid == 0) {
      if (a.overflow_mask) a.overflow_mask[q] = 1;
      if (a.overflow_count) atomicAdd(a.overflow_count, 1);
    }
    return;
  }
  const uint64_t *C = W32 ? nullptr : a.cand + base;
  const uint32_t *C32 = W32 ? a.cand32 + base : nullptr;
  const int64_t total = np + cnt;
  // segmented lists: the segments' key counts in LDS; wave w walks the
  // segments w, w + 4, ... (64 lanes per segment)
  __shared__ int32_t seg_cnt[VSK_MAX_SEG];
  const bool seg = a.seg_n != nullptr;
  if (seg) {
    for (int s = tid; s < a.nseg; s += SEL_THREADS) seg_cnt[s] = a.seg_n[q * a.nseg + s];
    __syncthreads();
  }
  const bool inreg = REG > 0 && !seg && total <= (int64_t)REG * SEL_THREADS;  // uniform
  uint64_t regs[REG > 0 ? REG : 1];
  if (inreg) {
#pragma unroll
    for (int r = 0; r < REG; ++r) {
      const int64_t i = tid + (int64_t)r * SEL_THREADS;
      regs[r] = i < total ? sel_elem<W32>(P, np, C, C32, i) : VSK_KEY_NONE;
    }
  }
  auto each_key = [&](auto &&f) {
    if (inreg) {
#pragma unroll
      for (int r = 0; r < REG; ++r)
        if (tid + (int64_t)r * SEL_THREADS < total) f(regs[r]);
      return;
    }
    if (!seg) {
      for (int64_t i = tid; i < total; i += SEL_THREADS) f(sel_elem<W32>(P, np, C, C32, i));
      return;
    }
    for (int64_t i = tid; i < np; i += SEL_THREADS) f(P[i]);
    if constexpr (SEGB > 0) {
      // keys past a segment's first 64 follow the batch
      const uint64_t *cq = a.cand + q * a.cap;
      for (int s0 = tid >> 6; s0 < a.nseg; s0 += SEGB * (SEL_THREADS / 64)) {
        uint64_t v[SEGB];
#pragma unroll
        for (int u = 0; u < SEGB; ++u) {
          const int s = s0 + u * (SEL_THREADS / 64);
          const int32_t ns = s < a.nseg ? seg_cnt[s] : 0;
          v[u] = lane < ns ? cq[(int64_t)s * a.seg_stride + lane] : VSK_KEY_NONE;
        }
#pragma unroll
        for (int u = 0; u < SEGB; ++u)
          if (v[u] != VSK_KEY_NONE) f(v[u]);
#pragma unroll
        for (int u = 0; u < SEGB; ++u) {
          const int s = s0 + u * (SEL_THREADS / 64);
          const int32_t ns = s < a.nseg ? seg_cnt[s] : 0;
          for (int32_t j = lane + 64; j < ns; j += 64) f(cq[(int64_t)s * a.seg_stride + j]);
        }
      }
      return;
    }
    for (int s = tid >> 6; s < a.nseg; s += SEL_THREADS / 64) {
      const uint64_t *cs = a.cand + q * a.cap + (int64_t)s * a.seg_stride;
      const int32_t ns = seg_cnt[s];
      for (int32_t j = lane; j < ns; j += 64) f(cs[j]);
    }
  };

  __shared__ SelShared sh;
  __shared__ uint64_t sel[VSK_MAX_K];
  __shared__ int sel_count;
  // Short cut for k <= 128 over a list in registers: each wave's k-th
  // smallest of its lanes' smallest keys (k <= 64) or of their two smallest
  // keys (k <= 128) has k keys at or below it, so the smallest of those
  // over the waves, B, does too; the k smallest keys are among the keys at
  // or below B (a few times k), which are sorted: by one wave in registers
  // (at most 512 of them), else by the block in LDS (at most 1,024).  More
  // of them, or fewer than k values in every wave, takes the radix search.
  // The output is sorted whether or not it was asked for.
  if (FAST && REG > 0 && inreg && k <= 128) {
    uint64_t wk;
    if (k <= 64) {
      uint64_t mn = VSK_KEY_NONE;
      each_key([&](uint64_t key) { mn = key < mn ? key : mn; });
      uint64_t v1[1] = {mn};
      wave_sort_u64<1>(v1);
      wk = __shfl(v1[0], k - 1);
    } else {
      uint64_t m1 = VSK_KEY_NONE, m2 = VSK_KEY_NONE;  // m1 <= m2
      each_key([&](uint64_t key) {
        const uint64_t lo = key < m1 ? key : m1, up = key < m1 ? m1 : key;
        m2 = up < m2 ? up : m2;
        m1 = lo;
      });
      uint64_t v2[2] = {m1, m2};
      wave_sort_u64<2>(v2);  // element e at lane e / 2, register e % 2
      const uint64_t c0 = __shfl(v2[0], (k - 1) >> 1), c1 = __shfl(v2[1], (k - 1) >> 1);
      wk = ((k - 1) & 1) ? c1 : c0;
    }
    if (lane == 0) sh.lo[tid >> 6] = wk;
    if (tid == 0) sel_count = 0;
    __syncthreads();
    uint64_t B = sh.lo[0];
#pragma unroll
    for (int i = 1; i < SEL_THREADS / 64; ++i) B = sh.lo[i] < B ? sh.lo[i] : B;
    if (B != VSK_KEY_NONE) {
      each_key([&](uint64_t key) {
        if (key <= B) {
          const int slot = atomicAdd(&sel_count, 1);
          if (slot < VSK_MAX_K) sel[slot] = key;
        }
      });
    }
    __syncthreads();
    const int c = sel_count;
    if (B != VSK_KEY_NONE && c > 512 && c <= VSK_MAX_K) {
      block_sort(sel, c);
      uint64_t *out = a.best_out + q * (int64_t)k;
      for (int i = tid; i < k; i += SEL_THREADS) out[i] = sel[i];
      if (tid == 0 && a.thresh) a.thresh[q] = sel[k - 1];
      return;
    }
    if (B != VSK_KEY_NONE && c <= 512) {
      if (tid < 64) {
        uint64_t *out = a.best_out + q * (int64_t)k;
        auto finish = [&](auto rtag) {
          constexpr int R = decltype(rtag)::value;
          uint64_t r[R];
#pragma unroll
          for (int i = 0; i < R; ++i) {
            const int e = lane * R + i;
            r[i] = e < c ? sel[e] : VSK_KEY_NONE;
          }
          wave_sort_u64<R>(r);
#pragma unroll
          for (int i = 0; i < R; ++i) {
            const int e = lane * R + i;
            if (e < k) out[e] = r[i];
            if (e == k - 1 && a.thresh) a.thresh[q] = r[i];
          }
        };
        if (c <= 64) finish(std::integral_constant<int, 1>{});
        else if (c <= 128) finish(std::integral_constant<int, 2>{});
        else if (c <= 256) finish(std::integral_constant<int, 4>{});
        else finish(std::integral_constant<int, 8>{});
      }
      return;
    }
    __syncthreads();  // sel_count and sh.lo are read; the radix search reuses them
  }
  uint64_t T, hi;
  bool take_all;
  radix_threshold(each_key, k, sh, T, take_all, hi);

  if (tid == 0) sel_count = 0;
  __syncthreads();
  each_key([&](uint64_t key) {
    if (key != VSK_KEY_NONE && (take_all || key <= T)) {
      int pos = atomicAdd(&sel_count, 1);
      if (pos < VSK_MAX_K) sel[pos] = key;
    }
  });
  __syncthreads();
  int m = sel_count;
  if (m > k) m = k;  // cannot happen with distinct keys; keeps LDS in range
  if (!a.sorted) {
    // the set and a threshold: T bounds the selected keys and no other key
    // lies at or below it (taken whole: the largest key)
    uint64_t *out = a.best_out + q * (int64_t)k;
    for (int i = tid; i < k; i += SEL_THREADS) out[i] = i < m ? sel[i] : VSK_KEY_NONE;
    if (tid == 0 && a.thresh) a.thresh[q] = m < k ? VSK_KEY_NONE : (take_all ? hi : T);
    return;
  }
  block_sort(sel, m);
  uint64_t *out = a.best_out + q * (int64_t)k;
  for (int i = tid; i < k; i += SEL_THREADS)
    out[i] = i < m ? sel[i] : VSK_KEY_NONE;
  if (tid == 0 && a.thresh) a.thresh[q] = (m >= k) ? sel[k - 1] : VSK_KEY_NONE;
}

// Short lists (at most 1,024 keys a query, counts given): one wave per
// query sorts its whole list in registers -- a bitonic network over 64 R
// keys, R a lane (R the smallest power of two holding the list), the
// partner of key e at distance j in the same lane when j < R, else in lane
// ^ j / R by a shuffle -- and writes the first k.  No LDS, no barrier.
template <int R>
__device__ void wave_sort_write(const uint64_t *C, int64_t n, int32_t k, uint64_t *out) {
  const int lane = threadIdx.x & 63;
  uint64_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t e = (int64_t)lane * R + r;
    v[r] = e < n ? C[e] : VSK_KEY_NONE;
  }
#pragma unroll
  for (int size = 2; size <= 64 * R; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      if (j < R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r & j) continue;
          const int e = lane * R + r;  // the lower of the pair
          const bool asc = (e & size) == 0;
          const uint64_t a = v[r], b = v[r + j];
          const bool sw = (a > b) == asc;
          v[r] = sw ? b : a;
          v[r + j] = sw ? a : b;
        }
      } else {
        const int lj = j / R;
        const bool lower = (lane & lj) == 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int e = lane * R + r;
          const bool asc = (e & size) == 0;
          const uint64_t p = __shfl_xor(v[r], lj);
          const uint64_t mn = v[r] < p ? v[r] : p, mx = v[r] < p ? p : v[r];
          v[r] = lower == asc ? mn : mx;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int e = lane * R + r;
    if (e < k) out[e] = v[r];
  }
}

__global__ __launch_bounds__(SEL_THREADS) void k_select_small(SelectArgs a) {
  const int64_t q = (int64_t)blockIdx.x * (SEL_THREADS / 64) + (threadIdx.x >> 6);
  if (q >= a.nq || (a.active && !a.active[q])) return;
  const uint64_t *C = a.cand + q * a.cap;
  int64_t n = a.counts[q];
  if (n > a.cap) n = a.cap;  // callers mark such queries inactive
  uint64_t *out = a.best_out + q * (int64_t)a.k;
  const int lane = threadIdx.x & 63;
  for (int i = lane + (int)(n < a.k ? n : a.k); i < a.k; i += 64) out[i] = VSK_KEY_NONE;
  if (n <= 64) wave_sort_write<1>(C, n, a.k, out);
  else if (n <= 128) wave_sort_write<2>(C, n, a.k, out);
  else if (n <= 256) wave_sort_write<4>(C, n, a.k, out);
  else if (n <= 512) wave_sort_write<8>(C, n, a.k, out);
  else wave_sort_write<16>(C, n, a.k, out);
}

// the margin gather (declared with MarginArgs).  Only the k-th smallest
// screened distance matters here, not which key holds it, so the search is
// a radix select over the 32-bit words themselves (ties counted): at most
// four 8-bit digits below the highest bit where the smallest and largest
// word differ, each a 256-bin histogram taken without branches (a word
// outside the prefix counts into one of 32 spare bins).  REG words per
// thread stay in registers when the list fits, loaded 16 bytes at a time;
// longer lists are read from memory on every pass.

struct WordShared {
  uint32_t hist[256 + 32];
  uint32_t lo[SEL_THREADS / 64], hi[SEL_THREADS / 64];
  uint32_t bucket, before, total;
};

// The k-th smallest of the words each(f) hands to f(word, index) (ties
// counted; kWordNone words skipped), kWordNone when there are fewer than k.
// stop_span > 0: the search may stop early once the words left in the
// k-th's bucket span less than stop_span as floats, returning the bucket's
// largest word (at or above the k-th).  Called by every thread of the block.
template <class Each>
__device__ uint32_t word_kth(Each &&each, uint32_t k, WordShared &sh, double stop_span) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t lo = kWordNone, hi = 0;
  each([&](uint32_t x, uint32_t) {
    if (x != kWordNone) {
      lo = x < lo ? x : lo;
      hi = x > hi ? x : hi;
    }
  });
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = min(lo, (uint32_t)__shfl_xor(lo, o));
    hi = max(hi, (uint32_t)__shfl_xor(hi, o));
  }
  if (lane == 0) {
    sh.lo[wv] = lo;
    sh.hi[wv] = hi;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < SEL_THREADS / 64; ++i) {
    lo = min(lo, sh.lo[i]);
    hi = max(hi, sh.hi[i]);
  }
  __syncthreads();  // sh.lo / sh.hi read by every thread
  if (lo == kWordNone) return kWordNone;
  uint32_t prefix = lo, mask = 0xFFFFFFFFu, need = k;
  int top = -1;
  if (lo != hi) {
    top = 31 - __builtin_clz(lo ^ hi);
    mask = top == 31 ? 0u : ~((2u << top) - 1u);
    prefix = lo & mask;
  }
  bool first = true;
  while (top >= 0) {
    const int width = top + 1 >= 8 ? 8 : top + 1;
    const int shift = top + 1 - width;
    const uint32_t dmask = (1u << width) - 1u;
    for (int i = tid; i < 256 + 32; i += SEL_THREADS) sh.hist[i] = 0;
    __syncthreads();
    // without branches: a word outside the prefix counts into one of 32
    // spare bins
    const uint32_t spare = 256u + (uint32_t)(lane & 31);
    each([&](uint32_t x, uint32_t) {
      const bool in = x != kWordNone && (x & mask) == prefix;
      atomicAdd(&sh.hist[in ? (x >> shift) & dmask : spare], 1u);
    });
    __syncthreads();
    if (tid < 64) {
      const uint32_t h0 = sh.hist[4 * lane], h1 = sh.hist[4 * lane + 1],
                     h2 = sh.hist[4 * lane + 2], h3 = sh.hist[4 * lane + 3];
      const uint32_t s4 = h0 + h1 + h2 + h3;
      uint32_t incl = s4;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
      }
      const uint32_t excl = incl - s4;
      if (lane == 63) sh.total = incl;
      if (excl < need && need <= incl) {
        const uint32_t hs[4] = {h0, h1, h2, h3};
        uint32_t before = excl;
        int j = 0;
        while (before + hs[j] < need) {
          before += hs[j];
          ++j;
        }
        sh.bucket = 4 * lane + j;
        sh.before = before;
      }
    }
    __syncthreads();
    if (first && sh.total < need) {
      __syncthreads();
      return kWordNone;  // fewer than k words
    }
    first = false;
    need -= sh.before;
    prefix |= sh.bucket << shift;
    mask |= dmask << shift;
    __syncthreads();  // every thread has read the shared values
    top = shift - 1;
    if (stop_span > 0 && top >= 0 &&
        (double)vsk_ord2f(prefix | ~mask) - (double)vsk_ord2f(prefix) < stop_span) {
      prefix |= ~mask;  // the bucket's largest word
      break;
    }
  }
  return prefix;
}

// One query's words, word i at W[i] for i < n (W 16-byte aligned, words
// readable up to the next multiple of 4): REG a thread in registers when
// they fit, loaded 16 bytes at a time, else read from memory on each pass.
template <int REG>
struct WordList {
  const uint32_t *W;
  int64_t n;
  bool inreg;
  int chunks;
  uint32_t w[REG];
  __device__ void load(const uint32_t *W_, int64_t n_) {
    W = W_;
    n = n_;
    inreg = n <= (int64_t)REG * SEL_THREADS;  // uniform
    chunks = (int)((n + 4 * SEL_THREADS - 1) / (4 * SEL_THREADS));
    if (!inreg) return;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < REG / 4; ++j) {
      const int64_t c = 4 * (tid + (int64_t)j * SEL_THREADS);
      uint4 v = make_uint4(kWordNone, kWordNone, kWordNone, kWordNone);
      if (c < n) v = *reinterpret_cast<const uint4 *>(W + c);
      w[4 * j] = c < n ? v.x : kWordNone;
      w[4 * j + 1] = c + 1 < n ? v.y : kWordNone;
      w[4 * j + 2] = c + 2 < n ? v.z : kWordNone;
      w[4 * j + 3] = c + 3 < n ? v.w : kWordNone;
    }
  }
  // f(word, index) over this thread's share (kWordNone for padding)
  template <class F>
  __device__ void each(F &&f) const {
    const int tid = threadIdx.x;
    if (inreg) {
#pragma unroll
      for (int j = 0; j < REG / 4; ++j) {
        if (j >= chunks) break;  // uniform
#pragma unroll
        for (int e = 0; e < 4; ++e) f(w[4 * j + e], 4 * (tid + j * SEL_THREADS) + e);
      }
      return;
    }
    for (int64_t i = tid; i < n; i += SEL_THREADS) f(W[i], (uint32_t)i);
  }
};

// One query's compact candidates (ScreenTailArgs::pcnt): probe slot p's are
// entries pre[p] .. pre[p + 1] - 1, stored from the slot's base pb[p] of the
// query's word segment W, with their rows' offsets in the list at the same
// places of R; an entry's position is pb[p] plus that offset.  pb and pre
// (np + 1 values) sit in LDS.  REG entries a thread in registers when they
// fit, else read from memory on each pass.
template <int REG>
struct CompactList {
  const uint32_t *W, *R;
  const int64_t *pb;
  const int32_t *pre;
  int np, n;
  bool inreg;
  uint32_t w[REG], pos[REG];
  __device__ void at(int e, uint32_t &x, uint32_t &i) const {
    int lo = 0, hi = np;  // the last slot whose first entry is at or below e
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pre[mid] <= e) lo = mid;
      else hi = mid;
    }
    const int64_t o = pb[lo] + (e - pre[lo]);
    x = W[o];
    i = (uint32_t)(pb[lo] + R[o]);
  }
  __device__ void load(const uint32_t *W_, const uint32_t *R_, const int64_t *pb_,
                       const int32_t *pre_, int np_) {
    W = W_;
    R = R_;
    pb = pb_;
    pre = pre_;
    np = np_;
    n = pre[np];
    inreg = n <= REG * SEL_THREADS;  // uniform
    if (!inreg) return;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < REG; ++j) {
      const int e = tid + j * SEL_THREADS;
      w[j] = kWordNone;
      pos[j] = 0;
      if (e < n) at(e, w[j], pos[j]);
    }
  }
  // f(word, position) over this thread's share (kWordNone for padding)
  template <class F>
  __device__ void each(F &&f) const {
    const int tid = threadIdx.x;
    if (inreg) {
#pragma unroll
      for (int j = 0; j < REG; ++j) {
        if (j * SEL_THREADS >= n) break;  // uniform
        f(w[j], pos[j]);
      }
      return;
    }
    for (int e = tid; e < n; e += SEL_THREADS) {
      uint32_t x, i;
      at(e, x, i);
      f(x, i);
    }
  }
};

// in-register bitonic sort of R 32-bit values a lane across the wave
// (value e at lane e / R, register e % R), ascending
template <int R>
__device__ void wave_sort_u32(uint32_t (&v)[R]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64 * R; size <<= 1) {
#pragma unroll
    for (int j = size >> 1; j > 0; j >>= 1) {
      if (j < R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r & j) continue;
          const bool asc = ((lane * R + r) & size) == 0;
          const uint32_t a = v[r], b = v[r + j];
          const bool sw = (a > b) == asc;
          v[r] = sw ? b : a;
          v[r + j] = sw ? a : b;
        }
      } else {
        const int lj = j / R;
        const bool lower = (lane & lj) == 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const bool asc = ((lane * R + r) & size) == 0;
          const uint32_t p = __shfl_xor(v[r], lj);
          const uint32_t mn = v[r] < p ? v[r] : p, mx = v[r] < p ? p : v[r];
          v[r] = lower == asc ? mn : mx;
        }
      }
    }
  }
}

// The k-th smallest word (ties counted; kWordNone when fewer than k) by a
// bound first: each wave's k-th smallest per-lane minimum has k words at or
// below it, so the smallest of those over the waves, T, does too, and the
// k-th smallest word is among the words at or below T -- usually a few
// times k of them, gathered into LDS and sorted by one wave.  k <= 64;
// more than 512 words at or below T (or fewer than k lanes holding words in
// every wave) falls back to word_kth.  Called by every thread of the block.
struct KthShared {
  WordShared w;
  uint32_t wmin[SEL_THREADS / 64];
  uint32_t g[512];
  int cnt;
  uint32_t kth;
};
template <class Each>
__device__ uint32_t word_kth_fast(Each &&each, uint32_t k, KthShared &sh, double stop_span) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (k == 0 || k > 64) return word_kth(each, k, sh.w, stop_span);
  uint32_t m = kWordNone;
  each([&](uint32_t x, uint32_t) { m = x < m ? x : m; });
  uint32_t v[1] = {m};
  wave_sort_u32<1>(v);
  const uint32_t wk = __shfl(v[0], (int)k - 1);
  if (lane == 0) sh.wmin[wv] = wk;
  if (tid == 0) sh.cnt = 0;
  __syncthreads();
  uint32_t T = sh.wmin[0];
#pragma unroll
  for (int i = 1; i < SEL_THREADS / 64; ++i) T = min(T, sh.wmin[i]);
  if (T == kWordNone) {  // no wave has k lanes holding words
    __syncthreads();
    return word_kth(each, k, sh.w, stop_span);
  }
  each([&](uint32_t x, uint32_t) {
    if (x <= T) {
      const int slot = atomicAdd(&sh.cnt, 1);
      if (slot < 512) sh.g[slot] = x;
    }
  });
  __syncthreads();
  const int c = sh.cnt;
  if (c > 512) {
    __syncthreads();
    return word_kth(each, k, sh.w, stop_span);
  }
  if (wv == 0) {
    // c >= k words; sort them in the smallest register width that holds them
    auto pick = [&](auto rtag) {
      constexpr int R = decltype(rtag)::value;
      uint32_t r[R];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int e = lane * R + i;
        r[i] = e < c ? sh.g[e] : kWordNone;
      }
      wave_sort_u32<R>(r);
      const int e = (int)k - 1;
#pragma unroll
      for (int i = 0; i < R; ++i)
        if (lane * R + i == e) sh.kth = r[i];
    };
    if (c <= 64) pick(std::integral_constant<int, 1>{});
    else if (c <= 128) pick(std::integral_constant<int, 2>{});
    else if (c <= 256) pick(std::integral_constant<int, 4>{});
    else pick(std::integral_constant<int, 8>{});
  }
  __syncthreads();
  const uint32_t kth = sh.kth;
  __syncthreads();  // every thread has read it
  return kth;
}

template <int REG>
__global__ __launch_bounds__(SEL_THREADS) void k_screen_margin(MarginArgs a) {
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  WordList<REG> L;
  L.load(a.words + (a.wseg ? a.wseg[q] : q * a.wstride), a.cnt ? a.cnt[q] : a.wn);
  auto each = [&](auto &&f) { L.each(f); };
  __shared__ KthShared sh;
  __shared__ int s_cnt;
  // the k-th smallest word (kWordNone: fewer than k words), or a word a
  // little above it: the search stops once the words left in the k-th's
  // bucket span less than 1/64 of the margin (the limit then only grows by
  // that much, and every key it adds is rescored like the others)
  const double eps = screen_eps_of(a.qnh[q], a.qnr[q], a.xh, a.xr, a.d, a.metric, a.nprod);
  const uint32_t kth = word_kth_fast(each, (uint32_t)a.k, sh, 0x1p-6 * eps);
  // every key when there are fewer than k, else those within the margin
  uint32_t lim_word = kWordNone - 1u;
  if (kth != kWordNone) {
    const double ak = vsk_ord2f(kth);
    const double lim = a.metric == VSK_METRIC_L2 ? (ak + eps) * (1.0 + 0x1p-20) + eps
                                                 : ak + 2.0 * eps;
    lim_word = vsk_f2ord(f_down(lim));
  }
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  uint64_t *out = a.out + q * (int64_t)a.cap;
  each([&](uint32_t x, uint32_t i) {
    if (x <= lim_word) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < a.cap) out[slot] = ((uint64_t)x << 32) | i;
    }
  });
  __syncthreads();
  if (tid == 0) {
    const int c = s_cnt;
    a.nout[q] = c;
    a.ok[q] = c <= a.cap ? 1 : 0;
    a.bad[q] = c <= a.cap ? 0 : 1;
    if (c > a.cap && a.nbad) atomicAdd(a.nbad, 1ull);
  }
}

void launch_screen_margin(vsk_ctx *ctx, const MarginArgs &a) {
  if (a.nq <= 0) return;
  KernelTimer t(ctx, "screen_margin");
  k_screen_margin<32><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  check_launch("screen_margin");
}

// the screen tail (declared with ScreenTailArgs)
__device__ inline float tail_exact(const float *x, const float *sq, int32_t ld, int32_t squared) {
#pragma clang fp contract(off)
  float acc = 0.f;
  for (int c0 = 0; c0 < ld; c0 += 32) {
    const int m = ld - c0 < 32 ? (ld - c0) >> 2 : 8;  // ld is a multiple of 4
    float4 xv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u < m) xv[u] = *reinterpret_cast<const float4 *>(x + c0 + 4 * u);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u < m) {
        const float4 qv = *reinterpret_cast<const float4 *>(sq + c0 + 4 * u);
        float t;
        t = qv.x - xv[u].x;
        acc = acc + t * t;
        t = qv.y - xv[u].y;
        acc = acc + t * t;
        t = qv.z - xv[u].z;
        acc = acc + t * t;
        t = qv.w - xv[u].w;
        acc = acc + t * t;
      }
  }
  return squared ? acc : sqrtf(acc);
}

__device__ inline int64_t tail_row(const ScreenTailArgs &t, int64_t q, int64_t p,
                                   const int64_t *lpb, const int64_t *llr);

// The exact keys of keys[0 .. c) in place, L lanes a key (L a power of two,
// 32 L >= ld): lane s of a group loads columns [32 s, 32 s + 32) of the
// row, so every load of a round is in flight at once, and the sequential
// sum passes from lane to lane -- lane s adds its 32 products to what lane
// s - 1 handed on -- which keeps the order of the one-thread sum.
__device__ void tail_rescore(uint64_t *keys, int c, const ScreenTailArgs &t, int64_t q,
                             const float *sq, const int64_t *lpb, const int64_t *llr) {
#pragma clang fp contract(off)
  const int L = t.ld <= 32 ? 1 : t.ld <= 64 ? 2 : t.ld <= 128 ? 4 : 8;
  const int tid = threadIdx.x, s = tid & (L - 1);
  const int c0 = 32 * s;
  const int m = t.ld - c0 >= 32 ? 8 : (t.ld > c0 ? (t.ld - c0) >> 2 : 0);  // ld: multiple of 4
  for (int b = 0; b < c; b += SEL_THREADS / L) {  // uniform
    const int i = b + tid / L;
    int64_t p = 0;
    float4 xv[8];
    if (i < c) {
      p = (int64_t)(uint32_t)keys[i];
      const float *x = t.rows + tail_row(t, q, p, lpb, llr) * t.ld + c0;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (u < m) xv[u] = *reinterpret_cast<const float4 *>(x + 4 * u);
    }
    float acc = 0.f;
    for (int step = 0; step < L; ++step) {  // uniform
      const float in = __shfl_up(acc, 1, L);
      if (s == step) {
        float a = step == 0 ? 0.f : in;
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (u < m) {
            const float4 qv = *reinterpret_cast<const float4 *>(sq + c0 + 4 * u);
            float d;
            d = qv.x - xv[u].x;
            a = a + d * d;
            d = qv.y - xv[u].y;
            a = a + d * d;
            d = qv.z - xv[u].z;
            a = a + d * d;
            d = qv.w - xv[u].w;
            a = a + d * d;
          }
        acc = a;
      }
    }
    if (i < c && s == L - 1) keys[i] = vsk_key(t.squared ? acc : sqrtf(acc), (uint32_t)p);
  }
}

// (lpb, llr: the query's probe bases and their lists' first rows, in LDS,
// or null to read them from memory)
__device__ inline int64_t tail_row(const ScreenTailArgs &t, int64_t q, int64_t p,
                                   const int64_t *lpb, const int64_t *llr) {
  if (!t.list_off) return p;
  if (lpb) {
    int lo = 0, hi = t.np;  // the last slot whose base is at or below p
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (lpb[mid] <= p) lo = mid;
      else hi = mid;
    }
    return llr[lo] + (p - lpb[lo]);
  }
  const int64_t *pb = t.pos_base + q * t.np;
  const int32_t *pr = t.probes + q * t.np;
  int lo = 0, hi = t.np;  // the last slot whose base is at or below p
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (pb[mid] <= p) lo = mid;
    else hi = mid;
  }
  return t.list_off[pr[lo]] + (p - pb[lo]);
}

// CMP: compact candidates (t.pcnt), 8 a thread in registers
template <int REG, bool CMP>
__global__ __launch_bounds__(SEL_THREADS) void k_screen_tail(ScreenTailArgs t) {
  const MarginArgs &a = t.m;
  const int64_t q = blockIdx.x;
  if (t.active && !t.active[q]) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t wbase = a.wseg ? a.wseg[q] : q * a.wstride;
  WordList<CMP ? 1 : REG> L;
  CompactList<CMP ? 8 : 1> C;
  if constexpr (!CMP) L.load(a.words + wbase, a.cnt ? a.cnt[q] : a.wn);
  auto each = [&](auto &&f) {
    if constexpr (CMP) C.each(f);
    else L.each(f);
  };
  __shared__ KthShared sh;
  __shared__ SelShared ssel;
  __shared__ uint64_t keys[VSK_MAX_K];
  __shared__ __attribute__((aligned(16))) float s_q[256];
  __shared__ int s_cnt;
  // the query's probe bases and their lists' first rows (a candidate's
  // row is found by a search over the bases: in LDS, not 7 dependent
  // global loads)
  __shared__ int64_t s_pb[256], s_lr[256];
  const bool lcache = t.list_off && t.np <= 256;
  if (lcache)
    for (int i = tid; i < t.np; i += SEL_THREADS) {
      s_pb[i] = t.pos_base[q * t.np + i];
      s_lr[i] = t.list_off[t.probes[q * t.np + i]];
    }
  const int64_t *lpb = lcache ? s_pb : nullptr, *llr = lcache ? s_lr : nullptr;
  // the query too, read while the k-th word is found
  for (int c = tid; c < t.ld; c += SEL_THREADS) s_q[c] = t.Q[q * t.ld + c];
  if constexpr (CMP) {
    // the probe slots' first entries (an exclusive scan of their kept
    // counts by wave 0, four slots a lane; np <= 256) and the total
    __shared__ int32_t s_pre[257];
    if (tid < 64) {
      const int64_t *pb = t.pos_base + q * t.np;
      int32_t v[4], sum = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = 4 * lane + u;
        v[u] = 0;
        if (p < t.np) {
          const int64_t size = (p + 1 < t.np ? pb[p + 1] : a.cnt[q]) - pb[p];
          v[u] = size > 0 ? t.pcnt[q * t.np + p] : 0;
        }
        sum += v[u];
      }
      int32_t incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      int32_t run = incl - sum;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = 4 * lane + u;
        if (p < t.np) s_pre[p] = run;
        run += v[u];
      }
      if (lane == 63) s_pre[t.np] = incl;
    }
    __syncthreads();
    C.load(a.words + wbase, t.prow + wbase, s_pb, s_pre, t.np);
  }
  const double eps = screen_eps_of(a.qnh[q], a.qnr[q], a.xh, a.xr, a.d, a.metric, a.nprod);
  const uint32_t kth = word_kth_fast(each, (uint32_t)a.k, sh, 0x1p-6 * eps);
  uint32_t lim_word = kWordNone - 1u;  // every key when there are fewer than k
  if (kth != kWordNone) {
    const double ak = vsk_ord2f(kth);
    const double lim = a.metric == VSK_METRIC_L2 ? (ak + eps) * (1.0 + 0x1p-20) + eps
                                                 : ak + 2.0 * eps;
    lim_word = vsk_f2ord(f_down(lim));
  }
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  each([&](uint32_t x, uint32_t i) {
    if (x <= lim_word) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < a.cap) keys[slot] = ((uint64_t)x << 32) | i;
    }
  });
  __syncthreads();
  const int c = s_cnt;
  const int32_t k = a.k;
  uint64_t *out = t.best_out + q * (int64_t)k;
  if (c <= a.cap) {
    tail_rescore(keys, c, t, q, s_q, lpb, llr);
    __syncthreads();
    if (tid < 64) {
      for (int i = c + lane; i < k; i += 64) out[i] = VSK_KEY_NONE;
      auto finish = [&](auto rtag) {
        constexpr int R = decltype(rtag)::value;
        uint64_t r[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
          const int e = lane * R + i;
          r[i] = e < c ? keys[e] : VSK_KEY_NONE;
        }
        wave_sort_u64<R>(r);
#pragma unroll
        for (int i = 0; i < R; ++i) {
          const int e = lane * R + i;
          if (e < k && e < c) out[e] = r[i];
        }
      };
      if (c <= 64) finish(std::integral_constant<int, 1>{});
      else if (c <= 128) finish(std::integral_constant<int, 2>{});
      else if (c <= 256) finish(std::integral_constant<int, 4>{});
      else if (c <= 512) finish(std::integral_constant<int, 8>{});
      else finish(std::integral_constant<int, 16>{});
    }
    return;
  }
  // more keys in the margin than the slots: every candidate's exact key,
  // then a radix selection over them
  if (tid == 0 && a.nbad) atomicAdd(a.nbad, 1ull);
  const int64_t base = t.seg_off ? t.seg_off[q] : q * t.all_n;
  const int64_t n = t.seg_off ? t.seg_off[q + 1] - base : t.all_n;
  uint64_t *A = t.all + base;
  // (a candidate the row filter excluded has the word kWordNone: no key;
  // compact candidates come from searches without a row filter)
  const uint32_t *W = a.words + wbase;
  for (int64_t i = tid; i < n; i += SEL_THREADS)
    A[i] = !CMP && W[i] == kWordNone
               ? VSK_KEY_NONE
               : vsk_key(tail_exact(t.rows + tail_row(t, q, i, lpb, llr) * t.ld, s_q, t.ld,
                                    t.squared),
                         (uint32_t)i);
  __threadfence_block();
  __syncthreads();
  auto each_key = [&](auto &&f) {
    for (int64_t i = tid; i < n; i += SEL_THREADS) f(A[i]);
  };
  uint64_t T, hi;
  bool take_all;
  radix_threshold(each_key, k, ssel, T, take_all, hi);
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  each_key([&](uint64_t key) {
    if (key != VSK_KEY_NONE && (take_all || key <= T)) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < VSK_MAX_K) keys[slot] = key;
    }
  });
  __syncthreads();
  int m = s_cnt;
  if (m > k) m = k;
  block_sort(keys, m);
  for (int i = tid; i < k; i += SEL_THREADS) out[i] = i < m ? keys[i] : VSK_KEY_NONE;
}

// The end of a wave's tail: the exact keys of the c <= 128 margin entries
// g[0 .. c) (position in the low 32 bits; row_of maps an entry to its row,
// called by every lane) -- the reference's sequential fp32 sum of (q - x)^2
// over the row, its square root unless squared -- one or two a lane, and
// the k smallest of them sorted into best_out[q]
template <class RowOf>
__device__ inline void wave_tail_finish(const ScreenTailArgs &t, int64_t q, const uint64_t *g,
                                        int32_t c, int32_t k, const float *sq, RowOf row_of) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  auto exact_key = [&](int e) -> uint64_t {
    const uint64_t ge = e < c ? g[e] : 0;
    const int64_t row = row_of(ge);
    if (e >= c) return VSK_KEY_NONE;
    const float *x = t.rows + row * t.ld;
    float acc = 0.f;
    for (int c0 = 0; c0 < t.ld; c0 += 64) {
      const int m = t.ld - c0 < 64 ? (t.ld - c0) >> 2 : 16;  // ld: multiple of 4
      float4 xv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < m) xv[u] = *reinterpret_cast<const float4 *>(x + c0 + 4 * u);
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < m) {
          const float4 qv = *reinterpret_cast<const float4 *>(sq + c0 + 4 * u);
          float d;
          d = qv.x - xv[u].x;
          acc = acc + d * d;
          d = qv.y - xv[u].y;
          acc = acc + d * d;
          d = qv.z - xv[u].z;
          acc = acc + d * d;
          d = qv.w - xv[u].w;
          acc = acc + d * d;
        }
    }
    return vsk_key(t.squared ? acc : sqrtf(acc), (uint32_t)ge);
  };
  uint64_t *out = t.best_out + q * (int64_t)k;
  if (c <= 64) {
    uint64_t key[1] = {exact_key(lane)};
    wave_sort_u64<1>(key);
    if (lane < k) out[lane] = key[0];
  } else {
    const uint64_t k0 = exact_key(lane), k1 = exact_key(lane + 64);
    uint64_t key[2] = {k0, k1};  // (any order: sorted next)
    wave_sort_u64<2>(key);       // element e at lane e / 2, register e % 2
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if (2 * lane + r < k) out[2 * lane + r] = key[r];
  }
}

// the margin limit of a k-th screened word (kWordNone: every word)
__device__ inline uint32_t tail_limit(uint32_t kth, double eps, int32_t metric) {
  if (kth == kWordNone) return kWordNone - 1u;
  const double ak = vsk_ord2f(kth);
  const double lim = metric == VSK_METRIC_L2 ? (ak + eps) * (1.0 + 0x1p-20) + eps : ak + 2.0 * eps;
  return vsk_f2ord(f_down(lim));
}

// The tail over compact candidates with a wave per query, for the common
// case: np <= 64, k <= 64, at most 512 kept candidates, at most 128 of them
// within the margin of the k-th (the k-th found from the per-lane minima
// with at most 64 words at or below their k-th).  A query outside that is
// marked in redo and left to k_screen_tail; every query's flag is written.
// The same margin, exact sums and keys as k_screen_tail, so the results are
// the same.  Four queries a workgroup, no block barrier.
constexpr int kTailWaveR = 8;  // kept candidates a lane
__global__ __launch_bounds__(256) void k_screen_tail_wave(ScreenTailArgs t, uint8_t *redo) {
#pragma clang fp contract(off)
  const MarginArgs &a = t.m;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t q = (int64_t)blockIdx.x * 4 + wv;
  if (q >= a.nq) return;
  __shared__ __attribute__((aligned(16))) float s_q[4][256];
  __shared__ uint64_t s_g[4][128];
  __shared__ uint8_t s_map[4][64 * kTailWaveR];
  const int np = t.np;
  const int64_t wbase = a.wseg[q];
  // lane p: probe slot p's base, its list's first row and its kept count
  int64_t pb = 0, lr = 0;
  int32_t cp = 0;
  if (lane < np) {
    pb = t.pos_base[q * np + lane];
    const int32_t l = t.probes[q * np + lane];
    lr = l >= 0 ? t.list_off[l] : 0;
  }
  const int64_t pnext = __shfl_down(pb, 1);
  if (lane < np) {
    const int64_t size = (lane + 1 < np ? pnext : a.cnt[q]) - pb;
    cp = size > 0 ? t.pcnt[q * np + lane] : 0;
  }
  int32_t incl = cp;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  const int32_t excl = incl - cp;
  const int32_t n = __shfl(incl, 63);
  if (n > 64 * kTailWaveR) {
    if (lane == 0) redo[q] = 1;
    return;
  }
  for (int c = lane; c < t.ld; c += 64) s_q[wv][c] = t.Q[q * t.ld + c];
  // entry e's probe slot: slot p marks entries excl .. incl - 1
  for (int p = 0; p < np; ++p) {
    const int32_t b = __builtin_amdgcn_readlane(excl, p), c = __builtin_amdgcn_readlane(cp, p);
    for (int i = lane; i < c; i += 64) s_map[wv][b + i] = (uint8_t)p;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const uint32_t *W = a.words + wbase, *R = t.prow + wbase;
  uint32_t w[kTailWaveR], ps[kTailWaveR];
  int sl[kTailWaveR];
#pragma unroll
  for (int r = 0; r < kTailWaveR; ++r) {
    const int e = lane + 64 * r;
    const int p = e < n ? s_map[wv][e] : 0;
    const int32_t pe = __shfl(excl, p);
    const int64_t pbp = __shfl(pb, p);
    w[r] = kWordNone;
    ps[r] = 0;
    sl[r] = p;
    if (e < n) {
      const int64_t o = pbp + (e - pe);
      w[r] = W[o];
      ps[r] = (uint32_t)(pbp + R[o]);
    }
  }
  // the k-th smallest word: at least k words are at or below the k-th
  // smallest per-lane minimum T, and it is among them
  const int32_t k = a.k;
  uint32_t kth = kWordNone;
  {
    uint32_t m = kWordNone;
#pragma unroll
    for (int r = 0; r < kTailWaveR; ++r) m = w[r] < m ? w[r] : m;
    uint32_t v[1] = {m};
    wave_sort_u32<1>(v);
    const uint32_t T = __shfl(v[0], k - 1);
    if (T != kWordNone) {
      int32_t c = 0;
#pragma unroll
      for (int r = 0; r < kTailWaveR; ++r) {
        const bool in = w[r] <= T;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
        const int32_t at = c + (int32_t)__builtin_amdgcn_mbcnt_hi(
                                   (uint32_t)(bal >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (in && at < 64) s_g[wv][at] = w[r];
        c += __builtin_popcountll(bal);
      }
      if (c > 64) {
        if (lane == 0) redo[q] = 1;
        return;
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      v[0] = lane < c ? (uint32_t)s_g[wv][lane] : kWordNone;
      wave_sort_u32<1>(v);
      kth = __shfl(v[0], k - 1);
    }
  }
  uint32_t lim_word = kWordNone - 1u;  // every key when there are fewer than k
  if (kth != kWordNone) {
    const double eps = screen_eps_of(a.qnh[q], a.qnr[q], a.xh, a.xr, a.d, a.metric, a.nprod);
    const double ak = vsk_ord2f(kth);
    const double lim = a.metric == VSK_METRIC_L2 ? (ak + eps) * (1.0 + 0x1p-20) + eps
                                                 : ak + 2.0 * eps;
    lim_word = vsk_f2ord(f_down(lim));
  }
  // the margin: up to 128 keys (probe slot, position), one or two a lane
  __builtin_amdgcn_wave_barrier();
  int32_t c = 0;
#pragma unroll
  for (int r = 0; r < kTailWaveR; ++r) {
    const bool in = w[r] <= lim_word;
    const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
    const int32_t at = c + (int32_t)__builtin_amdgcn_mbcnt_hi(
                               (uint32_t)(bal >> 32),
                               __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
    if (in && at < 128) s_g[wv][at] = ((uint64_t)(uint32_t)sl[r] << 32) | ps[r];
    c += __builtin_popcountll(bal);
  }
  if (c > 128) {
    if (lane == 0) redo[q] = 1;
    return;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  wave_tail_finish(t, q, s_g[wv], c, k, s_q[wv], [&](uint64_t g) -> int64_t {
    // (every lane takes part in the shuffles)
    const int gp = (int)(g >> 32);
    const int64_t gpb = __shfl(pb, gp), glr = __shfl(lr, gp);
    return glr + ((int64_t)(uint32_t)g - gpb);
  });
  if (lane == 0) redo[q] = 0;
}

// The tail of positional words without list slots (the probe's centroid
// words) with a wave per query, for k <= 64 and at most 4,096 words: the
// words are read in three passes (from cache after the first) rather than
// held.  Pass 1 takes each lane's minimum; T, the k-th smallest of those,
// has k words at or below it.  Pass 2 gathers every word within the margin
// of T (at most 128, with its position): they include the k smallest, so
// sorted they give the k-th word A_k, and those within the margin of A_k,
// a prefix of them, get their exact keys.  A query with more is marked in
// redo and left to k_screen_tail; every query's flag is written.
__global__ __launch_bounds__(256) void k_screen_tail_dense(ScreenTailArgs t, uint8_t *redo) {
  const MarginArgs &a = t.m;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t q = (int64_t)blockIdx.x * 4 + wv;
  if (q >= a.nq) return;
  __shared__ __attribute__((aligned(16))) float s_q[4][256];
  __shared__ uint64_t s_g[4][128];
  const uint32_t *W = a.words + q * a.wstride;
  const int n = (int)a.wn;
  for (int c = lane; c < t.ld; c += 64) s_q[wv][c] = t.Q[q * t.ld + c];
  // word 256 j + 4 lane + e of a pass (rows padded to 4 words)
  auto each = [&](auto &&f) {
#pragma unroll 4
    for (int j = 0; j < 16; ++j) {
      const int e0 = 256 * j + 4 * lane;
      uint4 v = make_uint4(kWordNone, kWordNone, kWordNone, kWordNone);
      if (e0 < n) v = *reinterpret_cast<const uint4 *>(W + e0);
      f(e0 < n ? v.x : kWordNone, e0);
      f(e0 + 1 < n ? v.y : kWordNone, e0 + 1);
      f(e0 + 2 < n ? v.z : kWordNone, e0 + 2);
      f(e0 + 3 < n ? v.w : kWordNone, e0 + 3);
    }
  };
  uint32_t m = kWordNone;
  each([&](uint32_t x, int) { m = x < m ? x : m; });
  const int32_t k = a.k;
  uint32_t v[1] = {m};
  wave_sort_u32<1>(v);
  const uint32_t T = __shfl(v[0], k - 1);
  const double eps = screen_eps_of(a.qnh[q], a.qnr[q], a.xh, a.xr, a.d, a.metric, a.nprod);
  const uint32_t limT = tail_limit(T, eps, a.metric);
  int32_t c = 0;
  each([&](uint32_t x, int e) {
    const bool in = x <= limT;
    const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
    const int32_t at = c + (int32_t)__builtin_amdgcn_mbcnt_hi(
                               (uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
    if (in && at < 128) s_g[wv][at] = ((uint64_t)x << 32) | (uint32_t)e;
    c += __builtin_popcountll(bal);
  });
  if (c > 128) {
    if (lane == 0) redo[q] = 1;
    return;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  // sorted by (word, position): the k-th word, and the margin a prefix
  uint32_t kth = kWordNone;
  if (c <= 64) {
    uint64_t r[1] = {lane < c ? s_g[wv][lane] : VSK_KEY_NONE};
    wave_sort_u64<1>(r);
    if (c >= k) kth = (uint32_t)(__shfl(r[0], k - 1) >> 32);
    __builtin_amdgcn_wave_barrier();
    if (lane < c) s_g[wv][lane] = r[0];
  } else {
    uint64_t r[2] = {s_g[wv][lane], lane + 64 < c ? s_g[wv][lane + 64] : VSK_KEY_NONE};
    wave_sort_u64<2>(r);  // element e at lane e / 2, register e % 2
    const uint64_t kk = __shfl(r[(k - 1) & 1], (k - 1) >> 1);
    kth = (uint32_t)(kk >> 32);
    __builtin_amdgcn_wave_barrier();
    if (2 * lane < c) s_g[wv][2 * lane] = r[0];
    if (2 * lane + 1 < c) s_g[wv][2 * lane + 1] = r[1];
  }
  const uint32_t lim = tail_limit(kth, eps, a.metric);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  int32_t cm = 0;  // the margin: the sorted entries whose word is within it
  for (int b = 0; b < c; b += 64) {
    const bool in = b + lane < c && (uint32_t)(s_g[wv][b + lane] >> 32) <= lim;
    cm += __builtin_popcountll(__builtin_amdgcn_ballot_w64(in));
  }
  // (keys carry the position; the exact key replaces the word)
  wave_tail_finish(t, q, s_g[wv], cm, k, s_q[wv],
                   [&](uint64_t g) -> int64_t { return (int64_t)(uint32_t)g; });
  if (lane == 0) redo[q] = 0;
}

void launch_screen_tail(vsk_ctx *ctx, const ScreenTailArgs &a, const char *name) {
  if (a.m.nq <= 0) return;
  if (a.m.k < 1 || a.m.k > VSK_MAX_K || a.m.cap > VSK_MAX_K || a.ld > 256)
    fail(VSK_ERR_INVALID_ARGUMENT, "screen tail: k, cap (<= 1024) or ld (<= 256) out of range");
  if (a.pcnt && (!a.list_off || a.np > 256 || !a.prow || !a.m.wseg || !a.m.cnt))
    fail(VSK_ERR_INVALID_ARGUMENT, "screen tail: compact candidates need list slots (np <= 256)");
  KernelTimer t(ctx, name);
  if (a.pcnt && a.np <= 64 && a.m.k <= 64 && !a.active) {
    // a wave per query, the block tail for the queries it leaves
    uint8_t *redo = static_cast<uint8_t *>(ctx->scratch_ptr("tail.redo", a.m.nq + 64));
    k_screen_tail_wave<<<(unsigned)ceil_div(a.m.nq, 4), 256, 0, ctx->stream>>>(a, redo);
    ScreenTailArgs b = a;
    b.active = redo;
    k_screen_tail<32, true><<<(unsigned)a.m.nq, SEL_THREADS, 0, ctx->stream>>>(b);
  } else if (!a.pcnt && !a.list_off && !a.m.wseg && !a.m.cnt && a.m.wn <= 4096 &&
             a.m.wstride % 4 == 0 && a.m.k <= 64 && !a.active) {
    // positional words (the probe's): the same, over three passes
    uint8_t *redo = static_cast<uint8_t *>(ctx->scratch_ptr("tail.redo", a.m.nq + 64));
    k_screen_tail_dense<<<(unsigned)ceil_div(a.m.nq, 4), 256, 0, ctx->stream>>>(a, redo);
    ScreenTailArgs b = a;
    b.active = redo;
    k_screen_tail<32, false><<<(unsigned)a.m.nq, SEL_THREADS, 0, ctx->stream>>>(b);
  } else if (a.pcnt)
    k_screen_tail<32, true><<<(unsigned)a.m.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  else
    k_screen_tail<32, false><<<(unsigned)a.m.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  check_launch(name);
}

// Exact top k by (word, index), sorted (declared with WordSelectArgs):
// word_kth finds the k-th smallest word V; every word below V is kept and,
// of the words equal to V, those with the smallest indices -- a second
// search over their indices when more are equal than the k still need.
template <int REG>
__global__ __launch_bounds__(SEL_THREADS) void k_select_words(WordSelectArgs a) {
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  if (a.active && !a.active[q]) return;
  WordList<REG> L;
  L.load(a.words + a.wseg[q], a.cnt[q]);
  auto each = [&](auto &&f) { L.each(f); };
  __shared__ KthShared sh;
  __shared__ uint64_t sel[VSK_MAX_K];
  __shared__ uint32_t s_less, s_eq;
  __shared__ int s_cnt;
  const uint32_t k = (uint32_t)a.k;
  const uint32_t V = word_kth_fast(each, k, sh, 0.0);
  uint32_t I = 0xFFFFFFFFu;  // the largest index kept among words equal to V
  if (V != kWordNone) {
    if (tid == 0) {
      s_less = 0;
      s_eq = 0;
    }
    __syncthreads();
    uint32_t less = 0, eq = 0;
    each([&](uint32_t x, uint32_t) {
      less += x < V ? 1u : 0u;
      eq += x == V ? 1u : 0u;
    });
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      less += __shfl_xor(less, o);
      eq += __shfl_xor(eq, o);
    }
    if (lane == 0) {
      atomicAdd(&s_less, less);
      atomicAdd(&s_eq, eq);
    }
    __syncthreads();
    const uint32_t need_eq = k - s_less;
    if (s_eq > need_eq) {
      I = word_kth([&](auto &&f) {
        L.each([&](uint32_t x, uint32_t i) { f(x == V ? i : kWordNone, i); });
      }, need_eq, sh.w, 0.0);
    }
  }
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  each([&](uint32_t x, uint32_t i) {
    const bool keep = x != kWordNone && (V == kWordNone || x < V || (x == V && i <= I));
    if (keep) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < VSK_MAX_K) sel[slot] = ((uint64_t)x << 32) | i;
    }
  });
  __syncthreads();
  int m = s_cnt;
  if (m > (int)k) m = (int)k;  // (exactly k, or fewer words in all)
  block_sort(sel, m);
  uint64_t *out = a.best_out + q * (int64_t)k;
  for (int i = tid; i < (int)k; i += SEL_THREADS) out[i] = i < m ? sel[i] : VSK_KEY_NONE;
}

void launch_select_words(vsk_ctx *ctx, const WordSelectArgs &a, const char *name) {
  if (a.nq <= 0) return;
  if (a.k < 1 || a.k > VSK_MAX_K)
    fail(VSK_ERR_INVALID_BUFFER_SIZE, "k out of range for selection");
  KernelTimer t(ctx, name);
  k_select_words<32><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  check_launch(name);
}

void launch_select(vsk_ctx *ctx, const SelectArgs &a, const char *name) {
  if (a.nq <= 0) return;
  if (a.k < 1 || a.k > VSK_MAX_K)
    fail(VSK_ERR_INVALID_BUFFER_SIZE, "k out of range for selection");
  KernelTimer t(ctx, name);
  if (a.small) {
    if (!a.counts || a.prev || a.seg_off || a.seg_n || a.cand32 || a.cap > 1024 || !a.sorted)
      fail(VSK_ERR_INVALID_ARGUMENT, "short-list selection takes counted lists of at most 1024");
    k_select_small<<<(unsigned)ceil_div(a.nq, SEL_THREADS / 64), SEL_THREADS, 0, ctx->stream>>>(a);
    check_launch(name);
    return;
  }
  // keys per query: the previous list (k) and up to cap candidates
  const int64_t most = a.cap + (a.prev ? a.k : 0);
  const bool fast = a.k <= 128 && !a.seg_n;
  if (a.cand32) {
    if (a.prev || a.seg_n) fail(VSK_ERR_INVALID_ARGUMENT, "32-bit lists take no previous list or segments");
    k_select<32, true><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  } else if (a.regs && !a.seg_off && most > 32 * SEL_THREADS) {
    if (fast)
      k_select<64, false, true><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
    else
      k_select<64, false><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  } else if (a.seg_off || a.regs) {
    if (fast)
      k_select<32, false, true><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
    else
      k_select<32, false><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  } else if (a.seg_n && a.nq < 4 * (int64_t)ctx->cu_count) {
    k_select<0, false, false, 8><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  } else {
    k_select<0, false><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  }
  check_launch(name);
}

int64_t default_cap(int32_t k) {
  int64_t c = 16384;
  while (c < 16ll * k) c <<= 1;
  return c;
}

int64_t screen_cap(int32_t k) {
  int64_t c = 2048;
  while (c < 4ll * k) c <<= 1;
  return c;
}

int64_t query_batch(const vsk_ctx *ctx, int64_t nq, int64_t cap) {
  // candidate buffers of one batch stay under the context's tile budget
  // (2 GiB of HBM, at least 64 queries; VSK_MAX_TILE_BYTES sets it, down to
  // one query a batch)
  const int64_t budget = ctx->max_tile_bytes > 0 ? ctx->max_tile_bytes : 2ll << 30;
  int64_t b = budget / (cap * (int64_t)sizeof(uint64_t));
  const int64_t least = ctx->max_tile_bytes > 0 ? 1 : 64;
  if (b < least) b = least;
  return nq < b ? nq : b;
}

int64_t tile_keys(const vsk_ctx *ctx, int64_t keys, int64_t bytes_per_key) {
  if (ctx->max_tile_bytes <= 0) return keys;
  const int64_t k = ctx->max_tile_bytes / bytes_per_key;
  return k < keys ? (k > 0 ? k : 1) : keys;
}

void progressive_topk(vsk_ctx *ctx, int64_t nq, int64_t n, int32_t k,
                      int64_t cap, const ScanFn &scan, uint64_t *best,
                      const char *select_name, int64_t max_growth,
                      const TopkWorkspace *ws) {
  if (nq <= 0) return;
  if (n <= 0) {
    fill_u64(ctx, best, nq * (int64_t)k, VSK_KEY_NONE);
    return;
  }
  // The first chunk is dense and taken by every query: its selection reads
  // no previous list and no counts (each query has exactly cap keys) and
  // writes every query's list and threshold, so neither needs clearing
  // (three fewer launches per call, which small problems notice).
  if (cap > n) cap = n;  // the whole database is one dense chunk
  TopkWorkspace w;
  if (ws) {
    w = *ws;
  } else {
    w.thresh = static_cast<uint64_t *>(ctx->scratch_ptr("topk.thresh", 8 * nq));
    w.cand = static_cast<uint64_t *>(
        ctx->scratch_ptr("topk.cand", sizeof(uint64_t) * (size_t)nq * cap));
    w.counts = static_cast<int32_t *>(ctx->scratch_ptr("topk.counts", 4 * nq));
    w.ovf_mask = static_cast<uint8_t *>(ctx->scratch_ptr("topk.ovfmask", nq + 64));
    w.seg_n = static_cast<int32_t *>(
        ctx->scratch_ptr("topk.segn", sizeof(int32_t) * (size_t)nq * VSK_MAX_SEG));
    w.ovf_count = static_cast<int32_t *>(ctx->scratch_ptr("topk.ovfcount", 64));
  }
  uint64_t *thresh = w.thresh, *cand = w.cand;
  int32_t *counts = w.counts, *seg_n = w.seg_n, *ovf_count = w.ovf_count;
  uint8_t *ovf_mask = w.ovf_mask;
  // Without topk_sync no chunk is checked from the host: an overflow only
  // counts into the context's call counter, which the call's final
  // synchronisation reads back (then the call runs again with checks).
  // (armed before the first filtered chunk: a search that is one dense
  // chunk has nothing to count, nor to read back)
  const bool defer = !ctx->topk_sync;

  int64_t r0 = 0;
  bool first = true;
  while (r0 < n) {
    int64_t c;
    if (first) {
      c = n < cap ? n : cap;
    } else {
      // expected survivors of a chunk of c rows after r0 rows are about
      // k*c/r0; keep that near cap/2
      int64_t factor = cap / (2 * (int64_t)k);
      if (max_growth > 0 && factor > max_growth) factor = max_growth;
      int64_t grow = r0 * factor;
      c = grow > cap ? grow : cap;
      if (c > n - r0) c = n - r0;
    }
    const bool dense = first;
    if (!dense) fill_i32(ctx, counts, nq, 0);
    if (!dense && defer && !ctx->ovf_armed) {
      fill_i32(ctx, ctx->ovf_dev, 1, 0);
      ctx->ovf_armed = true;
    }
    int32_t nseg = 0;
    int64_t seg_stride = 0;
    {
      ScanRequest rq{r0, r0 + c, thresh, nullptr, cand, cap, counts, dense};
      if (!dense && seg_n) {
        rq.seg_n = seg_n;
        rq.seg_nseg = &nseg;
        rq.seg_stride = &seg_stride;
      }
      scan(rq);
    }
    SelectArgs sa;
    sa.nq = nq;
    sa.k = k;
    sa.prev = dense ? nullptr : best;
    sa.cand = cand;
    sa.cap = cap;
    sa.counts = dense ? nullptr : counts;
    sa.best_out = best;
    sa.thresh = thresh;
    // only the last chunk's list is returned: the others stay unsorted
    sa.sorted = r0 + c >= n;
    // small dense lists (IVF probing over the centroids, small problems)
    // are read into registers once
    sa.regs = dense && cap <= 64 * SEL_THREADS;  // (no previous list)
    if (!dense) {
      if (defer) {
        // (the mask is written, never read)
        sa.overflow_count = ctx->ovf_dev;
      } else {
        fill_i32(ctx, ovf_count, 1, 0);
        fill_i32(ctx, reinterpret_cast<int32_t *>(ovf_mask), (nq + 3) / 4, 0);
        sa.overflow_count = ovf_count;
      }
      sa.overflow_mask = ovf_mask;
      if (nseg > 0) {
        sa.seg_n = seg_n;
        sa.nseg = nseg;
        sa.seg_stride = seg_stride;
      }
    }
    launch_select(ctx, sa, select_name);
    if (!dense && !defer) {
      int32_t h_ovf = 0;
      VSK_HIP(hipMemcpyAsync(&h_ovf, ovf_count, 4, hipMemcpyDeviceToHost,
                             ctx->stream));
      stream_sync(ctx);
      if (h_ovf > 0) {
        // queries whose survivors did not fit re-scan this chunk in
        // sub-chunks of cap rows, each kept whole
        for (int64_t s0 = r0; s0 < r0 + c; s0 += cap) {
          int64_t s1 = s0 + cap < r0 + c ? s0 + cap : r0 + c;
          fill_i32(ctx, counts, nq, (int32_t)(s1 - s0));
          scan(ScanRequest{s0, s1, thresh, ovf_mask, cand, cap, counts, true});
          SelectArgs sb = sa;
          sb.active = ovf_mask;
          sb.overflow_mask = nullptr;
          sb.overflow_count = nullptr;
          // a sub-chunk's keys are dense (cap a query), whatever the
          // filtered chunk's layout was
          sb.seg_n = nullptr;
          sb.nseg = 0;
          sb.seg_stride = 0;
          launch_select(ctx, sb, select_name);
        }
      }
    }
    r0 += c;
    first = false;
  }
}

}  // namespace vsk
