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
#include "vsk_api.hpp"

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

// REG: keys per thread held in registers when a query's list fits (REG x
// SEL_THREADS keys): every pass then reads registers, not the list again.
// The registers cost occupancy, so only callers whose lists are a few
// thousand keys (IVF candidate segments, a dense chunk as small as the IVF
// probe's centroids) take it.
// W32: the candidates are a.cand32 (no previous list)
template <int REG, bool W32>
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
    for (int s = tid >> 6; s < a.nseg; s += SEL_THREADS / 64) {
      const uint64_t *cs = a.cand + q * a.cap + (int64_t)s * a.seg_stride;
      const int32_t ns = seg_cnt[s];
      for (int32_t j = lane; j < ns; j += 64) f(cs[j]);
    }
  };

  __shared__ uint32_t hist[256];
  __shared__ uint64_t sel[VSK_MAX_K];
  __shared__ int sh_bucket, sh_take_all;
  __shared__ uint32_t sh_before, sh_bcount;
  __shared__ int sel_count;
  __shared__ uint64_t sh_lo[SEL_THREADS / 64], sh_hi[SEL_THREADS / 64];

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
    sh_lo[tid >> 6] = lo;
    sh_hi[tid >> 6] = hi;
  }
  __syncthreads();
  lo = sh_lo[0];
  hi = sh_hi[0];
#pragma unroll
  for (int wv = 1; wv < SEL_THREADS / 64; ++wv) {
    lo = sh_lo[wv] < lo ? sh_lo[wv] : lo;
    hi = sh_hi[wv] > hi ? sh_hi[wv] : hi;
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
    for (int i = tid; i < 256; i += SEL_THREADS) hist[i] = 0;
    __syncthreads();
    each_key([&](uint64_t key) {
      if (key != VSK_KEY_NONE && (key & mask) == prefix)
        atomicAdd(&hist[(uint32_t)(key >> shift) & dmask], 1u);
    });
    __syncthreads();
    if (tid < 64) {
      uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1],
               h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
      uint32_t s = h0 + h1 + h2 + h3;
      uint32_t incl = s;
      for (int o = 1; o < 64; o <<= 1) {
        uint32_t v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
      }
      uint32_t all = __shfl(incl, 63);
      uint32_t excl = incl - s;
      if (first && all <= (uint32_t)k) {
        if (lane == 0) sh_take_all = 1;
      } else {
        if (lane == 0) sh_take_all = 0;
        bool here = excl < (uint64_t)need && (uint64_t)need <= incl;
        if (here) {
          uint32_t hs[4] = {h0, h1, h2, h3};
          uint32_t before = excl;
          int j = 0;
          while (before + hs[j] < (uint64_t)need) {
            before += hs[j];
            ++j;
          }
          sh_bucket = 4 * lane + j;
          sh_before = before;
          sh_bcount = hs[j];
        }
      }
    }
    __syncthreads();
    if (sh_take_all) {
      take_all = true;
      break;
    }
    first = false;
    const uint32_t b = (uint32_t)sh_bucket;
    need -= sh_before;
    prefix |= (uint64_t)b << shift;
    mask |= (uint64_t)dmask << shift;
    const bool full = (uint64_t)sh_bcount == (uint64_t)need;
    __syncthreads();  // everyone has read the sh_* values
    if (full || shift == 0) {
      T = prefix | ~mask;
      break;
    }
    top = shift - 1;
  }

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
  uint64_t *out = a.best_out + q * (int64_t)k;
  for (int i = tid; i < k; i += SEL_THREADS)
    out[i] = i < m ? sel[i] : VSK_KEY_NONE;
  if (tid == 0 && a.thresh) a.thresh[q] = (m >= k) ? sel[k - 1] : VSK_KEY_NONE;
}

void launch_select(vsk_ctx *ctx, const SelectArgs &a, const char *name) {
  if (a.nq <= 0) return;
  if (a.k < 1 || a.k > VSK_MAX_K)
    fail(VSK_ERR_INVALID_BUFFER_SIZE, "k out of range for selection");
  KernelTimer t(ctx, name);
  // keys per query: the previous list (k) and up to cap candidates
  const int64_t most = a.cap + (a.prev ? a.k : 0);
  if (a.cand32) {
    if (a.prev || a.seg_n) fail(VSK_ERR_INVALID_ARGUMENT, "32-bit lists take no previous list or segments");
    k_select<32, true><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  } else if (a.regs && !a.seg_off && most > 32 * SEL_THREADS)
    k_select<64, false><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  else if (a.seg_off || a.regs)
    k_select<32, false><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
  else
    k_select<0, false><<<(unsigned)a.nq, SEL_THREADS, 0, ctx->stream>>>(a);
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

int64_t query_batch(int64_t nq, int64_t cap) {
  // candidate buffers of one batch stay under ~2 GiB of HBM
  const int64_t budget = 2ll << 30;
  int64_t b = budget / (cap * (int64_t)sizeof(uint64_t));
  if (b < 64) b = 64;
  return nq < b ? nq : b;
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
      fill_i32(ctx, ovf_count, 1, 0);
      fill_i32(ctx, reinterpret_cast<int32_t *>(ovf_mask), (nq + 3) / 4, 0);
      sa.overflow_mask = ovf_mask;
      sa.overflow_count = ovf_count;
      if (nseg > 0) {
        sa.seg_n = seg_n;
        sa.nseg = nseg;
        sa.seg_stride = seg_stride;
      }
    }
    launch_select(ctx, sa, select_name);
    if (!dense) {
      int32_t h_ovf = 0;
      VSK_HIP(hipMemcpyAsync(&h_ovf, ovf_count, 4, hipMemcpyDeviceToHost,
                             ctx->stream));
      VSK_HIP(hipStreamSynchronize(ctx->stream));
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
          launch_select(ctx, sb, select_name);
        }
      }
    }
    r0 += c;
    first = false;
  }
}

}  // namespace vsk
