// bin.hip -- binary quantization (one bit per dimension) and the Hamming
// top-k scan.
//
// Reference: quantizeVectors(scheme: .binary) ->
// AccelerateOptimizer.binaryQuantize (Acceleration/AccelerateOptimizer.swift:
// 447-481): bit i of a code is x_i > 0, in byte i/8 at bit i%8 (the Metal
// binaryQuantize, Acceleration/Metal/Shaders/QuantizationShaders.metal:
// 232-260, writes the same bits as little-endian 32-bit words).
// binaryHammingDistance (:285-305): popcount(q xor x) over the words.
//
// Layout in HBM: W 32-bit words per code, W a multiple of 4 (whole 16-byte
// loads); the padding bits are zero in every code and add nothing to a
// distance.
//
// Scan: a lane owns one database code (W registers) and walks the queries.
// The query words are the same for the whole wave, so they come by scalar
// loads and each word costs one v_xor_b32 and one v_bcnt_u32_b32 with a
// scalar operand; the codes are read from HBM once per launch whatever the
// number of queries.  The filter appends the keys <= the query's threshold
// with one atomic per (wave, query) that has any.
#include "flat.hpp"

struct vsk_bin {
  int64_t n = 0;
  int32_t d = 0;
  int32_t words = 0;  // 32-bit words per code (4, 8, 16 or 32)
  vsk::DevBuf codes;
  vsk::DevBuf pop;    // int32 per row: set bits of its code
};

namespace vsk {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

struct BinArgs {
  const uint32_t *X;  // rows, `words` words each
  const uint32_t *Q;  // queries, same stride
  int32_t words;
  int32_t nq;
  int64_t r0, r1;
  const uint64_t *thresh;
  const uint8_t *active;
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
  float *mat;  // distance matrix (nq x ldm), else null
  int64_t ldm;
};

constexpr int BIN_T = 256;

// (pointers as separate restrict arguments: the query words and thresholds
// are then provably never written by the kernel and load through the scalar
// cache; ACT: an active mask is given, which only the progressive top-k's
// overflow re-scans do)
template <int W, int MODE, bool ACT>
__global__ __launch_bounds__(BIN_T) void k_bin_scan(
    const uint32_t *__restrict__ X, const uint32_t *__restrict__ Q,
    const uint64_t *__restrict__ thresh, const uint8_t *__restrict__ active,
    uint64_t *__restrict__ cand, int32_t *__restrict__ counts, float *__restrict__ mat,
    BinArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = a.r0 + (int64_t)blockIdx.x * BIN_T + threadIdx.x;
  const bool rok = row < a.r1;
  uint32_t x[W];
  {
    const u4 *src = reinterpret_cast<const u4 *>(X + (rok ? row : a.r0) * W);
#pragma unroll
    for (int u = 0; u < W / 4; ++u) {
      const u4 v = src[u];
      x[4 * u] = v.x;
      x[4 * u + 1] = v.y;
      x[4 * u + 2] = v.z;
      x[4 * u + 3] = v.w;
    }
  }
  const uint64_t below = (1ull << lane) - 1ull;
  const uint32_t row32 = (uint32_t)row;
  // queries in blocks of QB: their words and thresholds are scalar loads
  // issued together, and the QB distances are independent chains
  constexpr int QB = 8;
  for (int32_t q0 = 0; q0 < a.nq; q0 += QB) {
    uint32_t dist[QB];
    uint64_t th[QB];
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      const int32_t q = q0 + j < a.nq ? q0 + j : a.nq - 1;  // past the end: a repeat
      if constexpr (MODE == MODE_FILTER) th[j] = thresh[q];
      const uint32_t *qw = Q + (int64_t)q * W;
      uint32_t s = 0;
#pragma unroll
      for (int w = 0; w < W; ++w) s += __builtin_popcount(x[w] ^ qw[w]);
      dist[j] = s;
    }
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      const int32_t q = q0 + j;
      if (q >= a.nq) break;
      if constexpr (ACT) {
        if (!active[q]) continue;
      }
      if constexpr (MODE == MODE_MATRIX) {
        if (rok) mat[(int64_t)q * a.ldm + row] = (float)dist[j];
      } else if constexpr (MODE == MODE_DENSE) {
        if (rok) cand[(int64_t)q * a.cap + (row - a.r0)] = vsk_key_i32((int32_t)dist[j], row32);
      } else {
        // key <= threshold on (distance, row): the distance settles all but
        // the tie with the threshold's own distance.  No threshold yet
        // (fewer than k keys, NONE) decodes to distance 0x7FFFFFFF, which
        // every distance is below.
        const uint32_t thd = (uint32_t)(th[j] >> 32) ^ 0x80000000u;
        const uint32_t thr = (uint32_t)th[j];
        const bool pass = rok & ((dist[j] < thd) | ((dist[j] == thd) & (row32 <= thr)));
        const uint64_t m = __builtin_amdgcn_ballot_w64(pass);
        if (m) {
          const int leader = __builtin_ctzll(m);
          int32_t base = 0;
          if (lane == leader) base = atomicAdd(&counts[q], (int32_t)__builtin_popcountll(m));
          base = __builtin_amdgcn_readlane(base, leader);
          if (pass) {
            const int64_t slot = base + __builtin_popcountll(m & below);
            if (slot < a.cap)
              cand[(int64_t)q * a.cap + slot] = vsk_key_i32((int32_t)dist[j], row32);
          }
        }
      }
    }
  }
}

template <int MODE, bool ACT>
static void launch_bin_mode(vsk_ctx *ctx, const BinArgs &a, unsigned grid) {
#define BIN_CASE(W)                                                                  \
  case W:                                                                            \
    k_bin_scan<W, MODE, ACT><<<grid, BIN_T, 0, ctx->stream>>>(                       \
        a.X, a.Q, a.thresh, a.active, a.cand, a.counts, a.mat, a);                   \
    break;
  switch (a.words) {
    BIN_CASE(4)
    BIN_CASE(8)
    BIN_CASE(12)
    BIN_CASE(16)
    BIN_CASE(20)
    BIN_CASE(24)
    BIN_CASE(28)
    BIN_CASE(32)
  default: fail(VSK_ERR_UNSUPPORTED, "binary codes of more than 1024 bits");
  }
#undef BIN_CASE
}

static void launch_bin(vsk_ctx *ctx, const BinArgs &a, int mode) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  const int64_t g = ceil_div(rows, BIN_T);
  if (g > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "too many rows");
  static const char *names[3] = {"bin_hamming_dense", "bin_hamming_filter",
                                 "bin_hamming_matrix"};
  KernelTimer t(ctx, names[mode], (double)a.nq * (double)rows);
  if (mode == MODE_DENSE && a.active)
    launch_bin_mode<MODE_DENSE, true>(ctx, a, (unsigned)g);
  else if (mode == MODE_DENSE)
    launch_bin_mode<MODE_DENSE, false>(ctx, a, (unsigned)g);
  else if (mode == MODE_FILTER && a.active)
    launch_bin_mode<MODE_FILTER, true>(ctx, a, (unsigned)g);
  else if (mode == MODE_FILTER)
    launch_bin_mode<MODE_FILTER, false>(ctx, a, (unsigned)g);
  else
    launch_bin_mode<MODE_MATRIX, false>(ctx, a, (unsigned)g);
  check_launch(names[mode]);
}

// ---------------------------------------------------------------------------
// The Hamming scan on the int8 matrix cores.  For 0/1 vectors
//   H(q, x) = |q| + |x| - 2 <q, x>,
// and <q, x> is an int8 dot product once every bit is spread to a byte.
// Layout as the int8 scan of sq8.hip: each wave keeps QT query tiles (16
// queries each) of KS 64-bit k-steps as v_mfma_i32_16x16x64_i8 B operands
// (expanded once) and streams 16-row A tiles of packed words, two blocks in
// flight; a lane's 16 bits of a k-step become 16 bytes by
// ((nibble * 0x204081) & 0x01010101) per dword (the four shifted copies of
// the nibble do not overlap, so nothing carries).  The filter ranks by
// 2<q, x> - |x| against the query's floor |q| - threshold: one multiply-add
// and one max per score, a ballot skips the blocks where nothing can pass.
// ---------------------------------------------------------------------------
typedef int i4 __attribute__((ext_vector_type(4)));

struct BinMArgs {
  const uint32_t *X;   // codes, `words` words per row
  const uint32_t *Q;   // query codes, same stride
  const int32_t *xpop; // set bits per row
  const int32_t *qpop; // set bits per query
  int64_t npop;        // entries of xpop (rows + 4 zero padding)
  int32_t words;
  int32_t nq;
  int64_t r0, r1, rows_per_split;
  const uint64_t *thresh;
  const uint8_t *active;
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
};

__device__ __forceinline__ i4 bin_expand16(uint32_t b) {
  i4 r;
  r.x = (int)(((b & 15u) * 0x204081u) & 0x01010101u);
  r.y = (int)((((b >> 4) & 15u) * 0x204081u) & 0x01010101u);
  r.z = (int)((((b >> 8) & 15u) * 0x204081u) & 0x01010101u);
  r.w = (int)((((b >> 12) & 15u) * 0x204081u) & 0x01010101u);
  return r;
}

// candidates staged per wave in LDS, appended 64 at a time (an atomic that
// returns a value would make the wave wait for its row prefetches)
constexpr int BM_WBUF = 512;

__device__ __forceinline__ void bm_flush(const BinMArgs &a, const uint64_t *lkey,
                                         const int32_t *lq, int32_t &nbuf, int lane) {
  for (int32_t e = lane; e < nbuf; e += 64) {
    const int32_t q = lq[e];
    const int c = atomicAdd(&a.counts[q], 1);
    if (c < a.cap) a.cand[(int64_t)q * a.cap + c] = lkey[e];
  }
  nbuf = 0;
}

// WPE: waves a SIMD holds (the register budget per wave)
template <int RT, int KS, int QT, bool DENSE, int WPE = 2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void k_bin_mfma(BinMArgs a, int32_t groups, int32_t splits_per_xcd) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
  const int grp = slot % groups;
  const int split = (slot / groups) * 8 + xcd;
  if (split >= 8 * splits_per_xcd) return;
  const int64_t s0 = a.r0 + (int64_t)split * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;
  const int64_t qw0 = ((int64_t)grp * 4 + w) * (QT * 16);
  if (qw0 >= a.nq) return;
  // this lane's 16 bits of k-step ks: word 2 ks + (lane >> 5), bits
  // 16 ((lane >> 4) & 1) ..
  const int wsel = lane >> 5, bsh = 16 * ((lane >> 4) & 1);

  i4 bq[QT][KS];
  int32_t floor_[QT], qp[QT], thd[QT];
  uint32_t trow[QT];
  bool qok[QT];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int64_t q = qw0 + 16 * j + (lane & 15);
    qok[j] = q < a.nq && (!a.active || a.active[q]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      bq[j][ks] = qok[j] ? bin_expand16(a.Q[q * a.words + 2 * ks + wsel] >> bsh)
                         : i4{0, 0, 0, 0};
    qp[j] = qok[j] ? a.qpop[q] : 0;
    const uint64_t th = (!DENSE && qok[j]) ? a.thresh[q] : VSK_KEY_NONE;
    thd[j] = (int32_t)((uint32_t)(th >> 32) ^ 0x80000000u);  // NONE: 0x7FFFFFFF
    trow[j] = (uint32_t)th;
    // H <= thd  <=>  2<q,x> - |x| >= |q| - thd
    floor_[j] = qok[j] ? qp[j] - thd[j] : 0x7FFFFFFF;
  }

  const int64_t nrows = s1 - s0;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.X + s0 * a.words), 0, (int32_t)(nrows * a.words * 4), 0x00020000);
  // the popcounts of a row group of 4 load as one 16-byte vector: the range
  // covers whole groups (within the padded array), so a group that straddles
  // the split's end is read whole and only its rows past the end are dropped
  int64_t npr = (nrows + 3) & ~3ll;
  if (npr > a.npop - s0) npr = a.npop - s0;
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.xpop + s0), 0, (int32_t)(npr * 4), 0x00020000);
  const int32_t lrow = ((int32_t)(lane & 15) * a.words + wsel) * 4;
  const int32_t lpop = 16 * (lane >> 4);  // bytes: rows 4 (lane >> 4) .. + 3
  uint32_t ar0[RT][KS], ar1[RT][KS];
  i4 xp0[RT], xp1[RT];
#define BM_LOAD(AR, XP, T)                                                          \
  _Pragma("unroll") for (int i = 0; i < RT; ++i) {                                 \
    _Pragma("unroll") for (int ks = 0; ks < KS; ++ks) AR[i][ks] =                  \
        __builtin_amdgcn_raw_buffer_load_b32(                                       \
            rx, (int32_t)((T) + 16 * i) * a.words * 4 + lrow, 8 * ks, 0);           \
    XP[i] = __builtin_bit_cast(                                                     \
        i4, __builtin_amdgcn_raw_buffer_load_b128(rp, (int32_t)((T) + 16 * i) * 4 + lpop, \
                                                  0, 0));                           \
  }
  __shared__ uint64_t s_key[4][DENSE ? 1 : BM_WBUF];
  __shared__ int32_t s_q[4][DENSE ? 1 : BM_WBUF];
  int32_t nbuf = 0;
  constexpr int32_t RB = 16 * RT;
  const int32_t nr = (int32_t)nrows;
  auto block = [&](const uint32_t (&ar)[RT][KS], const i4 (&xp)[RT], int64_t t0) {
    i4 acc[RT][QT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int j = 0; j < QT; ++j) acc[i][j] = i4{0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const i4 av = bin_expand16(ar[i][ks] >> bsh);
#pragma unroll
        for (int j = 0; j < QT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bq[j][ks], acc[i][j], 0, 0, 0);
      }
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int64_t rb = t0 + 16 * i + 4 * (lane >> 4);  // + r
      const int32_t xv[4] = {xp[i].x, xp[i].y, xp[i].z, xp[i].w};
      if constexpr (DENSE) {
#pragma unroll
        for (int j = 0; j < QT; ++j) {
          if (!qok[j]) continue;
          const int64_t q = qw0 + 16 * j + (lane & 15);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (rb + r < s1)
              a.cand[q * a.cap + (rb + r - a.r0)] =
                  vsk_key_i32(qp[j] + xv[r] - 2 * acc[i][j][r], (uint32_t)(rb + r));
        }
      } else {
#pragma unroll
        for (int j = 0; j < QT; ++j) {
          int32_t sc[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[r] = 2 * acc[i][j][r] - xv[r];
          const int32_t m01 = sc[0] > sc[1] ? sc[0] : sc[1];
          const int32_t m23 = sc[2] > sc[3] ? sc[2] : sc[3];
          const bool hit = (m01 > m23 ? m01 : m23) >= floor_[j];
          if (!__builtin_amdgcn_ballot_w64(hit)) continue;  // the common case
          const int32_t q = (int32_t)(qw0 + 16 * j + (lane & 15));
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            // (a lane whose query is past nq or inactive never passes: its
            // missing threshold would admit every row)
            const int32_t h = qp[j] - sc[r];
            const bool p = qok[j] && rb + r < s1 &&
                           (h < thd[j] || (h == thd[j] && (uint32_t)(rb + r) <= trow[j]));
            const uint64_t m = __builtin_amdgcn_ballot_w64(p);
            if (!m) continue;
            if (p) {
              const int32_t pos =
                  nbuf + (int32_t)__builtin_amdgcn_mbcnt_hi(
                             (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
              s_key[w][pos] = vsk_key_i32(h, (uint32_t)(rb + r));
              s_q[w][pos] = q;
            }
            nbuf += __builtin_popcountll(m);
          }
          if (nbuf > BM_WBUF - 256) bm_flush(a, s_key[w], s_q[w], nbuf, lane);
        }
      }
    }
  };
  BM_LOAD(ar0, xp0, 0);
  __builtin_amdgcn_sched_barrier(0);
  BM_LOAD(ar1, xp1, RB);
  __builtin_amdgcn_sched_barrier(0);
  for (int32_t t = 0; t < nr; t += 2 * RB) {
    block(ar0, xp0, s0 + t);
    BM_LOAD(ar0, xp0, t + 2 * RB);
    __builtin_amdgcn_sched_barrier(0);
    // the second block may lie past the split: it reads zeros and its rows
    // are dropped
    block(ar1, xp1, s0 + t + RB);
    BM_LOAD(ar1, xp1, t + 3 * RB);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (!DENSE && nbuf > 0) bm_flush(a, s_key[w], s_q[w], nbuf, lane);
#undef BM_LOAD
}

template <int RT, int KS, int QT, int WPE = 2>
static void launch_bm(vsk_ctx *ctx, const BinMArgs &a, bool dense) {
  const int64_t rows = a.r1 - a.r0;
  const int64_t qpg = 4 * QT * 16;  // queries per workgroup
  const int64_t groups = ceil_div(a.nq, qpg);
  int64_t splits = ceil_div(4096, groups);
  const int64_t max_splits = ceil_div(rows, 16 * RT);
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  BinMArgs b = a;
  b.rows_per_split = ceil_div(ceil_div(rows, splits), 16 * RT) * (16 * RT);
  // buffer offsets (row * words * 4, prefetch up to 4 blocks past the end)
  // stay within int32
  const int64_t max_rows = 0x7FFFFFFFll / (4ll * a.words) - 4 * 16 * RT;
  if (b.rows_per_split > max_rows) b.rows_per_split = max_rows / (16 * RT) * (16 * RT);
  splits = ceil_div(ceil_div(rows, b.rows_per_split), 8) * 8;
  const int64_t spx = splits / 8;
  const int64_t nblocks = 8 * spx * groups;
  if (nblocks > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "grid too large");
  if (dense)
    k_bin_mfma<RT, KS, QT, true, WPE><<<(unsigned)nblocks, 256, 0, ctx->stream>>>(b, (int32_t)groups,
                                                                            (int32_t)spx);
  else
    k_bin_mfma<RT, KS, QT, false, WPE><<<(unsigned)nblocks, 256, 0, ctx->stream>>>(b, (int32_t)groups,
                                                                             (int32_t)spx);
}

static void launch_bin_mfma(vsk_ctx *ctx, const BinMArgs &a, bool dense) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  static const char *names[2] = {"bin_mfma_filter", "bin_mfma_dense"};
  KernelTimer t(ctx, names[dense ? 1 : 0], (double)a.nq * (double)rows);
  switch (a.words) {
  // 128-bit codes: 64 queries a wave and three waves a SIMD (9 % faster
  // than 128 and two at 10M rows, 1,000 queries)
  case 4: launch_bm<2, 2, 4, 3>(ctx, a, dense); break;
  case 8: launch_bm<2, 4, 4>(ctx, a, dense); break;
  case 16: launch_bm<1, 8, 2>(ctx, a, dense); break;
  case 32: launch_bm<1, 16, 1>(ctx, a, dense); break;
  default: fail(VSK_ERR_UNSUPPORTED, "binary code width");
  }
  check_launch(names[dense ? 1 : 0]);
}

// bit i of row r: x[r][i] > 0, at word i/32, bit i%32 (little-endian bytes:
// byte i/8, bit i%8).  One wave per (row, 64 dimensions): the lanes read 64
// consecutive components (coalesced) and one ballot of x > 0 is the two
// words; lanes past d read 0, so padding bits are 0.
__global__ __launch_bounds__(256) void k_binary_encode(const float *x, int64_t n, int32_t d,
                                                       int32_t ld, int32_t words,
                                                       uint32_t *codes) {
  const int lane = threadIdx.x & 63;
  const int32_t chunks = (words + 1) / 2;  // 64-bit pieces per row
  const int64_t total = n * chunks;
  const int64_t wid = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t t = wid; t < total; t += nw) {
    const int64_t r = t / chunks;
    const int32_t c = (int32_t)(t - r * chunks);
    const int32_t j = 64 * c + lane;
    const float v = j < d ? x[r * ld + j] : 0.f;
    const uint64_t m = __builtin_amdgcn_ballot_w64(v > 0.f);
    if (lane < 2 && 2 * c + lane < words)
      codes[r * words + 2 * c + lane] = lane ? (uint32_t)(m >> 32) : (uint32_t)m;
  }
}

__global__ void k_bin_decode(const uint64_t *best, int64_t total, int32_t *dist,
                             int64_t *ids) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t key = best[i];
    if (key == VSK_KEY_NONE) {
      dist[i] = 0x7FFFFFFF;
      ids[i] = -1;
    } else {
      dist[i] = (int32_t)((uint32_t)(key >> 32) ^ 0x80000000u);
      ids[i] = (uint32_t)key;
    }
  }
}

static unsigned grid_n(int64_t n) {
  const int64_t g = ceil_div(n, 256);
  return (unsigned)(g < 1 ? 1 : (g > 16384 ? 16384 : g));
}

__global__ void k_bin_popcount(const uint32_t *codes, int64_t n, int32_t words,
                               int32_t *pop) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int32_t s = 0;
    for (int32_t w = 0; w < words; ++w) s += __builtin_popcount(codes[i * words + w]);
    pop[i] = s;
  }
}

static int32_t bin_words(int32_t d) {
  int32_t w = 4;
  while (w * 32 < d) w *= 2;
  return w;
}

// codes of ceil(d/8) bytes per row (host or device) -> words per row, zero
// padded, on the device
static const uint32_t *codes_to_words(vsk_ctx *ctx, const uint8_t *p, int64_t n,
                                      int32_t d, int32_t words, const std::string &slot) {
  const int32_t bytes = (d + 7) / 8;
  uint32_t *out = static_cast<uint32_t *>(
      ctx->scratch_ptr(slot, sizeof(uint32_t) * (size_t)n * words));
  if (bytes != words * 4) fill_i32(ctx, reinterpret_cast<int32_t *>(out), n * words, 0);
  copy_rows(ctx, out, (size_t)words * 4, p, bytes, bytes, n);
  return out;
}

}  // namespace vsk

using namespace vsk;

extern "C" {

vsk_status vsk_binary_encode(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                             uint8_t *codes) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no vectors");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(x && codes, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  CallScope cs(ctx);
  const int32_t ld = padded_ld(d);
  const float *dx = rows_to_device_padded(ctx, x, n, d, ld, "bin.x");
  const int32_t words = (d + 31) / 32;
  uint32_t *w = static_cast<uint32_t *>(
      ctx->scratch_ptr("bin.enc", sizeof(uint32_t) * (size_t)n * words));
  {
    KernelTimer t(ctx, "binary_encode", (double)n);
    const int64_t waves = n * ((words + 1) / 2);
    const int64_t g = ceil_div(waves, 4);
    k_binary_encode<<<(unsigned)(g < 65536 ? (g > 0 ? g : 1) : 65536), 256, 0, ctx->stream>>>(
        dx, n, d, ld, words, w);
    check_launch("binary_encode");
  }
  const int32_t bytes = (d + 7) / 8;
  copy_rows(ctx, codes, bytes, w, (size_t)words * 4, bytes, n);
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_bin_upload(vsk_ctx *ctx, const uint8_t *codes, int64_t n, int32_t d,
                          vsk_bin **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no codes");
  VSK_REQUIRE(d > 0 && d <= 1024, VSK_ERR_UNSUPPORTED, "binary codes of 1 to 1024 bits");
  VSK_REQUIRE(codes, VSK_ERR_INVALID_ARGUMENT, "codes is null");
  VSK_REQUIRE(n <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "a binary database holds at most 2^31-1 rows");
  CallScope cs(ctx);
  std::unique_ptr<vsk_bin> b(new vsk_bin());
  b->n = n;
  b->d = d;
  b->words = bin_words(d);
  b->codes.reserve(sizeof(uint32_t) * (size_t)n * b->words);
  const int32_t bytes = (d + 7) / 8;
  if (bytes != b->words * 4)
    fill_i32(ctx, b->codes.as<int32_t>(), n * b->words, 0);
  copy_rows(ctx, b->codes.p, (size_t)b->words * 4, codes, bytes, bytes, n);
  b->pop.reserve(sizeof(int32_t) * (size_t)(n + 4));
  fill_i32(ctx, b->pop.as<int32_t>() + n, 4, 0);
  k_bin_popcount<<<grid_n(n), 256, 0, ctx->stream>>>(b->codes.as<uint32_t>(), n, b->words,
                                                      b->pop.as<int32_t>());
  check_launch("bin_popcount");
  cs.finish();
  *out = b.release();
  VSK_API_END(ctx);
}

vsk_status vsk_bin_free(vsk_ctx *ctx, vsk_bin *bin) {
  VSK_API_BEGIN(ctx);
  stream_sync(ctx);
  delete bin;
  VSK_API_END(ctx);
}

static vsk_status bin_search_body(vsk_ctx *ctx, const vsk_bin *bin, const uint8_t *qcodes,
                          int64_t nq, int32_t k, int32_t *out_dist, int64_t *out_ids) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(bin, VSK_ERR_INVALID_ARGUMENT, "bin is null");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(qcodes && out_dist && out_ids, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(k >= 1, VSK_ERR_INVALID_ARGUMENT, "k must be >= 1");
  VSK_REQUIRE(k <= VSK_MAX_K, VSK_ERR_INVALID_BUFFER_SIZE, "k exceeds VSK_MAX_K");
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE, "too many queries");
  CallScope cs(ctx);
  const uint32_t *dq = codes_to_words(ctx, qcodes, nq, bin->d, bin->words, "bin.q");
  uint64_t *best = static_cast<uint64_t *>(
      ctx->scratch_ptr("bin.best", sizeof(uint64_t) * (size_t)nq * k));
  // the int8 matrix-core scan serves batches of queries (a wave holds 16 x
  // QT of them); a handful of queries take the popcount scan
  const bool mfma = nq >= 16 && !ctx->flat_no_screen;
  int32_t *qpop = nullptr;
  if (mfma) {
    qpop = static_cast<int32_t *>(ctx->scratch_ptr("bin.qpop", sizeof(int32_t) * (size_t)nq));
    k_bin_popcount<<<grid_n(nq), 256, 0, ctx->stream>>>(dq, nq, bin->words, qpop);
    check_launch("bin_popcount");
  }
  const int64_t cap = default_cap(k);
  const int64_t qb = query_batch(ctx, nq, cap);
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    BinArgs base{};
    base.X = bin->codes.as<uint32_t>();
    base.Q = dq + b0 * bin->words;
    base.words = bin->words;
    base.nq = (int32_t)nb;
    ScanFn scan = [&](const ScanRequest &r) {
      if (mfma) {
        BinMArgs m{};
        m.X = bin->codes.as<uint32_t>();
        m.Q = base.Q;
        m.xpop = bin->pop.as<int32_t>();
        m.qpop = qpop + b0;
        m.npop = bin->n + 4;
        m.words = bin->words;
        m.nq = base.nq;
        m.r0 = r.r0;
        m.r1 = r.r1;
        m.thresh = r.thresh;
        m.active = r.active;
        m.cand = r.cand;
        m.cap = r.cap;
        m.counts = r.counts;
        launch_bin_mfma(ctx, m, r.dense);
        return;
      }
      BinArgs a = base;
      a.r0 = r.r0;
      a.r1 = r.r1;
      a.thresh = r.thresh;
      a.active = r.active;
      a.cand = r.cand;
      a.cap = r.cap;
      a.counts = r.counts;
      launch_bin(ctx, a, r.dense ? MODE_DENSE : MODE_FILTER);
    };
    progressive_topk(ctx, nb, bin->n, k, cap, scan, best + b0 * k, "bin_select", 8);
  }
  OutputStage od(ctx, out_dist, sizeof(int32_t) * (size_t)nq * k, "out.bdist");
  OutputStage oi(ctx, out_ids, sizeof(int64_t) * (size_t)nq * k, "out.ids");
  {
    KernelTimer t(ctx, "bin_decode");
    k_bin_decode<<<grid_n(nq * k), 256, 0, ctx->stream>>>(best, nq * k, od.ptr<int32_t>(),
                                                          oi.ptr<int64_t>());
    check_launch("bin_decode");
  }
  od.copy_back();
  oi.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

// top-k overflow is checked at the call's end (topk_call)
vsk_status vsk_bin_search(vsk_ctx *ctx, const vsk_bin *bin, const uint8_t *qcodes,
                          int64_t nq, int32_t k, int32_t *out_dist, int64_t *out_ids) {
  return topk_call(ctx, [&] { return bin_search_body(ctx, bin, qcodes, nq, k, out_dist, out_ids); });
}

vsk_status vsk_bin_distances(vsk_ctx *ctx, const vsk_bin *bin, const uint8_t *qcodes,
                             int64_t nq, float *out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(bin, VSK_ERR_INVALID_ARGUMENT, "bin is null");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(qcodes && out, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE, "too many queries");
  CallScope cs(ctx);
  const uint32_t *dq = codes_to_words(ctx, qcodes, nq, bin->d, bin->words, "bin.q");
  OutputStage om(ctx, out, sizeof(float) * (size_t)nq * bin->n, "out.bmatrix");
  BinArgs a{};
  a.X = bin->codes.as<uint32_t>();
  a.Q = dq;
  a.words = bin->words;
  a.nq = (int32_t)nq;
  a.r0 = 0;
  a.r1 = bin->n;
  a.mat = om.ptr<float>();
  a.ldm = bin->n;
  launch_bin(ctx, a, MODE_MATRIX);
  om.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

}  // extern "C"
