// sq8.hip -- int8 scalar quantization: min/max training, encoding and the
// int8-MFMA scan with int32 accumulation fused with the top-k filter.
//
// Reference: ScalarQuantizer (Quantization/ScalarQuantizer.swift):
// calculateStatistics (:389-418, min/max over the values),
// calculateQuantizationParameters (:420-451, .int8: scale = 255/(max-min),
// offset = -min*scale - 128), quantizeToInt8 (:251-270, vDSP_vsmsa then
// vDSP_vfix8: x*scale + offset converted toward zero).  The reference has
// no distance over int8 codes; the scan ranks by the exact int32 score
// sum_j qcode_j * code_j (distance = -score), ties by row id.
//
// Scan kernel: the flat-search tiling on int8 -- a workgroup owns 64 queries
// and a slice of rows, 128-row tiles, 128-byte K stages in LDS, each wave a
// 32-row x 64-query block of 2x4 v_mfma_i32_16x16x32_i8 tiles.  Integer
// accumulation is exact, so scores and ids are bit-identical to the CPU.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "vsk_api.hpp"

struct vsk_sq8 {
  int64_t n = 0;
  int32_t d = 0, ldc = 0;  // ldc: row stride in bytes (multiple of 32)
  // row-major codes: kept only when there is no tiled copy (rows over 512
  // bytes); the tiled copy is then the one layout the scans read
  vsk::DevBuf codes;
  // the codes in 16-row blocks stored in MFMA operand order (see
  // k_sq8_tile); tks 64-byte k-steps a row, 0 if none
  vsk::DevBuf tiles;
  int32_t tks = 0;
};

namespace vsk {

typedef int i4 __attribute__((ext_vector_type(4)));

constexpr int SB_N = 128, SB_Q = 64, SB_K = 128;  // rows, queries, bytes
constexpr int SS = SB_K + 16;                     // LDS row stride (bytes)

struct Sq8Args {
  const int8_t *X;
  int64_t ldx;
  // tiled copy of X (16-row blocks of tks 1 KB k-steps), or null
  const int8_t *T;
  int32_t tks;
  const int8_t *Q;
  int64_t ldq;
  int32_t kbytes;  // padded code length (multiple of 32)
  int32_t nq;
  int64_t r0, r1, rows_per_split;
  const uint64_t *thresh;
  const uint8_t *active;
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
};

template <bool DENSE>
__global__ __launch_bounds__(256) void k_sq8_scan(Sq8Args a) {
  __shared__ __attribute__((aligned(16))) int8_t xs[SB_N * SS];
  __shared__ __attribute__((aligned(16))) int8_t qs[SB_Q * SS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t q0 = (int64_t)blockIdx.x * SB_Q;
  const int64_t s0 = a.r0 + (int64_t)blockIdx.y * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;
  int64_t qi[4];
  bool qok[4];
  uint64_t th[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    qi[j] = q0 + j * 16 + (lane & 15);
    qok[j] = qi[j] < a.nq && (!a.active || a.active[qi[j]]);
    th[j] = (!DENSE && qok[j]) ? a.thresh[qi[j]] : 0;
  }
  const int crow = tid >> 3, ccol = (tid & 7) * 16;
  for (int64_t t0 = s0; t0 < s1; t0 += SB_N) {
    i4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = i4{0, 0, 0, 0};
    for (int k0 = 0; k0 < a.kbytes; k0 += SB_K) {
      const bool kin = k0 + ccol < a.kbytes;
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        int64_t grow = t0 + u * 32 + crow;
        i4 v = (kin && grow < s1)
                   ? *reinterpret_cast<const i4 *>(a.X + grow * a.ldx + k0 + ccol)
                   : i4{0, 0, 0, 0};
        *reinterpret_cast<i4 *>(xs + (u * 32 + crow) * SS + ccol) = v;
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        int64_t gq = q0 + u * 32 + crow;
        i4 v = (kin && gq < a.nq)
                   ? *reinterpret_cast<const i4 *>(a.Q + gq * a.ldq + k0 + ccol)
                   : i4{0, 0, 0, 0};
        *reinterpret_cast<i4 *>(qs + (u * 32 + crow) * SS + ccol) = v;
      }
      __syncthreads();
      const int kend = a.kbytes - k0 < SB_K ? a.kbytes - k0 : SB_K;
      for (int kk = 0; kk < kend; kk += 32) {
        long af[2], bf[4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          af[i] = *reinterpret_cast<const long *>(
              xs + (w * 32 + i * 16 + (lane & 15)) * SS + kk + 8 * (lane >> 4));
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bf[j] = *reinterpret_cast<const long *>(
              qs + (j * 16 + (lane & 15)) * SS + kk + 8 * (lane >> 4));
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[i], bf[j],
                                                              acc[i][j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = t0 + w * 32 + i * 16 + 4 * (lane >> 4) + r;
        if (row >= s1) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!qok[j]) continue;
          const uint64_t key = vsk_key_i32(-acc[i][j][r], (uint32_t)row);
          if (DENSE) {
            a.cand[qi[j] * a.cap + (row - a.r0)] = key;
          } else if (key <= th[j]) {
            int slot = atomicAdd(&a.counts[qi[j]], 1);
            if (slot < a.cap) a.cand[qi[j] * a.cap + slot] = key;
          }
        }
      }
    }
  }
}

// Register-resident scan for codes up to 1024 bytes (the common case).
// Each wave keeps QT query tiles (16 queries each) of KS 64-byte k-steps as
// v_mfma_i32_16x16x64_i8 B operands in registers for the whole launch and
// streams 16-row A tiles of the database straight from memory (buffer loads,
// no LDS); the four waves of a workgroup hold different queries and read the
// same rows, which they share through L1.  The filter test is one integer
// compare per score against the query's score floor; the 64-bit key is built
// only where a score can pass.  Workgroup L runs on XCD L % 8, and the query
// groups of one row split are consecutive slots of one XCD so they share its
// L2.

// the first k-step takes the constant 0 as its accumulator operand (no
// register moves to clear the accumulators)
template <int RT, int KS, int QT>
__device__ __forceinline__ void sq8_mma(const i4 (&ar)[RT][KS],
                                        const i4 (&bq)[QT][KS],
                                        i4 (&acc)[RT][QT]) {
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < QT; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ar[i][0], bq[j][0], i4{0, 0, 0, 0},
                                                        0, 0, 0);
#pragma unroll
  for (int ks = 1; ks < KS; ++ks)
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int j = 0; j < QT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ar[i][ks], bq[j][ks],
                                                          acc[i][j], 0, 0, 0);
}

// Filtered candidates are staged per wave in LDS (SQ_WBUF entries) and
// appended to the global per-query lists only when the list fills and at
// the end, 64 at a time: an atomic that returns a value makes the wave wait
// for every memory operation it has in flight, row prefetches included.
constexpr int SQ_WBUF = 512;

__device__ __forceinline__ void sq8_flush(const Sq8Args &a, const uint64_t *lkey,
                                          const int32_t *lq, int32_t &nbuf,
                                          int lane) {
  for (int32_t e = lane; e < nbuf; e += 64) {
    const int32_t q = lq[e];
    const int c = atomicAdd(&a.counts[q], 1);
    if (c < a.cap) a.cand[(int64_t)q * a.cap + c] = lkey[e];
  }
  nbuf = 0;
}

// scores of rows t0 .. t0 + 16*RT - 1 (absolute ids) against the wave's
// queries: every key of valid rows in the dense chunk, else the keys that
// pass the query's threshold
template <int RT, int QT, bool DENSE>
__device__ __forceinline__ void sq8_epilogue(
    const Sq8Args &a, const i4 (&acc)[RT][QT], int64_t t0, int64_t s1,
    int lane, int64_t qw0, const bool (&qok)[QT], const int32_t (&smin)[QT],
    const uint64_t (&th)[QT], uint64_t *lkey, int32_t *lq, int32_t &nbuf) {
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int64_t rb = t0 + 16 * i + 4 * (lane >> 4);  // + r
    if (DENSE) {
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        if (!qok[j]) continue;
        const int64_t q = qw0 + 16 * j + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (rb + r < s1)
            a.cand[q * a.cap + (rb + r - a.r0)] =
                vsk_key_i32(-acc[i][j][r], (uint32_t)(rb + r));
      }
    }
  }
  if (DENSE) return;
  // filter: per query tile, the largest of the lane's 4 * RT scores first,
  // so the common case (nothing passes anywhere in the wave) is a few maxima,
  // one compare and one ballot per query tile
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    int32_t mx = acc[0][j][0];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = acc[i][j][r] > mx ? acc[i][j][r] : mx;
    if (!__builtin_amdgcn_ballot_w64(mx >= smin[j])) continue;  // the common case
    // key <= th[j]: a higher score, or the floor score at a row id not
    // above the threshold's.  Control flow stays wave-uniform so nbuf
    // stays uniform: passing keys take consecutive slots of the wave's
    // LDS list in lane order.
    const uint32_t trow = (uint32_t)th[j];
    const int32_t q = (int32_t)(qw0 + 16 * j + (lane & 15));
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int64_t rb = t0 + 16 * i + 4 * (lane >> 4);  // + r
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t v = acc[i][j][r];
        const bool p = rb + r < s1 &&
                       (v > smin[j] || (v == smin[j] && (uint32_t)(rb + r) <= trow));
        const uint64_t m = __builtin_amdgcn_ballot_w64(p);
        if (!m) continue;
        if (p) {
          const int32_t pos =
              nbuf + (int32_t)__builtin_amdgcn_mbcnt_hi(
                         (uint32_t)(m >> 32),
                         __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
          lkey[pos] = vsk_key_i32(-v, (uint32_t)(rb + r));
          lq[pos] = q;
        }
        nbuf += __builtin_popcountll(m);
      }
      if (nbuf > SQ_WBUF - 256) sq8_flush(a, lkey, lq, nbuf, lane);
    }
  }
}

template <int RT, int KS, int QT, bool DENSE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_sq8_reg(Sq8Args a, int32_t groups, int32_t splits_per_xcd) {
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
  const int kc = 16 * (lane >> 4);  // this lane's byte chunk of a k-step

  i4 bq[QT][KS];
  int32_t smin[QT];
  uint64_t th[QT];
  bool qok[QT];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int64_t q = qw0 + 16 * j + (lane & 15);
    qok[j] = q < a.nq && (!a.active || a.active[q]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int off = 64 * ks + kc;
      bq[j][ks] = (qok[j] && off < a.kbytes)
                      ? *reinterpret_cast<const i4 *>(a.Q + q * a.ldq + off)
                      : i4{0, 0, 0, 0};
    }
    th[j] = (!DENSE && qok[j]) ? a.thresh[q] : 0;
    // key <= th needs -score <= the distance half of th: score >= smin
    smin[j] = qok[j] ? -(int32_t)((uint32_t)(th[j] >> 32) ^ 0x80000000u)
                     : 0x7FFFFFFF;
  }

  const int64_t nrows = s1 - s0;
  // the tiled copy when there is one (as in k_sq8_pipe; s0 a multiple of 16)
  const bool tiled = a.T != nullptr;
  const __amdgpu_buffer_rsrc_t rx =
      tiled ? __builtin_amdgcn_make_buffer_rsrc(
                  (void *)(a.T + (s0 >> 4) * (KS * 1024)), 0,
                  (int32_t)(((nrows + 15) >> 4) * (KS * 1024)), 0x00020000)
            : __builtin_amdgcn_make_buffer_rsrc((void *)(a.X + s0 * a.ldx), 0,
                                                (int32_t)(nrows * a.ldx), 0x00020000);
  const int32_t rstep = tiled ? KS * 64 : (int32_t)a.ldx;
  const int32_t lrow = tiled ? lane * 16 : (int32_t)(lane & 15) * (int32_t)a.ldx + kc;
  const int32_t kstep = tiled ? 1024 : 64;
  i4 ar0[RT][KS], ar1[RT][KS];
#define SR_LOAD(AR, T)                                                       \
  _Pragma("unroll") for (int i = 0; i < RT; ++i)                          \
  _Pragma("unroll") for (int ks = 0; ks < KS; ++ks)                          \
      AR[i][ks] = __builtin_bit_cast(                                        \
          i4, __builtin_amdgcn_raw_buffer_load_b128(                         \
                  rx, (int32_t)((T) + 16 * i) * rstep + lrow, kstep * ks, 0))
  i4 acc[RT][QT];
  __shared__ uint64_t s_key[4][DENSE ? 1 : SQ_WBUF];
  __shared__ int32_t s_q[4][DENSE ? 1 : SQ_WBUF];
  int32_t nbuf = 0;  // wave-uniform count of staged candidates
  // two row blocks in flight: a block's buffer is refilled with the block
  // after next once its multiplies and filter are done.  Loads past the
  // split read zeros from the buffer descriptor, so they need no condition
  // (a conditional load would make the compiler wait for every load at the
  // loop head).
  constexpr int32_t RB = 16 * RT;
  const int32_t nr = (int32_t)nrows;
  // scheduling barriers keep the loads and multiplies in program order:
  // the first block's loads are issued before the second's (on entry as on
  // the loop's back edge), so the wait at the loop head covers only them
  SR_LOAD(ar0, 0);
  __builtin_amdgcn_sched_barrier(0);
  SR_LOAD(ar1, RB);
  __builtin_amdgcn_sched_barrier(0);
  for (int32_t t = 0; t < nr; t += 2 * RB) {
    sq8_mma<RT, KS, QT>(ar0, bq, acc);
    sq8_epilogue<RT, QT, DENSE>(a, acc, s0 + t, s1, lane, qw0, qok, smin, th,
                                s_key[w], s_q[w], nbuf);
    SR_LOAD(ar0, t + 2 * RB);
    __builtin_amdgcn_sched_barrier(0);
    // the second block may lie past the split: it reads zeros and the
    // epilogue drops its rows (no exit mid-body, which would make the
    // compiler carry the prefetch registers around the loop by copies)
    sq8_mma<RT, KS, QT>(ar1, bq, acc);
    sq8_epilogue<RT, QT, DENSE>(a, acc, s0 + t + RB, s1, lane, qw0, qok, smin,
                                th, s_key[w], s_q[w], nbuf);
    SR_LOAD(ar1, t + 3 * RB);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (!DENSE && nbuf > 0) sq8_flush(a, s_key[w], s_q[w], nbuf, lane);
#undef SR_LOAD
}

// Filter scan with the test software-pipelined: the two waves of a SIMD run
// the same code in step, so a test that follows its own block's multiplies
// leaves the matrix pipe idle while both waves test.  Here each wave
// multiplies row block b into one accumulator set while it tests block b-1
// in the other (the test's maxima and compares fill the MFMA shadow; the
// exact candidate path is a rare branch after the multiplies).  16-row
// blocks, NPF of them in flight in registers.
// does any lane hold a score >= its query's floor (wave-uniform)
template <int QT>
__device__ __forceinline__ bool sq8_any_pass(const i4 (&acc)[1][QT], const int32_t (&smin)[QT]) {
  uint64_t any = 0;
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const i4 v = acc[0][j];
    const int32_t m01 = v[0] > v[1] ? v[0] : v[1];
    const int32_t m23 = v[2] > v[3] ? v[2] : v[3];
    const int32_t mx = m01 > m23 ? m01 : m23;
    any |= __builtin_amdgcn_ballot_w64(mx >= smin[j]);
  }
  return any != 0;
}

// The tiled copy of a code matrix: 16-row block b, k-step ks (64 bytes of
// each row) is 1 KB at (b * ks_n + ks) KB, whose 16 bytes at 16 l hold row
// 16 b + (l & 15), bytes 64 ks + 16 (l >> 4): the v_mfma_i32_16x16x64_i8
// A operand of lane l.  Rows past n and bytes past ldc are zero.  A thread
// per 16 bytes, grid-stride.
__global__ __launch_bounds__(256) void k_sq8_tile(const int8_t *X, int64_t n, int32_t ldc,
                                                  int32_t ks_n, int64_t total, int8_t *T) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {  // 16-byte unit
    const int l = (int)(i & 63);
    const int64_t bk = i >> 6;  // block * ks_n + ks
    const int64_t b = bk / ks_n;
    const int ks = (int)(bk - b * ks_n);
    const int64_t row = 16 * b + (l & 15);
    const int32_t off = 64 * ks + 16 * (l >> 4);
    i4 v = i4{0, 0, 0, 0};
    if (row < n && off < ldc) v = *reinterpret_cast<const i4 *>(X + row * ldc + off);
    reinterpret_cast<i4 *>(T)[i] = v;
  }
}

// WPE: waves a SIMD holds (the register budget per wave)
template <int KS, int QT, int NPF, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void k_sq8_pipe(Sq8Args a, int32_t groups, int32_t splits_per_xcd) {
  constexpr int RT = 1;
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
  const int kc = 16 * (lane >> 4);  // this lane's byte chunk of a k-step

  i4 bq[QT][KS];
  int32_t smin[QT];
  uint64_t th[QT];
  bool qok[QT];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int64_t q = qw0 + 16 * j + (lane & 15);
    qok[j] = q < a.nq && (!a.active || a.active[q]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int off = 64 * ks + kc;
      bq[j][ks] = (qok[j] && off < a.kbytes)
                      ? *reinterpret_cast<const i4 *>(a.Q + q * a.ldq + off)
                      : i4{0, 0, 0, 0};
    }
    th[j] = qok[j] ? a.thresh[q] : 0;
    // key <= th needs -score <= the distance half of th: score >= smin
    smin[j] = qok[j] ? -(int32_t)((uint32_t)(th[j] >> 32) ^ 0x80000000u) : 0x7FFFFFFF;
  }

  const int64_t nrows = s1 - s0;
  // Row blocks come from the tiled copy when there is one: block b's k-step
  // ks is the 1 KB at (b * KS + ks) KB, lane l's 16 bytes at 16 l, so a
  // wave's load is contiguous (from the row-major codes the 16 lanes of a
  // quarter-wave touch 16 rows).  s0 is a multiple of 16 (launch_pipe).
  const bool tiled = a.T != nullptr;
  const __amdgpu_buffer_rsrc_t rx =
      tiled ? __builtin_amdgcn_make_buffer_rsrc(
                  (void *)(a.T + (s0 >> 4) * (KS * 1024)), 0,
                  (int32_t)(((nrows + 15) >> 4) * (KS * 1024)), 0x00020000)
            : __builtin_amdgcn_make_buffer_rsrc((void *)(a.X + s0 * a.ldx), 0,
                                                (int32_t)(nrows * a.ldx), 0x00020000);
  // byte offset of row T's block (T a multiple of 16) and this lane's part
  const int32_t rstep = tiled ? KS * 64 : (int32_t)a.ldx;
  const int32_t lrow = tiled ? lane * 16 : (int32_t)(lane & 15) * (int32_t)a.ldx + kc;
  const int32_t kstep = tiled ? 1024 : 64;
  i4 ar[NPF][RT][KS];
#define SP_LOAD(AR, T)                                                          \
  _Pragma("unroll") for (int ks = 0; ks < KS; ++ks) AR[0][ks] = __builtin_bit_cast( \
      i4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int32_t)(T) * rstep + lrow, \
                                                kstep * ks, 0))
  __shared__ uint64_t s_key[4][SQ_WBUF];
  __shared__ int32_t s_q[4][SQ_WBUF];
  int32_t nbuf = 0;  // wave-uniform count of staged candidates
  constexpr int32_t RB = 16;
  const int32_t nr = (int32_t)nrows;
  // A lane whose 4 scores of a query tile may pass (their largest reaches
  // the query's floor) queues them with their place (16-row block, tile,
  // lane) and the query's floor and threshold row; the queue is tested, a
  // block a lane, when full and at the end of the split, so the exact test
  // leaves the multiply pipeline once per SQ_QC blocks instead of once per
  // block that holds a candidate.
  constexpr int SQ_QC = 64;
  __shared__ i4 s_qv[4][SQ_QC];
  __shared__ int32_t s_qm[4][SQ_QC];
  __shared__ int2 s_qt[4][SQ_QC];
  int32_t qn = 0;  // queued blocks (wave-uniform)
  auto drain = [&]() {
    if (nbuf > SQ_WBUF - 4 * SQ_QC) sq8_flush(a, s_key[w], s_q[w], nbuf, lane);
    const bool has = lane < qn;
    const i4 v = has ? s_qv[w][lane] : i4{0, 0, 0, 0};
    const uint32_t pw = has ? (uint32_t)s_qm[w][lane] : 0u;
    const int2 st = has ? s_qt[w][lane] : int2{0x7FFFFFFF, 0};
    const int jj = (int)((pw >> 6) & 7u), sl = (int)(pw & 63u);
    const int32_t q = (int32_t)(qw0 + 16 * jj + (sl & 15));
    const int64_t rb = s0 + (int64_t)(pw >> 9) * RB + 4 * (sl >> 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = rb + r;
      const bool p = has && row < s1 &&
                     (v[r] > st.x || (v[r] == st.x && (uint32_t)row <= (uint32_t)st.y));
      const uint64_t m = __builtin_amdgcn_ballot_w64(p);
      if (!m) continue;
      if (p) {
        const int32_t pos = nbuf + (int32_t)__builtin_amdgcn_mbcnt_hi(
                                       (uint32_t)(m >> 32),
                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        s_key[w][pos] = vsk_key_i32(-v[r], (uint32_t)row);
        s_q[w][pos] = q;
      }
      nbuf += __builtin_popcountll(m);
    }
    qn = 0;
  };
  // block blk (16 rows from s0 + 16 blk) of accumulator set ac
  auto push = [&](const i4 (&ac)[1][QT], int32_t blk) {
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      const i4 v = ac[0][j];
      const int32_t m01 = v[0] > v[1] ? v[0] : v[1];
      const int32_t m23 = v[2] > v[3] ? v[2] : v[3];
      bool f = (m01 > m23 ? m01 : m23) >= smin[j];
      uint64_t bal = __builtin_amdgcn_ballot_w64(f);
      while (bal) {  // one pass unless the queue fills
        if (qn == SQ_QC) drain();
        const uint32_t pos = __builtin_amdgcn_mbcnt_hi(
            (uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        const int room = SQ_QC - qn;
        if (f && (int)pos < room) {
          const int e = qn + (int)pos;
          s_qv[w][e] = v;
          s_qm[w][e] = (blk << 9) | (j << 6) | lane;
          s_qt[w][e] = int2{smin[j], (int32_t)(uint32_t)th[j]};
        }
        const int n = __builtin_popcountll(bal);
        if (n <= room) {
          qn += n;
          break;
        }
        qn = SQ_QC;
        f = f && (int)pos >= room;
        bal = __builtin_amdgcn_ballot_w64(f);
      }
    }
  };
  i4 acc[2][RT][QT];
  // the "previous block" of the first: scores that pass no floor
#pragma unroll
  for (int j = 0; j < QT; ++j) acc[1][0][j] = i4{INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN};
#pragma unroll
  for (int p = 0; p < NPF; ++p) {
    SP_LOAD(ar[p], p * RB);
    __builtin_amdgcn_sched_barrier(0);
  }
  // block b: multiply into set b & 1 while testing block b - 1 (set
  // (b + 1) & 1), refill b's registers with block b + NPF, then the exact
  // path for block b - 1 if a score of it may pass.  A split is a whole
  // number of NPF-block steps (but the last), and blocks past it read zeros
  // whose rows the exact path drops.
#define SP_BLOCK(P)                                                             \
  do {                                                                          \
    constexpr int X = (P) & 1, Y = X ^ 1;                                       \
    sq8_mma<RT, KS, QT>(ar[P], bq, acc[X]);                                     \
    const bool hit = sq8_any_pass<QT>(acc[Y], smin);                            \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                          \
    _Pragma("unroll") for (int u = 0; u < QT * KS - 1; ++u) {                   \
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);                        \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                        \
    }                                                                           \
    __builtin_amdgcn_sched_barrier(0);                                          \
    SP_LOAD(ar[P], t + ((P) + NPF) * RB);                                       \
    __builtin_amdgcn_sched_barrier(0);                                          \
    if (hit) push(acc[Y], (t + ((P) - 1) * RB) >> 4);                          \
  } while (0)
  static_assert(NPF == 4, "four blocks per step: the register sets are fixed per position");
  for (int32_t t = 0; t < nr; t += NPF * RB) {
    SP_BLOCK(0);
    SP_BLOCK(1);
    SP_BLOCK(2);
    SP_BLOCK(3);
  }
#undef SP_BLOCK
#undef SP_LOAD
  // the last block (set 1: NPF is even)
  if (sq8_any_pass<QT>(acc[1], smin))
    push(acc[1], (((nr + NPF * RB - 1) / (NPF * RB)) * NPF * RB - RB) >> 4);
  if (qn) drain();
  if (nbuf > 0) sq8_flush(a, s_key[w], s_q[w], nbuf, lane);
}

template <int KS, int QT, int NPF, int WPE = 2>
static void launch_pipe(vsk_ctx *ctx, const Sq8Args &a) {
  const int64_t rows = a.r1 - a.r0;
  const int64_t qpg = 4 * QT * 16;  // queries per workgroup
  const int64_t groups = ceil_div(a.nq, qpg);
  // row splits: a multiple of 8 (one share per XCD), about 4096 workgroups
  int64_t splits = ceil_div(4096, groups);
  constexpr int64_t step = (int64_t)NPF * 16;  // rows per loop trip
  const int64_t max_splits = ceil_div(rows, step);
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  Sq8Args b = a;
  // the tiled copy holds 16-row blocks of this instance's k-steps
  if ((a.r0 & 15) || a.tks != KS) b.T = nullptr;
  if (!b.T && !b.X)
    fail(VSK_ERR_INVALID_ARGUMENT, "SQ8 scan: a chunk the tiled codes do not cover");
  b.rows_per_split = ceil_div(ceil_div(rows, splits), step) * step;
  // buffer offsets (row * ldx, or row * KS * 64 in the tiled copy; prefetch
  // up to 2 NPF blocks past the end) stay within int32
  const int64_t stride = b.T ? (int64_t)KS * 64 : a.ldx;
  // (and the filter queue's position word holds a 16-row block index of
  // 23 bits)
  const int64_t max_rows =
      std::min<int64_t>(0x7FFFFFFFll / stride - 2 * step, (int64_t)1 << 26);
  if (b.rows_per_split > max_rows) b.rows_per_split = max_rows / step * step;
  splits = ceil_div(ceil_div(rows, b.rows_per_split), 8) * 8;
  const int64_t spx = splits / 8;
  const int64_t nblocks = 8 * spx * groups;
  if (nblocks > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "grid too large");
  k_sq8_pipe<KS, QT, NPF, WPE><<<(unsigned)nblocks, 256, 0, ctx->stream>>>(b, (int32_t)groups,
                                                                      (int32_t)spx);
}

template <int RT, int KS, int QT>
static void launch_reg(vsk_ctx *ctx, const Sq8Args &a, bool dense) {
  const int64_t rows = a.r1 - a.r0;
  const int64_t qpg = 4 * QT * 16;  // queries per workgroup
  const int64_t groups = ceil_div(a.nq, qpg);
  // row splits: a multiple of 8 (one share per XCD), about 4096 workgroups
  int64_t splits = ceil_div(4096, groups);
  const int64_t max_splits = ceil_div(rows, 16 * RT);
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  Sq8Args b = a;
  // the tiled copy holds 16-row blocks of this instance's k-steps
  if ((a.r0 & 15) || a.tks != KS) b.T = nullptr;
  if (!b.T && !b.X)
    fail(VSK_ERR_INVALID_ARGUMENT, "SQ8 scan: a chunk the tiled codes do not cover");
  b.rows_per_split = ceil_div(ceil_div(rows, splits), 16 * RT) * (16 * RT);
  // buffer offsets (row * ldx, or row * KS * 64 in the tiled copy; prefetch
  // up to 4 blocks past the end) stay within int32
  const int64_t stride = b.T ? (int64_t)KS * 64 : a.ldx;
  const int64_t max_rows = 0x7FFFFFFFll / stride - 4 * 16 * RT;
  if (b.rows_per_split > max_rows)
    b.rows_per_split = max_rows / (16 * RT) * (16 * RT);
  splits = ceil_div(ceil_div(rows, b.rows_per_split), 8) * 8;
  const int64_t spx = splits / 8;
  const int64_t nblocks = 8 * spx * groups;
  if (nblocks > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "grid too large");
  if (dense)
    k_sq8_reg<RT, KS, QT, true><<<(unsigned)nblocks, 256, 0, ctx->stream>>>(
        b, (int32_t)groups, (int32_t)spx);
  else
    k_sq8_reg<RT, KS, QT, false><<<(unsigned)nblocks, 256, 0, ctx->stream>>>(
        b, (int32_t)groups, (int32_t)spx);
}

static void launch_sq8(vsk_ctx *ctx, Sq8Args a, bool dense) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  const int64_t qt = ceil_div(a.nq, SB_Q);
  int64_t splits = ceil_div(4096, qt);
  const int64_t max_splits = ceil_div(rows, SB_N);
  if (splits > max_splits) splits = max_splits;
  if (splits > 65535) splits = 65535;
  if (splits < 1) splits = 1;
  a.rows_per_split = ceil_div(ceil_div(rows, splits), SB_N) * SB_N;
  splits = ceil_div(rows, a.rows_per_split);
  dim3 grid((unsigned)qt, (unsigned)splits);
  KernelTimer t(ctx, dense ? "sq8_mfma_dense" : "sq8_mfma_filter",
                (double)a.nq * (double)rows);
  const int32_t ksteps = (a.kbytes + 63) / 64;
  // the filter scan pipelines its test (up to 512-byte codes; longer ones
  // leave no registers for four row blocks in flight)
  if (!dense && ksteps <= 8) {
    if (ksteps <= 1)
      launch_pipe<1, 8, 4>(ctx, a);
    else if (ksteps <= 2)
      // 64 queries a wave and three waves a SIMD: 4 % faster than 128 and
      // two at config 4 (the test's VALU work overlaps more MFMAs); 32
      // queries a wave read each row block too often
      launch_pipe<2, 4, 4, 3>(ctx, a);
    else if (ksteps <= 4)
      launch_pipe<4, 4, 4>(ctx, a);
    else
      launch_pipe<8, 2, 4>(ctx, a);
  } else if (ksteps <= 1)
    launch_reg<2, 1, 8>(ctx, a, dense);
  else if (ksteps <= 2)
    launch_reg<2, 2, 8>(ctx, a, dense);
  else if (ksteps <= 4)
    launch_reg<2, 4, 4>(ctx, a, dense);
  else if (ksteps <= 8)
    launch_reg<1, 8, 2>(ctx, a, dense);
  else if (ksteps <= 16)
    launch_reg<1, 16, 1>(ctx, a, dense);
  else if (dense)
    k_sq8_scan<true><<<grid, 256, 0, ctx->stream>>>(a);
  else
    k_sq8_scan<false><<<grid, 256, 0, ctx->stream>>>(a);
  check_launch("sq8_mfma_scan");
}

// per-block partial min/max per dimension
__global__ __launch_bounds__(256) void k_minmax_partial(const float *x,
                                                        int64_t n, int32_t d,
                                                        int64_t rows_per_block,
                                                        float *pmin,
                                                        float *pmax) {
  const int64_t r0 = blockIdx.x * rows_per_block;
  int64_t r1 = r0 + rows_per_block;
  if (r1 > n) r1 = n;
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    float mn = __int_as_float(0x7f800000), mx = -__int_as_float(0x7f800000);
    for (int64_t r = r0; r < r1; ++r) {
      float v = x[r * d + j];
      mn = v < mn ? v : mn;
      mx = v > mx ? v : mx;
    }
    pmin[(int64_t)blockIdx.x * d + j] = mn;
    pmax[(int64_t)blockIdx.x * d + j] = mx;
  }
}

// code = clamp(trunc(x * scale + offset)), multiply and add rounded apart
__global__ void k_sq8_encode(const float *x, int64_t n, int32_t d,
                             int32_t per_dim, const float *scale,
                             const float *offset, int8_t *codes, int32_t ldc) {
#pragma clang fp contract(off)
  const int64_t total = n * (int64_t)d;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / d;
    const int32_t j = (int32_t)(i - r * d);
    const float s = per_dim ? scale[j] : scale[0];
    const float o = per_dim ? offset[j] : offset[0];
    float t = x[i] * s;
    t = t + o;
    int8_t c;
    if (!(t > -128.0f))
      c = -128;
    else if (t >= 127.0f)
      c = 127;
    else
      c = (int8_t)(int32_t)t;
    codes[r * ldc + j] = c;
  }
}

// dequantizeFromInt8 (Quantization/ScalarQuantizer.swift:568-580):
// x = (Float(code) - offset) / scale, each operation rounded on its own
__global__ void k_sq8_dequantize(const int8_t *codes, int64_t n, int32_t d,
                                 int32_t per_dim, const float *scale,
                                 const float *offset, float *out) {
#pragma clang fp contract(off)
  const int64_t total = n * d;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t j = (int32_t)(i % d);
    const float s = per_dim ? scale[j] : scale[0];
    const float o = per_dim ? offset[j] : offset[0];
    out[i] = ((float)codes[i] - o) / s;
  }
}

__global__ void k_sq8_decode(const uint64_t *best, int64_t total,
                             int32_t *score, int64_t *ids) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t key = best[i];
    if (key == VSK_KEY_NONE) {
      score[i] = (int32_t)0x80000000;
      ids[i] = -1;
    } else {
      score[i] = -(int32_t)((uint32_t)(key >> 32) ^ 0x80000000u);
      ids[i] = (uint32_t)key;
    }
  }
}

// quantizeVectors(scheme: .scalar(bits:)) on the CPU path
// (Acceleration/AccelerateOptimizer.swift:387-430): per vector, min and max
// of its values, scale = (2^bits - 1) / (max - min) (1 when max == min),
// code_i = UInt8(min(max((x_i - min) * scale, 0), 255)), the conversion
// truncating toward zero.  One wave per row; min and max are exact in any
// order.
__global__ __launch_bounds__(256) void k_scalar_quantize_u8(const float *x, int64_t n,
                                                           int32_t d, float levels,
                                                           uint8_t *codes, float *scale,
                                                           float *minv) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const float *xr = x + row * d;
  float mn = __int_as_float(0x7f800000), mx = -__int_as_float(0x7f800000);
  for (int32_t j = lane; j < d; j += 64) {
    const float v = xr[j];
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o));
    mx = fmaxf(mx, __shfl_xor(mx, o));
  }
  const float range = mx - mn;
  const float s = range > 0.0f ? levels / range : 1.0f;
  uint8_t *cr = codes + row * d;
  for (int32_t j = lane; j < d; j += 64) {
    float t = xr[j] - mn;
    t = t * s;
    t = fminf(fmaxf(t, 0.0f), 255.0f);
    cr[j] = (uint8_t)(uint32_t)t;
  }
  if (lane == 0) {
    if (scale) scale[row] = s;
    if (minv) minv[row] = mn;
  }
}

static unsigned grid1(int64_t n) {
  int64_t g = ceil_div(n, 256);
  return (unsigned)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

// the reference's parameter formulas with each operation rounded on its own
static void sq8_params(float mn, float mx, float *s, float *o) {
#pragma clang fp contract(off)
  float range = mx - mn;
  float scale = range > 0.0f ? 255.0f / range : 1.0f;
  float t = -mn * scale;
  *s = scale;
  *o = t - 128.0f;
}

// codes (host or device, n x d) -> device buffer with row stride ldc
static const int8_t *codes_to_device(vsk_ctx *ctx, const int8_t *p, int64_t n,
                                     int32_t d, int32_t ldc,
                                     const std::string &slot) {
  bool dev = is_device_ptr(p);
  if (dev && ldc == d) return p;
  int8_t *out = static_cast<int8_t *>(ctx->scratch_ptr(slot, (size_t)n * ldc));
  if (ldc != d) fill_i32(ctx, reinterpret_cast<int32_t *>(out), n * ldc / 4, 0);
  copy_rows(ctx, out, ldc, p, d, d, n);
  return out;
}

// ---------------------------------------------------------------------------
// Scratch of the no-allocation search (vsk_sq8_search_noalloc): one static
// device array per GPU, held until the process ends.  Host code never passes
// `scratch` itself to a kernel (on the host the name is only a stand-in);
// it uses the device address hipGetSymbolAddress gives, per device, at
// context creation.  Every call on one GPU shares that GPU's array, so calls
// that overlap on one GPU (two contexts, two threads) race.
// ---------------------------------------------------------------------------
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_noalloc_mu;
static bool g_noalloc_done[NOALLOC_MAX_DEVICES];
static hipError_t g_noalloc_err[NOALLOC_MAX_DEVICES];
static unsigned char *g_noalloc_ptr[NOALLOC_MAX_DEVICES];

// Resolves the device address of this GPU's scratch array once per device;
// the device must be current.  Called by vsk_create.
void sq8_noalloc_setup(int device) {
  if (device < 0 || device >= NOALLOC_MAX_DEVICES) return;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (g_noalloc_done[device]) return;
  void *p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    p = nullptr;
  }
  g_noalloc_err[device] = e;
  g_noalloc_ptr[device] = static_cast<unsigned char *>(p);
  g_noalloc_done[device] = true;
}

static unsigned char *noalloc_scratch(int device) {
  VSK_REQUIRE(device >= 0 && device < NOALLOC_MAX_DEVICES, VSK_ERR_DEVICE_NOT_AVAILABLE,
              "device index beyond the no-allocation scratch table");
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  VSK_REQUIRE(g_noalloc_done[device], VSK_ERR_EXECUTION_FAILED,
              "no-allocation scratch not set up for this device");
  if (!g_noalloc_ptr[device])
    fail(VSK_ERR_EXECUTION_FAILED,
         std::string("hipGetSymbolAddress of the no-allocation scratch failed: ") +
             hipGetErrorString(g_noalloc_err[device]));
  return g_noalloc_ptr[device];
}

// bytes of one carved region, rounded to 256
static size_t region(size_t bytes) { return (bytes + 255) & ~size_t(255); }

}  // namespace vsk

using namespace vsk;

extern "C" {

vsk_status vsk_sq8_train(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                         int32_t per_dim, float *scale, float *offset) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no training vectors");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(x && scale && offset, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  CallScope cs(ctx);
  const float *dx = static_cast<const float *>(
      input_to_device(ctx, x, sizeof(float) * n * d, "sq8.x"));
  int64_t blocks = ceil_div(n, 4096);
  if (blocks > 4096) blocks = 4096;
  const int64_t rpb = ceil_div(n, blocks);
  blocks = ceil_div(n, rpb);
  float *pmin = static_cast<float *>(
      ctx->scratch_ptr("sq8.pmin", sizeof(float) * blocks * d));
  float *pmax = static_cast<float *>(
      ctx->scratch_ptr("sq8.pmax", sizeof(float) * blocks * d));
  {
    KernelTimer t(ctx, "sq8_minmax");
    k_minmax_partial<<<(unsigned)blocks, 256, 0, ctx->stream>>>(dx, n, d, rpb,
                                                                pmin, pmax);
    check_launch("sq8_minmax");
  }
  std::vector<float> hmin(blocks * d), hmax(blocks * d);
  VSK_HIP(hipMemcpyAsync(hmin.data(), pmin, 4 * hmin.size(),
                         hipMemcpyDeviceToHost, ctx->stream));
  VSK_HIP(hipMemcpyAsync(hmax.data(), pmax, 4 * hmax.size(),
                         hipMemcpyDeviceToHost, ctx->stream));
  cs.finish();
  std::vector<float> mn(d, INFINITY), mx(d, -INFINITY);
  for (int64_t b = 0; b < blocks; ++b)
    for (int32_t j = 0; j < d; ++j) {
      mn[j] = std::min(mn[j], hmin[b * d + j]);
      mx[j] = std::max(mx[j], hmax[b * d + j]);
    }
  std::vector<float> s(d), o(d);
  if (per_dim) {
    for (int32_t j = 0; j < d; ++j) sq8_params(mn[j], mx[j], &s[j], &o[j]);
  } else {
    float gmn = *std::min_element(mn.begin(), mn.end());
    float gmx = *std::max_element(mx.begin(), mx.end());
    sq8_params(gmn, gmx, &s[0], &o[0]);
  }
  const size_t cnt = per_dim ? d : 1;
  if (is_device_ptr(scale))
    VSK_HIP(hipMemcpy(scale, s.data(), 4 * cnt, hipMemcpyHostToDevice));
  else
    std::memcpy(scale, s.data(), 4 * cnt);
  if (is_device_ptr(offset))
    VSK_HIP(hipMemcpy(offset, o.data(), 4 * cnt, hipMemcpyHostToDevice));
  else
    std::memcpy(offset, o.data(), 4 * cnt);
  VSK_API_END(ctx);
}

vsk_status vsk_sq8_encode(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                          int32_t per_dim, const float *scale,
                          const float *offset, int8_t *codes) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no vectors");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(x && scale && offset && codes, VSK_ERR_INVALID_ARGUMENT,
              "null buffer");
  CallScope cs(ctx);
  const size_t cnt = per_dim ? d : 1;
  const float *dx = static_cast<const float *>(
      input_to_device(ctx, x, sizeof(float) * n * d, "sq8.x"));
  const float *ds = static_cast<const float *>(
      input_to_device(ctx, scale, 4 * cnt, "sq8.scale"));
  const float *dof = static_cast<const float *>(
      input_to_device(ctx, offset, 4 * cnt, "sq8.offset"));
  OutputStage oc(ctx, codes, (size_t)n * d, "out.codes");
  {
    KernelTimer t(ctx, "sq8_encode");
    k_sq8_encode<<<grid1(n * d), 256, 0, ctx->stream>>>(
        dx, n, d, per_dim, ds, dof, oc.ptr<int8_t>(), d);
    check_launch("sq8_encode");
  }
  oc.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_sq8_decode(vsk_ctx *ctx, const int8_t *codes, int64_t n, int32_t d,
                          int32_t per_dim, const float *scale, const float *offset,
                          float *out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no codes");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(codes && scale && offset && out, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  CallScope cs(ctx);
  const size_t cnt = per_dim ? d : 1;
  const int8_t *dc = static_cast<const int8_t *>(
      input_to_device(ctx, codes, (size_t)n * d, "sq8.dcodes"));
  const float *ds = static_cast<const float *>(
      input_to_device(ctx, scale, 4 * cnt, "sq8.scale"));
  const float *dof = static_cast<const float *>(
      input_to_device(ctx, offset, 4 * cnt, "sq8.offset"));
  OutputStage ox(ctx, out, sizeof(float) * (size_t)n * d, "out.decoded");
  {
    KernelTimer t(ctx, "sq8_dequantize");
    k_sq8_dequantize<<<grid1(n * d), 256, 0, ctx->stream>>>(dc, n, d, per_dim, ds, dof,
                                                           ox.ptr<float>());
    check_launch("sq8_dequantize");
  }
  ox.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_scalar_quantize_u8(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                                  int32_t bits, uint8_t *codes, float *scale, float *minv) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no vectors");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(x && codes, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(bits >= 1 && bits <= 8, VSK_ERR_INVALID_ARGUMENT, "bits must be in 1..8");
  VSK_REQUIRE(n <= 0x7FFFFFFFll * 4, VSK_ERR_INVALID_BUFFER_SIZE, "too many vectors");
  CallScope cs(ctx);
  const float *dx = static_cast<const float *>(
      input_to_device(ctx, x, sizeof(float) * (size_t)n * d, "squ8.x"));
  OutputStage oc(ctx, codes, (size_t)n * d, "squ8.codes");
  OutputStage os(ctx, scale, scale ? sizeof(float) * (size_t)n : 0, "squ8.scale");
  OutputStage om(ctx, minv, minv ? sizeof(float) * (size_t)n : 0, "squ8.min");
  {
    KernelTimer t(ctx, "scalar_quantize_u8", (double)n);
    k_scalar_quantize_u8<<<(unsigned)ceil_div(n, 4), 256, 0, ctx->stream>>>(
        dx, n, d, (float)((1 << bits) - 1), oc.ptr<uint8_t>(),
        scale ? os.ptr<float>() : nullptr, minv ? om.ptr<float>() : nullptr);
    check_launch("scalar_quantize_u8");
  }
  oc.copy_back();
  if (scale) os.copy_back();
  if (minv) om.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_sq8_upload(vsk_ctx *ctx, const int8_t *codes, int64_t n,
                          int32_t d, vsk_sq8 **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no codes");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(codes, VSK_ERR_INVALID_ARGUMENT, "codes is null");
  VSK_REQUIRE(n <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "a database holds at most 2^31-1 rows");
  std::unique_ptr<vsk_sq8> db(new vsk_sq8());
  db->n = n;
  db->d = d;
  db->ldc = (d + 31) & ~31;  // whole 32-byte MFMA k-steps
  CallScope cs(ctx);
  db->codes.reserve((size_t)n * db->ldc);
  if (db->ldc != d)
    fill_i32(ctx, db->codes.as<int32_t>(), n * db->ldc / 4, 0);
  copy_rows(ctx, db->codes.p, db->ldc, codes, d, d, n);
  // the filter scan's tiled copy (codes of up to 512 bytes, its range), in
  // the k-steps of the scan instance that takes this width (1, 2, 4 or 8;
  // the extra ones are zero)
  int32_t ks_n = 1;
  while (ks_n * 64 < db->ldc) ks_n <<= 1;
  if (ks_n <= 8) {
    const int64_t units = ceil_div(n, 16) * ks_n * 64;
    db->tiles.reserve((size_t)units * 16);
    db->tks = ks_n;
    k_sq8_tile<<<grid1(units), 256, 0, ctx->stream>>>(db->codes.as<int8_t>(), n, db->ldc, ks_n,
                                                      units, db->tiles.as<int8_t>());
    check_launch("sq8_tile");
  }
  cs.finish();
  // one layout in memory: every chunk a search scans starts on a 16-row
  // boundary (the chunk sizes are multiples of 16), so the tiled copy
  // serves every scan and the row-major codes go
  if (db->tks) db->codes.release();
  *out = db.release();
  VSK_API_END(ctx);
}

vsk_status vsk_sq8_free(vsk_ctx *ctx, vsk_sq8 *db) {
  if (ctx) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
  }
  delete db;
  return VSK_OK;
}

static vsk_status sq8_search_body(vsk_ctx *ctx, const vsk_sq8 *db,
                          const int8_t *qcodes, int64_t nq, int32_t k,
                          int32_t *out_score, int64_t *out_ids) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(db, VSK_ERR_INVALID_ARGUMENT, "db is null");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(qcodes && out_score && out_ids, VSK_ERR_INVALID_ARGUMENT,
              "null buffer");
  VSK_REQUIRE(k >= 1, VSK_ERR_INVALID_ARGUMENT, "k must be >= 1");
  VSK_REQUIRE(k <= VSK_MAX_K, VSK_ERR_INVALID_BUFFER_SIZE,
              "k exceeds VSK_MAX_K");
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "too many queries");
  CallScope cs(ctx);
  const int8_t *dq = codes_to_device(ctx, qcodes, nq, db->d, db->ldc, "sq8.q");
  uint64_t *best = static_cast<uint64_t *>(
      ctx->scratch_ptr("sq8.best", sizeof(uint64_t) * nq * k));
  const int64_t cap = default_cap(k);
  const int64_t qb = query_batch(ctx, nq, cap);
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    Sq8Args base{};
    base.X = db->codes.p ? db->codes.as<int8_t>() : nullptr;
    base.ldx = db->ldc;
    base.T = db->tks ? db->tiles.as<int8_t>() : nullptr;
    base.tks = db->tks;
    base.Q = dq + b0 * db->ldc;
    base.ldq = db->ldc;
    base.kbytes = db->ldc;
    base.nq = (int32_t)nb;
    ScanFn scan = [&](const ScanRequest &r) {
      Sq8Args a = base;
      a.r0 = r.r0;
      a.r1 = r.r1;
      a.thresh = r.thresh;
      a.active = r.active;
      a.cand = r.cand;
      a.cap = r.cap;
      a.counts = r.counts;
      launch_sq8(ctx, a, r.dense);
    };
    // chunks grow at most 8x, so the running threshold is tight before the
    // bulk of the rows is scanned (the filter epilogue is cheap only when
    // few scores pass)
    progressive_topk(ctx, nb, db->n, k, cap, scan, best + b0 * k, "sq8_select", 8);
  }
  OutputStage os(ctx, out_score, sizeof(int32_t) * nq * k, "out.score");
  OutputStage oi(ctx, out_ids, sizeof(int64_t) * nq * k, "out.ids");
  {
    KernelTimer t(ctx, "sq8_decode");
    k_sq8_decode<<<grid1(nq * k), 256, 0, ctx->stream>>>(
        best, nq * k, os.ptr<int32_t>(), oi.ptr<int64_t>());
    check_launch("sq8_decode");
  }
  os.copy_back();
  oi.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

// top-k overflow is checked at the call's end (topk_call)
vsk_status vsk_sq8_search(vsk_ctx *ctx, const vsk_sq8 *db,
                          const int8_t *qcodes, int64_t nq, int32_t k,
                          int32_t *out_score, int64_t *out_ids) {
  return topk_call(ctx, [&] { return sq8_search_body(ctx, db, qcodes, nq, k, out_score, out_ids); });
}

static vsk_status sq8_search_noalloc_body(vsk_ctx *ctx, const vsk_sq8 *db,
                                  const int8_t *qcodes, int64_t nq, int32_t k,
                                  int32_t *out_score, int64_t *out_ids) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(db, VSK_ERR_INVALID_ARGUMENT, "db is null");
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(qcodes && out_score && out_ids, VSK_ERR_INVALID_ARGUMENT,
              "null buffer");
  VSK_REQUIRE(k >= 1, VSK_ERR_INVALID_ARGUMENT, "k must be >= 1");
  VSK_REQUIRE(k <= VSK_MAX_K, VSK_ERR_INVALID_BUFFER_SIZE,
              "k exceeds VSK_MAX_K");
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "too many queries");
  // staging a host buffer would need device memory: only device buffers
  VSK_REQUIRE(is_device_ptr(qcodes) && is_device_ptr(out_score) && is_device_ptr(out_ids),
              VSK_ERR_INVALID_ARGUMENT,
              "vsk_sq8_search_noalloc takes device buffers only (qcodes, out_score, out_ids)");
  unsigned char *base = noalloc_scratch(ctx->device);
  const int64_t cap = std::min<int64_t>(default_cap(k), db->n);
  const bool pad = db->ldc != db->d;
  // scratch per query: best keys, threshold, candidates, count, overflow
  // flag, the padded query codes; fixed: overflow counter + slack
  const size_t fixed = 6 * 256 + 64 + 256;
  const size_t per_q = sizeof(uint64_t) * (size_t)k + 8 + sizeof(uint64_t) * (size_t)cap + 4 +
                       1 + (pad ? (size_t)db->ldc : 0);
  int64_t qb = (int64_t)((NOALLOC_SCRATCH_BYTES - fixed) / per_q);
  if (qb > nq) qb = nq;
  if (qb < 1)
    fail(VSK_ERR_INVALID_BUFFER_SIZE,
         "one query needs " + std::to_string(per_q + fixed) +
             " bytes of scratch, more than the no-allocation maximum of " +
             std::to_string(NOALLOC_SCRATCH_BYTES) + " bytes (k or d too large)");
  // carve the array for a batch of qb queries
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    unsigned char *p = base + off;
    off += region(bytes);
    return p;
  };
  uint64_t *best = reinterpret_cast<uint64_t *>(carve(sizeof(uint64_t) * (size_t)qb * k));
  TopkWorkspace ws;
  ws.thresh = reinterpret_cast<uint64_t *>(carve(8 * (size_t)qb));
  ws.cand = reinterpret_cast<uint64_t *>(carve(sizeof(uint64_t) * (size_t)qb * cap));
  ws.counts = reinterpret_cast<int32_t *>(carve(4 * (size_t)qb));
  ws.ovf_mask = carve((size_t)qb + 64);
  ws.ovf_count = reinterpret_cast<int32_t *>(carve(64));
  ws.seg_n = nullptr;  // the SQ8 scans append; no segmented lists
  int8_t *qpad = pad ? reinterpret_cast<int8_t *>(carve((size_t)qb * db->ldc)) : nullptr;
  if (off > NOALLOC_SCRATCH_BYTES)
    fail(VSK_ERR_INVALID_BUFFER_SIZE, "no-allocation scratch layout exceeds its maximum");

  CallScope cs(ctx);
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    const int8_t *dq = qcodes + b0 * db->d;
    if (pad) {
      // zero padding adds 0 to every dot product
      fill_i32(ctx, reinterpret_cast<int32_t *>(qpad), nb * db->ldc / 4, 0);
      VSK_HIP(hipMemcpy2DAsync(qpad, db->ldc, dq, db->d, db->d, (size_t)nb,
                               hipMemcpyDeviceToDevice, ctx->stream));
      dq = qpad;
    }
    Sq8Args a0{};
    a0.X = db->codes.p ? db->codes.as<int8_t>() : nullptr;
    a0.ldx = db->ldc;
    a0.T = db->tks ? db->tiles.as<int8_t>() : nullptr;
    a0.tks = db->tks;
    a0.Q = dq;
    a0.ldq = db->ldc;
    a0.kbytes = db->ldc;
    a0.nq = (int32_t)nb;
    ScanFn scan = [&](const ScanRequest &r) {
      Sq8Args a = a0;
      a.r0 = r.r0;
      a.r1 = r.r1;
      a.thresh = r.thresh;
      a.active = r.active;
      a.cand = r.cand;
      a.cap = r.cap;
      a.counts = r.counts;
      launch_sq8(ctx, a, r.dense);
    };
    progressive_topk(ctx, nb, db->n, k, cap, scan, best, "sq8_select", 8, &ws);
    KernelTimer t(ctx, "sq8_decode");
    k_sq8_decode<<<grid1(nb * k), 256, 0, ctx->stream>>>(best, nb * k, out_score + b0 * k,
                                                         out_ids + b0 * k);
    check_launch("sq8_decode");
  }
  cs.finish();
  VSK_API_END(ctx);
}

// top-k overflow is checked at the call's end (topk_call)
vsk_status vsk_sq8_search_noalloc(vsk_ctx *ctx, const vsk_sq8 *db,
                                  const int8_t *qcodes, int64_t nq, int32_t k,
                                  int32_t *out_score, int64_t *out_ids) {
  return topk_call(ctx, [&] { return sq8_search_noalloc_body(ctx, db, qcodes, nq, k, out_score, out_ids); });
}

}  // extern "C"
