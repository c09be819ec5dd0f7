// flat_bf16x3.hip -- the flat dot-product kernels (L2^2, L2, cosine,
// normalised cosine, dot) on gfx950's bf16 MFMA with fp32-level accuracy.
//
// Every fp32 operand v is split once into two bf16 numbers, hi = bf16(v)
// and lo = bf16(v - hi) (v - hi is exact in fp32), so v = hi + lo + e with
// |e| <= 2^-18 |v|.  A product is formed from three bf16 MFMA products,
//   q.x ~= qh.xh + qh.xl + ql.xh,
// accumulated in fp32; the dropped ql.xl term and the split errors are
// below 2^-16 of |q_i x_i| per term, far inside the 1e-4 relative bar of the
// fp32 path, while v_mfma_f32_16x16x32_bf16 runs 16x the fp32 MFMA rate.
//
// The rows are split once when the database is first searched (hi and lo
// planes, bf16, row stride ldb = roundup(d, 32)); queries per call.
//
// Tiling: a workgroup (4 waves) owns 128 queries and a slice of rows walked
// in 128-row tiles; each wave a 64-row x 64-query block of 4x4 16x16 tiles;
// two workgroups per CU.  Per 32-dim stage the workgroup stages hi and lo
// of its 128 rows and 128 queries in LDS (64-byte rows, 16-byte chunks
// XOR-swizzled so operand reads and staging writes are free of bank
// conflicts) through buffer loads whose range check zeroes rows past the
// slice.  LDS is double-buffered: while a stage is consumed by the MFMAs,
// the next one is written to the other buffer from registers and the one
// after is loaded from memory, with one barrier per stage.
#include "flat.hpp"

namespace vsk {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int XB_N = 128;   // rows per tile
constexpr int XB_Q = 128;   // queries per workgroup
constexpr int XB_K = 32;    // dims per LDS stage (one MFMA k-step)
constexpr int XR = 64;      // LDS row stride in bytes (chunks XOR-swizzled)
constexpr int XB_GQ = 16;   // query tiles per XCD group
constexpr int kBufFlags = 0x00020000;  // buffer descriptor word 3 (raw, dword data)

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

// hi = bf16(v) and (when lo is given) lo = bf16(v - hi) planes of an
// (n x ld) fp32 matrix, zero-padded to ldb columns, one wave per row.  With
// nhi: |hi| and |v - hi| of each row (v - hi is exact in fp32; squares
// summed in double, square root scaled up by 1e-12 and rounded up), and
// their maxima over the rows in maxbits[0..1] (float bits, atomic max).
__global__ __launch_bounds__(256) void k_split_rows(
    const float *x, int64_t n, int32_t d, int32_t ld, uint16_t *hi,
    uint16_t *lo, int32_t ldb, float *nhi, float *nres, uint32_t *maxbits) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  uint32_t mh = 0, mr = 0;
  for (int64_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < n;
       r += (int64_t)gridDim.x * 4) {
    double sh = 0.0, sr = 0.0;
    for (int32_t c = lane; c < ldb; c += 64) {
      const float v = c < d ? x[r * ld + c] : 0.f;
      const uint16_t h = bf16_rn(v);
      const float hv = __uint_as_float((uint32_t)h << 16);
      const float rv = v - hv;
      hi[r * ldb + c] = h;
      if (lo) lo[r * ldb + c] = bf16_rn(rv);
      sh += (double)hv * (double)hv;
      sr += (double)rv * (double)rv;
    }
    if (nhi || maxbits) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        sh += __shfl_xor(sh, o);
        sr += __shfl_xor(sr, o);
      }
      const float a = f_up(sqrt(sh) * (1.0 + 1e-12));
      const float b = f_up(sqrt(sr) * (1.0 + 1e-12));
      if (lane == 0 && nhi) {
        nhi[r] = a;
        nres[r] = b;
      }
      mh = __float_as_uint(a) > mh ? __float_as_uint(a) : mh;
      mr = __float_as_uint(b) > mr ? __float_as_uint(b) : mr;
    }
  }
  if (maxbits && lane == 0 && (mh | mr)) {
    atomicMax(&maxbits[0], mh);
    atomicMax(&maxbits[1], mr);
  }
}

template <int MODE, int METRIC>
__device__ inline void emit_x(const FlatArgs &a, int64_t qi, int64_t row,
                              float dist, uint64_t th) {
  if constexpr (MODE == MODE_MATRIX) {
    a.mat[qi * a.ldm + row] = METRIC == VSK_METRIC_L2 ? sqrtf(dist) : dist;
  } else {
    const uint64_t key = vsk_key(dist, (uint32_t)row);
    if constexpr (MODE == MODE_DENSE) {
      a.cand[qi * a.cap + (row - a.r0)] = key;
    } else if (key <= th) {
      int slot = atomicAdd(&a.counts[qi], 1);
      if (slot < a.cap) a.cand[qi * a.cap + slot] = key;
    }
  }
}

template <int METRIC>
__device__ inline float dist_from_dot(float dot, float qa, float xa) {
  if constexpr (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2)
    return fmaxf(qa + xa - 2.0f * dot, 0.0f);
  else if constexpr (METRIC == VSK_METRIC_COSINE)
    return 1.0f - dot / (qa * xa + 1e-8f);
  else if constexpr (METRIC == VSK_METRIC_COSINE_NORMALIZED)
    return 1.0f - dot;
  else
    return -dot;
}

// LDS byte offset of 16-byte chunk c (0..3) of tile row r: chunk positions
// are XOR-swizzled with (r >> 1) & 3.  Measured on gfx950: with this layout
// the MFMA operand reads (rows r..r+15 at one chunk) and the staging
// writes run without bank conflicts, while plain 64- or 80-byte rows take
// about four conflict cycles per ds_read_b128.
__device__ __forceinline__ int swz(int r, int c) {
  return r * XR + ((c ^ ((r >> 1) & 3)) << 4);
}

// The MFMAs of one 32-dim k-step from a staged LDS tile for a wave's
// 64-row x 64-query block: lane l holds row/query (l & 15), k = 8*(l >> 4)
// .. +7; for each 16-row block the three products are issued as three
// passes over its 4 query tiles, so two MFMAs that update one accumulator
// are 4 issues apart.
// PASSES == 1: the hi products only (the screen), over a 64-dim stage
// whose second 32 dims sit where the lo planes go; two_k false when the
// stage's second half lies past the padded dimension.
template <int PASSES>
__device__ __forceinline__ void x3_mfma(f4 (&acc)[4][4], const uint8_t *buf,
                                        int wr, int wq, int lane,
                                        bool two_k = true) {
  const uint8_t *xh_s = buf, *xl_s = buf + XB_N * XR;
  const uint8_t *qh_s = buf + 2 * XB_N * XR, *ql_s = buf + (2 * XB_N + XB_Q) * XR;
  const int cl = lane >> 4;
  bf8 bh[4], bl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int off = swz(wq * 64 + j * 16 + (lane & 15), cl);
    bh[j] = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(qh_s + off));
    if constexpr (PASSES == 3)
      bl[j] = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(ql_s + off));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int off = swz(wr * 64 + i * 16 + (lane & 15), cl);
    const bf8 ah = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(xh_s + off));
    if constexpr (PASSES == 3) {
      const bf8 al = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(xl_s + off));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl[j], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh[j], acc[i][j], 0, 0, 0);
  }
  if constexpr (PASSES == 1) {
    if (!two_k) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int off = swz(wq * 64 + j * 16 + (lane & 15), cl);
      bl[j] = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(ql_s + off));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int off = swz(wr * 64 + i * 16 + (lane & 15), cl);
      const bf8 ah = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(xl_s + off));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl[j], acc[i][j], 0, 0, 0);
    }
  }
}

template <int MODE, int METRIC, int PASSES>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_flat_bf16x3(FlatArgs a, SplitPtrs s) {
  // two stage buffers of {row hi, row lo, query hi, query lo}
  constexpr int STAGE_BYTES = 2 * (XB_N + XB_Q) * XR;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 1, wq = w >> 1;
  // XCD-aware placement: workgroup L runs on XCD L % 8; XCD x owns row
  // splits x, x+8, ... and walks them in groups of XB_GQ query tiles, so the
  // workgroups resident on one XCD share few row slices and few query tiles
  // in its L2
  const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
  const int sx = a.splits_per_xcd;
  const int grp = slot / (XB_GQ * sx), rem = slot - grp * (XB_GQ * sx);
  const int qtile = grp * XB_GQ + rem % XB_GQ;
  const int split = (rem / XB_GQ) * 8 + xcd;
  const int64_t q0 = (int64_t)qtile * XB_Q;
  if (q0 >= a.nq) return;
  const int64_t s0 = a.r0 + (int64_t)split * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;
  const int64_t qw = q0 + wq * 64 + (lane & 15);  // query of tile j: qw + 16 j
  // staging: 4 threads per 64-byte row segment, rows crow and crow + 64
  const int crow = tid >> 2, cch = tid & 3;
  // dims per LDS stage: 32 (three passes over hi and lo) or 64 (one pass,
  // the second 32 dims of hi in the lo slots)
  constexpr int SK = PASSES == 1 ? 2 * XB_K : XB_K;
  const int nst = (s.kb + SK - 1) / SK;
  const int32_t qbytes =
      (int32_t)(((a.nq - q0) < XB_Q ? (a.nq - q0) : XB_Q) * s.ldqb * 2);
  const __amdgpu_buffer_rsrc_t rqh =
      __builtin_amdgcn_make_buffer_rsrc((void *)(s.qh + q0 * s.ldqb), 0, qbytes, kBufFlags);
  const __amdgpu_buffer_rsrc_t rql =
      __builtin_amdgcn_make_buffer_rsrc((void *)(s.ql + q0 * s.ldqb), 0, qbytes, kBufFlags);
  const int32_t ox0 = crow * (int32_t)s.ldxb * 2 + cch * 16;
  const int32_t ox1 = ox0 + 64 * (int32_t)s.ldxb * 2;
  const int32_t oq0 = crow * (int32_t)s.ldqb * 2 + cch * 16;
  const int32_t oq1 = oq0 + 64 * (int32_t)s.ldqb * 2;
  const int w0 = swz(crow, cch), w1 = swz(64 + crow, cch);

  for (int64_t t0 = s0; t0 < s1; t0 += XB_N) {
    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    // buffer resources over this tile's rows: offsets past the valid range
    // read as zero, so partial tiles need no predicates
    const int32_t xbytes = (int32_t)((s1 - t0) * s.ldxb * 2);
    const __amdgpu_buffer_rsrc_t rxh =
        __builtin_amdgcn_make_buffer_rsrc((void *)(s.xh + t0 * s.ldxb), 0, xbytes, kBufFlags);
    const __amdgpu_buffer_rsrc_t rxl =
        __builtin_amdgcn_make_buffer_rsrc((void *)(s.xl + t0 * s.ldxb), 0, xbytes, kBufFlags);
#define X3_LD(RS, OFF, K) \
  __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(RS, OFF, (K) * 2, 0))
    // three register slots of staged loads (stage s in slot s mod 3): a
    // stage's loads are issued three stages before they are written to LDS,
    // which covers the latency of L2 misses
    uint4 axh0, axh1, axl0, axl1, aqh0, aqh1, aql0, aql1;
    uint4 bxh0, bxh1, bxl0, bxl1, bqh0, bqh1, bql0, bql1;
    uint4 cxh0, cxh1, cxl0, cxl1, cqh0, cqh1, cql0, cql1;
#define X3_LOAD(P, ST)                                                        \
  do {                                                                        \
    const int k_ = (ST) * SK;                                                 \
    P##xh0 = X3_LD(rxh, ox0, k_);                                             \
    P##xh1 = X3_LD(rxh, ox1, k_);                                             \
    P##qh0 = X3_LD(rqh, oq0, k_);                                             \
    P##qh1 = X3_LD(rqh, oq1, k_);                                             \
    if constexpr (PASSES == 3) {                                              \
      P##xl0 = X3_LD(rxl, ox0, k_);                                           \
      P##xl1 = X3_LD(rxl, ox1, k_);                                           \
      P##ql0 = X3_LD(rql, oq0, k_);                                           \
      P##ql1 = X3_LD(rql, oq1, k_);                                           \
    } else {                                                                  \
      P##xl0 = X3_LD(rxh, ox0, k_ + XB_K);                                    \
      P##xl1 = X3_LD(rxh, ox1, k_ + XB_K);                                    \
      P##ql0 = X3_LD(rqh, oq0, k_ + XB_K);                                    \
      P##ql1 = X3_LD(rqh, oq1, k_ + XB_K);                                    \
    }                                                                         \
  } while (0)
#define X3_STORE(P, BUF)                                                      \
  do {                                                                        \
    uint8_t *b_ = (BUF);                                                      \
    *reinterpret_cast<uint4 *>(b_ + w0) = P##xh0;                             \
    *reinterpret_cast<uint4 *>(b_ + w1) = P##xh1;                             \
    *reinterpret_cast<uint4 *>(b_ + 2 * XB_N * XR + w0) = P##qh0;             \
    *reinterpret_cast<uint4 *>(b_ + 2 * XB_N * XR + w1) = P##qh1;             \
    *reinterpret_cast<uint4 *>(b_ + XB_N * XR + w0) = P##xl0;                 \
    *reinterpret_cast<uint4 *>(b_ + XB_N * XR + w1) = P##xl1;                 \
    *reinterpret_cast<uint4 *>(b_ + (2 * XB_N + XB_Q) * XR + w0) = P##ql0;    \
    *reinterpret_cast<uint4 *>(b_ + (2 * XB_N + XB_Q) * XR + w1) = P##ql1;    \
  } while (0)
    // One step: stage S+1 (slot P) goes into the other LDS buffer while
    // stage S is consumed (every wave finished reading that buffer at the
    // barrier closing stage S-1), then slot P is refilled with stage S+4.
    // Steps past the last stage only keep the barrier count in step; loads
    // past the padded dimension read the next row or zeros (buffer range
    // check) and are never used.
#define X3_STEP(S, P)                                                         \
  do {                                                                        \
    const int s_ = (S);                                                       \
    if (s_ + 1 < nst) X3_STORE(P, lds + ((s_ + 1) & 1) * STAGE_BYTES);        \
    if (s_ < nst)                                                             \
      x3_mfma<PASSES>(acc, lds + (s_ & 1) * STAGE_BYTES, wr, wq, lane,        \
                      s_ * SK + XB_K < s.kb);                                 \
    X3_LOAD(P, s_ + 4);                                                       \
    __builtin_amdgcn_sched_barrier(0);                                        \
    __syncthreads();                                                          \
  } while (0)
    // prologue: stage 0 in buffer 0, stages 1, 2, 3 loading in slot order
    __syncthreads();  // the previous tile's last reads are done
    X3_LOAD(a, 0);
    X3_STORE(a, lds);
    __builtin_amdgcn_sched_barrier(0);
    X3_LOAD(b, 1);
    __builtin_amdgcn_sched_barrier(0);
    X3_LOAD(c, 2);
    __builtin_amdgcn_sched_barrier(0);
    X3_LOAD(a, 3);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    for (int st = 0; st < nst; st += 3) {
      X3_STEP(st, b);
      X3_STEP(st + 1, c);
      X3_STEP(st + 2, a);
    }
#undef X3_STEP
#undef X3_STORE
#undef X3_LOAD
#undef X3_LD
    // D[row = 4*(lane/16) + r][query = lane%16] of each 16x16 tile
    const bool full = t0 + XB_N <= s1;
    const int64_t rbase = t0 + wr * 64 + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t qi = qw + 16 * j;
      if (qi >= a.nq || (a.active && !a.active[qi])) continue;
      const uint64_t th = MODE == MODE_FILTER ? a.thresh[qi] : 0;
      const float qa = a.qaux ? a.qaux[qi] : 0.f;
      if constexpr (MODE == MODE_FILTER) {
        // fast path: the threshold as a distance; a key can only pass when
        // its distance is <= that (ties are settled by the exact key)
        const uint32_t th_hi = (uint32_t)(th >> 32);
        const float th_f = th_hi == 0xFFFFFFFFu ? __int_as_float(0x7f800000)
                                                 : vsk_ord2f(th_hi);
        bool any = false;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            // rows past the slice (zeros) read the last row's norm: they
            // can only send the tile to the exact test below
            const int64_t rr = rbase + i * 16 + r;
            const float xa = a.xaux ? a.xaux[rr < s1 ? rr : s1 - 1] : 0.f;
            any |= dist_from_dot<METRIC>(acc[i][j][r], qa, xa) <= th_f;
          }
        if (!any) continue;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t row = rbase + i * 16 + r;
          if (!full && row >= s1) continue;
          const float xa = a.xaux ? a.xaux[row] : 0.f;
          const float dist = dist_from_dot<METRIC>(acc[i][j][r], qa, xa);
          emit_x<MODE, METRIC>(a, qi, row, dist, th);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The screen's one-pass kernel: 256-row x 256-query workgroup tiles.
//
// A workgroup is 8 waves; wave w owns rows 64*(w & 3) .. +63 and queries
// 128*(w >> 2) .. +127 of the tile (4 x 8 tiles of 16x16, 128 fp32
// accumulators per lane).  Each LDS stage holds 64 dims (two MFMA k-steps)
// of the tile's 256 rows and 256 queries as 128-byte rows of eight 16-byte
// chunks, chunk c of row r stored at position c ^ ((r >> 1) & 7): the 16
// lanes of one ds_read_b128 phase (rows r..r+15, one chunk) and of one
// staging write (rows r, r+1, all chunks) then touch 16 distinct bank
// quads.  Two stage buffers (128 KB); the stage after next is loaded into
// registers while the current one is multiplied.  Filtered candidates go
// through per-wave LDS lists (24 KB).  Per MFMA this moves half
// the global bytes and two thirds of the LDS bytes of the 128 x 128 tile.
// Filtered candidates of one wave, staged in LDS (SC_CAP entries of key and
// query) and appended to the global per-query lists 64 entries per atomic
// round trip: an atomic that returns a value makes the wave wait for all
// its memory operations in flight, the prefetched stages included.  Calls
// are made in wave-uniform control flow, so the count n stays uniform.
constexpr int SC_CAP = 256;
struct WaveCands {
  uint64_t *key;
  int32_t *q;
  int32_t n;
};

__device__ __forceinline__ void wc_flush(WaveCands &wc, const FlatArgs &a,
                                         int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int32_t e = lane; e < wc.n; e += 64) {
    const int32_t q = wc.q[e];
    const int c = atomicAdd(&a.counts[q], 1);
    if (c < a.cap) a.cand[(int64_t)q * a.cap + c] = wc.key[e];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  wc.n = 0;
}

// append the passing lanes' keys in lane order; flush when fewer than 64
// slots would be left
__device__ __forceinline__ void wc_push(WaveCands &wc, const FlatArgs &a,
                                        bool pass, uint64_t key, int32_t q,
                                        int lane) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(pass);
  if (!m) return;
  if (pass) {
    const int32_t pos =
        wc.n + (int32_t)__builtin_amdgcn_mbcnt_hi(
                   (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    wc.key[pos] = key;
    wc.q[pos] = q;
  }
  wc.n += __builtin_popcountll(m);
  if (wc.n > SC_CAP - 64) wc_flush(wc, a, lane);
}

constexpr int XS_N = 256, XS_Q = 256, XS_K = 64, XS_R = 128;
constexpr int XS_STAGE = (XS_N + XS_Q) * XS_R;  // bytes per stage buffer
// two stage buffers, then the 8 waves' candidate lists (keys, queries)
constexpr int XS_LDS = 2 * XS_STAGE + 8 * SC_CAP * (8 + 4);

__device__ __forceinline__ int swz8(int r, int c) {
  return r * XS_R + ((c ^ ((r >> 1) & 7)) << 4);
}

template <int MODE, int METRIC>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_flat_screen(FlatArgs a, SplitPtrs s) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 3, wq = w >> 2;
  const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
  const int sx = a.splits_per_xcd;
  const int grp = slot / (XB_GQ * sx), rem = slot - grp * (XB_GQ * sx);
  const int qtile = grp * XB_GQ + rem % XB_GQ;
  const int split = (rem / XB_GQ) * 8 + xcd;
  const int64_t q0 = (int64_t)qtile * XS_Q;
  if (q0 >= a.nq) return;
  const int64_t s0 = a.r0 + (int64_t)split * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;
  const int64_t qw = q0 + wq * 128 + (lane & 15);  // query of tile j: qw + 16 j
  // staging: thread t moves chunk t & 7 of rows (t >> 3) + 64 u, u = 0..3
  const int crow = tid >> 3, cch = tid & 7;
  const int nst = (s.kb + XS_K - 1) / XS_K;
  const int32_t qbytes =
      (int32_t)(((a.nq - q0) < XS_Q ? (a.nq - q0) : XS_Q) * s.ldqb * 2);
  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc((void *)(s.qh + q0 * s.ldqb), 0, qbytes, kBufFlags);
  const int32_t ldx2 = (int32_t)s.ldxb * 2, ldq2 = (int32_t)s.ldqb * 2;
  const int32_t ox = crow * ldx2 + cch * 16, oq = crow * ldq2 + cch * 16;
  int wpos[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) wpos[u] = swz8(crow + 64 * u, cch);
  const int cl = lane >> 4;
  WaveCands wc;
  wc.key = reinterpret_cast<uint64_t *>(lds + 2 * XS_STAGE) + w * SC_CAP;
  wc.q = reinterpret_cast<int32_t *>(lds + 2 * XS_STAGE + 8 * SC_CAP * 8) + w * SC_CAP;
  wc.n = 0;

  for (int64_t t0 = s0; t0 < s1; t0 += XS_N) {
    f4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    const int32_t xbytes = (int32_t)((s1 - t0) * s.ldxb * 2);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)(s.xh + t0 * s.ldxb), 0, xbytes, kBufFlags);
    uint4 px[4], pq[4];
#define XS_LOAD(ST)                                                           \
  do {                                                                        \
    const int kb_ = (ST) * XS_K * 2;                                          \
    _Pragma("unroll") for (int u = 0; u < 4; ++u) {                           \
      px[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(\
                                            rx, ox + 64 * u * ldx2, kb_, 0)); \
      pq[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(\
                                            rq, oq + 64 * u * ldq2, kb_, 0)); \
    }                                                                         \
  } while (0)
#define XS_STORE(BUF)                                                         \
  do {                                                                        \
    uint8_t *b_ = (BUF);                                                      \
    _Pragma("unroll") for (int u = 0; u < 4; ++u) {                           \
      *reinterpret_cast<uint4 *>(b_ + wpos[u]) = px[u];                       \
      *reinterpret_cast<uint4 *>(b_ + XS_N * XS_R + wpos[u]) = pq[u];         \
    }                                                                         \
  } while (0)
    __syncthreads();  // the previous tile's last reads are done
    XS_LOAD(0);
    XS_STORE(lds);
    XS_LOAD(1);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
      const uint8_t *cur = lds + (st & 1) * XS_STAGE;
      // stage st+1 goes into the other buffer while this one is consumed
      // (every wave finished reading it at the barrier closing stage st-1);
      // loads past the padded dimension are never stored
      if (st + 1 < nst) {
        XS_STORE(lds + ((st + 1) & 1) * XS_STAGE);
        XS_LOAD(st + 2);
      }
      const uint8_t *xs_ = cur, *qs_ = cur + XS_N * XS_R;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        if (kk == 1 && st * XS_K + 32 >= s.kb) break;  // past the padding
        bf8 b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          b[j] = __builtin_bit_cast(
              bf8, *reinterpret_cast<const uint4 *>(
                       qs_ + swz8(wq * 128 + j * 16 + (lane & 15), kk * 4 + cl)));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bf8 av = __builtin_bit_cast(
              bf8, *reinterpret_cast<const uint4 *>(
                       xs_ + swz8(wr * 64 + i * 16 + (lane & 15), kk * 4 + cl)));
#pragma unroll
          for (int j = 0; j < 8; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b[j], acc[i][j], 0, 0, 0);
        }
      }
      __syncthreads();
    }
#undef XS_STORE
#undef XS_LOAD
    // D[row = 4*(lane/16) + r][query = lane%16] of each 16x16 tile
    const bool full = t0 + XS_N <= s1;
    const int64_t rbase = t0 + wr * 64 + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t qi = qw + 16 * j;
      const bool qok = qi < a.nq && (!a.active || a.active[qi]);
      const float qa = (qok && a.qaux) ? a.qaux[qi] : 0.f;
      if constexpr (MODE == MODE_DENSE) {
        if (!qok) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t row = rbase + i * 16 + r;
            if (!full && row >= s1) continue;
            const float xa = a.xaux ? a.xaux[row] : 0.f;
            a.cand[qi * a.cap + (row - a.r0)] =
                vsk_key(dist_from_dot<METRIC>(acc[i][j][r], qa, xa), (uint32_t)row);
          }
      } else {
        // a key can only pass when its distance is <= the threshold's (ties
        // are settled by the exact key): one compare per score, and the
        // exact test only in the (row block, r) steps where a lane passes
        const uint64_t th = qok ? a.thresh[qi] : 0;
        const uint32_t th_hi = (uint32_t)(th >> 32);
        const float th_f = th_hi == 0xFFFFFFFFu ? __int_as_float(0x7f800000)
                                                 : vsk_ord2f(th_hi);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t row = rbase + i * 16 + r;
            const bool in = qok && (full || row < s1);
            const float xa = (in && a.xaux) ? a.xaux[row] : 0.f;
            const float dist = dist_from_dot<METRIC>(acc[i][j][r], qa, xa);
            const bool maybe = in && dist <= th_f;
            if (!__builtin_amdgcn_ballot_w64(maybe)) continue;  // the common case
            const uint64_t key = vsk_key(dist, (uint32_t)row);
            wc_push(wc, a, maybe && key <= th, key, (int32_t)qi, lane);
          }
      }
    }
  }
  if constexpr (MODE == MODE_FILTER) {
    if (wc.n > 0) wc_flush(wc, a, lane);
  }
}

template <int METRIC>
static void launch_s(vsk_ctx *ctx, unsigned grid, const FlatArgs &a,
                     const SplitPtrs &s, int mode) {
  const size_t lds = XS_LDS;
  if (mode == MODE_DENSE)
    k_flat_screen<MODE_DENSE, METRIC><<<grid, 512, lds, ctx->stream>>>(a, s);
  else
    k_flat_screen<MODE_FILTER, METRIC><<<grid, 512, lds, ctx->stream>>>(a, s);
}

void launch_flat_screen(vsk_ctx *ctx, FlatArgs a, const SplitPtrs &s, int mode) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  if (mode == MODE_MATRIX) fail(VSK_ERR_UNSUPPORTED, "the screen has no matrix mode");
  static bool lds_set = false;
  if (!lds_set) {
    const int bytes = XS_LDS;
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_DENSE, VSK_METRIC_L2SQ>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_FILTER, VSK_METRIC_L2SQ>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_DENSE, VSK_METRIC_L2>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_FILTER, VSK_METRIC_L2>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_DENSE, VSK_METRIC_COSINE_NORMALIZED>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_FILTER, VSK_METRIC_COSINE_NORMALIZED>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_DENSE, VSK_METRIC_DOT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    VSK_HIP(hipFuncSetAttribute(
        reinterpret_cast<const void *>(k_flat_screen<MODE_FILTER, VSK_METRIC_DOT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    lds_set = true;
  }
  const int64_t qt = ceil_div(a.nq, XS_Q);
  // row splits: a multiple of 8 (one share per XCD), about 2048 workgroups
  // (one per CU at a time)
  int64_t splits = ceil_div(2048, qt);
  const int64_t max_splits = ceil_div(rows, XS_N);
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  a.rows_per_split = ceil_div(ceil_div(rows, splits), XS_N) * XS_N;
  splits = ceil_div(ceil_div(rows, a.rows_per_split), 8) * 8;
  a.splits_per_xcd = (int32_t)(splits / 8);
  const int64_t groups = ceil_div(qt, XB_GQ);
  const int64_t nblocks = 8 * a.splits_per_xcd * groups * XB_GQ;
  if (nblocks > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "grid too large");
  static const char *names[2] = {"flat_screen_dense", "flat_screen_filter"};
  KernelTimer t(ctx, names[mode], (double)a.nq * (double)rows);
  switch (a.metric) {
  case VSK_METRIC_L2SQ: launch_s<VSK_METRIC_L2SQ>(ctx, (unsigned)nblocks, a, s, mode); break;
  case VSK_METRIC_L2: launch_s<VSK_METRIC_L2>(ctx, (unsigned)nblocks, a, s, mode); break;
  case VSK_METRIC_COSINE_NORMALIZED:
    launch_s<VSK_METRIC_COSINE_NORMALIZED>(ctx, (unsigned)nblocks, a, s, mode);
    break;
  case VSK_METRIC_DOT: launch_s<VSK_METRIC_DOT>(ctx, (unsigned)nblocks, a, s, mode); break;
  default: fail(VSK_ERR_UNSUPPORTED, "metric without a one-pass screen");
  }
  check_launch(names[mode]);
}

template <int METRIC, int PASSES>
static void launch_x(vsk_ctx *ctx, unsigned grid, const FlatArgs &a,
                     const SplitPtrs &s, int mode) {
  if (mode == MODE_DENSE)
    k_flat_bf16x3<MODE_DENSE, METRIC, PASSES><<<grid, 256, 0, ctx->stream>>>(a, s);
  else if (mode == MODE_FILTER)
    k_flat_bf16x3<MODE_FILTER, METRIC, PASSES><<<grid, 256, 0, ctx->stream>>>(a, s);
  else if constexpr (PASSES == 3)
    k_flat_bf16x3<MODE_MATRIX, METRIC, 3><<<grid, 256, 0, ctx->stream>>>(a, s);
  else
    fail(VSK_ERR_UNSUPPORTED, "the one-pass screen has no matrix mode");
}

void split_bf16(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
                uint16_t *hi, uint16_t *lo, int32_t ldb, float *nhi,
                float *nres, uint32_t *maxbits) {
  if (n <= 0) return;
  int64_t g = ceil_div(n, 4);
  if (g > 16384) g = 16384;
  KernelTimer t(ctx, "split_bf16");
  k_split_rows<<<(unsigned)g, 256, 0, ctx->stream>>>(x, n, d, ld, hi, lo, ldb,
                                                     nhi, nres, maxbits);
  check_launch("split_bf16");
}

void launch_flat_bf16x3(vsk_ctx *ctx, FlatArgs a, const SplitPtrs &s, int mode,
                        int passes) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  const int64_t qt = ceil_div(a.nq, XB_Q);
  // row splits: a multiple of 8 (one share per XCD), enough workgroups to
  // fill the chip; trailing splits may be empty
  int64_t splits = ceil_div(4096, qt);
  const int64_t max_splits = ceil_div(rows, XB_N);
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  a.rows_per_split = ceil_div(ceil_div(rows, splits), XB_N) * XB_N;
  splits = ceil_div(ceil_div(rows, a.rows_per_split), 8) * 8;
  a.splits_per_xcd = (int32_t)(splits / 8);
  const int64_t groups = ceil_div(qt, XB_GQ);
  const int64_t nblocks = 8 * a.splits_per_xcd * groups * XB_GQ;
  if (nblocks > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "grid too large");
  const unsigned grid = (unsigned)nblocks;
  static const char *names[2][3] = {
      {"flat_bf16x3_dense", "flat_bf16x3_filter", "flat_bf16x3_matrix"},
      {"flat_screen_dense", "flat_screen_filter", "flat_screen_matrix"}};
  const char *name = names[passes == 1][mode];
  KernelTimer t(ctx, name, (double)a.nq * (double)rows);
  if (passes == 1) {
    switch (a.metric) {
    case VSK_METRIC_L2SQ: launch_x<VSK_METRIC_L2SQ, 1>(ctx, grid, a, s, mode); break;
    case VSK_METRIC_L2: launch_x<VSK_METRIC_L2, 1>(ctx, grid, a, s, mode); break;
    case VSK_METRIC_COSINE_NORMALIZED:
      launch_x<VSK_METRIC_COSINE_NORMALIZED, 1>(ctx, grid, a, s, mode);
      break;
    case VSK_METRIC_DOT: launch_x<VSK_METRIC_DOT, 1>(ctx, grid, a, s, mode); break;
    default: fail(VSK_ERR_UNSUPPORTED, "metric without a one-pass screen");
    }
  } else {
    switch (a.metric) {
    case VSK_METRIC_L2SQ: launch_x<VSK_METRIC_L2SQ, 3>(ctx, grid, a, s, mode); break;
    case VSK_METRIC_L2: launch_x<VSK_METRIC_L2, 3>(ctx, grid, a, s, mode); break;
    case VSK_METRIC_COSINE: launch_x<VSK_METRIC_COSINE, 3>(ctx, grid, a, s, mode); break;
    case VSK_METRIC_COSINE_NORMALIZED:
      launch_x<VSK_METRIC_COSINE_NORMALIZED, 3>(ctx, grid, a, s, mode);
      break;
    default: launch_x<VSK_METRIC_DOT, 3>(ctx, grid, a, s, mode); break;
    }
  }
  check_launch(name);
}

}  // namespace vsk
