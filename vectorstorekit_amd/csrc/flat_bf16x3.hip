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
#include <type_traits>

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
// s_waitcnt immediates (gfx9 layout: vmcnt [3:0], expcnt [6:4], lgkmcnt [11:8]):
// everything, and vector memory down to 8 outstanding
constexpr int kWaitAll = 0x0000;
constexpr int kWaitVm8 = 0x0F78;


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
// quads.  Two stage buffers (128 KB); the next stage is copied into the
// other one by buffer loads that write LDS directly while the current one
// is multiplied.  Filter mode appends each query's surviving keys to its
// slots of the candidate array; on L2 and L2^2 the blocks of scores that
// may pass wait in a per-wave LDS queue (17 KB) and are tested in batches.
// Per MFMA this moves half the global bytes and two thirds of the LDS bytes
// of the 128 x 128 tile.
constexpr int XS_N = 256, XS_Q = 256, XS_K = 64, XS_R = 128;
// query tiles per XCD group: the 32 workgroups resident on an XCD then hold
// 4 query tiles (1.5 MB of bf16 queries at d = 768) and 8 row slices
constexpr int XS_GQ = 4;
constexpr int XS_STAGE = (XS_N + XS_Q) * XS_R;  // bytes per stage buffer
// two stage buffers, then per query: slot limit, slot count, active flag,
// |q|^2 or |q| (metric), threshold as a distance, threshold key, index of
// the first reserved slot in the candidate array
constexpr int XS_LDS = 2 * XS_STAGE + 6 * XS_Q * 4 + 2 * XS_Q * 8;
// MODE_TOP2: a (smallest key, second smallest distance) slot per row wave
// and query
// and the row norms of four row tiles (copied with the tile's first stage)
constexpr int XS_LDS_TOP2 = XS_LDS + 4 * XS_Q * (8 + 4) + 4 * XS_N * 4;
static_assert(XS_LDS_TOP2 <= 160 * 1024, "LDS of one workgroup");
// filter mode on L2 and L2^2: the row norms of four row tiles in LDS too (a
// global load in the epilogue would wait for every stage copy in flight)
constexpr int XS_LDS_XA = XS_LDS + 4 * XS_N * 4;
// filter mode on L2 and L2^2: after the row norms, a queue per wave of up to
// XS_QCAP blocks (a lane's 16 scores of one query, 64 bytes) and a position
// word for each
constexpr int XS_QCAP = 32;
constexpr int XS_LDS_QUEUE = XS_LDS_XA + 8 * XS_QCAP * (64 + 4);
static_assert(XS_LDS_QUEUE <= 160 * 1024, "LDS of one workgroup");
template <int MODE, int METRIC>
constexpr bool xs_norms_in_lds() {
  return MODE == MODE_TOP2 ||
         (MODE == MODE_FILTER && (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2 ||
                                  METRIC == VSK_METRIC_COSINE));
}

__device__ __forceinline__ float top2_keydist(uint64_t k) {
  return k == VSK_KEY_NONE ? __int_as_float(0x7f800000) : vsk_ord2f((uint32_t)(k >> 32));
}
// (k, m2) := the smallest key and the second smallest distance of the union
// of two such pairs
__device__ __forceinline__ void top2_merge(uint64_t &k, float &m2, uint64_t ko, float mo) {
  const uint64_t hi = ko < k ? k : ko;
  k = ko < k ? ko : k;
  m2 = fminf(fminf(m2, mo), top2_keydist(hi));
}

// The lane index, computed where it is used and opaque to the compiler:
// kept live from a kernel's start under register pressure it is spilled,
// and its reload waits for every stage copy in flight.
__device__ __forceinline__ int lane_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

__device__ __forceinline__ int swz8(int r, int c) {
  return r * XS_R + ((c ^ ((r >> 1) & 7)) << 4);
}

// QR (planes of at most 128 dims, two stages a tile): the workgroup's
// queries are copied into LDS once and stay there (64 KB where the second
// stage buffer's query half was), and each stage copies only its 256 rows,
// into one of two 32 KB row buffers: half the copies per stage.
template <int MODE, int METRIC, bool QR = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_flat_screen(FlatArgs a, SplitPtrs s) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wr = w & 3, wq = w >> 2;
  const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
  const int sx = a.splits_per_xcd;
  // sx == 0: one split, workgroup L takes query tile L over every row (the
  // argmin with many queries: the rows stay in every XCD's L2, each query is
  // read once)
  // qx > 0: split-major, XCD x taking query tiles x*qx .. x*qx+qx-1 over
  // every split in turn
  const int qx = a.qtiles_per_xcd;
  const int grp = sx ? slot / (XS_GQ * sx) : 0, rem = sx ? slot - grp * (XS_GQ * sx) : 0;
  const int qtile = qx ? xcd * qx + slot % qx : (sx ? grp * XS_GQ + rem % XS_GQ : L);
  const int split = qx ? slot / qx : (sx ? (rem / XS_GQ) * 8 + xcd : 0);
  const int64_t q0 = (int64_t)qtile * XS_Q;
  if (q0 >= a.nq) return;
  const int64_t s0 = a.r0 + (int64_t)split * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;
  const int nst = (s.kb + XS_K - 1) / XS_K;
  const int32_t qbytes =
      (int32_t)(((a.nq - q0) < XS_Q ? (a.nq - q0) : XS_Q) * s.ldqb * 2);
  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc((void *)(s.qh + q0 * s.ldqb), 0, qbytes, kBufFlags);
  const int32_t ldx2 = (int32_t)s.ldxb * 2;  // the query plane has the same pitch
  const int cl = lane >> 4;
  // filter appends: the workgroup takes a.sub slots of each of its
  // queries' candidate lists up front (one device atomic per query, not one
  // per candidate: device-scope atomics are slow on the XCD-split L2) and
  // fills them through LDS counters; unused slots become NONE, which the
  // selection ignores, and a query whose slots overflow gets a count past
  // cap, so the selection re-scans it
  // The queries' flags, norms and thresholds are read once into LDS: in
  // the epilogue a global load would wait (in-order vector memory counter)
  // for every stage prefetch in flight, eight times per tile.
  // (The slot addresses are read from LDS where used: computed from the
  // query index, the compiler would hoist all eight out of the loops and
  // keep them live.)
  int32_t *s_lim = reinterpret_cast<int32_t *>(lds + 2 * XS_STAGE);
  int32_t *s_cnt = s_lim + XS_Q;
  int32_t *s_ok = s_cnt + XS_Q;
  float *s_qa = reinterpret_cast<float *>(s_ok + XS_Q);
  float *s_thf = s_qa + XS_Q;
  float *s_tdot = s_thf + XS_Q;
  uint64_t *s_th = reinterpret_cast<uint64_t *>(s_tdot + XS_Q);
  int64_t *s_pb = reinterpret_cast<int64_t *>(s_th + XS_Q);
  uint64_t *s_t1 = reinterpret_cast<uint64_t *>(lds + XS_LDS);  // [4][XS_Q]
  float *s_t2 = reinterpret_cast<float *>(s_t1 + 4 * XS_Q);
  // [4][XS_N]: |x|^2 of row tile t in slot t & 3
  float *s_xa = MODE == MODE_TOP2 ? s_t2 + 4 * XS_Q : reinterpret_cast<float *>(lds + XS_LDS);
  constexpr bool XA = xs_norms_in_lds<MODE, METRIC>();
  constexpr bool XS_SHIFT =
      MODE == MODE_FILTER && (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2);
  if constexpr (MODE == MODE_TOP2) {
    for (int i = tid; i < 4 * XS_Q; i += 512) {
      s_t1[i] = VSK_KEY_NONE;
      s_t2[i] = __int_as_float(0x7f800000);
    }
  }
  if (tid < XS_Q) {
    const int64_t q = q0 + tid;
    const bool ok = q < a.nq && (!a.active || a.active[q]);
    s_ok[tid] = ok ? 1 : 0;
    s_qa[tid] = (ok && a.qaux) ? a.qaux[q] : 0.f;
    if constexpr (MODE == MODE_FILTER) {
      const uint64_t th = ok ? a.thresh[q] : 0;
      const uint32_t th_hi = (uint32_t)(th >> 32);
      s_th[tid] = th;
      const float thf = !ok ? -__int_as_float(0x7f800000)
                            : (th_hi == 0xFFFFFFFFu ? __int_as_float(0x7f800000)
                                                    : vsk_ord2f(th_hi));
      s_thf[tid] = thf;
      // the same bound on the raw dot product (normalised cosine: a dot
      // below 1 - thf less a margin of the rounding of 1 - dot cannot pass;
      // dot: -dot <= thf exactly when dot >= -thf)
      if constexpr (METRIC == VSK_METRIC_COSINE_NORMALIZED) {
        const double t = 1.0 - (double)thf;
        const double m = t - 0x1p-22 * (fabs((double)thf) > 1.0 ? fabs((double)thf) : 1.0);
        float f = (float)m;
        if ((double)f > m) f = __uint_as_float(f > 0.f ? __float_as_uint(f) - 1u
                                               : (f < 0.f ? __float_as_uint(f) + 1u
                                                          : 0x80000001u));
        s_tdot[tid] = f;
      } else if constexpr (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2) {
        // L2: a score can pass the exact test (fma(-2, dot, qa + xa), its
        // max with 0, <= thf) only when dot - xa/2 >= (qa - thf)/2 less a
        // margin for the roundings of both forms.  A passing row has
        // (|x| - 1.01|q|)^2 <= 0.03 |q|^2 + thf + 1 (|dot| <= 1.01 |q||x| for
        // the bf16 products), which bounds its |x|^2 by xq2 below; every
        // rounding is then within 2^-22 (thf + qa + xq2 + 1), and the margin
        // takes four times that.
        const double qa = (double)s_qa[tid], t = (double)thf;
        float f;
        if (!ok) {
          f = __int_as_float(0x7f800000);
        } else if (th_hi == 0xFFFFFFFFu) {
          f = -__int_as_float(0x7f800000);
        } else {
          const double xq = 1.01 * sqrt(qa) + sqrt(0.03 * qa + fabs(t) + 1.0);
          const double m = 0.5 * (qa - t) - 0x1p-20 * (fabs(t) + qa + xq * xq + 1.0);
          f = (float)m;
          if ((double)f > m) f = __uint_as_float(f > 0.f ? __float_as_uint(f) - 1u
                                                 : (f < 0.f ? __float_as_uint(f) + 1u
                                                            : 0x80000001u));
        }
        s_tdot[tid] = f;
      } else if constexpr (METRIC == VSK_METRIC_COSINE) {
        // cosine (with the reference's epsilon): a <= thf is
        // dot >= (1 - thf) den, den = |q||x| + 1e-8 > 0; the bound t2 on
        // dot / den sits 2^-20 (1 + |1 - thf|) below 1 - thf, more than
        // the roundings of either form, so no score whose exact test below
        // passes is under it
        float f;
        if (!ok) {
          f = __int_as_float(0x7f800000);
        } else if (th_hi == 0xFFFFFFFFu) {
          f = -__int_as_float(0x7f800000);
        } else {
          const double t = 1.0 - (double)thf;
          const double m = t - 0x1p-20 * (1.0 + fabs(t));
          f = (float)m;
          if ((double)f > m) f = __uint_as_float(f > 0.f ? __float_as_uint(f) - 1u
                                                 : (f < 0.f ? __float_as_uint(f) + 1u
                                                            : 0x80000001u));
        }
        s_tdot[tid] = f;
      } else {
        s_tdot[tid] = -thf;
      }
      // segmented: this split's fixed segment; else slots taken from the
      // query's append counter
      const int64_t base = a.seg_n ? (int64_t)split * a.sub
                                   : (ok ? atomicAdd(&a.counts[q], a.sub) : a.cap);
      const int64_t room = a.cap - base;
      s_lim[tid] = (int32_t)(room < a.sub ? (room > 0 ? room : 0) : a.sub);
      s_pb[tid] = q * a.cap + base;
      s_cnt[tid] = 0;
    }
  }
  __syncthreads();

  // Staging: the stages of all tiles of the slice form one sequence, and
  // stage g goes into buffer g & 1 by buffer loads that write LDS directly
  // (no registers): wave w moves the 8-row units 4w+u (u = 0..3) of the row
  // half and of the query half, lane l the 16-byte chunk that belongs at
  // position (row 8U + l/8, slot l%8) of the swizzled layout.  The MFMA
  // operands of the next half-stage are read one step ahead into the second
  // register set, so the MFMAs never wait on LDS, and the next tile's first
  // stages are in flight during this tile's epilogue.
  // Wait rules: a wave waits for its own copies (vector memory counter)
  // and for its own operand reads (LDS counter), then the barrier makes
  // every wave's copies visible and ends every wave's reads of the buffer
  // the next copy overwrites.
  // (units 4w+u and 4w+u+2 differ by 16 rows, the same swizzle: one lane
  // offset per parity of u, the row step in the scalar offset)
  int32_t voff[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int r = 8 * (4 * w + u) + (lane >> 3);
    voff[u] = r * ldx2 + (((lane & 7) ^ ((r >> 1) & 7)) << 4);
  }
  int dst = 0;          // next stage to copy: stage dst of the tile at dt0
  int64_t dt0 = s0;     // (past the slice: zero-length rows, nothing read)
  int dtile = 0;        // index of that tile in the slice
  int dbuf = 0;
  auto copy_next = [&]() {
    const int64_t left = s1 - dt0;
    const int64_t rows = left < XS_N ? (left > 0 ? left : 0) : XS_N;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(s.xh + dt0 * s.ldxb), 0, (int32_t)(rows * ldx2), kBufFlags);
    if constexpr (XA) {
      if (dst == 0 && w < 4) {
        // the tile's row norms, 64 per wave (rows past the slice read 0)
        const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(a.xaux + dt0), 0, (int32_t)(rows * 4), kBufFlags);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rn, (__attribute__((address_space(3))) void *)(s_xa + (dtile & 3) * XS_N + 64 * w),
            4, lane * 4, w * 256, 0, 0);
      }
    }
    const int32_t kofs = dst * XS_K * 2;
    // waves 0-3 issue the stage's 64 copies (QR: 32), 16 (8) each: their
    // own units and those of wave w + 4, 128 rows further (the same
    // swizzle); the other four waves only multiply (fewer waves issuing
    // memory instructions measured faster)
    if (w < 4) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint8_t *bx = lds + dbuf * (QR ? XS_N * XS_R : XS_STAGE) + 4 * (w + 4 * h) * 1024;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int32_t so = kofs + (u >> 1) * 16 * ldx2 + h * 128 * ldx2;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rx, (__attribute__((address_space(3))) void *)(bx + u * 1024), 16, voff[u & 1], so,
              0, 0);
          if constexpr (!QR)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rq, (__attribute__((address_space(3))) void *)(bx + XS_N * XS_R + u * 1024), 16,
                voff[u & 1], so, 0, 0);
        }
      }
    }
    dbuf ^= 1;
    if (++dst == nst) {
      dst = 0;
      dt0 += XS_N;
      ++dtile;
    }
  };
  // the rows and the queries of stage g
  auto rows_of = [&](int gg) -> const uint8_t * {
    return lds + (gg & 1) * (QR ? XS_N * XS_R : XS_STAGE);
  };
  auto queries_of = [&](int gg) -> const uint8_t * {
    if constexpr (QR)
      return lds + 2 * XS_N * XS_R + (nst == 2 ? (gg & 1) : 0) * XS_Q * XS_R;
    else
      return lds + (gg & 1) * XS_STAGE + XS_N * XS_R;
  };
  // operands: two sets, this step's and the next one's (read one step ahead)
  bf8 ra[2][4], rb[2][8];
  auto read_ops = [&](int gg, int kk, int n) {
    const uint8_t *bq = queries_of(gg), *bx = rows_of(gg);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      rb[n][j] = __builtin_bit_cast(
          bf8, *reinterpret_cast<const uint4 *>(
                   bq + swz8(wq * 128 + j * 16 + (lane & 15), kk * 4 + cl)));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[n][i] = __builtin_bit_cast(
          bf8, *reinterpret_cast<const uint4 *>(
                   bx + swz8(wr * 64 + i * 16 + (lane & 15), kk * 4 + cl)));
  };
  if constexpr (QR) {
    // the queries' stages, once (in the layout of a stage's query half)
    if (w < 4) {
      for (int hh = 0; hh < nst; ++hh) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint8_t *bq = lds + 2 * XS_N * XS_R + hh * XS_Q * XS_R + 4 * (w + 4 * h) * 1024;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int32_t so = hh * XS_K * 2 + (u >> 1) * 16 * ldx2 + h * 128 * ldx2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rq, (__attribute__((address_space(3))) void *)(bq + u * 1024), 16, voff[u & 1],
                so, 0, 0);
          }
        }
      }
    }
  }
  copy_next();
  copy_next();
  __builtin_amdgcn_s_waitcnt(kWaitVm8);  // this wave's copies of stage 0
  __builtin_amdgcn_s_barrier();
  // L2 filter: a lane whose block of 16 scores may pass (its largest
  // score clears the query's bound) puts the block in its wave's queue,
  // with the block's position (tile, query column, lane).  The queue is
  // drained, one block a lane, when full and at the end of the slice: the
  // per-score test and the exact keys then run once for up to XS_QCAP
  // blocks instead of once per flagged block.  (Rows per split stay below
  // 2^31, so the tile index fits in 23 bits.)
  int qn = 0;  // blocks in the queue (wave-uniform)
  float *q_val = reinterpret_cast<float *>(lds + XS_LDS_XA) + w * XS_QCAP * 16;
  int32_t *q_pos = reinterpret_cast<int32_t *>(lds + XS_LDS_XA + 8 * XS_QCAP * 64) + w * XS_QCAP;
  auto drain = [&]() {
    const int ln = lane_here();
    if (ln < qn) {
      const uint32_t pw = (uint32_t)q_pos[ln];
      const int jj = (int)((pw >> 6) & 7u), sl = (int)(pw & 63u);
      const int lq = wq * 128 + 16 * jj + (sl & 15);
      const f4 *src = reinterpret_cast<const f4 *>(q_val + ln * 16);
      const f4 v0 = src[0], v1 = src[1], v2 = src[2], v3 = src[3];
      const bool ok = s_ok[lq] != 0;
      const float td = s_tdot[lq];
      const float qa = a.qaux ? s_qa[lq] : 0.f;
      const uint64_t th = s_th[lq];
      uint32_t m = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        m |= (v0[r] < td) ? 0u : (1u << r);
        m |= (v1[r] < td) ? 0u : (1u << (4 + r));
        m |= (v2[r] < td) ? 0u : (1u << (8 + r));
        m |= (v3[r] < td) ? 0u : (1u << (12 + r));
      }
      if (!ok) m = 0;
      const int64_t rb = s0 + (int64_t)(pw >> 9) * XS_N + wr * 64 + 4 * (sl >> 4);
      while (m) {
        const int b = __builtin_ctz(m);
        m &= m - 1;
        const int64_t row = rb + 16 * (b >> 2) + (b & 3);
        if (row >= s1) continue;  // past the slice
        // |q|^2 - 2 (dot - |x|^2/2), one rounding
        const float dist = fmaxf(__builtin_fmaf(-2.0f, q_val[ln * 16 + b], qa), 0.0f);
        const uint64_t key = vsk_key(dist, (uint32_t)row);
        if (key <= th) {
          const int pos = atomicAdd(&s_cnt[lq], 1);
          if (pos < s_lim[lq]) a.cand[s_pb[lq] + pos] = key;
        }
      }
    }
    qn = 0;
  };
  int g = 0;  // stage of the sequence being multiplied
  int tcur = 0;  // index of the tile being multiplied
  for (int64_t t0 = s0; t0 < s1; t0 += XS_N, ++tcur) {
    // the tile's first operands are read here rather than before the
    // previous epilogue, which then has the registers to itself
    read_ops(g, 0, 0);
    // the accumulators start at zero, or in filter mode on L2 and L2^2 at
    // -|x|^2/2 of the lane's rows (the tile's norms reached LDS with its
    // first stage): acc is then dot - |x|^2/2, the quantity the filter's
    // bound is on
    f4 acc[4][8];
    const int xl = XS_SHIFT ? lane_here() : lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f4 init = f4{0.f, 0.f, 0.f, 0.f};
      if constexpr (XS_SHIFT)
        init = *reinterpret_cast<const f4 *>(s_xa + (tcur & 3) * XS_N + wr * 64 +
                                             4 * (xl >> 4) + 16 * i) *
               -0.5f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = init;
    }
#define XS_MMA(N)                                                               \
  do {                                                                          \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                             \
      _Pragma("unroll") for (int j = 0; j < 8; ++j) acc[i][j] =                 \
          __builtin_amdgcn_mfma_f32_16x16x32_bf16(ra[N][i], rb[N][j], acc[i][j], 0, 0, 0); \
    }                                                                           \
  } while (0)
    // (the operand reads are spread over the MFMAs: as a block, the eight
    // waves' reads fill the LDS queue and hold up the MFMA issue)
    for (int st = 0; st < nst; ++st, ++g) {
      read_ops(g, 1, 1);
      XS_MMA(0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(kWaitAll);  // own copies of stage g+1, own reads of cur
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // stage g+1 (at a tile's last stage the next tile's first one, read
      // again at its start: unconditional, so the reads can interleave)
      read_ops(g + 1, 0, 0);
      // stage g+2 into cur
      copy_next();
      XS_MMA(1);
      __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);  // the copies first
#pragma unroll
      for (int t = 0; t < 12; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#undef XS_MMA
    // D[row = 4*(lane/16) + r][query = lane%16] of each 16x16 tile
    const bool full = t0 + XS_N <= s1;
    const int64_t rbase = t0 + wr * 64 + 4 * (lane >> 4);
    // this lane's query state: query j at element 16 j (a constant offset)
    const int lq0 = wq * 128 + (lane & 15);
    const int32_t *l_ok = s_ok + lq0, *l_lim = s_lim + lq0;
    int32_t *l_cnt = s_cnt + lq0;
    const float *l_qa = s_qa + lq0, *l_thf = s_thf + lq0, *l_tdot = s_tdot + lq0;
    // rows of this lane inside the slice: bit 4i+r for row rbase + 16i + r
    uint32_t vmask = 0xFFFFu;
    if (!full) {
      vmask = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (rbase + i * 16 + r < s1) vmask |= 1u << (4 * i + r);
    }
    const uint64_t *l_th = s_th + lq0;
    const int64_t *l_pb = s_pb + lq0;
    uint64_t *l_t1 = s_t1 + wr * XS_Q + lq0;
    float *l_t2 = s_t2 + wr * XS_Q + lq0;
    // L2 filter: the eight query columns' bounds read at once (read one at
    // a time, each test waits for its read)
    float tdv[8];
    if constexpr (MODE == MODE_FILTER && XS_SHIFT) {
#pragma unroll
      for (int j = 0; j < 8; ++j) tdv[j] = l_tdot[16 * j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t qi = q0 + lq0 + 16 * j;
      const float qa = a.qaux ? l_qa[16 * j] : 0.f;
      if constexpr (MODE == MODE_DENSE) {
        if (!l_ok[16 * j]) continue;
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
      } else if constexpr (MODE == MODE_TOP2) {
        // The screened distance less the query's constant |q|^2,
        // t = |x|^2 - 2 q.x (one FMA), with this lane's slot (lane group cl,
        // score e) in its 6 low mantissa bits: min and median-of-three then
        // keep the two smallest and the first one's position.  The packing
        // moves t by under 64 ulp, within 2^-17 (|q| + |x|)^2, which the
        // argmin's bound adds; equal screened distances stay within that of
        // each other, so the bound test still refuses to decide them.
        const float inf = __int_as_float(0x7f800000);
        float m1 = inf, m2 = inf;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int e = 4 * i + r;
            const float xa = s_xa[(tcur & 3) * XS_N + wr * 64 + 4 * cl + 16 * i + r];
            float t = __builtin_fmaf(-2.0f, acc[i][j][r], xa);
            t = __uint_as_float((__float_as_uint(t) & ~63u) | (uint32_t)e);
            if (!full) t = ((vmask >> e) & 1u) ? t : inf;
            m2 = __builtin_amdgcn_fmed3f(m1, m2, t);
            m1 = fminf(m1, t);
          }
        // the lane group in bits 4-5 (all 16 scores share it)
        if (m1 < inf) m1 = __uint_as_float(__float_as_uint(m1) | (uint32_t)(cl << 4));
        // the four lane groups hold other rows of the same query
#pragma unroll
        for (int mk = 16; mk <= 32; mk <<= 1) {
          const float o1 = __shfl_xor(m1, mk), o2 = __shfl_xor(m2, mk);
          m2 = fminf(fmaxf(m1, o1), fminf(m2, o2));
          m1 = fminf(m1, o1);
        }
        if (cl == 0 && l_ok[16 * j]) {
          uint64_t k1 = VSK_KEY_NONE;
          if (m1 < inf) {
            const uint32_t pos = __float_as_uint(m1) & 63u;
            const int64_t row = t0 + wr * 64 + 4 * (pos >> 4) + 16 * ((pos & 15) >> 2) + (pos & 3);
            k1 = vsk_key(fmaxf(qa + m1, 0.f), (uint32_t)row);
          }
          const float a2 = m2 < inf ? fmaxf(qa + m2, 0.f) : inf;
          // this wave's own slot
          uint64_t k = l_t1[16 * j];
          float t2 = l_t2[16 * j];
          top2_merge(k, t2, k1, a2);
          l_t1[16 * j] = k;
          l_t2[16 * j] = t2;
        }
      } else {
        // a key can only pass when its distance is <= the threshold's (ties
        // are settled by the exact key): one compare per score, and the
        // exact test only in the (row block, r) steps where a lane passes
        // fast test, one compare per score: bit 4i+r of m for a score that
        // may pass (NaN included); rows past the slice masked off
        if constexpr (XS_SHIFT) {
          // acc holds dot - |x|^2/2, the quantity the bound is on; the
          // block's largest score first (a NaN score is dropped by the max:
          // it needs a non-finite input, whose bound is not finite, so such
          // a query fails the screen's check and is redone exactly)
          const float tdot = tdv[j];
          float mx = acc[0][j][0];
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, acc[i][j][r]);
          uint64_t bal = __builtin_amdgcn_ballot_w64(!(mx < tdot));
          while (bal) {  // (the common case skips it)
            if (qn == XS_QCAP) drain();
            const uint32_t pos = __builtin_amdgcn_mbcnt_hi(
                (uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            const int ln = lane_here();
            const bool mine = ((bal >> ln) & 1u) && (int)pos < XS_QCAP - qn;
            if (mine) {
              f4 *dst = reinterpret_cast<f4 *>(q_val + (qn + (int)pos) * 16);
#pragma unroll
              for (int i = 0; i < 4; ++i) dst[i] = acc[i][j];
              q_pos[qn + (int)pos] =
                  (int32_t)(((uint32_t)tcur << 9) | ((uint32_t)j << 6) | (uint32_t)ln);
            }
            const uint64_t took = __builtin_amdgcn_ballot_w64(mine);
            qn = __builtin_amdgcn_readfirstlane(qn + __builtin_popcountll(took));
            bal &= ~took;
          }
          continue;
        }
        uint32_t m = 0;
        if constexpr (METRIC == VSK_METRIC_COSINE_NORMALIZED || METRIC == VSK_METRIC_DOT) {
          const float tdot = l_tdot[16 * j];
          // the block's largest dot first: when it is below the bound in
          // every lane, no score of the block can pass (one compare and a
          // ballot instead of sixteen).  A NaN score is dropped by the max;
          // it needs a non-finite input, whose bound is not finite, so such
          // a query fails the screen's check and is redone exactly.
          float mx = acc[0][j][0];
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, acc[i][j][r]);
          if (!__builtin_amdgcn_ballot_w64(!(mx < tdot))) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              m |= (acc[i][j][r] < tdot) ? 0u : (1u << (4 * i + r));
        } else if constexpr (METRIC == VSK_METRIC_COSINE) {
          // dot - t2 (|q||x| + 1e-8) >= 0 with the row norms from LDS; the
          // block's largest first (a NaN score is dropped by the max: it
          // needs a non-finite input, whose query fails the screen's check)
          const float t2 = l_tdot[16 * j];
          float mx = -__int_as_float(0x7f800000);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float xn = s_xa[(tcur & 3) * XS_N + wr * 64 + 4 * cl + 16 * i + r];
              mx = fmaxf(mx, __builtin_fmaf(-t2, __builtin_fmaf(qa, xn, 1e-8f), acc[i][j][r]));
            }
          if (!__builtin_amdgcn_ballot_w64(!(mx < 0.f))) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float xn = s_xa[(tcur & 3) * XS_N + wr * 64 + 4 * cl + 16 * i + r];
              m |= (__builtin_fmaf(-t2, __builtin_fmaf(qa, xn, 1e-8f), acc[i][j][r]) < 0.f)
                       ? 0u
                       : (1u << (4 * i + r));
            }
        } else {
          const float th_f = l_thf[16 * j];
          // the block's largest dot - |x|^2/2 first, against the query's
          // bound on it (with its margin, no score whose exact test below
          // passes is under it): when it is below in every lane, no score of
          // the block can pass.  A NaN score is dropped by the max; it needs
          // a non-finite input, whose bound is not finite, so such a query
          // fails the screen's check and is redone exactly.
          const float tdot = l_tdot[16 * j];
          float mx = -__int_as_float(0x7f800000);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              mx = fmaxf(mx, acc[i][j][r] -
                                 0.5f * s_xa[(tcur & 3) * XS_N + wr * 64 + 4 * cl + 16 * i + r]);
          if (!__builtin_amdgcn_ballot_w64(!(mx < tdot))) continue;
          // the same bound per score: a superset of the scores whose exact
          // test below passes (the exact key test then decides each one)
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              // (rows past the slice read 0 and are masked off below)
              const float xa = s_xa[(tcur & 3) * XS_N + wr * 64 + 4 * cl + 16 * i + r];
              m |= (acc[i][j][r] - 0.5f * xa < tdot) ? 0u : (1u << (4 * i + r));
            }
          (void)th_f;
        }
        m &= vmask;
        if (!__builtin_amdgcn_ballot_w64(m != 0)) continue;  // the common case
        if (m && l_ok[16 * j]) {
          // the few candidates of this lane: exact key test
          const uint64_t th = l_th[16 * j];
          const int32_t lim = l_lim[16 * j];
          const int64_t pb = l_pb[16 * j];
          // this query's 16 scores of the lane as named values behind an
          // empty asm: a select between two loads of one array would be
          // folded into one dynamically indexed load, which sends the array
          // (and with it the accumulators) to scratch memory
          float c0 = acc[0][j][0], c1 = acc[0][j][1], c2 = acc[0][j][2], c3 = acc[0][j][3];
          float c4 = acc[1][j][0], c5 = acc[1][j][1], c6 = acc[1][j][2], c7 = acc[1][j][3];
          float c8 = acc[2][j][0], c9 = acc[2][j][1], c10 = acc[2][j][2], c11 = acc[2][j][3];
          float c12 = acc[3][j][0], c13 = acc[3][j][1], c14 = acc[3][j][2], c15 = acc[3][j][3];
          asm volatile("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3), "+v"(c4), "+v"(c5),
                       "+v"(c6), "+v"(c7));
          asm volatile("" : "+v"(c8), "+v"(c9), "+v"(c10), "+v"(c11), "+v"(c12), "+v"(c13),
                       "+v"(c14), "+v"(c15));
          while (m) {
            const int b = __builtin_ctz(m);
            m &= m - 1;
            const bool b0 = b & 1, b1 = b & 2, b2 = b & 4;
            const float s0 = b0 ? c1 : c0, s1 = b0 ? c3 : c2, s2 = b0 ? c5 : c4,
                        s3 = b0 ? c7 : c6, s4 = b0 ? c9 : c8, s5 = b0 ? c11 : c10,
                        s6 = b0 ? c13 : c12, s7 = b0 ? c15 : c14;
            const float u0 = b1 ? s1 : s0, u1 = b1 ? s3 : s2, u2 = b1 ? s5 : s4,
                        u3 = b1 ? s7 : s6;
            const float w0 = b2 ? u1 : u0, w1 = b2 ? u3 : u2;
            const float dot = (b & 8) ? w1 : w0;
            const int64_t row = rbase + 16 * (b >> 2) + (b & 3);
            float dist;
            if constexpr (XS_SHIFT) {
              // |q|^2 - 2 (dot - |x|^2/2), one rounding
              dist = fmaxf(__builtin_fmaf(-2.0f, dot, qa), 0.0f);
            } else {
              float xa = 0.f;
              if constexpr (XA)
                xa = s_xa[(tcur & 3) * XS_N + wr * 64 + 4 * cl + 16 * (b >> 2) + (b & 3)];
              else if (a.xaux)
                xa = a.xaux[row];
              dist = dist_from_dot<METRIC>(dot, qa, xa);
            }
            const uint64_t key = vsk_key(dist, (uint32_t)row);
            if (key <= th) {
              const int pos = atomicAdd(&l_cnt[16 * j], 1);
              if (pos < lim) a.cand[pb + pos] = key;
            }
          }
        }
      }
    }
  }
  // the copies issued past the slice end land before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  if constexpr (MODE == MODE_FILTER && XS_SHIFT) {
    if (qn) drain();
  }
  if constexpr (MODE == MODE_TOP2) {
    __syncthreads();
    if (tid < XS_Q && s_ok[tid]) {
      uint64_t k = s_t1[tid];
      float t2 = s_t2[tid];
#pragma unroll
      for (int u = 1; u < 4; ++u) top2_merge(k, t2, s_t1[u * XS_Q + tid], s_t2[u * XS_Q + tid]);
      a.cand[(q0 + tid) * a.ldm + split] = k;
      a.mat[(q0 + tid) * a.ldm + split] = t2;
    }
  }
  if constexpr (MODE == MODE_FILTER) {
    __syncthreads();
    if (tid < XS_Q && s_ok[tid]) {
      const int32_t n = s_cnt[tid];
      const int32_t lim = s_lim[tid];
      // past the slots: the query re-scans the chunk
      if (n > lim) atomicAdd(&a.counts[q0 + tid], (int32_t)a.cap + 1);
      if (a.seg_n) {
        a.seg_n[(q0 + tid) * (int64_t)(8 * a.splits_per_xcd) + split] = n < lim ? n : lim;
      } else if (n <= lim) {
        const int64_t pb = s_pb[tid];
        for (int32_t i = n; i < lim; ++i) a.cand[pb + i] = VSK_KEY_NONE;
      }
    }
  }
}

// dynamic LDS of each mode: the stage buffers and the queries' state, then
// the row norms (filter mode on L2, L2^2 and cosine) and the candidate
// queue (filter mode on L2 and L2^2), or the argmin's slots
template <int MODE, int METRIC>
constexpr int xs_lds_bytes() {
  if constexpr (MODE == MODE_TOP2) return XS_LDS_TOP2;
  if constexpr (MODE == MODE_FILTER && (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2))
    return XS_LDS_QUEUE;
  if constexpr (xs_norms_in_lds<MODE, METRIC>()) return XS_LDS_XA;
  return XS_LDS;
}

template <int MODE, int METRIC, bool QR>
static void set_lds() {
  VSK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(k_flat_screen<MODE, METRIC, QR>),
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              xs_lds_bytes<MODE, METRIC>()));
}

template <int METRIC, bool QR>
static void set_lds_metric() {
  set_lds<MODE_DENSE, METRIC, QR>();
  set_lds<MODE_FILTER, METRIC, QR>();
  if constexpr (METRIC == VSK_METRIC_L2SQ) set_lds<MODE_TOP2, METRIC, QR>();
}

template <int METRIC, bool QR>
static void launch_s(vsk_ctx *ctx, unsigned grid, const FlatArgs &a,
                     const SplitPtrs &s, int mode) {
  if constexpr (METRIC == VSK_METRIC_L2SQ) {
    if (mode == MODE_TOP2) {
      k_flat_screen<MODE_TOP2, METRIC, QR>
          <<<grid, 512, xs_lds_bytes<MODE_TOP2, METRIC>(), ctx->stream>>>(a, s);
      return;
    }
  }
  if (mode == MODE_TOP2) fail(VSK_ERR_UNSUPPORTED, "the screen's argmin mode is L2^2 only");
  if (mode == MODE_DENSE)
    k_flat_screen<MODE_DENSE, METRIC, QR>
        <<<grid, 512, xs_lds_bytes<MODE_DENSE, METRIC>(), ctx->stream>>>(a, s);
  else
    k_flat_screen<MODE_FILTER, METRIC, QR>
        <<<grid, 512, xs_lds_bytes<MODE_FILTER, METRIC>(), ctx->stream>>>(a, s);
}

// planes of at most 128 dims (two stages a tile) keep the queries in LDS
template <int METRIC>
static void launch_s(vsk_ctx *ctx, unsigned grid, const FlatArgs &a, const SplitPtrs &s,
                     int mode) {
  if (s.kb <= 2 * XS_K)
    launch_s<METRIC, true>(ctx, grid, a, s, mode);
  else
    launch_s<METRIC, false>(ctx, grid, a, s, mode);
}

void launch_flat_screen(vsk_ctx *ctx, FlatArgs a, const SplitPtrs &s, int mode,
                        int32_t *nseg, int64_t *stride) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  if (mode == MODE_MATRIX || mode == MODE_ARGMIN)
    fail(VSK_ERR_UNSUPPORTED, "the screen has no matrix or VALU argmin mode");
  if (s.ldqb != s.ldxb || s.kb > s.ldxb || (s.kb & 63))
    fail(VSK_ERR_INVALID_ARGUMENT, "screen planes need one pitch and a padded dimension");
  static bool lds_set = false;
  if (!lds_set) {
    set_lds_metric<VSK_METRIC_L2SQ, false>();
    set_lds_metric<VSK_METRIC_L2SQ, true>();
    set_lds_metric<VSK_METRIC_L2, false>();
    set_lds_metric<VSK_METRIC_L2, true>();
    set_lds_metric<VSK_METRIC_COSINE_NORMALIZED, false>();
    set_lds_metric<VSK_METRIC_COSINE_NORMALIZED, true>();
    set_lds_metric<VSK_METRIC_DOT, false>();
    set_lds_metric<VSK_METRIC_DOT, true>();
    set_lds_metric<VSK_METRIC_COSINE, false>();
    set_lds_metric<VSK_METRIC_COSINE, true>();
    lds_set = true;
  }
  const int64_t qt = ceil_div(a.nq, XS_Q);
  // Row splits, a multiple of 8 (one share per XCD).  One workgroup fills a
  // CU, so the launch runs in rounds of cu_count workgroups: take the split
  // count with the fewest (rounds x tiles per split), the fewer splits on a
  // tie, up to about 8 rounds.  (Filter mode: at most cap/32 - 7 splits, so
  // that every split's workgroup reserves at least 32 slots per query.)
  const int64_t tiles = ceil_div(rows, XS_N);
  int64_t top = 8 * ceil_div(8 * (int64_t)ctx->cu_count, 8 * qt);
  if (top > 8 * ceil_div(tiles, 8)) top = 8 * ceil_div(tiles, 8);
  if (mode == MODE_FILTER && top > (a.cap / 32 - 7) / 8 * 8) top = (a.cap / 32 - 7) / 8 * 8;
  if (top < 8) top = 8;
  int64_t splits = 8, best = -1;
  for (int64_t sp = 8; sp <= top; sp += 8) {
    const int64_t tps = ceil_div(tiles, sp);
    const int64_t used = ceil_div(tiles, tps);
    const int64_t cost = ceil_div(qt * used, (int64_t)ctx->cu_count) * tps;
    if (best < 0 || cost < best) {
      best = cost;
      splits = sp;
    }
  }
  // Order of the (query tile, split) workgroups.  Split-major (XCD x takes
  // query tiles x*qx .. x*qx+qx-1 over every split in turn) when the query
  // tiles divide evenly over the XCDs, to within 1/32: all XCDs then stream
  // the same rows at a time, read from HBM once and served to the other XCDs
  // by the memory-side cache.  (Measured at 1M x 768, 10,000 queries: 7%
  // faster than the group order.)  Otherwise groups of XS_GQ query tiles
  // over the splits that each XCD owns: every XCD gets an equal share.
  a.qtiles_per_xcd = 0;
  if (mode != MODE_TOP2) {
    const int64_t qx = ceil_div(qt, 8);
    if (32 * (8 * qx - qt) <= qt) a.qtiles_per_xcd = (int32_t)qx;
  }
  a.rows_per_split = ceil_div(tiles, splits) * XS_N;
  a.splits_per_xcd = (int32_t)(splits / 8);
  if (mode == MODE_TOP2 && qt >= 2 * (int64_t)ctx->cu_count) {
    // enough query tiles to fill the chip twice: one split over every row
    splits = 1;
    a.rows_per_split = tiles * XS_N;
    a.splits_per_xcd = 0;
  }
  // reserved slots per (workgroup, query), all splits within cap
  a.sub = 0;
  if (mode == MODE_FILTER) {
    // (the filter queue keeps a block's tile index in 23 bits)
    if (a.rows_per_split >= (int64_t)1 << 31)
      fail(VSK_ERR_INVALID_BUFFER_SIZE, "row split too long for the screen's filter");
    const int64_t sub = a.cap / splits < 256 ? a.cap / splits : 256;
    if (sub < 1) fail(VSK_ERR_INVALID_BUFFER_SIZE, "candidate capacity too small");
    a.sub = (int32_t)sub;
  }
  if (mode == MODE_TOP2) {
    // one (key, distance) pair per query and split: the caller merges them
    a.ldm = splits;
    if (nseg) *nseg = (int32_t)splits;
  }
  if (mode != MODE_FILTER || splits > VSK_MAX_SEG || !nseg || !stride) a.seg_n = nullptr;
  if (a.seg_n) {
    // splits without rows launch no writes: their segments start empty
    fill_i32(ctx, a.seg_n, (int64_t)a.nq * splits, 0);
    *nseg = (int32_t)splits;
    *stride = a.sub;
  }
  const int64_t groups = ceil_div(qt, XS_GQ);
  const int64_t nblocks = a.qtiles_per_xcd ? 8 * (int64_t)a.qtiles_per_xcd * splits
                         : a.splits_per_xcd ? 8 * a.splits_per_xcd * groups * XS_GQ : qt;
  if (nblocks > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "grid too large");
  static const char *names[5] = {"flat_screen_dense", "flat_screen_filter", "",
                                 "", "flat_screen_top2"};
  KernelTimer t(ctx, names[mode], (double)a.nq * (double)rows);
  switch (a.metric) {
  case VSK_METRIC_L2SQ: launch_s<VSK_METRIC_L2SQ>(ctx, (unsigned)nblocks, a, s, mode); break;
  case VSK_METRIC_L2: launch_s<VSK_METRIC_L2>(ctx, (unsigned)nblocks, a, s, mode); break;
  case VSK_METRIC_COSINE_NORMALIZED:
    launch_s<VSK_METRIC_COSINE_NORMALIZED>(ctx, (unsigned)nblocks, a, s, mode);
    break;
  case VSK_METRIC_DOT: launch_s<VSK_METRIC_DOT>(ctx, (unsigned)nblocks, a, s, mode); break;
  case VSK_METRIC_COSINE: launch_s<VSK_METRIC_COSINE>(ctx, (unsigned)nblocks, a, s, mode); break;
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
