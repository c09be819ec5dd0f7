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

// hi/lo planes of an (n x ld) fp32 matrix, zero-padded to ldb columns
__global__ void k_split_bf16(const float *x, int64_t n, int32_t d, int32_t ld,
                             uint16_t *hi, uint16_t *lo, int32_t ldb) {
#pragma clang fp contract(off)
  const int64_t total = n * (int64_t)ldb;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / ldb;
    const int32_t c = (int32_t)(i - r * ldb);
    const float v = c < d ? x[r * ld + c] : 0.f;
    const uint16_t h = bf16_rn(v);
    const float hv = __uint_as_float((uint32_t)h << 16);
    hi[i] = h;
    lo[i] = bf16_rn(v - hv);
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
__device__ __forceinline__ void x3_mfma(f4 (&acc)[4][4], const uint8_t *buf,
                                        int wr, int wq, int lane) {
  const uint8_t *xh_s = buf, *xl_s = buf + XB_N * XR;
  const uint8_t *qh_s = buf + 2 * XB_N * XR, *ql_s = buf + (2 * XB_N + XB_Q) * XR;
  const int cl = lane >> 4;
  bf8 bh[4], bl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int off = swz(wq * 64 + j * 16 + (lane & 15), cl);
    bh[j] = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(qh_s + off));
    bl[j] = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(ql_s + off));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int off = swz(wr * 64 + i * 16 + (lane & 15), cl);
    const bf8 ah = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(xh_s + off));
    const bf8 al = __builtin_bit_cast(bf8, *reinterpret_cast<const uint4 *>(xl_s + off));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh[j], acc[i][j], 0, 0, 0);
  }
}

template <int MODE, int METRIC>
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
  const int nst = s.kb / XB_K;
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
    uint4 pxh0, pxh1, pxl0, pxl1, pqh0, pqh1, pql0, pql1;
#define X3_LOAD(ST)                                                           \
  do {                                                                        \
    const int k_ = (ST) * XB_K;                                               \
    pxh0 = X3_LD(rxh, ox0, k_);                                               \
    pxl0 = X3_LD(rxl, ox0, k_);                                               \
    pxh1 = X3_LD(rxh, ox1, k_);                                               \
    pxl1 = X3_LD(rxl, ox1, k_);                                               \
    pqh0 = X3_LD(rqh, oq0, k_);                                               \
    pql0 = X3_LD(rql, oq0, k_);                                               \
    pqh1 = X3_LD(rqh, oq1, k_);                                               \
    pql1 = X3_LD(rql, oq1, k_);                                               \
  } while (0)
#define X3_STORE(BUF)                                                         \
  do {                                                                        \
    uint8_t *b_ = (BUF);                                                      \
    *reinterpret_cast<uint4 *>(b_ + w0) = pxh0;                               \
    *reinterpret_cast<uint4 *>(b_ + w1) = pxh1;                               \
    *reinterpret_cast<uint4 *>(b_ + XB_N * XR + w0) = pxl0;                   \
    *reinterpret_cast<uint4 *>(b_ + XB_N * XR + w1) = pxl1;                   \
    *reinterpret_cast<uint4 *>(b_ + 2 * XB_N * XR + w0) = pqh0;               \
    *reinterpret_cast<uint4 *>(b_ + 2 * XB_N * XR + w1) = pqh1;               \
    *reinterpret_cast<uint4 *>(b_ + (2 * XB_N + XB_Q) * XR + w0) = pql0;      \
    *reinterpret_cast<uint4 *>(b_ + (2 * XB_N + XB_Q) * XR + w1) = pql1;      \
  } while (0)
    // prologue: stage 0 in buffer 0, stage 1 in registers
    __syncthreads();  // the previous tile's last reads are done
    X3_LOAD(0);
    X3_STORE(lds);
    if (nst > 1) X3_LOAD(1);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
      uint8_t *cur = lds + (st & 1) * STAGE_BYTES;
      uint8_t *nxt = lds + ((st + 1) & 1) * STAGE_BYTES;
      // stage st+1 goes into the other buffer while this one is consumed
      // (every wave finished reading it at the barrier closing stage st-1)
      if (st + 1 < nst) {
        X3_STORE(nxt);
        if (st + 2 < nst) X3_LOAD(st + 2);
      }
      x3_mfma(acc, cur, wr, wq, lane);
      __syncthreads();
    }
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
            const float xa = a.xaux ? a.xaux[rbase + i * 16 + r] : 0.f;
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

template <int METRIC>
static void launch_x(vsk_ctx *ctx, unsigned grid, const FlatArgs &a,
                     const SplitPtrs &s, int mode) {
  if (mode == MODE_DENSE)
    k_flat_bf16x3<MODE_DENSE, METRIC><<<grid, 256, 0, ctx->stream>>>(a, s);
  else if (mode == MODE_FILTER)
    k_flat_bf16x3<MODE_FILTER, METRIC><<<grid, 256, 0, ctx->stream>>>(a, s);
  else
    k_flat_bf16x3<MODE_MATRIX, METRIC><<<grid, 256, 0, ctx->stream>>>(a, s);
}

void split_bf16(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
                uint16_t *hi, uint16_t *lo, int32_t ldb) {
  if (n <= 0) return;
  int64_t g = ceil_div(n * (int64_t)ldb, 256);
  if (g > 16384) g = 16384;
  KernelTimer t(ctx, "split_bf16");
  k_split_bf16<<<(unsigned)g, 256, 0, ctx->stream>>>(x, n, d, ld, hi, lo, ldb);
  check_launch("split_bf16");
}

void launch_flat_bf16x3(vsk_ctx *ctx, FlatArgs a, const SplitPtrs &s, int mode) {
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
  static const char *names[3] = {"flat_bf16x3_dense", "flat_bf16x3_filter",
                                 "flat_bf16x3_matrix"};
  KernelTimer t(ctx, names[mode], (double)a.nq * (double)rows);
  switch (a.metric) {
  case VSK_METRIC_L2SQ: launch_x<VSK_METRIC_L2SQ>(ctx, grid, a, s, mode); break;
  case VSK_METRIC_L2: launch_x<VSK_METRIC_L2>(ctx, grid, a, s, mode); break;
  case VSK_METRIC_COSINE: launch_x<VSK_METRIC_COSINE>(ctx, grid, a, s, mode); break;
  case VSK_METRIC_COSINE_NORMALIZED:
    launch_x<VSK_METRIC_COSINE_NORMALIZED>(ctx, grid, a, s, mode);
    break;
  default: launch_x<VSK_METRIC_DOT>(ctx, grid, a, s, mode); break;
  }
  check_launch(names[mode]);
}

}  // namespace vsk
