// flat.hpp -- the flat scan kernels' launch interface, shared by the flat
// search, IVF probing/assignment and the PQ re-rank.
#pragma once

#include "vsk_api.hpp"

namespace vsk {

// internal metric: sqrt(sum (q-x)^2) summed in dimension order without FMA
// (bit-identical to a sequential fp32 loop; VALU kernel)
constexpr int32_t METRIC_L2_EXACT = 100;

enum { MODE_DENSE = 0, MODE_FILTER = 1, MODE_MATRIX = 2, MODE_ARGMIN = 3 };

struct FlatArgs {
  const float *X;
  int64_t ldx;
  const float *Q;
  int64_t ldq;
  const float *xaux;  // |x|^2 (L2), |x| (cosine), else null
  const float *qaux;  // same for queries
  int32_t kdim;       // padded dimension (multiple of 4)
  int32_t nq;
  int64_t r0, r1;
  int64_t rows_per_split;
  int32_t metric;
  const uint64_t *thresh;
  const uint8_t *active;
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
  float *mat;  // MODE_MATRIX output, row-major nq x ldm
  int64_t ldm;
  int32_t splits_per_xcd;  // bf16x3 kernel: row splits owned by each XCD
};

// bf16 hi/lo operand planes of the bf16x3 kernel
struct SplitPtrs {
  const uint16_t *xh, *xl;  // row planes, stride ldxb
  const uint16_t *qh, *ql;  // query planes, stride ldqb
  int64_t ldxb, ldqb;
  int32_t kb;               // padded dimension (multiple of 32)
};
// hi = bf16(x), lo = bf16(x - hi) of an (n x ld) fp32 matrix, ldb columns
void split_bf16(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
                uint16_t *hi, uint16_t *lo, int32_t ldb);
void launch_flat_bf16x3(vsk_ctx *ctx, FlatArgs a, const SplitPtrs &s, int mode);

// launch one scan over rows [a.r0, a.r1) of a.X for the a.nq queries of a.Q
// (mode MODE_*; argmin output only for MODE_ARGMIN).  a.rows_per_split is
// chosen here.
void launch_flat(vsk_ctx *ctx, FlatArgs a, int mode, int32_t *argmin);

// exact top-k of queries dq (device, stride db->ld) over a resident
// database; best: nq*k keys
void flat_topk_device(vsk_ctx *ctx, const vsk_db *db, const float *dq,
                      int64_t nq, int32_t k, int32_t metric, uint64_t *best);

}  // namespace vsk
