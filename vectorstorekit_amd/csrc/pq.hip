// pq.hip -- product quantization: distance tables (LUT), encoding, the ADC
// scan with the tables resident in LDS, and the exact re-rank.
//
// Reference: ProductQuantizer (Quantization/ProductQuantizer.swift):
// precomputeDistanceTables (:209-233) -- table[m][c] =
// euclideanDistanceSquared(query segment m, codeword c) (:362-369,
// sequential sum of squared differences); DistanceTables.computeDistance
// (Quantization/ProductQuantizerTypes.swift:14-20) -- sqrt of the sum of
// table[m][code_m] over m ascending; Codebook.encode
// (Quantization/ProductQuantizerCodebook.swift:12-30) -- argmin with strict
// '<'.  The reference has no batch scan and no re-rank; the re-rank uses the
// reference's exact CPU distance formulas
// (Acceleration/AccelerateOptimizer.swift:251-383) summed in index order.
//
// Every floating-point sum here is formed in the reference's order with
// separate multiply and add roundings (no FMA), so tables, ADC sums, re-rank
// distances and ids are bit-identical to the CPU.
//
// ADC scan: a workgroup holds the tables of several queries in LDS and
// streams a slice of the code rows; a thread owns a row, loads its code
// bytes once and accumulates one sum per query; each sum is keyed (sum, row)
// and goes through the same threshold filter / append as the flat scan.
// k_pq_adc16 serves M = 16, ksub = 256 (8 queries, tables interleaved four
// queries to a 16-byte half entry, survivors staged in LDS); k_pq_adc any other
// shape.  Ranking is on the sum (sqrt is monotone); sqrt is applied to the
// outputs only.
#include "flat.hpp"

struct vsk_pq {
  int32_t M = 0, ksub = 0, dsub = 0, d = 0;
  vsk::DevBuf codebooks;  // M x ksub x dsub fp32
  std::vector<float> host_codebooks;  // the same, for identity checks and files
  vsk::DevBuf codes;      // n x M uint8
  int64_t n = 0, cap_rows = 0;
  // the bf16 screen of the ADC scan: the decoded rows x^ (each segment's
  // codeword) as a bf16 plane of xldb columns, |x^|^2 per row, and the
  // maxima over the rows of |bf16(x^)| and |x^ - bf16(x^)|; made by the
  // first screened search and again when rows were added since (xrows)
  mutable vsk::DevBuf xplane, xsq;
  mutable int32_t xldb = 0;
  mutable int64_t xrows = 0;
  mutable double xh_max = 0, xr_max = 0;
};

namespace vsk {

// decode (Quantization/ProductQuantizer.swift:142-160, the codeword of each
// segment; productDequantize, QuantizationShaders.metal:177-198): out[i][j]
// = codebook[j / dsub][code[i][j / dsub]][j % dsub]
__global__ void k_pq_decode(const uint8_t *codes, int64_t n, const float *cb, int32_t M,
                            int32_t ksub, int32_t dsub, float *out) {
  const int64_t d = (int64_t)M * dsub, total = n * d;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / d;
    const int32_t j = (int32_t)(i - r * d), m = j / dsub;
    out[i] = cb[((int64_t)m * ksub + codes[r * M + m]) * dsub + (j - m * dsub)];
  }
}

constexpr int PQ_QG = 4;  // queries per ADC workgroup

// lut[q][m][c], one thread per entry
__global__ void k_pq_lut(const float *q, int64_t nq, int32_t ldq,
                         const float *cb, int32_t M, int32_t ksub, int32_t dsub,
                         float *lut) {
#pragma clang fp contract(off)
  const int64_t total = nq * (int64_t)M * ksub;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t qi = i / ((int64_t)M * ksub);
    const int32_t mc = (int32_t)(i - qi * (int64_t)M * ksub);
    const int32_t m = mc / ksub;
    const float *qs = q + qi * ldq + m * dsub;
    const float *c = cb + (int64_t)mc * dsub;
    float s = 0.f;
    for (int j = 0; j < dsub; ++j) {
      float t = qs[j] - c[j];
      s = s + t * t;
    }
    lut[i] = s;
  }
}

// lut[q][m][c] for segment lengths DS up to 32: block (query batch, m),
// thread c = codeword c (codebooks hold at most 256) with the codeword in
// registers; the batch's query segments are wave-uniform loads, and each
// (q, m) row of the table is one coalesced store.  The sums are the same as
// k_pq_lut's (j ascending, no FMA).
constexpr int PQL_QB = 64;  // queries per block
template <int DS>
__global__ __launch_bounds__(256) void k_pq_lut_seg(const float *q, int64_t nq, int32_t ldq,
                                                    const float *cb, int32_t M, int32_t ksub,
                                                    float *lut) {
#pragma clang fp contract(off)
  const int32_t m = blockIdx.y;
  const int64_t qa = (int64_t)blockIdx.x * PQL_QB;
  const int64_t qb = qa + PQL_QB < nq ? qa + PQL_QB : nq;
  const int32_t c = threadIdx.x;
  if (c >= ksub) return;
  float cw[DS];
  const float *cp = cb + ((int64_t)m * ksub + c) * DS;
#pragma unroll
  for (int j = 0; j < DS; ++j) cw[j] = cp[j];
  for (int64_t qi = qa; qi < qb; ++qi) {
    const float *qs = q + qi * ldq + (int64_t)m * DS;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < DS; ++j) {
      const float t = qs[j] - cw[j];
      s = s + t * t;
    }
    lut[(qi * M + m) * ksub + c] = s;
  }
}

// codes[i][m] = argmin_c |x_m - C_m[c]|^2 (strict '<': the first minimum
// wins), each sum over j in ascending order without FMA.  Block (bx, m):
// codebook m staged in LDS (every lane reads the same codeword, a broadcast),
// one row per thread with its segment in registers when DS (compile-time
// dsub) is nonzero.
template <int DS>
__global__ __launch_bounds__(256) void k_pq_encode_lds(
    const float *x, int64_t n, int32_t ldx, const float *cb, int32_t M,
    int32_t ksub, int32_t dsub, uint8_t *codes) {
#pragma clang fp contract(off)
  extern __shared__ float s_cb[];  // ksub x dsub
  const int32_t m = blockIdx.y;
  const int32_t ds = DS > 0 ? DS : dsub;
  const float *cbm = cb + (int64_t)m * ksub * ds;
  for (int32_t i = threadIdx.x; i < ksub * ds; i += blockDim.x) s_cb[i] = cbm[i];
  __syncthreads();
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < n;
       r += (int64_t)gridDim.x * blockDim.x) {
    const float *xs = x + r * ldx + (int64_t)m * ds;
    float best = __int_as_float(0x7f800000);
    int32_t bc = 0;
    if constexpr (DS > 0) {
      float xv[DS];
#pragma unroll
      for (int j = 0; j < DS; ++j) xv[j] = xs[j];
      for (int32_t c = 0; c < ksub; ++c) {
        const float *cw = s_cb + c * DS;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < DS; ++j) {
          float t = xv[j] - cw[j];
          acc = acc + t * t;
        }
        if (acc < best) {
          best = acc;
          bc = c;
        }
      }
    } else {
      for (int32_t c = 0; c < ksub; ++c) {
        const float *cw = s_cb + c * ds;
        float acc = 0.f;
        for (int j = 0; j < ds; ++j) {
          float t = xs[j] - cw[j];
          acc = acc + t * t;
        }
        if (acc < best) {
          best = acc;
          bc = c;
        }
      }
    }
    codes[r * M + m] = (uint8_t)bc;
  }
}

// same result for codebooks too large for LDS: one thread per (row, m),
// codewords read from global memory
__global__ void k_pq_encode(const float *x, int64_t n, int32_t ldx,
                            const float *cb, int32_t M, int32_t ksub,
                            int32_t dsub, uint8_t *codes) {
#pragma clang fp contract(off)
  const int64_t total = n * (int64_t)M;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / M;
    const int32_t m = (int32_t)(i - r * M);
    const float *xs = x + r * ldx + m * dsub;
    float best = __int_as_float(0x7f800000);
    int32_t bc = 0;
    for (int32_t c = 0; c < ksub; ++c) {
      const float *cw = cb + ((int64_t)m * ksub + c) * dsub;
      float acc = 0.f;
      for (int j = 0; j < dsub; ++j) {
        float t = xs[j] - cw[j];
        acc = acc + t * t;
      }
      if (acc < best) {
        best = acc;
        bc = c;
      }
    }
    codes[i] = (uint8_t)bc;
  }
}

static unsigned grid1(int64_t n) {
  int64_t g = ceil_div(n, 256);
  return (unsigned)(g < 16384 ? (g > 0 ? g : 1) : 16384);
}

static void launch_encode(vsk_ctx *ctx, const vsk_pq *pq, const float *dx,
                          int64_t n, uint8_t *codes) {
  const size_t lds = sizeof(float) * (size_t)pq->ksub * pq->dsub;
  KernelTimer t(ctx, "pq_encode", (double)n * pq->M);
  if (lds <= 64 * 1024) {
    int64_t bx = ceil_div(n, 256);
    if (bx > 2048) bx = 2048;
    dim3 grid((unsigned)bx, (unsigned)pq->M);
    switch (pq->dsub) {
      case 4:
        k_pq_encode_lds<4><<<grid, 256, lds, ctx->stream>>>(
            dx, n, pq->d, pq->codebooks.as<float>(), pq->M, pq->ksub, pq->dsub, codes);
        break;
      case 8:
        k_pq_encode_lds<8><<<grid, 256, lds, ctx->stream>>>(
            dx, n, pq->d, pq->codebooks.as<float>(), pq->M, pq->ksub, pq->dsub, codes);
        break;
      case 16:
        k_pq_encode_lds<16><<<grid, 256, lds, ctx->stream>>>(
            dx, n, pq->d, pq->codebooks.as<float>(), pq->M, pq->ksub, pq->dsub, codes);
        break;
      default:
        k_pq_encode_lds<0><<<grid, 256, lds, ctx->stream>>>(
            dx, n, pq->d, pq->codebooks.as<float>(), pq->M, pq->ksub, pq->dsub, codes);
    }
  } else {
    k_pq_encode<<<grid1(n * pq->M), 256, 0, ctx->stream>>>(
        dx, n, pq->d, pq->codebooks.as<float>(), pq->M, pq->ksub, pq->dsub, codes);
  }
  check_launch("pq_encode");
}

struct AdcArgs {
  const uint8_t *codes;
  int32_t M, ksub;
  const float *lut;  // [nq][M][ksub]
  int32_t nq;
  int64_t r0, r1, rows_per_split;
  const uint64_t *thresh;
  const uint8_t *active;
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
};

template <bool DENSE, bool M16>
__global__ __launch_bounds__(256) void k_pq_adc(AdcArgs a) {
  extern __shared__ float lut_s[];  // PQ_QG x M x ksub
  const int64_t q0 = (int64_t)blockIdx.x * PQ_QG;
  const int64_t s0 = a.r0 + (int64_t)blockIdx.y * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1) return;
  const int tsz = a.M * a.ksub;
  for (int i = threadIdx.x; i < PQ_QG * tsz; i += blockDim.x) {
    const int j = i / tsz;
    lut_s[i] = (q0 + j < a.nq) ? a.lut[(q0 + j) * tsz + (i - j * tsz)] : 0.f;
  }
  bool qok[PQ_QG];
  uint64_t th[PQ_QG];
#pragma unroll
  for (int j = 0; j < PQ_QG; ++j) {
    qok[j] = q0 + j < a.nq && (!a.active || a.active[q0 + j]);
    th[j] = (!DENSE && qok[j]) ? a.thresh[q0 + j] : 0;
  }
  __syncthreads();
  for (int64_t r = s0 + threadIdx.x; r < s1; r += blockDim.x) {
    float s[PQ_QG];
#pragma unroll
    for (int j = 0; j < PQ_QG; ++j) s[j] = 0.f;
    if constexpr (M16) {
      const uint4 cw = *reinterpret_cast<const uint4 *>(a.codes + r * 16);
      const uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const int c = (w4[m >> 2] >> (8 * (m & 3))) & 0xFF;
#pragma unroll
        for (int j = 0; j < PQ_QG; ++j)
          s[j] = s[j] + lut_s[j * tsz + m * a.ksub + c];
      }
    } else {
      const uint8_t *cr = a.codes + r * a.M;
      for (int m = 0; m < a.M; ++m) {
        const int c = cr[m];
#pragma unroll
        for (int j = 0; j < PQ_QG; ++j)
          s[j] = s[j] + lut_s[j * tsz + m * a.ksub + c];
      }
    }
#pragma unroll
    for (int j = 0; j < PQ_QG; ++j) {
      if (!qok[j]) continue;
      const int64_t qi = q0 + j;
      const uint64_t key = vsk_key(s[j], (uint32_t)r);
      if (DENSE) {
        a.cand[qi * a.cap + (r - a.r0)] = key;
      } else if (key <= th[j]) {
        int slot = atomicAdd(&a.counts[qi], 1);
        if (slot < a.cap) a.cand[qi * a.cap + slot] = key;
      }
    }
  }
}

static void launch_adc(vsk_ctx *ctx, AdcArgs a, bool dense) {
  const int64_t rows = a.r1 - a.r0;
  if (rows <= 0 || a.nq <= 0) return;
  const int64_t qt = ceil_div(a.nq, PQ_QG);
  int64_t splits = ceil_div(8192, qt);
  const int64_t max_splits = ceil_div(rows, 1024);
  if (splits > max_splits) splits = max_splits;
  if (splits > 65535) splits = 65535;
  if (splits < 1) splits = 1;
  a.rows_per_split = ceil_div(rows, splits);
  splits = ceil_div(rows, a.rows_per_split);
  dim3 grid((unsigned)qt, (unsigned)splits);
  const size_t lds = sizeof(float) * PQ_QG * a.M * a.ksub;
  const bool m16 = a.M == 16;
  KernelTimer t(ctx, dense ? "pq_adc_dense" : "pq_adc_filter",
                (double)a.nq * (double)rows);
  if (dense) {
    if (m16)
      k_pq_adc<true, true><<<grid, 256, lds, ctx->stream>>>(a);
    else
      k_pq_adc<true, false><<<grid, 256, lds, ctx->stream>>>(a);
  } else {
    if (m16)
      k_pq_adc<false, true><<<grid, 256, lds, ctx->stream>>>(a);
    else
      k_pq_adc<false, false><<<grid, 256, lds, ctx->stream>>>(a);
  }
  check_launch("pq_adc_scan");
}

// ADC scan for the common shape M = 16, ksub = 256 (16-byte code rows).
// A workgroup of 8 waves holds the tables of 8 queries in LDS, interleaved
// four queries to a 16-byte entry (entry [g][m][c] = table[m][c] of queries
// 4g..4g+3), so one ds_read_b128 serves four queries and the entries of one
// m spread over all 16 four-bank groups.  A thread owns a code row: one
// 16-byte load, 32 LDS reads, the eight sums in m order (bit-exact).
// Filter mode reserves `sub` slots of each query's candidate list up front
// (one device atomic per query, not one per survivor: the counters of the
// 8,000 survivors of a query would otherwise serialise at one L2 address)
// and fills them through LDS counters; unused slots become NONE and a query
// whose slots overflow gets a count past cap (the chunk is re-scanned).
// Workgroup L runs on XCD L % 8; the query groups of one row split are
// consecutive slots of one XCD, so they share its L2 for the code rows.
constexpr int PQ16_QG = 8, PQ16_T = 512;
typedef float pq_f4 __attribute__((ext_vector_type(4)));
// LDS (static, so every table address is known at compile time and its
// segment offset folds into the read's immediate): the tables as two
// halves of 16 x 256 entries of 16 bytes, entry (m, c) of half h holding
// queries 4h..4h+3 of the group (a 16-byte stride keeps random codes spread
// over all 16 bank quads), then the survivor
// staging of each wave (key, then slot << 3 | query), then per query: first
// slot, threshold key, slot limit, slot count, active flag.
constexpr int PQ16_TAB = 2 * 16 * 256 * 16;
// filter survivors are staged per wave in LDS and stored in bulk: a global
// store between the prefetch loads and their use would make every use wait
// for all of them (one vector memory counter for loads and stores, which
// may then complete out of order)
constexpr int PQ16_WBUF = 256;
constexpr int PQ16_WAVES = PQ16_T / 64;
constexpr int PQ16_KEYS = PQ16_TAB;
constexpr int PQ16_META = PQ16_KEYS + PQ16_WAVES * PQ16_WBUF * 8;
constexpr int PQ16_STATE = PQ16_META + PQ16_WAVES * PQ16_WBUF * 4;
constexpr int PQ16_LDS = PQ16_STATE + PQ16_QG * (3 * 4 + 2 * 8);
static_assert(PQ16_LDS <= 160 * 1024, "LDS of one workgroup");

struct Adc16Args {
  const uint8_t *codes;
  const float *lut;  // [nq][16][256]
  int32_t nq, nqg, splits_per_xcd, sub;
  int64_t r0, r1, rows_per_split;
  const uint64_t *thresh;
  const uint8_t *active;
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
};

template <bool DENSE>
__global__ __launch_bounds__(PQ16_T) void k_pq_adc16(Adc16Args a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) uint8_t lds[PQ16_LDS];
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  uint64_t *w_key = reinterpret_cast<uint64_t *>(lds + PQ16_KEYS) + wv * PQ16_WBUF;
  uint32_t *w_meta = reinterpret_cast<uint32_t *>(lds + PQ16_META) + wv * PQ16_WBUF;
  int64_t *s_pb = reinterpret_cast<int64_t *>(lds + PQ16_STATE);
  uint64_t *s_th = reinterpret_cast<uint64_t *>(s_pb + PQ16_QG);
  int32_t *s_lim = reinterpret_cast<int32_t *>(s_th + PQ16_QG);
  int32_t *s_cnt = s_lim + PQ16_QG, *s_ok = s_cnt + PQ16_QG;
  const int L = blockIdx.x, xcd = L & 7, slot = L >> 3;
  const int qg = slot % a.nqg;
  const int split = (slot / a.nqg) * 8 + xcd;
  const int64_t q0 = (int64_t)qg * PQ16_QG;
  const int64_t s0 = a.r0 + (int64_t)split * a.rows_per_split;
  int64_t s1 = s0 + a.rows_per_split;
  if (s1 > a.r1) s1 = a.r1;
  if (s0 >= s1 || q0 >= a.nq) return;
  {
    // entry e = 4096 h + 256 m + c holds lut[q0 + 4h + 0..3][m][c]
    float4 *w = reinterpret_cast<float4 *>(lds);
    for (int e = tid; e < 2 * 4096; e += PQ16_T) {
      const int h = e >> 12, mc = e & 4095;
      float v[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int64_t q = q0 + 4 * h + jj;
        v[jj] = q < a.nq ? a.lut[q * 4096 + mc] : 0.f;
      }
      w[e] = float4{v[0], v[1], v[2], v[3]};
    }
  }
  if (tid < PQ16_QG) {
    const int64_t q = q0 + tid;
    const bool ok = q < a.nq && (!a.active || a.active[q]);
    s_ok[tid] = ok ? 1 : 0;
    s_th[tid] = (ok && !DENSE) ? a.thresh[q] : VSK_KEY_NONE;
    if constexpr (!DENSE) {
      const int64_t base = ok ? atomicAdd(&a.counts[q], a.sub) : a.cap;
      const int64_t room = a.cap - base;
      s_lim[tid] = (int32_t)(room < a.sub ? (room > 0 ? room : 0) : a.sub);
      s_pb[tid] = q * a.cap + base;
      s_cnt[tid] = 0;
    }
  }
  __syncthreads();
  // threshold of each query as a sum: a row can pass only if its sum is at
  // most this (NaN sums fail the compare and are kept for the exact key
  // test, which orders them last); inactive queries: -inf, so only NaN
  // sums reach the key test, which then drops them by the flag
  float thf[PQ16_QG];
  uint64_t thk[PQ16_QG];
  bool ok[PQ16_QG];
#pragma unroll
  for (int j = 0; j < PQ16_QG; ++j) {
    const uint64_t th = s_th[j];
    thk[j] = th;
    ok[j] = s_ok[j] != 0;
    const uint32_t hi = (uint32_t)(th >> 32);
    thf[j] = !ok[j] ? -__int_as_float(0x7f800000)
                    : (hi == 0xFFFFFFFFu ? __int_as_float(0x7f800000) : vsk_ord2f(hi));
  }
  // code rows of this split through a buffer descriptor (reads past the
  // split return 0)
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.codes + s0 * 16), 0, (int32_t)((s1 - s0) * 16), 0x00020000);
  // block b = rows s0 + 512 b + tid; every lane runs the same number of
  // blocks (rows past the split read as zeros and are masked at the end)
  auto load_blk = [&](int b) {
    return __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(rc, (b * PQ16_T + tid) * 16, 0, 0));
  };
  int wcnt = 0;  // this wave's staged survivors (wave-uniform)
  auto flush = [&]() {
    for (int i = lane; i < wcnt; i += 64) {
      const uint32_t meta = w_meta[i];
      const int j = (int)(meta & 7u), pos = (int)(meta >> 3);
      if (pos < s_lim[j]) a.cand[s_pb[j] + pos] = w_key[i];
    }
    wcnt = 0;
    // the stores complete here, so none is pending beside the prefetch loads
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  };
  uint32_t hi_base = 65536;
  asm volatile("" : "+s"(hi_base));
  // one row: 32 table reads (16 bytes each, four queries), the eight sums in
  // m order, then the filter or the dense store
  auto row = [&](int b, const uint4 cw) {
    const int64_t r = s0 + (int64_t)b * PQ16_T + tid;
    const bool valid = r < s1;
    const uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
    float sa[4] = {0.f, 0.f, 0.f, 0.f}, sb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const uint32_t c = (w4[m >> 2] >> (8 * (m & 3))) & 0xFFu;
      // (a native 4-vector: one 16-byte read each; the HIP float4 struct is
      // split into scalar loads, some of which come back 4 bytes wide)
      // the second half lies past the 16-bit immediate offset: its base
      // comes from a register (one add per code), the segment offsets of
      // both halves fold into the reads
      const pq_f4 va = *reinterpret_cast<const pq_f4 *>(lds + m * 4096 + c * 16);
      const pq_f4 vb =
          *reinterpret_cast<const pq_f4 *>(lds + hi_base + m * 4096 + c * 16);
      sa[0] = sa[0] + va[0];
      sa[1] = sa[1] + va[1];
      sa[2] = sa[2] + va[2];
      sa[3] = sa[3] + va[3];
      sb[0] = sb[0] + vb[0];
      sb[1] = sb[1] + vb[1];
      sb[2] = sb[2] + vb[2];
      sb[3] = sb[3] + vb[3];
    }
    const float sum[PQ16_QG] = {sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
#pragma unroll
    for (int j = 0; j < PQ16_QG; ++j) {
      if constexpr (DENSE) {
        if (ok[j] && valid)
          a.cand[(q0 + j) * a.cap + (r - a.r0)] = vsk_key(sum[j], (uint32_t)r);
      } else {
        // one compare per (row, query) in the common case of no survivor
        const bool maybe = !(sum[j] > thf[j]);
        if (!__builtin_amdgcn_ballot_w64(maybe)) continue;
        const uint64_t key = vsk_key(sum[j], (uint32_t)r);
        const bool pass = maybe && valid && ok[j] && key <= thk[j];
        const uint64_t mask = __builtin_amdgcn_ballot_w64(pass);
        if (mask == 0) continue;
        if (pass) {
          const int pos = atomicAdd(&s_cnt[j], 1);
          const int at = wcnt + (int)__builtin_amdgcn_mbcnt_hi(
                                    (uint32_t)(mask >> 32),
                                    __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
          w_key[at] = key;
          w_meta[at] = ((uint32_t)pos << 3) | (uint32_t)j;
        }
        wcnt += __builtin_popcountll(mask);
        if (wcnt > PQ16_WBUF - 64) flush();
      }
    }
  };
  // four code buffers, each reloaded right after its row is consumed: the
  // load of block b+4 is in flight while blocks b+1..b+3 are processed (a
  // rotation of registers instead would wait for the load just issued)
  const int nblk = (int)((s1 - s0 + PQ16_T - 1) / PQ16_T);
  uint4 c0 = load_blk(0), c1 = load_blk(1), c2 = load_blk(2), c3 = load_blk(3);
  // (no early exit between the four: a conditional reload makes every
  // trip wait for all loads in flight; splits are whole multiples of 8
  // blocks except a chunk's last)
  for (int b = 0; b < nblk; b += 4) {
    row(b, c0);
    c0 = load_blk(b + 4);
    row(b + 1, c1);
    c1 = load_blk(b + 5);
    row(b + 2, c2);
    c2 = load_blk(b + 6);
    row(b + 3, c3);
    c3 = load_blk(b + 7);
  }
  if constexpr (!DENSE) {
    flush();
    __syncthreads();
#pragma unroll 1
    for (int j = 0; j < PQ16_QG; ++j) {
      if (!ok[j]) continue;
      const int32_t n = s_cnt[j], lim = s_lim[j];
      if (n > lim) {
        if (tid == 0) atomicAdd(&a.counts[q0 + j], (int32_t)a.cap + 1);
      } else {
        for (int32_t i = n + tid; i < lim; i += PQ16_T) a.cand[s_pb[j] + i] = VSK_KEY_NONE;
      }
    }
  }
}

static void launch_adc16(vsk_ctx *ctx, const AdcArgs &in, bool dense) {
  const int64_t rows = in.r1 - in.r0;
  if (rows <= 0 || in.nq <= 0) return;
  Adc16Args a;
  a.codes = in.codes;
  a.lut = in.lut;
  a.nq = in.nq;
  a.nqg = (int32_t)ceil_div(in.nq, PQ16_QG);
  a.r0 = in.r0;
  a.r1 = in.r1;
  a.thresh = in.thresh;
  a.active = in.active;
  a.cand = in.cand;
  a.cap = in.cap;
  a.counts = in.counts;
  // Row splits, a multiple of 8: the fewest (rounds of one workgroup per CU
  // x rows per split), up to about 8 rounds, each split at least 4,096 rows
  // (the tables are 128 KB per workgroup); filter mode keeps at least 64
  // reserved slots per (split, query).
  const int64_t unit = PQ16_T * 8;
  const int64_t units = ceil_div(rows, unit);
  int64_t top = 8 * ceil_div(8 * (int64_t)ctx->cu_count, 8 * (int64_t)a.nqg);
  if (top > 8 * ceil_div(units, 8)) top = 8 * ceil_div(units, 8);
  if (!dense && top > in.cap / 64 / 8 * 8) top = in.cap / 64 / 8 * 8;
  if (top < 8) top = 8;
  int64_t splits = 8, best = -1;
  for (int64_t sp = 8; sp <= top; sp += 8) {
    const int64_t ups = ceil_div(units, sp);
    const int64_t used = ceil_div(units, ups);
    const int64_t cost = ceil_div((int64_t)a.nqg * used, (int64_t)ctx->cu_count) * ups;
    if (best < 0 || cost < best) {
      best = cost;
      splits = sp;
    }
  }
  a.rows_per_split = ceil_div(units, splits) * unit;
  a.splits_per_xcd = (int32_t)(splits / 8);
  a.sub = dense ? 0 : (int32_t)(in.cap / splits);
  if (!dense && a.sub < 1) fail(VSK_ERR_INVALID_BUFFER_SIZE, "candidate capacity too small");
  const int64_t nblocks = (int64_t)a.nqg * splits;
  if (nblocks > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "grid too large");
  KernelTimer t(ctx, dense ? "pq_adc_dense" : "pq_adc_filter", (double)in.nq * (double)rows);
  if (dense)
    k_pq_adc16<true><<<(unsigned)nblocks, PQ16_T, 0, ctx->stream>>>(a);
  else
    k_pq_adc16<false><<<(unsigned)nblocks, PQ16_T, 0, ctx->stream>>>(a);
  check_launch("pq_adc16");
}

// ---------------------------------------------------------------------------
// The ADC scan through the bf16 matrix cores.  The ADC distance of a row is
// a sequential fp32 sum of d squared differences q_j - x^_j (segment by
// segment, then over the segments), x^ the row's decoded codewords: the
// same kind of sum the flat screen's L2^2 bound covers.  So the flat screen
// kernel runs over the decoded rows (a bf16 plane) and keeps every row whose
// screened distance a(x) is within eps(q) of the query's exact threshold
// key: a row whose ADC key is at most that threshold has a(x) <= ADC + eps.
// The survivors' keys are then rescored exactly (the LUT sum in m order,
// as the LUT scan adds it) and those above the threshold dropped, so the
// selection sees exactly the keys the LUT scan would have kept.
// ---------------------------------------------------------------------------

// decoded rows: M lanes per row (M divides 64), lane m decodes segment m
template <int DS>
__global__ __launch_bounds__(256) void k_pq_plane(const uint8_t *codes, int64_t n, int32_t M,
                                                  int32_t ksub, const float *cb, int32_t ldb,
                                                  uint16_t *plane, float *sq,
                                                  uint32_t *maxbits) {
#pragma clang fp contract(off)
  const int rpb = 256 / M;
  const int m = threadIdx.x % M;
  const int64_t r = (int64_t)blockIdx.x * rpb + threadIdx.x / M;
  const bool valid = r < n;
  float s2 = 0.f;
  double sh = 0.0, sr = 0.0;
  if (valid) {
    const float *c = cb + ((int64_t)m * ksub + codes[r * M + m]) * DS;
    uint16_t h[DS];
#pragma unroll
    for (int j = 0; j < DS; ++j) {
      const float v = c[j];
      h[j] = bf16_rn(v);
      const float hv = __uint_as_float((uint32_t)h[j] << 16);
      const float rv = v - hv;
      s2 = s2 + v * v;
      sh += (double)hv * (double)hv;
      sr += (double)rv * (double)rv;
    }
    uint16_t *dst = plane + r * ldb + m * DS;
    if constexpr (DS % 2 == 0) {
#pragma unroll
      for (int j = 0; j < DS; j += 2)
        *reinterpret_cast<uint32_t *>(dst + j) = (uint32_t)h[j] | ((uint32_t)h[j + 1] << 16);
    } else {
#pragma unroll
      for (int j = 0; j < DS; ++j) dst[j] = h[j];
    }
  }
  // the row's sums over its M lanes (aligned groups within the wave)
  for (int o = M >> 1; o > 0; o >>= 1) {
    s2 += __shfl_xor(s2, o);
    sh += __shfl_xor(sh, o);
    sr += __shfl_xor(sr, o);
  }
  if (valid && m == 0) sq[r] = s2;
  uint32_t mh = valid ? __float_as_uint(f_up(sqrt(sh) * (1.0 + 1e-12))) : 0u;
  uint32_t mr = valid ? __float_as_uint(f_up(sqrt(sr) * (1.0 + 1e-12))) : 0u;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t a = __shfl_xor(mh, o), b = __shfl_xor(mr, o);
    mh = a > mh ? a : mh;
    mr = b > mr ? b : mr;
  }
  if ((threadIdx.x & 63) == 0 && (mh | mr)) {
    atomicMax(&maxbits[0], mh);
    atomicMax(&maxbits[1], mr);
  }
}

// the screen's filter threshold of each query: its exact threshold's
// distance plus eps(q), every row id (NONE stays NONE).  eps is the flat
// screen's L2^2 bound with x^ for x: 2 e_dot + (2d + 8) u (|q| + |x^|)^2,
// where e_dot = |qh||dx| + |dq||xh| + |dq||dx| + 2(d-1)u|qh||xh| bounds the
// bf16 dot's error and the second term the rounding of |q|^2, |x^|^2, the
// screen's last operations and the ADC sum itself (at most d + 2 roundings of
// a sum bounded by (|q| + |x^|)^2).
__global__ void k_pq_screen_thresh(const uint64_t *thresh, int64_t nq, const float *qnh,
                                   const float *qnr, double xh, double xr, int32_t d,
                                   uint64_t *out) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nq) return;
  const uint64_t t = thresh[q];
  if (t == VSK_KEY_NONE) {
    out[q] = VSK_KEY_NONE;
    return;
  }
  const double eps = screen_eps_of(qnh[q], qnr[q], xh, xr, d, VSK_METRIC_L2SQ);
  const double lim = (double)vsk_ord2f((uint32_t)(t >> 32)) + eps;
  out[q] = vsk_key(f_up(lim), 0xFFFFFFFFu);
}

// exact ADC keys of the screen's survivors, in place (a workgroup per
// query, its table in LDS): the sum of lut[q][m][code_m] in m order from
// 0, as the LUT scan adds it; keys above the exact threshold become NONE.
// A row's M code bytes load as whole 4- or 16-byte words.  Segmented lists
// (seg_n) or appended ones (counts, capped at cap).
template <int M>
__global__ __launch_bounds__(256) void k_pq_rescore_keys(
    const uint8_t *codes, int32_t ksub, const float *lut, const uint64_t *thresh,
    const uint8_t *active, uint64_t *cand, int64_t cap, const int32_t *counts,
    const int32_t *seg_n, int32_t nseg, int64_t seg_stride) {
#pragma clang fp contract(off)
  extern __shared__ float lut_s[];  // M x ksub
  const int64_t q = blockIdx.x;
  if (active && !active[q]) return;
  const int mk = M * ksub;
  for (int i = threadIdx.x; i < mk; i += 256) lut_s[i] = lut[q * mk + i];
  __syncthreads();
  const uint64_t th = thresh[q];
  constexpr int NW = M >= 4 ? M / 4 : 1;  // 32-bit words per code row
  auto rescore = [&](uint64_t &key) {
    if (key == VSK_KEY_NONE) return;
    const uint32_t row = (uint32_t)key;
    const uint8_t *c = codes + (int64_t)row * M;
    uint32_t w[NW];
    if constexpr (M >= 16) {
#pragma unroll
      for (int i = 0; i < M / 16; ++i) {
        const uint4 v = reinterpret_cast<const uint4 *>(c)[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
      }
    } else if constexpr (M >= 4) {
#pragma unroll
      for (int i = 0; i < NW; ++i) w[i] = reinterpret_cast<const uint32_t *>(c)[i];
    } else {
      w[0] = 0;
#pragma unroll
      for (int m = 0; m < M; ++m) w[0] |= (uint32_t)c[m] << (8 * m);
    }
    float s = 0.f;
#pragma unroll
    for (int m = 0; m < M; ++m) s = s + lut_s[m * ksub + ((w[m >> 2] >> (8 * (m & 3))) & 0xFFu)];
    const uint64_t ek = vsk_key(s, row);
    key = ek <= th ? ek : VSK_KEY_NONE;
  };
  // four keys a lane at a time: their loads (key, then code row) in
  // flight together rather than one key's chain after another's
  auto rescore4 = [&](uint64_t *p, int64_t i, int64_t n, int64_t step) {
    uint64_t k4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) k4[u] = i + u * step < n ? p[i + u * step] : VSK_KEY_NONE;
#pragma unroll
    for (int u = 0; u < 4; ++u) rescore(k4[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i + u * step < n) p[i + u * step] = k4[u];
  };
  uint64_t *base = cand + q * cap;
  if (seg_n) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int sgi = w; sgi < nseg; sgi += 4) {
      const int32_t ns = seg_n[q * nseg + sgi];
      uint64_t *cs = base + (int64_t)sgi * seg_stride;
      for (int32_t i = lane; i < ns; i += 256) rescore4(cs, i, ns, 64);
    }
  } else {
    int64_t cnt = counts[q];
    if (cnt > cap) return;  // overflowed: the chunk is re-scanned whole
    for (int64_t i = threadIdx.x; i < cnt; i += 1024) rescore4(base, i, cnt, 256);
  }
}

// the decoded plane of the screen, made when missing or stale
static void pq_screen_plane(vsk_ctx *ctx, const vsk_pq *pq) {
  if (pq->xrows == pq->n && pq->xplane.p) return;
  const int32_t ldb = (pq->d + 63) & ~63;
  pq->xplane.reserve(sizeof(uint16_t) * (size_t)pq->n * ldb);
  pq->xsq.reserve(sizeof(float) * (size_t)pq->n);
  uint16_t *plane = pq->xplane.as<uint16_t>();
  if (ldb > pq->d) fill_i32(ctx, reinterpret_cast<int32_t *>(plane), (int64_t)pq->n * ldb / 2, 0);
  uint32_t *mb = static_cast<uint32_t *>(ctx->scratch_ptr("pq.planemax", 2 * sizeof(uint32_t)));
  fill_i32(ctx, reinterpret_cast<int32_t *>(mb), 2, 0);
  const int64_t rpb = 256 / pq->M;
  const unsigned grid = (unsigned)ceil_div(pq->n, rpb);
  {
    KernelTimer t(ctx, "pq_screen_plane", (double)pq->n);
    const float *cb = pq->codebooks.as<float>();
    const uint8_t *codes = pq->codes.as<uint8_t>();
    float *sq = pq->xsq.as<float>();
    switch (pq->dsub) {
    case 1: k_pq_plane<1><<<grid, 256, 0, ctx->stream>>>(codes, pq->n, pq->M, pq->ksub, cb, ldb, plane, sq, mb); break;
    case 2: k_pq_plane<2><<<grid, 256, 0, ctx->stream>>>(codes, pq->n, pq->M, pq->ksub, cb, ldb, plane, sq, mb); break;
    case 4: k_pq_plane<4><<<grid, 256, 0, ctx->stream>>>(codes, pq->n, pq->M, pq->ksub, cb, ldb, plane, sq, mb); break;
    case 8: k_pq_plane<8><<<grid, 256, 0, ctx->stream>>>(codes, pq->n, pq->M, pq->ksub, cb, ldb, plane, sq, mb); break;
    case 16: k_pq_plane<16><<<grid, 256, 0, ctx->stream>>>(codes, pq->n, pq->M, pq->ksub, cb, ldb, plane, sq, mb); break;
    default: k_pq_plane<32><<<grid, 256, 0, ctx->stream>>>(codes, pq->n, pq->M, pq->ksub, cb, ldb, plane, sq, mb); break;
    }
    check_launch("pq_screen_plane");
  }
  uint32_t hb[2];
  VSK_HIP(hipMemcpyAsync(hb, mb, sizeof(hb), hipMemcpyDeviceToHost, ctx->stream));
  stream_sync(ctx);
  pq->xh_max = __builtin_bit_cast(float, hb[0]);
  pq->xr_max = __builtin_bit_cast(float, hb[1]);
  pq->xldb = ldb;
  pq->xrows = pq->n;
}

// the screen serves a search of nq queries: segments of at most 32 values
// whose count divides a wave, and a problem large enough that the screen's
// fixed launches pay (forced by VSK_FLAT_KERNEL=screen, off by =exact)
static bool pq_screen_applies(const vsk_ctx *ctx, const vsk_pq *pq, int64_t nq) {
  if (ctx->flat_no_screen || ctx->flat_fp32 || ctx->exact_only) return false;
  if (pq->M < 1 || pq->M > 64 || (64 % pq->M) != 0) return false;
  if (pq->dsub != 1 && pq->dsub != 2 && pq->dsub != 4 && pq->dsub != 8 && pq->dsub != 16 &&
      pq->dsub != 32)
    return false;
  if (pq->n >= 0x7FFFFFFFll) return false;
  return ctx->flat_force_screen || (double)nq * (double)pq->n * pq->d >= (double)(1ll << 30);
}

// exact distance of each ADC candidate, summed in index order (no FMA).
// A workgroup takes 256 candidates of one query, a wave 64 of them: per
// block of 64 dimensions the wave gathers its rows in 256-byte segments (16
// lanes per row, coalesced) and the query's block into its LDS tile, then
// every lane continues the sequential sums of its own row from there.
constexpr int RR_W = 64;         // dimensions per gathered block
constexpr int RR_LD = RR_W + 4;  // LDS row stride (floats)
typedef float rr_f4 __attribute__((ext_vector_type(4)));

template <int METRIC>
__global__ __launch_bounds__(256) void k_rerank(const uint64_t *adc_best, int32_t kadc,
                                                const float *q, int32_t ldq,
                                                const float *x, int32_t ldx, int32_t d,
                                                uint64_t *out) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float tile[4][65 * RR_LD];  // rows, then the query
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t qi = blockIdx.x;
  const int32_t c = blockIdx.y * 256 + threadIdx.x;
  const uint64_t key = c < kadc ? adc_best[qi * kadc + c] : VSK_KEY_NONE;
  const bool valid = key != VSK_KEY_NONE;
  if (!__builtin_amdgcn_ballot_w64(valid)) {
    if (c < kadc) out[qi * kadc + c] = VSK_KEY_NONE;
    return;
  }
  const uint32_t row = (uint32_t)key;
  const float *qr = q + qi * ldq;
  float *t = tile[w];
  const int seg = lane & 15, sub = lane >> 4;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;  // the metric's sums (cosine: q.x, q.q, x.x)
  // the rows this lane gathers: candidates sub, sub + 4, ..., sub + 60 (a
  // missing candidate reads row 0, a segment past the row end is clamped
  // into it; neither is summed).  All loads are unconditional, so the 16
  // row segments and the query values of a block are in flight together,
  // and the next block's loads run while this one is summed.
  const uint32_t my_row = valid ? row : 0u;
  const float *src[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) src[i] = x + (int64_t)__shfl(my_row, sub + 4 * i) * ldx;
  const int32_t cmax = ldx - 4;
  rr_f4 buf[16];
  float qb[4];  // query values of the block (rows have stride d, not padded)
  {
    const int32_t col = 4 * seg < cmax ? 4 * seg : cmax;
#pragma unroll
    for (int i = 0; i < 16; ++i) buf[i] = *reinterpret_cast<const rr_f4 *>(src[i] + col);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int32_t qc = 4 * seg + e;
      qb[e] = qr[qc < d ? qc : d - 1];
    }
  }
  for (int32_t j0 = 0; j0 < d; j0 += RR_W) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      *reinterpret_cast<rr_f4 *>(t + (sub + 4 * i) * RR_LD + 4 * seg) = buf[i];
    if (sub == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) t[64 * RR_LD + 4 * seg + e] = qb[e];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {
      // the next block (the last one reloads itself)
      const int32_t jnext = j0 + RR_W < d ? j0 + RR_W : j0;
      const int32_t col = jnext + 4 * seg < cmax ? jnext + 4 * seg : cmax;
#pragma unroll
      for (int i = 0; i < 16; ++i) buf[i] = *reinterpret_cast<const rr_f4 *>(src[i] + col);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int32_t qc = jnext + 4 * seg + e;
        qb[e] = qr[qc < d ? qc : d - 1];
      }
    }
    const int32_t jn = d - j0 < RR_W ? d - j0 : RR_W;
    const float *xr = t + lane * RR_LD, *qv = t + 64 * RR_LD;
    for (int32_t j = 0; j < jn; ++j) {
      const float a = qv[j], b = xr[j];
      if constexpr (METRIC == VSK_METRIC_L1) {
        s0 = s0 + fabsf(a - b);
      } else if constexpr (METRIC == VSK_METRIC_L2SQ || METRIC == VSK_METRIC_L2) {
        const float tt = a - b;
        s0 = s0 + tt * tt;
      } else if constexpr (METRIC == VSK_METRIC_COSINE) {
        s0 = s0 + a * b;
        s1 = s1 + a * a;
        s2 = s2 + b * b;
      } else {
        s0 = s0 + a * b;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  if (c >= kadc) return;
  if (!valid) {
    out[qi * kadc + c] = VSK_KEY_NONE;
    return;
  }
  float dist;
  if constexpr (METRIC == VSK_METRIC_L1 || METRIC == VSK_METRIC_L2SQ) {
    dist = s0;
  } else if constexpr (METRIC == VSK_METRIC_L2) {
    dist = sqrtf(s0);
  } else if constexpr (METRIC == VSK_METRIC_COSINE) {
    float den = sqrtf(s1) * sqrtf(s2);
    den = den + 1e-8f;
    dist = 1.0f - s0 / den;
  } else if constexpr (METRIC == VSK_METRIC_COSINE_NORMALIZED) {
    dist = 1.0f - s0;
  } else {
    dist = -s0;
  }
  out[qi * kadc + c] = vsk_key(dist, row);
}

static void launch_rerank(vsk_ctx *ctx, const uint64_t *best, int64_t nq, int32_t kadc,
                          const float *q, int32_t ldq, const float *x, int32_t ldx,
                          int32_t d, int32_t metric, uint64_t *out) {
  if (nq > 0x7FFFFFFF) fail(VSK_ERR_INVALID_BUFFER_SIZE, "too many queries");
  const dim3 grid((unsigned)nq, (unsigned)ceil_div(kadc, 256));
  switch (metric) {
#define RR_CASE(M)                                                                 \
  case M:                                                                          \
    k_rerank<M><<<grid, 256, 0, ctx->stream>>>(best, kadc, q, ldq, x, ldx, d, out); \
    break;
    RR_CASE(VSK_METRIC_L1)
    RR_CASE(VSK_METRIC_L2SQ)
    RR_CASE(VSK_METRIC_L2)
    RR_CASE(VSK_METRIC_COSINE)
    RR_CASE(VSK_METRIC_COSINE_NORMALIZED)
    RR_CASE(VSK_METRIC_DOT)
#undef RR_CASE
    default: fail(VSK_ERR_INVALID_ARGUMENT, "unknown re-rank metric");
  }
  check_launch("pq_rerank");
}

static void require_pq(const vsk_pq *pq) {
  VSK_REQUIRE(pq, VSK_ERR_INVALID_ARGUMENT, "pq is null");
}

// q (host or device, nq x d) -> device, stride d
static const float *pq_queries(vsk_ctx *ctx, const vsk_pq *pq, const float *q,
                               int64_t nq) {
  return static_cast<const float *>(
      input_to_device(ctx, q, sizeof(float) * nq * pq->d, "pq.q"));
}

static void pq_lut_device(vsk_ctx *ctx, const vsk_pq *pq, const float *dq,
                          int64_t nq, float *lut) {
  KernelTimer t(ctx, "pq_lut");
  const dim3 grid((unsigned)ceil_div(nq, PQL_QB), (unsigned)pq->M);
  const float *cb = pq->codebooks.as<float>();
  if (ceil_div(nq, PQL_QB) > 0x7FFFFFFF || pq->M > 65535)
    fail(VSK_ERR_INVALID_BUFFER_SIZE, "too many queries or segments");
  if (pq->ksub > 256) fail(VSK_ERR_INVALID_ARGUMENT, "codebooks hold at most 256 codewords");
  switch (pq->dsub) {
  case 1: k_pq_lut_seg<1><<<grid, 256, 0, ctx->stream>>>(dq, nq, pq->d, cb, pq->M, pq->ksub, lut); break;
  case 2: k_pq_lut_seg<2><<<grid, 256, 0, ctx->stream>>>(dq, nq, pq->d, cb, pq->M, pq->ksub, lut); break;
  case 4: k_pq_lut_seg<4><<<grid, 256, 0, ctx->stream>>>(dq, nq, pq->d, cb, pq->M, pq->ksub, lut); break;
  case 8: k_pq_lut_seg<8><<<grid, 256, 0, ctx->stream>>>(dq, nq, pq->d, cb, pq->M, pq->ksub, lut); break;
  case 16: k_pq_lut_seg<16><<<grid, 256, 0, ctx->stream>>>(dq, nq, pq->d, cb, pq->M, pq->ksub, lut); break;
  case 32: k_pq_lut_seg<32><<<grid, 256, 0, ctx->stream>>>(dq, nq, pq->d, cb, pq->M, pq->ksub, lut); break;
  default:
    k_pq_lut<<<grid1(nq * pq->M * pq->ksub), 256, 0, ctx->stream>>>(
        dq, nq, pq->d, cb, pq->M, pq->ksub, pq->dsub, lut);
  }
  check_launch("pq_lut");
}

}  // namespace vsk

using namespace vsk;

extern "C" {

vsk_status vsk_pq_create(vsk_ctx *ctx, const float *codebooks, int32_t M,
                         int32_t ksub, int32_t dsub, vsk_pq **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(codebooks, VSK_ERR_NOT_TRAINED, "no codebooks (not trained)");
  VSK_REQUIRE(M > 0 && dsub > 0, VSK_ERR_INVALID_ARGUMENT,
              "segments and segment dimension must be positive");
  VSK_REQUIRE(ksub >= 1 && ksub <= 256, VSK_ERR_INVALID_ARGUMENT,
              "codebook size must be in [1, 256] (8-bit codes)");
  VSK_REQUIRE((int64_t)PQ_QG * M * ksub * 4 <= 64 * 1024, VSK_ERR_UNSUPPORTED,
              "M * ksub too large for LDS-resident distance tables");
  std::unique_ptr<vsk_pq> pq(new vsk_pq());
  pq->M = M;
  pq->ksub = ksub;
  pq->dsub = dsub;
  pq->d = M * dsub;
  CallScope cs(ctx);
  const size_t bytes = sizeof(float) * (size_t)M * ksub * dsub;
  pq->codebooks.reserve(bytes);
  VSK_HIP(hipMemcpyAsync(pq->codebooks.p, codebooks, bytes, hipMemcpyDefault,
                         ctx->stream));
  pq->host_codebooks.resize((size_t)M * ksub * dsub);
  VSK_HIP(hipMemcpyAsync(pq->host_codebooks.data(), pq->codebooks.p, bytes,
                         hipMemcpyDeviceToHost, ctx->stream));
  cs.finish();
  *out = pq.release();
  VSK_API_END(ctx);
}

vsk_status vsk_pq_upload(vsk_ctx *ctx, const float *codebooks,
                         const uint8_t *codes, int64_t n, int32_t M,
                         int32_t dsub, vsk_pq **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(n >= 0, VSK_ERR_INVALID_ARGUMENT, "row count is negative");
  vsk_pq *pq = nullptr;
  vsk_status st = vsk_pq_create(ctx, codebooks, M, 256, dsub, &pq);
  if (st != VSK_OK) return st;
  if (n > 0) {
    st = vsk_pq_add_codes(ctx, pq, codes, n);
    if (st != VSK_OK) {
      vsk_pq_free(ctx, pq);  // keeps the add's message
      return st;
    }
  }
  *out = pq;
  VSK_API_END(ctx);
}

vsk_status vsk_pq_free(vsk_ctx *ctx, vsk_pq *pq) {
  if (ctx) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
  }
  delete pq;
  return VSK_OK;
}

vsk_status vsk_pq_encode(vsk_ctx *ctx, const vsk_pq *pq, const float *x,
                         int64_t n, uint8_t *codes) {
  VSK_API_BEGIN(ctx);
  require_pq(pq);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no vectors");
  VSK_REQUIRE(x && codes, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  CallScope cs(ctx);
  const float *dx = static_cast<const float *>(
      input_to_device(ctx, x, sizeof(float) * n * pq->d, "pq.x"));
  OutputStage oc(ctx, codes, (size_t)n * pq->M, "out.codes");
  launch_encode(ctx, pq, dx, n, oc.ptr<uint8_t>());
  oc.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_pq_decode(vsk_ctx *ctx, const vsk_pq *pq, const uint8_t *codes,
                         int64_t n, float *out) {
  VSK_API_BEGIN(ctx);
  require_pq(pq);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no codes");
  VSK_REQUIRE(codes && out, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  CallScope cs(ctx);
  const uint8_t *dc = static_cast<const uint8_t *>(
      input_to_device(ctx, codes, (size_t)n * pq->M, "pq.dcodes"));
  OutputStage ox(ctx, out, sizeof(float) * (size_t)n * pq->d, "out.decoded");
  {
    KernelTimer t(ctx, "pq_decode", (double)n);
    const int64_t total = n * pq->d;
    const int64_t g = ceil_div(total, 256);
    k_pq_decode<<<(unsigned)(g < 16384 ? (g > 0 ? g : 1) : 16384), 256, 0, ctx->stream>>>(
        dc, n, pq->codebooks.as<float>(), pq->M, pq->ksub, pq->dsub, ox.ptr<float>());
    check_launch("pq_decode");
  }
  ox.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

vsk_status vsk_pq_add_codes(vsk_ctx *ctx, vsk_pq *pq, const uint8_t *codes,
                            int64_t n) {
  VSK_API_BEGIN(ctx);
  require_pq(pq);
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "no codes");
  VSK_REQUIRE(codes, VSK_ERR_INVALID_ARGUMENT, "codes is null");
  VSK_REQUIRE(pq->n + n <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "a code database holds at most 2^31-1 rows");
  CallScope cs(ctx);
  const int64_t need = pq->n + n;
  if (need > pq->cap_rows) {
    int64_t cap = std::max<int64_t>(need, pq->cap_rows + pq->cap_rows / 2);
    auto nb = std::make_unique<DevBuf>();
    nb->reserve((size_t)cap * pq->M + 16);
    if (pq->n > 0)
      VSK_HIP(hipMemcpyAsync(nb->p, pq->codes.p, (size_t)pq->n * pq->M,
                             hipMemcpyDeviceToDevice, ctx->stream));
    stream_sync(ctx);
    std::swap(pq->codes.p, nb->p);
    std::swap(pq->codes.bytes, nb->bytes);
    pq->cap_rows = cap;
  }
  VSK_HIP(hipMemcpyAsync(pq->codes.as<uint8_t>() + pq->n * pq->M, codes,
                         (size_t)n * pq->M, hipMemcpyDefault, ctx->stream));
  cs.finish();
  pq->n = need;
  VSK_API_END(ctx);
}

vsk_status vsk_pq_lut(vsk_ctx *ctx, const vsk_pq *pq, const float *q,
                      int64_t nq, float *lut) {
  VSK_API_BEGIN(ctx);
  require_pq(pq);
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(q && lut, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  CallScope cs(ctx);
  const float *dq = pq_queries(ctx, pq, q, nq);
  OutputStage ol(ctx, lut, sizeof(float) * nq * pq->M * pq->ksub, "out.lut");
  pq_lut_device(ctx, pq, dq, nq, ol.ptr<float>());
  ol.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

static vsk_status pq_search_body(vsk_ctx *ctx, const vsk_pq *pq, const float *q,
                         int64_t nq, int32_t k_adc, int32_t k,
                         int32_t rerank_metric, const vsk_db *rerank_db,
                         float *out_dist, int64_t *out_ids) {
  VSK_API_BEGIN(ctx);
  require_pq(pq);
  VSK_REQUIRE(nq > 0, VSK_ERR_EMPTY_INPUT, "no queries");
  VSK_REQUIRE(pq->n > 0, VSK_ERR_EMPTY_INPUT, "no codes added");
  VSK_REQUIRE(q && out_dist && out_ids, VSK_ERR_INVALID_ARGUMENT,
              "null buffer");
  VSK_REQUIRE(k >= 1 && k_adc >= 1, VSK_ERR_INVALID_ARGUMENT,
              "k and k_adc must be >= 1");
  VSK_REQUIRE(k <= VSK_MAX_K && k_adc <= VSK_MAX_K,
              VSK_ERR_INVALID_BUFFER_SIZE, "k exceeds VSK_MAX_K");
  const bool rerank = rerank_db && rerank_metric >= 0;
  if (rerank) {
    VSK_REQUIRE(metric_valid(rerank_metric), VSK_ERR_INVALID_ARGUMENT,
                "unknown re-rank metric");
    VSK_REQUIRE(rerank_metric != VSK_METRIC_HAMMING, VSK_ERR_UNSUPPORTED,
                "the re-rank has no hamming metric");
    VSK_REQUIRE(rerank_db->d == pq->d, VSK_ERR_DIMENSION_MISMATCH,
                "re-rank rows have another dimension");
    VSK_REQUIRE(rerank_db->n >= pq->n, VSK_ERR_DIMENSION_MISMATCH,
                "re-rank rows do not cover every code row");
  }
  VSK_REQUIRE(nq <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "too many queries");
  CallScope cs(ctx);
  const float *dq = pq_queries(ctx, pq, q, nq);
  float *lut = static_cast<float *>(
      ctx->scratch_ptr("pq.lut", sizeof(float) * nq * pq->M * pq->ksub));
  pq_lut_device(ctx, pq, dq, nq, lut);
  uint64_t *best = static_cast<uint64_t *>(
      ctx->scratch_ptr("pq.best", sizeof(uint64_t) * nq * k_adc));
  // the bf16 screen: decoded rows (kept with the codes), the queries' bf16
  // plane and norms, a threshold slot per query.  Its chunks grow at most
  // 4-8x: the survivors (k_adc times the growth, plus the bound's band) then
  // stay well inside the screen's 256 slots per (row split, query), whose
  // overflow costs a dense re-scan (measured at config 5: 8,192 slots,
  // growth 4, 2 % faster than 16,384 and growth 8)
  const bool screen = pq_screen_applies(ctx, pq, nq);
  const int64_t cap = screen ? std::max<int64_t>(default_cap(k_adc) / 2, 4 * (int64_t)k_adc)
                             : default_cap(k_adc);
  const int64_t qb = query_batch(ctx, nq, cap);
  ArgminQueries qp;
  uint64_t *sthr = nullptr;
  if (screen) {
    pq_screen_plane(ctx, pq);
    qp = argmin_queries(ctx, dq, nq, pq->d, pq->d, "pq.sq");
    sthr = static_cast<uint64_t *>(ctx->scratch_ptr("pq.sthr", sizeof(uint64_t) * nq));
  }
  for (int64_t b0 = 0; b0 < nq; b0 += qb) {
    const int64_t nb = nq - b0 < qb ? nq - b0 : qb;
    AdcArgs base{};
    base.codes = pq->codes.as<uint8_t>();
    base.M = pq->M;
    base.ksub = pq->ksub;
    base.lut = lut + b0 * pq->M * pq->ksub;
    base.nq = (int32_t)nb;
    ScanFn scan = [&](const ScanRequest &r) {
      if (!r.dense && screen) {
        // filtered chunks: the bf16 screen over the decoded rows, then the
        // survivors' exact keys
        k_pq_screen_thresh<<<(unsigned)ceil_div(nb, 256), 256, 0, ctx->stream>>>(
            r.thresh, nb, qp.qnh + b0, qp.qnr + b0, pq->xh_max, pq->xr_max, pq->d, sthr);
        check_launch("pq_screen_thresh");
        FlatArgs f{};
        f.xaux = pq->xsq.as<float>();
        f.qaux = qp.qsq + b0;
        f.kdim = pq->xldb;
        f.nq = (int32_t)nb;
        f.r0 = r.r0;
        f.r1 = r.r1;
        f.metric = VSK_METRIC_L2SQ;
        f.thresh = sthr;
        f.active = r.active;
        f.cand = r.cand;
        f.cap = r.cap;
        f.counts = r.counts;
        f.seg_n = r.seg_n;
        SplitPtrs sp{};
        sp.xh = pq->xplane.as<uint16_t>();
        sp.qh = qp.qh + b0 * qp.ldb;
        sp.ldxb = pq->xldb;
        sp.ldqb = qp.ldb;
        sp.kb = pq->xldb;
        int32_t nseg = 0;
        int64_t stride = 0;
        launch_flat_screen(ctx, f, sp, MODE_FILTER, r.seg_n ? &nseg : nullptr,
                           r.seg_n ? &stride : nullptr);
        if (r.seg_nseg) *r.seg_nseg = nseg;
        if (r.seg_stride) *r.seg_stride = stride;
        {
          KernelTimer t(ctx, "pq_screen_rescore");
          const size_t lds = sizeof(float) * pq->M * pq->ksub;
          const int32_t *sn = nseg > 0 ? r.seg_n : nullptr;
          const uint8_t *cd = pq->codes.as<uint8_t>();
#define PQ_RESCORE(MM)                                                                  \
  k_pq_rescore_keys<MM><<<(unsigned)nb, 256, lds, ctx->stream>>>(                       \
      cd, pq->ksub, base.lut, r.thresh, r.active, r.cand, r.cap, r.counts, sn, nseg, stride)
          switch (pq->M) {
          case 1: PQ_RESCORE(1); break;
          case 2: PQ_RESCORE(2); break;
          case 4: PQ_RESCORE(4); break;
          case 8: PQ_RESCORE(8); break;
          case 16: PQ_RESCORE(16); break;
          case 32: PQ_RESCORE(32); break;
          default: PQ_RESCORE(64); break;
          }
#undef PQ_RESCORE
          check_launch("pq_screen_rescore");
        }
        return;
      }
      AdcArgs a = base;
      a.r0 = r.r0;
      a.r1 = r.r1;
      a.thresh = r.thresh;
      a.active = r.active;
      a.cand = r.cand;
      a.cap = r.cap;
      a.counts = r.counts;
      if (pq->M == 16 && pq->ksub == 256)
        launch_adc16(ctx, a, r.dense);
      else
        launch_adc(ctx, a, r.dense);
    };
    progressive_topk(ctx, nb, pq->n, k_adc, cap, scan, best + b0 * k_adc,
                     "pq_select", screen ? 8 : 0);
  }
  OutputStage od(ctx, out_dist, sizeof(float) * nq * k, "out.dist");
  OutputStage oi(ctx, out_ids, sizeof(int64_t) * nq * k, "out.ids");
  if (rerank) {
    uint64_t *rk = static_cast<uint64_t *>(
        ctx->scratch_ptr("pq.rerank", sizeof(uint64_t) * nq * k_adc));
    {
      KernelTimer t(ctx, "pq_rerank");
      launch_rerank(ctx, best, nq, k_adc, dq, pq->d, rerank_db->x.as<float>(),
                    rerank_db->ld, pq->d, rerank_metric, rk);
    }
    uint64_t *fin = static_cast<uint64_t *>(
        ctx->scratch_ptr("pq.final", sizeof(uint64_t) * nq * k));
    SelectArgs sa;
    sa.nq = nq;
    sa.k = k;
    sa.cand = rk;
    sa.cap = k_adc;
    sa.best_out = fin;
    launch_select(ctx, sa, "pq_rerank_select");
    decode_keys(ctx, fin, nq * (int64_t)k, false, nullptr, od.ptr<float>(),
                oi.ptr<int64_t>());
  } else if (k <= k_adc) {
    uint64_t *fin = static_cast<uint64_t *>(
        ctx->scratch_ptr("pq.final", sizeof(uint64_t) * nq * k));
    SelectArgs sa;  // first k of the sorted ADC list
    sa.nq = nq;
    sa.k = k;
    sa.cand = best;
    sa.cap = k_adc;
    sa.best_out = fin;
    launch_select(ctx, sa, "pq_rerank_select");
    decode_keys(ctx, fin, nq * (int64_t)k, true, nullptr, od.ptr<float>(),
                oi.ptr<int64_t>());
  } else {
    fail(VSK_ERR_INVALID_ARGUMENT, "k > k_adc needs a re-rank database");
  }
  od.copy_back();
  oi.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

// top-k overflow is checked at the call's end (topk_call)
vsk_status vsk_pq_search(vsk_ctx *ctx, const vsk_pq *pq, const float *q,
                         int64_t nq, int32_t k_adc, int32_t k,
                         int32_t rerank_metric, const vsk_db *rerank_db,
                         float *out_dist, int64_t *out_ids) {
  return topk_call(ctx, [&] { return pq_search_body(ctx, pq, q, nq, k_adc, k, rerank_metric, rerank_db, out_dist, out_ids); });
}

}  // extern "C"

namespace vsk {

int32_t pq_shape(const vsk_pq *pq, int32_t *M, int32_t *ksub) {
  *M = pq->M;
  *ksub = pq->ksub;
  return pq->d;
}

bool pq_shape_matches(const vsk_pq *pq, int32_t d, int32_t M, int32_t ksub) {
  return pq && pq->d == d && pq->M == M && pq->ksub == ksub;
}

const std::vector<float> &pq_host_codebooks(const vsk_pq *pq, int32_t *dsub) {
  *dsub = pq->dsub;
  return pq->host_codebooks;
}

}  // namespace vsk
