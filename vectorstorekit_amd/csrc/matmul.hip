// matrixMultiply (Acceleration/MetalAccelerationEngine.swift:209-229) on the
// VALU: c = a . b with every entry summed over the inner dimension in order
// from 0, a product and then a sum (no FMA), as the reference's CPU loop
// adds it (Acceleration/Metal/MetalMatrixCompute.swift:791-806).  The MPS
// path of the reference leaves its summation order unspecified; this order
// makes the result the oracle's bit for bit.
//
// A workgroup of 256 threads owns a 64 x 64 tile of c; thread (ty, tx) owns
// rows 4 ty .. 4 ty + 3 and columns 4 tx .. 4 tx + 3, 16 running sums.  The
// inner dimension goes in steps of 32: the step's 64 x 32 block of a is
// stored transposed in LDS (t-major, so a thread's four rows are one 16-byte
// read) and the 32 x 64 block of b as is (a thread's four columns are one
// 16-byte read, the 16 threads of a row of the tile reading 256 contiguous
// bytes).  Per t: two LDS reads, 16 multiplies, 16 adds.  Entries past m, n
// or k read 0: a sum that starts at +0 never becomes -0 when 0 * 0 is
// added, so the padding changes no result.
#include "vsk_api.hpp"

namespace vsk {
namespace {

constexpr int MM_T = 64;        // tile rows and columns
constexpr int MM_K = 32;        // inner step
constexpr int MM_LDA = MM_T + 4;  // padded row of the transposed a block

__global__ __launch_bounds__(256) void k_matmul_seq(const float *__restrict__ A,
                                                    const float *__restrict__ B,
                                                    float *__restrict__ C, int64_t m,
                                                    int32_t k, int64_t n,
                                                    int64_t tiles_n, int64_t tiles) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float sa[MM_K * MM_LDA];
  __shared__ __attribute__((aligned(16))) float sb[MM_K * MM_T];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int64_t r0 = (tile / tiles_n) * MM_T, c0 = (tile % tiles_n) * MM_T;
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[r][c] = 0.f;
    for (int32_t t0 = 0; t0 < k; t0 += MM_K) {
      // a block: element e = tid + 256 i is row e / 32, column e % 32 (a
      // row's 32 floats are 128 contiguous bytes)
#pragma unroll
      for (int i = 0; i < MM_T * MM_K / 256; ++i) {
        const int e = tid + 256 * i;
        const int rr = e >> 5, tt = e & 31;
        const int64_t row = r0 + rr;
        const int32_t t = t0 + tt;
        sa[tt * MM_LDA + rr] = (row < m && t < k) ? A[row * k + t] : 0.f;
      }
      // b block: element e is row e / 64, column e % 64
#pragma unroll
      for (int i = 0; i < MM_T * MM_K / 256; ++i) {
        const int e = tid + 256 * i;
        const int tt = e >> 6, cc = e & 63;
        const int32_t t = t0 + tt;
        const int64_t col = c0 + cc;
        sb[tt * MM_T + cc] = (t < k && col < n) ? B[(int64_t)t * n + col] : 0.f;
      }
      __syncthreads();
#pragma unroll 8
      for (int tt = 0; tt < MM_K; ++tt) {
        const float4 av = *reinterpret_cast<const float4 *>(sa + tt * MM_LDA + 4 * ty);
        const float4 bv = *reinterpret_cast<const float4 *>(sb + tt * MM_T + 4 * tx);
        const float a4[4] = {av.x, av.y, av.z, av.w};
        const float b4[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float p = a4[r] * b4[c];
            acc[r][c] = acc[r][c] + p;
          }
      }
      __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = r0 + 4 * ty + r;
      if (row >= m) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t col = c0 + 4 * tx + c;
        if (col < n) C[row * n + col] = acc[r][c];
      }
    }
  }
}

}  // namespace
}  // namespace vsk

using namespace vsk;

extern "C" {

vsk_status vsk_matrix_multiply(vsk_ctx *ctx, const float *a, int64_t m, int32_t k,
                               const float *b, int64_t n, float *c) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(a && b && c, VSK_ERR_INVALID_ARGUMENT, "null buffer");
  VSK_REQUIRE(m >= 0 && k >= 0 && n >= 0, VSK_ERR_INVALID_ARGUMENT, "negative dimension");
  VSK_REQUIRE(m > 0 && k > 0 && n > 0, VSK_ERR_EMPTY_INPUT, "empty matrix");
  VSK_REQUIRE(m <= (int64_t)1 << 40 && n <= (int64_t)1 << 40, VSK_ERR_INVALID_BUFFER_SIZE,
              "matrix too large");
  CallScope cs(ctx);
  const float *da = static_cast<const float *>(
      input_to_device(ctx, a, sizeof(float) * (size_t)m * (size_t)k, "mm.a"));
  const float *db = static_cast<const float *>(
      input_to_device(ctx, b, sizeof(float) * (size_t)k * (size_t)n, "mm.b"));
  OutputStage oc(ctx, c, sizeof(float) * (size_t)m * (size_t)n, "out.mm");
  const int64_t tiles_n = ceil_div(n, MM_T);
  const int64_t tiles = ceil_div(m, MM_T) * tiles_n;
  const int64_t grid = tiles < 65536 ? tiles : 65536;
  {
    KernelTimer t(ctx, "matmul_seq", (double)m * (double)n * (double)k);
    k_matmul_seq<<<(unsigned)grid, 256, 0, ctx->stream>>>(da, db, oc.ptr<float>(), m, k, n,
                                                          tiles_n, tiles);
    check_launch("matmul_seq");
  }
  oc.copy_back();
  cs.finish();
  VSK_API_END(ctx);
}

}  // extern "C"
