// peaks.hip -- measured ceilings of this GPU for the rooflines the bench
// reports: dense bf16 and int8 matrix-core rates, and HBM copy bandwidth.
// Each is timed with HIP events on the context's stream over a few hundred
// milliseconds of work at most.  The bandwidths are what kernels here can
// reach, well under the 8 TB/s datasheet figure (about 5.1 TB/s copying
// and 5.7 TB/s reading on the MI355X boxes used).
//
// The MFMA loops run two waves per SIMD (at most 256 registers each, so the
// accumulators stay in VGPRs) and keep 32 (bf16) and 16 (int8) independent accumulators per
// wave: with 8, a k-step that adds to a result issued 8 multiplies earlier
// stalls the matrix pipe (measured: int8 2.6 POP/s with 8 chains, 4.3 with
// 16).  Operands stay in registers; every accumulator feeds the stored
// checksum, so no multiply is dead code.  The copy streams 2 GiB through
// 16-byte loads and stores (bytes read plus bytes written over its time),
// the read pass the same 2 GiB.
#include "vsk_api.hpp"

namespace vsk {
namespace {

typedef float pk_f4 __attribute__((ext_vector_type(4)));
typedef int pk_i4 __attribute__((ext_vector_type(4)));
typedef __bf16 pk_bf8 __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_peak_bf16(int iters, float *out) {
  const int lane = threadIdx.x & 63;
  pk_bf8 a[4], b[8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) a[i][e] = (__bf16)(float)((lane + i + e) & 7);
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) b[j][e] = (__bf16)(float)((j + e) & 3);
  pk_f4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = pk_f4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_peak_i8(int iters, int *out) {
  const int lane = threadIdx.x & 63;
  pk_i4 a[2], b[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) a[i] = pk_i4{lane + i, 1, 2, 3};
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = pk_i4{j, lane, 3, 1};
  pk_i4 acc[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = pk_i4{0, 0, 0, 0};
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  int s = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// four 16-byte loads in flight per thread before their stores, both
// non-temporal (n is a multiple of 4 * 256 * gridDim.x, so every access is
// in bounds).  Measured on
// MI355X: 5.1 TB/s; cached accesses reach 4.5 TB/s, with one load in
// flight per thread or four.
typedef unsigned pk_u4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_peak_copy(const pk_u4 *src, pk_u4 *dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += 4 * stride) {
    pk_u4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < 4; ++u) __builtin_nontemporal_store(v[u], dst + i + u * stride);
  }
}

// reads only: four 16-byte loads in flight per thread, folded into a value
// that is stored only if it matches a constant (so the loads stay live)
__global__ __launch_bounds__(256) void k_peak_read(const pk_u4 *src, int64_t n, unsigned *out) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  unsigned x = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += 4 * stride) {
    const pk_u4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    x ^= a[0] ^ b[1] ^ c[2] ^ d[3];
  }
  if (x == 0x9E3779B9u) out[blockIdx.x] = x;
}

}  // namespace
}  // namespace vsk

using namespace vsk;

extern "C" vsk_status vsk_measure_peaks(vsk_ctx *ctx, vsk_peaks *out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  hipDeviceProp_t p;
  VSK_HIP(hipGetDeviceProperties(&p, ctx->device));
  // 8 waves per CU (two 256-thread workgroups), four rounds of them
  const int blocks = p.multiProcessorCount * 2 * 4;
  const int64_t copy_bytes = (int64_t)1 << 31;
  DevBuf sink, src, dst;
  sink.reserve((size_t)blocks * 256 * 4);
  src.reserve((size_t)copy_bytes);
  dst.reserve((size_t)copy_bytes);
  VSK_HIP(hipMemsetAsync(src.p, 1, (size_t)copy_bytes, ctx->stream));
  struct Events {
    hipEvent_t a = nullptr, b = nullptr;
    ~Events() {
      if (a) (void)hipEventDestroy(a);
      if (b) (void)hipEventDestroy(b);
    }
  } ev;
  VSK_HIP(hipEventCreate(&ev.a));
  VSK_HIP(hipEventCreate(&ev.b));
  hipEvent_t e0 = ev.a, e1 = ev.b;
  // the best of three timed launches after one warm-up
  auto time_ms = [&](auto launch) {
    launch();
    float best = 1e30f;
    for (int r = 0; r < 3; ++r) {
      VSK_HIP(hipEventRecord(e0, ctx->stream));
      launch();
      VSK_HIP(hipEventRecord(e1, ctx->stream));
      VSK_HIP(hipEventSynchronize(e1));
      float ms = 0.f;
      VSK_HIP(hipEventElapsedTime(&ms, e0, e1));
      if (ms < best) best = ms;
    }
    return (double)best;
  };
  const int iters = 2000;
  const double waves = blocks * 4.0;
  const double tb = time_ms([&] {
    k_peak_bf16<<<blocks, 256, 0, ctx->stream>>>(iters, sink.as<float>());
  });
  out->bf16_tflops = waves * iters * 32 * (2.0 * 16 * 16 * 32) / (tb * 1e9);
  const double ti = time_ms([&] {
    k_peak_i8<<<blocks, 256, 0, ctx->stream>>>(iters, sink.as<int>());
  });
  out->int8_tops = waves * iters * 16 * (2.0 * 16 * 16 * 64) / (ti * 1e9);
  // the copied span: a whole number of the grid's 4-load steps
  const int cgrid = p.multiProcessorCount * 32;
  const int64_t unit = 4 * 256 * (int64_t)cgrid;
  const int64_t n16 = copy_bytes / 16 / unit * unit;
  const double moved = 16.0 * (double)n16;
  const double tc = time_ms([&] {
    k_peak_copy<<<cgrid, 256, 0, ctx->stream>>>(src.as<pk_u4>(), dst.as<pk_u4>(), n16);
  });
  out->hbm_gbs = 2.0 * moved / (tc * 1e6);
  const double tr = time_ms([&] {
    k_peak_read<<<cgrid, 256, 0, ctx->stream>>>(src.as<pk_u4>(), n16, sink.as<unsigned>());
  });
  out->hbm_read_gbs = moved / (tr * 1e6);
  check_launch("measure_peaks");
  VSK_API_END(ctx);
}
