// sort.hip -- segmented sort of 64-bit keys (rocPRIM's segmented radix
// sort), for the IVF probe that ranks every centroid of a query.
#include "flat.hpp"

#include <rocprim/device/device_segmented_radix_sort.hpp>

namespace vsk {

// segment offsets s * len, s = 0..nseg
__global__ void k_segment_offsets(int64_t *off, int64_t nseg, int64_t len) {
  const int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (s <= nseg) off[s] = s * len;
}

void segmented_sort_u64(vsk_ctx *ctx, const uint64_t *in, uint64_t *out, int64_t nseg,
                        int64_t len) {
  if (nseg <= 0 || len <= 0) return;
  if (nseg * len > (int64_t)INT32_MAX)
    fail(VSK_ERR_INVALID_BUFFER_SIZE, "segmented sort: more than 2^31 - 1 keys");
  int64_t *off = static_cast<int64_t *>(
      ctx->scratch_ptr("sort.off", sizeof(int64_t) * (size_t)(nseg + 1)));
  k_segment_offsets<<<(unsigned)ceil_div(nseg + 1, 256), 256, 0, ctx->stream>>>(off, nseg,
                                                                               len);
  check_launch("segment_offsets");
  size_t bytes = 0;
  VSK_HIP(rocprim::segmented_radix_sort_keys(
      nullptr, bytes, in, out, (unsigned)(nseg * len), (unsigned)nseg, off, off + 1, 0, 64,
      ctx->stream));
  void *tmp = ctx->scratch_ptr("sort.tmp", bytes);
  KernelTimer t(ctx, "segmented_sort");
  VSK_HIP(rocprim::segmented_radix_sort_keys(
      tmp, bytes, in, out, (unsigned)(nseg * len), (unsigned)nseg, off, off + 1, 0, 64, ctx->stream));
  check_launch("segmented_sort");
}

}  // namespace vsk
