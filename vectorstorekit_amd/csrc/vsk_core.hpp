// vsk_core.hpp -- context, errors, device buffers and the composite
// (distance, tie) key shared by every kernel of the library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "vsk_hip.h"

namespace vsk {

// ---------------------------------------------------------------------------
// errors: every internal failure throws Error; the C entry points catch it,
// store the message on the context and return the code.
// ---------------------------------------------------------------------------
struct Error {
  vsk_status code;
  std::string msg;
};

[[noreturn]] void fail(vsk_status code, const std::string &msg);
void check_hip(hipError_t e, const char *what, const char *file, int line);
// Fault injection from the host (VSK_FAULT=alloc:<n>, launch:<n> or
// sync:<n>, read when a context is created): the n-th device allocation,
// kernel launch check or end-of-call synchronisation of that context fails
// as HIP would report it (out of memory; execution failed), once.  The
// kernels themselves run normally; only the report is forced, so error
// mapping and recovery can be tested without faulting the GPU.
enum FaultKind { FAULT_NONE = 0, FAULT_ALLOC = 1, FAULT_LAUNCH = 2, FAULT_SYNC = 3 };
void fault_point(int kind);
}  // namespace vsk
struct vsk_ctx;
namespace vsk {
// the context whose API call runs on this thread (fault counting), for the
// duration of the call: no other code sees a context that may since have
// been destroyed
vsk_ctx *set_fault_ctx(vsk_ctx *c);  // returns the previous one
struct FaultCtxScope {
  vsk_ctx *prev;  // an enclosing API call's context (nested calls)
  explicit FaultCtxScope(vsk_ctx *c) : prev(set_fault_ctx(c)) {}
  ~FaultCtxScope() { set_fault_ctx(prev); }
  FaultCtxScope(const FaultCtxScope &) = delete;
  FaultCtxScope &operator=(const FaultCtxScope &) = delete;
};
#define VSK_HIP(expr) ::vsk::check_hip((expr), #expr, __FILE__, __LINE__)
#define VSK_REQUIRE(cond, code, msg)                                          \
  do {                                                                        \
    if (!(cond)) ::vsk::fail((code), (msg));                                   \
  } while (0)

// ---------------------------------------------------------------------------
// device memory
// ---------------------------------------------------------------------------
struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  ~DevBuf();
  void reserve(size_t b);  // grow (contents not kept)
  void release();
  template <class T> T *as() const { return static_cast<T *>(p); }
};

bool is_device_ptr(const void *p);

}  // namespace vsk

// ---------------------------------------------------------------------------
// context (one HIP stream; per-call scratch slots; event profiling)
// ---------------------------------------------------------------------------
struct vsk_ctx {
  int device = 0;
  int cu_count = 256;  // compute units of the device
  hipStream_t stream = nullptr;
  // a second stream for work a call overlaps with its own kernels (created
  // on first use, default priority; every call still returns synchronised)
  hipStream_t aux = nullptr;
  hipStream_t aux_stream();
  // a small pinned host buffer for asynchronous read-backs (grown on use)
  void *pinned = nullptr;
  size_t pinned_bytes = 0;
  void *pinned_ptr(size_t bytes);
  std::string last_error;
  float last_ms = 0.f;
  hipEvent_t call_begin = nullptr, call_end = nullptr;

  // scratch buffers, reused across calls, keyed by purpose
  std::map<std::string, std::unique_ptr<vsk::DevBuf>> scratch;
  void *scratch_ptr(const std::string &key, size_t bytes);

  // flat top-k path, from the environment VSK_FLAT_KERNEL at context
  // creation: unset = one-pass bf16 screen with exact fp32 rescore where the
  // metric allows it (the exact sequential scan alone for small problems,
  // bf16x3 elsewhere); "screen" = the screen at every size; "bf16x3" =
  // bf16x3 split MFMA only; "fp32" = fp32 MFMA only
  bool flat_fp32 = false;
  bool flat_no_screen = false;
  bool flat_force_screen = false;
  // VSK_MAX_TILE_BYTES: the largest working buffer a query batch may take
  // (candidate keys and words); searches split their queries into batches
  // under it, as MetalDistanceCompute chunks queries under its buffer limit
  // (Acceleration/Metal/MetalDistanceCompute.swift:371-380, 450-473).  0:
  // the defaults (2 GiB of candidate keys, at least 64 queries a batch)
  int64_t max_tile_bytes = 0;
  // "exact": no bf16 screen anywhere -- the exact scans alone (flat search
  // on the exact VALU kernel for its screenable metrics, IVF's exact probe
  // and list scans, PQ's LUT scan over the codes, the exact argmin)
  bool exact_only = false;
  // VSK_IVF_COMPACT=0: the screened IVF list scan keeps every candidate's
  // word at its position instead of the candidates under each query's
  // bound, compacted (the two give the same results)
  bool ivf_no_compact = false;
  // VSK_FAULT: the kind of event to fail, at which occurrence, seen so far
  int fault_kind = 0;
  int64_t fault_at = 0, fault_seen = 0;

  // Top-k overflow without a read-back per chunk (progressive_topk): unless
  // topk_sync is set, a filtered chunk whose survivors overflow a query's
  // slots only counts into ovf_dev (the query keeps its earlier list, so
  // later work stays well defined); CallScope::finish reads the count with
  // the call's final synchronisation into topk_overflowed, and the entry
  // point then runs the call again with topk_sync (a check after each
  // chunk, and the overflowing queries re-scan it in sub-chunks).  Both
  // buffers are made with the context, so no call allocates them.
  int32_t *ovf_dev = nullptr;   // device counter
  int32_t *ovf_host = nullptr;  // pinned copy (8 ints: [0] the count)
  bool ovf_armed = false;       // ovf_dev cleared for this call
  bool topk_sync = false;
  bool topk_overflowed = false;
  // host waits for the stream in the current (outermost) API call
  int32_t sync_count = 0;

  // queries the last vsk_search_flat redid in the screen's fallback tiers
  // (indices into that call's queries, ascending): [0] the wider screen,
  // [1] the exact scan over every row
  std::vector<int64_t> screen_redo[2];

  // profiling
  bool profile = false;
  // when not empty, only the timers of these names record (and no work
  // count is read back from the device)
  std::vector<std::string> profile_only;
  bool timed(const char *name) const {
    if (!profile) return false;
    if (profile_only.empty()) return true;
    for (const auto &s : profile_only)
      if (s == name) return true;
    return false;
  }
  // device-side work counters are kept only under full profiling
  bool count_work() const { return profile && profile_only.empty(); }
  struct Pending {
    int stat;
    hipEvent_t a, b;
    double work;
    int work_slot;  // >= 0: the work count read back into work_pinned[slot]
  };
  // pinned slots for work counts the device computes (profiling only)
  static constexpr int kWorkSlots = 1024;
  int64_t *work_pinned = nullptr;
  int work_used = 0;
  std::vector<Pending> pending;
  std::vector<hipEvent_t> event_pool;
  // the kernel timers' events: timing only, recorded without the system-scope
  // fence (no cache write-back and invalidation between the timed kernels);
  // read after the call's stream synchronisation
  std::vector<hipEvent_t> timer_pool;
  std::vector<vsk_kernel_stat> stats;
  std::map<std::string, int> stat_index;
  hipEvent_t take_event();
  hipEvent_t take_timer_event();
  void resolve_pending();
  // the pending timings of a call that failed: their events back to the
  // pool, unread
  void drop_pending();
};

struct vsk_db {
  int64_t n = 0;
  int32_t d = 0;
  int32_t ld = 0;  // row stride in floats (multiple of 4, >= d; zero padded)
  vsk::DevBuf x;       // n x ld fp32
  vsk::DevBuf sqnorm;  // n: sum x^2 (fp32)
  vsk::DevBuf norm;    // n: sqrt(sum x^2)
  // bf16 hi/lo planes for the bf16 MFMA kernels, built on first use (the
  // lo plane only for the bf16x3 kernel; the screen reads hi alone), and
  // the maxima over the rows of |hi| and |x - hi| (the screen's bound)
  mutable vsk::DevBuf split, split_lo;
  // the reference's |x| per row (seq_norms), built when the exact cosine
  // first needs it
  mutable vsk::DevBuf seqnorm;
  // the screen's bound for cosine: maxima over the rows with 0 < |x| of
  // |bf16(x)| / |x| and |x - bf16(x)| / |x| (|x| the fp32 norm above);
  // cos_state 0 = not made, 1 = made, -1 = a row's norm is too small or not
  // finite for the bound (cosine then takes the exact scan)
  mutable int32_t cos_state = 0;
  mutable float cos_rel_hi = 0.f, cos_rel_res = 0.f;
  mutable int32_t ldb = 0;
  mutable float split_max_hi = 0.f, split_max_res = 0.f;
};

namespace vsk {

// RAII marker for one API call: records the call's begin/end events,
// synchronises the stream at the end and resolves profiling events.
struct CallScope {
  vsk_ctx *ctx;
  explicit CallScope(vsk_ctx *c);
  void finish();  // sync + timing; call before returning results
};

// Runs an API entry point's body with deferred top-k overflow checks (see
// vsk_ctx::topk_sync); when a query overflowed, the body runs once more
// with a check after every chunk.  Nested calls leave the decision to the
// outermost one.
template <class F> vsk_status topk_call(vsk_ctx *ctx, F &&body) {
  if (!ctx) return VSK_ERR_INVALID_ARGUMENT;
  if (ctx->topk_sync) return body();
  ctx->topk_overflowed = false;
  vsk_status st = body();
  if (st == VSK_OK && ctx->topk_overflowed) {
    const int32_t waits = ctx->sync_count;  // (the second run counts afresh)
    ctx->topk_overflowed = false;
    ctx->topk_sync = true;
    st = body();
    ctx->topk_sync = false;
    ctx->sync_count += waits;
  }
  ctx->topk_overflowed = false;
  return st;
}

// Times one kernel launch when profiling is on.
struct KernelTimer {
  vsk_ctx *ctx;
  int stat = -1;
  hipEvent_t a = nullptr;
  double work = 0;
  hipStream_t stream = nullptr;
  // times on stream s (default: the context's stream)
  const int64_t *work_dev = nullptr;
  KernelTimer(vsk_ctx *c, const char *name, double work_items = 0, hipStream_t s = nullptr);
  // the work count is a device value, final once the timed launch ends
  void device_work(const int64_t *p) { work_dev = p; }
  ~KernelTimer();
};

// check the last launch on the stream
void check_launch(const char *name);
// the host waits for the context's stream (counted per API call)
void stream_sync(vsk_ctx *ctx);

// staging of caller buffers: a device pointer is used as is, a host
// pointer is copied through a scratch slot.
const void *input_to_device(vsk_ctx *ctx, const void *p, size_t bytes,
                            const std::string &slot);
struct OutputStage {
  vsk_ctx *ctx;
  void *user;
  void *dev;
  size_t bytes;
  bool host;
  OutputStage(vsk_ctx *c, void *user_ptr, size_t nbytes,
              const std::string &slot);
  template <class T> T *ptr() const { return static_cast<T *>(dev); }
  void copy_back();  // enqueue device->host copy when user is host memory
};

// rows x row_bytes from src (row pitch src_pitch) to dst (dst_pitch) on the
// context's stream; either side may be host memory.  A host side moves in
// whole chunks through a device staging slot and the pitch change runs as a
// device-to-device copy, so narrow rows never become one transfer per row.
void copy_rows(vsk_ctx *ctx, void *dst, size_t dst_pitch, const void *src,
               size_t src_pitch, size_t row_bytes, int64_t rows);

// pad rows of a (rows x d) fp32 matrix to stride ld on the device
const float *rows_to_device_padded(vsk_ctx *ctx, const float *p, int64_t rows,
                                   int32_t d, int32_t ld,
                                   const std::string &slot);

inline int32_t padded_ld(int32_t d) { return (d + 3) & ~3; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool metric_valid(int32_t m);

// fill kernels (used instead of hipMemsetAsync so callers may capture the
// stream into a graph)
void fill_u64(vsk_ctx *ctx, uint64_t *p, int64_t n, uint64_t v);
void fill_i32(vsk_ctx *ctx, int32_t *p, int64_t n, int32_t v);

// row norms of an (n x ld) matrix over its first d columns:
// sq[i] = sum x^2 (fp32), nrm[i] = sqrt(sq[i]); either may be null.
void row_norms(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
               float *sq, float *nrm);
// norms[i] = sqrtf of the squares of row i summed in dimension order without
// FMA: the |x| of the reference's cosine, bit for bit
void seq_norms(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
               float *norms);

}  // namespace vsk

// ---------------------------------------------------------------------------
// composite sort key: (distance, tie) packed in a uint64 whose unsigned order
// equals ascending distance then ascending tie key.  The distance's fp32
// bits are mapped to an order-preserving uint32 (negatives flipped, -0
// folded onto +0, NaN sorted after +inf).
// ---------------------------------------------------------------------------
#define VSK_KEY_NONE 0xFFFFFFFFFFFFFFFFull

__host__ __device__ inline uint32_t vsk_f2ord(float f) {
  if (f == 0.0f) f = 0.0f;          // -0 -> +0
  if (f != f) return 0xFFFFFFFFu;   // NaN last
  uint32_t u;
#ifdef __HIP_DEVICE_COMPILE__
  u = __float_as_uint(f);
#else
  __builtin_memcpy(&u, &f, 4);
#endif
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__host__ __device__ inline float vsk_ord2f(uint32_t o) {
  uint32_t u = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
  float f;
#ifdef __HIP_DEVICE_COMPILE__
  f = __uint_as_float(u);
#else
  __builtin_memcpy(&f, &u, 4);
#endif
  return f;
}
__host__ __device__ inline uint64_t vsk_key(float dist, uint32_t tie) {
  return ((uint64_t)vsk_f2ord(dist) << 32) | (uint64_t)tie;
}
// int32 distance (SQ8: -score) keyed the same way
__host__ __device__ inline uint64_t vsk_key_i32(int32_t dist, uint32_t tie) {
  return ((uint64_t)((uint32_t)dist ^ 0x80000000u) << 32) | (uint64_t)tie;
}
