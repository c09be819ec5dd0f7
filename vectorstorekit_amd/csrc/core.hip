// core.hip -- context, staging of caller buffers, event profiling, small
// utility kernels (fills, row norms, key decoding) and the flat database.
#include <cstdlib>
#include <cstring>

#include "vsk_api.hpp"
#include "vsk_core.hpp"

namespace vsk {

[[noreturn]] void fail(vsk_status code, const std::string &msg) {
  throw Error{code, msg};
}

void check_hip(hipError_t e, const char *what, const char *file, int line) {
  if (e == hipSuccess) return;
  char buf[512];
  snprintf(buf, sizeof buf, "%s failed: %s (%s:%d)", what, hipGetErrorString(e),
           file, line);
  vsk_status code = VSK_ERR_EXECUTION_FAILED;
  if (e == hipErrorOutOfMemory) code = VSK_ERR_OUT_OF_MEMORY;
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
    code = VSK_ERR_DEVICE_NOT_AVAILABLE;
  fail(code, buf);
}

DevBuf::~DevBuf() { release(); }
void DevBuf::release() {
  if (p) (void)hipFree(p);
  p = nullptr;
  bytes = 0;
}
namespace {
thread_local vsk_ctx *t_fault_ctx = nullptr;
}
vsk_ctx *set_fault_ctx(vsk_ctx *c) {
  vsk_ctx *p = t_fault_ctx;
  t_fault_ctx = c;
  return p;
}
void fault_point(int kind) {
  vsk_ctx *c = t_fault_ctx;
  if (!c || c->fault_kind != kind) return;
  if (++c->fault_seen != c->fault_at) return;
  static const char *names[] = {"", "allocation", "launch", "synchronisation"};
  fail(kind == FAULT_ALLOC ? VSK_ERR_OUT_OF_MEMORY : VSK_ERR_EXECUTION_FAILED,
       std::string("injected fault (VSK_FAULT): ") + names[kind] + " " +
           std::to_string(c->fault_at));
}

void DevBuf::reserve(size_t b) {
  if (b <= bytes && p) return;
  release();
  fault_point(FAULT_ALLOC);
  size_t want = b ? b : 1;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    p = nullptr;
    fail(VSK_ERR_OUT_OF_MEMORY,
         "device allocation of " + std::to_string(want) + " bytes failed");
  }
  bytes = want;
}

bool is_device_ptr(const void *p) {
  if (!p) return false;
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return attr.type == hipMemoryTypeDevice;
}

CallScope::CallScope(vsk_ctx *c) : ctx(c) {
  VSK_HIP(hipEventRecord(ctx->call_begin, ctx->stream));
}
void stream_sync(vsk_ctx *ctx) {
  ++ctx->sync_count;
  VSK_HIP(hipStreamSynchronize(ctx->stream));
}

void CallScope::finish() {
  if (ctx->aux) VSK_HIP(hipStreamSynchronize(ctx->aux));
  // the deferred top-k overflow count comes back with the final sync
  const bool armed = ctx->ovf_armed;
  if (armed)
    VSK_HIP(hipMemcpyAsync(ctx->ovf_host, ctx->ovf_dev, sizeof(int32_t),
                           hipMemcpyDeviceToHost, ctx->stream));
  VSK_HIP(hipEventRecord(ctx->call_end, ctx->stream));
  stream_sync(ctx);
  if (armed) {
    ctx->ovf_armed = false;
    if (ctx->ovf_host[0] > 0) ctx->topk_overflowed = true;
  }
  float ms = 0.f;
  VSK_HIP(hipEventElapsedTime(&ms, ctx->call_begin, ctx->call_end));
  ctx->last_ms = ms;
  ctx->resolve_pending();
  fault_point(FAULT_SYNC);
}

KernelTimer::KernelTimer(vsk_ctx *c, const char *name, double work_items, hipStream_t s)
    : ctx(c), work(work_items), stream(s ? s : c->stream) {
  if (!ctx->timed(name)) return;
  auto it = ctx->stat_index.find(name);
  if (it == ctx->stat_index.end()) {
    vsk_kernel_stat s;
    memset(&s, 0, sizeof s);
    snprintf(s.name, sizeof s.name, "%s", name);
    ctx->stats.push_back(s);
    it = ctx->stat_index.emplace(name, (int)ctx->stats.size() - 1).first;
  }
  stat = it->second;
  a = ctx->take_timer_event();
  VSK_HIP(hipEventRecord(a, stream));
}
KernelTimer::~KernelTimer() {
  if (stat < 0) return;
  hipEvent_t b = ctx->take_timer_event();
  if (hipEventRecord(b, stream) != hipSuccess) {
    ctx->timer_pool.push_back(a);
    ctx->timer_pool.push_back(b);
    return;
  }
  int slot = -1;
  if (work_dev && ctx->count_work()) {
    if (!ctx->work_pinned &&
        hipHostMalloc(reinterpret_cast<void **>(&ctx->work_pinned),
                      sizeof(int64_t) * vsk_ctx::kWorkSlots, hipHostMallocDefault) != hipSuccess)
      ctx->work_pinned = nullptr;
    if (ctx->work_pinned && ctx->work_used < vsk_ctx::kWorkSlots &&
        hipMemcpyAsync(ctx->work_pinned + ctx->work_used, work_dev, sizeof(int64_t),
                       hipMemcpyDeviceToHost, stream) == hipSuccess)
      slot = ctx->work_used++;
  }
  ctx->pending.push_back({stat, a, b, work, slot});
}

void check_launch(const char *name) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    fail(VSK_ERR_EXECUTION_FAILED,
         std::string("launch of ") + name + " failed: " + hipGetErrorString(e));
  fault_point(FAULT_LAUNCH);
}

const void *input_to_device(vsk_ctx *ctx, const void *p, size_t bytes,
                            const std::string &slot) {
  if (bytes == 0 || is_device_ptr(p)) return p;
  void *d = ctx->scratch_ptr(slot, bytes);
  VSK_HIP(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, ctx->stream));
  return d;
}

OutputStage::OutputStage(vsk_ctx *c, void *user_ptr, size_t nbytes,
                         const std::string &slot)
    : ctx(c), user(user_ptr), bytes(nbytes) {
  host = !is_device_ptr(user_ptr);
  dev = host ? ctx->scratch_ptr(slot, nbytes) : user_ptr;
}
void OutputStage::copy_back() {
  if (host && bytes)
    VSK_HIP(hipMemcpyAsync(user, dev, bytes, hipMemcpyDeviceToHost,
                           ctx->stream));
}

void copy_rows(vsk_ctx *ctx, void *dst, size_t dst_pitch, const void *src,
               size_t src_pitch, size_t row_bytes, int64_t rows) {
  if (rows <= 0 || row_bytes == 0) return;
  const bool sdev = is_device_ptr(src), ddev = is_device_ptr(dst);
  const bool dense = src_pitch == row_bytes && dst_pitch == row_bytes;
  const hipMemcpyKind kind =
      sdev ? (ddev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost)
           : (ddev ? hipMemcpyHostToDevice : hipMemcpyHostToHost);
  if (dense) {
    VSK_HIP(hipMemcpyAsync(dst, src, row_bytes * (size_t)rows, kind,
                           ctx->stream));
    return;
  }
  if (sdev && ddev) {
    VSK_HIP(hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, row_bytes,
                             (size_t)rows, kind, ctx->stream));
    return;
  }
  VSK_REQUIRE(sdev || ddev, VSK_ERR_INVALID_ARGUMENT,
              "host-to-host row copy is not supported");
  VSK_REQUIRE(!sdev || dst_pitch == row_bytes, VSK_ERR_INVALID_ARGUMENT,
              "host destination rows must be packed");
  // one side is host memory: move whole chunks in one transfer each and do
  // the pitch change on the device
  const size_t host_pitch = sdev ? dst_pitch : src_pitch;
  const size_t chunk_bytes = size_t(64) << 20;
  int64_t chunk = (int64_t)(chunk_bytes / host_pitch);
  if (chunk < 1) chunk = 1;
  if (chunk > rows) chunk = rows;
  char *stage = static_cast<char *>(
      ctx->scratch_ptr("stage.rows", host_pitch * (size_t)chunk));
  for (int64_t r = 0; r < rows; r += chunk) {
    const int64_t m = rows - r < chunk ? rows - r : chunk;
    const size_t span = host_pitch * (size_t)(m - 1) + row_bytes;
    if (!sdev) {
      VSK_HIP(hipMemcpyAsync(stage, static_cast<const char *>(src) + r * src_pitch,
                             span, hipMemcpyHostToDevice, ctx->stream));
      VSK_HIP(hipMemcpy2DAsync(static_cast<char *>(dst) + r * dst_pitch,
                               dst_pitch, stage, src_pitch, row_bytes,
                               (size_t)m, hipMemcpyDeviceToDevice,
                               ctx->stream));
    } else {
      VSK_HIP(hipMemcpy2DAsync(stage, dst_pitch,
                               static_cast<const char *>(src) + r * src_pitch,
                               src_pitch, row_bytes, (size_t)m,
                               hipMemcpyDeviceToDevice, ctx->stream));
      VSK_HIP(hipMemcpyAsync(static_cast<char *>(dst) + r * dst_pitch, stage,
                             span, hipMemcpyDeviceToHost, ctx->stream));
    }
  }
}

const float *rows_to_device_padded(vsk_ctx *ctx, const float *p, int64_t rows,
                                   int32_t d, int32_t ld,
                                   const std::string &slot) {
  if (rows == 0) return nullptr;
  bool dev = is_device_ptr(p);
  // used in place when already laid out (kernels load 16-byte vectors)
  if (dev && ld == d && (reinterpret_cast<uintptr_t>(p) & 15) == 0) return p;
  float *out = static_cast<float *>(
      ctx->scratch_ptr(slot, sizeof(float) * (size_t)rows * ld));
  if (ld != d)
    fill_i32(ctx, reinterpret_cast<int32_t *>(out), rows * (int64_t)ld, 0);
  copy_rows(ctx, out, sizeof(float) * ld, p, sizeof(float) * d,
            sizeof(float) * d, rows);
  return out;
}

bool metric_valid(int32_t m) {
  return m >= VSK_METRIC_L2SQ && m <= VSK_METRIC_HAMMING;
}

// ---------------------------------------------------------------------------
// utility kernels
// ---------------------------------------------------------------------------
__global__ void k_fill_u64(uint64_t *p, int64_t n, uint64_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}
__global__ void k_fill_i32(int32_t *p, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}
static unsigned fill_grid(int64_t n) {
  int64_t g = ceil_div(n, 256);
  return (unsigned)(g < 4096 ? (g > 0 ? g : 1) : 4096);
}
void fill_u64(vsk_ctx *ctx, uint64_t *p, int64_t n, uint64_t v) {
  if (n <= 0) return;
  k_fill_u64<<<fill_grid(n), 256, 0, ctx->stream>>>(p, n, v);
  check_launch("fill_u64");
}
void fill_i32(vsk_ctx *ctx, int32_t *p, int64_t n, int32_t v) {
  if (n <= 0) return;
  k_fill_i32<<<fill_grid(n), 256, 0, ctx->stream>>>(p, n, v);
  check_launch("fill_i32");
}

// one wave per row: lane-strided partial sums, then a butterfly reduction
__global__ __launch_bounds__(256) void k_row_norms(const float *x, int64_t n,
                                                   int32_t d, int32_t ld,
                                                   float *sq, float *nrm) {
  const int lane = threadIdx.x & 63;
  int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const float *r = x + row * ld;
  float s = 0.f;
  for (int j = lane; j < d; j += 64) s += r[j] * r[j];
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) {
    if (sq) sq[row] = s;
    if (nrm) nrm[row] = sqrtf(s);
  }
}
void row_norms(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
               float *sq, float *nrm) {
  if (n <= 0) return;
  k_row_norms<<<(unsigned)ceil_div(n, 4), 256, 0, ctx->stream>>>(x, n, d, ld,
                                                                   sq, nrm);
  check_launch("row_norms");
}

// normalizeVectors (Acceleration/Metal/Shaders/DistanceShaders.metal:
// 403-429): m = sqrt(sum x_i^2) + 1e-8 with the squares added in dimension
// order (no FMA), then x_i <- x_i / m, a division per component.  One lane
// per row keeps the sequential sum; each wave stages 64 rows x 32 columns
// at a time through LDS so the row reads stay coalesced.
constexpr int NRM_COLS = 32;
// With norms, the same sequential sums give norms[row] = sqrt(sum x_i^2)
// and the rows are left as they are: the reference's |x| (cosine,
// Acceleration/AccelerateOptimizer.swift:305-316 restated sequentially).
__global__ __launch_bounds__(256) void k_normalize_rows(float *x, int64_t n,
                                                       int32_t d, int32_t ld,
                                                       float *norms) {
#pragma clang fp contract(off)
  __shared__ float tile[4][64][NRM_COLS + 1];
  __shared__ float mag[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + w) * 64;
  // every wave reaches the barriers; a wave past the last row has no rows
  const int rows = n - row0 >= 64 ? 64 : (n > row0 ? (int)(n - row0) : 0);
  float s = 0.f;
  for (int32_t c0 = 0; c0 < d; c0 += NRM_COLS) {
    // lanes 0-31 read one row's 32 columns, lanes 32-63 the next row's
#pragma unroll 4
    for (int j = 0; j < 32; ++j) {
      const int r = 2 * j + (lane >> 5), c = c0 + (lane & 31);
      tile[w][r][lane & 31] = (r < rows && c < d) ? x[(row0 + r) * ld + c] : 0.f;
    }
    __syncthreads();
    const int cn = d - c0 < NRM_COLS ? d - c0 : NRM_COLS;
    for (int c = 0; c < cn; ++c) {
      const float v = tile[w][lane][c];
      s = s + v * v;
    }
    __syncthreads();
  }
  if (norms) {
    if (lane < rows) norms[row0 + lane] = sqrtf(s);
    return;
  }
  mag[w][lane] = sqrtf(s) + 1e-8f;
  __syncthreads();
  if (rows == 0) return;
  for (int r = 0; r < rows; ++r) {
    const float m = mag[w][r];
    float *xr = x + (row0 + r) * ld;
    for (int32_t c = lane; c < d; c += 64) xr[c] = xr[c] / m;
  }
}

void seq_norms(vsk_ctx *ctx, const float *x, int64_t n, int32_t d, int32_t ld,
               float *norms) {
  if (n <= 0) return;
  k_normalize_rows<<<(unsigned)ceil_div(n, 256), 256, 0, ctx->stream>>>(
      const_cast<float *>(x), n, d, ld, norms);
  check_launch("seq_norms");
}

// decode composite keys into (distance, id) outputs
__global__ void k_decode_f32(const uint64_t *best, int64_t total, int32_t mode,
                             const int64_t *id_map, float *out_dist,
                             int64_t *out_ids) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    uint64_t key = best[i];
    if (key == VSK_KEY_NONE) {
      out_dist[i] = __int_as_float(0x7f800000);
      out_ids[i] = -1;
      continue;
    }
    float dist = vsk_ord2f((uint32_t)(key >> 32));
    if (mode == 1) dist = sqrtf(fmaxf(dist, 0.f));
    uint32_t tie = (uint32_t)key;
    out_dist[i] = dist;
    out_ids[i] = id_map ? id_map[tie] : (int64_t)tie;
  }
}
void decode_keys(vsk_ctx *ctx, const uint64_t *best, int64_t total,
                 bool sqrt_out, const int64_t *id_map, float *out_dist,
                 int64_t *out_ids) {
  if (total <= 0) return;
  KernelTimer t(ctx, "decode_keys");
  k_decode_f32<<<fill_grid(total), 256, 0, ctx->stream>>>(
      best, total, sqrt_out ? 1 : 0, id_map, out_dist, out_ids);
  check_launch("decode_keys");
}

}  // namespace vsk

// ---------------------------------------------------------------------------
// vsk_ctx members
// ---------------------------------------------------------------------------
void *vsk_ctx::scratch_ptr(const std::string &key, size_t bytes) {
  auto &b = scratch[key];
  if (!b) b.reset(new vsk::DevBuf());
  if (b->bytes < bytes || !b->p) {
    // a buffer in use by queued work must not be freed under it
    ++sync_count;
    VSK_HIP(hipStreamSynchronize(stream));
    if (aux) VSK_HIP(hipStreamSynchronize(aux));
    b->reserve(bytes + bytes / 8);
  }
  return b->p;
}
hipStream_t vsk_ctx::aux_stream() {
  if (!aux) VSK_HIP(hipStreamCreate(&aux));
  return aux;
}
void *vsk_ctx::pinned_ptr(size_t bytes) {
  if (pinned_bytes < bytes) {
    if (pinned) {
      ++sync_count;
      VSK_HIP(hipStreamSynchronize(stream));
      if (aux) VSK_HIP(hipStreamSynchronize(aux));
      (void)hipHostFree(pinned);
      pinned = nullptr;
      pinned_bytes = 0;
    }
    VSK_HIP(hipHostMalloc(&pinned, bytes, hipHostMallocDefault));
    pinned_bytes = bytes;
  }
  return pinned;
}
hipEvent_t vsk_ctx::take_event() {
  if (!event_pool.empty()) {
    hipEvent_t e = event_pool.back();
    event_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  VSK_HIP(hipEventCreate(&e));
  return e;
}
hipEvent_t vsk_ctx::take_timer_event() {
  if (!timer_pool.empty()) {
    hipEvent_t e = timer_pool.back();
    timer_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  VSK_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
  return e;
}
void vsk_ctx::drop_pending() {
  for (auto &p : pending) {
    timer_pool.push_back(p.a);
    timer_pool.push_back(p.b);
  }
  pending.clear();
  work_used = 0;
}

void vsk_ctx::resolve_pending() {
  for (auto &p : pending) {
    float ms = 0.f;
    if (p.stat < (int)stats.size() && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
      stats[p.stat].launches += 1;
      stats[p.stat].total_ms += ms;
      stats[p.stat].work += p.work_slot >= 0 ? (double)work_pinned[p.work_slot] : p.work;
    }
    timer_pool.push_back(p.a);
    timer_pool.push_back(p.b);
  }
  pending.clear();
  work_used = 0;
}

// ---------------------------------------------------------------------------
// C ABI: context, profiling, flat database
// ---------------------------------------------------------------------------
using namespace vsk;

extern "C" {

vsk_status vsk_create(int32_t device, vsk_ctx **out) {
  if (!out) return VSK_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    (void)hipGetLastError();
    return VSK_ERR_DEVICE_NOT_AVAILABLE;
  }
  if (device < 0 || device >= count) return VSK_ERR_DEVICE_NOT_AVAILABLE;
  if (hipSetDevice(device) != hipSuccess) return VSK_ERR_DEVICE_NOT_AVAILABLE;
  // the device address of this GPU's no-allocation scratch (sq8.hip), once
  // per device; a failure is reported by the entry point that needs it
  sq8_noalloc_setup(device);
  vsk_ctx *c = new vsk_ctx();
  c->device = device;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
      cus > 0)
    c->cu_count = cus;
  const char *fk = getenv("VSK_FLAT_KERNEL");
  c->flat_fp32 = fk && strcmp(fk, "fp32") == 0;
  c->flat_no_screen = fk && (c->flat_fp32 || strcmp(fk, "bf16x3") == 0);
  c->flat_force_screen = fk && strcmp(fk, "screen") == 0;
  c->exact_only = fk && strcmp(fk, "exact") == 0;
  const char *ic = getenv("VSK_IVF_COMPACT");
  c->ivf_no_compact = ic && strcmp(ic, "0") == 0;
  if (const char *tb = getenv("VSK_MAX_TILE_BYTES")) {
    const long long v = atoll(tb);
    if (v > 0) c->max_tile_bytes = v;
  }
  if (const char *ff = getenv("VSK_FAULT")) {
    const char *colon = strchr(ff, ':');
    const long long at = colon ? atoll(colon + 1) : 0;
    const size_t len = colon ? (size_t)(colon - ff) : strlen(ff);
    int kind = 0;
    if (len == 5 && strncmp(ff, "alloc", 5) == 0) kind = FAULT_ALLOC;
    if (len == 6 && strncmp(ff, "launch", 6) == 0) kind = FAULT_LAUNCH;
    if (len == 4 && strncmp(ff, "sync", 4) == 0) kind = FAULT_SYNC;
    if (kind && at > 0) {
      c->fault_kind = kind;
      c->fault_at = at;
    }
  }
  // a blocking stream: it orders itself after work on the null stream, so
  // device buffers produced there (e.g. by torch) are complete when read
  if (hipStreamCreate(&c->stream) != hipSuccess ||
      hipEventCreate(&c->call_begin) != hipSuccess ||
      hipEventCreate(&c->call_end) != hipSuccess ||
      hipMalloc(reinterpret_cast<void **>(&c->ovf_dev), 256) != hipSuccess ||
      hipHostMalloc(reinterpret_cast<void **>(&c->ovf_host), 8 * sizeof(int32_t),
                    hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    if (c->ovf_dev) (void)hipFree(c->ovf_dev);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    if (c->call_begin) (void)hipEventDestroy(c->call_begin);
    if (c->call_end) (void)hipEventDestroy(c->call_end);
    delete c;
    return VSK_ERR_DEVICE_NOT_AVAILABLE;
  }
  *out = c;
  return VSK_OK;
}

vsk_status vsk_destroy(vsk_ctx *ctx) {
  if (!ctx) return VSK_OK;
  if (t_fault_ctx == ctx) t_fault_ctx = nullptr;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->aux) (void)hipStreamSynchronize(ctx->aux);
  ctx->resolve_pending();
  for (auto e : ctx->event_pool) (void)hipEventDestroy(e);
  for (auto e : ctx->timer_pool) (void)hipEventDestroy(e);
  if (ctx->aux) (void)hipStreamDestroy(ctx->aux);
  if (ctx->pinned) (void)hipHostFree(ctx->pinned);
  if (ctx->work_pinned) (void)hipHostFree(ctx->work_pinned);
  if (ctx->ovf_host) (void)hipHostFree(ctx->ovf_host);
  if (ctx->ovf_dev) (void)hipFree(ctx->ovf_dev);
  ctx->scratch.clear();
  (void)hipEventDestroy(ctx->call_begin);
  (void)hipEventDestroy(ctx->call_end);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return VSK_OK;
}

vsk_status vsk_configure(vsk_ctx *ctx, const vsk_config *cfg) {
  if (!ctx || !cfg) return VSK_ERR_INVALID_ARGUMENT;
  if (cfg->kernel < VSK_KERNEL_AUTO || cfg->kernel > VSK_KERNEL_FP32 || cfg->max_tile_bytes < 0) {
    ctx->last_error = "invalid configuration";
    return VSK_ERR_INVALID_ARGUMENT;
  }
  ctx->flat_fp32 = cfg->kernel == VSK_KERNEL_FP32;
  ctx->flat_no_screen = cfg->kernel == VSK_KERNEL_FP32 || cfg->kernel == VSK_KERNEL_BF16X3;
  ctx->flat_force_screen = cfg->kernel == VSK_KERNEL_SCREEN;
  ctx->exact_only = cfg->kernel == VSK_KERNEL_EXACT;
  ctx->profile = cfg->enable_profiling != 0;
  ctx->max_tile_bytes = cfg->max_tile_bytes;
  return VSK_OK;
}

vsk_status vsk_get_config(const vsk_ctx *ctx, vsk_config *cfg) {
  if (!ctx || !cfg) return VSK_ERR_INVALID_ARGUMENT;
  cfg->kernel = ctx->flat_fp32           ? VSK_KERNEL_FP32
                : ctx->flat_no_screen    ? VSK_KERNEL_BF16X3
                : ctx->flat_force_screen ? VSK_KERNEL_SCREEN
                : ctx->exact_only        ? VSK_KERNEL_EXACT
                                         : VSK_KERNEL_AUTO;
  cfg->enable_profiling = ctx->profile ? 1 : 0;
  cfg->max_tile_bytes = ctx->max_tile_bytes;
  return VSK_OK;
}

const char *vsk_last_error(const vsk_ctx *ctx) {
  return ctx ? ctx->last_error.c_str() : "null context";
}
void *vsk_stream(vsk_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }
float vsk_last_kernel_ms(const vsk_ctx *ctx) { return ctx ? ctx->last_ms : 0.f; }
int32_t vsk_last_sync_count(const vsk_ctx *ctx) { return ctx ? ctx->sync_count : 0; }

vsk_status vsk_last_screen_redo(const vsk_ctx *ctx, int32_t tier, int64_t *out,
                                int64_t cap, int64_t *count) {
  if (!ctx || !count || (tier != 1 && tier != 2) || cap < 0 || (cap > 0 && !out))
    return VSK_ERR_INVALID_ARGUMENT;
  const auto &rec = ctx->screen_redo[tier - 1];
  *count = (int64_t)rec.size();
  const int64_t m = cap < *count ? cap : *count;
  for (int64_t i = 0; i < m; ++i) out[i] = rec[(size_t)i];
  return VSK_OK;
}

vsk_status vsk_device_info(vsk_ctx *ctx, vsk_caps *caps) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(caps, VSK_ERR_INVALID_ARGUMENT, "caps is null");
  hipDeviceProp_t p;
  VSK_HIP(hipGetDeviceProperties(&p, ctx->device));
  memset(caps, 0, sizeof *caps);
  snprintf(caps->name, sizeof caps->name, "%s", p.name);
  snprintf(caps->arch, sizeof caps->arch, "%s", p.gcnArchName);
  caps->device = ctx->device;
  caps->compute_units = p.multiProcessorCount;
  caps->wavefront_size = p.warpSize;
  caps->lds_bytes_per_block = (int32_t)p.sharedMemPerBlock;
  caps->global_mem_bytes = (int64_t)p.totalGlobalMem;
  caps->clock_khz = p.clockRate;
  caps->memory_clock_khz = p.memoryClockRate;
  caps->memory_bus_width_bits = p.memoryBusWidth;
  VSK_API_END(ctx);
}

vsk_status vsk_profile_enable(vsk_ctx *ctx, int32_t on) {
  if (!ctx) return VSK_ERR_INVALID_ARGUMENT;
  ctx->profile = on != 0;
  return VSK_OK;
}
vsk_status vsk_profile_only(vsk_ctx *ctx, const char *names) {
  if (!ctx) return VSK_ERR_INVALID_ARGUMENT;
  ctx->profile_only.clear();
  if (!names) return VSK_OK;
  std::string cur;
  for (const char *p = names;; ++p) {
    if (*p == ',' || *p == 0) {
      if (!cur.empty()) ctx->profile_only.push_back(cur);
      cur.clear();
      if (*p == 0) break;
    } else {
      cur.push_back(*p);
    }
  }
  return VSK_OK;
}
vsk_status vsk_profile_reset(vsk_ctx *ctx) {
  if (!ctx) return VSK_ERR_INVALID_ARGUMENT;
  // timings of a failed call that were never resolved name stats that are
  // about to go
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  ctx->drop_pending();
  ctx->stats.clear();
  ctx->stat_index.clear();
  return VSK_OK;
}
int32_t vsk_profile_count(const vsk_ctx *ctx) {
  return ctx ? (int32_t)ctx->stats.size() : 0;
}
vsk_status vsk_profile_get(const vsk_ctx *ctx, int32_t i,
                           vsk_kernel_stat *out) {
  if (!ctx || !out || i < 0 || i >= (int32_t)ctx->stats.size())
    return VSK_ERR_INVALID_ARGUMENT;
  *out = ctx->stats[i];
  return VSK_OK;
}

vsk_status vsk_db_upload_f32(vsk_ctx *ctx, const float *x, int64_t n, int32_t d,
                             int32_t flags, vsk_db **out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(out, VSK_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  VSK_REQUIRE(n > 0, VSK_ERR_EMPTY_INPUT, "database has no rows");
  VSK_REQUIRE(d > 0, VSK_ERR_INVALID_ARGUMENT, "dimension must be positive");
  VSK_REQUIRE(d <= (1 << 24), VSK_ERR_INVALID_BUFFER_SIZE, "at most 2^24 dimensions");
  VSK_REQUIRE(x, VSK_ERR_INVALID_ARGUMENT, "x is null");
  VSK_REQUIRE(n <= 0x7FFFFFFFll, VSK_ERR_INVALID_BUFFER_SIZE,
              "a database holds at most 2^31-1 rows");
  VSK_REQUIRE((flags & ~VSK_DB_NORMALIZE) == 0, VSK_ERR_INVALID_ARGUMENT,
              "unknown flags");
  std::unique_ptr<vsk_db> db(new vsk_db());
  db->n = n;
  db->d = d;
  db->ld = padded_ld(d);
  CallScope cs(ctx);
  db->x.reserve(sizeof(float) * (size_t)n * db->ld);
  if (db->ld != d)
    fill_i32(ctx, db->x.as<int32_t>(), n * (int64_t)db->ld, 0);
  copy_rows(ctx, db->x.p, sizeof(float) * db->ld, x, sizeof(float) * d,
            sizeof(float) * d, n);
  if (flags & VSK_DB_NORMALIZE) {
    k_normalize_rows<<<(unsigned)ceil_div(n, 256), 256, 0, ctx->stream>>>(
        db->x.as<float>(), n, d, db->ld, nullptr);
    check_launch("normalize_rows");
  }
  db->sqnorm.reserve(sizeof(float) * n);
  db->norm.reserve(sizeof(float) * n);
  row_norms(ctx, db->x.as<float>(), n, d, db->ld, db->sqnorm.as<float>(),
            db->norm.as<float>());
  cs.finish();
  *out = db.release();
  VSK_API_END(ctx);
}

vsk_status vsk_db_free(vsk_ctx *ctx, vsk_db *db) {
  if (ctx) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
  }
  delete db;
  return VSK_OK;
}

vsk_status vsk_db_info(const vsk_db *db, int64_t *n, int32_t *d) {
  if (!db) return VSK_ERR_INVALID_ARGUMENT;
  if (n) *n = db->n;
  if (d) *d = db->d;
  return VSK_OK;
}

vsk_status vsk_db_read_f32(vsk_ctx *ctx, const vsk_db *db, int64_t row0,
                           int64_t count, float *out) {
  VSK_API_BEGIN(ctx);
  VSK_REQUIRE(db && out, VSK_ERR_INVALID_ARGUMENT, "null argument");
  VSK_REQUIRE(row0 >= 0 && count >= 0 && row0 + count <= db->n,
              VSK_ERR_INVALID_ARGUMENT, "row range out of bounds");
  if (count == 0) return VSK_OK;
  CallScope cs(ctx);
  copy_rows(ctx, out, sizeof(float) * db->d, db->x.as<float>() + row0 * db->ld,
            sizeof(float) * db->ld, sizeof(float) * db->d, count);
  cs.finish();
  VSK_API_END(ctx);
}

}  // extern "C"
