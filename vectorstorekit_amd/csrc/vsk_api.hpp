// vsk_api.hpp -- entry-point boilerplate and the shared top-k machinery.
#pragma once

#include <functional>

#include "vsk_core.hpp"

// Every C entry point runs its body inside VSK_API_BEGIN / VSK_API_END: the
// context's device is made current and internal errors become status codes.
#define VSK_API_BEGIN(ctx)                                                    \
  if (!(ctx)) return VSK_ERR_INVALID_ARGUMENT;                                \
  const ::vsk::FaultCtxScope vsk_fault_scope_(ctx);                           \
  if (!vsk_fault_scope_.prev) (ctx)->sync_count = 0;                          \
  try {                                                                       \
    (ctx)->last_error.clear();                                                \
    VSK_HIP(hipSetDevice((ctx)->device));

#define VSK_API_END(ctx)                                                      \
  }                                                                           \
  catch (const ::vsk::Error &e) {                                             \
    (ctx)->last_error = e.msg;                                                \
    (ctx)->ovf_armed = false;                                                 \
    (void)hipStreamSynchronize((ctx)->stream);                                \
    if ((ctx)->aux) (void)hipStreamSynchronize((ctx)->aux);                   \
    (void)hipGetLastError();                                                  \
    (ctx)->drop_pending();                                                    \
    return e.code;                                                            \
  }                                                                           \
  catch (const std::exception &e) {                                           \
    (ctx)->last_error = e.what();                                             \
    (ctx)->ovf_armed = false;                                                 \
    (void)hipStreamSynchronize((ctx)->stream);                                \
    (ctx)->drop_pending();                                                    \
    return VSK_ERR_EXECUTION_FAILED;                                          \
  }                                                                           \
  return VSK_OK;

namespace vsk {

// ---------------------------------------------------------------------------
// top-k selection over composite keys (select.hip)
// ---------------------------------------------------------------------------
// Segment q holds, in this order, prev[q*k .. q*k+k) (VSK_KEY_NONE entries
// are ignored; prev may be null) and the candidates
//   cand[base .. base+count)   base = seg_off ? seg_off[q] : q*cap
//                              count = counts ? counts[q]
//                                      : seg_off ? seg_off[q+1]-seg_off[q]
//                                      : cap
// All keys of a segment must be distinct.  The k smallest are written
// sorted to best_out[q*k ..] (VSK_KEY_NONE-padded; may alias prev) and
// thresh[q] (optional) receives the k-th key (VSK_KEY_NONE if fewer).
// If counts[q] > cap (only with uniform stride) the segment overflowed: its
// outputs are left untouched, overflow_mask[q] = 1 and *overflow_count is
// incremented.  Segments with active && !active[q] are skipped.
struct SelectArgs {
  int64_t nq = 0;
  int32_t k = 0;
  const uint64_t *prev = nullptr;
  const uint64_t *cand = nullptr;
  // 32-bit distances instead of cand (no prev): key = (value << 32) | the
  // value's index in its query's list
  const uint32_t *cand32 = nullptr;
  int64_t cap = 0;
  const int64_t *seg_off = nullptr;
  const int32_t *counts = nullptr;
  uint64_t *best_out = nullptr;
  uint64_t *thresh = nullptr;
  const uint8_t *active = nullptr;
  uint8_t *overflow_mask = nullptr;
  int32_t *overflow_count = nullptr;
  // segmented lists: query q's candidates are segments s = 0..nseg-1 at
  // cand[q*cap + s*seg_stride], seg_n[q*nseg + s] keys each (counts then
  // only flags overflow)
  const int32_t *seg_n = nullptr;
  int32_t nseg = 0;
  int64_t seg_stride = 0;
  bool regs = false;  // small lists: the register-resident variant
  // short counted lists (cap <= 1024, sorted output, no thresh): one wave
  // per query sorts the whole list
  bool small = false;
  // false: best_out gets the k smallest keys in no particular order and
  // thresh a key T with exactly those k keys <= T (a chunk's list that only
  // the next chunk's selection reads)
  bool sorted = true;
};
void launch_select(vsk_ctx *ctx, const SelectArgs &a, const char *name);

// maximum segments per query of a segmented scan
constexpr int32_t VSK_MAX_SEG = 512;

// A scan kernel over database rows [r0, r1) that, for each active query q,
// either writes the key of every row to cand[q*cap + (row - r0)] (dense) or
// appends the keys <= thresh[q] to cand[q*cap + atomicAdd(&counts[q], 1)]
// (keys past cap are dropped, counts keeps counting).
struct ScanRequest {
  int64_t r0, r1;
  const uint64_t *thresh;
  const uint8_t *active;  // null: all queries active
  uint64_t *cand;
  int64_t cap;
  int32_t *counts;
  bool dense;
  // a filter scan may write segmented lists instead (see SelectArgs): it
  // fills seg_n (nq x VSK_MAX_SEG) and reports its layout in *seg_nseg and
  // *seg_stride; left at 0, the lists are the appended kind
  int32_t *seg_n = nullptr;
  int32_t *seg_nseg = nullptr;
  int64_t *seg_stride = nullptr;
};
using ScanFn = std::function<void(const ScanRequest &)>;

// Device buffers of one progressive_topk call, for callers that bring their
// own memory (nothing is allocated then).  cand holds nq*cap keys with cap
// already clamped to the row count; seg_n may be null (appended lists only).
struct TopkWorkspace {
  uint64_t *thresh = nullptr;    // nq
  uint64_t *cand = nullptr;      // nq * cap
  int32_t *counts = nullptr;     // nq
  uint8_t *ovf_mask = nullptr;   // roundup(nq, 4) + 64
  int32_t *ovf_count = nullptr;  // 1
  int32_t *seg_n = nullptr;      // nq * VSK_MAX_SEG, or null
};

// Exact top-k over n rows for nq queries by streaming the rows in growing
// chunks: the first chunk is kept whole, later chunks only keep rows that
// beat the running k-th key of their query; a query whose survivors
// overflow cap re-scans the chunk in whole sub-chunks.  best: nq*k keys
// (device), sorted ascending per query on return.  A chunk after the first
// holds at most cap/(2k) times the rows already seen, and at most max_growth
// times when that is positive.
// ws: the buffers to use (sized for nq and min(cap, n)); null = the
// context's scratch slots.
void progressive_topk(vsk_ctx *ctx, int64_t nq, int64_t n, int32_t k,
                      int64_t cap, const ScanFn &scan, uint64_t *best,
                      const char *select_name, int64_t max_growth = 0,
                      const TopkWorkspace *ws = nullptr);

// candidate buffer capacity per query used by the progressive scans
int64_t default_cap(int32_t k);
// candidate slots per query of the bf16 screen: chunks grow about 2-4x (the
// survivors of a chunk are about k times the growth), so a small first dense
// chunk and its selection, at a few more launches; measured at 1M x 768 with
// 10,000 queries and k = 100 (kept 364): 5% faster than default_cap
int64_t screen_cap(int32_t k);
// largest query batch whose candidate buffers (cap keys a query) fit the
// context's tile budget
int64_t query_batch(const vsk_ctx *ctx, int64_t nq, int64_t cap);
// keys of bytes_per_key bytes a batch may hold: at most keys, and under
// VSK_MAX_TILE_BYTES when it is set
int64_t tile_keys(const vsk_ctx *ctx, int64_t keys, int64_t bytes_per_key);

// decode keys: dist = float of the key (sqrt when sqrt_out), id =
// id_map ? id_map[tie] : tie; VSK_KEY_NONE -> (+inf, -1)
void decode_keys(vsk_ctx *ctx, const uint64_t *best, int64_t total,
                 bool sqrt_out, const int64_t *id_map, float *out_dist,
                 int64_t *out_ids);

// Resolves, once per device (the device current), the device address of the
// static scratch array that vsk_sq8_search_noalloc uses (sq8.hip).
void sq8_noalloc_setup(int device);

}  // namespace vsk
