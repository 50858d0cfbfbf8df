// One MoE layer of the global-table path in one call: the stage entry points
// enqueued back to back on one stream, the workspace split between them.
#include <mutex>

#include "tm_internal.h"

// Scratch of tm_table_forward_noalloc: the layer workspace as a static device
// array (each GPU the library runs on holds its own copy until the process
// ends).  Host code never passes the array's name to a kernel -- on the host
// it is only a stand-in -- but the per-device address hipGetSymbolAddress
// returns for it.
static __device__ __align__(256) unsigned char scratch[TM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Three plans share one workspace layout: the general one (tm_project,
// tm_search_global, tm_keep_select as exported), the fused top-1 one (packed
// keys and partial query norms: column-split projection carrying the router
// and the key reset, search merging by atomic minimum, keep select decoding
// the keys; for up to 4096 tokens the search decodes the keys and the
// combine ranks the keep set), and the decode plan (n <= 64: split
// projection, stream search, one finishing launch, or all three in one
// launch).  The first kSync bytes hold the plans' arrival counters and flags
// at the same offset for every n and plan: zero before the first call on a
// workspace, and left zero (counters) or at this workspace's generation
// (flags) by every call.  The decode plan's split projection uses counters
// 0 .. 63, the one-launch decode plan words 64 .. 3071, the ranked top-1
// plan one per query tile, kTmCntStride words apart, from kTileCnt on.
constexpr size_t kSync = TM_LAYER_SYNC_BYTES;
constexpr int kTileCnt = 3072;  // past the one-launch decode plan's words
constexpr int kMaxTiles = 32;
static_assert((kTileCnt + kMaxTiles * kTmCntStride) * 4 <= (int)kSync, "sync region");

struct WsLayout {
  size_t sync, project, search, keep, keys, qn_part, part, total;
};

WsLayout layout(const tm_table_layer *t, int64_t n, int32_t nn) {
  WsLayout w;
  w.sync = kSync;
  w.project = align_up(tm_project_workspace_size(n, t->hidden, t->dim));
  w.search = align_up(tm_search_global_workspace_size(n, t->n_cent, t->dim, nn));
  w.keep = align_up(tm_keep_select_workspace_size(n));
  const size_t nkeys = tm_internal_decode_keys(n);  // decode plan: replicated best keys
  w.keys = align_up((nkeys > (size_t)n ? nkeys : (size_t)n) * sizeof(uint64_t));
  const size_t qn_floats = tm_internal_decode_qn_floats(n, t->dim);  // decode plan: one partial per 16 columns
  w.qn_part = align_up((qn_floats > (size_t)n * 4 ? qn_floats : (size_t)n * 4) * sizeof(float));
  w.part = n <= 64 ? align_up(tm_internal_decode_part_bytes(n, t->dim)) : 0;
  w.total = w.sync + w.project + w.search + w.keep + w.keys + w.qn_part + w.part;
  return w;
}

// Region offsets (the sync region first).
struct WsPtrs {
  char *project, *search, *keep, *keys, *qn_part, *part;
  uint32_t *sync;
};

WsPtrs ptrs(const WsLayout &w, char *ws) {
  WsPtrs p;
  p.sync = reinterpret_cast<uint32_t *>(ws);
  p.project = ws + w.sync;
  p.search = p.project + w.project;
  p.keep = p.search + w.search;
  p.keys = p.keep + w.keep;
  p.qn_part = p.keys + w.keys;
  p.part = p.qn_part + w.qn_part;
  return p;
}

// The ranked top-1 plan: the keep set is ranked in the combine, each token's
// workgroup reading all n distances, so n is kept moderate.
bool ranked_ok(const tm_table_layer *t, const tm_layer_io *io) {
  const int64_t n = io->n_tokens;
  if (n > 4096) return false;
  const int64_t tiles = tm_internal_search_decode_tiles(t->dtype, n, t->n_cent, t->dim, t->ld_c, t->dim);
  return tiles > 0 && tiles <= kMaxTiles &&
         tm_internal_combine_rank_ok(t->dtype, t->hidden, io->slot_out, io->so_b, io->so_s, io->router_top_k,
                                     t->values, t->ld_v, io->dist, io->residual, io->ld_r, io->out, io->ld_o);
}

// The general plan's ranked form: a top-1 layer of at most 4096 tokens skips
// the keep-select launch and ranks the keep set in the combine (its
// search writes the distances the combine reads).
bool general_ranked_ok(const tm_table_layer *t, const tm_layer_io *io) {
  const int64_t n = io->n_tokens;
  return io->n_nearest == 1 && n > 0 && n <= 4096 &&
         tm_internal_combine_rank_ok(t->dtype, t->hidden, io->slot_out, io->so_b, io->so_s, io->router_top_k,
                                     t->values, t->ld_v, io->dist, io->residual, io->ld_r, io->out, io->ld_o);
}

bool fused_top1_ok(const tm_table_layer *t, const tm_layer_io *io) {
  const int64_t n = io->n_tokens;
  return io->n_nearest == 1 &&
         tm_internal_project_cols_ok(t->dtype, io->x, n, t->hidden, io->ld_x, t->proj_vis, t->bias_vis,
                                     t->proj_txt, t->bias_txt, t->ps_h, t->ps_d, t->dim, io->q, t->dim) &&
         tm_internal_search_keys_ok(t->dtype, n, t->n_cent, t->ld_c, t->dim, 1) && tm_internal_keep_keys_ok(n);
}

int record(void *const *events, int i, hipStream_t s) {
  if (events == nullptr || events[i] == nullptr) return TM_OK;
  const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(events[i]), s);
  if (e != hipSuccess) return tm_fail(TM_EHIP, "tm_table_forward: hipEventRecord: %s", hipGetErrorString(e));
  return TM_OK;
}

// Stages 0-4 of the fused top-1 plan (events 0..4 bracket router, projection,
// search, keep select).  Ranked form (large n, up to 4096 tokens): the wide
// search decodes the keys itself and the combine ranks the keep set, so the
// keep stage has no launch (events 3 and 4 coincide).
int fused_top1_stages(const tm_table_layer *t, const tm_layer_io *io, const WsLayout &w, char *ws,
                      const tm_route_args &ra, bool route_fused, bool ranked, int64_t n_keep, void *const *ev,
                      hipStream_t s) {
  const int64_t n = io->n_tokens;
  const WsPtrs p = ptrs(w, ws);
  uint64_t *keys = reinterpret_cast<uint64_t *>(p.keys);
  float *qn_part = reinterpret_cast<float *>(p.qn_part);
  int st;
  if ((st = record(ev, 0, s)) != TM_OK) return st;
  if (!route_fused && (st = tm_topk_softmax(io->router_logits, n, io->n_experts, io->ld_logits, io->router_top_k,
                                            0, io->weights, io->expert_ids, s)) != TM_OK)
    return st;
  if ((st = record(ev, 1, s)) != TM_OK) return st;
  if ((st = tm_internal_project_cols(t->dtype, io->x, n, t->hidden, io->ld_x, io->is_vision, t->proj_vis,
                                     t->bias_vis, t->proj_txt, t->bias_txt, t->ps_h, t->ps_d, t->dim, io->q, t->dim,
                                     qn_part, keys, route_fused ? &ra : nullptr, s)) != TM_OK)
    return st;
  if ((st = record(ev, 2, s)) != TM_OK) return st;
  const int32_t parts = (int32_t)tm_internal_project_cols_parts(t->dim, n, t->hidden);
  if (ranked) {  // the search decodes the keys; the keep set is ranked in the combine
    if ((st = tm_internal_search_decode(t->dtype, io->q, n, t->dim, t->cents, t->n_cent, t->ld_c, t->c_sqnorm,
                                        t->dim, t->metric, keys, qn_part, parts, io->dist, io->idx, io->q_sqnorm,
                                        p.sync + kTileCnt, s)) != TM_OK)
      return st;
    return record(ev, 3, s);
  }
  if ((st = tm_internal_search_keys(t->dtype, io->q, n, t->dim, t->cents, t->n_cent, t->ld_c, t->c_sqnorm, t->dim,
                                    t->metric, keys, s)) != TM_OK)
    return st;
  if ((st = record(ev, 3, s)) != TM_OK) return st;
  return tm_internal_keep_keys(keys, qn_part, parts, t->metric, n, n_keep, io->dist, io->idx, io->q_sqnorm, io->keep,
                               s);
}

// Stages 0-4 of the decode plan (n <= 64): split projection (+ router, + key
// reset), stream search, and the finishing launch that merges, ranks the keep
// set and combines; events 3 and 4 coincide (the keep select rides in the
// finishing launch), event 5 is recorded by the caller.
int decode_stages(const tm_table_layer *t, const tm_layer_io *io, const WsLayout &w, char *ws,
                  const tm_route_args &ra, bool route_fused, int64_t n_keep, void *const *ev, bool wait_plans,
                  hipStream_t s) {
  const int64_t n = io->n_tokens;
  const WsPtrs p = ptrs(w, ws);
  const tm_decode_ws dw{reinterpret_cast<uint64_t *>(p.search), reinterpret_cast<uint64_t *>(p.keys),
                        reinterpret_cast<float *>(p.qn_part), p.part, p.sync};
  int st;
  if ((st = record(ev, 0, s)) != TM_OK) return st;
  if (!route_fused && (st = tm_topk_softmax(io->router_logits, n, io->n_experts, io->ld_logits, io->router_top_k,
                                            0, io->weights, io->expert_ids, s)) != TM_OK)
    return st;
  if ((st = record(ev, 1, s)) != TM_OK) return st;
  return tm_internal_decode_forward(t, io, dw, route_fused ? &ra : nullptr, n_keep, ev, wait_plans, s);
}

// Stages 0-4 of the general plan: the exported entry points; the router rides
// in the search's split-merge launch when it can.  Ranked: no keep-select
// launch (events 3 and 4 coincide; the combine ranks the keep set).
int general_stages(const tm_table_layer *t, const tm_layer_io *io, const WsLayout &w, char *ws,
                   const tm_route_args &ra, bool route_fused, bool ranked, int64_t n_keep, void *const *ev,
                   hipStream_t s) {
  const int64_t n = io->n_tokens;
  int st;
  if ((st = record(ev, 0, s)) != TM_OK) return st;
  if (!route_fused && (st = tm_topk_softmax(io->router_logits, n, io->n_experts, io->ld_logits, io->router_top_k,
                                            0, io->weights, io->expert_ids, s)) != TM_OK)
    return st;
  if ((st = record(ev, 1, s)) != TM_OK) return st;
  const WsPtrs p = ptrs(w, ws);
  if ((st = tm_project(t->dtype, io->x, n, t->hidden, io->ld_x, io->is_vision, t->proj_vis, t->bias_vis,
                       t->proj_txt, t->bias_txt, t->ps_h, t->ps_d, t->dim, 0, 1e-6f, io->q, t->dim, io->q_sqnorm,
                       w.project ? p.project : nullptr, w.project, s)) != TM_OK)
    return st;
  if ((st = record(ev, 2, s)) != TM_OK) return st;
  if (route_fused)
    st = tm_internal_search_route(t->dtype, io->q, n, t->dim, io->q_sqnorm, t->cents, t->n_cent, t->ld_c,
                                  t->c_sqnorm, t->dim, io->n_nearest, t->metric, io->dist, io->idx, p.search,
                                  w.search, &ra, s);
  else
    st = tm_search_global(t->dtype, io->q, n, t->dim, io->q_sqnorm, t->cents, t->n_cent, t->ld_c, t->c_sqnorm,
                          t->dim, io->n_nearest, t->metric, io->dist, io->idx, p.search, w.search, s);
  if (st != TM_OK) return st;
  if ((st = record(ev, 3, s)) != TM_OK || ranked) return st;
  return tm_keep_select(io->dist, n, io->n_nearest, n_keep, io->keep, w.keep ? p.keep : nullptr, w.keep, s);
}

}  // namespace

namespace {

// Per-device address of `scratch` and whether its counter region has been
// cleared by a launch (set-up of tm_table_forward_noalloc on each device).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];
bool g_scratch_cleared[kMaxDevices];

__global__ void clear_sync_kernel(uint32_t *p) {
  for (unsigned i = threadIdx.x; i < kSync / 4; i += blockDim.x) p[i] = 0u;
}

// The current device's scratch address; on a device's first call, looks it
// up and enqueues the clear of the arrival counters on `s` (a kernel, not a
// memset, so a caller may capture the call into a graph).
int scratch_for_current_device(hipStream_t s, void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return tm_fail(TM_EHIP, "tm_table_forward_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  TM_REQUIRE(dev >= 0 && dev < kMaxDevices, TM_EINVAL_ARG, "tm_table_forward_noalloc: device %d beyond %d", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return tm_fail(TM_EHIP, "tm_table_forward_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                     hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  if (!g_scratch_cleared[dev]) {
    hipLaunchKernelGGL(clear_sync_kernel, dim3(1), dim3(256), 0, s, static_cast<uint32_t *>(g_scratch_ptr[dev]));
    TM_LAUNCH_CHECK("tm_table_forward_noalloc(clear)");
    g_scratch_cleared[dev] = true;
  }
  *out = g_scratch_ptr[dev];
  return TM_OK;
}

}  // namespace

extern "C" size_t tm_struct_size(int32_t which) {
  return which == 0 ? sizeof(tm_table_layer) : (which == 1 ? sizeof(tm_layer_io) : 0);
}

extern "C" size_t tm_table_forward_workspace_size(const tm_table_layer *table, int64_t n_tokens, int32_t n_nearest) {
  if (table == nullptr || n_tokens <= 0) return 0;
  return layout(table, n_tokens, n_nearest).total;
}

namespace {

// tm_table_forward; `wait_plans` false keeps every launch free of waits on
// other workgroups (the decode plan runs as three launches), so no result
// depends on all of a launch's workgroups being resident together.
int table_forward(const tm_table_layer *t, const tm_layer_io *io, void *workspace, size_t workspace_bytes,
                  void *const *stage_events, bool wait_plans, tm_stream_t stream) {
  TM_REQUIRE(t && io, TM_EINVAL_ARG, "tm_table_forward: null descriptor");
  const int64_t n = io->n_tokens;
  TM_REQUIRE(n >= 0, TM_EINVAL_SHAPE, "tm_table_forward: negative token count");
  if (n == 0) return TM_OK;
  TM_REQUIRE(io->weights && io->expert_ids && io->q && io->q_sqnorm && io->dist && io->idx && io->keep,
             TM_EINVAL_ARG, "tm_table_forward: intermediate buffers missing");
  const WsLayout w = layout(t, n, io->n_nearest);
  TM_REQUIRE(workspace != nullptr || w.total == 0, TM_EWORKSPACE, "tm_table_forward: workspace missing");
  TM_REQUIRE(workspace_bytes >= w.total, TM_EWORKSPACE, "tm_table_forward: workspace %zu bytes < %zu",
             workspace_bytes, w.total);
  char *ws = static_cast<char *>(workspace);
  hipStream_t s = tm_hip_stream(stream);
  // The router's results are only consumed by the combine: without stage
  // events it rides in another launch (its own launch would be a few
  // latency-bound workgroups that leave the chip idle) and its stage interval
  // is empty.
  const tm_route_args ra{io->router_logits, io->ld_logits, io->n_experts, io->router_top_k, io->weights,
                         io->expert_ids};
  const bool route_fused = stage_events == nullptr && tm_internal_route_fusable(&ra);
  const int64_t n_keep = tm_keep_count(n, io->keep_rate);
  TM_REQUIRE((io->flags & ~TM_LAYER_NO_COMBINE) == 0, TM_EINVAL_ARG, "tm_table_forward: unknown flags 0x%x",
             (unsigned)io->flags);
  const bool combine = (io->flags & TM_LAYER_NO_COMBINE) == 0;
  int st;
  if (combine && tm_internal_decode_ok(t, io)) {  // the finishing launch also combines
    if ((st = decode_stages(t, io, w, ws, ra, route_fused, n_keep, stage_events, wait_plans, s)) != TM_OK)
      return st;
    return record(stage_events, 5, s);
  }
  const bool fused = fused_top1_ok(t, io);
  // ranked plans decide the keep set in the combine
  const bool ranked = combine && (fused ? ranked_ok(t, io) : general_ranked_ok(t, io));
  st = fused ? fused_top1_stages(t, io, w, ws, ra, route_fused, ranked, n_keep, stage_events, s)
             : general_stages(t, io, w, ws, ra, route_fused, ranked, n_keep, stage_events, s);
  if (st != TM_OK) return st;
  if ((st = record(stage_events, 4, s)) != TM_OK) return st;
  if (!combine) return record(stage_events, 5, s);
  if (ranked)
    st = tm_internal_combine_rank(t->dtype, n, t->hidden, io->slot_out, io->so_b, io->so_s, io->weights,
                                  io->router_top_k, io->router_top_k, t->values, t->n_cent, t->ld_v, io->idx,
                                  io->dist, io->residual, io->ld_r, io->out, io->ld_o, n_keep, io->keep, s);
  else
    st = tm_gather_combine(t->dtype, n, t->hidden, io->keep, io->slot_out, io->so_b, io->so_s, io->weights,
                           io->router_top_k, io->router_top_k, t->values, t->n_cent, t->ld_v, io->idx, io->dist,
                           io->n_nearest, io->n_nearest, io->residual, io->ld_r, io->out, io->ld_o, stream);
  if (st != TM_OK) return st;
  return record(stage_events, 5, s);
}

}  // namespace

extern "C" int tm_table_forward(const tm_table_layer *t, const tm_layer_io *io, void *workspace,
                                size_t workspace_bytes, void *const *stage_events, tm_stream_t stream) {
  return table_forward(t, io, workspace, workspace_bytes, stage_events, true, stream);
}

extern "C" int tm_table_forward_noalloc(const tm_table_layer *t, const tm_layer_io *io, tm_stream_t stream) {
  TM_REQUIRE(t && io, TM_EINVAL_ARG, "tm_table_forward_noalloc: null descriptor");
  TM_REQUIRE(io->n_tokens >= 0, TM_EINVAL_SHAPE, "tm_table_forward_noalloc: negative token count");
  if (io->n_tokens == 0) return TM_OK;
  const size_t need = layout(t, io->n_tokens, io->n_nearest).total;
  TM_REQUIRE(need <= (size_t)TM_NOALLOC_SCRATCH_BYTES, TM_EWORKSPACE,
             "tm_table_forward_noalloc: the layer needs %zu bytes of scratch > TM_NOALLOC_SCRATCH_BYTES (%zu)", need,
             (size_t)TM_NOALLOC_SCRATCH_BYTES);
  void *ws = nullptr;
  const int st = scratch_for_current_device(tm_hip_stream(stream), &ws);
  if (st != TM_OK) return st;
  // No plan whose workgroups wait for each other: such a wait that runs out
  // is reported only in the workspace's error word, which a caller of this
  // entry point cannot read.
  return table_forward(t, io, ws, (size_t)TM_NOALLOC_SCRATCH_BYTES, nullptr, false, stream);
}
