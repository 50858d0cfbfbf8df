// Library-internal entry points shared between translation units (not part
// of the C ABI; hidden from the shared object's symbol table).
#pragma once

#include "tm_common.h"

// Router arguments for a launch that also routes (see tm_route_token).
struct tm_route_args {
  const float *logits;
  int64_t ld;
  int32_t n_experts;
  int32_t top_k;
  float *out_w;
  int64_t *out_ids;
};

// True when the router shape can ride in another launch: 64 or 128 experts,
// top_k <= 8, 16-byte aligned logits rows.
__attribute__((visibility("hidden"))) bool tm_internal_route_fusable(const tm_route_args *ra);

// tm_search_global whose split-merge launch also routes the n tokens (extra
// workgroups after the merging ones).  `ra` must be fusable.
__attribute__((visibility("hidden"))) int tm_internal_search_route(
    int32_t dtype, const void *q, int64_t n_tokens, int64_t ld_q, const float *q_sqnorm, const void *cents,
    int64_t n_cent, int64_t ld_c, const float *c_sqnorm, int32_t dim, int32_t top_k, int32_t metric,
    float *out_dist, int64_t *out_idx, void *workspace, size_t workspace_bytes, const tm_route_args *ra,
    hipStream_t stream);

// Column-split projection of packed P (no normalisation): q rows plus the
// partial squared norms qn_part[g][row] of column group g (dim / 64 groups,
// added in group order by the consumer).  With `keys` set, also resets the
// rows' packed top-1 search keys to ~0; with `ra` set, the launch also routes
// the n tokens (`ra` must be fusable).
__attribute__((visibility("hidden"))) bool tm_internal_project_cols_ok(
    int32_t dtype, const void *x, int64_t n, int32_t hidden, int64_t ld_x, const void *pv, const void *bv,
    const void *pt, const void *bt, int64_t ps_h, int64_t ps_d, int32_t dim, const void *q, int64_t ld_q);
__attribute__((visibility("hidden"))) size_t tm_internal_project_cols_parts(int32_t dim, int64_t n, int32_t hidden);
__attribute__((visibility("hidden"))) int tm_internal_project_cols(
    int32_t dtype, const void *x, int64_t n, int32_t hidden, int64_t ld_x, const uint8_t *is_vision,
    const void *pv, const void *bv, const void *pt, const void *bt, int64_t ps_h, int64_t ps_d, int32_t dim,
    void *q, int64_t ld_q, float *qn_part, uint64_t *keys, const tm_route_args *ra, hipStream_t stream);

// Top-1 global search that merges its centroid ranges by an atomic minimum of
// packed keys (orderable(dp) << 32 | centroid) into keys[n] (reset to ~0
// beforehand): no split-merge launch.  Only the shapes that run the pipelined
// top-1 kernel qualify.
__attribute__((visibility("hidden"))) bool tm_internal_search_keys_ok(int32_t dtype, int64_t n, int64_t n_cent,
                                                                      int64_t ld_c, int32_t dim, int32_t top_k);
__attribute__((visibility("hidden"))) int tm_internal_search_keys(
    int32_t dtype, const void *q, int64_t n, int64_t ld_q, const void *cents, int64_t n_cent, int64_t ld_c,
    const float *c_sqnorm, int32_t dim, int32_t metric, uint64_t *keys, hipStream_t stream);

// The same search for large n (wide kernel: 8-wave workgroups, one per CU):
// the workgroup that finishes a 256-query tile last also decodes the tile's
// keys into dist[i], idx[i] and q_sqnorm[i] (|q|^2 = the sum of `parts`
// partial norms qn_part[p][i]).  `cnt` holds one arrival counter per tile
// (cnt[tile * kTmCntStride]), zero before the call and left zero.  tm_internal_search_decode_tiles gives
// the tile count (0: shape not supported).
// Arrival counters handed to tm_internal_search_decode sit kTmCntStride words
// apart (one 128-byte line each: 256 workgroups count on 16 counters, and
// counters sharing a line serialise one another).
constexpr int kTmCntStride = 32;
__attribute__((visibility("hidden"))) int64_t tm_internal_search_decode_tiles(int32_t dtype, int64_t n,
                                                                              int64_t n_cent, int64_t ld_q,
                                                                              int64_t ld_c, int32_t dim);
__attribute__((visibility("hidden"))) int tm_internal_search_decode(
    int32_t dtype, const void *q, int64_t n, int64_t ld_q, const void *cents, int64_t n_cent, int64_t ld_c,
    const float *c_sqnorm, int32_t dim, int32_t metric, uint64_t *keys, const float *qn_part, int32_t parts,
    float *out_dist, int64_t *out_idx, float *out_qn, uint32_t *cnt, hipStream_t stream);

// tm_gather_combine for top-1 tables whose keep set is not yet known: each
// token's workgroup ranks its distance among all n (larger first, ties ->
// lower index), keeps the token when fewer than n_keep are ahead of it and
// writes keep[i] (the set tm_keep_select gives).  Shapes: 16-bit data,
// top_k 6 or 8, contiguous 16-byte aligned dist.
__attribute__((visibility("hidden"))) bool tm_internal_combine_rank_ok(int32_t dtype, int32_t hidden,
                                                                       const void *slot_out, int64_t so_b,
                                                                       int64_t so_s, int32_t top_k,
                                                                       const void *values, int64_t ld_v,
                                                                       const float *dist, const void *residual,
                                                                       int64_t ld_r, const void *out, int64_t ld_o);
__attribute__((visibility("hidden"))) int tm_internal_combine_rank(
    int32_t dtype, int64_t n_tokens, int32_t hidden, const void *slot_out, int64_t so_b, int64_t so_s,
    const float *weights, int64_t ld_w, int32_t top_k, const void *values, int64_t n_cent, int64_t ld_v,
    const int64_t *idx, const float *dist, const void *residual, int64_t ld_r, void *out, int64_t ld_o,
    int64_t n_keep, uint8_t *keep_out, hipStream_t stream);

// tm_keep_select over the distances the packed keys give (|q|^2 = the sum of
// `parts` partial norms qn_part[p][i]); also writes dist[i], idx[i] and
// q_sqnorm[i].  n <= 16384.
__attribute__((visibility("hidden"))) bool tm_internal_keep_keys_ok(int64_t n);
__attribute__((visibility("hidden"))) int tm_internal_keep_keys(const uint64_t *keys, const float *qn_part,
                                                                int32_t parts, int32_t metric, int64_t n,
                                                                int64_t n_keep, float *out_dist,
                                                                int64_t *out_idx, float *out_qn,
                                                                uint8_t *out_keep, hipStream_t stream);

// Leading dimension of the decode plan's best-key replicas: each replica
// starts on a 128-byte line of its own (16 keys), so the atomic minima on
// different replicas never meet on one line.
__host__ __device__ inline int64_t tm_key_stride(int64_t n) { return (n + 15) / 16 * 16; }

// Decode plan, search stage: the small-batch stream kernel (n <= 64) alone.
// Split s writes the sorted top-k lists of its centroid range into
// lists[(s * n + r) * list_len] and the best key of each query into
// keys[(s % key_rep) * tm_key_stride(n) + r] by atomic minimum (every replica
// reset to ~0 beforehand).  tm_internal_stream_nsplit gives the split count (0 when the
// shape is not a stream shape); list_len is 1, 4 or 8 for top_k 1, 2..4, 5..8.
__attribute__((visibility("hidden"))) int64_t tm_internal_stream_nsplit(int64_t n, int64_t n_cent, int32_t dim,
                                                                        int32_t top_k);
__attribute__((visibility("hidden"))) int tm_internal_search_stream(
    int32_t dtype, const void *q, int64_t n, int64_t ld_q, const void *cents, int64_t n_cent, int64_t ld_c,
    const float *c_sqnorm, int32_t dim, int32_t top_k, int32_t metric, uint64_t *lists, uint64_t *keys,
    int32_t key_rep, hipStream_t stream);

// Decode plan of tm_table_forward (n <= 64): three launches — split
// projection (+ router, + key reset), stream search, and one finishing launch
// that merges the lists, ranks the keep set and gathers/combines per (token,
// row chunk).  With stage events, events 2 / 3 / 4 are recorded after the
// projection / search / search (the keep select rides in the finishing
// launch).  `cnt` holds one arrival counter per (16-row tile, 16-column
// block): zero before the first call, left zero by every call.  With
// `one_launch` false the plan never takes its one-launch form (whose
// workgroups wait for each other and need to be resident together): the
// three launches hand data on only through the last arrival of each group.
struct tm_decode_ws {
  uint64_t *lists;  // search lists [nsplit][n][list_len]
  uint64_t *keys;   // best keys [tm_internal_decode_keys(n)]
  float *qn_blk;    // partial |q|^2 [n][dim / 16]
  void *part;       // projection partials [tm_internal_decode_part_bytes]
  uint32_t *cnt;    // arrival counters [ceil(n / 16) * dim / 16] (<= 64)
};
__attribute__((visibility("hidden"))) bool tm_internal_decode_ok(const tm_table_layer *t, const tm_layer_io *io);
__attribute__((visibility("hidden"))) size_t tm_internal_decode_qn_floats(int64_t n, int32_t dim);
__attribute__((visibility("hidden"))) size_t tm_internal_decode_keys(int64_t n);
__attribute__((visibility("hidden"))) size_t tm_internal_decode_part_bytes(int64_t n, int32_t dim);
__attribute__((visibility("hidden"))) int tm_internal_decode_forward(const tm_table_layer *t, const tm_layer_io *io,
                                                                     const tm_decode_ws &w, const tm_route_args *ra,
                                                                     int64_t n_keep, void *const *stage_events,
                                                                     bool one_launch, hipStream_t stream);
