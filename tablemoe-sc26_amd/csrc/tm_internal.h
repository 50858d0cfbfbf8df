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
