// Library-internal entry points shared between translation units (not part
// of the C ABI; hidden from the shared object's symbol table).
#pragma once

#include "tm_common.h"

#define TM_NOT_FUSED (-1)

// Keep selection plus the router in one launch (routing workgroups after the
// selecting one).  TM_OK when launched, TM_NOT_FUSED when the shapes do not
// qualify (64 or 128 experts, top_k <= 8, 16-byte aligned logits rows).
__attribute__((visibility("hidden"))) int tm_internal_keep_route(
    const float *score, int64_t n, int64_t ld_score, int64_t n_keep, uint8_t *out_keep, const float *logits,
    int64_t ld_logits, int32_t n_experts, int32_t top_k, float *out_w, int64_t *out_ids, hipStream_t stream);
