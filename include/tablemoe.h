/*
 * tablemoe.h -- C ABI of the MI355X (gfx950) table-search path of TableMoE.
 *
 * Every entry point takes device pointers, element counts, element strides
 * and a HIP stream (hipStream_t passed as void*; NULL = the legacy default
 * stream), enqueues its kernels on that stream and returns without a host
 * synchronisation.  Nothing here allocates device memory: outputs and
 * workspaces are caller-provided.  No global mutable state; calls on
 * different streams are independent as long as their buffers are.
 *
 * Return value: TM_OK or one of the TM_E* codes below; tm_last_error()
 * gives a message for the calling thread's last failure.
 *
 * Booleans are bytes (0/1), as torch.bool.  Indices are int64 (torch.long).
 * "dtype" selects the element type of the model-dtype operands:
 * TM_DT_F32, TM_DT_F16 or TM_DT_BF16.
 *
 * Two families of entry points:
 *   - reference semantics ("mode R"): the per-(expert, modality) tables of
 *     table_moe/cache_engine (keys [E,2,K,d], values [E,2,K,H]), gated
 *     dot/cosine search, expert keep masks, slot combine, online window.
 *   - global-table semantics ("mode G"): one table of C centroids [C,d] with
 *     cached outputs [C,H]; L2 top-k search, token keep-by-distance, gather +
 *     combine + residual.  These serve the north-star configs; the reference
 *     has no counterpart beyond the reference entry points they generalise,
 *     cited on each.
 */
#ifndef TABLEMOE_H
#define TABLEMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define TM_OK 0
#define TM_EINVAL_SHAPE 1 /* a size or stride is out of range             */
#define TM_EINVAL_DTYPE 2 /* unsupported dtype tag for this entry point   */
#define TM_EINVAL_ARG 3   /* a required pointer is NULL, bad enum value   */
#define TM_EHIP 4         /* a HIP runtime call failed (launch error)     */
#define TM_EWORKSPACE 5   /* workspace missing or too small               */

/* ---- dtype tags ------------------------------------------------------ */
#define TM_DT_F32 0
#define TM_DT_F16 1
#define TM_DT_BF16 2

/* ---- hit comparators (max score vs threshold) ------------------------ */
#define TM_CMP_GE 0 /* hit = max >= threshold */
#define TM_CMP_GT 1 /* hit = max >  threshold */

/* ---- metrics of the global table ------------------------------------- */
#define TM_METRIC_L2 0  /* ascending ||q - c||^2 */
#define TM_METRIC_DOT 1 /* descending q . c      */

/* ---- renormalisation targets ----------------------------------------- */
#define TM_TARGET_ONE 0      /* surviving weights rescaled to sum 1           */
#define TM_TARGET_ORIG_SUM 1 /* rescaled to the row's original sum (DeepSeek) */
#define TM_TARGET_GIVEN 2    /* rescaled to a caller-given per-row target     */

typedef void *tm_stream_t;

/* Library version (major*10000 + minor*100 + patch). */
int tm_version(void);
/* Static string naming a status code. */
const char *tm_status_string(int status);
/* Message of the calling thread's last failing call ("" if none). */
const char *tm_last_error(void);

/* ======================================================================
 * a1 -- router softmax + top-k.
 * Replaces qwen_topk_softmax (table_moe/ops/qwen_topk_softmax.py:122-154;
 * binding table_moe/ops/csrc/qwen_topk_softmax/qwen_topk_softmax_bindings.cpp:5-23).
 * logits [n_tokens, n_experts] fp32 (row stride ld_logits); outputs
 * [n_tokens, top_k] contiguous: fp32 softmax probabilities in descending
 * order (ties -> lower expert id) and int64 expert ids.  renormalize != 0
 * divides the k weights by their sum (clamped to 1e-20), as normalize_topk.
 * Limits: 1 <= top_k <= min(n_experts, 32), n_experts <= 4096.
 * ====================================================================== */
int tm_topk_softmax(const float *logits, int64_t n_tokens, int32_t n_experts, int64_t ld_logits,
                    int32_t top_k, int32_t renormalize, float *out_weights, int64_t *out_ids,
                    tm_stream_t stream);

/* ======================================================================
 * a4 -- projection of hidden states into the PCA space.
 * Replaces VectorSearchEngine._project_queries_into + _normalize_last_dim
 * (table_moe/cache_engine/search.py:476-498, :12-21).
 * q[b] = dtype(x[b] @ P_m + bias_m), m = vision if is_vision[b] else text
 * (is_vision NULL: all vision; proj_txt/bias_txt NULL: the vision pair is
 * shared).  normalize != 0: q = dtype(fp32(q / dtype(||q||))) and rows with
 * ||q|| <= eps become 0.  x [n, hidden] (row stride ld_x), bias_m [dim],
 * P_m element (h, j) at P_m[h*ps_h + j*ps_d] with ps_d == 1 (the reference's
 * row-major [hidden, dim]) or ps_h == 1 (a k-contiguous transposed copy),
 * or ps_h == ps_d == 0: P_m in the packed layout written by tm_project_pack
 * (F16/BF16, the fast path: every matrix-core operand is one contiguous
 * load).  q_out [n, dim] (row stride ld_q).  q_sqnorm (nullable) receives
 * sum_j q[b,j]^2 in fp32 of the stored (rounded) q.
 * workspace (nullable): >= tm_project_workspace_size(n, hidden, dim) bytes
 * lets the strided layouts split `hidden` over workgroups (fp32 partials
 * summed in a fixed order, so results do not depend on it); without it one
 * workgroup walks all of `hidden` for its rows.  The packed layout needs no
 * workspace.
 * Limits: dim <= 256; hidden % 8 == 0 and dim in {16, 32, 64, 128, 256} for
 * F16/BF16 (MFMA path; required for the packed layout, whose bias pointers
 * must also be 16-byte aligned).
 * ====================================================================== */
size_t tm_project_workspace_size(int64_t n_tokens, int32_t hidden, int32_t dim);

/* Packed projection layout (no reference counterpart: an on-device re-layout
 * of the reference's [hidden, dim] PCA matrix, made once when a table is
 * loaded).  For k-step t < ceil(hidden/32), column block c < dim/16 and lane
 * l < 64, the 8 elements at 16-byte chunk (t*(dim/16) + c)*64 + l are
 * P[32t + 8(l/16) + e][16c + l%16], e = 0..7, zero where the row index
 * reaches `hidden`.  Source element (h, j) at src[h*ps_h + j*ps_d] (any
 * strides).  Limits: F16/BF16, dim in {16, 32, 64, 128, 256}. */
size_t tm_project_packed_size(int32_t hidden, int32_t dim, int32_t dtype);
int tm_project_pack(int32_t dtype, const void *src, int32_t hidden, int32_t dim, int64_t ps_h, int64_t ps_d,
                    void *packed, size_t packed_bytes, tm_stream_t stream);
int tm_project(int32_t dtype, const void *x, int64_t n_tokens, int32_t hidden, int64_t ld_x,
               const uint8_t *is_vision, const void *proj_vis, const void *bias_vis,
               const void *proj_txt, const void *bias_txt, int64_t ps_h, int64_t ps_d,
               int32_t dim, int32_t normalize, float eps, void *q_out, int64_t ld_q, float *q_sqnorm,
               void *workspace, size_t workspace_bytes, tm_stream_t stream);

/* ======================================================================
 * a5/a6/a7 -- gated search of each reused (token, slot) in the table of its
 * routed expert and modality.
 * Replaces the prefill/decode offline search of VectorSearchEngine
 * (table_moe/cache_engine/search.py:515-602 cosine, :661-697 dot, Triton
 * kernels :35-256).
 * For b < n_tokens, s < top_k: searched = reuse[b,s] (reuse NULL: all) and
 * s >= col_offset and 0 <= sel[b,s] < n_experts.  If searched:
 * score_c = q[b] . keys[sel[b,s], m(b), c] (fp32 accumulation), max over
 * c < n_centroids (first index on ties), hit = max >= thr (TM_CMP_GE) or
 * > thr (TM_CMP_GT), thr = thr_vision or thr_text by modality.
 * Writes every (b, s): (1, argmax) on a hit, (0, 0) otherwise.
 * keys element strides (ks_e, ks_m, ks_c), unit stride along dim.
 * Limits: dim <= 256, n_centroids <= 65536.
 * ====================================================================== */
int tm_search_gated(int32_t dtype, const void *q_low, int64_t n_tokens, int64_t ld_q,
                    const void *keys, int64_t n_experts, int64_t n_centroids, int32_t dim,
                    int64_t ks_e, int64_t ks_m, int64_t ks_c, const int64_t *sel, int32_t top_k,
                    int64_t ss_b, int64_t ss_s, const uint8_t *is_vision, const uint8_t *reuse,
                    int64_t rs_b, int64_t rs_s, int32_t col_offset, float thr_vision,
                    float thr_text, int32_t cmp, uint8_t *out_hit, int64_t *out_idx,
                    int64_t os_b, int64_t os_s, tm_stream_t stream);

/* ======================================================================
 * a8 -- decode hybrid search: online window first, offline table second.
 * Replaces VectorSearchEngine.search_decode_hybrid /
 * search_decode_hybrid_bs1_into (table_moe/cache_engine/search.py:839-954,
 * :987-1105; Triton kernel :258-385; fallback :778-806).
 * Slots s >= keep_k of each token b are searched.  Online (n_online_valid > 0):
 * score_j = x[b] . online_keys[j] for j < n_online_valid, (max, first argmax j*);
 * if max > 0: on_idx[b] = j*, and slot s is an online hit when sel[b,s] is
 * among online_ids[j*, 0:online_topk] (on_slot = first matching position).
 * Slots that are not online hits are searched offline with the raw
 * projection q = dtype(x @ P_m + bias_m) against keys with hit = max >= 0.
 * All outputs are written for every (b, s): on_hit/off_hit 0, on_slot/off_idx
 * 0, on_idx -1 where nothing was found.  q_out (nullable, row stride
 * ld_q_out) receives the projected queries when any slot is searched.
 * workspace: >= tm_search_hybrid_workspace_size(n_tokens, hidden, dim) bytes
 * (16-byte aligned): fp32 projection partials and window scores.
 * Limits: n_online_valid <= 1024, online_topk <= 64, dim <= 256.
 * ====================================================================== */
size_t tm_search_hybrid_workspace_size(int64_t n_tokens, int32_t hidden, int32_t dim);
int tm_search_hybrid(int32_t dtype, const void *x, int64_t n_tokens, int32_t hidden, int64_t ld_x,
                     const uint8_t *is_vision, const void *proj_vis, const void *bias_vis,
                     const void *proj_txt, const void *bias_txt, int64_t ps_h, int64_t ps_d,
                     int32_t dim, const void *online_keys, int64_t ld_online, int32_t n_online_valid,
                     const int64_t *online_ids, int32_t online_topk, int64_t ld_online_ids,
                     const void *keys, int64_t n_experts, int64_t n_centroids, int64_t ks_e,
                     int64_t ks_m, int64_t ks_c, const int64_t *sel, int32_t top_k, int64_t ss_b,
                     int64_t ss_s, int32_t keep_k, uint8_t *on_hit, int64_t *on_idx,
                     uint8_t *off_hit, int64_t *off_idx, int64_t *on_slot, int64_t os_b,
                     int64_t os_s, void *q_out, int64_t ld_q_out, void *workspace, size_t workspace_bytes,
                     tm_stream_t stream);

/* ======================================================================
 * a3 -- keep masks.
 * tm_fixed_keep_mask replaces build_fixed_keep_mask / build_decode_keep_mask
 * (table_moe/skip/pruning.py:4-15, :51-52): out[b,s] = s < keep_k.
 * tm_expert_keep_mask replaces build_prefill_keep_mask
 * (table_moe/skip/pruning.py:18-48): score[e] = sum of attn[b]*w[b,s] over
 * slots routed to e (attn NULL: w[b,s]/n_tokens), summed in a fixed order;
 * the max(1, int(n_active*keep_rate)) highest-scoring activated experts are
 * kept (equal scores: lower id first); out[b,s] = kept(sel[b,s]).
 * workspace: >= tm_expert_keep_mask_workspace_size(n_tokens, n_experts).
 * Limits: n_experts <= 1024.
 * ====================================================================== */
int tm_fixed_keep_mask(int64_t n_tokens, int32_t top_k, int32_t keep_k, uint8_t *out,
                       tm_stream_t stream);
size_t tm_expert_keep_mask_workspace_size(int64_t n_tokens, int32_t n_experts);
int tm_expert_keep_mask(const int64_t *sel, const float *weights, const float *attn,
                        int64_t n_tokens, int32_t top_k, int32_t n_experts, double keep_rate,
                        uint8_t *out_mask, float *out_expert_scores, void *workspace,
                        size_t workspace_bytes, tm_stream_t stream);

/* ======================================================================
 * a11 -- surviving-weight renormalisation.
 * Replaces renormalize_surviving_weights (table_moe/skip/pruning.py:55-73).
 * out[b,:] = (w*m) / sum(w*m) * target, 0 for rows whose kept sum is not > 0;
 * target = 1 (TM_TARGET_ONE), the row's original sum (TM_TARGET_ORIG_SUM) or
 * target[b * ld_t] (TM_TARGET_GIVEN, dtype of the weights).
 * Each step rounds to the weights' dtype as the torch ops do.
 * w [n, k] (row stride ld_w), mask [n, k] (row stride ld_m), out contiguous.
 * ====================================================================== */
int tm_renormalize(int32_t dtype, const void *weights, int64_t ld_w, const uint8_t *mask,
                   int64_t ld_m, int64_t n_tokens, int32_t top_k, int32_t target_mode,
                   const void *target, int64_t ld_t, void *out, tm_stream_t stream);

/* ======================================================================
 * a10 -- gather of cached rows.
 * Replaces HybridStorageManager.gather_values / gather_values_decode_bs1
 * (table_moe/cache_engine/manager.py:212-228).
 * out[dst(i)] = values[eids[i], mids[i], cids[i]] (a row of `hidden`
 * elements), dst(i) = dst_rows[i] (NULL: i).  mids NULL: modality
 * `modality`.  values element strides (vs_e, vs_m, vs_c), unit along hidden.
 * out has n_out_rows rows of stride ld_out; a destination outside
 * [0, n_out_rows) is skipped, a source index out of range zero-fills its row.
 * ====================================================================== */
int tm_gather_rows(int32_t dtype, const void *values, int64_t n_experts, int64_t n_centroids,
                   int32_t hidden, int64_t vs_e, int64_t vs_m, int64_t vs_c, const int64_t *eids,
                   const int64_t *mids, int32_t modality, const int64_t *cids, int64_t n_rows,
                   const int64_t *dst_rows, void *out, int64_t n_out_rows, int64_t ld_out,
                   tm_stream_t stream);

/* ======================================================================
 * a10+a11 -- fused gather + combine of one MoE layer's slots (reference
 * semantics), with optional residual.
 * Fuses the collected-buffer fill and the weighted sum of
 * QwenMoeWrapperCached.forward (table_moe/models/qwen3_vl_moe/cached_layers.py:
 * 439-465) and DeepSeekMoeWrapperCached.forward
 * (table_moe/models/deepseek_vl2/deepseek_layers.py:695-729):
 * slot (b,s) source = computed[b,s] if compute_mask, else
 * online_values[on_idx[b], on_slot[b,s]] if on_hit, else
 * values[sel[b,s], m(b), off_idx[b,s]] if off_hit, else dropped.
 * Surviving weights renormalised per target_mode (rounded to dtype for
 * TM_TARGET_ONE, as the reference's .to(dtype)), y = sum_s w~ * source in fp32,
 * out = dtype(y) or dtype(residual + y).
 * computed [n, k, hidden] (strides cs_b, cs_s), weights fp32 [n, k]
 * (row stride ld_w), masks/indices [n, k] with row stride ld_m,
 * online_values [W, online_topk, hidden] (strides ov_w, ov_s) or NULL.
 * ====================================================================== */
int tm_slot_combine(int32_t dtype, int64_t n_tokens, int32_t top_k, int32_t hidden,
                    const float *weights, int64_t ld_w, const uint8_t *compute_mask,
                    const void *computed, int64_t cs_b, int64_t cs_s, const uint8_t *off_hit,
                    const int64_t *off_idx, const int64_t *sel, int64_t ld_m,
                    const uint8_t *is_vision, const void *values, int64_t n_experts,
                    int64_t n_centroids, int64_t vs_e, int64_t vs_m, int64_t vs_c,
                    const uint8_t *on_hit, const int64_t *on_idx, const int64_t *on_slot,
                    const void *online_values, int64_t n_online, int32_t online_topk,
                    int64_t ov_w, int64_t ov_s, int32_t target_mode, const void *residual,
                    int64_t ld_r, void *out, int64_t ld_out, tm_stream_t stream);

/* ======================================================================
 * a12 -- online window ring-buffer write.
 * Replaces the copies of HybridStorageManager.update_online_cache /
 * update_online_cache_bs1 (table_moe/cache_engine/manager.py:89-155).
 * Row i < n_rows goes to ring row (start + i) % ring_size: keys <- hidden[i],
 * ids <- ids[i] (-1 where valid[i,s] == 0), values <- outputs[i] (0 where
 * invalid).  valid NULL: all valid.  n_rows <= ring_size.  The caller keeps
 * the host-side ring pointer (as the reference does).
 * ====================================================================== */
int tm_online_update(int32_t dtype, const void *hidden, int64_t ld_h, const int64_t *ids,
                     int64_t ld_ids, const void *outputs, int64_t os_b, int64_t os_s,
                     const uint8_t *valid, int64_t ld_valid, int64_t n_rows, int32_t top_k,
                     int32_t hidden_dim, int64_t start, int64_t ring_size, void *ring_keys,
                     int64_t *ring_ids, void *ring_values, tm_stream_t stream);

/* ======================================================================
 * Mode G (global table) -- north-star kernels (1)-(4).
 * ====================================================================== */

/* ||c||^2 of each centroid in fp32 (table load time). */
int tm_centroid_sqnorms(int32_t dtype, const void *cents, int64_t n_cent, int32_t dim,
                        int64_t ld_c, float *out, tm_stream_t stream);

/* (1)+(2): nearest centroids of each query.
 * Generalises the offline search (table_moe/cache_engine/search.py:566-602)
 * to one global table with L2 or dot metric and top-k.
 * q [n, dim] dtype (row stride ld_q); cents [C, dim] (row stride ld_c);
 * q_sqnorm (nullable: computed) and c_sqnorm (required for L2) fp32.
 * L2: dist = ||q||^2 - 2 q.c + ||c||^2 in fp32, ascending; DOT: q.c
 * descending; ties -> lower centroid index.  out_dist/out_idx [n, top_k].
 * workspace >= tm_search_global_workspace_size(...).
 * Limits: dim in {64, 128, 256}, 1 <= top_k <= 8; dtype F16 or BF16 (matrix
 * cores) or F32 (fp32 FMAs in dimension order: the CPU-reference config);
 * 16-byte aligned rows. */
size_t tm_search_global_workspace_size(int64_t n_tokens, int64_t n_cent, int32_t dim,
                                       int32_t top_k);
int tm_search_global(int32_t dtype, const void *q, int64_t n_tokens, int64_t ld_q,
                     const float *q_sqnorm, const void *cents, int64_t n_cent, int64_t ld_c,
                     const float *c_sqnorm, int32_t dim, int32_t top_k, int32_t metric,
                     float *out_dist, int64_t *out_idx, void *workspace, size_t workspace_bytes,
                     tm_stream_t stream);

/* (3): keep the n_keep tokens of largest score (ties -> lower token index);
 * out_keep[i] = 1 for kept tokens.  tm_keep_count gives
 * max(1, floor(n * keep_rate)) clamped to n (table_moe/skip/pruning.py:45).
 * score: fp32 [n] with row stride ld_score (e.g. column 0 of [n, top_k]). */
int64_t tm_keep_count(int64_t n, double keep_rate);
size_t tm_keep_select_workspace_size(int64_t n);
int tm_keep_select(const float *score, int64_t n, int64_t ld_score, int64_t n_keep,
                   uint8_t *out_keep, void *workspace, size_t workspace_bytes,
                   tm_stream_t stream);

/* (4): gather + combine + residual.
 * out[i] = dtype(residual[i] + y_i), y_i = sum_s w~[i,s] * slot_out[i,s]
 * (w~ = w / sum w) for kept tokens; y_i = sum_j beta_ij values[idx[i,j]]
 * (beta ~ 1/(dist+1e-6), normalised; beta = 1 for n_nearest = 1) otherwise.
 * residual NULL: no residual.  slot_out is read only for kept tokens.
 * Strides: slot_out (so_b, so_s), values ld_v, residual ld_r, out ld_o,
 * weights ld_w, idx/dist ld_idx. */
int tm_gather_combine(int32_t dtype, int64_t n_tokens, int32_t hidden, const uint8_t *keep,
                      const void *slot_out, int64_t so_b, int64_t so_s, const float *weights,
                      int64_t ld_w, int32_t top_k, const void *values, int64_t n_cent,
                      int64_t ld_v, const int64_t *idx, const float *dist, int64_t ld_idx,
                      int32_t n_nearest, const void *residual, int64_t ld_r, void *out,
                      int64_t ld_o, tm_stream_t stream);

/* (3)+(4) in one launch for top-1 tables: tm_gather_combine (n_nearest = 1)
 * with the keep set decided from `dist` (fp32 [n], contiguous) instead of
 * read: token i is kept when fewer than n_keep tokens are ahead of it (a
 * larger distance, or the same at a lower index) -- the set tm_keep_select
 * gives -- and out_keep[i] is written.  No single counterpart in the
 * reference: it replaces the keep selection (table_moe/skip/pruning.py:45
 * count) followed by the gather + combine of tm_gather_combine.  dtype F16
 * or BF16, top_k 6 or 8, hidden <= 2048 and a multiple of 8, 16-byte aligned
 * rows and dist; each token's workgroup reads all n distances (the work grows
 * as n^2), so n_tokens <= TM_RANKED_MAX_TOKENS (TM_EINVAL_SHAPE beyond: run
 * tm_keep_select + tm_gather_combine instead). */
#define TM_RANKED_MAX_TOKENS 16384
int tm_gather_combine_ranked(int32_t dtype, int64_t n_tokens, int32_t hidden, const void *slot_out,
                             int64_t so_b, int64_t so_s, const float *weights, int64_t ld_w, int32_t top_k,
                             const void *values, int64_t n_cent, int64_t ld_v, const int64_t *idx,
                             const float *dist, const void *residual, int64_t ld_r, void *out, int64_t ld_o,
                             int64_t n_keep, uint8_t *out_keep, tm_stream_t stream);

/* ======================================================================
 * Online window, decode step of one token: the slot combine of
 * tm_slot_combine (n_tokens = 1) and the ring write of tm_online_update in
 * one launch.  Replaces the tail of QwenMoeWrapperCached._forward_decode_bs1
 * (table_moe/models/qwen3_vl_moe/cached_layers.py:213-267: online/offline
 * fills of collected, effective weights, matmul) together with
 * update_online_cache_bs1 (table_moe/cache_engine/manager.py:89-106).
 * Slot sources, coefficients and `out` are exactly tm_slot_combine's; then
 * ring row `ring_row` takes x (online_keys row stride = hidden), the slot
 * ids (-1 where the slot did not survive) and each slot's source row (zeros
 * where dropped).  A source in the overwritten row itself is read first.
 * top_k = online_topk <= 8; 16-byte aligned rows.  The caller advances its
 * ring pointer (as the reference's host-side online_ptr).
 * ====================================================================== */
int tm_decode_combine_update(int32_t dtype, int32_t top_k, int32_t hidden, const float *weights,
                             const uint8_t *compute_mask, const void *computed, int64_t cs_s, const uint8_t *off_hit,
                             const int64_t *off_idx, const int64_t *sel, const uint8_t *is_vision, const void *values,
                             int64_t n_experts, int64_t n_centroids, int64_t vs_e, int64_t vs_m, int64_t vs_c,
                             const uint8_t *on_hit, const int64_t *on_idx, const int64_t *on_slot,
                             void *online_values, int64_t n_online, int32_t online_topk, int64_t ov_w, int64_t ov_s,
                             int32_t target_mode, const void *residual, void *out, const void *x, void *online_keys,
                             int64_t *online_ids, int64_t ring_row, tm_stream_t stream);

/* ======================================================================
 * Importance for the expert-level keep rule: attention probabilities of the
 * last query over every key, averaged over heads.
 * Replaces HybridQwen3Attention._compute_and_cache_importance
 * (models/qwen3_vl_moe/hybrid_attention.py:111-146) and the DeepSeek
 * _cache_last_token_attention (models/deepseek_vl2/deepseek_attention.py:
 * 206-249); feeds tm_expert_keep_mask's `attn`.
 * q(b, h, d) = q[b*qs_b + h*qs_h + d]; k(b, t, g, d) = k[b*ks_b + t*ks_s +
 * g*ks_h + d]; head h reads KV head h / (n_heads / n_kv_heads) (the
 * reference's repeat_interleave).  Score of key t:
 *   TM_SCORE_MODEL  dtype(dtype(q . k) * scale)  (torch.matmul in the model
 *                   dtype, then `* scaling` in the model dtype: Qwen)
 *   TM_SCORE_F32    fp32(q . k) * scale          (fp32 einsum: DeepSeek)
 * (fp32 accumulation).  Keys with key_mask[b*km_b + t] == 0 get probability
 * 0 and leave the normalisation.  p = softmax over t in fp32;
 * out[b*ld_out + j] = mean over heads of p at key n_keys - out_len + j.
 * head_dim in {64, 128, 192, 256}; n_heads <= 256; n_keys <= 524288.
 * Workspace: tm_importance_workspace_size (scores and chunk statistics).
 * ====================================================================== */
#define TM_SCORE_MODEL 0
#define TM_SCORE_F32 1
size_t tm_importance_workspace_size(int64_t batch, int32_t n_heads, int64_t n_keys);
int tm_last_query_importance(int32_t dtype, const void *q, int64_t qs_b, int64_t qs_h, const void *k, int64_t ks_b,
                             int64_t ks_s, int64_t ks_h, int64_t batch, int32_t n_heads, int32_t n_kv_heads,
                             int32_t head_dim, int64_t n_keys, float scale, int32_t score_mode,
                             const uint8_t *key_mask, int64_t km_b, int64_t out_len, float *out, int64_t ld_out,
                             void *workspace, size_t workspace_bytes, tm_stream_t stream);

/* ======================================================================
 * Recompute path -- the SwiGLU expert MLP of the slots that are recomputed.
 * tm_expert_swiglu replaces fused_moe_ffn_fp16_into
 * (table_moe/ops/csrc/fp16_fused_expert/fp16_fused_moe_mlp.cu:107-274,
 * called by maybe_run_fp16_fused_expert, table_moe/ops/fp16_fused_expert.py:
 * 223-257) for one expert and any row count; tm_group_slots +
 * tm_grouped_swiglu replace the per-expert loop of
 * models/qwen3_vl_moe/cached_layers.py:431-437 (index_select the expert's
 * tokens, run the expert, scatter into collected[token, slot]).
 * Per row: g = dtype(x W1^T), f = dtype(silu(g) * (x W3^T)) (the up
 * projection unrounded, silu in fp32: the SiLU-mul epilogue of
 * fp16_epilogue_utils.h:51-125), y = dtype(f W2^T).  fp32 accumulation on
 * bf16/fp16 matrix cores.  Weights as nn.Linear stores them: W1, W3
 * [n_experts, inter, hidden], W2 [n_experts, hidden, inter], contiguous.
 * hidden and inter must be multiples of 128, inter * hidden < 2^30; x,
 * out, addend rows and the weights 16-byte aligned (row strides and
 * tm_grouped_swiglu's row_out offsets multiples of 8 elements: rows are
 * written in 16-byte pieces).  Workspace: the [rows, inter] intermediate
 * (tm_swiglu_workspace_size).
 * ====================================================================== */
size_t tm_swiglu_workspace_size(int64_t max_rows, int32_t inter, int32_t dtype);
int tm_expert_swiglu(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                     const void *w1, const void *w3, const void *w2, int32_t inter, void *out, int64_t ld_out,
                     void *workspace, size_t workspace_bytes, tm_stream_t stream);
/* tm_expert_swiglu with an addend folded into the down projection's
 * epilogue: y = dtype(addend + f W2^T) (fp32 sum, one rounding), addend
 * [n_rows, hidden] with row stride ld_add, not overlapping `out`.
 * For a DeepSeek layer's shared experts (models/deepseek_vl2/
 * deepseek_layers.py:743 adds them to the routed output, which the decoder
 * layer adds to the residual): with the residual as the addend, the shared
 * MLP writes residual + shared in one pass, and the table combine
 * (tm_gather_combine) adds the routed part on top. */
int tm_expert_swiglu_add(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                         const void *w1, const void *w3, const void *w2, int32_t inter, const void *addend,
                         int64_t ld_add, void *out, int64_t ld_out, void *workspace, size_t workspace_bytes,
                         tm_stream_t stream);
/* Buckets the recomputed (token, slot) pairs by expert, on the device (no
 * host sync): pair (b, s) is recomputed when mask[b*ms_b + s*ms_s] != 0
 * (ms_s = 0: a per-token flag) and 0 <= ids[b*ld_ids + s] < n_experts.
 * Writes expert_offsets [n_experts + 1], one row per pair (row_token = b,
 * row_out = b*so_b + s*so_s: the element offset of its output row), and
 * tiles [2 + 2*tm_group_slots_tiles(n_tokens*top_k, n_experts)]: row count,
 * tile count, then each 256-row tile's expert and first row.  The order of
 * rows inside an expert is unspecified; results do not depend on it.
 * so_b and so_s must be multiples of 8 elements (TM_EINVAL_SHAPE
 * otherwise). */
int64_t tm_group_slots_tiles(int64_t max_rows, int32_t n_experts);
int tm_group_slots(const int64_t *ids, int64_t n_tokens, int32_t top_k, int64_t ld_ids, const uint8_t *mask,
                   int64_t ms_b, int64_t ms_s, int32_t n_experts, int64_t so_b, int64_t so_s,
                   int32_t *expert_offsets, int32_t *row_token, int64_t *row_out, int32_t *tiles,
                   tm_stream_t stream);
/* tm_group_slots over several workgroups (no counterpart in the reference:
 * the same outputs, with the ids read by many CUs instead of one): for
 * 1 <= n_tokens <= 8192, 1 <= top_k <= 8 and 1 <= n_experts <= 256 two
 * launches -- per-workgroup expert counts into `workspace`
 * (tm_group_slots_workspace_size bytes, 16-byte aligned; TM_EWORKSPACE if
 * smaller), then the placement of each workgroup's rows after those of the
 * workgroups before it; other shapes run tm_group_slots (the workspace is
 * not used, and tm_group_slots_workspace_size returns 0).  Same contract as
 * tm_group_slots: the offsets, tile list and the set of rows of each expert
 * are the same; the order of rows inside an expert is unspecified. */
size_t tm_group_slots_workspace_size(int64_t n_tokens, int32_t top_k, int32_t n_experts);
int tm_group_slots_ws(const int64_t *ids, int64_t n_tokens, int32_t top_k, int64_t ld_ids, const uint8_t *mask,
                      int64_t ms_b, int64_t ms_s, int32_t n_experts, int64_t so_b, int64_t so_s,
                      int32_t *expert_offsets, int32_t *row_token, int64_t *row_out, int32_t *tiles,
                      void *workspace, size_t workspace_bytes, tm_stream_t stream);
/* The MLP of every grouped row: row r (expert e by expert_offsets) reads
 * x[row_token[r]] and writes out[row_out[r] .. + hidden).  max_rows bounds
 * the row count (n_tokens * top_k of the tm_group_slots call). */
int tm_grouped_swiglu(int32_t dtype, const void *x, int64_t ld_x, int32_t hidden, int32_t inter,
                      int32_t n_experts, const void *w1, const void *w3, const void *w2, int64_t max_rows,
                      const int32_t *expert_offsets, const int32_t *row_token, const int64_t *row_out,
                      const int32_t *tiles, void *out, void *workspace, size_t workspace_bytes,
                      tm_stream_t stream);
/* Packed expert weights (no counterpart in the reference: a device layout
 * of the same weights for tm_grouped_swiglu_packed).  Each tile of rows
 * that one GEMM workgroup multiplies keeps its place in the nn.Linear
 * layout but is reordered by 32-column stage, so a stage of the tile is one
 * contiguous block in the order the GEMM stages it through LDS (the plain
 * layout reads a 64-byte piece of each of the tile's rows per stage).
 * role TM_PACK_GATE_UP: w is W1 or W3 [n_experts, inter, hidden]; role
 * TM_PACK_DOWN: w is W2 [n_experts, hidden, inter].  out has w's size and
 * must not overlap it; pack once per weight set.  F16/BF16. */
#define TM_PACK_GATE_UP 0
#define TM_PACK_DOWN 1
int tm_expert_pack_weights(int32_t dtype, const void *w, int32_t n_experts, int32_t hidden, int32_t inter,
                           int32_t role, void *out, tm_stream_t stream);
/* tm_grouped_swiglu on weights packed by tm_expert_pack_weights (w1p and
 * w3p with TM_PACK_GATE_UP, w2p with TM_PACK_DOWN); the same results bit for
 * bit.  Its workspace holds the intermediate as whole 256-row tiles, each
 * stored stage by stage like the packed weights:
 * tm_grouped_swiglu_packed_workspace_size bytes. */
size_t tm_grouped_swiglu_packed_workspace_size(int64_t max_rows, int32_t inter, int32_t n_experts, int32_t dtype);
/* tm_expert_swiglu / tm_expert_swiglu_add (addend nullable) on one expert's
 * weights packed by tm_expert_pack_weights with n_experts = 1 (a DeepSeek
 * layer's shared experts); the same results bit for bit.  Workspace:
 * tm_grouped_swiglu_packed_workspace_size(n_rows, inter, 1, dtype). */
int tm_expert_swiglu_packed(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                            const void *w1p, const void *w3p, const void *w2p, int32_t inter, const void *addend,
                            int64_t ld_add, void *out, int64_t ld_out, void *workspace, size_t workspace_bytes,
                            tm_stream_t stream);
int tm_grouped_swiglu_packed(int32_t dtype, const void *x, int64_t ld_x, int32_t hidden, int32_t inter,
                             int32_t n_experts, const void *w1p, const void *w3p, const void *w2p, int64_t max_rows,
                             const int32_t *expert_offsets, const int32_t *row_token, const int64_t *row_out,
                             const int32_t *tiles, void *out, void *workspace, size_t workspace_bytes,
                             tm_stream_t stream);

/* ======================================================================
 * Mode G -- one MoE layer of the table path in ONE call.
 * Enqueues, back to back on `stream`: tm_topk_softmax (router) ->
 * tm_project -> tm_search_global -> tm_keep_select (n_keep =
 * tm_keep_count(n, keep_rate)) -> tm_gather_combine, with the semantics of
 * each of those entry points (for top-1 batches of up to 4096 tokens the
 * last two run as tm_gather_combine_ranked).  One FFI call per layer keeps host overhead
 * out of the layer time.  The table descriptor is fixed per layer; the I/O
 * descriptor names the token batch, the caller's output and intermediate
 * buffers.  `stage_events` (nullable) is an array of 6 hipEvent_t recorded
 * before the router and after each stage (timing hook).
 * ====================================================================== */
typedef struct tm_table_layer {
  int32_t dtype;            /* TM_DT_BF16, TM_DT_F16 or TM_DT_F32          */
  int32_t metric;           /* TM_METRIC_L2 or TM_METRIC_DOT               */
  int32_t dim;              /* PCA dimension (64, 128 or 256)              */
  int32_t hidden;           /* model hidden size                           */
  int64_t n_cent;           /* centroids                                   */
  const void *cents;        /* [n_cent, dim], row stride ld_c              */
  int64_t ld_c;
  const float *c_sqnorm;    /* [n_cent] (tm_centroid_sqnorms)              */
  const void *values;       /* cached outputs [n_cent, hidden], ld_v       */
  int64_t ld_v;
  const void *proj_vis;     /* P_m as in tm_project (ps_h, ps_d)           */
  const void *bias_vis;
  const void *proj_txt;     /* nullable: shared with vision                */
  const void *bias_txt;
  int64_t ps_h, ps_d;
} tm_table_layer;

typedef struct tm_layer_io {
  int64_t n_tokens;
  const void *x;            /* [n, hidden], row stride ld_x                */
  int64_t ld_x;
  const uint8_t *is_vision; /* [n] nullable (all vision)                   */
  const float *router_logits; /* [n, n_experts] fp32, row stride ld_logits */
  int64_t ld_logits;
  int32_t n_experts;
  int32_t router_top_k;
  int32_t n_nearest;        /* 1..8                                        */
  int32_t flags;            /* 0 or TM_LAYER_NO_COMBINE                    */
  double keep_rate;
  const void *slot_out;     /* [n, router_top_k, hidden] strides so_b, so_s */
  int64_t so_b, so_s;
  const void *residual;     /* [n, hidden] nullable, row stride ld_r       */
  int64_t ld_r;
  void *out;                /* [n, hidden], row stride ld_o                */
  int64_t ld_o;
  /* intermediates, caller buffers (contiguous): */
  float *weights;           /* [n, router_top_k]                           */
  int64_t *expert_ids;      /* [n, router_top_k]                           */
  void *q;                  /* [n, dim]                                    */
  float *q_sqnorm;          /* [n]                                         */
  float *dist;              /* [n, n_nearest]                              */
  int64_t *idx;             /* [n, n_nearest]                              */
  uint8_t *keep;            /* [n]                                         */
} tm_layer_io;

/* tm_layer_io.flags: stop after the keep set (weights, expert_ids, q,
 * q_sqnorm, dist, idx and keep are written; slot_out, residual and out are
 * not used), so a caller can recompute the kept tokens' slots and then run
 * tm_gather_combine itself (a DeepSeek-style layer whose recompute and
 * shared experts sit between the keep selection and the combine). */
#define TM_LAYER_NO_COMBINE 1

/* sizeof(tm_table_layer) for which == 0, sizeof(tm_layer_io) for which == 1
 * (lets a binding check its mirror of the two structs). */
size_t tm_struct_size(int32_t which);
/* Workspace of tm_table_forward.  Its first TM_LAYER_SYNC_BYTES bytes hold
 * arrival counters and flags (batches of at most 64 tokens hand the
 * projection and the search results between workgroups; larger top-1 batches
 * decode each query tile's search result in the tile's last workgroup): they
 * must be zero before the first call on a workspace (allocate it
 * zero-filled); every call leaves the counters zero and the flags at a
 * generation the next call continues from.  Calls that share one workspace
 * must not overlap (one stream).
 *
 * Batches of at most 64 tokens may run as one launch whose workgroups wait
 * for each other (bounded waits; the launch assumes its 128 workgroups can
 * be resident together, as on an otherwise idle device).  A wait that runs
 * out (20 ms) adds one to the uint32 at byte TM_LAYER_SYNC_ERR_BYTE of the
 * workspace; that call's outputs are then undefined (the row chunks the
 * waiting workgroup writes are NaN).  The library never clears the word
 * (zero = no wait ever ran out).  The return code cannot report such a
 * failure (the call returns before the kernels run): a caller that shares
 * the device with other work must read the word after the calls complete
 * and discard the outputs of any call during which it grew.  A workgroup of
 * such a call that started late may leave flags that a later call would
 * take for its own: after the word grew, zero the first
 * TM_LAYER_SYNC_BYTES of the workspace (the word included) before the next
 * call on it. */
#define TM_LAYER_SYNC_BYTES 16384
#define TM_LAYER_SYNC_ERR_BYTE 3584
size_t tm_table_forward_workspace_size(const tm_table_layer *table, int64_t n_tokens, int32_t n_nearest);
int tm_table_forward(const tm_table_layer *table, const tm_layer_io *io, void *workspace,
                     size_t workspace_bytes, void *const *stage_events, tm_stream_t stream);

/* ======================================================================
 * tm_table_forward without a workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same semantics and results as tm_table_forward (no stage events), except
 * that it never takes a plan whose workgroups wait for each other (batches
 * of at most 64 tokens run the decode plan as three launches): its results
 * do not depend on the device being otherwise idle, and there is no error
 * word to read.  The workspace is a static device array of
 * TM_NOALLOC_SCRATCH_BYTES inside the library (one per GPU, held until the
 * process ends; looked up, and its
 * arrival counters cleared by a kernel on `stream`, on the first call on
 * each device).  A layer whose tm_table_forward_workspace_size exceeds
 * TM_NOALLOC_SCRATCH_BYTES is rejected with TM_EWORKSPACE.  Allocates
 * nothing.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race.
 * ====================================================================== */
#define TM_NOALLOC_SCRATCH_BYTES (16u << 20)
int tm_table_forward_noalloc(const tm_table_layer *table, const tm_layer_io *io, tm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TABLEMOE_H */
