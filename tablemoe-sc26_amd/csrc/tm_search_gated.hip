// Reference-semantics ("mode R") searches over the per-(expert, modality)
// tables keys[E, 2, K, d]:
//   - tm_search_gated: the prefill/decode offline search (cosine or raw dot,
//     threshold gate) from already projected queries
//     (table_moe/cache_engine/search.py:515-602, :661-697; Triton :35-256);
//   - tm_search_hybrid: the decode online-window + offline search with the
//     projection fused (search.py:839-954, :987-1105, :778-806; Triton :258-385).
//
// Scores are fp32 sums in a fixed order; the arg-max keeps the first index
// among equal maxima, as torch.max / tl.max(return_indices) do.
#include "tm_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxDim = 256;

// Best (max score, first index) of the wave over the n_cent rows of one table.
// qv: the query in LDS as fp32.  Lane l takes centroids l, l+64, ...
template <int DT, bool VEC>
__device__ __forceinline__ void wave_table_argmax(const typename Elem<DT>::T *table, int64_t ks_c,
                                                  int64_t n_cent, int dim, const float *qv,
                                                  float &best, int &best_i) {
  const int lane = threadIdx.x & 63;
  best = -__builtin_huge_valf();
  best_i = 0x7fffffff;
  for (int64_t c = lane; c < n_cent; c += 64) {
    const typename Elem<DT>::T *row = table + c * ks_c;
    float acc = 0.f;
    if constexpr (VEC) {
      for (int j = 0; j < dim; j += 8) {
        float v[8];
        tm_load8<DT>(row + j, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(qv[j + i], v[i], acc);
      }
    } else {
      for (int j = 0; j < dim; ++j) acc = fmaf(qv[j], Elem<DT>::to_f(row[j]), acc);
    }
    if (acc > best) { best = acc; best_i = (int)c; }
  }
  tm_wave_argmax(best, best_i);
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void gated_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t n, int64_t ld_q,
    const typename Elem<DT>::T *__restrict__ keys, int64_t n_exp, int64_t n_cent, int dim, int64_t ks_e,
    int64_t ks_m, int64_t ks_c, const int64_t *__restrict__ sel, int top_k, int64_t ss_b, int64_t ss_s,
    const uint8_t *__restrict__ is_vision, const uint8_t *__restrict__ reuse, int64_t rs_b, int64_t rs_s,
    int col_offset, float thr_v, float thr_t, int cmp, uint8_t *__restrict__ out_hit,
    int64_t *__restrict__ out_idx, int64_t os_b, int64_t os_s) {
  __shared__ float qsh[kThreads / 64][kMaxDim];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t pair = (int64_t)blockIdx.x * (kThreads / 64) + wave;
  const int64_t b = pair / top_k;
  const int s = (int)(pair % top_k);
  if (b >= n) return;  // whole wave
  const int64_t e = sel[b * ss_b + s * ss_s];
  const bool searched = s >= col_offset && (reuse == nullptr || reuse[b * rs_b + s * rs_s]) &&
                        e >= 0 && e < n_exp;
  const int64_t o = b * os_b + s * os_s;
  if (!searched) {
    if (lane == 0) { out_hit[o] = 0; out_idx[o] = 0; }
    return;
  }
  const bool vis = is_vision == nullptr || is_vision[b];
  for (int j = lane; j < dim; j += 64) qsh[wave][j] = Elem<DT>::to_f(q[b * ld_q + j]);
  // qsh is private to this wave: a wave-level barrier suffices.
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  float best;
  int best_i;
  wave_table_argmax<DT, VEC>(keys + e * ks_e + (vis ? 0 : 1) * ks_m, ks_c, n_cent, dim, qsh[wave], best,
                             best_i);
  const float thr = vis ? thr_v : thr_t;
  const bool hit = (cmp == TM_CMP_GE) ? (best >= thr) : (best > thr);
  if (lane == 0) {
    out_hit[o] = hit ? 1 : 0;
    out_idx[o] = hit ? (int64_t)best_i : 0;
  }
}

// Decode hybrid search: one workgroup per token.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void hybrid_kernel(
    const typename Elem<DT>::T *__restrict__ x, int hidden, int64_t ld_x, const uint8_t *__restrict__ is_vision,
    const typename Elem<DT>::T *__restrict__ pv, const typename Elem<DT>::T *__restrict__ bv,
    const typename Elem<DT>::T *__restrict__ pt, const typename Elem<DT>::T *__restrict__ bt, int64_t ps_h,
    int64_t ps_d, int dim, const typename Elem<DT>::T *__restrict__ on_keys, int64_t ld_on, int n_valid,
    const int64_t *__restrict__ on_ids, int on_topk, int64_t ld_on_ids,
    const typename Elem<DT>::T *__restrict__ keys, int64_t n_exp, int64_t n_cent, int64_t ks_e, int64_t ks_m,
    int64_t ks_c, const int64_t *__restrict__ sel, int top_k, int64_t ss_b, int64_t ss_s, int keep_k,
    uint8_t *__restrict__ on_hit, int64_t *__restrict__ on_idx, uint8_t *__restrict__ off_hit,
    int64_t *__restrict__ off_idx, int64_t *__restrict__ on_slot, int64_t os_b, int64_t os_s,
    typename Elem<DT>::T *__restrict__ q_ws) {
  using T = typename Elem<DT>::T;
  extern __shared__ float xsh[];        // hidden floats
  __shared__ float on_sc[1024];         // online scores
  __shared__ float part[kThreads];      // projection partials
  __shared__ float qsh[kMaxDim];
  __shared__ int s_jstar, s_valid_on;
  __shared__ uint8_t s_onhit[64];
  __shared__ int s_onslot[64];
  __shared__ int s_need_offline;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x;
  const bool vis = is_vision == nullptr || is_vision[b];
  const T *xr = x + b * ld_x;
  for (int h = tid; h < hidden; h += kThreads) xsh[h] = Elem<DT>::to_f(xr[h]);
  if (tid == 0) s_need_offline = 0;
  __syncthreads();

  // 1) online window scores x . online_keys[j]
  for (int j = wave; j < n_valid; j += kThreads / 64) {
    const T *kr = on_keys + (int64_t)j * ld_on;
    float acc = 0.f;
    for (int h = lane; h < hidden; h += 64) acc = fmaf(xsh[h], Elem<DT>::to_f(kr[h]), acc);
    acc = tm_wave_sum(acc);
    if (lane == 0) on_sc[j] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    float mx = -__builtin_huge_valf();
    int js = -1;
    for (int j = 0; j < n_valid; ++j)
      if (on_sc[j] > mx) { mx = on_sc[j]; js = j; }
    const int valid_on = (n_valid > 0 && mx > 0.f) ? 1 : 0;
    s_jstar = js;
    s_valid_on = valid_on;
    on_idx[b] = valid_on ? js : -1;
  }
  __syncthreads();
  // 2) online hits of the searched slots
  if (tid < top_k) {
    const int s = tid;
    uint8_t hit = 0;
    int slot = 0;
    if (s >= keep_k && s_valid_on) {
      const int64_t e = sel[b * ss_b + s * ss_s];
      const int64_t *ids = on_ids + (int64_t)s_jstar * ld_on_ids;
      for (int t = 0; t < on_topk; ++t) {
        if (ids[t] == e) { hit = 1; slot = t; break; }
      }
    }
    s_onhit[s] = hit;
    s_onslot[s] = slot;
    if (s >= keep_k && !hit) atomicOr(&s_need_offline, 1);
  }
  __syncthreads();
  // 3) raw projection q = dtype(x @ P_m + bias_m) (only if an offline search remains)
  if (s_need_offline) {
    const T *P = vis ? pv : pt;
    const T *bias = vis ? bv : bt;
    const int nparts = kThreads / dim;
    const int col = tid % dim, p = tid / dim;
    float acc = 0.f;
    if (p < nparts) {
      const int h0 = (int)(((int64_t)hidden * p) / nparts), h1 = (int)(((int64_t)hidden * (p + 1)) / nparts);
      for (int h = h0; h < h1; ++h) acc = fmaf(xsh[h], Elem<DT>::to_f(P[(int64_t)h * ps_h + (int64_t)col * ps_d]), acc);
    }
    part[tid] = acc;
    __syncthreads();
    if (tid < dim) {
      float sum = 0.f;
      for (int pp = 0; pp < nparts; ++pp) sum += part[pp * dim + tid];
      const float v = tm_round<DT>(sum + Elem<DT>::to_f(bias[tid]));
      qsh[tid] = v;
      q_ws[b * dim + tid] = Elem<DT>::from_f(v);
    }
    __syncthreads();
    // 4) offline search of the remaining slots, one wave per slot
    for (int s = keep_k + wave; s < top_k; s += kThreads / 64) {
      if (s_onhit[s]) continue;
      const int64_t e = sel[b * ss_b + s * ss_s];
      uint8_t hit = 0;
      int64_t idx = 0;
      if (e >= 0 && e < n_exp) {
        float best;
        int best_i;
        wave_table_argmax<DT, VEC>(keys + e * ks_e + (vis ? 0 : 1) * ks_m, ks_c, n_cent, dim, qsh, best,
                                   best_i);
        hit = best >= 0.f;
        idx = hit ? best_i : 0;
      }
      if (lane == 0) {
        off_hit[b * os_b + s * os_s] = hit;
        off_idx[b * os_b + s * os_s] = idx;
      }
    }
  }
  // 5) the remaining outputs
  if (tid < top_k) {
    const int s = tid;
    const int64_t o = b * os_b + s * os_s;
    on_hit[o] = s_onhit[s];
    on_slot[o] = s_onhit[s] ? s_onslot[s] : 0;
    if (s < keep_k || s_onhit[s] || !s_need_offline) {
      off_hit[o] = 0;
      off_idx[o] = 0;
    }
  }
}

}  // namespace

extern "C" int tm_search_gated(int32_t dtype, const void *q_low, int64_t n_tokens, int64_t ld_q,
                               const void *keys, int64_t n_experts, int64_t n_centroids, int32_t dim,
                               int64_t ks_e, int64_t ks_m, int64_t ks_c, const int64_t *sel, int32_t top_k,
                               int64_t ss_b, int64_t ss_s, const uint8_t *is_vision, const uint8_t *reuse,
                               int64_t rs_b, int64_t rs_s, int32_t col_offset, float thr_vision,
                               float thr_text, int32_t cmp, uint8_t *out_hit, int64_t *out_idx,
                               int64_t os_b, int64_t os_s, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && top_k >= 0 && dim >= 1 && dim <= kMaxDim && n_centroids >= 1 &&
                 n_centroids <= 65536 && n_experts >= 1 && ld_q >= dim,
             TM_EINVAL_SHAPE, "tm_search_gated: bad sizes (dim %d, K %lld)", dim, (long long)n_centroids);
  TM_REQUIRE(cmp == TM_CMP_GE || cmp == TM_CMP_GT, TM_EINVAL_ARG, "tm_search_gated: bad comparator");
  const int64_t pairs = n_tokens * top_k;
  if (pairs == 0) return TM_OK;
  TM_REQUIRE(q_low && keys && sel && out_hit && out_idx, TM_EINVAL_ARG, "tm_search_gated: null pointer");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const bool vec = dim % 8 == 0 && tm_aligned16(keys) && (ks_e * E) % 16 == 0 && (ks_m * E) % 16 == 0 &&
                     (ks_c * E) % 16 == 0;
    dim3 grid((unsigned)tm_cdiv(pairs, kThreads / 64)), block(kThreads);
    auto launch = [&](auto vec_tag) {
      constexpr bool VEC = decltype(vec_tag)::value;
      hipLaunchKernelGGL((gated_kernel<DT, VEC>), grid, block, 0, tm_hip_stream(stream),
                         static_cast<const T *>(q_low), n_tokens, ld_q, static_cast<const T *>(keys),
                         n_experts, n_centroids, dim, ks_e, ks_m, ks_c, sel, top_k, ss_b, ss_s, is_vision,
                         reuse, rs_b, rs_s, col_offset, thr_vision, thr_text, cmp, out_hit, out_idx, os_b,
                         os_s);
    };
    if (vec) launch(std::true_type{});
    else launch(std::false_type{});
    TM_LAUNCH_CHECK("tm_search_gated");
    return TM_OK;
  });
}

extern "C" int tm_search_hybrid(int32_t dtype, const void *x, int64_t n_tokens, int32_t hidden, int64_t ld_x,
                                const uint8_t *is_vision, const void *proj_vis, const void *bias_vis,
                                const void *proj_txt, const void *bias_txt, int64_t ps_h, int64_t ps_d,
                                int32_t dim, const void *online_keys, int64_t ld_online, int32_t n_online_valid,
                                const int64_t *online_ids, int32_t online_topk, int64_t ld_online_ids,
                                const void *keys, int64_t n_experts, int64_t n_centroids, int64_t ks_e,
                                int64_t ks_m, int64_t ks_c, const int64_t *sel, int32_t top_k, int64_t ss_b,
                                int64_t ss_s, int32_t keep_k, uint8_t *on_hit, int64_t *on_idx,
                                uint8_t *off_hit, int64_t *off_idx, int64_t *on_slot, int64_t os_b,
                                int64_t os_s, void *workspace, size_t workspace_bytes, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && hidden >= 1 && hidden <= 16384 && ld_x >= hidden && dim >= 1 && dim <= kMaxDim &&
                 n_centroids >= 1 && n_centroids <= 65536 && n_experts >= 1 && top_k >= 0 && top_k <= 64,
             TM_EINVAL_SHAPE, "tm_search_hybrid: bad sizes");
  TM_REQUIRE(n_online_valid >= 0 && n_online_valid <= 1024 && online_topk >= 0 && online_topk <= 64,
             TM_EINVAL_SHAPE, "tm_search_hybrid: online window too large");
  TM_REQUIRE(ps_h == 1 || ps_d == 1, TM_EINVAL_SHAPE, "tm_search_hybrid: projection needs a unit stride");
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(x && proj_vis && bias_vis && keys && sel && on_hit && on_idx && off_hit && off_idx && on_slot,
             TM_EINVAL_ARG, "tm_search_hybrid: null pointer");
  TM_REQUIRE((proj_txt == nullptr) == (bias_txt == nullptr), TM_EINVAL_ARG,
             "tm_search_hybrid: proj_txt and bias_txt must both be set or both be NULL");
  TM_REQUIRE(n_online_valid == 0 || (online_keys && online_ids), TM_EINVAL_ARG,
             "tm_search_hybrid: online window pointers missing");
  TM_REQUIRE(n_tokens < (int64_t)0x7fffffff, TM_EINVAL_SHAPE, "tm_search_hybrid: too many tokens");
  if (keep_k < 0) keep_k = 0;
  if (keep_k > top_k) keep_k = top_k;
  // nothing searched: outputs are only cleared (on_idx = -1), no window lookup
  if (keep_k == top_k) n_online_valid = 0;
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const size_t need = (size_t)n_tokens * dim * E;
    TM_REQUIRE(workspace && workspace_bytes >= need, TM_EWORKSPACE,
               "tm_search_hybrid: workspace %zu bytes < %zu", workspace_bytes, need);
    const bool vec = dim % 8 == 0 && tm_aligned16(keys) && (ks_e * E) % 16 == 0 && (ks_m * E) % 16 == 0 &&
                     (ks_c * E) % 16 == 0;
    const T *pt = static_cast<const T *>(proj_txt ? proj_txt : proj_vis);
    const T *bt = static_cast<const T *>(proj_txt ? bias_txt : bias_vis);
    const size_t shmem = (size_t)hidden * sizeof(float);
    auto launch = [&](auto vec_tag) {
      constexpr bool VEC = decltype(vec_tag)::value;
      hipLaunchKernelGGL((hybrid_kernel<DT, VEC>), dim3((unsigned)n_tokens), dim3(kThreads), shmem,
                         tm_hip_stream(stream), static_cast<const T *>(x), hidden, ld_x, is_vision,
                         static_cast<const T *>(proj_vis), static_cast<const T *>(bias_vis), pt, bt, ps_h, ps_d,
                         dim, static_cast<const T *>(online_keys), ld_online, n_online_valid, online_ids,
                         online_topk, ld_online_ids, static_cast<const T *>(keys), n_experts, n_centroids,
                         ks_e, ks_m, ks_c, sel, top_k, ss_b, ss_s, keep_k, on_hit, on_idx, off_hit, off_idx,
                         on_slot, os_b, os_s, static_cast<T *>(workspace));
    };
    if (vec) launch(std::true_type{});
    else launch(std::false_type{});
    TM_LAUNCH_CHECK("tm_search_hybrid");
    return TM_OK;
  });
}
