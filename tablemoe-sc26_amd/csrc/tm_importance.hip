// Importance scoring for the expert-level keep rule: the attention
// probabilities of the last query over every key, averaged over heads.
//
// Replaces HybridQwen3Attention._compute_and_cache_importance
// (models/qwen3_vl_moe/hybrid_attention.py:111-146: scores = (last_q K^T) in
// the model dtype, times `scaling` in the model dtype, softmax in fp32, mean
// over heads) and the DeepSeek variant _cache_last_token_attention
// (models/deepseek_vl2/deepseek_attention.py:206-249: fp32 scores, padded
// keys excluded, the last query_length keys kept).  Its output feeds
// tm_expert_keep_mask (the reference's build_prefill_keep_mask).
//
// Two launches.  scores_kernel: one workgroup per (512-key chunk, head,
// batch row); 8 lanes per key (each lane a D / 8 slice, fp32 products summed
// in lane order, then an 8-lane DPP tree), the chunk's scores to the
// workspace and its softmax statistics (max m_c, l_c = sum exp(s - m_c)).
// Chunk c of head h gets block id c + n_chunks * h, and the heads that share a
// KV head are consecutive, so with 8 chunks the KV chunk they read lands on one
// XCD.  mean_kernel: one thread per output key; per head, M = max_c m_c and
// L = sum_c l_c exp(m_c - M), p = exp(s - M) / L, then the heads' p summed in
// head order and divided by the head count.
#include "tm_internal.h"
#include "tm_route_dev.h"

namespace {

constexpr int kChunk = 512;    // keys per workgroup of scores_kernel
constexpr int kThreads = 256;  // 32 keys per pass (8 lanes each)
constexpr int kMaxHeads = 256;
constexpr int kMaxChunks = 1024;

template <int DT, int CH>
__global__ __launch_bounds__(kThreads) void scores_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t qs_b, int64_t qs_h, const typename Elem<DT>::T *__restrict__ k,
    int64_t ks_b, int64_t ks_s, int64_t ks_h, int n_heads, int groups, int64_t n_keys, float scale, int score_mode,
    const uint8_t *__restrict__ key_mask, int64_t km_b, float *__restrict__ sc, float2 *__restrict__ stats) {
  using T = typename Elem<DT>::T;
  // head dim 64 * CH: lane `sub` of a key's 8 lanes holds chunks sub, sub + 8, ... (8 elements each)
  const int c = (int)blockIdx.x, h = (int)blockIdx.y;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x, sub = tid & 7, grp = tid >> 3;
  const int kvh = h / groups;
  float qv[CH][8];
#pragma unroll
  for (int j = 0; j < CH; ++j) tm_load8<DT>(q + b * qs_b + (int64_t)h * qs_h + (j * 8 + sub) * 8, qv[j]);

  __shared__ float red_m[kThreads / 64], red_l[kThreads / 64];
  float m = -__builtin_huge_valf();
  float sv[kChunk / 32];
  bool ok[kChunk / 32];
  const int64_t t0 = (int64_t)c * kChunk;
#pragma unroll
  for (int it = 0; it < kChunk / 32; ++it) {
    const int64_t t = t0 + it * 32 + grp;
    const int64_t tc = t < n_keys ? t : n_keys - 1;
    const T *kr = k + b * ks_b + tc * ks_s + (int64_t)kvh * ks_h;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      float kv[8];
      tm_load8<DT>(kr + (j * 8 + sub) * 8, kv);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fmaf(qv[j][i], kv[i], acc);
    }
    acc += tm_g8f<kG8Steps[0]>(acc);
    acc += tm_g8f<kG8Steps[1]>(acc);
    acc += tm_g8f<kG8Steps[2]>(acc);
    const float s = score_mode == TM_SCORE_MODEL ? tm_round<DT>(tm_round<DT>(acc) * scale) : acc * scale;
    const bool valid = t < n_keys && (key_mask == nullptr || key_mask[b * km_b + tc] != 0);
    sv[it] = s;
    ok[it] = valid;
    m = valid ? fmaxf(m, s) : m;
    if (sub == 0 && t < n_keys) sc[(b * n_heads + h) * n_keys + t] = s;
  }
  // chunk max, then the sum of exp(s - max) over the valid keys
  m = tm_wave_max(m);
  if ((tid & 63) == 0) red_m[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  float l = 0.f;
  if (sub == 0) {
#pragma unroll
    for (int it = 0; it < kChunk / 32; ++it) l += ok[it] ? expf(sv[it] - m) : 0.f;
  }
  l = tm_wave_sum(l);
  if ((tid & 63) == 0) red_l[tid >> 6] = l;
  __syncthreads();
  if (tid == 0) {
    const float lt = ((red_l[0] + red_l[1]) + red_l[2]) + red_l[3];
    stats[(b * n_heads + h) * gridDim.x + c] = make_float2(m, lt);
  }
}

__global__ __launch_bounds__(kThreads) void mean_kernel(const float *__restrict__ sc, const float2 *__restrict__ stats,
                                                       int n_heads, int n_chunks, int64_t n_keys,
                                                       const uint8_t *__restrict__ key_mask, int64_t km_b,
                                                       int64_t out_len, float *__restrict__ out, int64_t ld_out) {
  __shared__ float hm[kMaxHeads], hl[kMaxHeads];
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  for (int h = tid; h < n_heads; h += kThreads) {  // combine the chunk statistics of head h
    const float2 *st = stats + (b * n_heads + h) * n_chunks;
    float M = -__builtin_huge_valf();
    for (int cc = 0; cc < n_chunks; ++cc) M = fmaxf(M, st[cc].x);
    float L = 0.f;
    if (M != -__builtin_huge_valf())
      for (int cc = 0; cc < n_chunks; ++cc) L += st[cc].y * expf(st[cc].x - M);
    hm[h] = M;
    hl[h] = L;
  }
  __syncthreads();
  const int64_t j = (int64_t)blockIdx.x * kThreads + tid;
  if (j >= out_len) return;
  const int64_t t = n_keys - out_len + j;
  const bool valid = key_mask == nullptr || key_mask[b * km_b + t] != 0;
  float acc = 0.f;
  for (int h = 0; h < n_heads; ++h) {
    const float s = sc[(b * n_heads + h) * n_keys + t];
    acc += (valid && hl[h] > 0.f) ? expf(s - hm[h]) / hl[h] : 0.f;
  }
  out[b * ld_out + j] = acc / (float)n_heads;
}

template <int DT, int CH>
void launch_scores(const void *q, int64_t qs_b, int64_t qs_h, const void *k, int64_t ks_b, int64_t ks_s, int64_t ks_h,
                   int64_t batch, int n_heads, int groups, int64_t n_keys, float scale, int score_mode,
                   const uint8_t *key_mask, int64_t km_b, float *sc, float2 *stats, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const dim3 grid((unsigned)tm_cdiv(n_keys, kChunk), (unsigned)n_heads, (unsigned)batch);
  hipLaunchKernelGGL((scores_kernel<DT, CH>), grid, dim3(kThreads), 0, s, static_cast<const T *>(q), qs_b, qs_h,
                     static_cast<const T *>(k), ks_b, ks_s, ks_h, n_heads, groups, n_keys, scale, score_mode,
                     key_mask, km_b, sc, stats);
}

}  // namespace

extern "C" size_t tm_importance_workspace_size(int64_t batch, int32_t n_heads, int64_t n_keys) {
  if (batch <= 0 || n_heads <= 0 || n_keys <= 0) return 0;
  const size_t scores = (size_t)batch * n_heads * n_keys * sizeof(float);
  const size_t stats = (size_t)batch * n_heads * tm_cdiv(n_keys, kChunk) * sizeof(float2);
  return (scores + 255) / 256 * 256 + stats;
}

extern "C" int tm_last_query_importance(int32_t dtype, const void *q, int64_t qs_b, int64_t qs_h, const void *k,
                                        int64_t ks_b, int64_t ks_s, int64_t ks_h, int64_t batch, int32_t n_heads,
                                        int32_t n_kv_heads, int32_t head_dim, int64_t n_keys, float scale,
                                        int32_t score_mode, const uint8_t *key_mask, int64_t km_b, int64_t out_len,
                                        float *out, int64_t ld_out, void *workspace, size_t workspace_bytes,
                                        tm_stream_t stream) {
  TM_REQUIRE(batch >= 0 && n_heads >= 1 && n_heads <= kMaxHeads && n_kv_heads >= 1 && n_heads % n_kv_heads == 0 &&
                 n_keys >= 0 && tm_cdiv(n_keys, kChunk) <= kMaxChunks && out_len >= 0 && out_len <= n_keys &&
                 ld_out >= out_len && batch < 65536,
             TM_EINVAL_SHAPE, "tm_last_query_importance: bad sizes (heads <= %d, keys <= %d)", kMaxHeads,
             kMaxChunks * kChunk);
  TM_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 192 || head_dim == 256, TM_EINVAL_SHAPE,
             "tm_last_query_importance: head_dim %d not in {64, 128, 192, 256}", head_dim);
  TM_REQUIRE(score_mode == TM_SCORE_MODEL || score_mode == TM_SCORE_F32, TM_EINVAL_ARG,
             "tm_last_query_importance: bad score mode");
  if (batch == 0 || n_keys == 0 || out_len == 0) return TM_OK;
  TM_REQUIRE(q && k && out, TM_EINVAL_ARG, "tm_last_query_importance: null pointer");
  const size_t need = tm_importance_workspace_size(batch, n_heads, n_keys);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need && tm_aligned16(workspace), TM_EWORKSPACE,
             "tm_last_query_importance: workspace %zu bytes < %zu", workspace_bytes, need);
  hipStream_t s = tm_hip_stream(stream);
  float *sc = static_cast<float *>(workspace);
  const size_t sc_bytes = ((size_t)batch * n_heads * n_keys * sizeof(float) + 255) / 256 * 256;
  float2 *stats = reinterpret_cast<float2 *>(static_cast<char *>(workspace) + sc_bytes);
  const int groups = n_heads / n_kv_heads;
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    const int E = Elem<DT>::kBytes;
    TM_REQUIRE(tm_aligned16(q) && tm_aligned16(k) && (qs_b * E) % 16 == 0 && (qs_h * E) % 16 == 0 &&
                   (ks_b * E) % 16 == 0 && (ks_s * E) % 16 == 0 && (ks_h * E) % 16 == 0,
               TM_EINVAL_SHAPE, "tm_last_query_importance: q/k rows must be 16-byte aligned");
    if constexpr (DT == TM_DT_F32) {
      TM_REQUIRE(score_mode == TM_SCORE_F32, TM_EINVAL_ARG, "tm_last_query_importance: fp32 inputs score in fp32");
    }
    switch (head_dim) {
      case 64: launch_scores<DT, 1>(q, qs_b, qs_h, k, ks_b, ks_s, ks_h, batch, n_heads, groups, n_keys, scale, score_mode, key_mask, km_b, sc, stats, s); break;
      case 128: launch_scores<DT, 2>(q, qs_b, qs_h, k, ks_b, ks_s, ks_h, batch, n_heads, groups, n_keys, scale, score_mode, key_mask, km_b, sc, stats, s); break;
      case 192: launch_scores<DT, 3>(q, qs_b, qs_h, k, ks_b, ks_s, ks_h, batch, n_heads, groups, n_keys, scale, score_mode, key_mask, km_b, sc, stats, s); break;
      default: launch_scores<DT, 4>(q, qs_b, qs_h, k, ks_b, ks_s, ks_h, batch, n_heads, groups, n_keys, scale, score_mode, key_mask, km_b, sc, stats, s); break;
    }
    TM_LAUNCH_CHECK("tm_last_query_importance(scores)");
    hipLaunchKernelGGL(mean_kernel, dim3((unsigned)tm_cdiv(out_len, kThreads), (unsigned)batch), dim3(kThreads), 0,
                       s, sc, stats, (int)n_heads, (int)tm_cdiv(n_keys, kChunk), n_keys, key_mask, km_b, out_len, out,
                       ld_out);
    TM_LAUNCH_CHECK("tm_last_query_importance(mean)");
    return TM_OK;
  });
}
