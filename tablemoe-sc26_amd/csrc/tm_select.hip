// Selection kernels: keep-rate radix select (north-star kernel (3)), the
// reference's keep masks (table_moe/skip/pruning.py) and surviving-weight
// renormalisation.
#include "tm_internal.h"
#include "tm_keep_dev.h"

namespace {

// ---------------------------------------------------------------------------
// block-wide exclusive scan of one uint32 per thread (blockDim.x % 64 == 0)
// ---------------------------------------------------------------------------
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *wave_tot, uint32_t &total) {
  constexpr int NW = NT / 64;
  static_assert(NW % 4 == 0, "wave totals are read four at a time");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t inc = tm_wave_incl_scan(v);
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  // every thread adds up the totals of the waves before its own (no second
  // barrier; the callers do not write wave_tot again before their next barrier)
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NW; w += 4) {
    const uint4 t = *reinterpret_cast<const uint4 *>(&wave_tot[w]);
    const uint32_t tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      all += tv[e];
      before += (w + e < wave) ? tv[e] : 0u;
    }
  }
  total = all;
  return before + inc - v;
}

// ---------------------------------------------------------------------------
// (3) keep the n_keep largest scores; ties -> lower token index.
// One workgroup; thread t owns the contiguous token range [t*per, (t+1)*per)
// and caches its order-preserving uint32 keys in registers (n <= 16384).
// Four 8-bit radix passes find the boundary key T and how many copies of T
// are kept: each pass builds a 256-bin histogram of the keys still matching
// the known high bits (one private histogram per wave, so nearby distances
// sharing their high digits only contend within a wave), the wave histograms
// are summed bin-parallel, and wave 0 locates the bin holding the n_keep-th largest key
// with a reverse prefix sum (4 bins per lane).  A block scan over the tokens
// in index order keeps the first of the tied ones.
// ---------------------------------------------------------------------------
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelRegs = 16;

__global__ __launch_bounds__(kSelThreads) void keep_select_kernel(const float *__restrict__ score,
                                                                  int64_t n, int64_t ld,
                                                                  int64_t n_keep,
                                                                  uint8_t *__restrict__ out) {
  __shared__ uint32_t whist[kSelWaves][256];  // per-wave private histograms
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_mask;
  __shared__ int64_t s_remaining;
  __shared__ __align__(16) uint32_t wave_tot[kSelWaves + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t per = (n + kSelThreads - 1) / kSelThreads;
  const int64_t lo = tid * per;
  const int64_t hi = (lo + per < n) ? lo + per : n;
  const int cnt = (int)(hi > lo ? hi - lo : 0);

  if (n_keep <= 0 || n_keep >= n) {
    const uint8_t v = n_keep > 0 ? 1 : 0;
    for (int64_t i = lo; i < hi; ++i) out[i] = v;
    return;
  }
  const bool cached = per <= kSelRegs;  // uniform
  uint32_t keys[kSelRegs];
  if (cached) {
#pragma unroll
    for (int j = 0; j < kSelRegs; ++j) keys[j] = (j < cnt) ? tm_orderable(score[(lo + j) * ld]) : 0u;
  }
  auto key_at = [&](int j) -> uint32_t {
    if (cached) {
      uint32_t k = 0;
#pragma unroll
      for (int u = 0; u < kSelRegs; ++u)
        if (u == j) k = keys[u];
      return k;
    }
    return tm_orderable(score[(lo + j) * ld]);
  };

  if (tid == 0) { s_prefix = 0; s_mask = 0; s_remaining = n_keep; }
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = lane; b < 256; b += 64) whist[wave][b] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    if (cached) {
#pragma unroll
      for (int j = 0; j < kSelRegs; ++j)
        if (j < cnt && (keys[j] & mask) == prefix) atomicAdd(&whist[wave][(keys[j] >> shift) & 255u], 1u);
    } else {
      for (int j = 0; j < cnt; ++j) {
        const uint32_t k = key_at(j);
        if ((k & mask) == prefix) atomicAdd(&whist[wave][(k >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (tid < 256) {  // thread t sums bin t over the waves
      uint32_t acc = 0;
#pragma unroll
      for (int w = 0; w < kSelWaves; ++w) acc += whist[w][tid];
      hist[tid] = acc;
    }
    __syncthreads();
    if (wave == 0) {
      uint32_t hb[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) hb[b] = hist[4 * lane + b];
      const uint32_t t = hb[0] + hb[1] + hb[2] + hb[3];
      uint32_t incl = t;  // sum over lanes >= this lane (bins >= 4*lane)
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_down(incl, o, 64);
        if (lane + o < 64) incl += v;
      }
      const int64_t rem = s_remaining;
      int64_t above = (int64_t)(incl - t);
#pragma unroll
      for (int b = 3; b >= 0; --b) {
        if (above < rem && rem <= above + (int64_t)hb[b]) {
          s_prefix = prefix | ((uint32_t)(4 * lane + b) << shift);
          s_mask = mask | (255u << shift);
          s_remaining = rem - above;
        }
        above += hb[b];
      }
    }
    __syncthreads();
  }
  const uint32_t T = s_prefix;
  const int64_t keep_eq = s_remaining;  // copies of T to keep, >= 1
  uint32_t eq = 0;
  for (int j = 0; j < cnt; ++j) eq += (key_at(j) == T);
  uint32_t total;
  uint32_t rank = block_exclusive_scan<kSelThreads>(eq, wave_tot, total);
  for (int j = 0; j < cnt; ++j) {
    const uint32_t key = key_at(j);
    uint8_t k = 0;
    if (key > T) {
      k = 1;
    } else if (key == T) {
      k = ((int64_t)rank < keep_eq) ? 1 : 0;
      ++rank;
    }
    out[lo + j] = k;
  }
}

// ---------------------------------------------------------------------------
// (3), fast form for n <= kSelThreads * kKeepRegs: same result as
// keep_select_kernel (tm_keep_select_fast in one 1024-thread workgroup).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kSelThreads) void keep_select_fast_kernel(const float *__restrict__ score, int64_t n,
                                                                       int64_t ld, int64_t n_keep,
                                                                       uint8_t *__restrict__ out, KeySrc ks) {
  __shared__ KeepSmem<kSelThreads> sm;
  tm_keep_select_fast<kSelThreads>(score, n, ld, n_keep, out, ks, sm);
}

// ---------------------------------------------------------------------------
// a3: build_fixed_keep_mask (pruning.py:4-15)
// ---------------------------------------------------------------------------
__global__ void fixed_keep_kernel(int64_t total, int top_k, int keep_k, uint8_t *out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < total) out[i] = ((int)(i % top_k) < keep_k) ? 1 : 0;
}

// ---------------------------------------------------------------------------
// a3: build_prefill_keep_mask (pruning.py:18-48), deterministic.
// Pass 1: per chunk of kEntries (token, slot) entries, each expert's partial
// score sum (entries in order) and selection count.  Pass 2 (one
// workgroup): each expert's chunk sums in a fixed order, ranking, mask.
// Every loop issues its loads ahead of their use: a loop that loads and
// uses one value per iteration waits a memory (or LDS) round trip each time.
// ---------------------------------------------------------------------------
constexpr int kEntries = 256;  // (token, slot) entries per chunk

__global__ __launch_bounds__(256) void expert_partial_kernel(
    const int64_t *__restrict__ sel, const float *__restrict__ w, const float *__restrict__ attn,
    int64_t n, int top_k, int n_experts, int64_t tok_per_chunk, float *__restrict__ part_sum,
    uint32_t *__restrict__ part_cnt) {
  __shared__ int4 s_sel[kEntries / 4];
  __shared__ float4 s_val[kEntries / 4];
  const int64_t t0 = (int64_t)blockIdx.x * tok_per_chunk;
  const int64_t t1 = (t0 + tok_per_chunk < n) ? t0 + tok_per_chunk : n;
  const int ne = (int)((t1 - t0) * top_k);
  const float nf = (float)n;
  int *ss = reinterpret_cast<int *>(s_sel);
  float *sv = reinterpret_cast<float *>(s_val);
  for (int j = threadIdx.x; j < kEntries; j += blockDim.x) {
    int ev = -1;
    float v = 0.f;
    if (j < ne) {
      const int64_t b = t0 + j / top_k;
      const int64_t e = sel[t0 * top_k + j];
      ev = (e >= 0 && e < n_experts) ? (int)e : -1;
      const float wv = w[t0 * top_k + j];
      v = attn ? attn[b] * wv : wv / nf;
    }
    ss[j] = ev;  // entries past the chunk match no expert
    sv[j] = v;
  }
  __syncthreads();
  const int nq = (ne + 3) / 4;
  for (int e = threadIdx.x; e < n_experts; e += blockDim.x) {
    float acc = 0.f;
    uint32_t cnt = 0;
#pragma unroll 8
    for (int q = 0; q < nq; ++q) {  // broadcast reads, entries in order
      const int4 s4 = s_sel[q];
      const float4 v4 = s_val[q];
      acc = s4.x == e ? acc + v4.x : acc;
      acc = s4.y == e ? acc + v4.y : acc;
      acc = s4.z == e ? acc + v4.z : acc;
      acc = s4.w == e ? acc + v4.w : acc;
      cnt += (uint32_t)(s4.x == e) + (uint32_t)(s4.y == e) + (uint32_t)(s4.z == e) + (uint32_t)(s4.w == e);
    }
    part_sum[(int64_t)blockIdx.x * n_experts + e] = acc;
    part_cnt[(int64_t)blockIdx.x * n_experts + e] = cnt;
  }
}

constexpr int kRankThreads = 1024;
constexpr int kMaxExperts = 1024;
constexpr int kRankPass = 128;                         // experts per pass
constexpr int kRankShares = kRankThreads / kRankPass;  // threads per expert (8)
constexpr int kRankBatch = 16;                         // loads issued before any is used

__global__ __launch_bounds__(kRankThreads) void expert_rank_kernel(
    const int64_t *__restrict__ sel, int64_t n, int top_k, int n_experts, int64_t nchunk,
    const float *__restrict__ part_sum, const uint32_t *__restrict__ part_cnt, double keep_rate,
    uint8_t *__restrict__ out_mask, float *__restrict__ out_scores) {
  __shared__ float score[kMaxExperts];
  __shared__ uint8_t active[kMaxExperts];
  __shared__ uint8_t kept[kMaxExperts];
  __shared__ float sh_sum[kRankShares][kRankPass];
  __shared__ uint32_t sh_cnt[kRankShares][kRankPass];
  __shared__ __align__(16) uint32_t wave_tot[kRankThreads / 64 + 1];
  const int tid = threadIdx.x;
  const int sub = tid / kRankPass;  // share of the chunks / experts this thread takes
  const int el = tid % kRankPass;   // expert within the pass: a wave reads consecutive experts
  // Expert e's score: share sub adds chunks sub, sub + 8, ... in increasing
  // order; the 8 shares are then added in share order.
  for (int e0 = 0; e0 < n_experts; e0 += kRankPass) {
    const int e = e0 + el;
    const int ee = e < n_experts ? e : n_experts - 1;
    float s = 0.f;
    uint32_t c = 0;
    for (int64_t k0 = sub; k0 < nchunk; k0 += (int64_t)kRankShares * kRankBatch) {
      float v[kRankBatch];
      uint32_t cc[kRankBatch];
#pragma unroll
      for (int u = 0; u < kRankBatch; ++u) {
        const int64_t k = k0 + (int64_t)u * kRankShares;
        const int64_t kk = k < nchunk ? k : nchunk - 1;
        v[u] = part_sum[kk * n_experts + ee];
        cc[u] = part_cnt[kk * n_experts + ee];
      }
#pragma unroll
      for (int u = 0; u < kRankBatch; ++u) {
        const bool in = k0 + (int64_t)u * kRankShares < nchunk;
        s = in ? s + v[u] : s;
        c += in ? cc[u] : 0u;
      }
    }
    sh_sum[sub][el] = s;
    sh_cnt[sub][el] = c;
    __syncthreads();
    if (sub == 0 && e < n_experts) {
      float t = 0.f;
      uint32_t tc = 0;
#pragma unroll
      for (int q = 0; q < kRankShares; ++q) {
        t += sh_sum[q][el];
        tc += sh_cnt[q][el];
      }
      score[e] = t;
      active[e] = tc > 0;
      if (out_scores) out_scores[e] = t;
    }
    __syncthreads();
  }
  uint32_t my_active = 0;
  for (int e = tid; e < n_experts; e += kRankThreads) my_active += active[e];
  uint32_t n_active;
  (void)block_exclusive_scan<kRankThreads>(my_active, wave_tot, n_active);
  int64_t num_keep = (int64_t)((double)n_active * keep_rate);
  if (num_keep < 1) num_keep = 1;
  if (num_keep > (int64_t)n_active) num_keep = n_active;
  // Rank of each active expert among the active ones (higher score first,
  // ties to the lower id): share sub counts the experts o = sub, sub + 8, ...
  // ahead of e, branch-free, reading 8 of them before using any.
  for (int e0 = 0; e0 < n_experts; e0 += kRankPass) {
    const int e = e0 + el;
    const int ee = e < n_experts ? e : n_experts - 1;
    const float se = score[ee];
    uint32_t r = 0;
    for (int o0 = sub; o0 < n_experts; o0 += kRankShares * 8) {
      float so[8];
      uint32_t ao[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int o = o0 + u * kRankShares;
        const int oo = o < n_experts ? o : 0;
        so[u] = score[oo];
        ao[u] = (o < n_experts) ? active[oo] : 0u;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int o = o0 + u * kRankShares;
        r += (ao[u] != 0u && (so[u] > se || (so[u] == se && o < e))) ? 1u : 0u;
      }
    }
    sh_cnt[sub][el] = r;
    __syncthreads();
    if (sub == 0 && e < n_experts) {
      uint32_t rank = 0;
#pragma unroll
      for (int q = 0; q < kRankShares; ++q) rank += sh_cnt[q][el];
      kept[e] = (active[e] && (int64_t)rank < num_keep) ? 1 : 0;
    }
    __syncthreads();
  }
  const int64_t total = n * top_k;
  constexpr int kMaskBatch = 16;  // ids loaded before any is used
  for (int64_t i0 = tid; i0 < total; i0 += (int64_t)kRankThreads * kMaskBatch) {
    int64_t ev[kMaskBatch];
#pragma unroll
    for (int u = 0; u < kMaskBatch; ++u) {
      const int64_t i = i0 + (int64_t)u * kRankThreads;
      ev[u] = sel[i < total ? i : total - 1];
    }
#pragma unroll
    for (int u = 0; u < kMaskBatch; ++u) {
      const int64_t i = i0 + (int64_t)u * kRankThreads;
      if (i < total) out_mask[i] = (ev[u] >= 0 && ev[u] < n_experts) ? kept[ev[u]] : 0;
    }
  }
}

// ---------------------------------------------------------------------------
// a11: renormalize_surviving_weights (pruning.py:55-73), one thread per row.
// ---------------------------------------------------------------------------
template <int DT>
__global__ void renormalize_kernel(const typename Elem<DT>::T *__restrict__ w, int64_t ld_w,
                                   const uint8_t *__restrict__ mask, int64_t ld_m, int64_t n,
                                   int top_k, int target_mode, const typename Elem<DT>::T *__restrict__ target,
                                   int64_t ld_t, typename Elem<DT>::T *__restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n) return;
  const typename Elem<DT>::T *wr = w + b * ld_w;
  const uint8_t *mr = mask + b * ld_m;
  float kept = 0.f, full = 0.f;
  for (int s = 0; s < top_k; ++s) {
    const float v = Elem<DT>::to_f(wr[s]);
    full += v;
    if (mr[s]) kept += v;
  }
  kept = tm_round<DT>(kept);
  float tgt = 1.f;
  if (target_mode == TM_TARGET_ORIG_SUM) tgt = tm_round<DT>(full);
  else if (target_mode == TM_TARGET_GIVEN) tgt = Elem<DT>::to_f(target[b * ld_t]);
  typename Elem<DT>::T *o = out + b * top_k;
  const bool valid = kept > 0.f;
  for (int s = 0; s < top_k; ++s) {
    float r = 0.f;
    if (valid && mr[s]) {
      r = tm_round<DT>(Elem<DT>::to_f(wr[s]) / kept);
      if (target_mode != TM_TARGET_ONE) r = tm_round<DT>(r * tgt);
    }
    o[s] = Elem<DT>::from_f(r);
  }
}

}  // namespace

// ===========================================================================
extern "C" int64_t tm_keep_count(int64_t n, double keep_rate) {
  if (n <= 0) return 0;
  int64_t k = (int64_t)((double)n * keep_rate);
  if (k < 1) k = 1;
  if (k > n) k = n;
  return k;
}

extern "C" size_t tm_keep_select_workspace_size(int64_t n) {
  (void)n;
  return 0;
}

extern "C" int tm_keep_select(const float *score, int64_t n, int64_t ld_score, int64_t n_keep,
                              uint8_t *out_keep, void *workspace, size_t workspace_bytes,
                              tm_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  TM_REQUIRE(n >= 0 && n < ((int64_t)1 << 31) && ld_score >= 1, TM_EINVAL_SHAPE,
             "tm_keep_select: bad sizes n=%lld", (long long)n);
  if (n == 0) return TM_OK;
  TM_REQUIRE(score && out_keep, TM_EINVAL_ARG, "tm_keep_select: null pointer");
  if (n <= (int64_t)kSelThreads * kKeepRegs)
    hipLaunchKernelGGL(keep_select_fast_kernel, dim3(1), dim3(kSelThreads), 0, tm_hip_stream(stream),
                       score, n, ld_score, n_keep, out_keep, KeySrc{});
  else
    hipLaunchKernelGGL(keep_select_kernel, dim3(1), dim3(kSelThreads), 0, tm_hip_stream(stream),
                       score, n, ld_score, n_keep, out_keep);
  TM_LAUNCH_CHECK("tm_keep_select");
  return TM_OK;
}

extern "C" int tm_fixed_keep_mask(int64_t n_tokens, int32_t top_k, int32_t keep_k, uint8_t *out,
                                  tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && top_k >= 0, TM_EINVAL_SHAPE, "tm_fixed_keep_mask: bad sizes");
  const int64_t total = n_tokens * top_k;
  if (total == 0) return TM_OK;
  TM_REQUIRE(out, TM_EINVAL_ARG, "tm_fixed_keep_mask: null pointer");
  hipLaunchKernelGGL(fixed_keep_kernel, dim3((unsigned)tm_cdiv(total, 256)), dim3(256), 0,
                     tm_hip_stream(stream), total, top_k, keep_k, out);
  TM_LAUNCH_CHECK("tm_fixed_keep_mask");
  return TM_OK;
}

static int64_t expert_tok_per_chunk(int32_t top_k) {
  int64_t t = kEntries / (top_k > 0 ? top_k : 1);
  return t < 1 ? 1 : t;
}

extern "C" size_t tm_expert_keep_mask_workspace_size(int64_t n_tokens, int32_t n_experts) {
  // sized for the largest chunk count (top_k = 32)
  if (n_tokens <= 0 || n_experts <= 0) return 0;
  const int64_t nchunk = tm_cdiv(n_tokens, expert_tok_per_chunk(32));
  return (size_t)nchunk * (size_t)n_experts * (sizeof(float) + sizeof(uint32_t));
}

extern "C" int tm_expert_keep_mask(const int64_t *sel, const float *weights, const float *attn,
                                   int64_t n_tokens, int32_t top_k, int32_t n_experts,
                                   double keep_rate, uint8_t *out_mask, float *out_expert_scores,
                                   void *workspace, size_t workspace_bytes, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && top_k >= 1 && top_k <= 32 && n_experts >= 1 && n_experts <= kMaxExperts,
             TM_EINVAL_SHAPE, "tm_expert_keep_mask: bad sizes (top_k %d, experts %d)", top_k, n_experts);
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(sel && weights && out_mask, TM_EINVAL_ARG, "tm_expert_keep_mask: null pointer");
  const int64_t tpc = expert_tok_per_chunk(top_k);
  const int64_t nchunk = tm_cdiv(n_tokens, tpc);
  const size_t need = (size_t)nchunk * (size_t)n_experts * (sizeof(float) + sizeof(uint32_t));
  TM_REQUIRE(workspace && workspace_bytes >= need, TM_EWORKSPACE,
             "tm_expert_keep_mask: workspace %zu bytes < %zu", workspace_bytes, need);
  float *part_sum = static_cast<float *>(workspace);
  uint32_t *part_cnt = reinterpret_cast<uint32_t *>(part_sum + nchunk * n_experts);
  hipStream_t s = tm_hip_stream(stream);
  hipLaunchKernelGGL(expert_partial_kernel, dim3((unsigned)nchunk), dim3(256), 0, s, sel, weights,
                     attn, n_tokens, top_k, n_experts, tpc, part_sum, part_cnt);
  TM_LAUNCH_CHECK("tm_expert_keep_mask(partial)");
  hipLaunchKernelGGL(expert_rank_kernel, dim3(1), dim3(kRankThreads), 0, s, sel, n_tokens, top_k,
                     n_experts, nchunk, part_sum, part_cnt, keep_rate, out_mask, out_expert_scores);
  TM_LAUNCH_CHECK("tm_expert_keep_mask(rank)");
  return TM_OK;
}

extern "C" int tm_renormalize(int32_t dtype, const void *weights, int64_t ld_w, const uint8_t *mask,
                              int64_t ld_m, int64_t n_tokens, int32_t top_k, int32_t target_mode,
                              const void *target, int64_t ld_t, void *out, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && top_k >= 0 && ld_w >= top_k && ld_m >= top_k, TM_EINVAL_SHAPE,
             "tm_renormalize: bad sizes");
  TM_REQUIRE(target_mode >= TM_TARGET_ONE && target_mode <= TM_TARGET_GIVEN, TM_EINVAL_ARG,
             "tm_renormalize: bad target mode %d", target_mode);
  if (n_tokens == 0 || top_k == 0) return TM_OK;
  TM_REQUIRE(weights && mask && out && (target_mode != TM_TARGET_GIVEN || target), TM_EINVAL_ARG,
             "tm_renormalize: null pointer");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    hipLaunchKernelGGL((renormalize_kernel<DT>), dim3((unsigned)tm_cdiv(n_tokens, 256)), dim3(256), 0,
                       tm_hip_stream(stream), static_cast<const T *>(weights), ld_w, mask, ld_m,
                       n_tokens, top_k, target_mode, static_cast<const T *>(target), ld_t,
                       static_cast<T *>(out));
    TM_LAUNCH_CHECK("tm_renormalize");
    return TM_OK;
  });
}

bool tm_internal_keep_keys_ok(int64_t n) { return n > 0 && n <= (int64_t)kSelThreads * kKeepRegs; }

int tm_internal_keep_keys(const uint64_t *keys, const float *qn_part, int32_t parts, int32_t metric, int64_t n,
                          int64_t n_keep, float *out_dist, int64_t *out_idx, float *out_qn, uint8_t *out_keep,
                          hipStream_t stream) {
  TM_REQUIRE(tm_internal_keep_keys_ok(n) && parts >= 1 && parts <= 4, TM_EINVAL_SHAPE,
             "tm_table_forward: keep select from keys: bad sizes");
  TM_REQUIRE(keys && qn_part && out_dist && out_idx && out_qn && out_keep && tm_aligned16(keys) &&
                 tm_aligned16(qn_part),
             TM_EINVAL_ARG, "tm_table_forward: keep select from keys: bad buffers");
  const KeySrc ks{keys, qn_part, parts, metric == TM_METRIC_L2 ? 1 : 0, out_dist, out_idx, out_qn};
  hipLaunchKernelGGL(keep_select_fast_kernel, dim3(1), dim3(kSelThreads), 0, stream, nullptr, n, (int64_t)1,
                     n_keep, out_keep, ks);
  TM_LAUNCH_CHECK("tm_table_forward(keep)");
  return TM_OK;
}
