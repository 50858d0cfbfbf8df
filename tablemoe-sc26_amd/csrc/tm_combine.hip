// Gather / combine kernels: cached-row gather (a10), the mode-G gather +
// combine + residual (north-star kernel (4)), the reference-semantics fused
// slot combine (a10+a11) and the online-window ring write (a12).
//
// All are HBM-bound row streams: one workgroup of 256 threads per output row,
// 16-byte vector loads/stores (8 bf16/fp16 or 2x4 fp32 per thread per step)
// when every row pointer is 16-byte aligned, element loops otherwise.
#include "tm_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxSrc = 64;

// y[h] = sum_j coef[j] * src_j[h] (+ residual), for one row, fp32 accumulate.
template <int DT, bool VEC>
__device__ __forceinline__ void combine_row(const typename Elem<DT>::T *const *src, const float *coef,
                                            int nsrc, const typename Elem<DT>::T *residual,
                                            typename Elem<DT>::T *dst, int hidden) {
  if constexpr (VEC) {
    for (int h0 = threadIdx.x * 8; h0 < hidden; h0 += kThreads * 8) {
      float acc[8];
      if (residual) {
        tm_load8<DT>(residual + h0, acc);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.f;
      }
      for (int j = 0; j < nsrc; ++j) {
        float v[8];
        tm_load8<DT>(src[j] + h0, v);
        const float c = coef[j];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(c, v[i], acc[i]);
      }
      tm_store8<DT>(dst + h0, acc);
    }
  } else {
    for (int h = threadIdx.x; h < hidden; h += kThreads) {
      float acc = residual ? Elem<DT>::to_f(residual[h]) : 0.f;
      for (int j = 0; j < nsrc; ++j) acc = fmaf(coef[j], Elem<DT>::to_f(src[j][h]), acc);
      dst[h] = Elem<DT>::from_f(acc);
    }
  }
}

// ---------------------------------------------------------------------------
// a10: out[dst(i)] = values[e, m, c]
// ---------------------------------------------------------------------------
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(
    const typename Elem<DT>::T *__restrict__ values, int64_t n_exp, int64_t n_cent, int hidden,
    int64_t vs_e, int64_t vs_m, int64_t vs_c, const int64_t *__restrict__ eids,
    const int64_t *__restrict__ mids, int modality, const int64_t *__restrict__ cids,
    const int64_t *__restrict__ dst_rows, typename Elem<DT>::T *__restrict__ out, int64_t n_out,
    int64_t ld_out) {
  using T = typename Elem<DT>::T;
  const int64_t i = blockIdx.x;
  const int64_t e = eids[i], c = cids[i];
  const int64_t m = mids ? mids[i] : modality;
  const int64_t d = dst_rows ? dst_rows[i] : i;
  if (d < 0 || d >= n_out) return;  // whole workgroup
  T *dst = out + d * ld_out;
  const bool ok = e >= 0 && e < n_exp && m >= 0 && m < 2 && c >= 0 && c < n_cent;
  const T *src = values + e * vs_e + m * vs_m + c * vs_c;
  const float one = 1.f;
  combine_row<DT, VEC>(&src, &one, ok ? 1 : 0, nullptr, dst, hidden);
}

// ---------------------------------------------------------------------------
// (4) mode G: out[b] = residual[b] + (keep ? sum_s w~ E[b,s] : sum_j beta V[idx])
//
// One workgroup per token row.  The row's sources and coefficients depend on
// the row only, so every wave derives them itself from wave-uniform loads (no
// LDS hand-off, no barrier).  Fast path: at most 8 sources; all 16-byte loads
// of a chunk are issued before the FMAs so they are in flight together.
// ---------------------------------------------------------------------------
constexpr int kFastSrc = 8;
constexpr int kRankTokens = 1;  // tokens per workgroup of the ranked combine
constexpr int kRowsPerGroup = 1;  // rows per workgroup of the fast kernel (more in flight per CU with 1)

// Sources and coefficients of one row (wave-uniform).
template <int DT>
struct RowPlan {
  const typename Elem<DT>::T *src[kFastSrc];
  float coef[kFastSrc];
  bool use[kFastSrc];
};

template <int DT>
__device__ __forceinline__ void plan_row(RowPlan<DT> &p, int64_t b, const uint8_t *keep,
                                         const typename Elem<DT>::T *slot_out, int64_t so_b, int64_t so_s,
                                         const float *w, int64_t ld_w, int top_k,
                                         const typename Elem<DT>::T *values, int64_t n_cent, int64_t ld_v,
                                         const int64_t *idx, const float *dist, int64_t ld_idx, int nn) {
  // every metadata load of the row is issued before any is used
  float wv[kFastSrc], dv[kFastSrc];
  int64_t cv[kFastSrc];
  const bool kept = keep[b] != 0;
#pragma unroll
  for (int j = 0; j < kFastSrc; ++j) {
    wv[j] = (j < top_k) ? w[b * ld_w + j] : 0.f;
    cv[j] = (j < nn) ? idx[b * ld_idx + j] : -1;
    dv[j] = (j < nn && nn > 1) ? dist[b * ld_idx + j] : 0.f;
  }
  if (kept) {
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < kFastSrc; ++s) sum += wv[s];
#pragma unroll
    for (int s = 0; s < kFastSrc; ++s) {
      p.use[s] = s < top_k && sum > 0.f;
      p.coef[s] = p.use[s] ? wv[s] / sum : 0.f;
      p.src[s] = slot_out + b * so_b + (int64_t)s * so_s;
    }
  } else {
    float inv_sum = 0.f;
#pragma unroll
    for (int j = 0; j < kFastSrc; ++j) {
      p.use[j] = cv[j] >= 0 && cv[j] < n_cent;
      p.src[j] = values + (p.use[j] ? cv[j] : 0) * ld_v;
      p.coef[j] = (p.use[j] && nn > 1) ? 1.f / (dv[j] + 1e-6f) : (p.use[j] ? 1.f : 0.f);
      inv_sum += p.coef[j];
    }
    if (nn > 1) {
#pragma unroll
      for (int j = 0; j < kFastSrc; ++j) p.coef[j] = p.use[j] ? p.coef[j] / inv_sum : 0.f;
    }
  }
}

// One workgroup streams kRowsPerGroup rows; the next row's plan (metadata
// loads) is formed before the current row's data is combined, and all 16-byte
// loads of a chunk are issued before the FMAs.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void gather_combine_fast_kernel(
    int64_t n, int hidden, const uint8_t *__restrict__ keep, const typename Elem<DT>::T *__restrict__ slot_out,
    int64_t so_b, int64_t so_s, const float *__restrict__ w, int64_t ld_w, int top_k,
    const typename Elem<DT>::T *__restrict__ values, int64_t n_cent, int64_t ld_v,
    const int64_t *__restrict__ idx, const float *__restrict__ dist, int64_t ld_idx, int nn,
    const typename Elem<DT>::T *__restrict__ residual, int64_t ld_r,
    typename Elem<DT>::T *__restrict__ out, int64_t ld_o) {
  using T = typename Elem<DT>::T;
  const int64_t b0 = (int64_t)blockIdx.x * kRowsPerGroup;
  const int64_t b1 = (b0 + kRowsPerGroup < n) ? b0 + kRowsPerGroup : n;
  RowPlan<DT> cur, nxt;
  plan_row<DT>(cur, b0, keep, slot_out, so_b, so_s, w, ld_w, top_k, values, n_cent, ld_v, idx, dist, ld_idx, nn);
  for (int64_t b = b0; b < b1; ++b) {
    if (b + 1 < b1)
      plan_row<DT>(nxt, b + 1, keep, slot_out, so_b, so_s, w, ld_w, top_k, values, n_cent, ld_v, idx, dist,
                   ld_idx, nn);
    const T *res_row = residual ? residual + b * ld_r : nullptr;
    T *dst = out + b * ld_o;
    if constexpr (VEC) {
      for (int h0 = threadIdx.x * 8; h0 < hidden; h0 += kThreads * 8) {
        float v[kFastSrc][8];
#pragma unroll
        for (int j = 0; j < kFastSrc; ++j)
          if (cur.use[j]) tm_load8<DT>(cur.src[j] + h0, v[j]);
        float acc[8];
        if (res_row) {
          tm_load8<DT>(res_row + h0, acc);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = 0.f;
        }
#pragma unroll
        for (int j = 0; j < kFastSrc; ++j)
          if (cur.use[j]) {
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = fmaf(cur.coef[j], v[j][i], acc[i]);
          }
        tm_store8<DT>(dst + h0, acc);
      }
    } else {
      for (int h = threadIdx.x; h < hidden; h += kThreads) {
        float acc = res_row ? Elem<DT>::to_f(res_row[h]) : 0.f;
#pragma unroll
        for (int j = 0; j < kFastSrc; ++j)
          if (cur.use[j]) acc = fmaf(cur.coef[j], Elem<DT>::to_f(cur.src[j][h]), acc);
        dst[h] = Elem<DT>::from_f(acc);
      }
    }
    cur = nxt;
  }
}

// Shape-specialised path (top_k = TK recomputed slots, NN nearest centroids,
// 2-byte types, 16-byte aligned rows): the keep flag selects one of two
// wave-uniform branches, and inside each every source load is unconditional,
// so all of a chunk's loads are in flight together (a load behind a per-source
// branch makes the compiler wait for everything outstanding at the join).
// Slot outputs and the output are streamed once: non-temporal accesses;
// gathered value rows (centroids repeat) and the residual use ordinary loads
// (a non-temporal residual made the ranked combine ~0.7 us slower).
// Same arithmetic as gather_combine_fast_kernel: fp32 accumulation starting
// from the residual, sources added in order with fmaf, one rounding.
// Keep decisions when the keep set is ranked in the combine: token b is
// kept when fewer than n_keep tokens are ahead of it (a larger distance, or
// the same at a lower index), the set the radix select gives.  One pass over
// the n distances (contiguous, 16-byte aligned) serves the TPB tokens of the
// workgroup (token b0 + g for g < TPB; TPB * 256 threads).
struct RankKeep {
  int64_t n;
  int64_t n_keep;
  uint8_t *keep_out;
};

// The distances, kRankVec 16-byte vectors per thread and pass, plus (first
// pass) one scalar per thread for the n % 4 last: every load uses a clamped
// index (no load is conditional, so none makes the wave wait where it is
// issued) and a pass's loads are in flight together; values past n are
// loaded but count as a key no token is behind.  With n < 4 the vectors come
// from a zero vector of their own.  n <= kRankOnePass: one pass, straight-
// line code (the layer's sizes).
constexpr int kRankVec = 4;
__device__ float4 g_rank_pad;

template <int TPB>
constexpr int64_t kRankOnePass = 4LL * kRankVec * TPB * kThreads;

struct RankPass {
  float4 v[kRankVec];
  float tail;
};

template <int TPB>
__device__ __forceinline__ RankPass rank_load(const float *__restrict__ dist, int64_t n, int64_t base) {
  constexpr int NT = TPB * kThreads;
  const int64_t n4 = n >> 2;
  const float4 *d4 = n4 > 0 ? reinterpret_cast<const float4 *>(dist) : &g_rank_pad;
  const int64_t last = n4 > 0 ? n4 - 1 : 0;
  RankPass r;
#pragma unroll
  for (int u = 0; u < kRankVec; ++u) {
    const int64_t i = base + threadIdx.x + (int64_t)u * NT;
    r.v[u] = d4[i < last ? i : last];
  }
  const int64_t j = 4 * n4 + threadIdx.x;
  r.tail = dist[j < n ? j : n - 1];
  return r;
}

// Keep decision of token b0 + g: dist_first is the first pass (rank_load at
// base 0), loaded by the caller before its other loads so that it retires
// first; ONE: n <= kRankOnePass<TPB>, no further pass.
template <int TPB, bool ONE>
__device__ __forceinline__ bool rank_keep(const float *__restrict__ dist, int64_t n, int64_t n_keep, int64_t b0,
                                          int g, const RankPass &dist_first) {
  constexpr int NT = TPB * kThreads;
  constexpr int NW = NT / 64;
  __shared__ uint32_t s_ahead[NW][TPB];
  uint32_t kb[TPB];
#pragma unroll
  for (int t = 0; t < TPB; ++t) kb[t] = tm_orderable(dist[b0 + t < n ? b0 + t : n - 1]);
  uint32_t ahead[TPB];
#pragma unroll
  for (int t = 0; t < TPB; ++t) ahead[t] = 0;
  // every key of a real distance is >= orderable(-inf) > 0: key 0 is ahead of
  // no token and ties with none
  auto count = [&](uint32_t k, int64_t j) {
#pragma unroll
    for (int t = 0; t < TPB; ++t)
      ahead[t] += (uint32_t)(k > kb[t]) | ((uint32_t)(k == kb[t]) & (uint32_t)(j < b0 + t));
  };
  const int64_t n4 = n >> 2;
  auto count_pass = [&](const RankPass &r, int64_t base) {
#pragma unroll
    for (int u = 0; u < kRankVec; ++u) {
      const int64_t i = base + threadIdx.x + (int64_t)u * NT;
      const bool in = i < n4;
      count(in ? tm_orderable(r.v[u].x) : 0u, 4 * i);
      count(in ? tm_orderable(r.v[u].y) : 0u, 4 * i + 1);
      count(in ? tm_orderable(r.v[u].z) : 0u, 4 * i + 2);
      count(in ? tm_orderable(r.v[u].w) : 0u, 4 * i + 3);
    }
  };
  count_pass(dist_first, 0);
  const int64_t jt = 4 * n4 + threadIdx.x;
  count(jt < n ? tm_orderable(dist_first.tail) : 0u, jt);
  if constexpr (!ONE) {
    for (int64_t base = (int64_t)kRankVec * NT; base < n4; base += (int64_t)kRankVec * NT)
      count_pass(rank_load<TPB>(dist, n, base), base);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int t = 0; t < TPB; ++t) {
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)tm_wave_incl_scan(ahead[t]), 63);
    if (lane == 0) s_ahead[wave][t] = a;
  }
  __syncthreads();
  uint32_t total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) total += s_ahead[w][g];
  return (int64_t)total < n_keep;
}

template <int DT, int TK, int NN>
__global__ __launch_bounds__(kThreads, 8) void gather_combine_tk_kernel(
    int hidden, const uint8_t *__restrict__ keep, const typename Elem<DT>::T *__restrict__ slot_out, int64_t so_b,
    int64_t so_s, const float *__restrict__ w, int64_t ld_w, const typename Elem<DT>::T *__restrict__ values,
    int64_t n_cent, int64_t ld_v, const int64_t *__restrict__ idx, const float *__restrict__ dist, int64_t ld_idx,
    const typename Elem<DT>::T *__restrict__ residual, int64_t ld_r, typename Elem<DT>::T *__restrict__ out,
    int64_t ld_o) {
  using T = typename Elem<DT>::T;
  const int64_t b = blockIdx.x;
  const T *res_row = residual ? residual + b * ld_r : nullptr;
  T *dst = out + b * ld_o;
  if (keep[b]) {  // uniform
    float coef[TK];
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s) {
      coef[s] = w[b * ld_w + s];
      sum += coef[s];
    }
    const bool any = sum > 0.f;  // rows whose weights sum to 0 contribute nothing
#pragma unroll
    for (int s = 0; s < TK; ++s) coef[s] = coef[s] / sum;
    const T *src = slot_out + b * so_b;
    for (int h0 = threadIdx.x * 8; h0 < hidden; h0 += kThreads * 8) {
      float acc[8];
      if (res_row) {
        tm_load8<DT>(res_row + h0, acc);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.f;
      }
      if (any) {
        tm_u32x4 raw[TK];  // 16-bit values until used: 4 registers per slot instead of 8
#pragma unroll
        for (int s = 0; s < TK; ++s)
          raw[s] = __builtin_nontemporal_load(reinterpret_cast<const tm_u32x4 *>(src + (int64_t)s * so_s + h0));
#pragma unroll
        for (int s = 0; s < TK; ++s) {
          const T *e = reinterpret_cast<const T *>(&raw[s]);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = fmaf(coef[s], Elem<DT>::to_f(e[i]), acc[i]);
        }
      }
      tm_store8_nt<DT>(dst + h0, acc);
    }
  } else {
    const T *src[NN];
    float coef[NN];
    bool ok[NN];
    float inv_sum = 0.f;
#pragma unroll
    for (int j = 0; j < NN; ++j) {
      const int64_t c = idx[b * ld_idx + j];
      ok[j] = c >= 0 && c < n_cent;
      src[j] = values + (ok[j] ? c : 0) * ld_v;
      coef[j] = ok[j] ? ((NN > 1) ? 1.f / (dist[b * ld_idx + j] + 1e-6f) : 1.f) : 0.f;
      inv_sum += coef[j];
    }
    if (NN > 1) {
#pragma unroll
      for (int j = 0; j < NN; ++j) coef[j] = ok[j] ? coef[j] / inv_sum : 0.f;
    }
    for (int h0 = threadIdx.x * 8; h0 < hidden; h0 += kThreads * 8) {
      float acc[8];
      if (res_row) {
        tm_load8<DT>(res_row + h0, acc);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.f;
      }
      float v[NN][8];
#pragma unroll
      for (int j = 0; j < NN; ++j) tm_load8<DT>(src[j] + h0, v[j]);
#pragma unroll
      for (int j = 0; j < NN; ++j) {
        if (ok[j]) {  // uniform; the loads above are already issued
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = fmaf(coef[j], v[j][i], acc[i]);
        }
      }
      tm_store8_nt<DT>(dst + h0, acc);
    }
  }
}

// 8 consecutive elements as loaded: 16-bit values stay packed (one 16-byte
// vector), fp32 takes two vectors; converted where they are used.
template <int DT>
struct Raw8 {
  tm_u32x4 w[Elem<DT>::kBytes / 2];
  __device__ __forceinline__ float at(int i) const {
    return Elem<DT>::to_f(reinterpret_cast<const typename Elem<DT>::T *>(&w[0])[i]);
  }
};

template <int DT, bool NT>
__device__ __forceinline__ Raw8<DT> raw_load8(const typename Elem<DT>::T *p) {
  Raw8<DT> r;
  const tm_u32x4 *v = reinterpret_cast<const tm_u32x4 *>(p);
#pragma unroll
  for (int k = 0; k < Elem<DT>::kBytes / 2; ++k) r.w[k] = NT ? __builtin_nontemporal_load(v + k) : v[k];
  return r;
}

// Top-1 combine that also decides the keep set (rank_keep), TPB tokens per
// workgroup (256 threads each, one 8-element chunk per thread: hidden <=
// 2048), so the distances are read once per TPB tokens.  The arithmetic is
// gather_combine_tk_kernel's (NN = 1).
//
// Two dependent memory round trips per workgroup: every load whose address
// is known at entry goes out first -- the first pass of distances, then the
// residual chunk, the token's router weights and its centroid id -- with
// clamped addresses, so no load is conditional and none makes the wave wait
// where it is issued (loads retire in order: the distances, issued first,
// are counted while the others are still in flight).  Once the ranking
// decided, the token's TK slot chunks (kept) or its value chunk (replaced)
// are loaded, all before the first is used; sources a token does not take
// are loaded and masked out by a select, not skipped by a branch.
template <int DT, int TK, int TPB, bool ONE>
__global__ __launch_bounds__(TPB * kThreads, 8) void gather_combine_rank_kernel(
    int hidden, const typename Elem<DT>::T *__restrict__ slot_out, int64_t so_b, int64_t so_s,
    const float *__restrict__ w, int64_t ld_w, const typename Elem<DT>::T *__restrict__ values, int64_t n_cent,
    int64_t ld_v, const int64_t *__restrict__ idx, const float *__restrict__ dist,
    const typename Elem<DT>::T *__restrict__ residual, int64_t ld_r, typename Elem<DT>::T *__restrict__ out,
    int64_t ld_o, RankKeep rk) {
  using T = typename Elem<DT>::T;
  // one token per workgroup: its index, row addresses, weights and centroid
  // are wave-uniform (scalar registers and loads)
  const int g = TPB == 1 ? 0 : threadIdx.x / kThreads;
  const int64_t b0 = (int64_t)blockIdx.x * TPB;
  const int64_t b = b0 + g;
  const int h0 = (threadIdx.x % kThreads) * 8;
  const bool act = h0 < hidden && b < rk.n;
  const int64_t bc = b < rk.n ? b : rk.n - 1;
  const int hc = h0 < hidden ? h0 : hidden - 8;
  const RankPass d0 = rank_load<TPB>(dist, rk.n, 0);
  __builtin_amdgcn_sched_barrier(0);  // the distances first: they are needed first
  // without a residual the output row stands in as a valid address (not used)
  const Raw8<DT> res = raw_load8<DT, false>(residual ? residual + bc * ld_r + hc : out + bc * ld_o + hc);
  float wt[TK];
#pragma unroll
  for (int s = 0; s < TK; ++s) wt[s] = w[bc * ld_w + s];
  const int64_t c = idx[bc];
  // every load above is issued before the counting starts (the compiler
  // barrier keeps the weights' and centroid's loads from sinking into the
  // branches that use them)
  asm volatile("" ::: "memory");
  const bool kept = rank_keep<TPB, ONE>(dist, rk.n, rk.n_keep, b0, g, d0);
  if (!act) return;
  if (h0 == 0) rk.keep_out[b] = kept ? 1 : 0;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = residual ? res.at(i) : 0.f;
  if (kept) {  // uniform over the token's 256 threads
    const T *src = slot_out + b * so_b + h0;
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s) sum += wt[s];
    const bool any = sum > 0.f;  // rows whose weights sum to 0 contribute nothing
    // 16-bit rows: all TK chunks in flight before the first is used; fp32
    // rows (8 registers a chunk) in two halves
    constexpr int GRP = sizeof(T) == 2 ? TK : TK / 2;
#pragma unroll
    for (int s0 = 0; s0 < TK; s0 += GRP) {
      Raw8<DT> sv[GRP];
#pragma unroll
      for (int s = 0; s < GRP; ++s) sv[s] = raw_load8<DT, true>(src + (int64_t)(s0 + s) * so_s);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < GRP; ++s) {
        const float coef = wt[s0 + s] / sum;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = any ? fmaf(coef, sv[s].at(i), acc[i]) : acc[i];
      }
    }
  } else {
    const bool ok = c >= 0 && c < n_cent;
    const Raw8<DT> val = raw_load8<DT, false>(values + (ok ? c : 0) * ld_v + h0);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = ok ? fmaf(1.f, val.at(i), acc[i]) : acc[i];
  }
  tm_store8_nt<DT>(out + b * ld_o + h0, acc);
}

// gather_combine_tk_kernel with one 8-element chunk per thread (hidden <=
// 8 * kTk1MaxThreads, a block of round64(hidden / 8) threads), in two
// dependent memory round trips: the keep byte first, then every other load
// whose address is known at entry (the residual chunk with a clamped
// address, the router weights, centroid ids and distances as scalar loads),
// and once the keep byte is in, all of the branch's source chunks before the
// first is used (sources a row does not take are loaded and masked out by a
// select).  The loop kernel walks a chunk at a time, each behind a residual
// load the compiler waits for where it is issued.  Same arithmetic.
constexpr int kTk1MaxThreads = 1024;

template <int DT, int TK, int NN>
__global__ __launch_bounds__(kTk1MaxThreads, 8) void gather_combine_tk1_kernel(
    int hidden, const uint8_t *__restrict__ keep, const typename Elem<DT>::T *__restrict__ slot_out, int64_t so_b,
    int64_t so_s, const float *__restrict__ w, int64_t ld_w, const typename Elem<DT>::T *__restrict__ values,
    int64_t n_cent, int64_t ld_v, const int64_t *__restrict__ idx, const float *__restrict__ dist, int64_t ld_idx,
    const typename Elem<DT>::T *__restrict__ residual, int64_t ld_r, typename Elem<DT>::T *__restrict__ out,
    int64_t ld_o) {
  using T = typename Elem<DT>::T;
  const int64_t b = blockIdx.x;
  const int h0 = threadIdx.x * 8;
  const bool act = h0 < hidden;
  const int hc = act ? h0 : hidden - 8;
  const uint8_t kp = keep[b];
  __builtin_amdgcn_sched_barrier(0);  // the keep byte first: it is needed first
  // without a residual the output row stands in as a valid address (not used)
  Raw8<DT> res = raw_load8<DT, false>(residual ? residual + b * ld_r + hc : out + b * ld_o + hc);
  float wt[TK];
#pragma unroll
  for (int s = 0; s < TK; ++s) wt[s] = w[b * ld_w + s];
  int64_t c[NN];
  float dj[NN];
#pragma unroll
  for (int j = 0; j < NN; ++j) {
    c[j] = idx[b * ld_idx + j];
    dj[j] = NN > 1 ? dist[b * ld_idx + j] : 0.f;
  }
  // The weights, ids and distances (scalar loads) are taken here, where the
  // branch waits for the keep byte anyway: left to itself the compiler moves
  // them into the branch, in front of its source loads.
#pragma unroll
  for (int s = 0; s < TK; ++s) asm volatile("" : "+s"(wt[s]));
#pragma unroll
  for (int j = 0; j < NN; ++j) asm volatile("" : "+s"(c[j]), "+s"(dj[j]));
  float acc[8];
  // The residual is converted only after the branch's source loads are
  // issued (the empty asm keeps the conversion, common to both branches,
  // from being hoisted above the branch).
  auto take_res = [&] {
#pragma unroll
    for (int k = 0; k < Elem<DT>::kBytes / 2; ++k) asm volatile("" : "+v"(res.w[k]));
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = residual ? res.at(i) : 0.f;
  };
  if (kp) {  // uniform
    const T *src = slot_out + b * so_b + hc;
    Raw8<DT> sv[TK];
#pragma unroll
    for (int s = 0; s < TK; ++s) sv[s] = raw_load8<DT, true>(src + (int64_t)s * so_s);
    __builtin_amdgcn_sched_barrier(0);  // all TK chunks in flight before the residual or any of them is used
    take_res();
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s) sum += wt[s];
    const bool any = sum > 0.f;  // rows whose weights sum to 0 contribute nothing
#pragma unroll
    for (int s = 0; s < TK; ++s) {
      const float coef = wt[s] / sum;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = any ? fmaf(coef, sv[s].at(i), acc[i]) : acc[i];
    }
  } else {
    bool ok[NN];
    Raw8<DT> v[NN];
#pragma unroll
    for (int j = 0; j < NN; ++j) {
      ok[j] = c[j] >= 0 && c[j] < n_cent;
      v[j] = raw_load8<DT, false>(values + (ok[j] ? c[j] : 0) * ld_v + hc);
    }
    __builtin_amdgcn_sched_barrier(0);
    take_res();
    float coef[NN];
    float inv_sum = 0.f;
#pragma unroll
    for (int j = 0; j < NN; ++j) {
      coef[j] = ok[j] ? ((NN > 1) ? 1.f / (dj[j] + 1e-6f) : 1.f) : 0.f;
      inv_sum += coef[j];
    }
    if (NN > 1) {
#pragma unroll
      for (int j = 0; j < NN; ++j) coef[j] = ok[j] ? coef[j] / inv_sum : 0.f;
    }
#pragma unroll
    for (int j = 0; j < NN; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = ok[j] ? fmaf(coef[j], v[j].at(i), acc[i]) : acc[i];
  }
  if (act) tm_store8_nt<DT>(out + b * ld_o + h0, acc);
}

// General path (more than 8 sources): sources staged through LDS.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void gather_combine_kernel(
    int hidden, const uint8_t *__restrict__ keep, const typename Elem<DT>::T *__restrict__ slot_out,
    int64_t so_b, int64_t so_s, const float *__restrict__ w, int64_t ld_w, int top_k,
    const typename Elem<DT>::T *__restrict__ values, int64_t n_cent, int64_t ld_v,
    const int64_t *__restrict__ idx, const float *__restrict__ dist, int64_t ld_idx, int nn,
    const typename Elem<DT>::T *__restrict__ residual, int64_t ld_r,
    typename Elem<DT>::T *__restrict__ out, int64_t ld_o) {
  using T = typename Elem<DT>::T;
  __shared__ const T *s_src[kMaxSrc];
  __shared__ float s_coef[kMaxSrc];
  __shared__ int s_nsrc;
  const int64_t b = blockIdx.x;
  if (threadIdx.x == 0) {
    int ns = 0;
    if (keep[b]) {
      float sum = 0.f;
      for (int s = 0; s < top_k; ++s) sum += w[b * ld_w + s];
      if (sum > 0.f) {
        for (int s = 0; s < top_k; ++s) {
          s_src[ns] = slot_out + b * so_b + s * so_s;
          s_coef[ns] = w[b * ld_w + s] / sum;
          ++ns;
        }
      }
    } else {
      float inv_sum = 0.f;
      for (int j = 0; j < nn; ++j) {
        const int64_t c = idx[b * ld_idx + j];
        if (c >= 0 && c < n_cent) inv_sum += (nn > 1) ? 1.f / (dist[b * ld_idx + j] + 1e-6f) : 1.f;
      }
      for (int j = 0; j < nn; ++j) {
        const int64_t c = idx[b * ld_idx + j];
        if (c >= 0 && c < n_cent) {
          s_src[ns] = values + c * ld_v;
          s_coef[ns] = (nn > 1) ? (1.f / (dist[b * ld_idx + j] + 1e-6f)) / inv_sum : 1.f;
          ++ns;
        }
      }
    }
    s_nsrc = ns;
  }
  __syncthreads();
  combine_row<DT, VEC>(s_src, s_coef, s_nsrc, residual ? residual + b * ld_r : nullptr, out + b * ld_o,
                       hidden);
}

// ---------------------------------------------------------------------------
// a10+a11 reference-semantics slot combine (cached_layers.py:439-465,
// deepseek_layers.py:695-729).
// ---------------------------------------------------------------------------
// combine_row for at most kSlotSrc sources (16-byte rows): every source load
// of a chunk is issued before the first is used (the sources past nsrc read
// the output row itself and are not added), so a token's rows stream in one
// round trip instead of one per source.
constexpr int kSlotSrc = 8;

template <int DT>
__device__ __forceinline__ void combine_row_few(const typename Elem<DT>::T *const *src, const float *coef, int nsrc,
                                                const typename Elem<DT>::T *residual, typename Elem<DT>::T *dst,
                                                int hidden) {
  using T = typename Elem<DT>::T;
  const T *p[kSlotSrc];
  float c[kSlotSrc];
#pragma unroll
  for (int j = 0; j < kSlotSrc; ++j) {
    p[j] = j < nsrc ? src[j] : dst;
    c[j] = j < nsrc ? coef[j] : 0.f;
  }
  for (int h0 = threadIdx.x * 8; h0 < hidden; h0 += kThreads * 8) {
    float acc[8];
    if (residual) {
      tm_load8<DT>(residual + h0, acc);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.f;
    }
    uint4 raw[kSlotSrc];
#pragma unroll
    for (int j = 0; j < kSlotSrc; ++j) raw[j] = *reinterpret_cast<const uint4 *>(p[j] + h0);
#pragma unroll
    for (int j = 0; j < kSlotSrc; ++j) {
      const T *e = reinterpret_cast<const T *>(&raw[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = j < nsrc ? fmaf(c[j], Elem<DT>::to_f(e[i]), acc[i]) : acc[i];
    }
    tm_store8<DT>(dst + h0, acc);
  }
}

// a10+a11: one workgroup per token.  Lane s < top_k loads slot s's flags,
// ids and weight (every load issued at once, whatever the flags say); the
// source of the slot is the table row (off_hit), else the online window row
// (on_hit), else the recomputed row (compute_mask), else none.  Thread 0
// then forms the renormalised coefficients in slot order from LDS.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void slot_combine_kernel(
    int top_k, int hidden, const float *__restrict__ w, int64_t ld_w,
    const uint8_t *__restrict__ compute_mask, const typename Elem<DT>::T *__restrict__ computed,
    int64_t cs_b, int64_t cs_s, const uint8_t *__restrict__ off_hit, const int64_t *__restrict__ off_idx,
    const int64_t *__restrict__ sel, int64_t ld_m, const uint8_t *__restrict__ is_vision,
    const typename Elem<DT>::T *__restrict__ values, int64_t n_exp, int64_t n_cent, int64_t vs_e,
    int64_t vs_m, int64_t vs_c, const uint8_t *__restrict__ on_hit, const int64_t *__restrict__ on_idx,
    const int64_t *__restrict__ on_slot, const typename Elem<DT>::T *__restrict__ online_values,
    int64_t n_online, int online_topk, int64_t ov_w, int64_t ov_s, int target_mode,
    const typename Elem<DT>::T *__restrict__ residual, int64_t ld_r, typename Elem<DT>::T *__restrict__ out,
    int64_t ld_o) {
  using T = typename Elem<DT>::T;
  __shared__ const T *s_src[kMaxSrc];
  __shared__ float s_coef[kMaxSrc];
  __shared__ const T *s_p[kMaxSrc];
  __shared__ float s_w[kMaxSrc];
  __shared__ int s_nsrc;
  const int64_t b = blockIdx.x;
  const int t = threadIdx.x;
  if (t < top_k) {
    const int64_t mi = b * ld_m + t;
    const uint8_t fh = off_hit ? off_hit[mi] : 0;
    const uint8_t oh = on_hit ? on_hit[mi] : 0;
    const uint8_t cm = compute_mask ? compute_mask[mi] : 0;
    const int64_t e = off_hit ? sel[mi] : -1;
    const int64_t c = off_hit ? off_idx[mi] : -1;
    const int64_t r = on_hit ? on_idx[b] : -1;
    const int64_t jo = on_hit ? on_slot[mi] : -1;
    const float ws = w[b * ld_w + t];
    const int m = (is_vision == nullptr || is_vision[b]) ? 0 : 1;
    const T *p = nullptr;
    if (fh) {
      if (e >= 0 && e < n_exp && c >= 0 && c < n_cent) p = values + e * vs_e + m * vs_m + c * vs_c;
    } else if (oh) {
      if (r >= 0 && r < n_online && jo >= 0 && jo < online_topk) p = online_values + r * ov_w + jo * ov_s;
    } else if (cm) {
      p = computed + b * cs_b + t * cs_s;
    }
    s_p[t] = p;
    s_w[t] = ws;
  }
  __syncthreads();
  if (t == 0) {
    float kept = 0.f, full = 0.f;
    for (int s = 0; s < top_k; ++s) {
      full += s_w[s];
      if (s_p[s]) kept += s_w[s];
    }
    int ns = 0;
    if (kept > 0.f) {
      for (int s = 0; s < top_k; ++s) {
        if (!s_p[s]) continue;
        float cf = s_w[s] / kept;
        if (target_mode == TM_TARGET_ORIG_SUM) cf = cf * full;
        else cf = tm_round<DT>(cf);
        s_src[ns] = s_p[s];
        s_coef[ns] = cf;
        ++ns;
      }
    }
    s_nsrc = ns;
  }
  __syncthreads();
  const T *res = residual ? residual + b * ld_r : nullptr;
  if constexpr (VEC) {
    if (top_k <= kSlotSrc) {  // uniform
      combine_row_few<DT>(s_src, s_coef, s_nsrc, res, out + b * ld_o, hidden);
      return;
    }
  }
  combine_row<DT, VEC>(s_src, s_coef, s_nsrc, res, out + b * ld_o, hidden);
}

// ---------------------------------------------------------------------------
// Decode step of one token (reference _forward_decode_bs1,
// cached_layers.py:161-269): the slot combine above plus the ring write of
// update_online_cache_bs1 (manager.py:89-106) in one launch.  Ring row r
// takes the token's hidden row, its expert ids (-1 for slots that did not
// survive) and each slot's source row (zeros when dropped).  Every thread
// loads all sources of its 8 columns before it writes them, so a source in
// ring row r itself (the window's oldest entry) is read before it is
// overwritten; other threads never touch those columns.
// ---------------------------------------------------------------------------
constexpr int kDecodeSlots = 8;

template <int DT>
__global__ __launch_bounds__(kThreads) void slot_combine_update_kernel(
    int top_k, int hidden, const float *__restrict__ w, const uint8_t *__restrict__ compute_mask,
    const typename Elem<DT>::T *__restrict__ computed, int64_t cs_s, const uint8_t *__restrict__ off_hit,
    const int64_t *__restrict__ off_idx, const int64_t *__restrict__ sel, const uint8_t *__restrict__ is_vision,
    const typename Elem<DT>::T *__restrict__ values, int64_t n_exp, int64_t n_cent, int64_t vs_e, int64_t vs_m,
    int64_t vs_c, const uint8_t *__restrict__ on_hit, const int64_t *__restrict__ on_idx,
    const int64_t *__restrict__ on_slot, typename Elem<DT>::T *online_values, int64_t n_online, int online_topk,
    int64_t ov_w, int64_t ov_s, int target_mode, const typename Elem<DT>::T *__restrict__ residual,
    typename Elem<DT>::T *__restrict__ out, const typename Elem<DT>::T *__restrict__ x,
    typename Elem<DT>::T *__restrict__ ring_keys, int64_t *__restrict__ ring_ids, int64_t r) {
  using T = typename Elem<DT>::T;
  __shared__ const T *s_src[kDecodeSlots];
  __shared__ float s_coef[kDecodeSlots];
  __shared__ float s_w[kDecodeSlots];
  const int t = threadIdx.x;
  if (t < top_k) {  // lane s: slot s's flags, ids and weight, every load issued at once
    const uint8_t fh = off_hit ? off_hit[t] : 0;
    const uint8_t oh = on_hit ? on_hit[t] : 0;
    const uint8_t cm = compute_mask ? compute_mask[t] : 0;
    const int64_t e = sel[t];
    const int64_t c = off_hit ? off_idx[t] : -1;
    const int64_t rr = on_hit ? on_idx[0] : -1;
    const int64_t j = on_hit ? on_slot[t] : -1;
    const float ws = w[t];
    const int m = (is_vision == nullptr || is_vision[0]) ? 0 : 1;
    const T *p = nullptr;
    if (fh) {
      if (e >= 0 && e < n_exp && c >= 0 && c < n_cent) p = values + e * vs_e + m * vs_m + c * vs_c;
    } else if (oh) {
      if (rr >= 0 && rr < n_online && j >= 0 && j < online_topk) p = online_values + rr * ov_w + j * ov_s;
    } else if (cm) {
      p = computed + t * cs_s;
    }
    s_src[t] = p;
    s_w[t] = ws;
    ring_ids[r * online_topk + t] = p ? e : -1;
  }
  __syncthreads();
  if (t == 0) {  // the coefficients as slot_combine_kernel forms them (sums in slot order)
    float kept = 0.f, full = 0.f;
    for (int s = 0; s < top_k; ++s) {
      full += s_w[s];
      if (s_src[s]) kept += s_w[s];
    }
    for (int s = 0; s < top_k; ++s) {
      float c = 0.f;
      if (s_src[s] && kept > 0.f) {
        c = s_w[s] / kept;
        c = (target_mode == TM_TARGET_ORIG_SUM) ? c * full : tm_round<DT>(c);
      }
      s_coef[s] = c;
    }
  }
  __syncthreads();
  const T *src[kDecodeSlots];
  bool use[kDecodeSlots];
  float cf[kDecodeSlots];
#pragma unroll
  for (int s = 0; s < kDecodeSlots; ++s) {
    use[s] = s < top_k && s_src[s] != nullptr;
    src[s] = use[s] ? s_src[s] : x;  // dropped slots read the token's own row and store zeros
    cf[s] = s < top_k ? s_coef[s] : 0.f;
  }
  for (int h0 = t * 8; h0 < hidden; h0 += kThreads * 8) {
    tm_u32x4 raw[kDecodeSlots];
#pragma unroll
    for (int s = 0; s < kDecodeSlots; ++s) raw[s] = *reinterpret_cast<const tm_u32x4 *>(src[s] + h0);
    float xin[8], acc[8];
    tm_load8<DT>(x + h0, xin);
    if (residual) {
      tm_load8<DT>(residual + h0, acc);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.f;
    }
    // every source row of the chunk is loaded before any is used (the
    // compiler would otherwise move a load into the branch of its use)
#pragma unroll
    for (int s = 0; s < kDecodeSlots; ++s) asm volatile("" : "+v"(raw[s]));
    float v[kDecodeSlots][8];
#pragma unroll
    for (int s = 0; s < kDecodeSlots; ++s) {
      const T *ev = reinterpret_cast<const T *>(&raw[s]);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[s][i] = use[s] ? Elem<DT>::to_f(ev[i]) : 0.f;
    }
#pragma unroll
    for (int s = 0; s < kDecodeSlots; ++s)  // sources in slot order, as combine_row adds them
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = use[s] ? fmaf(cf[s], v[s][i], acc[i]) : acc[i];
    tm_store8<DT>(out + h0, acc);
    tm_store8<DT>(ring_keys + r * (int64_t)hidden + h0, xin);
#pragma unroll
    for (int s = 0; s < kDecodeSlots; ++s)
      if (s < top_k) tm_store8<DT>(online_values + r * ov_w + s * ov_s + h0, v[s]);
  }
}

// ---------------------------------------------------------------------------
// a12: ring write of the online window
// ---------------------------------------------------------------------------
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void online_update_kernel(
    const typename Elem<DT>::T *__restrict__ hidden_in, int64_t ld_h, const int64_t *__restrict__ ids,
    int64_t ld_ids, const typename Elem<DT>::T *__restrict__ outputs, int64_t os_b, int64_t os_s,
    const uint8_t *__restrict__ valid, int64_t ld_valid, int top_k, int hidden, int64_t start,
    int64_t ring_size, typename Elem<DT>::T *__restrict__ ring_keys, int64_t *__restrict__ ring_ids,
    typename Elem<DT>::T *__restrict__ ring_values) {
  using T = typename Elem<DT>::T;
  const int64_t i = blockIdx.x;
  const int64_t r = (start + i) % ring_size;
  if (threadIdx.x < top_k) {
    const int s = threadIdx.x;
    const bool ok = valid == nullptr || valid[i * ld_valid + s];
    ring_ids[r * top_k + s] = ok ? ids[i * ld_ids + s] : -1;
  }
  const float one = 1.f;
  const T *hsrc = hidden_in + i * ld_h;
  combine_row<DT, VEC>(&hsrc, &one, 1, nullptr, ring_keys + r * hidden, hidden);
  for (int s = 0; s < top_k; ++s) {
    const bool ok = valid == nullptr || valid[i * ld_valid + s];
    const T *src = outputs + i * os_b + s * os_s;
    combine_row<DT, VEC>(&src, &one, ok ? 1 : 0, nullptr, ring_values + (r * top_k + s) * hidden, hidden);
  }
}

template <int DT>
constexpr int64_t vec_elems() { return 16 / Elem<DT>::kBytes; }

// True when rows starting at `base` with element stride `ld` are 16-byte aligned.
static bool rows_aligned(const void *base, int64_t ld, int elem_bytes) {
  return base == nullptr || (tm_aligned16(base) && ((ld * elem_bytes) % 16 == 0));
}

}  // namespace

// ===========================================================================
extern "C" int tm_gather_rows(int32_t dtype, const void *values, int64_t n_experts, int64_t n_centroids,
                              int32_t hidden, int64_t vs_e, int64_t vs_m, int64_t vs_c,
                              const int64_t *eids, const int64_t *mids, int32_t modality,
                              const int64_t *cids, int64_t n_rows, const int64_t *dst_rows, void *out,
                              int64_t n_out_rows, int64_t ld_out, tm_stream_t stream) {
  TM_REQUIRE(n_rows >= 0 && hidden > 0 && ld_out >= hidden && n_out_rows >= 0, TM_EINVAL_SHAPE,
             "tm_gather_rows: bad sizes");
  if (n_rows == 0) return TM_OK;
  TM_REQUIRE(values && eids && cids && out, TM_EINVAL_ARG, "tm_gather_rows: null pointer");
  TM_REQUIRE(n_rows < (int64_t)0x7fffffff, TM_EINVAL_SHAPE, "tm_gather_rows: too many rows");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const bool vec = hidden % 8 == 0 && tm_aligned16(values) && (vs_e * E) % 16 == 0 &&
                     (vs_m * E) % 16 == 0 && (vs_c * E) % 16 == 0 && rows_aligned(out, ld_out, E);
    auto V = static_cast<const T *>(values);
    auto O = static_cast<T *>(out);
    if (vec)
      hipLaunchKernelGGL((gather_rows_kernel<DT, true>), dim3((unsigned)n_rows), dim3(kThreads), 0,
                         tm_hip_stream(stream), V, n_experts, n_centroids, hidden, vs_e, vs_m, vs_c,
                         eids, mids, modality, cids, dst_rows, O, n_out_rows, ld_out);
    else
      hipLaunchKernelGGL((gather_rows_kernel<DT, false>), dim3((unsigned)n_rows), dim3(kThreads), 0,
                         tm_hip_stream(stream), V, n_experts, n_centroids, hidden, vs_e, vs_m, vs_c,
                         eids, mids, modality, cids, dst_rows, O, n_out_rows, ld_out);
    TM_LAUNCH_CHECK("tm_gather_rows");
    return TM_OK;
  });
}

// Launch of the shape-specialised combine when (top_k, n_nearest) matches.
#define TM_GC_TK(TK_, NN_)                                                                                     \
  if (top_k == TK_ && n_nearest == NN_) {                                                                      \
    if (hidden <= 8 * kTk1MaxThreads)                                                                          \
      hipLaunchKernelGGL((gather_combine_tk1_kernel<DT, TK_, NN_>), grid, dim3(tk1_threads), 0, s, hidden,    \
                         keep, static_cast<const T *>(slot_out), so_b, so_s, weights, ld_w,                    \
                         static_cast<const T *>(values), n_cent, ld_v, idx, dist, ld_idx,                       \
                         static_cast<const T *>(residual), ld_r, static_cast<T *>(out), ld_o);                  \
    else                                                                                                       \
      hipLaunchKernelGGL((gather_combine_tk_kernel<DT, TK_, NN_>), grid, block, 0, s, hidden, keep,            \
                         static_cast<const T *>(slot_out), so_b, so_s, weights, ld_w,                           \
                         static_cast<const T *>(values), n_cent, ld_v, idx, dist, ld_idx,                       \
                         static_cast<const T *>(residual), ld_r, static_cast<T *>(out), ld_o);                  \
    TM_LAUNCH_CHECK("tm_gather_combine");                                                                      \
    return TM_OK;                                                                                              \
  }

extern "C" int tm_gather_combine(int32_t dtype, int64_t n_tokens, int32_t hidden, const uint8_t *keep,
                                 const void *slot_out, int64_t so_b, int64_t so_s, const float *weights,
                                 int64_t ld_w, int32_t top_k, const void *values, int64_t n_cent,
                                 int64_t ld_v, const int64_t *idx, const float *dist, int64_t ld_idx,
                                 int32_t n_nearest, const void *residual, int64_t ld_r, void *out,
                                 int64_t ld_o, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && hidden > 0 && top_k >= 1 && top_k <= kMaxSrc && n_nearest >= 1 &&
                 n_nearest <= kMaxSrc && ld_o >= hidden && ld_v >= hidden && ld_w >= top_k &&
                 ld_idx >= n_nearest,
             TM_EINVAL_SHAPE, "tm_gather_combine: bad sizes");
  TM_REQUIRE(n_tokens < (int64_t)0x7fffffff, TM_EINVAL_SHAPE, "tm_gather_combine: too many tokens");
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(keep && slot_out && weights && values && idx && out && (n_nearest == 1 || dist),
             TM_EINVAL_ARG, "tm_gather_combine: null pointer");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const bool vec = hidden % 8 == 0 && tm_aligned16(slot_out) && (so_b * E) % 16 == 0 &&
                     (so_s * E) % 16 == 0 && rows_aligned(values, ld_v, E) &&
                     rows_aligned(residual, ld_r, E) && rows_aligned(out, ld_o, E);
    const bool fast = top_k <= kFastSrc && n_nearest <= kFastSrc;
    if constexpr (Elem<DT>::kBytes == 2) {
      if (vec) {
        const dim3 grid((unsigned)n_tokens), block(kThreads);
        const unsigned tk1_threads = (unsigned)((hidden / 8 + 63) / 64 * 64);  // one chunk per thread
        hipStream_t s = tm_hip_stream(stream);
        TM_GC_TK(8, 1)
        TM_GC_TK(8, 4)
        TM_GC_TK(6, 1)
        TM_GC_TK(6, 4)
      }
    }
    auto launch = [&](auto vec_tag) {
      constexpr bool VEC = decltype(vec_tag)::value;
      if (fast)
        hipLaunchKernelGGL((gather_combine_fast_kernel<DT, VEC>), dim3((unsigned)tm_cdiv(n_tokens, kRowsPerGroup)),
                           dim3(kThreads), 0, tm_hip_stream(stream), n_tokens, hidden, keep,
                           static_cast<const T *>(slot_out), so_b,
                           so_s, weights, ld_w, top_k, static_cast<const T *>(values), n_cent, ld_v, idx,
                           dist, ld_idx, n_nearest, static_cast<const T *>(residual), ld_r,
                           static_cast<T *>(out), ld_o);
      else
        hipLaunchKernelGGL((gather_combine_kernel<DT, VEC>), dim3((unsigned)n_tokens), dim3(kThreads), 0,
                           tm_hip_stream(stream), hidden, keep, static_cast<const T *>(slot_out), so_b,
                           so_s, weights, ld_w, top_k, static_cast<const T *>(values), n_cent, ld_v, idx,
                           dist, ld_idx, n_nearest, static_cast<const T *>(residual), ld_r,
                           static_cast<T *>(out), ld_o);
    };
    if (vec) launch(std::true_type{});
    else launch(std::false_type{});
    TM_LAUNCH_CHECK("tm_gather_combine");
    return TM_OK;
  });
}

#undef TM_GC_TK

extern "C" int tm_gather_combine_ranked(int32_t dtype, int64_t n_tokens, int32_t hidden, const void *slot_out,
                                        int64_t so_b, int64_t so_s, const float *weights, int64_t ld_w,
                                        int32_t top_k, const void *values, int64_t n_cent, int64_t ld_v,
                                        const int64_t *idx, const float *dist, const void *residual, int64_t ld_r,
                                        void *out, int64_t ld_o, int64_t n_keep, uint8_t *out_keep,
                                        tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && hidden > 0 && ld_w >= top_k && ld_o >= hidden && ld_v >= hidden, TM_EINVAL_SHAPE,
             "tm_gather_combine_ranked: bad sizes");
  // each token's workgroup reads all n distances: the work grows as n^2
  TM_REQUIRE(n_tokens <= TM_RANKED_MAX_TOKENS, TM_EINVAL_SHAPE,
             "tm_gather_combine_ranked: %lld tokens > %d (use tm_keep_select + tm_gather_combine)",
             (long long)n_tokens, TM_RANKED_MAX_TOKENS);
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(dtype == TM_DT_BF16 || dtype == TM_DT_F16, TM_EINVAL_DTYPE,
             "tm_gather_combine_ranked: dtype must be F16 or BF16");
  TM_REQUIRE(slot_out && weights && values && idx && dist && out && out_keep, TM_EINVAL_ARG,
             "tm_gather_combine_ranked: null pointer");
  TM_REQUIRE(tm_internal_combine_rank_ok(dtype, hidden, slot_out, so_b, so_s, top_k, values, ld_v, dist, residual,
                                         ld_r, out, ld_o),
             TM_EINVAL_SHAPE,
             "tm_gather_combine_ranked: needs top_k 6 or 8, hidden <= 2048 and a multiple of 8, aligned rows");
  return tm_internal_combine_rank(dtype, n_tokens, hidden, slot_out, so_b, so_s, weights, ld_w, top_k, values,
                                  n_cent, ld_v, idx, dist, residual, ld_r, out, ld_o, n_keep, out_keep,
                                  tm_hip_stream(stream));
}

bool tm_internal_combine_rank_ok(int32_t dtype, int32_t hidden, const void *slot_out, int64_t so_b, int64_t so_s,
                                 int32_t top_k, const void *values, int64_t ld_v, const float *dist,
                                 const void *residual, int64_t ld_r, const void *out, int64_t ld_o) {
  if (!(dtype == TM_DT_BF16 || dtype == TM_DT_F16 || dtype == TM_DT_F32) || !(top_k == 6 || top_k == 8) ||
      hidden <= 0 || hidden > kThreads * 8)
    return false;
  const int E = dtype == TM_DT_F32 ? 4 : 2;
  return hidden % 8 == 0 && tm_aligned16(slot_out) && (so_b * E) % 16 == 0 && (so_s * E) % 16 == 0 &&
         rows_aligned(values, ld_v, E) && rows_aligned(residual, ld_r, E) && rows_aligned(out, ld_o, E) &&
         ld_o >= hidden && ld_v >= hidden && dist != nullptr && tm_aligned16(dist);
}

int tm_internal_combine_rank(int32_t dtype, int64_t n_tokens, int32_t hidden, const void *slot_out, int64_t so_b,
                             int64_t so_s, const float *weights, int64_t ld_w, int32_t top_k, const void *values,
                             int64_t n_cent, int64_t ld_v, const int64_t *idx, const float *dist,
                             const void *residual, int64_t ld_r, void *out, int64_t ld_o, int64_t n_keep,
                             uint8_t *keep_out, hipStream_t s) {
  TM_REQUIRE(tm_internal_combine_rank_ok(dtype, hidden, slot_out, so_b, so_s, top_k, values, ld_v, dist, residual,
                                         ld_r, out, ld_o) &&
                 n_tokens > 0 && n_tokens < (int64_t)0x7fffffff && ld_w >= top_k,
             TM_EINVAL_SHAPE, "tm_table_forward: combine shape not supported by the ranked path");
  TM_REQUIRE(weights && idx && keep_out && values && slot_out && out, TM_EINVAL_ARG,
             "tm_table_forward: combine: null pointer");
  const RankKeep rk{n_tokens, n_keep, keep_out};
  auto launch = [&](auto dt_tag, auto tk_tag) {
    constexpr int DT = decltype(dt_tag)::value;
    constexpr int TK = decltype(tk_tag)::value;
    using T = typename Elem<DT>::T;
    auto kern = n_tokens <= kRankOnePass<kRankTokens> ? gather_combine_rank_kernel<DT, TK, kRankTokens, true>
                                                        : gather_combine_rank_kernel<DT, TK, kRankTokens, false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)tm_cdiv(n_tokens, kRankTokens)), dim3(kRankTokens * kThreads), 0, s,
                       hidden, static_cast<const T *>(slot_out), so_b, so_s, weights, ld_w,
                       static_cast<const T *>(values), n_cent, ld_v, idx, dist, static_cast<const T *>(residual),
                       ld_r, static_cast<T *>(out), ld_o, rk);
  };
  using BF = std::integral_constant<int, TM_DT_BF16>;
  using HF = std::integral_constant<int, TM_DT_F16>;
  using F32 = std::integral_constant<int, TM_DT_F32>;
  using K8 = std::integral_constant<int, 8>;
  using K6 = std::integral_constant<int, 6>;
  if (dtype == TM_DT_BF16)
    top_k == 8 ? launch(BF{}, K8{}) : launch(BF{}, K6{});
  else if (dtype == TM_DT_F16)
    top_k == 8 ? launch(HF{}, K8{}) : launch(HF{}, K6{});
  else
    top_k == 8 ? launch(F32{}, K8{}) : launch(F32{}, K6{});
  TM_LAUNCH_CHECK("tm_table_forward(combine)");
  return TM_OK;
}

extern "C" int tm_slot_combine(int32_t dtype, int64_t n_tokens, int32_t top_k, int32_t hidden,
                               const float *weights, int64_t ld_w, const uint8_t *compute_mask,
                               const void *computed, int64_t cs_b, int64_t cs_s, const uint8_t *off_hit,
                               const int64_t *off_idx, const int64_t *sel, int64_t ld_m,
                               const uint8_t *is_vision, const void *values, int64_t n_experts,
                               int64_t n_centroids, int64_t vs_e, int64_t vs_m, int64_t vs_c,
                               const uint8_t *on_hit, const int64_t *on_idx, const int64_t *on_slot,
                               const void *online_values, int64_t n_online, int32_t online_topk,
                               int64_t ov_w, int64_t ov_s, int32_t target_mode, const void *residual,
                               int64_t ld_r, void *out, int64_t ld_out, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && top_k >= 1 && top_k <= kMaxSrc && hidden > 0 && ld_w >= top_k &&
                 ld_m >= top_k && ld_out >= hidden,
             TM_EINVAL_SHAPE, "tm_slot_combine: bad sizes");
  TM_REQUIRE(target_mode == TM_TARGET_ONE || target_mode == TM_TARGET_ORIG_SUM, TM_EINVAL_ARG,
             "tm_slot_combine: bad target mode %d", target_mode);
  TM_REQUIRE(n_tokens < (int64_t)0x7fffffff, TM_EINVAL_SHAPE, "tm_slot_combine: too many tokens");
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(weights && out, TM_EINVAL_ARG, "tm_slot_combine: null pointer");
  TM_REQUIRE(!compute_mask || computed, TM_EINVAL_ARG, "tm_slot_combine: compute_mask needs computed");
  TM_REQUIRE(!off_hit || (off_idx && sel && values), TM_EINVAL_ARG,
             "tm_slot_combine: off_hit needs off_idx, sel and values");
  TM_REQUIRE(!on_hit || (on_idx && on_slot && online_values), TM_EINVAL_ARG,
             "tm_slot_combine: on_hit needs on_idx, on_slot and online_values");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const bool vec = hidden % 8 == 0 && (computed == nullptr || (tm_aligned16(computed) && (cs_b * E) % 16 == 0 &&
                                                                  (cs_s * E) % 16 == 0)) &&
                     (values == nullptr || (tm_aligned16(values) && (vs_e * E) % 16 == 0 &&
                                            (vs_m * E) % 16 == 0 && (vs_c * E) % 16 == 0)) &&
                     (online_values == nullptr || (tm_aligned16(online_values) && (ov_w * E) % 16 == 0 &&
                                                   (ov_s * E) % 16 == 0)) &&
                     rows_aligned(residual, ld_r, E) && rows_aligned(out, ld_out, E);
    auto launch = [&](auto vec_tag) {
      constexpr bool VEC = decltype(vec_tag)::value;
      hipLaunchKernelGGL((slot_combine_kernel<DT, VEC>), dim3((unsigned)n_tokens), dim3(kThreads), 0,
                         tm_hip_stream(stream), top_k, hidden, weights, ld_w, compute_mask,
                         static_cast<const T *>(computed), cs_b, cs_s, off_hit, off_idx, sel, ld_m,
                         is_vision, static_cast<const T *>(values), n_experts, n_centroids, vs_e, vs_m,
                         vs_c, on_hit, on_idx, on_slot, static_cast<const T *>(online_values), n_online,
                         online_topk, ov_w, ov_s, target_mode, static_cast<const T *>(residual), ld_r,
                         static_cast<T *>(out), ld_out);
    };
    if (vec) launch(std::true_type{});
    else launch(std::false_type{});
    TM_LAUNCH_CHECK("tm_slot_combine");
    return TM_OK;
  });
}

extern "C" int tm_online_update(int32_t dtype, const void *hidden, int64_t ld_h, const int64_t *ids,
                                int64_t ld_ids, const void *outputs, int64_t os_b, int64_t os_s,
                                const uint8_t *valid, int64_t ld_valid, int64_t n_rows, int32_t top_k,
                                int32_t hidden_dim, int64_t start, int64_t ring_size, void *ring_keys,
                                int64_t *ring_ids, void *ring_values, tm_stream_t stream) {
  TM_REQUIRE(n_rows >= 0 && ring_size > 0 && n_rows <= ring_size && top_k >= 0 && top_k <= kThreads &&
                 hidden_dim > 0 && start >= 0 && start < ring_size,
             TM_EINVAL_SHAPE, "tm_online_update: bad sizes (rows %lld, ring %lld, start %lld)",
             (long long)n_rows, (long long)ring_size, (long long)start);
  if (n_rows == 0) return TM_OK;
  TM_REQUIRE(hidden && ids && outputs && ring_keys && ring_ids && ring_values, TM_EINVAL_ARG,
             "tm_online_update: null pointer");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const bool vec = hidden_dim % 8 == 0 && rows_aligned(hidden, ld_h, E) && tm_aligned16(outputs) &&
                     (os_b * E) % 16 == 0 && (os_s * E) % 16 == 0 && tm_aligned16(ring_keys) &&
                     tm_aligned16(ring_values);
    auto launch = [&](auto vec_tag) {
      constexpr bool VEC = decltype(vec_tag)::value;
      hipLaunchKernelGGL((online_update_kernel<DT, VEC>), dim3((unsigned)n_rows), dim3(kThreads), 0,
                         tm_hip_stream(stream), static_cast<const T *>(hidden), ld_h, ids, ld_ids,
                         static_cast<const T *>(outputs), os_b, os_s, valid, ld_valid, top_k, hidden_dim,
                         start, ring_size, static_cast<T *>(ring_keys), ring_ids, static_cast<T *>(ring_values));
    };
    if (vec) launch(std::true_type{});
    else launch(std::false_type{});
    TM_LAUNCH_CHECK("tm_online_update");
    return TM_OK;
  });
}

extern "C" int tm_decode_combine_update(int32_t dtype, int32_t top_k, int32_t hidden, const float *weights,
                                        const uint8_t *compute_mask, const void *computed, int64_t cs_s,
                                        const uint8_t *off_hit, const int64_t *off_idx, const int64_t *sel,
                                        const uint8_t *is_vision, const void *values, int64_t n_experts,
                                        int64_t n_centroids, int64_t vs_e, int64_t vs_m, int64_t vs_c,
                                        const uint8_t *on_hit, const int64_t *on_idx, const int64_t *on_slot,
                                        void *online_values, int64_t n_online, int32_t online_topk, int64_t ov_w,
                                        int64_t ov_s, int32_t target_mode, const void *residual, void *out,
                                        const void *x, void *online_keys, int64_t *online_ids, int64_t ring_row,
                                        tm_stream_t stream) {
  TM_REQUIRE(top_k >= 1 && top_k <= kDecodeSlots && hidden > 0 && hidden % 8 == 0 && top_k == online_topk &&
                 n_online >= 1 && ring_row >= 0 && ring_row < n_online && ov_w >= (int64_t)top_k * ov_s &&
                 ov_s >= hidden,
             TM_EINVAL_SHAPE, "tm_decode_combine_update: bad sizes (top_k <= %d, hidden %% 8 == 0, ring row in range)",
             kDecodeSlots);
  TM_REQUIRE(target_mode == TM_TARGET_ONE || target_mode == TM_TARGET_ORIG_SUM, TM_EINVAL_ARG,
             "tm_decode_combine_update: bad target mode %d", target_mode);
  TM_REQUIRE(weights && out && x && online_values && online_keys && online_ids, TM_EINVAL_ARG,
             "tm_decode_combine_update: null pointer");
  TM_REQUIRE(!compute_mask || computed, TM_EINVAL_ARG, "tm_decode_combine_update: compute_mask needs computed");
  TM_REQUIRE(!off_hit || (off_idx && sel && values), TM_EINVAL_ARG,
             "tm_decode_combine_update: off_hit needs off_idx, sel and values");
  TM_REQUIRE(sel, TM_EINVAL_ARG, "tm_decode_combine_update: sel is required (the ring stores the ids)");
  TM_REQUIRE(!on_hit || (on_idx && on_slot), TM_EINVAL_ARG, "tm_decode_combine_update: on_hit needs on_idx, on_slot");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const bool aligned = tm_aligned16(out) && tm_aligned16(x) && tm_aligned16(online_keys) &&
                         tm_aligned16(online_values) && (ov_w * E) % 16 == 0 && (ov_s * E) % 16 == 0 &&
                         (computed == nullptr || (tm_aligned16(computed) && (cs_s * E) % 16 == 0)) &&
                         (values == nullptr || (tm_aligned16(values) && (vs_e * E) % 16 == 0 &&
                                                (vs_m * E) % 16 == 0 && (vs_c * E) % 16 == 0)) &&
                         (residual == nullptr || tm_aligned16(residual));
    TM_REQUIRE(aligned, TM_EINVAL_SHAPE, "tm_decode_combine_update: rows must be 16-byte aligned");
    hipLaunchKernelGGL((slot_combine_update_kernel<DT>), dim3(1), dim3(kThreads), 0, tm_hip_stream(stream), top_k,
                       hidden, weights, compute_mask, static_cast<const T *>(computed), cs_s, off_hit, off_idx, sel,
                       is_vision, static_cast<const T *>(values), n_experts, n_centroids, vs_e, vs_m, vs_c, on_hit,
                       on_idx, on_slot, static_cast<T *>(online_values), n_online, online_topk, ov_w, ov_s,
                       target_mode, static_cast<const T *>(residual), static_cast<T *>(out),
                       static_cast<const T *>(x), static_cast<T *>(online_keys), online_ids, ring_row);
    TM_LAUNCH_CHECK("tm_decode_combine_update");
    return TM_OK;
  });
}
