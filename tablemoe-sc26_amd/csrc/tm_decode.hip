// Decode plan of the one-call layer (tm_table_forward, n <= 64 tokens).
//
// A decode step moves a few MB (the centroid table, one P, a handful of rows)
// and each stage of the general plan is latency-bound on a few workgroups
// (the projection of 32 tokens ran on 2 workgroups, each streaming all of P).
// Here the layer is three launches, each spread over many workgroups:
//
//  1. project_split_kernel: one wave per (16-row tile, 16-column block, one
//     of kSlices slices of `hidden`); it issues all of its operand loads at
//     once, runs one MFMA chain and publishes its 16 x 16 fp32 partial.  The
//     last wave of a (tile, block) group to arrive (counter in the workspace,
//     reset by that wave) adds the partials in slice order, adds the bias,
//     rounds once (q = dtype(x P + bias), the contract of tm_project) and
//     writes q and the block's partial |q|^2.  The launch also resets the
//     rows' best keys and carries the router's workgroups.
//  2. search_stream_kernel (tm_search_global.hip): per-split sorted lists,
//     and each query's best key by 64-bit atomic minimum into one of kKeyRep
//     replicas (split % kKeyRep), so few workgroups contend for an address.
//  3. decode_finish_kernel: one wave per (token, 512-element row chunk).  It
//     ranks the token's best distance among the n tokens' (keep rule of
//     tm_keep_select: larger distance first, ties to the lower token index),
//     merges the token's split lists (the K smallest packed keys, a set, so
//     the same keys as merge_kernel), and combines its row chunk exactly as
//     gather_combine_tk_kernel does (fp32 from the residual, sources in order,
//     one rounding).  The chunk-0 wave also writes dist, idx, keep and |q|^2.
//
// Given the same q, every output equals the stage calls'; q itself may differ
// from tm_project's in the last bit (another fp32 summation order).
#include "tm_internal.h"
#include "tm_mfma.h"
#include "tm_route_dev.h"

namespace {

constexpr int kSlices = 8;     // hidden slices of the projection: one wave (workgroup) each
constexpr int kRound = 16;     // k-steps of operand loads issued together per wave
constexpr int kKeyRep = 8;     // replicas of the best-key array (spreads the search's atomics)
constexpr int kChunk = 512;    // row elements per finishing wave (64 lanes x 8)
constexpr int kMaxLists = 4;   // split lists per lane in the finishing kernel (nsplit <= 256)

struct SliceRoute {
  tm_route_args a;
  int64_t first;  // first router workgroup (0 = none)
};

// KPW > 0: every slice is exactly KPW whole k-steps (hidden == 32 * kSlices *
// KPW), so the loads and MFMAs carry no guards (a guard lets the compiler
// sink each load into its own branch and wait for it there).  KPW == 0: any
// hidden (multiple of 8), guarded rounds of kRound k-steps.
template <int DT, int DIM, int RVPL, int KPW>
__global__ __launch_bounds__(64) void project_split_kernel(
    const typename Elem<DT>::T *__restrict__ x, int64_t n, int hidden, int64_t ld_x,
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ pv,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ pt,
    const typename Elem<DT>::T *__restrict__ bt, typename Elem<DT>::T *__restrict__ q, int64_t ld_q,
    float *__restrict__ qn_blk, uint64_t *__restrict__ keys, float4 *part, uint32_t *cnt, SliceRoute sr) {
  using T = typename Elem<DT>::T;
  constexpr int NCB = DIM / 16;
  constexpr int S = kSlices;
  const int lane = threadIdx.x;
  if constexpr (RVPL > 0) {
    if ((int64_t)blockIdx.x >= sr.first) {  // uniform: router workgroup, 8 tokens
      const int64_t tok = ((int64_t)blockIdx.x - sr.first) * 8 + (lane >> 3);
      tm_route_token<RVPL, 8>(sr.a.logits, n, sr.a.ld, sr.a.top_k, 0, sr.a.out_w, sr.a.out_ids, tok, lane & 7);
      return;
    }
  }
  const int sl = (int)(blockIdx.x % S);           // hidden slice
  const int64_t g = (int64_t)(blockIdx.x / S);    // (tile, column block) group
  const int cb = (int)(g % NCB);
  const int64_t row0 = (g / NCB) * 16;
  const int64_t arow = row0 + (lane & 15);
  const bool arow_ok = arow < n;
  const T *xrow = x + (arow_ok ? arow : 0) * ld_x;

  const int nks = (hidden + 31) / 32;
  const int per = (nks + S - 1) / S;
  const int ks_begin = sl * per;
  const int ks_end = (ks_begin + per < nks) ? ks_begin + per : nks;
  const int klast = ks_end - 1;  // >= 0 (an empty slice clamps to the last k-step and multiplies nothing)
  const int kq = 8 * (lane >> 4);

  // modality of the tile's rows first: the operand loads depend on it
  const uint8_t *vsrc = is_vision ? is_vision + (arow_ok ? arow : 0) : reinterpret_cast<const uint8_t *>(x);
  const uint8_t vis_byte = *vsrc;
  // the reducer's bias values, loaded now so their latency hides behind the slice
  const int col = cb * 16 + (lane & 15);
  const float bias_v = Elem<DT>::to_f(bv[col]);
  const float bias_t = Elem<DT>::to_f(bt[col]);
  const int amod = !arow_ok ? 2 : ((is_vision == nullptr || vis_byte) ? 0 : 1);
  const uint32_t vis_bits = (uint32_t)(__ballot(amod == 0) & 0xFFFFull);
  const uint32_t txt_bits = (uint32_t)(__ballot(amod == 1) & 0xFFFFull);

  tm_f32x4 fin = tm_f32x4{0.f, 0.f, 0.f, 0.f};
  auto run_pass = [&](const T *P, uint32_t rows_of_pass) {
    const uint4 *pf = reinterpret_cast<const uint4 *>(P) + lane;
    tm_f32x4 acc = tm_f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (KPW > 0) {
      uint4 ar[KPW], br[KPW];
#pragma unroll
      for (int j = 0; j < KPW; ++j) {
        ar[j] = *reinterpret_cast<const uint4 *>(xrow + (ks_begin + j) * 32 + kq);
        br[j] = pf[((int64_t)(ks_begin + j) * NCB + cb) * 64];
      }
#pragma unroll
      for (int j = 0; j < KPW; ++j) acc = tm_mfma16x16x32<DT>(ar[j], br[j], acc);
    } else {
    for (int r0 = ks_begin; r0 < ks_end; r0 += kRound) {  // uniform; one round for hidden <= 32 * S * kRound
      uint4 ar[kRound], br[kRound];
      bool kin[kRound];
#pragma unroll
      for (int j = 0; j < kRound; ++j) {  // every load of the round in flight together
        const int kc = r0 + j < klast ? r0 + j : klast;
        const int kraw = kc * 32 + kq;
        kin[j] = kraw < hidden;
        const int k = kraw < hidden - 8 ? kraw : hidden - 8;
        ar[j] = *reinterpret_cast<const uint4 *>(xrow + k);
        br[j] = pf[((int64_t)kc * NCB + cb) * 64];
      }
#pragma unroll
      for (int j = 0; j < kRound; ++j)
        if (r0 + j < ks_end)  // uniform
          acc = tm_mfma16x16x32<DT>(kin[j] ? ar[j] : make_uint4(0, 0, 0, 0), br[j], acc);
    }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if ((rows_of_pass >> (4 * (lane >> 4) + i)) & 1u) fin[i] = acc[i];
  };
  if (vis_bits) run_pass(pv, vis_bits);  // uniform branches
  if (txt_bits) run_pass(pt, txt_bits);

  // reset the tile's best keys (every replica) for the search launch
  if (cb == 0 && lane < 16 && arow_ok)
    for (int r = sl; r < kKeyRep; r += S) keys[(int64_t)r * n + arow] = ~0ull;

  // Publish this slice's 16 x 16 partial (fragment order), then count the
  // arrival.  The partials and the counter move through agent-scope relaxed
  // atomics, which are coherent across the XCDs' L2 caches per location; the
  // workgroup-scope fences keep the order (stores complete before the count,
  // the count before the partials are read) without the L2 write-back and
  // invalidate an agent-scope fence performs.
  uint64_t *pp = reinterpret_cast<uint64_t *>(part) + ((g * S + sl) * 64 + lane) * 2;
  __hip_atomic_store(pp, ((uint64_t)__float_as_uint(fin[1]) << 32) | __float_as_uint(fin[0]), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(pp + 1, ((uint64_t)__float_as_uint(fin[3]) << 32) | __float_as_uint(fin[2]), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);  // both stores acknowledged before the count
  uint32_t ticket = 0;
  if (lane == 0) ticket = __hip_atomic_fetch_add(cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ticket = (uint32_t)__builtin_amdgcn_readfirstlane((int)ticket);
  if (ticket != S - 1) return;  // uniform: not the last slice of the group
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (lane == 0) __hip_atomic_store(cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next call

  // Last arrival: the S partials added in slice order, bias, one rounding.
  uint64_t pv2[S][2];
#pragma unroll
  for (int s2 = 0; s2 < S; ++s2) {
    const uint64_t *src = reinterpret_cast<const uint64_t *>(part) + ((g * S + s2) * 64 + lane) * 2;
    pv2[s2][0] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    pv2[s2][1] = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < S; ++s2) {
    v[0] += __uint_as_float((uint32_t)pv2[s2][0]);
    v[1] += __uint_as_float((uint32_t)(pv2[s2][0] >> 32));
    v[2] += __uint_as_float((uint32_t)pv2[s2][1]);
    v[3] += __uint_as_float((uint32_t)(pv2[s2][1] >> 32));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * (lane >> 4) + i;
    const bool vis = (vis_bits >> r) & 1u;
    v[i] = tm_round<DT>(v[i] + (vis ? bias_v : bias_t));
    // |q|^2 over this block's 16 columns: the squares summed over the 16 lanes of the row group
    float sq = v[i] * v[i];
    sq += __shfl_xor(sq, 1, 64);
    sq += __shfl_xor(sq, 2, 64);
    sq += __shfl_xor(sq, 4, 64);
    sq += __shfl_xor(sq, 8, 64);
    const int64_t gr = row0 + r;
    if (gr < n) {
      q[gr * ld_q + col] = Elem<DT>::from_f(v[i]);
      if ((lane & 15) == 0) qn_blk[gr * NCB + cb] = sq;
    }
  }
}

// |q|^2 from the NCB block partials, added as the butterfly of the row
// epilogue adds its lanes: pairwise, adjacent blocks first.
template <int NCB>
__device__ __forceinline__ float qn_tree(float (&b)[NCB]) {
#pragma unroll
  for (int w = NCB; w > 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w / 2; ++i) b[i] = b[2 * i] + b[2 * i + 1];
  return b[0];
}

// The K smallest of two ascending K-lists, ascending (bitonic min-merge).
template <int K>
__device__ __forceinline__ void merge_min_k(uint64_t (&a)[K], const uint64_t (&b)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) a[i] = a[i] < b[K - 1 - i] ? a[i] : b[K - 1 - i];
#pragma unroll
  for (int d = K / 2; d > 0; d >>= 1)
#pragma unroll
    for (int i = 0; i < K; ++i)
      if ((i & d) == 0) {
        const uint64_t lo = a[i] < a[i + d] ? a[i] : a[i + d];
        const uint64_t hi = a[i] < a[i + d] ? a[i + d] : a[i];
        a[i] = lo;
        a[i + d] = hi;
      }
}

template <int DT, int TK, int NN, int NCB, int ML>
__global__ __launch_bounds__(64) void decode_finish_kernel(
    int64_t n, int hidden, int n_chunks, const uint64_t *__restrict__ keys, const float *__restrict__ qn_blk,
    const uint64_t *__restrict__ lists, int64_t nsplit, int l2, int64_t n_keep,
    const typename Elem<DT>::T *__restrict__ slot_out, int64_t so_b, int64_t so_s, const float *__restrict__ w,
    const typename Elem<DT>::T *__restrict__ values, int64_t n_cent, int64_t ld_v,
    const typename Elem<DT>::T *__restrict__ residual, int64_t ld_r, typename Elem<DT>::T *__restrict__ out,
    int64_t ld_o, float *__restrict__ out_dist, int64_t *__restrict__ out_idx, float *__restrict__ out_qn,
    uint8_t *__restrict__ out_keep) {
  using T = typename Elem<DT>::T;
  constexpr int K = NN;  // list length of the search (1 or 4)
  const int lane = threadIdx.x;
  const int b = (int)(blockIdx.x / n_chunks);  // token (uniform)
  const int ch = (int)(blockIdx.x % n_chunks);
  const int h0 = ch * kChunk + lane * 8;
  const int hl = h0 < hidden ? h0 : hidden - 8;  // lanes past the row re-read its last 16 bytes, store nothing

  // every load that does not depend on another is issued first
  const int jl = lane < n ? lane : (int)n - 1;
  uint64_t kr[kKeyRep];
#pragma unroll
  for (int r = 0; r < kKeyRep; ++r) kr[r] = keys[(int64_t)r * n + jl];
  float qb[NCB];
#pragma unroll
  for (int c = 0; c < NCB; c += 4) {
    const float4 f = *reinterpret_cast<const float4 *>(qn_blk + (int64_t)jl * NCB + c);
    qb[c] = f.x; qb[c + 1] = f.y; qb[c + 2] = f.z; qb[c + 3] = f.w;
  }
  uint64_t lst[K];
#pragma unroll
  for (int j = 0; j < K; ++j) lst[j] = ~0ull;
  if constexpr (K > 1) {
#pragma unroll
    for (int m = 0; m < ML; ++m) {
      const int64_t s = lane + 64 * m;
      const uint64_t *src = lists + ((s < nsplit ? s : nsplit - 1) * n + b) * K;
      uint64_t o[K];
#pragma unroll
      for (int j = 0; j < K; j += 2) {
        const uint4 v = *reinterpret_cast<const uint4 *>(src + j);
        o[j] = ((uint64_t)v.y << 32) | v.x;
        o[j + 1] = ((uint64_t)v.w << 32) | v.z;
      }
#pragma unroll
      for (int j = 0; j < K; ++j) o[j] = s < nsplit ? o[j] : ~0ull;
      merge_min_k<K>(lst, o);
    }
  }
  float wv[TK];
#pragma unroll
  for (int s = 0; s < TK; ++s) wv[s] = w[(int64_t)b * TK + s];
  float acc[8];
  if (residual) {
    tm_load8_nt<DT>(residual + (int64_t)b * ld_r + hl, acc);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  }

  // keep rank of token b among the n tokens' best distances
  uint64_t kj = kr[0];
#pragma unroll
  for (int r = 1; r < kKeyRep; ++r) kj = kr[r] < kj ? kr[r] : kj;
  const float qn_j = qn_tree<NCB>(qb);
  int64_t ix_j;
  const float d_j = tm_key_to_dist(kj, qn_j, l2 != 0, ix_j);
  const uint32_t key_j = tm_orderable(d_j);
  const uint32_t key_b = (uint32_t)__builtin_amdgcn_readlane((int)key_j, b);
  const float qn_b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qn_j), b));
  const bool ahead = lane < n && (key_j > key_b || (key_j == key_b && lane < b));
  const int rank = __popcll(__ballot(ahead));
  const bool kept = n_keep >= n ? true : (n_keep <= 0 ? false : rank < n_keep);

  // top-NN keys of token b
  if constexpr (K > 1) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      uint64_t other[K];
#pragma unroll
      for (int j = 0; j < K; ++j) other[j] = __shfl_xor(lst[j], o, 64);
      merge_min_k<K>(lst, other);
    }
  } else {
    lst[0] = (uint64_t)__builtin_amdgcn_readlane((int)(uint32_t)kj, b) |
             ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(kj >> 32), b) << 32);
  }
  float dn[NN];
  int64_t cn[NN];
#pragma unroll
  for (int j = 0; j < NN; ++j) dn[j] = tm_key_to_dist(lst[j], qn_b, l2 != 0, cn[j]);

  if (ch == 0 && lane == 0) {
#pragma unroll
    for (int j = 0; j < NN; ++j) {
      out_dist[(int64_t)b * NN + j] = dn[j];
      out_idx[(int64_t)b * NN + j] = cn[j];
    }
    out_keep[b] = kept ? 1 : 0;
    out_qn[b] = qn_b;
  }

  T *dst = out + (int64_t)b * ld_o + hl;
  if (kept) {  // uniform
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s) sum += wv[s];
    const bool any = sum > 0.f;
    float coef[TK];
#pragma unroll
    for (int s = 0; s < TK; ++s) coef[s] = wv[s] / sum;
    if (any) {
      const T *src = slot_out + (int64_t)b * so_b + hl;
      float v[TK][8];
#pragma unroll
      for (int s = 0; s < TK; ++s) tm_load8_nt<DT>(src + (int64_t)s * so_s, v[s]);
#pragma unroll
      for (int s = 0; s < TK; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(coef[s], v[s][i], acc[i]);
    }
  } else {
    const T *src[NN];
    float coef[NN];
    bool okc[NN];
    float inv_sum = 0.f;
#pragma unroll
    for (int j = 0; j < NN; ++j) {
      okc[j] = cn[j] >= 0 && cn[j] < n_cent;
      src[j] = values + (okc[j] ? cn[j] : 0) * ld_v + hl;
      coef[j] = okc[j] ? ((NN > 1) ? 1.f / (dn[j] + 1e-6f) : 1.f) : 0.f;
      inv_sum += coef[j];
    }
    if (NN > 1) {
#pragma unroll
      for (int j = 0; j < NN; ++j) coef[j] = okc[j] ? coef[j] / inv_sum : 0.f;
    }
    float v[NN][8];
#pragma unroll
    for (int j = 0; j < NN; ++j) tm_load8<DT>(src[j], v[j]);
#pragma unroll
    for (int j = 0; j < NN; ++j)
      if (okc[j]) {  // uniform; the loads above are already issued
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(coef[j], v[j][i], acc[i]);
      }
  }
  if (h0 < hidden) tm_store8_nt<DT>(dst, acc);
}

template <int DT, int DIM, int RVPL, int KPW>
void launch_split(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w, const tm_route_args *ra,
                  hipStream_t s) {
  using T = typename Elem<DT>::T;
  const int64_t n = io->n_tokens;
  SliceRoute sr{};
  int64_t blocks = tm_cdiv(n, 16) * (DIM / 16) * kSlices;
  if (RVPL > 0) {
    sr.a = *ra;
    sr.first = blocks;
    blocks += tm_cdiv(n, 8);
  }
  const void *pt = t->proj_txt ? t->proj_txt : t->proj_vis;
  const void *bt = t->proj_txt ? t->bias_txt : t->bias_vis;
  hipLaunchKernelGGL((project_split_kernel<DT, DIM, RVPL, KPW>), dim3((unsigned)blocks), dim3(64), 0, s,
                     static_cast<const T *>(io->x), n, t->hidden, io->ld_x, io->is_vision,
                     static_cast<const T *>(t->proj_vis), static_cast<const T *>(t->bias_vis),
                     static_cast<const T *>(pt), static_cast<const T *>(bt), static_cast<T *>(io->q),
                     (int64_t)t->dim, w.qn_blk, w.keys, reinterpret_cast<float4 *>(w.part), w.cnt, sr);
}

template <int DT, int DIM, int RVPL>
void launch_split_kpw(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w,
                      const tm_route_args *ra, hipStream_t s) {
  const int h = t->hidden;
  const int kpw = (h % (32 * kSlices) == 0) ? h / (32 * kSlices) : 0;
  switch (kpw) {  // the model hidden sizes 1024, 2048, 2560, 3584, 4096
    case 4: launch_split<DT, DIM, RVPL, 4>(t, io, w, ra, s); break;
    case 8: launch_split<DT, DIM, RVPL, 8>(t, io, w, ra, s); break;
    case 10: launch_split<DT, DIM, RVPL, 10>(t, io, w, ra, s); break;
    case 14: launch_split<DT, DIM, RVPL, 14>(t, io, w, ra, s); break;
    case 16: launch_split<DT, DIM, RVPL, 16>(t, io, w, ra, s); break;
    default: launch_split<DT, DIM, RVPL, 0>(t, io, w, ra, s); break;
  }
}

template <int DT, int DIM>
void launch_split_route(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w,
                        const tm_route_args *ra, hipStream_t s) {
  if (ra == nullptr)
    launch_split_kpw<DT, DIM, 0>(t, io, w, ra, s);
  else if (ra->n_experts == 64)
    launch_split_kpw<DT, DIM, 8>(t, io, w, ra, s);
  else
    launch_split_kpw<DT, DIM, 16>(t, io, w, ra, s);
}

template <int DT, int TK, int NN, int NCB, int ML>
void launch_finish(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w, int64_t nsplit,
                   int64_t n_keep, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const int64_t n = io->n_tokens;
  const int n_chunks = (int)tm_cdiv(t->hidden, kChunk);
  hipLaunchKernelGGL((decode_finish_kernel<DT, TK, NN, NCB, ML>), dim3((unsigned)(n * n_chunks)), dim3(64), 0, s,
                     n, t->hidden, n_chunks, w.keys, w.qn_blk, w.lists, nsplit, t->metric == TM_METRIC_L2 ? 1 : 0, n_keep,
                     static_cast<const T *>(io->slot_out), io->so_b, io->so_s, io->weights,
                     static_cast<const T *>(t->values), t->n_cent, t->ld_v, static_cast<const T *>(io->residual),
                     io->ld_r, static_cast<T *>(io->out), io->ld_o, io->dist, io->idx, io->q_sqnorm, io->keep);
}

template <int DT, int TK, int NN, int NCB>
void finish_ml(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w, int64_t nsplit,
               int64_t n_keep, hipStream_t s) {
  if (NN == 1 || nsplit <= 64)
    launch_finish<DT, TK, NN, NCB, 1>(t, io, w, nsplit, n_keep, s);
  else if (nsplit <= 128)
    launch_finish<DT, TK, NN, NCB, 2>(t, io, w, nsplit, n_keep, s);
  else
    launch_finish<DT, TK, NN, NCB, kMaxLists>(t, io, w, nsplit, n_keep, s);
}

template <int DT, int TK, int NCB>
void finish_nn(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w, int64_t nsplit,
               int64_t n_keep, hipStream_t s) {
  if (io->n_nearest == 1)
    finish_ml<DT, TK, 1, NCB>(t, io, w, nsplit, n_keep, s);
  else
    finish_ml<DT, TK, 4, NCB>(t, io, w, nsplit, n_keep, s);
}

template <int DT, int NCB>
void finish_tk(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w, int64_t nsplit,
               int64_t n_keep, hipStream_t s) {
  if (io->router_top_k == 8)
    finish_nn<DT, 8, NCB>(t, io, w, nsplit, n_keep, s);
  else
    finish_nn<DT, 6, NCB>(t, io, w, nsplit, n_keep, s);
}

bool rows16(const void *base, int64_t ld) {
  return base == nullptr || (tm_aligned16(base) && (ld * 2) % 16 == 0);
}

}  // namespace

size_t tm_internal_decode_qn_floats(int64_t n, int32_t dim) { return (size_t)n * (size_t)(dim / 16); }
size_t tm_internal_decode_keys(int64_t n) { return (size_t)kKeyRep * (size_t)n; }
size_t tm_internal_decode_part_bytes(int64_t n, int32_t dim) {
  return (size_t)tm_cdiv(n, 16) * (size_t)(dim / 16) * kSlices * 64 * sizeof(float4);
}

bool tm_internal_decode_ok(const tm_table_layer *t, const tm_layer_io *io) {
  const int64_t n = io->n_tokens;
  const bool packed = t->ps_h == 0 && t->ps_d == 0;
  const int64_t nsplit = tm_internal_stream_nsplit(n, t->n_cent, t->dim, io->n_nearest);
  return (t->dtype == TM_DT_BF16 || t->dtype == TM_DT_F16) && packed &&
         (t->dim == 64 || t->dim == 128 || t->dim == 256) && n >= 1 && n <= 64 && nsplit > 0 &&
         (io->n_nearest == 1 || (io->n_nearest == 4 && nsplit <= 64 * kMaxLists)) &&
         (io->router_top_k == 6 || io->router_top_k == 8) && t->hidden >= 8 && t->hidden % 8 == 0 &&
         io->ld_x >= t->hidden && rows16(io->x, io->ld_x) && t->proj_vis && t->bias_vis &&
         tm_aligned16(t->proj_vis) && tm_aligned16(t->bias_vis) && (t->proj_txt == nullptr) == (t->bias_txt == nullptr) &&
         (t->proj_txt == nullptr || (tm_aligned16(t->proj_txt) && tm_aligned16(t->bias_txt))) &&
         tm_aligned16(io->q) && io->slot_out && tm_aligned16(io->slot_out) && (io->so_b * 2) % 16 == 0 &&
         (io->so_s * 2) % 16 == 0 && t->values && rows16(t->values, t->ld_v) && t->ld_v >= t->hidden &&
         rows16(io->residual, io->ld_r) && (io->residual == nullptr || io->ld_r >= t->hidden) && io->out &&
         rows16(io->out, io->ld_o) && io->ld_o >= t->hidden && t->ld_c >= t->dim && t->n_cent < (int64_t)0x7fffffff;
}

int tm_internal_decode_forward(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w,
                               const tm_route_args *ra, int64_t n_keep, void *const *ev, hipStream_t s) {
  auto record = [&](int i) -> int {
    if (ev == nullptr || ev[i] == nullptr) return TM_OK;
    const hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(ev[i]), s);
    return e == hipSuccess ? TM_OK : tm_fail(TM_EHIP, "tm_table_forward: hipEventRecord: %s", hipGetErrorString(e));
  };
  TM_REQUIRE(tm_internal_decode_ok(t, io), TM_EINVAL_SHAPE, "tm_table_forward: shape not supported by the decode plan");
  TM_REQUIRE(ra == nullptr || tm_internal_route_fusable(ra), TM_EINVAL_ARG,
             "tm_table_forward: router shape cannot be fused");
  TM_REQUIRE(w.lists && w.keys && w.qn_blk && w.part && w.cnt, TM_EINVAL_ARG,
             "tm_table_forward: decode workspace missing");
  const int64_t n = io->n_tokens;
  const int64_t nsplit = tm_internal_stream_nsplit(n, t->n_cent, t->dim, io->n_nearest);
  int st = TM_DISPATCH_DTYPE(t->dtype, DT, [&] {
    if constexpr (DT != TM_DT_F32) {
      switch (t->dim) {
        case 64: launch_split_route<DT, 64>(t, io, w, ra, s); break;
        case 128: launch_split_route<DT, 128>(t, io, w, ra, s); break;
        default: launch_split_route<DT, 256>(t, io, w, ra, s); break;
      }
      TM_LAUNCH_CHECK("tm_table_forward(project)");
    }
    return TM_OK;
  });
  if (st != TM_OK || (st = record(2)) != TM_OK) return st;
  if ((st = tm_internal_search_stream(t->dtype, io->q, n, t->dim, t->cents, t->n_cent, t->ld_c, t->c_sqnorm, t->dim,
                                      io->n_nearest, t->metric, w.lists, w.keys, kKeyRep, s)) != TM_OK)
    return st;
  if ((st = record(3)) != TM_OK || (st = record(4)) != TM_OK) return st;
  return TM_DISPATCH_DTYPE(t->dtype, DT, [&] {
    if constexpr (DT != TM_DT_F32) {
      switch (t->dim) {
        case 64: finish_tk<DT, 4>(t, io, w, nsplit, n_keep, s); break;
        case 128: finish_tk<DT, 8>(t, io, w, nsplit, n_keep, s); break;
        default: finish_tk<DT, 16>(t, io, w, nsplit, n_keep, s); break;
      }
      TM_LAUNCH_CHECK("tm_table_forward(finish)");
    }
    return TM_OK;
  });
}
