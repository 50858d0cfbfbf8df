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
//     replicas (split % kKeyRep, each replica on a 128-byte line of its
//     own), so few workgroups contend for a line.
//  3. decode_finish_kernel: one wave per (token, 512-element row chunk).  It
//     ranks the token's best distance among the n tokens' (keep rule of
//     tm_keep_select: larger distance first, ties to the lower token index),
//     takes the K smallest keys of the token's split lists (wave_min_k: a
//     set, so the same keys as merge_kernel), and combines its row chunk exactly as
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
constexpr int kStreamChunkD = 128;  // centroids per search split (tm_internal_stream_nsplit's split size)

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

  // modality of the tile's rows (which P each row multiplies)
  const uint8_t *vsrc = is_vision ? is_vision + (arow_ok ? arow : 0) : reinterpret_cast<const uint8_t *>(x);
  const uint8_t vis_byte = *vsrc;
  // the reducer's bias values, loaded now so their latency hides behind the slice
  const int col = cb * 16 + (lane & 15);
  const float bias_v = Elem<DT>::to_f(bv[col]);
  const float bias_t = Elem<DT>::to_f(bt[col]);

  tm_f32x4 fin = tm_f32x4{0.f, 0.f, 0.f, 0.f};
  // whole-k-step slices: x and both modalities' P loaded at once, so no P
  // load waits for the modality byte
  constexpr int KA = KPW > 0 ? KPW : 1;
  uint4 xa[KA], pva[KA], pta[KA];
  if constexpr (KPW > 0) {
    const uint4 *pvf = reinterpret_cast<const uint4 *>(pv) + lane;
    const uint4 *ptf = reinterpret_cast<const uint4 *>(pt) + lane;
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      xa[j] = *reinterpret_cast<const uint4 *>(xrow + (ks_begin + j) * 32 + kq);
      pva[j] = pvf[((int64_t)(ks_begin + j) * NCB + cb) * 64];
      pta[j] = ptf[((int64_t)(ks_begin + j) * NCB + cb) * 64];
    }
  }
  const int amod = !arow_ok ? 2 : ((is_vision == nullptr || vis_byte) ? 0 : 1);
  const uint32_t vis_bits = (uint32_t)(__ballot(amod == 0) & 0xFFFFull);
  const uint32_t txt_bits = (uint32_t)(__ballot(amod == 1) & 0xFFFFull);
  auto run_pass = [&](const T *P, uint32_t rows_of_pass) {
    const uint4 *pf = reinterpret_cast<const uint4 *>(P) + lane;
    tm_f32x4 acc = tm_f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (KPW > 0) {
      const bool is_v = P == pv;  // uniform
#pragma unroll
      for (int j = 0; j < KPW; ++j) acc = tm_mfma16x16x32<DT>(xa[j], is_v ? pva[j] : pta[j], acc);
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
    for (int r = sl; r < kKeyRep; r += S) keys[(int64_t)r * tm_key_stride(n) + arow] = ~0ull;

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

// Wave minimum of a 64-bit value, in every lane: DPP exchanges inside each
// 16-lane row (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror: every lane then holds its row's minimum), then the four row
// minima read into scalars.  Every lane of the wave must call it.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_min64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  return o < v ? o : v;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  v = dpp_min64<0xB1>(v);
  v = dpp_min64<0x4E>(v);
  v = dpp_min64<0x141>(v);
  v = dpp_min64<0x140>(v);
  uint64_t m = ~0ull;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t x = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * r) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 16 * r) << 32);
    m = x < m ? x : m;
  }
  return m;
}

// The K smallest keys of the wave, ascending, in every lane, from each lane's
// ascending K-list: K rounds of a wave minimum over the lists' heads, the lane
// that holds it popping its head.  Keys are unique (the centroid index is the
// low word), so one lane pops; empty entries (~0) pop in every lane holding
// one and stay ~0.  The same K keys as a merge of all the lists.
template <int K>
__device__ __forceinline__ void wave_min_k(uint64_t (&l)[K]) {
  uint64_t top[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const uint64_t m = wave_min_u64(l[0]);
    top[j] = m;
    if (j + 1 < K) {
      const bool pop = l[0] == m;
#pragma unroll
      for (int i = 0; i + 1 < K; ++i) l[i] = pop ? l[i + 1] : l[i];
      l[K - 1] = pop ? ~0ull : l[K - 1];
    }
  }
#pragma unroll
  for (int j = 0; j < K; ++j) l[j] = top[j];
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
  for (int r = 0; r < kKeyRep; ++r) kr[r] = keys[(int64_t)r * tm_key_stride(n) + jl];
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
    tm_load8<DT>(residual + (int64_t)b * ld_r + hl, acc);
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
    wave_min_k<K>(lst);
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

// ---------------------------------------------------------------------------
// One-launch decode plan (decode_fused_kernel): the three launches above as
// three phases of one launch of kFusedWGs four-wave workgroups.  A phase
// whose inputs come from other workgroups waits on a grid-wide flag.
//   A  projection (project_split_kernel's work): one row tile: (tile, column
//      block) group g runs on workgroup G - 1 - g, two slices per wave, added
//      through LDS; more rows: one slice per wave, spread over workgroups, the
//      group's last wave adds the partials.  The wave that finishes a group
//      writes q and the block's |q|^2 and raises the group's flag; a
//      workgroup goes on once one wave saw every group's flag.
//   B  workgroup s < nsplit searches split s (search_stream_kernel's work) and
//      publishes its lists and best keys; every workgroup then counts itself
//      on one of kSubCnt sub-counters, the last arrival of each raises that
//      sub-group's done flag, and a workgroup goes on once one wave saw every
//      sub-group's flag.
//   C  wave 3 - t / G of workgroup t % G finishes task t = (token, row
//      chunk) (decode_finish_kernel's work, the same arithmetic); counting
//      the waves from the other end keeps the routing these waves do off the
//      projection waves.
// What does not depend on another workgroup is loaded before the first wait:
// the split's centroid rows and norms, the task's residual chunk and slot
// rows, and the weights when the router ran in its own launch.  Otherwise each
// finishing wave routes its own token (tm_route_compute, the router kernel's
// routine, so the same bits) while the projection runs.
//
// Flags carry a generation: every wave reads gen at the start, a flag raised
// in this call holds gen + 1 and workgroup 0 advances gen once it saw every
// sub-group's done flag (every workgroup has read gen by then), so no flag is
// ever cleared; each counter is cleared by the arrival that
// completes it.  Data handed between workgroups moves through agent-scope
// atomic loads and stores, which the hardware performs at one point of
// coherence per address for every XCD (the loads bypass the non-coherent
// per-XCD L2), and the counts through agent-scope atomics.  A producer's
// s_waitcnt vmcnt(0) (gfx9 counts stores and returnless atomics in vmcnt)
// returns only after its stores are acknowledged, and only then does it
// count; a consumer loads only after it saw the flag.  Agent-scope
// release/acquire fences would write back and invalidate whole L2s
// instead (measured at microseconds per launch).  Every wait polls with a
// bound of kSpinTicks ticks of the 100 MHz constant clock: a wait that runs
// out counts on the err word, and that workgroup's output chunks are
// written as NaN, so a launch whose workgroups could not all be resident at
// once (another kernel filling the device) ends with flagged outputs instead
// of hanging.
// ---------------------------------------------------------------------------
constexpr int kFusedWGs = 128;
constexpr int kSubCnt = 8;     // sub-counters of the search arrival
constexpr int kSubRep = 2;     // copies of each sub-group's done flag (the pollers spread over them)
constexpr int kLine = 32;      // words per 128-byte line: each hot word on a line of its own
constexpr uint64_t kSpinTicks = 2000000;  // 20 ms
static_assert(kFusedWGs % kSubCnt == 0, "whole sub-counter groups");
static_assert(kSubCnt <= 64, "one polling lane per sub-group");
// word offsets in the layer workspace's sync region (words 0 .. 63 belong to
// the other plans' counters)
constexpr int kWGen = 64;
constexpr int kWSsub = kWGen + 2 * kLine;                  // (one spare line after the generation)
constexpr int kWDone = kWSsub + kSubCnt * kLine;           // the sub-groups' done flags, one line each
constexpr int kWErr = kWDone + kSubCnt * kSubRep * kLine;
constexpr int kMaxGroups = 64 / 16 * 128 / 16;  // (64 rows / 16) x (d 128 / 16)
constexpr int kWGrp = kWErr + kLine;                   // the projection groups' counters, one line each
constexpr int kWFlagA = kWGrp + kMaxGroups * kLine;    // the projection groups' q-ready flags, one line each
static_assert(kWFlagA + kMaxGroups * kLine <= 3072, "the ranked top-1 plan's counters follow");
static_assert(kWErr * 4 == TM_LAYER_SYNC_ERR_BYTE, "documented err word");

struct FusedArgs {
  int64_t n, nsplit, n_cent, ld_c, n_keep, ld_x, ld_logits, so_b, so_s, ld_v, ld_r, ld_o;
  int hidden, n_chunks, l2, routed, n_experts, has_res;
  const void *x;
  const uint8_t *is_vision;
  const void *pv, *bv, *pt, *bt;
  void *q;
  float *qn_blk;
  float4 *part;
  const void *cents;
  const float *c_sqnorm;
  uint64_t *lists, *keys;
  const float *logits;
  float *w;      // router outputs (routed) or the router weights (input)
  int64_t *ids;  // router outputs (routed)
  const void *slot_out, *values, *residual;
  void *out;
  float *out_dist;
  int64_t *out_idx;
  float *out_qn;
  uint8_t *out_keep;
  uint32_t *sync;
};

__device__ __forceinline__ uint64_t coh_ld(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_st(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_st32(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t coh_add(uint32_t *p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Phase A of decode_fused_kernel: project_split_kernel's work (hidden ==
// 32 * kSlices * KPW) in one of two layouts, chosen by the batch:
//  - one row tile (n <= 16): (tile, column block) group g runs on one
//    workgroup, wave w taking slices 2w and 2w + 1; the group's kSlices fp32
//    partials are added in slice order through LDS and wave 0 finishes q.
//  - more rows: one slice per wave, the slices of a group spread over
//    workgroups; each publishes its partial by coherent stores and counts it
//    on the group, and the group's last wave adds the partials in slice order
//    and finishes q.  (A whole group on one workgroup moves 160 KB of operands
//    through one CU at 16 real rows, which costs more than the hand-off.)
// Both add the same partials in the same order: the same q, bit for bit.
// fused_project_loads issues every operand load of the wave at once -- x, the
// first modality's P (text with a modality mask, vision without; no load waits
// for the modality byte) and the biases -- and fused_project_task multiplies
// (loading the other modality's P only when the tile holds a row of it),
// reduces, writes q and the block's |q|^2 by coherent stores and raises the
// group's q-ready flag.
template <int DT, int KPW, bool OT>
struct ProjOps {
  static constexpr int NK = OT ? 2 * KPW : KPW;  // k-steps per wave: two slices in the one-tile layout
  uint4 x[NK], p1[NK];  // p1: the first modality's P (text with a modality mask, else vision)
  typename Elem<DT>::T bias_v, bias_t;  // raw: converted where used
  uint8_t vis;
};

// k-steps ks0 .. ks0 + NK - 1 of group g
template <int DT, int DIM, int KPW, bool OT>
__device__ __forceinline__ void fused_project_loads(const FusedArgs &a, int64_t g, int ks0, int lane,
                                                    ProjOps<DT, KPW, OT> &o) {
  constexpr int NK = ProjOps<DT, KPW, OT>::NK;
  using T = typename Elem<DT>::T;
  constexpr int NCB = DIM / 16;
  const int64_t n = a.n;
  const int cb = (int)(g % NCB);
  const int64_t arow = (g / NCB) * 16 + (lane & 15);
  const bool arow_ok = arow < n;
  const T *x = static_cast<const T *>(a.x);
  const T *xrow = x + (arow_ok ? arow : 0) * a.ld_x;
  const int kq = 8 * (lane >> 4);
  const uint8_t *vsrc = a.is_vision ? a.is_vision + (arow_ok ? arow : 0) : reinterpret_cast<const uint8_t *>(x);
  o.vis = *vsrc;
  const int col = cb * 16 + (lane & 15);
  o.bias_v = static_cast<const T *>(a.bv)[col];
  o.bias_t = static_cast<const T *>(a.bt)[col];
  // the first modality's P only (text when there is a modality mask: decode
  // batches are text; vision without one); fused_project_task loads the
  // other when its tile holds a row of it
  const uint4 *p1f = reinterpret_cast<const uint4 *>(a.is_vision ? a.pt : a.pv) + lane;
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    o.x[j] = *reinterpret_cast<const uint4 *>(xrow + (ks0 + j) * 32 + kq);
    o.p1[j] = p1f[((int64_t)(ks0 + j) * NCB + cb) * 64];
  }
}

// OT: the one-tile layout (every wave of the workgroup calls it: it holds a
// barrier), `sw` = the wave; else slice `sw` of the spread layout.
template <int DT, int DIM, int KPW, bool OT>
__device__ __forceinline__ void fused_project_task(const FusedArgs &a, int64_t g, int sw, uint32_t g0v, int lane,
                                                   const ProjOps<DT, KPW, OT> &o, tm_f32x4 (*red)[64]) {
  constexpr int NK = ProjOps<DT, KPW, OT>::NK;
  constexpr bool two = OT;
  using T = typename Elem<DT>::T;
  constexpr int NCB = DIM / 16;
  constexpr int S = kSlices;
  static_assert(S == 8, "4 waves x 2 slices");
  const int64_t n = a.n;
  const int cb = (int)(g % NCB);
  const int64_t row0 = (g / NCB) * 16;
  const int64_t arow = row0 + (lane & 15);
  const bool arow_ok = arow < n;
  const int sl0 = two ? 2 * sw : sw;  // first slice of this wave
  const int amod = !arow_ok ? 2 : ((a.is_vision == nullptr || o.vis) ? 0 : 1);
  const uint32_t vis_bits = (uint32_t)(__ballot(amod == 0) & 0xFFFFull);
  const uint32_t txt_bits = (uint32_t)(__ballot(amod == 1) & 0xFFFFull);
  tm_f32x4 fin[2];
  fin[0] = tm_f32x4{0.f, 0.f, 0.f, 0.f};
  fin[1] = tm_f32x4{0.f, 0.f, 0.f, 0.f};
  auto run_pass = [&](const uint4 (&br)[NK], uint32_t rows_of_pass) {
#pragma unroll
    for (int h = 0; h < NK / KPW; ++h) {  // one fp32 partial per slice, as project_split_kernel's waves
      tm_f32x4 acc = tm_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KPW; ++j) acc = tm_mfma16x16x32<DT>(o.x[h * KPW + j], br[h * KPW + j], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if ((rows_of_pass >> (4 * (lane >> 4) + i)) & 1u) fin[h][i] = acc[i];
    }
  };
  // uniform branches: the first modality's rows from the loaded P; rows of
  // the other (vision rows of a masked batch) after a load of its P
  const uint32_t first_bits = a.is_vision ? txt_bits : vis_bits;
  const uint32_t second_bits = a.is_vision ? vis_bits : 0u;
  if (first_bits) run_pass(o.p1, first_bits);
  if (second_bits) {
    const int ks0 = sl0 * KPW;
    const uint4 *pvf = reinterpret_cast<const uint4 *>(a.pv) + lane;
    uint4 p2[NK];
#pragma unroll
    for (int j = 0; j < NK; ++j) p2[j] = pvf[((int64_t)(ks0 + j) * NCB + cb) * 64];
    run_pass(p2, second_bits);
  }

  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (two) {
    red[sl0][lane] = fin[0];
    red[sl0 + 1][lane] = fin[1];
    __syncthreads();
    if (sw != 0) return;
    // the tile's best keys (every replica) reset for phase B, acknowledged
    // with q before the group's flag
    if (cb == 0) {
#pragma unroll
      for (int e = lane; e < 16 * kKeyRep; e += 64) {
        const int64_t r = row0 + (e & 15);
        if (r < n) coh_st(a.keys + (int64_t)(e >> 4) * tm_key_stride(n) + r, ~0ull);
      }
    }
    // wave 0: the S partials added in slice order
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2) {
      const tm_f32x4 p = red[s2][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += p[i];
    }
  } else {
    // reset the tile's best keys (replicas s, s + S, ... for slice s) for
    // phase B, acknowledged with the partial before the count
    if (cb == 0 && lane < 16 && arow_ok)
      for (int r = sl0; r < kKeyRep; r += S) coh_st(a.keys + (int64_t)r * tm_key_stride(n) + arow, ~0ull);
    // publish this slice's partial, count it on the group
    uint64_t *pp = reinterpret_cast<uint64_t *>(a.part) + ((g * S + sl0) * 64 + lane) * 2;
    coh_st(pp, ((uint64_t)__float_as_uint(fin[0][1]) << 32) | __float_as_uint(fin[0][0]));
    coh_st(pp + 1, ((uint64_t)__float_as_uint(fin[0][3]) << 32) | __float_as_uint(fin[0][2]));
    __builtin_amdgcn_s_waitcnt(0);
    uint32_t ticket = 0;
    if (lane == 0) ticket = coh_add(a.sync + kWGrp + g * kLine);
    ticket = (uint32_t)__builtin_amdgcn_readfirstlane((int)ticket);
    if (ticket != S - 1) return;  // uniform: not the group's last slice
    if (lane == 0) coh_st32(a.sync + kWGrp + g * kLine, 0u);
    // the group's last wave: the S partials added in slice order
    uint64_t pv2[S][2];
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2) {
      const uint64_t *src = reinterpret_cast<const uint64_t *>(a.part) + ((g * S + s2) * 64 + lane) * 2;
      pv2[s2][0] = coh_ld(src);
      pv2[s2][1] = coh_ld(src + 1);
    }
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2) {
      v[0] += __uint_as_float((uint32_t)pv2[s2][0]);
      v[1] += __uint_as_float((uint32_t)(pv2[s2][0] >> 32));
      v[2] += __uint_as_float((uint32_t)pv2[s2][1]);
      v[3] += __uint_as_float((uint32_t)(pv2[s2][1] >> 32));
    }
  }
  // bias, one rounding
  const float bias_v = Elem<DT>::to_f(o.bias_v), bias_t = Elem<DT>::to_f(o.bias_t);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * (lane >> 4) + i;
    const bool vis = (vis_bits >> r) & 1u;
    v[i] = tm_round<DT>(v[i] + (vis ? bias_v : bias_t));
    float sq = v[i] * v[i];
    sq += __shfl_xor(sq, 1, 64);
    sq += __shfl_xor(sq, 2, 64);
    sq += __shfl_xor(sq, 4, 64);
    sq += __shfl_xor(sq, 8, 64);
    const int64_t gr = row0 + r;
    if (gr < n && (lane & 15) == 0) coh_st32(reinterpret_cast<uint32_t *>(a.qn_blk + gr * NCB + cb), __float_as_uint(sq));
  }
  // q in 8-byte pieces: lane l writes row 4 (l / 16) + l % 4, columns 4 ((l % 16) / 4) .. + 3 of the block
  uint64_t piece = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float y = __shfl(v[i], (lane & ~3) + t, 64);
      if (i == (lane & 3)) piece |= (uint64_t)__builtin_bit_cast(uint16_t, Elem<DT>::from_f(y)) << (16 * t);
    }
  const int64_t qrow = row0 + 4 * (lane >> 4) + (lane & 3);
  if (qrow < n)
    coh_st(reinterpret_cast<uint64_t *>(static_cast<T *>(a.q) + qrow * DIM + cb * 16 + 4 * ((lane & 15) >> 2)), piece);
  __builtin_amdgcn_s_waitcnt(0);  // q and |q|^2 of the block acknowledged before its flag
  const uint32_t gen = (uint32_t)__builtin_amdgcn_readfirstlane((int)g0v);
  if (lane == 0) coh_st32(a.sync + kWFlagA + g * kLine, gen + 1);
}

template <int DT, int DIM, int KPW, int K, int TK, bool OT>
__global__ __launch_bounds__(256) void decode_fused_kernel(FusedArgs a) {
  using T = typename Elem<DT>::T;
  constexpr int KS = DIM / 16;
  constexpr int NCB = DIM / 16;
  constexpr int S = kSlices;
  constexpr int NN = K;
  __shared__ uint64_t merge_buf[4][K][64];
  __shared__ uint4 q_lds[64 * DIM / 8];
  __shared__ tm_f32x4 red[kSlices][64];  // the projection group's slice partials
  __shared__ uint32_t s_ok;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wg = (int)blockIdx.x;
  const int G = (int)gridDim.x;
  const int64_t n = a.n;
  uint32_t *const sync = a.sync;

  // Loads in the order they are needed (vmcnt retires them in order): the
  // projection task's operands, the split's centroid block and norms, the
  // finishing task's rows, then this call's generation.  Every one is
  // unconditional (clamped or redirected addresses): a load under a branch
  // makes the compiler wait for it, and for all loads before it, right there.
  // Projection, one row tile (n <= 16): group ga = G - 1 - wg (16-row tile,
  // 16-column block) on the last workgroups (the finishing tasks, and the
  // routing they do, start at workgroup 0), two slices per wave.  More rows:
  // task of (wave, workgroup): position L = wave * G + wg holds group
  // 8 (L / 64) + L % 8, slice (L / 8) % 8, so a group's S slices run on
  // workgroups congruent mod 8 (one XCD under the dispatcher's round robin).
  static_assert(S == 8 && NCB == 8, "64 slices per row tile");
  constexpr bool one_tile = OT;  // the launch picks it: n <= 16
  const int64_t la = (int64_t)wave * G + wg;
  const int64_t ta = (8 * (la / 64) + la % 8) * S + (la / 8) % 8;
  const int64_t ga = one_tile ? (int64_t)(G - 1 - wg) : ta / S;
  const int sw = one_tile ? wave : (int)(ta % S);
  const bool has_a = one_tile ? ga < NCB : ta < ((n + 15) / 16) * NCB * S;  // uniform per wave
  ProjOps<DT, KPW, OT> po;
  if (has_a) fused_project_loads<DT, DIM, KPW, OT>(a, ga, (one_tile ? 2 * sw : sw) * KPW, lane, po);

  const bool has_split = wg < a.nsplit;  // uniform
  const int64_t c_begin = (int64_t)wg * kStreamChunkD;
  const int64_t c_end = (c_begin + kStreamChunkD < a.n_cent) ? c_begin + kStreamChunkD : a.n_cent;
  const int64_t c0 = c_begin + 32 * wave;
  const T *cents = static_cast<const T *>(a.cents);
  uint4 af[KS];
  {
    const int64_t cr = c0 + (lane & 31);
    const int64_t crr = cr < a.n_cent ? cr : a.n_cent - 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      af[ks] = *reinterpret_cast<const uint4 *>(cents + crr * a.ld_c + ks * 16 + 8 * (lane >> 5));
  }
  float pen[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t cm = c0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    pen[i] = a.c_sqnorm[cm < a.n_cent ? cm : a.n_cent - 1];  // a readable stand-in for the dot metric
  }

  const int ntc = (int)n * a.n_chunks;
  const int tc = (3 - wave) * G + wg;  // from the last wave down: the first waves take the projection
  const bool has_c = tc < ntc;  // uniform per wave
  const int b = has_c ? tc / a.n_chunks : 0;
  const int ch = has_c ? tc % a.n_chunks : 0;
  const int h0 = ch * kChunk + lane * 8;
  const int hl = h0 < a.hidden ? h0 : a.hidden - 8;
  // the finishing task's rows, kept raw (converting them here would make the
  // compiler wait for them here)
  tm_u32x4 rrow, srow[TK];
  float wv[TK];
  if (has_c) {
    rrow = *reinterpret_cast<const tm_u32x4 *>(static_cast<const T *>(a.residual) + (int64_t)b * a.ld_r + hl);
    const T *src = static_cast<const T *>(a.slot_out) + (int64_t)b * a.so_b + hl;
#pragma unroll
    for (int s = 0; s < TK; ++s)
      srow[s] = __builtin_nontemporal_load(reinterpret_cast<const tm_u32x4 *>(src + (int64_t)s * a.so_s));
#pragma unroll
    for (int s = 0; s < TK; ++s) wv[s] = a.w[(int64_t)b * TK + s];  // replaced by the routing below when routed
  }

  // this call's generation: moved to a scalar only where it is used, so no
  // wait for it (and for every load before it) lands here
  uint32_t g0v = 0;
  if (lane == 0) g0v = __hip_atomic_load(sync + kWGen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  auto g0 = [&] { return (uint32_t)__builtin_amdgcn_readfirstlane((int)g0v); };

  // ---- phase A: projection task ----
  if (has_a) fused_project_task<DT, DIM, KPW, OT>(a, ga, sw, g0v, lane, po, red);
  if (!a.l2) {
#pragma unroll
    for (int i = 0; i < 16; ++i) pen[i] = 0.f;
  }
  // the finishing wave routes its token
  if (a.routed && has_c) {
    float kw[8];
    int ki[8];
    float wsum;
    if (a.n_experts == 64)
      tm_route_compute<8, 8>(a.logits, n, a.ld_logits, TK, b, lane & 7, kw, ki, wsum);
    else
      tm_route_compute<16, 8>(a.logits, n, a.ld_logits, TK, b, lane & 7, kw, ki, wsum);
#pragma unroll
    for (int s = 0; s < TK; ++s) wv[s] = kw[s];
    if (ch == 0 && lane == 0) {
#pragma unroll
      for (int s = 0; s < TK; ++s) {
        a.w[(int64_t)b * TK + s] = kw[s];
        a.ids[(int64_t)b * TK + s] = ki[s];
      }
    }
  }
  // A kept token's row chunk: the residual plus its recomputed slot rows
  // weighted by the renormalised router weights.
  T *const dst = static_cast<T *>(a.out) + (int64_t)b * a.ld_o + hl;
  auto kept_row = [&](float (&acc)[8]) {
    const T *e = reinterpret_cast<const T *>(&rrow);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = a.has_res ? Elem<DT>::to_f(e[i]) : 0.f;
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s) sum += wv[s];
    const bool any = sum > 0.f;
    float coef[TK];
#pragma unroll
    for (int s = 0; s < TK; ++s) coef[s] = wv[s] / sum;
    if (any) {
#pragma unroll
      for (int s = 0; s < TK; ++s) {
        const T *es = reinterpret_cast<const T *>(&srow[s]);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(coef[s], Elem<DT>::to_f(es[i]), acc[i]);
      }
    }
  };
  // Every token kept (n_keep >= n, as for one token at the reference keep
  // rates): the rows need nothing from the search, so the finishing waves
  // store them now; after the waits only chunk 0 of each token writes the
  // search outputs (and a wait that ran out rewrites the rows as NaN).
  const bool all_kept = a.n_keep >= n;  // uniform
  if (has_c && all_kept) {
    float acc[8];
    kept_row(acc);
    if (h0 < a.hidden) tm_store8_nt<DT>(dst, acc);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t cm = c0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    pen[i] = cm < c_end ? pen[i] : __builtin_huge_valf();
  }

  // ---- wait for q: wave 0's lane g polls group g's flag ----
  __syncthreads();
  if (wave == 0) {
    const int ngroups = (int)((n + 15) / 16) * NCB;
    const uint32_t want = g0() + 1;
    const uint32_t *f = sync + kWFlagA + (lane < ngroups ? lane : 0) * kLine;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    bool ok = true;
    while (__ballot(lane < ngroups && __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != want) != 0) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) { ok = false; break; }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      if (!ok) coh_add(sync + kWErr);
      s_ok = ok ? 1u : 0u;
    }
  }
  __syncthreads();
  bool poison = s_ok == 0u;

  // ---- phase B: search split wg ----
  if (has_split) {  // uniform
    const bool two = n > 32;
    const T *q = static_cast<const T *>(a.q);
    // q (32 or 64 rows) comes into LDS once per workgroup, 16-byte chunk j
    // of row r at r * CH + (j ^ (r % CH)) (conflict-free fragment reads)
    constexpr int CH = DIM / 8;
    const int rows = two ? 64 : 32;
    // every chunk's loads are issued before the first is written (a loop that
    // loads and writes one chunk per iteration waits a round trip each time);
    // rows past n read row n - 1
    constexpr int kQIt = 64 * CH / 256;
    uint64_t qlo[kQIt], qhi[kQIt];
#pragma unroll
    for (int it = 0; it < kQIt; ++it) {
      const int c = tid + it * 256;
      const int r = c / CH, j = c % CH;
      const int64_t rr = r < n ? r : n - 1;
      const uint64_t *src = reinterpret_cast<const uint64_t *>(q + rr * DIM + j * 8);
      qlo[it] = coh_ld(src);
      qhi[it] = coh_ld(src + 1);
    }
#pragma unroll
    for (int it = 0; it < kQIt; ++it) {
      const int c = tid + it * 256;
      const int r = c / CH, j = c % CH;
      if (c < rows * CH)
        q_lds[r * CH + (j ^ (r % CH))] = make_uint4((uint32_t)qlo[it], (uint32_t)(qlo[it] >> 32), (uint32_t)qhi[it],
                                                    (uint32_t)(qhi[it] >> 32));
    }
    __syncthreads();
    auto q_slab = [&](int sl, uint4 (&qf)[KS]) {
      const int r = sl * 32 + (lane & 31);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[ks] = q_lds[r * CH + ((2 * ks + (lane >> 5)) ^ (r % CH))];
    };
    tm_f32x16 sacc[2];
    sacc[0] = tm_f32x16{};
    sacc[1] = tm_f32x16{};
    {
      uint4 qf[KS];
      q_slab(0, qf);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sacc[0] = tm_mfma32x32x16<DT>(af[ks], qf[ks], sacc[0]);
    }
    if (two) {  // uniform: rows 32 .. 63
      uint4 qf[KS];
      q_slab(1, qf);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sacc[1] = tm_mfma32x32x16<DT>(af[ks], qf[ks], sacc[1]);
    }
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      if (sl == 1 && !two) break;  // uniform
      uint64_t l[K];
#pragma unroll
      for (int j = 0; j < K; ++j) l[j] = ~0ull;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int c = (int)c0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        const float dp = a.l2 ? fmaf(-2.f, sacc[sl][i], pen[i]) : (pen[i] - sacc[sl][i]);
        uint64_t xk = dp == __builtin_huge_valf() ? ~0ull : (((uint64_t)tm_orderable(dp) << 32) | (uint32_t)c);
#pragma unroll
        for (int j = 0; j < K; ++j) {  // compare-swap chain (no branch)
          const uint64_t lo = l[j] < xk ? l[j] : xk;
          xk = l[j] < xk ? xk : l[j];
          l[j] = lo;
        }
      }
      uint64_t o[K];
#pragma unroll
      for (int j = 0; j < K; ++j) o[j] = __shfl_xor(l[j], 32, 64);
      merge_min_k<K>(l, o);
      if (lane < 32) {
#pragma unroll
        for (int j = 0; j < K; ++j) merge_buf[wave][j][sl * 32 + lane] = l[j];
      }
    }
    __syncthreads();
    if (tid < (two ? 64 : 32)) {
      const int r = tid;
      uint64_t l[K];
#pragma unroll
      for (int j = 0; j < K; ++j) l[j] = merge_buf[0][j][r];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        uint64_t o[K];
#pragma unroll
        for (int j = 0; j < K; ++j) o[j] = merge_buf[w][j][r];
        merge_min_k<K>(l, o);
      }
      if (r < n) {
        if constexpr (K > 1) {
          uint64_t *dst = a.lists + ((int64_t)wg * n + r) * K;
#pragma unroll
          for (int j = 0; j < K; ++j) coh_st(dst + j, l[j]);
        }
        atomicMin(reinterpret_cast<unsigned long long *>(a.keys + (int64_t)(wg % kKeyRep) * tm_key_stride(n) + r),
                  (unsigned long long)l[0]);
      }
    }
  }
  // ---- arrival, then wait for every split ----
  __builtin_amdgcn_s_waitcnt(0);  // this thread's list stores and key minima performed
  __syncthreads();
  if (tid == 0) {
    const uint32_t t = coh_add(sync + kWSsub + (wg % kSubCnt) * kLine);
    if (t == (uint32_t)(G / kSubCnt - 1)) {  // the sub-group's last arrival raises its done flags
      coh_st32(sync + kWSsub + (wg % kSubCnt) * kLine, 0u);
      for (int r = 0; r < kSubRep; ++r) coh_st32(sync + kWDone + ((wg % kSubCnt) * kSubRep + r) * kLine, g0() + 1);
    }
  }
  if (wave == 0) {  // lane i polls sub-group i's done flag (replica wg % kSubRep)
    const uint32_t *f = sync + kWDone + ((lane % kSubCnt) * kSubRep + wg % kSubRep) * kLine;
    const uint32_t want = g0() + 1;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    bool ok = true;
    for (;;) {
      uint32_t v = want;
      if (lane < kSubCnt) v = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__ballot(v != want) == 0) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) { ok = false; break; }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      if (!ok) coh_add(sync + kWErr);
      // workgroup 0 advances the generation (the next call's flags want
      // gen + 2; every wave of this call read gen at its start, and the next
      // launch starts after this one ends), also after a wait that ran out,
      // so flags this call raised are never taken for the next call's
      if (wg == 0) coh_st32(sync + kWGen, g0() + 1);
      s_ok = ok ? 1u : 0u;
    }
  }
  __syncthreads();
  poison = poison || s_ok == 0u;
  if (!has_c) return;  // uniform per wave
  if (all_kept && ch != 0) {  // the row chunk is stored
    if (poison && h0 < a.hidden) {
      float nan8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) nan8[i] = __builtin_nanf("");
      tm_store8_nt<DT>(dst, nan8);
    }
    return;
  }

  // ---- phase C: token b, row chunk ch ----
  const int jl = lane < n ? lane : (int)n - 1;
  uint64_t kr[kKeyRep];
#pragma unroll
  for (int r = 0; r < kKeyRep; ++r) kr[r] = coh_ld(a.keys + (int64_t)r * tm_key_stride(n) + jl);
  float qb[NCB];
#pragma unroll
  for (int c = 0; c < NCB; c += 2) {
    const uint64_t u = coh_ld(reinterpret_cast<const uint64_t *>(a.qn_blk + (int64_t)jl * NCB + c));
    qb[c] = __uint_as_float((uint32_t)u);
    qb[c + 1] = __uint_as_float((uint32_t)(u >> 32));
  }
  uint64_t lst[K];
#pragma unroll
  for (int j = 0; j < K; ++j) lst[j] = ~0ull;
  if constexpr (K > 1) {
    // both halves of the split lists are loaded before either is merged
    // (unconditional loads of clamped addresses, masked afterwards)
    uint64_t o[2][K];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int64_t s = lane + 64 * m;
      const uint64_t *src = a.lists + ((s < a.nsplit ? s : a.nsplit - 1) * n + b) * K;
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const uint64_t v = coh_ld(src + j);
        o[m][j] = s < a.nsplit ? v : ~0ull;
      }
    }
    merge_min_k<K>(lst, o[0]);
    if (a.nsplit > 64) merge_min_k<K>(lst, o[1]);  // uniform
  }

  // keep rank of token b among the n tokens' best distances
  uint64_t kj = kr[0];
#pragma unroll
  for (int r = 1; r < kKeyRep; ++r) kj = kr[r] < kj ? kr[r] : kj;
  const float qn_j = qn_tree<NCB>(qb);
  int64_t ix_j;
  const float d_j = tm_key_to_dist(kj, qn_j, a.l2 != 0, ix_j);
  const uint32_t key_j = tm_orderable(d_j);
  const uint32_t key_b = (uint32_t)__builtin_amdgcn_readlane((int)key_j, b);
  const float qn_b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qn_j), b));
  const bool ahead = lane < n && (key_j > key_b || (key_j == key_b && lane < b));
  const int rank = __popcll(__ballot(ahead));
  const int64_t n_keep = a.n_keep;
  const bool kept = n_keep >= n ? true : (n_keep <= 0 ? false : rank < n_keep);

  if constexpr (K > 1) {
    wave_min_k<K>(lst);
  } else {
    lst[0] = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)kj, b) |
             ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(kj >> 32), b) << 32);
  }
  float dn[NN];
  int64_t cn[NN];
#pragma unroll
  for (int j = 0; j < NN; ++j) dn[j] = tm_key_to_dist(lst[j], qn_b, a.l2 != 0, cn[j]);

  if (ch == 0 && lane == 0) {
#pragma unroll
    for (int j = 0; j < NN; ++j) {
      a.out_dist[(int64_t)b * NN + j] = dn[j];
      a.out_idx[(int64_t)b * NN + j] = cn[j];
    }
    a.out_keep[b] = kept ? 1 : 0;
    a.out_qn[b] = qn_b;
  }

  if (all_kept && !poison) return;  // the row chunk is stored
  float acc[8];
  if (kept) {  // uniform
    kept_row(acc);
  } else {
    {
      const T *e = reinterpret_cast<const T *>(&rrow);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = a.has_res ? Elem<DT>::to_f(e[i]) : 0.f;
    }
    const T *values = static_cast<const T *>(a.values);
    const T *src[NN];
    float coef[NN];
    bool okc[NN];
    float inv_sum = 0.f;
#pragma unroll
    for (int j = 0; j < NN; ++j) {
      okc[j] = cn[j] >= 0 && cn[j] < a.n_cent;
      src[j] = values + (okc[j] ? cn[j] : 0) * a.ld_v + hl;
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
  if (poison) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __builtin_nanf("");
  }
  if (h0 < a.hidden) tm_store8_nt<DT>(dst, acc);
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

template <int DT, int KPW, int K, int TK>
void launch_fused(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w, const tm_route_args *ra,
                  int64_t nsplit, int64_t n_keep, hipStream_t s) {
  FusedArgs a{};
  a.n = io->n_tokens;
  a.nsplit = nsplit;
  a.n_cent = t->n_cent;
  a.ld_c = t->ld_c;
  a.n_keep = n_keep;
  a.ld_x = io->ld_x;
  a.hidden = t->hidden;
  a.n_chunks = (int)tm_cdiv(t->hidden, kChunk);
  a.l2 = t->metric == TM_METRIC_L2 ? 1 : 0;
  a.routed = ra != nullptr ? 1 : 0;
  a.n_experts = ra != nullptr ? ra->n_experts : 0;
  a.logits = ra != nullptr ? ra->logits : nullptr;
  a.ld_logits = ra != nullptr ? ra->ld : 0;
  a.x = io->x;
  a.is_vision = io->is_vision;
  a.pv = t->proj_vis;
  a.bv = t->bias_vis;
  a.pt = t->proj_txt ? t->proj_txt : t->proj_vis;
  a.bt = t->proj_txt ? t->bias_txt : t->bias_vis;
  a.q = io->q;
  a.qn_blk = w.qn_blk;
  a.part = reinterpret_cast<float4 *>(w.part);
  a.cents = t->cents;
  // stand-ins keep every prologue load unconditional: the norms (dot
  // metric) read the centroid bytes, the residual (none) reads slot rows
  a.c_sqnorm = t->c_sqnorm ? t->c_sqnorm : static_cast<const float *>(t->cents);
  a.lists = w.lists;
  a.keys = w.keys;
  a.w = io->weights;
  a.ids = io->expert_ids;
  a.slot_out = io->slot_out;
  a.so_b = io->so_b;
  a.so_s = io->so_s;
  a.values = t->values;
  a.ld_v = t->ld_v;
  a.has_res = io->residual != nullptr ? 1 : 0;
  a.residual = io->residual ? io->residual : io->slot_out;
  a.ld_r = io->residual ? io->ld_r : 0;
  a.out = io->out;
  a.ld_o = io->ld_o;
  a.out_dist = io->dist;
  a.out_idx = io->idx;
  a.out_qn = io->q_sqnorm;
  a.out_keep = io->keep;
  a.sync = w.cnt;
  if (a.n <= 16)  // one row tile: the projection groups reduce in LDS
    hipLaunchKernelGGL((decode_fused_kernel<DT, 128, KPW, K, TK, true>), dim3(kFusedWGs), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((decode_fused_kernel<DT, 128, KPW, K, TK, false>), dim3(kFusedWGs), dim3(256), 0, s, a);
}

template <int DT, int KPW>
void fused_nn_tk(const tm_table_layer *t, const tm_layer_io *io, const tm_decode_ws &w, const tm_route_args *ra,
                 int64_t nsplit, int64_t n_keep, hipStream_t s) {
  const bool tk8 = io->router_top_k == 8;
  if (io->n_nearest == 1)
    tk8 ? launch_fused<DT, KPW, 1, 8>(t, io, w, ra, nsplit, n_keep, s)
        : launch_fused<DT, KPW, 1, 6>(t, io, w, ra, nsplit, n_keep, s);
  else
    tk8 ? launch_fused<DT, KPW, 4, 8>(t, io, w, ra, nsplit, n_keep, s)
        : launch_fused<DT, KPW, 4, 6>(t, io, w, ra, nsplit, n_keep, s);
}

// The one-launch plan's shapes (on top of tm_internal_decode_ok): d = 128,
// hidden 2048 or 2560, at most kFusedWGs search splits, a fused router of 64
// or 128 experts (or weights from a router launch).
bool fused_ok(const tm_table_layer *t, const tm_layer_io *io, const tm_route_args *ra, int64_t nsplit) {
  return t->dim == 128 && (t->hidden == 2048 || t->hidden == 2560) && nsplit >= 1 && nsplit <= kFusedWGs &&
         (ra == nullptr || ((ra->n_experts == 64 || ra->n_experts == 128) && ra->top_k == io->router_top_k)) &&
         (t->metric == TM_METRIC_DOT || t->c_sqnorm != nullptr) && io->weights && io->expert_ids;
}

bool rows16(const void *base, int64_t ld) {
  return base == nullptr || (tm_aligned16(base) && (ld * 2) % 16 == 0);
}

}  // namespace

size_t tm_internal_decode_qn_floats(int64_t n, int32_t dim) { return (size_t)n * (size_t)(dim / 16); }
size_t tm_internal_decode_keys(int64_t n) { return (size_t)kKeyRep * (size_t)tm_key_stride(n); }
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
                               const tm_route_args *ra, int64_t n_keep, void *const *ev, bool one_launch,
                               hipStream_t s) {
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
  if (one_launch && ev == nullptr && fused_ok(t, io, ra, nsplit)) {  // one launch
    const int kpw = t->hidden / (32 * kSlices);
    if (t->dtype == TM_DT_BF16)
      kpw == 8 ? fused_nn_tk<TM_DT_BF16, 8>(t, io, w, ra, nsplit, n_keep, s)
               : fused_nn_tk<TM_DT_BF16, 10>(t, io, w, ra, nsplit, n_keep, s);
    else
      kpw == 8 ? fused_nn_tk<TM_DT_F16, 8>(t, io, w, ra, nsplit, n_keep, s)
               : fused_nn_tk<TM_DT_F16, 10>(t, io, w, ra, nsplit, n_keep, s);
    TM_LAUNCH_CHECK("tm_table_forward(decode)");
    return TM_OK;
  }
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
