// Reference-semantics ("mode R") searches over the per-(expert, modality)
// tables keys[E, 2, K, d]:
//   - tm_search_gated: the prefill/decode offline search (cosine or raw dot,
//     threshold gate) from already projected queries
//     (table_moe/cache_engine/search.py:515-602, :661-697; Triton :35-256);
//   - tm_search_hybrid: the decode online-window + offline search with the
//     projection fused (search.py:839-954, :987-1105, :778-806; Triton :258-385).
//
// Scores are fp32 sums of the model-dtype products; the arg-max keeps the
// first index among equal maxima, as torch.max / tl.max(return_indices) do.
//
// tm_search_gated runs gated_seg_kernel for 16-bit tables whose dimension is
// a multiple of 16: the reference's grid is one program per (token, slot),
// each streaming its whole 256 x 64 table (at Qwen prefill ~13k searched
// pairs x 32 KiB); here the pairs that share a table are searched together.
// A workgroup owns one expert and one chunk of tokens: it scans the chunk's
// slots for that expert, compacts the searched pairs per modality into LDS,
// and scores them 32 at a time on the matrix cores (v_mfma_f32_32x32x16:
// A = 32 table rows, B = the 32 pairs' queries), its four waves splitting
// the table's 32-row blocks; every table row is read once per 32 pairs.
#include "tm_common.h"
#include "tm_mfma.h"

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
  if constexpr (VEC && Elem<DT>::kBytes == 2) {
    if (dim == 64) {  // the reference's table width: a lane's rows in groups of 4, all of a group's loads in flight
      for (int64_t c0 = lane; c0 < n_cent; c0 += 4 * 64) {
        uint4 raw[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          int64_t c = c0 + 64 * u;
          c = c < n_cent ? c : n_cent - 1;  // clamped in bounds; masked below
          const uint4 *row = reinterpret_cast<const uint4 *>(table + c * ks_c);
#pragma unroll
          for (int t = 0; t < 8; ++t) raw[u][t] = row[t];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t c = c0 + 64 * u;
          float acc = 0.f;
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const typename Elem<DT>::T *e = reinterpret_cast<const typename Elem<DT>::T *>(&raw[u][t]);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc = fmaf(qv[8 * t + i], Elem<DT>::to_f(e[i]), acc);
          }
          if (c < n_cent && acc > best) { best = acc; best_i = (int)c; }
        }
      }
      tm_wave_argmax(best, best_i);
      return;
    }
  }
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

// ---------------------------------------------------------------------------
// Segment-grouped gated search (16-bit tables, DIM % 16 == 0).
// ---------------------------------------------------------------------------
constexpr int kSegThreads = 256;

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load and store of the wave (its fence), which
// would drain the next block's query prefetch and this block's result stores
// at each barrier; the exchanges here go through LDS alone.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
constexpr int kSegList = 8192;  // pair slots per workgroup (LDS); tokens per chunk <= kSegList / top_k

// REG: tables of at most 256 rows with DIM <= 128 -- each wave loads its
// (at most two) 32-row blocks of every modality table that has pairs once,
// right after the scan, and keeps them in registers for all pair blocks.
template <int DT, int DIM, bool REG>
__global__ __launch_bounds__(kSegThreads) void gated_seg_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t n, int64_t ld_q,
    const typename Elem<DT>::T *__restrict__ keys, int64_t n_exp, int64_t n_cent, int64_t ks_e, int64_t ks_m,
    int64_t ks_c, const int64_t *__restrict__ sel, int top_k, int64_t ss_b, int64_t ss_s,
    const uint8_t *__restrict__ is_vision, const uint8_t *__restrict__ reuse, int64_t rs_b, int64_t rs_s,
    int col_offset, float thr_v, float thr_t, int cmp, uint8_t *__restrict__ out_hit,
    int64_t *__restrict__ out_idx, int64_t os_b, int64_t os_s, int64_t tok_per_wg) {
  using T = typename Elem<DT>::T;
  constexpr int KS = DIM / 16;  // k-steps
  __shared__ uint32_t list[kSegList];  // vision pairs from the front, text pairs from the back
  __shared__ int cnt[2];
  __shared__ float red_v[4][32];
  __shared__ int red_i[4][32];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t e = blockIdx.x;
  const int64_t b0 = (int64_t)blockIdx.y * tok_per_wg;
  const int64_t b1 = b0 + tok_per_wg < n ? b0 + tok_per_wg : n;
  if (tid < 2) cnt[tid] = 0;
  __syncthreads();
  // 1) scan: pairs routed to expert e (and, in expert 0's workgroups, pairs
  // whose id is out of range); searched ones are listed, the rest written
  // as (0, 0) here -- every pair is written by exactly one workgroup.  A
  // thread takes tokens tid, tid + 256, ... and loads the slot ids of
  // kScanTok of them (up to kScanSlots slots each) before testing any, so
  // the loads are in flight together; pair p = token * top_k + slot.
  constexpr int kScanTok = 4, kScanSlots = 8;
  const int ntok = (int)(b1 - b0);
  auto row_ptr = [&](int m, int64_t cb) {
    int64_t c = cb + (lane & 31);
    c = c < n_cent ? c : n_cent - 1;  // rows past the table re-read its last row (masked below)
    return keys + e * ks_e + m * ks_m + c * ks_c + 8 * (lane >> 5);
  };
  // the pair's searched flag and modality, from values already loaded
  auto test_pair = [&](int bl, int s, int64_t ex, bool rflag, bool vflag) {
    const bool valid = ex >= 0 && ex < n_exp;
    if (ex == e || (!valid && e == 0)) {
      const int64_t b = b0 + bl;
      const bool searched = valid && s >= col_offset && rflag;
      if (searched) {
        const int m = vflag ? 0 : 1;
        const int pos = atomicAdd(&cnt[m], 1);
        list[m == 0 ? pos : kSegList - 1 - pos] = (uint32_t)(bl * top_k + s);
      } else {
        const int64_t o = b * os_b + s * os_s;
        out_hit[o] = 0;
        out_idx[o] = 0;
      }
    }
  };
  const bool fast = top_k == kScanSlots && ss_s == 1 && ss_b == kScanSlots &&
                    (reuse == nullptr || (rs_s == 1 && rs_b == kScanSlots)) &&
                    (reinterpret_cast<uintptr_t>(sel) & 15) == 0 &&
                    (reuse == nullptr || (reinterpret_cast<uintptr_t>(reuse) & 1) == 0);
  if (fast) {  // uniform
    // 1) coalesced scan of contiguous [n][8] ids: 4 lanes per token, 2 slots
    // each (one 16-byte load of ids, one 2-byte load of reuse flags); a pass
    // covers 64 tokens and every pass's loads are issued before any test.
    constexpr int kPasses = 16;
    const int q4 = lane & 3, s0 = 2 * q4;
    for (int t0 = 0; t0 < ntok; t0 += kPasses * 64) {
      uint4 idv[kPasses];
      uint16_t rfv[kPasses];
      uint8_t vfv[kPasses];
#pragma unroll
      for (int u = 0; u < kPasses; ++u) {
        const int bl = t0 + u * 64 + (tid >> 2);
        const int64_t b = b0 + (bl < ntok ? bl : ntok - 1);  // clamped: every load is in bounds
        idv[u] = *reinterpret_cast<const uint4 *>(sel + b * kScanSlots + s0);
        rfv[u] = reuse == nullptr ? (uint16_t)0x0101 : *reinterpret_cast<const uint16_t *>(reuse + b * kScanSlots + s0);
        vfv[u] = is_vision == nullptr ? (uint8_t)1 : is_vision[b];
      }
      // Every pass's loads are issued before the first test: the values are
      // inputs of these empty statements (without them the scheduler sinks
      // loads toward their tests and their latencies add up: 31 vs 21 us).
#pragma unroll
      for (int u = 0; u < kPasses; ++u)
        asm volatile("" ::"v"(idv[u].x), "v"(idv[u].z), "v"((uint32_t)rfv[u]), "v"((uint32_t)vfv[u]));
      // test, branch-free: bit 2u + h of mv / mt marks a searched vision /
      // text pair of expert e (token t0 + 64u + tid / 4, slot s0 + h); zmask
      // marks e's pairs that are not searched (zero outputs, written below)
      const uint32_t e32 = (uint32_t)e, nexp32 = (uint32_t)n_exp;
      const int tl = tid >> 2;
      const bool col_ok[2] = {s0 >= col_offset, s0 + 1 >= col_offset};
      uint32_t mv = 0, mt = 0, zmask = 0;
      if (e32 != 0) {  // uniform: a pair is e's exactly when its id equals e (e < n_exp: valid)
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
          const uint32_t out = t0 + u * 64 + tl < ntok ? 0u : 1u;  // clamped rows past the chunk
          const bool text = vfv[u] == 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t lo = h == 0 ? idv[u].x : idv[u].z, hi = h == 0 ? idv[u].y : idv[u].w;
            const bool mine = ((lo ^ e32) | hi | out) == 0;
            const bool searched = mine && col_ok[h] && ((rfv[u] >> (8 * h)) & 0xffu) != 0;
            const uint32_t bit = 1u << (2 * u + h);
            zmask |= (mine && !searched) ? bit : 0u;
            mv |= (searched && !text) ? bit : 0u;
            mt |= (searched && text) ? bit : 0u;
          }
        }
      } else {  // expert 0 also takes the pairs whose id is out of range (zero outputs)
#pragma unroll
        for (int u = 0; u < kPasses; ++u) {
          const bool in = t0 + u * 64 + tl < ntok;
          const bool text = vfv[u] == 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t lo = h == 0 ? idv[u].x : idv[u].z, hi = h == 0 ? idv[u].y : idv[u].w;
            const bool valid = hi == 0 && lo < nexp32;  // negative ids have hi != 0
            const bool mine = in && (!valid || lo == 0);
            const bool searched = mine && valid && col_ok[h] && ((rfv[u] >> (8 * h)) & 0xffu) != 0;
            const uint32_t bit = 1u << (2 * u + h);
            zmask |= (mine && !searched) ? bit : 0u;
            mv |= (searched && !text) ? bit : 0u;
            mt |= (searched && text) ? bit : 0u;
          }
        }
      }
      auto token_of = [&](int k) { return t0 + (k >> 1) * 64 + tl; };
      while (zmask != 0) {  // rare: zero outputs of e's pairs that are not searched
        const int k = __builtin_ctz(zmask);
        zmask &= zmask - 1;
        const int64_t o = (b0 + token_of(k)) * os_b + (int64_t)(s0 + (k & 1)) * os_s;
        out_hit[o] = 0;
        out_idx[o] = 0;
      }
      // append: one LDS atomic per wave and modality (positions from a wave
      // prefix sum of the per-lane counts), then each lane writes its pairs
      const uint32_t cv = (uint32_t)__builtin_popcount(mv), ct = (uint32_t)__builtin_popcount(mt);
      const uint32_t iv = tm_wave_incl_scan(cv), it = tm_wave_incl_scan(ct);
      const uint32_t tv = (uint32_t)__builtin_amdgcn_readlane((int)iv, 63);
      const uint32_t tt = (uint32_t)__builtin_amdgcn_readlane((int)it, 63);
      int bv = 0, bt = 0;
      if (lane == 63) {
        if (tv) bv = atomicAdd(&cnt[0], (int)tv);
        if (tt) bt = atomicAdd(&cnt[1], (int)tt);
      }
      int pv = __builtin_amdgcn_readlane(bv, 63) + (int)(iv - cv);
      int pt = __builtin_amdgcn_readlane(bt, 63) + (int)(it - ct);
      while (mv != 0) {
        const int k = __builtin_ctz(mv);
        mv &= mv - 1;
        list[pv++] = (uint32_t)(token_of(k) * kScanSlots + s0 + (k & 1));
      }
      while (mt != 0) {
        const int k = __builtin_ctz(mt);
        mt &= mt - 1;
        list[kSegList - 1 - pt++] = (uint32_t)(token_of(k) * kScanSlots + s0 + (k & 1));
      }
    }
  } else {
    // 1) scan: a thread takes tokens tid, tid + 256, ... and loads the slot
    // ids, reuse flags and modality bytes of kScanTok of them (up to
    // kScanSlots slots each) before testing any: every load is in flight
    // together and no test waits on a load of its own.
    for (int t0 = 0; t0 < ntok; t0 += kSegThreads * kScanTok) {
      int64_t ex[kScanTok][kScanSlots];
      uint8_t rf[kScanTok][kScanSlots];
      uint8_t vf[kScanTok];
  #pragma unroll
      for (int u = 0; u < kScanTok; ++u) {
        const int bl = t0 + u * kSegThreads + tid;
        const int64_t b = b0 + (bl < ntok ? bl : ntok - 1);  // clamped: every load is in bounds
  #pragma unroll
        for (int s = 0; s < kScanSlots; ++s) {
          const int sc = s < top_k ? s : top_k - 1;
          ex[u][s] = sel[b * ss_b + sc * ss_s];
          rf[u][s] = reuse == nullptr ? (uint8_t)1 : reuse[b * rs_b + sc * rs_s];
        }
        vf[u] = is_vision == nullptr ? (uint8_t)1 : is_vision[b];
      }
  #pragma unroll
      for (int u = 0; u < kScanTok; ++u) {
        const int bl = t0 + u * kSegThreads + tid;
        if (bl >= ntok) continue;
  #pragma unroll
        for (int s = 0; s < kScanSlots; ++s)
          if (s < top_k) test_pair(bl, s, ex[u][s], rf[u][s] != 0, vf[u] != 0);
        for (int s = kScanSlots; s < top_k; ++s) {
          const int64_t b = b0 + bl;
          test_pair(bl, s, sel[b * ss_b + s * ss_s], reuse == nullptr || reuse[b * rs_b + s * rs_s],
                    vf[u] != 0);
        }
      }
    }
  }
  lds_barrier();  // the list and the counts are complete (the pair stores may still fly)
  const int counts[2] = {cnt[0], cnt[1]};
  uint4 kreg[REG ? 2 : 1][REG ? 2 : 1][KS];
  if constexpr (REG) {  // the tables that have pairs, held in registers for every block
#pragma unroll
    for (int m = 0; m < 2; ++m)
      if (counts[m] > 0)  // uniform
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
          const T *krow = row_ptr(m, (int64_t)wave * 32 + bi * 128);
#pragma unroll
          for (int t = 0; t < KS; ++t) kreg[m][bi][t] = *reinterpret_cast<const uint4 *>(krow + 16 * t);
        }
  }
  // 2) search, 32 pairs of one modality at a time: the vision blocks, then
  // the text blocks; each block's queries are loaded while the previous
  // block is scored
  const int nbv = (counts[0] + 31) >> 5, nb = nbv + ((counts[1] + 31) >> 5);
  auto block_pair = [&](int i, int &m, int &j, int &jj, uint32_t &p) {
    m = i < nbv ? 0 : 1;
    const int c_m = counts[m];
    const int blk = (i < nbv ? i : i - nbv) * 32;
    j = blk + (lane & 31);
    jj = j < c_m ? j : blk;  // past the end: the block's first pair (result dropped)
    p = list[m == 0 ? jj : kSegList - 1 - jj];
  };
  auto load_q = [&](uint32_t p, uint4 (&f)[KS]) {
    const T *qrow = q + (b0 + (int64_t)(p / (uint32_t)top_k)) * ld_q + 8 * (lane >> 5);
#pragma unroll
    for (int t = 0; t < KS; ++t) f[t] = *reinterpret_cast<const uint4 *>(qrow + 16 * t);
  };
  uint4 qf[KS], qn[KS];
  if (nb > 0) {  // uniform
    int m0, j0, jj0;
    uint32_t p0;
    block_pair(0, m0, j0, jj0, p0);
    load_q(p0, qn);
  }
  for (int i = 0; i < nb; ++i) {  // uniform
    int m, j, jj;
    uint32_t p;
    block_pair(i, m, j, jj, p);
    const int c_m = counts[m];
#pragma unroll
    for (int t = 0; t < KS; ++t) qf[t] = qn[t];
    if (i + 1 < nb) {  // uniform: the next block's queries fly while this one is scored
      int m1, j1, jj1;
      uint32_t p1;
      block_pair(i + 1, m1, j1, jj1, p1);
      load_q(p1, qn);
    }
    {
      float best = -__builtin_huge_valf();
      int best_i = 0x7fffffff;
      auto score_block = [&](const uint4 (&kf)[KS], int64_t cb) {
        tm_f32x16 acc{};
#pragma unroll
        for (int t = 0; t < KS; ++t) acc = tm_mfma32x32x16<DT>(kf[t], qf[t], acc);
        // lane holds pair (lane % 32) against rows 8(i/4) + 4(lane/32) + i%4 of
        // the block, ascending in i; selects, not branches (the first of equal
        // maxima stays)
        const int c0 = (int)cb + 4 * (lane >> 5), nc = (int)n_cent;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int ci = c0 + 8 * (i >> 2) + (i & 3);
          const float v = acc[i];
          const bool take = (ci < nc) & (v > best);
          best = take ? v : best;
          best_i = take ? ci : best_i;
        }
      };
      if constexpr (REG) {
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
          const int64_t cb = (int64_t)wave * 32 + bi * 128;
          if (cb < n_cent) {  // uniform per wave
            if (m == 0)  // uniform: constant register indices on both sides
              score_block(kreg[0][bi], cb);
            else
              score_block(kreg[1][bi], cb);
          }
        }
      } else {
        for (int64_t cb = (int64_t)wave * 32; cb < n_cent; cb += 4 * 32) {  // uniform per wave
          const T *krow = row_ptr(m, cb);
          uint4 kf[KS];
#pragma unroll
          for (int t = 0; t < KS; ++t) kf[t] = *reinterpret_cast<const uint4 *>(krow + 16 * t);
          score_block(kf, cb);
        }
      }
      const float ov = __shfl_xor(best, 32, 64);  // lanes l and l ^ 32 hold the same pair
      const int oi = __shfl_xor(best_i, 32, 64);
      if (ov > best || (ov == best && oi < best_i)) {
        best = ov;
        best_i = oi;
      }
      if (lane < 32) {
        red_v[wave][lane] = best;
        red_i[wave][lane] = best_i;
      }
      lds_barrier();
      if (wave == 0 && lane < 32 && j < c_m) {
        float v = red_v[0][lane];
        int bi = red_i[0][lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) {  // waves hold interleaved blocks: ties go to the lower index
          const float wv = red_v[w][lane];
          const int wi = red_i[w][lane];
          if (wv > v || (wv == v && wi < bi)) {
            v = wv;
            bi = wi;
          }
        }
        const int64_t b = b0 + (int64_t)(p / (uint32_t)top_k);
        const int s = (int)(p % (uint32_t)top_k);
        const float thr = m == 0 ? thr_v : thr_t;
        const bool hit = (cmp == TM_CMP_GE) ? (v >= thr) : (v > thr);
        const int64_t o = b * os_b + s * os_s;
        out_hit[o] = hit ? 1 : 0;
        out_idx[o] = hit ? (int64_t)bi : 0;
      }
      lds_barrier();  // red_* are rewritten by the next block
    }
  }
}

// Tokens per workgroup chunk of gated_seg_kernel: about 512 workgroups over
// the experts, at most kSegList / top_k tokens (the LDS pair list), at least
// 64 tokens per chunk unless the batch is smaller.
int64_t seg_tokens_per_wg(int64_t n, int64_t n_exp, int top_k) {
  const int64_t cap = kSegList / top_k;
  int64_t chunks = tm_cdiv(512, n_exp);
  const int64_t by_size = tm_cdiv(n, 64);
  chunks = chunks < by_size ? chunks : by_size;
  if (chunks < 1) chunks = 1;
  int64_t tok = tm_cdiv(n, chunks);
  return tok < cap ? tok : cap;
}

// ---------------------------------------------------------------------------
// Decode hybrid search, two launches.
//  hybrid_partial_kernel: grid (token, slice): each workgroup stages the
//    token's x in LDS, writes the fp32 projection partial of its slice of
//    `hidden` (every column) and the online-window scores of its share of
//    the window rows.
//  hybrid_finish_kernel: one workgroup per token: q = dtype(sum of the slice
//    partials in slice order + bias) (one rounding), the window arg-max and
//    online hits, then the offline search of the remaining slots (one wave
//    per slot) and every output.
// Workspace: partials [n][G][dim] fp32, then window scores [n][kMaxOnline].
// ---------------------------------------------------------------------------
constexpr int kMaxOnline = 1024;
constexpr int kHybRowsPerSlice = 128;
constexpr int kHybMaxSlices = 16;
constexpr int kHybMaxOnTopk = 16;  // window rows' ids compared from registers up to this many
constexpr int kFinThreads = 512;   // hybrid_finish_kernel: q waves, the window wave, 8 search waves

inline int hybrid_slices(int hidden) {
  int g = hidden / kHybRowsPerSlice;
  return g < 1 ? 1 : (g > kHybMaxSlices ? kHybMaxSlices : g);
}
inline int hybrid_slice_rows(int hidden, int g) { return (int)(tm_cdiv(tm_cdiv(hidden, g), 8) * 8); }

template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void hybrid_partial_kernel(
    const typename Elem<DT>::T *__restrict__ x, int hidden, int64_t ld_x, const uint8_t *__restrict__ is_vision,
    const typename Elem<DT>::T *__restrict__ pv, const typename Elem<DT>::T *__restrict__ pt, int64_t ps_h,
    int64_t ps_d, int dim, int slice_rows, int need_proj, const typename Elem<DT>::T *__restrict__ on_keys,
    int64_t ld_on, int n_valid, float *__restrict__ partial, float *__restrict__ scores) {
  using T = typename Elem<DT>::T;
  extern __shared__ float xsh[];  // hidden floats
  __shared__ float red[kThreads];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x;
  const int g = blockIdx.y, G = gridDim.y;
  const T *xr = x + b * ld_x;
  // (unrolled loops below: several iterations' loads are in flight together)
#pragma unroll 8
  for (int h = tid; h < hidden; h += kThreads) xsh[h] = Elem<DT>::to_f(xr[h]);
  __syncthreads();
  // projection partial over rows [h0, h1) of this slice, every column
  if (need_proj) {  // uniform
    const bool vis = is_vision == nullptr || is_vision[b];
    const T *P = vis ? pv : pt;
    const int h0 = g * slice_rows;
    const int h1 = h0 + slice_rows < hidden ? h0 + slice_rows : hidden;
    const int parts = kThreads / dim;  // >= 1
    const int col = tid % dim, part = tid / dim;
    float acc = 0.f;
    if (part < parts && h0 < h1) {
      const int per = (h1 - h0 + parts - 1) / parts;
      const int a0 = h0 + part * per;
      const int a1 = a0 + per < h1 ? a0 + per : h1;
      if (VEC && ps_h == 1) {  // k-contiguous copy: each thread's rows are one contiguous run
        const T *src = P + (int64_t)col * ps_d;
        int h = a0;
#pragma unroll 4
        for (; h + 8 <= a1; h += 8) {
          float v[8];
          tm_load8<DT>(src + h, v);
#pragma unroll
          for (int u = 0; u < 8; ++u) acc = fmaf(xsh[h + u], v[u], acc);
        }
        for (; h < a1; ++h) acc = fmaf(xsh[h], Elem<DT>::to_f(src[h]), acc);
      } else {
        for (int h = a0; h < a1; ++h)
          acc = fmaf(xsh[h], Elem<DT>::to_f(P[(int64_t)h * ps_h + (int64_t)col * ps_d]), acc);
      }
    }
    red[tid] = acc;
    __syncthreads();
    if (tid < dim) {
      float sum = 0.f;
      for (int pp = 0; pp < parts; ++pp) sum += red[pp * dim + tid];  // parts in order
      partial[((int64_t)b * G + g) * dim + tid] = sum;
    }
  }
  // online scores of window rows g, g + G, ...: one wave per row
  for (int j = g + G * wave; j < n_valid; j += G * (kThreads / 64)) {
    const T *kr = on_keys + (int64_t)j * ld_on;
    float acc = 0.f;
    if (VEC) {
#pragma unroll 4
      for (int h = 8 * lane; h + 8 <= hidden; h += 8 * 64) {
        float v[8];
        tm_load8<DT>(kr + h, v);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fmaf(xsh[h + u], v[u], acc);
      }
      for (int h = (hidden / 8) * 8 + lane; h < hidden; h += 64) acc = fmaf(xsh[h], Elem<DT>::to_f(kr[h]), acc);
    } else {
      for (int h = lane; h < hidden; h += 64) acc = fmaf(xsh[h], Elem<DT>::to_f(kr[h]), acc);
    }
    acc = tm_wave_sum(acc);
    if (lane == 0) scores[(int64_t)b * kMaxOnline + j] = acc;
  }
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kFinThreads) void hybrid_finish_kernel(
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ bv,
    const typename Elem<DT>::T *__restrict__ bt, int dim, int n_slices, const float *__restrict__ partial,
    const float *__restrict__ scores, int n_valid, const int64_t *__restrict__ on_ids, int on_topk,
    int64_t ld_on_ids, const typename Elem<DT>::T *__restrict__ keys, int64_t n_exp, int64_t n_cent, int64_t ks_e,
    int64_t ks_m, int64_t ks_c, const int64_t *__restrict__ sel, int top_k, int64_t ss_b, int64_t ss_s, int keep_k,
    uint8_t *__restrict__ on_hit, int64_t *__restrict__ on_idx, uint8_t *__restrict__ off_hit,
    int64_t *__restrict__ off_idx, int64_t *__restrict__ on_slot, int64_t os_b, int64_t os_s,
    typename Elem<DT>::T *__restrict__ q_out, int64_t ld_q_out) {
  __shared__ float qsh[kMaxDim];
  __shared__ int s_jstar, s_valid_on;
  __shared__ uint8_t s_onhit[64];
  __shared__ int s_onslot[64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x;
  const bool vis = is_vision == nullptr || is_vision[b];
  const bool need_proj = keep_k < top_k;
  // the slot's expert id, loaded first (used after the first barrier)
  const int64_t my_e = tid < top_k ? sel[b * ss_b + tid * ss_s] : 0;
  // 1) q = dtype(sum of the slice partials + bias): every slice's partial is
  // requested before any is added (in slice order, as before)
  if (need_proj && tid < dim) {
    float pv[kHybMaxSlices];
#pragma unroll
    for (int g = 0; g < kHybMaxSlices; ++g) {
      const int gc = g < n_slices ? g : n_slices - 1;
      pv[g] = partial[((int64_t)b * n_slices + gc) * dim + tid];
    }
    const float bias = Elem<DT>::to_f((vis ? bv : bt)[tid]);
    float sum = 0.f;
#pragma unroll
    for (int g = 0; g < kHybMaxSlices; ++g)
      if (g < n_slices) sum += pv[g];
    const float v = tm_round<DT>(sum + bias);
    qsh[tid] = v;
    if (q_out != nullptr) q_out[b * ld_q_out + tid] = Elem<DT>::from_f(v);
  }
  // 2) window arg-max (first index of the maximum) on wave 4, beside the q waves
  if (wave == 4) {
    float mx = -__builtin_huge_valf();
    int js = 0x7fffffff;
    for (int j = lane; j < n_valid; j += 64) {
      const float v = scores[(int64_t)b * kMaxOnline + j];
      if (v > mx) { mx = v; js = j; }
    }
    tm_wave_argmax(mx, js);
    if (lane == 0) {
      const int valid_on = (n_valid > 0 && mx > 0.f) ? 1 : 0;
      s_jstar = valid_on ? js : -1;
      s_valid_on = valid_on;
      on_idx[b] = valid_on ? js : -1;
    }
  }
  __syncthreads();
  // 3) online hits of the searched slots: the window row's ids all requested
  // at once, then the first match
  if (tid < top_k) {
    const int s = tid;
    uint8_t hit = 0;
    int slot = 0;
    if (s >= keep_k && s_valid_on) {
      const int64_t *ids = on_ids + (int64_t)s_jstar * ld_on_ids;
      if (on_topk <= kHybMaxOnTopk) {
        int64_t v[kHybMaxOnTopk];
#pragma unroll
        for (int t = 0; t < kHybMaxOnTopk; ++t) v[t] = ids[t < on_topk ? t : 0];
#pragma unroll
        for (int t = kHybMaxOnTopk - 1; t >= 0; --t)  // descending: the first match wins
          if (t < on_topk && v[t] == my_e) { hit = 1; slot = t; }
      } else {
        for (int t = 0; t < on_topk; ++t) {
          if (ids[t] == my_e) { hit = 1; slot = t; break; }
        }
      }
    }
    s_onhit[s] = hit;
    s_onslot[s] = slot;
  }
  __syncthreads();
  // 4) offline search of the remaining slots, one wave per slot (8 waves);
  // every output written
  for (int s = wave; s < top_k; s += kFinThreads / 64) {
    const int64_t o = b * os_b + s * os_s;
    uint8_t hit = 0;
    int64_t idx = 0;
    if (s >= keep_k && !s_onhit[s]) {  // uniform per wave
      const int64_t e = sel[b * ss_b + s * ss_s];
      if (e >= 0 && e < n_exp) {
        float best;
        int best_i;
        wave_table_argmax<DT, VEC>(keys + e * ks_e + (vis ? 0 : 1) * ks_m, ks_c, n_cent, dim, qsh, best, best_i);
        hit = best >= 0.f;
        idx = hit ? best_i : 0;
      }
    }
    if (lane == 0) {
      off_hit[o] = hit;
      off_idx[o] = idx;
      on_hit[o] = s_onhit[s];
      on_slot[o] = s_onhit[s] ? s_onslot[s] : 0;
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
    if constexpr (E == 2) {
      const int64_t tok = top_k <= kSegList ? seg_tokens_per_wg(n_tokens, n_experts, top_k) : 0;
      const int64_t chunks = tok > 0 ? tm_cdiv(n_tokens, tok) : 0;
      const bool seg = vec && dim % 16 == 0 && tm_aligned16(q_low) && (ld_q * E) % 16 == 0 && tok > 0 &&
                       chunks <= 65535 && n_experts <= 0x7fffffff && n_centroids < 0x7fffffff;
      if (seg) {
        const dim3 sgrid((unsigned)n_experts, (unsigned)chunks);
        auto go = [&](auto dim_tag) {
          constexpr int D = decltype(dim_tag)::value;
          auto launch_seg = [&](auto reg_tag) {
            constexpr bool R = decltype(reg_tag)::value;
            hipLaunchKernelGGL((gated_seg_kernel<DT, D, R>), sgrid, dim3(kSegThreads), 0, tm_hip_stream(stream),
                               static_cast<const T *>(q_low), n_tokens, ld_q, static_cast<const T *>(keys),
                               n_experts, n_centroids, ks_e, ks_m, ks_c, sel, top_k, ss_b, ss_s, is_vision, reuse,
                               rs_b, rs_s, col_offset, thr_vision, thr_text, cmp, out_hit, out_idx, os_b, os_s, tok);
          };
          if constexpr (D <= 128) {
            if (n_centroids <= 256) {
              launch_seg(std::true_type{});
              return;
            }
          }
          launch_seg(std::false_type{});
        };
        bool launched = true;
        switch (dim) {
          case 16: go(std::integral_constant<int, 16>{}); break;
          case 32: go(std::integral_constant<int, 32>{}); break;
          case 64: go(std::integral_constant<int, 64>{}); break;
          case 128: go(std::integral_constant<int, 128>{}); break;
          case 256: go(std::integral_constant<int, 256>{}); break;
          default: launched = false;
        }
        if (launched) {
          TM_LAUNCH_CHECK("tm_search_gated");
          return TM_OK;
        }
      }
    }
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

extern "C" size_t tm_search_hybrid_workspace_size(int64_t n_tokens, int32_t hidden, int32_t dim) {
  if (n_tokens <= 0 || hidden <= 0 || dim <= 0) return 0;
  return (size_t)n_tokens * ((size_t)hybrid_slices(hidden) * (size_t)dim + kMaxOnline) * sizeof(float);
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
                                int64_t os_s, void *q_out, int64_t ld_q_out, void *workspace, size_t workspace_bytes,
                                tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && hidden >= 1 && hidden <= 16384 && ld_x >= hidden && dim >= 1 && dim <= kMaxDim &&
                 n_centroids >= 1 && n_centroids <= 65536 && n_experts >= 1 && top_k >= 0 && top_k <= 64,
             TM_EINVAL_SHAPE, "tm_search_hybrid: bad sizes");
  TM_REQUIRE(n_online_valid >= 0 && n_online_valid <= kMaxOnline && online_topk >= 0 && online_topk <= 64,
             TM_EINVAL_SHAPE, "tm_search_hybrid: online window too large");
  TM_REQUIRE(ps_h == 1 || ps_d == 1, TM_EINVAL_SHAPE, "tm_search_hybrid: projection needs a unit stride");
  TM_REQUIRE(q_out == nullptr || ld_q_out >= dim, TM_EINVAL_SHAPE, "tm_search_hybrid: bad q_out stride");
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(x && proj_vis && bias_vis && keys && sel && on_hit && on_idx && off_hit && off_idx && on_slot,
             TM_EINVAL_ARG, "tm_search_hybrid: null pointer");
  TM_REQUIRE((proj_txt == nullptr) == (bias_txt == nullptr), TM_EINVAL_ARG,
             "tm_search_hybrid: proj_txt and bias_txt must both be set or both be NULL");
  TM_REQUIRE(n_online_valid == 0 || (online_keys && online_ids), TM_EINVAL_ARG,
             "tm_search_hybrid: online window pointers missing");
  TM_REQUIRE(n_tokens < 65536 * 32768LL, TM_EINVAL_SHAPE, "tm_search_hybrid: too many tokens");
  if (keep_k < 0) keep_k = 0;
  if (keep_k > top_k) keep_k = top_k;
  // nothing searched: outputs are only cleared (on_idx = -1), no window lookup
  if (keep_k == top_k) n_online_valid = 0;
  const size_t need = tm_search_hybrid_workspace_size(n_tokens, hidden, dim);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need && tm_aligned16(workspace), TM_EWORKSPACE,
             "tm_search_hybrid: workspace %zu bytes < %zu", workspace_bytes, need);
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    using T = typename Elem<DT>::T;
    const int E = Elem<DT>::kBytes;
    const bool vec = dim % 8 == 0 && tm_aligned16(keys) && (ks_e * E) % 16 == 0 && (ks_m * E) % 16 == 0 &&
                     (ks_c * E) % 16 == 0 && tm_aligned16(x) && (ld_x * E) % 16 == 0 &&
                     (n_online_valid == 0 || (tm_aligned16(online_keys) && (ld_online * E) % 16 == 0)) &&
                     (ps_h != 1 || (tm_aligned16(proj_vis) && (proj_txt == nullptr || tm_aligned16(proj_txt)) &&
                                    (ps_d * E) % 16 == 0));
    const T *pt = static_cast<const T *>(proj_txt ? proj_txt : proj_vis);
    const T *bt = static_cast<const T *>(proj_txt ? bias_txt : bias_vis);
    const int G = hybrid_slices(hidden);
    float *partial = static_cast<float *>(workspace);
    float *scores = partial + (size_t)n_tokens * G * dim;
    hipStream_t s = tm_hip_stream(stream);
    auto launch = [&](auto vec_tag) {
      constexpr bool VEC = decltype(vec_tag)::value;
      hipLaunchKernelGGL((hybrid_partial_kernel<DT, VEC>), dim3((unsigned)n_tokens, (unsigned)G), dim3(kThreads),
                         (size_t)hidden * sizeof(float), s, static_cast<const T *>(x), hidden, ld_x, is_vision,
                         static_cast<const T *>(proj_vis), pt, ps_h, ps_d, dim, hybrid_slice_rows(hidden, G),
                         keep_k < top_k ? 1 : 0, static_cast<const T *>(online_keys), ld_online, n_online_valid,
                         partial, scores);
      hipLaunchKernelGGL((hybrid_finish_kernel<DT, VEC>), dim3((unsigned)n_tokens), dim3(kFinThreads), 0, s, is_vision,
                         static_cast<const T *>(bias_vis), bt, dim, G, partial, scores, n_online_valid, online_ids,
                         online_topk, ld_online_ids, static_cast<const T *>(keys), n_experts, n_centroids, ks_e, ks_m,
                         ks_c, sel, top_k, ss_b, ss_s, keep_k, on_hit, on_idx, off_hit, off_idx, on_slot, os_b, os_s,
                         static_cast<T *>(q_out), ld_q_out);
    };
    if (vec) launch(std::true_type{});
    else launch(std::false_type{});
    TM_LAUNCH_CHECK("tm_search_hybrid");
    return TM_OK;
  });
}
