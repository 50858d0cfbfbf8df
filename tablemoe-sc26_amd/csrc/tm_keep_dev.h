// Keep-rate selection of the n_keep largest of n <= NT * kKeepRegs scores
// (ties -> lower index) as a block-level device routine, and the decoding of
// packed top-1 search keys into distances (also used by the search kernel
// that decodes its own keys).
#pragma once

#include "tm_common.h"

constexpr int kKeepRegs = 16;    // scores per thread
constexpr int kKeepBins = 4096;  // one 12-bit radix digit
constexpr int kKeepDigit = 12;
constexpr int kKeepPasses = 3;   // 32-bit keys: at most three 12-bit digits

// Sum over the wave of `v` for lanes below `nl` (one LDS read per wave when
// `v` comes from shared memory, then DPP; no all-lane broadcast reads).
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)tm_wave_incl_scan(v), 63);
}

// Optional source of the scores: packed top-1 search keys of the layer call
// (see tm_key_to_dist) with the query norms as `parts` partial sums; the
// kernel then also writes each token's distance, centroid and |q|^2.
struct KeySrc {
  const uint64_t *keys;  // null: scores come from `score`
  const float *qn_part;  // [parts][n]
  int parts;
  int l2;
  float *out_dist;
  int64_t *out_idx;
  float *out_qn;
};

// |q|^2 from the column-group partials in the order of a lane-pair tree over
// the groups (the order a whole-row reduction across lanes adds them).
__device__ __forceinline__ float qn_sum(float a0, float a1, float a2, float a3, int parts) {
  if (parts == 1) return a0;
  if (parts == 2) return a0 + a1;
  return (a0 + a1) + (a2 + a3);
}

// LDS of the routine: one histogram per radix pass (cleared up front), the
// per-wave totals of the block scans and the boundary found by each pass.
template <int NT>
struct __align__(16) KeepSmem {
  uint32_t hist[kKeepPasses][kKeepBins];
  uint32_t wave_tot[NT / 64];
  uint32_t s_min[NT / 64], s_max[NT / 64];
  uint2 s_sel;  // (boundary prefix, keys still to keep at it)
};

// Fast form of keep select (north-star kernel (3)).  A block min/max first
// finds the highest bit in which the keys differ (the bits above it are
// common: for distances, the sign and most of the exponent), then radix
// passes of up to 12 bits walk down from there over one 4096-bin histogram
// per pass (usually two passes).  The boundary bin is found with one block
// scan over the bins in descending order (thread t owns the BPT = 4096 / NT
// bins of rank NT - 1 - t).  Ties at the boundary: lower token index first.
// Thread t owns the contiguous score range [t * per, (t + 1) * per).  With
// `ks.keys` set, the scores are decoded from packed top-1 search keys and the
// routine also writes each token's distance, centroid and |q|^2.
template <int NT>
__device__ __forceinline__ void tm_keep_select_fast(const float *__restrict__ score, int64_t n, int64_t ld,
                                                    int64_t n_keep, uint8_t *__restrict__ out, const KeySrc &ks,
                                                    KeepSmem<NT> &sm) {
  constexpr int NW = NT / 64;
  constexpr int BPT = kKeepBins / NT;
  static_assert(NT % 64 == 0 && NW <= 64 && BPT % 4 == 0 && kKeepPasses * kKeepBins % (4 * NT) == 0, "block shape");
  // One histogram per pass, all cleared up front while the keys load; every
  // LDS value that all threads need is read by one lane per wave and spread
  // with DPP (LDS instruction issue, not bandwidth, bounds this kernel).
  uint32_t(&hist)[kKeepPasses][kKeepBins] = sm.hist;
  uint32_t *wave_tot = sm.wave_tot;
  uint32_t *s_min = sm.s_min, *s_max = sm.s_max;
  uint2 &s_sel = sm.s_sel;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (int)((n + NT - 1) / NT);
  const int64_t lo = (int64_t)tid * per;
  const int64_t hi = (lo + per < n) ? lo + per : n;
  const int cnt = (int)(hi > lo ? hi - lo : 0);

  float sc[kKeepRegs];  // key source: this thread's distances
  if (ks.keys != nullptr) {  // uniform
    uint64_t kv[kKeepRegs];
    float qn[kKeepRegs];
    if (per == 4 && cnt == 4 && ks.parts <= 4 && (n & 3) == 0) {  // 16-byte loads (lo is a multiple of 4)
      const uint4 k01 = *reinterpret_cast<const uint4 *>(ks.keys + lo);
      const uint4 k23 = *reinterpret_cast<const uint4 *>(ks.keys + lo + 2);
      kv[0] = ((uint64_t)k01.y << 32) | k01.x; kv[1] = ((uint64_t)k01.w << 32) | k01.z;
      kv[2] = ((uint64_t)k23.y << 32) | k23.x; kv[3] = ((uint64_t)k23.w << 32) | k23.z;
      float4 qp[4] = {};
#pragma unroll
      for (int p = 0; p < 4; ++p)
        if (p < ks.parts) qp[p] = *reinterpret_cast<const float4 *>(ks.qn_part + (int64_t)p * n + lo);
      const float a[4][4] = {{qp[0].x, qp[0].y, qp[0].z, qp[0].w}, {qp[1].x, qp[1].y, qp[1].z, qp[1].w},
                             {qp[2].x, qp[2].y, qp[2].z, qp[2].w}, {qp[3].x, qp[3].y, qp[3].z, qp[3].w}};
#pragma unroll
      for (int j = 0; j < 4; ++j) qn[j] = qn_sum(a[0][j], a[1][j], a[2][j], a[3][j], ks.parts);
    } else {
#pragma unroll
      for (int j = 0; j < kKeepRegs; ++j)
        if (j < cnt) {
          kv[j] = ks.keys[lo + j];
          float a[4];
#pragma unroll
          for (int p = 0; p < 4; ++p) a[p] = p < ks.parts ? ks.qn_part[(int64_t)p * n + lo + j] : 0.f;
          qn[j] = qn_sum(a[0], a[1], a[2], a[3], ks.parts);
        }
    }
#pragma unroll
    for (int j = 0; j < kKeepRegs; ++j)
      if (j < cnt) {
        int64_t ix;
        sc[j] = tm_key_to_dist(kv[j], qn[j], ks.l2 != 0, ix);
        ks.out_dist[lo + j] = sc[j];
        ks.out_idx[lo + j] = ix;
        ks.out_qn[lo + j] = qn[j];
      }
  }

  if (n_keep <= 0 || n_keep >= n) {
    const uint8_t v = n_keep > 0 ? 1 : 0;
    for (int64_t i = lo; i < hi; ++i) out[i] = v;
    return;
  }
  if (n <= 64) {  // uniform: one wave ranks the keys directly (no LDS, no barrier)
    if (wave == 0) {
      const uint32_t key = lane < n ? tm_orderable(ks.keys ? sc[0] : score[(int64_t)lane * ld]) : 0u;
      uint32_t rank = 0;  // keys ahead of this one: larger, or equal at a lower index
      for (int j = 0; j < (int)n; ++j) {
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)key, j);
        rank += (kj > key || (kj == key && j < lane)) ? 1u : 0u;
      }
      if (lane < n) out[lane] = rank < (uint32_t)n_keep ? 1 : 0;
    }
    return;
  }
  {
    uint4 *h4 = reinterpret_cast<uint4 *>(&hist[0][0]);
#pragma unroll
    for (int i = 0; i < kKeepPasses * kKeepBins / 4 / NT; ++i) h4[tid + i * NT] = make_uint4(0, 0, 0, 0);
  }
  uint32_t keys[kKeepRegs];
  const bool vec4 = per == 4 && (ks.keys != nullptr || (ld == 1 && (reinterpret_cast<uintptr_t>(score) & 15) == 0));  // uniform
  if (ks.keys != nullptr) {
#pragma unroll
    for (int j = 0; j < kKeepRegs; ++j) keys[j] = (j < cnt) ? tm_orderable(sc[j]) : 0u;
  } else if (vec4 && cnt == 4) {
    const float4 f = *reinterpret_cast<const float4 *>(score + lo);
    keys[0] = tm_orderable(f.x); keys[1] = tm_orderable(f.y); keys[2] = tm_orderable(f.z); keys[3] = tm_orderable(f.w);
#pragma unroll
    for (int j = 4; j < kKeepRegs; ++j) keys[j] = 0u;
  } else {
#pragma unroll
    for (int j = 0; j < kKeepRegs; ++j) keys[j] = (j < cnt) ? tm_orderable(score[(lo + j) * ld]) : 0u;
  }
  uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int j = 0; j < kKeepRegs; ++j)
    if (j < cnt) {
      kmin = keys[j] < kmin ? keys[j] : kmin;
      kmax = keys[j] > kmax ? keys[j] : kmax;
    }
  kmin = tm_wave_min_u32(kmin);
  kmax = tm_wave_max_u32(kmax);
  if (lane == 0) { s_min[wave] = kmin; s_max[wave] = kmax; }
  __syncthreads();
  kmin = tm_wave_min_u32(lane < NW ? s_min[lane] : 0xffffffffu);
  kmax = tm_wave_max_u32(lane < NW ? s_max[lane] : 0u);
  uint32_t prefix = kmin & kmax, mask = 0u;  // common high bits
  int top = -1;
  if (kmin != kmax) {
    top = 31 - __builtin_clz(kmin ^ kmax);  // highest differing bit
    mask = (top == 31) ? 0u : (0xffffffffu << (top + 1));
    prefix &= mask;
  } else {
    mask = 0xffffffffu;
    prefix = kmin;
  }
  uint32_t rem = (uint32_t)n_keep;  // keys still to keep among those matching `prefix`
  int pass = 0;
  for (int hi_bit = top; hi_bit >= 0; hi_bit -= kKeepDigit, ++pass) {  // uniform trip count (<= 3)
    const int w = hi_bit + 1 < kKeepDigit ? hi_bit + 1 : kKeepDigit;
    const int shift = hi_bit + 1 - w;
    const uint32_t dmask = (1u << w) - 1u;
    uint32_t *h = hist[pass];
#pragma unroll
    for (int j = 0; j < kKeepRegs; ++j)
      if (j < cnt && (keys[j] & mask) == prefix) atomicAdd(&h[(keys[j] >> shift) & dmask], 1u);
    __syncthreads();
    // thread t owns bins BPT*r .. BPT*r+BPT-1 of rank r = NT-1-t (descending bin order across threads)
    const int r = NT - 1 - tid;
    uint32_t hb[BPT];
#pragma unroll
    for (int q4 = 0; q4 < BPT / 4; ++q4) {
      const uint4 hb4 = *reinterpret_cast<const uint4 *>(&h[BPT * r + 4 * q4]);
      hb[4 * q4] = hb4.x; hb[4 * q4 + 1] = hb4.y; hb[4 * q4 + 2] = hb4.z; hb[4 * q4 + 3] = hb4.w;
    }
    uint32_t tsum = 0;
#pragma unroll
    for (int b = 0; b < BPT; ++b) tsum += hb[b];
    const uint32_t inc = tm_wave_incl_scan(tsum);
    if (lane == 63) wave_tot[wave] = inc;
    __syncthreads();
    uint32_t above = wave_sum_u32(lane < wave ? wave_tot[lane] : 0u) + inc - tsum;  // keys in higher bins
#pragma unroll
    for (int b = BPT - 1; b >= 0; --b) {
      if (above < rem && rem <= above + hb[b]) s_sel = make_uint2(prefix | ((uint32_t)(BPT * r + b) << shift), rem - above);
      above += hb[b];
    }
    __syncthreads();
    // (the next pass writes wave_tot and s_sel only after its first barrier)
    const uint2 sel = s_sel;
    prefix = sel.x;
    rem = sel.y;
    mask |= dmask << shift;
  }
  const uint32_t T = prefix;  // the boundary key; `rem` copies of it are kept (>= 1)
  uint32_t eq = 0;
#pragma unroll
  for (int j = 0; j < kKeepRegs; ++j) eq += (j < cnt && keys[j] == T) ? 1u : 0u;
  const uint32_t inc = tm_wave_incl_scan(eq);
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  uint32_t rank = wave_sum_u32(lane < wave ? wave_tot[lane] : 0u) + inc - eq;  // copies of T at lower indices
  uint32_t packed = 0;
#pragma unroll
  for (int j = 0; j < kKeepRegs; ++j) {
    uint32_t k = 0;
    if (j < cnt) {
      if (keys[j] > T) {
        k = 1;
      } else if (keys[j] == T) {
        k = rank < rem ? 1u : 0u;
        ++rank;
      }
    }
    if (j < 4) packed |= k << (8 * j);
    if (!(vec4 && cnt == 4) && j < cnt) out[lo + j] = (uint8_t)k;
  }
  if (vec4 && cnt == 4 && (reinterpret_cast<uintptr_t>(out) & 3) == 0)
    *reinterpret_cast<uint32_t *>(out + lo) = packed;
  else if (vec4 && cnt == 4)
    for (int j = 0; j < 4; ++j) out[lo + j] = (uint8_t)((packed >> (8 * j)) & 1u);
}
