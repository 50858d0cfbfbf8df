// Router top-k softmax for one token held by an 8-lane group: the device
// routine shared by the router kernel and the fused projection launch.
#pragma once

#include "tm_common.h"

// Exchange within 8-lane groups by DPP (VALU, no LDS round trip): quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror (lane i <-> 7-i).  After the
// three steps of a symmetric reduction every lane of the group holds the result.
template <int CTRL>
__device__ __forceinline__ float tm_g8f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int tm_g8i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kG8Steps[3] = {0xB1, 0x4E, 0x141};

// Rows of 8*VPL experts (VPL % 4 == 0): lane `sub` (0..7) of the token's
// group holds the contiguous experts [sub*VPL, sub*VPL + VPL), loaded as
// VPL/4 unconditional 16-byte loads (the group reads the row as one
// contiguous span; a row past n re-reads the last row and writes nothing).
// fp32 softmax (max, exp, sum, divide), then top_k rounds of an arg-max whose
// ties go to the lower expert id; the winner is masked out after each round.
// The group's lane 0 keeps the winners (top_k <= KM) and writes them once.
// Every lane of the wave must call this (the reductions are 8-lane DPP exchanges).
// tm_route_compute leaves the winners in every lane of the group (kw, ki;
// entries past top_k unset) and their sum in wsum; tm_route_token also writes
// them.
template <int VPL, int KM>
__device__ __forceinline__ void tm_route_compute(const float *__restrict__ logits, int64_t n, int64_t ld, int top_k,
                                                 int64_t row, int sub, float (&kw)[KM], int (&ki)[KM],
                                                 float &wsum) {
  static_assert(VPL % 4 == 0, "whole 16-byte loads");
  const bool valid = row < n;
  const float *lr = logits + (valid ? row : n - 1) * ld + sub * VPL;
  float v[VPL];
#pragma unroll
  for (int j = 0; j < VPL / 4; ++j) {
    const float4 f = *reinterpret_cast<const float4 *>(lr + 4 * j);
    v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
  }
  float mx = v[0];
#pragma unroll
  for (int j = 1; j < VPL; ++j) mx = fmaxf(mx, v[j]);
  mx = fmaxf(mx, tm_g8f<kG8Steps[0]>(mx));
  mx = fmaxf(mx, tm_g8f<kG8Steps[1]>(mx));
  mx = fmaxf(mx, tm_g8f<kG8Steps[2]>(mx));
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    v[j] = expf(v[j] - mx);
    sum += v[j];
  }
  sum += tm_g8f<kG8Steps[0]>(sum);
  sum += tm_g8f<kG8Steps[1]>(sum);
  sum += tm_g8f<kG8Steps[2]>(sum);
#pragma unroll
  for (int j = 0; j < VPL; ++j) v[j] = v[j] / sum;
  wsum = 0.f;
  for (int k = 0; k < top_k; ++k) {
    float bv = -2.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (v[j] > bv) { bv = v[j]; bi = sub * VPL + j; }
    }
    {
      float ov = tm_g8f<kG8Steps[0]>(bv);
      int oi = tm_g8i<kG8Steps[0]>(bi);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      ov = tm_g8f<kG8Steps[1]>(bv);
      oi = tm_g8i<kG8Steps[1]>(bi);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      ov = tm_g8f<kG8Steps[2]>(bv);
      oi = tm_g8i<kG8Steps[2]>(bi);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (bi / VPL == sub) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
        if (j == bi % VPL) v[j] = -1.f;
    }
#pragma unroll
    for (int u = 0; u < KM; ++u)
      if (u == k) { kw[u] = bv; ki[u] = bi; }
    wsum += bv;
  }
}

template <int VPL, int KM>
__device__ __forceinline__ void tm_route_token(const float *__restrict__ logits, int64_t n, int64_t ld, int top_k,
                                               int renorm, float *__restrict__ out_w,
                                               int64_t *__restrict__ out_ids, int64_t row, int sub) {
  float kw[KM];
  int ki[KM];
  float wsum;
  tm_route_compute<VPL, KM>(logits, n, ld, top_k, row, sub, kw, ki, wsum);
  const bool valid = row < n;
  if (sub == 0 && valid) {
    const float d = renorm ? fmaxf(wsum, 1e-20f) : 1.f;
    float *ow = out_w + row * top_k;
    int64_t *oi = out_ids + row * top_k;
#pragma unroll
    for (int u = 0; u < KM; ++u) {
      if (u < top_k) {
        ow[u] = renorm ? kw[u] / d : kw[u];
        oi[u] = ki[u];
      }
    }
  }
}
