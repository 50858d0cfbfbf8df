// Internal helpers shared by the gfx950 kernels of the table-search path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tablemoe.h"

// ---------------------------------------------------------------------------
// error reporting (tm_runtime.hip)
// ---------------------------------------------------------------------------
int tm_fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void tm_clear_error();

#define TM_REQUIRE(cond, status, ...)          \
  do {                                         \
    if (!(cond)) return tm_fail(status, __VA_ARGS__); \
  } while (0)

#define TM_LAUNCH_CHECK(name)                                                          \
  do {                                                                                 \
    hipError_t e_ = hipGetLastError();                                                 \
    if (e_ != hipSuccess)                                                              \
      return tm_fail(TM_EHIP, "%s: kernel launch failed: %s", name, hipGetErrorString(e_)); \
  } while (0)

static inline hipStream_t tm_hip_stream(tm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

static inline int64_t tm_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// element types
// ---------------------------------------------------------------------------
__device__ __forceinline__ float tm_bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

__device__ __forceinline__ uint16_t tm_f32_to_bf16(float f) {
  // v_cvt_pk_bf16_f32: round half to even; a NaN keeps its sign and upper
  // payload bits with the quiet bit set, i.e. (bits >> 16) | 0x40.  Checked
  // against that software rule over all 2^32 fp32 bit patterns on gfx950.
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <int DT>
struct Elem;

template <>
struct Elem<TM_DT_F32> {
  using T = float;
  static constexpr int kBytes = 4;
  __device__ __forceinline__ static float to_f(T v) { return v; }
  __device__ __forceinline__ static T from_f(float f) { return f; }
};

template <>
struct Elem<TM_DT_F16> {
  using T = _Float16;
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static float to_f(T v) { return (float)v; }
  __device__ __forceinline__ static T from_f(float f) { return (_Float16)f; }
};

template <>
struct Elem<TM_DT_BF16> {
  using T = uint16_t;
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static float to_f(T v) { return tm_bf16_to_f32(v); }
  __device__ __forceinline__ static T from_f(float f) { return tm_f32_to_bf16(f); }
};

// Round an fp32 value to the element type and back (the rounding a torch op
// producing a tensor of that dtype applies).
template <int DT>
__device__ __forceinline__ float tm_round(float f) {
  return Elem<DT>::to_f(Elem<DT>::from_f(f));
}

// 16-byte vector load/store of consecutive elements, converted to/from fp32.
// 2-byte types move 8 elements, fp32 moves 4 (called twice for 8).
template <int DT>
__device__ __forceinline__ void tm_load8(const typename Elem<DT>::T *p, float (&v)[8]) {
  if constexpr (Elem<DT>::kBytes == 2) {
    uint4 r = *reinterpret_cast<const uint4 *>(p);
    const typename Elem<DT>::T *e = reinterpret_cast<const typename Elem<DT>::T *>(&r);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elem<DT>::to_f(e[i]);
  } else {
    float4 a = *reinterpret_cast<const float4 *>(p);
    float4 b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <int DT>
__device__ __forceinline__ void tm_store8(typename Elem<DT>::T *p, const float (&v)[8]) {
  if constexpr (Elem<DT>::kBytes == 2) {
    uint4 r;
    typename Elem<DT>::T *e = reinterpret_cast<typename Elem<DT>::T *>(&r);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = Elem<DT>::from_f(v[i]);
    *reinterpret_cast<uint4 *>(p) = r;
  } else {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4 *>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Streaming variants: non-temporal 16-byte accesses for data read or
// written once (kept out of the caches' working set); fp32 moves 8 elements
// as two of them.
typedef unsigned int tm_u32x4 __attribute__((ext_vector_type(4)));
typedef float tm_f32x4_nt __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ void tm_load8_nt(const typename Elem<DT>::T *p, float (&v)[8]) {
  if constexpr (Elem<DT>::kBytes == 2) {
    const tm_u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const tm_u32x4 *>(p));
    const typename Elem<DT>::T *e = reinterpret_cast<const typename Elem<DT>::T *>(&r);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elem<DT>::to_f(e[i]);
  } else {
    const tm_f32x4_nt a = __builtin_nontemporal_load(reinterpret_cast<const tm_f32x4_nt *>(p));
    const tm_f32x4_nt b = __builtin_nontemporal_load(reinterpret_cast<const tm_f32x4_nt *>(p + 4));
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <int DT>
__device__ __forceinline__ void tm_store8_nt(typename Elem<DT>::T *p, const float (&v)[8]) {
  if constexpr (Elem<DT>::kBytes == 2) {
    tm_u32x4 r;
    typename Elem<DT>::T *e = reinterpret_cast<typename Elem<DT>::T *>(&r);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = Elem<DT>::from_f(v[i]);
    __builtin_nontemporal_store(r, reinterpret_cast<tm_u32x4 *>(p));
  } else {
    __builtin_nontemporal_store(tm_f32x4_nt{v[0], v[1], v[2], v[3]}, reinterpret_cast<tm_f32x4_nt *>(p));
    __builtin_nontemporal_store(tm_f32x4_nt{v[4], v[5], v[6], v[7]}, reinterpret_cast<tm_f32x4_nt *>(p + 4));
  }
}

// True when a pointer is aligned for tm_load8/tm_store8 of this type.
static inline bool tm_aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define TM_DISPATCH_DTYPE(dtype, DT, ...)                                     \
  [&]() -> int {                                                              \
    switch (dtype) {                                                          \
      case TM_DT_F32: { constexpr int DT = TM_DT_F32; return __VA_ARGS__(); } \
      case TM_DT_F16: { constexpr int DT = TM_DT_F16; return __VA_ARGS__(); } \
      case TM_DT_BF16: { constexpr int DT = TM_DT_BF16; return __VA_ARGS__(); } \
      default: return tm_fail(TM_EINVAL_DTYPE, "unsupported dtype tag %d", (int)dtype); \
    }                                                                         \
  }()

// ---------------------------------------------------------------------------
// ordering keys
// ---------------------------------------------------------------------------
// Monotone map of fp32 to uint32: a < b (as floats, no NaN) <=> key(a) < key(b).
__device__ __forceinline__ uint32_t tm_orderable(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float tm_from_orderable(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// A packed search key (orderable(dp) << 32 | centroid) of one query turned
// into its output: dp = -2 * (q.c - |c|^2 / 2) for L2 (distance |q|^2 + dp,
// clamped at 0), dp = -q.c for DOT (score -dp).  Key ~0 (no candidate) gives
// index -1 and the worst distance.
__device__ __forceinline__ float tm_key_to_dist(uint64_t key, float qn, bool l2, int64_t &idx) {
  if (key == ~0ull) {
    idx = -1;
    return l2 ? __builtin_huge_valf() : -__builtin_huge_valf();
  }
  const float dp = tm_from_orderable((uint32_t)(key >> 32));
  idx = (int64_t)(uint32_t)key;
  return l2 ? fmaxf(qn + dp, 0.f) : -dp;
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
// DPP (data-parallel primitives, gfx9): row_shr:n reads lane i-n of the same
// 16-lane row, row_bcast:15 / row_bcast:31 read lane 15 / 31 of the previous
// row(s).  Lanes whose source is outside the row keep `old`.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t tm_dpp(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, ROW_MASK, 0xF, false);
}
// Inclusive prefix sum over the wave (11 VALU ops, no LDS).
__device__ __forceinline__ uint32_t tm_wave_incl_scan(uint32_t v) {
  v += tm_dpp<0x111>(0u, v);        // row_shr:1
  v += tm_dpp<0x112>(0u, v);        // row_shr:2
  v += tm_dpp<0x114>(0u, v);        // row_shr:4
  v += tm_dpp<0x118>(0u, v);        // row_shr:8
  v += tm_dpp<0x142, 0xA>(0u, v);   // row_bcast:15 into rows 1, 3
  v += tm_dpp<0x143, 0xC>(0u, v);   // row_bcast:31 into rows 2, 3
  return v;
}
// Minimum / maximum over the wave, returned in every lane.
__device__ __forceinline__ uint32_t tm_wave_min_u32(uint32_t v) {
  v = min(v, tm_dpp<0x111>(v, v));
  v = min(v, tm_dpp<0x112>(v, v));
  v = min(v, tm_dpp<0x114>(v, v));
  v = min(v, tm_dpp<0x118>(v, v));
  v = min(v, tm_dpp<0x142, 0xA>(v, v));
  v = min(v, tm_dpp<0x143, 0xC>(v, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t tm_wave_max_u32(uint32_t v) {
  v = max(v, tm_dpp<0x111>(v, v));
  v = max(v, tm_dpp<0x112>(v, v));
  v = max(v, tm_dpp<0x114>(v, v));
  v = max(v, tm_dpp<0x118>(v, v));
  v = max(v, tm_dpp<0x142, 0xA>(v, v));
  v = max(v, tm_dpp<0x143, 0xC>(v, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ float tm_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float tm_wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// (value, index) arg-max with ties to the lower index.
__device__ __forceinline__ void tm_wave_argmax(float &v, int &i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, 64);
    int oi = __shfl_xor(i, o, 64);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
  }
}
__device__ __forceinline__ uint64_t tm_wave_min_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t ov = __shfl_xor(v, o, 64);
    v = ov < v ? ov : v;
  }
  return v;
}
