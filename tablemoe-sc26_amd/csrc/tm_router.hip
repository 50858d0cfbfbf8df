// a1: router softmax + top-k (replaces the qwen_topk_softmax extension,
// table_moe/ops/qwen_topk_softmax.py:122-154).
//
// fp32 softmax (max, exp, sum, divide), then top_k rounds of an arg-max whose
// ties go to the lower expert id; the winner is masked out after each round.
// Rows of up to 256 experts use 8 lanes per token; wider rows one wave.
#include "tm_route_dev.h"

namespace {

constexpr int kThreads = 256;

template <int VPL>
__global__ __launch_bounds__(kThreads) void topk_softmax_kernel(const float *__restrict__ logits,
                                                                int64_t n, int n_exp, int64_t ld,
                                                                int top_k, int renorm,
                                                                float *__restrict__ out_w,
                                                                int64_t *__restrict__ out_ids) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= n) return;  // whole wave
  const float *lr = logits + row * ld;
  float v[VPL];
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = j * 64 + lane;
    v[j] = (e < n_exp) ? lr[e] : -__builtin_huge_valf();
    mx = fmaxf(mx, v[j]);
  }
  mx = tm_wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = j * 64 + lane;
    v[j] = (e < n_exp) ? expf(v[j] - mx) : 0.f;
    sum += v[j];
  }
  sum = tm_wave_sum(sum);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = j * 64 + lane;
    v[j] = (e < n_exp) ? v[j] / sum : -1.f;
  }
  float wsum = 0.f;
  float *ow = out_w + row * top_k;
  int64_t *oi = out_ids + row * top_k;
  for (int k = 0; k < top_k; ++k) {
    float bv = -2.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (v[j] > bv) { bv = v[j]; bi = j * 64 + lane; }
    }
    tm_wave_argmax(bv, bi);
    if ((bi & 63) == lane) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
        if (j == (bi >> 6)) v[j] = -1.f;
    }
    if (lane == 0) {
      ow[k] = bv;
      oi[k] = bi;
    }
    wsum += bv;
  }
  if (renorm && lane == 0) {
    const float d = fmaxf(wsum, 1e-20f);
    for (int k = 0; k < top_k; ++k) ow[k] = ow[k] / d;
  }
}

// Narrow rows (E <= 256): 8 lanes per token, 8 tokens per wave.  Lane `sub`
// holds experts sub, sub+8, ... (coalesced across the row's lanes); the
// reductions and each top-k round use 3 butterfly steps inside the 8-lane
// group.
template <int VPL>
__global__ __launch_bounds__(kThreads) void topk_softmax_group_kernel(const float *__restrict__ logits,
                                                                      int64_t n, int n_exp, int64_t ld,
                                                                      int top_k, int renorm,
                                                                      float *__restrict__ out_w,
                                                                      int64_t *__restrict__ out_ids) {
  const int lane = threadIdx.x & 63;
  const int sub = lane & 7;
  const int64_t row = ((int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)) * 8 + (lane >> 3);
  const bool valid = row < n;  // invalid rows still join the group shuffles
  const float *lr = logits + (valid ? row : 0) * ld;
  float v[VPL];
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = j * 8 + sub;
    v[j] = (valid && e < n_exp) ? lr[e] : -__builtin_huge_valf();
    mx = fmaxf(mx, v[j]);
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = j * 8 + sub;
    v[j] = (e < n_exp && valid) ? expf(v[j] - mx) : 0.f;
    sum += v[j];
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o, 64);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = j * 8 + sub;
    v[j] = (e < n_exp && valid) ? v[j] / sum : -1.f;
  }
  float wsum = 0.f;
  float *ow = out_w + (valid ? row : 0) * top_k;
  int64_t *oi = out_ids + (valid ? row : 0) * top_k;
  for (int k = 0; k < top_k; ++k) {
    float bv = -2.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (v[j] > bv) { bv = v[j]; bi = j * 8 + sub; }
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi2 = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi2 < bi)) { bv = ov; bi = oi2; }
    }
    if ((bi & 7) == sub) {
#pragma unroll
      for (int j = 0; j < VPL; ++j)
        if (j == (bi >> 3)) v[j] = -1.f;
    }
    if (sub == 0 && valid) {
      ow[k] = bv;
      oi[k] = bi;
    }
    wsum += bv;
  }
  if (renorm && sub == 0 && valid) {
    const float d = fmaxf(wsum, 1e-20f);
    for (int k = 0; k < top_k; ++k) ow[k] = ow[k] / d;
  }
}

// Rows of 64, 128 or 256 experts with 16-byte aligned rows: tm_route_token,
// 8 tokens per 64-thread workgroup.
template <int VPL, int KM>
__global__ __launch_bounds__(64) void topk_softmax_vec_kernel(const float *__restrict__ logits, int64_t n, int64_t ld,
                                                             int top_k, int renorm, float *__restrict__ out_w,
                                                             int64_t *__restrict__ out_ids) {
  const int lane = threadIdx.x & 63;
  tm_route_token<VPL, KM>(logits, n, ld, top_k, renorm, out_w, out_ids, (int64_t)blockIdx.x * 8 + (lane >> 3),
                          lane & 7);
}

}  // namespace

extern "C" int tm_topk_softmax(const float *logits, int64_t n_tokens, int32_t n_experts,
                               int64_t ld_logits, int32_t top_k, int32_t renormalize,
                               float *out_weights, int64_t *out_ids, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && n_experts >= 1 && n_experts <= 4096 && ld_logits >= n_experts,
             TM_EINVAL_SHAPE, "tm_topk_softmax: bad sizes (experts %d)", n_experts);
  TM_REQUIRE(top_k >= 1 && top_k <= 32 && top_k <= n_experts, TM_EINVAL_SHAPE,
             "tm_topk_softmax: top_k %d out of range", top_k);
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(logits && out_weights && out_ids, TM_EINVAL_ARG, "tm_topk_softmax: null pointer");
  dim3 grid((unsigned)tm_cdiv(n_tokens, kThreads / 64)), block(kThreads);
  hipStream_t s = tm_hip_stream(stream);
  // one wave (8 tokens) per workgroup: spreads small batches over more CUs
  const dim3 ggrid((unsigned)tm_cdiv(n_tokens, 8)), gblock(64);
  const bool vec4 = tm_aligned16(logits) && ld_logits % 4 == 0;
#define TM_ROUTER_VEC(E_, VPL_)                                                                                \
  if (vec4 && n_experts == E_) {                                                                              \
    if (top_k <= 8)                                                                                           \
      hipLaunchKernelGGL((topk_softmax_vec_kernel<VPL_, 8>), ggrid, gblock, 0, s, logits, n_tokens, ld_logits,  \
                         top_k, renormalize, out_weights, out_ids);                                          \
    else                                                                                                      \
      hipLaunchKernelGGL((topk_softmax_vec_kernel<VPL_, 32>), ggrid, gblock, 0, s, logits, n_tokens, ld_logits, \
                         top_k, renormalize, out_weights, out_ids);                                          \
    TM_LAUNCH_CHECK("tm_topk_softmax");                                                                       \
    return TM_OK;                                                                                             \
  }
  TM_ROUTER_VEC(64, 8)
  TM_ROUTER_VEC(128, 16)
  TM_ROUTER_VEC(256, 32)
#undef TM_ROUTER_VEC
  if (n_experts <= 64)
    hipLaunchKernelGGL(topk_softmax_group_kernel<8>, ggrid, gblock, 0, s, logits, n_tokens, n_experts, ld_logits, top_k, renormalize, out_weights, out_ids);
  else if (n_experts <= 128)
    hipLaunchKernelGGL(topk_softmax_group_kernel<16>, ggrid, gblock, 0, s, logits, n_tokens, n_experts, ld_logits, top_k, renormalize, out_weights, out_ids);
  else if (n_experts <= 256)
    hipLaunchKernelGGL(topk_softmax_group_kernel<32>, ggrid, gblock, 0, s, logits, n_tokens, n_experts, ld_logits, top_k, renormalize, out_weights, out_ids);
  else if (n_experts <= 1024)
    hipLaunchKernelGGL(topk_softmax_kernel<16>, grid, block, 0, s, logits, n_tokens, n_experts, ld_logits, top_k, renormalize, out_weights, out_ids);
  else
    hipLaunchKernelGGL(topk_softmax_kernel<64>, grid, block, 0, s, logits, n_tokens, n_experts, ld_logits, top_k, renormalize, out_weights, out_ids);
  TM_LAUNCH_CHECK("tm_topk_softmax");
  return TM_OK;
}
