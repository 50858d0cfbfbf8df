// a4: projection of hidden states into the PCA space (+ optional L2 normalise).
//
// q[b] = dtype(x[b] @ P_m + bias_m), one rounding after fp32 accumulation,
// as torch.addmm in the model dtype (table_moe/cache_engine/search.py:484,492).
// Normalisation follows _normalize_last_dim (search.py:12-21): the norm is
// rounded to dtype, the quotient is an fp32 division rounded to dtype, and
// rows with norm <= eps become zero.
//
// MFMA path (F16/BF16): a workgroup owns 32 token rows and all `DIM` output
// columns.  Hidden is walked in 64-wide stages: the x tile is staged in LDS
// row-major, the P tile transposed (k-contiguous per output column) so both
// MFMA operands are 16-byte LDS reads.  Tiles that mix modalities run one
// pass per modality and keep each row's own result.
#include "tm_mfma.h"

namespace {

constexpr int kBM = 32;
constexpr int kBK = 64;
constexpr int kPad = 8;
constexpr int kThreads = 256;

template <int DT, int DIM, bool PK>
__global__ __launch_bounds__(kThreads) void project_mfma_kernel(
    const typename Elem<DT>::T *__restrict__ x, int64_t n, int hidden, int64_t ld_x,
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ pv,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ pt,
    const typename Elem<DT>::T *__restrict__ bt, int64_t ps_h, int64_t ps_d, int normalize,
    float eps, typename Elem<DT>::T *__restrict__ q, int64_t ld_q, float *__restrict__ q_sqnorm) {
  using T = typename Elem<DT>::T;
  constexpr int NBLK = (kBM / 16) * (DIM / 16);          // 16x16 output blocks
  constexpr int PER_WAVE = (NBLK + 3) / 4;
  __shared__ __attribute__((aligned(16))) T xs[kBM][kBK + kPad];
  __shared__ __attribute__((aligned(16))) T ps[DIM][kBK + kPad];
  __shared__ float qs[kBM][DIM + 1];
  __shared__ uint8_t row_mod[kBM];
  __shared__ int mod_present[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * kBM;

  if (tid < 2) mod_present[tid] = 0;
  __syncthreads();
  if (tid < kBM) {
    int64_t r = row0 + tid;
    uint8_t m = 0;
    if (r < n) {
      m = (is_vision == nullptr || is_vision[r]) ? 0 : 1;
      atomicOr(&mod_present[m], 1);
    }
    row_mod[tid] = m;
  }
  __syncthreads();

  for (int m = 0; m < 2; ++m) {
    if (!mod_present[m]) continue;  // uniform across the workgroup
    const T *P = (m == 0) ? pv : pt;
    const T *bias = (m == 0) ? bv : bt;

    tm_f32x4 acc[PER_WAVE];
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) acc[i] = tm_f32x4{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < hidden; k0 += kBK) {
      // x tile: 32 rows x 64 elements = 256 chunks of 8.
      {
        const int r = tid >> 3, c8 = (tid & 7) * 8;
        const int64_t gr = row0 + r;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (gr < n && k0 + c8 < hidden)
          v = *reinterpret_cast<const uint4 *>(x + gr * ld_x + k0 + c8);
        *reinterpret_cast<uint4 *>(&xs[r][c8]) = v;
      }
      // P tile, transposed into ps[j][h].
      if constexpr (PK) {
        for (int ci = tid; ci < DIM * (kBK / 8); ci += kThreads) {
          const int j = ci / (kBK / 8), h0 = (ci % (kBK / 8)) * 8;
          uint4 v = make_uint4(0, 0, 0, 0);
          if (k0 + h0 < hidden) v = *reinterpret_cast<const uint4 *>(P + (int64_t)j * ps_d + k0 + h0);
          *reinterpret_cast<uint4 *>(&ps[j][h0]) = v;
        }
      } else {
        for (int ci = tid; ci < kBK * (DIM / 8); ci += kThreads) {
          const int h = ci / (DIM / 8), j0 = (ci % (DIM / 8)) * 8;
          uint4 v = make_uint4(0, 0, 0, 0);
          if (k0 + h < hidden) v = *reinterpret_cast<const uint4 *>(P + (int64_t)(k0 + h) * ps_h + j0);
          const T *e = reinterpret_cast<const T *>(&v);
#pragma unroll
          for (int i = 0; i < 8; ++i) ps[j0 + i][h] = e[i];
        }
      }
      __syncthreads();
#pragma unroll
      for (int ks = 0; ks < kBK / 32; ++ks) {
        const int kk = ks * 32 + 8 * (lane >> 4);
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
          const int b = wave + 4 * i;
          if (b < NBLK) {
            const int rb = b % (kBM / 16), cb = b / (kBM / 16);
            uint4 a = *reinterpret_cast<const uint4 *>(&xs[rb * 16 + (lane & 15)][kk]);
            uint4 bb = *reinterpret_cast<const uint4 *>(&ps[cb * 16 + (lane & 15)][kk]);
            acc[i] = tm_mfma16x16x32<DT>(a, bb, acc[i]);
          }
        }
      }
      __syncthreads();
    }
    // bias + rounding; keep the rows of this modality.
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int b = wave + 4 * i;
      if (b < NBLK) {
        const int rb = b % (kBM / 16), cb = b / (kBM / 16);
        const int col = cb * 16 + (lane & 15);
        const float bcol = Elem<DT>::to_f(bias[col]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb * 16 + 4 * (lane >> 4) + r;
          if (row_mod[row] == m) qs[row][col] = tm_round<DT>(acc[i][r] + bcol);
        }
      }
    }
    __syncthreads();
  }

  // Row epilogue: 8 threads per row, DIM/8 columns each.
  constexpr int CPT = DIM / 8;
  const int row = tid >> 3, part = tid & 7;
  const int64_t gr = row0 + row;
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    float v = qs[row][part * CPT + c];
    ss = fmaf(v, v, ss);
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  ss += __shfl_xor(ss, 4, 64);
  float scale_den = 1.f;
  bool zero_row = false;
  if (normalize) {
    const float norm = tm_round<DT>(sqrtf(ss));
    const float eps_dt = tm_round<DT>(eps);
    zero_row = !(norm > eps_dt);
    scale_den = fmaxf(norm, eps_dt);
  }
  float ss_out = 0.f;
  if (gr < n) {
    T *dst = q + gr * ld_q + part * CPT;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      float v = qs[row][part * CPT + c];
      if (normalize) v = zero_row ? 0.f : tm_round<DT>(v / scale_den);
      ss_out = fmaf(v, v, ss_out);
      dst[c] = Elem<DT>::from_f(v);
    }
  }
  if (q_sqnorm != nullptr) {
    ss_out += __shfl_xor(ss_out, 1, 64);
    ss_out += __shfl_xor(ss_out, 2, 64);
    ss_out += __shfl_xor(ss_out, 4, 64);
    if (part == 0 && gr < n) q_sqnorm[gr] = ss_out;
  }
}

// Generic path (any dtype, dim <= 256): one thread per output element,
// sequential fp32 accumulation over hidden.  Every thread reaches every
// barrier; inactive threads carry zeros.
template <int DT>
__global__ __launch_bounds__(kThreads) void project_scalar_kernel(
    const typename Elem<DT>::T *__restrict__ x, int64_t n, int hidden, int64_t ld_x,
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ pv,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ pt,
    const typename Elem<DT>::T *__restrict__ bt, int64_t ps_h, int64_t ps_d, int dim, int normalize,
    float eps, typename Elem<DT>::T *__restrict__ q, int64_t ld_q, float *__restrict__ q_sqnorm) {
  using T = typename Elem<DT>::T;
  __shared__ float vals[kThreads];
  __shared__ float rowss[kThreads];
  const int rows_per_block = kThreads / dim;
  const int tid = threadIdx.x;
  const int lr = tid / dim, col = tid % dim;
  const int64_t row = (int64_t)blockIdx.x * rows_per_block + lr;
  const bool active = lr < rows_per_block && row < n;
  float v = 0.f;
  if (active) {
    const bool vis = is_vision == nullptr || is_vision[row];
    const T *P = vis ? pv : pt;
    const T *bias = vis ? bv : bt;
    const T *xr = x + row * ld_x;
    float acc = 0.f;
    for (int h = 0; h < hidden; ++h)
      acc = fmaf(Elem<DT>::to_f(xr[h]), Elem<DT>::to_f(P[(int64_t)h * ps_h + (int64_t)col * ps_d]), acc);
    v = tm_round<DT>(acc + Elem<DT>::to_f(bias[col]));
  }
  vals[tid] = v;
  __syncthreads();
  if (active && col == 0) {
    float ss = 0.f;
    for (int c = 0; c < dim; ++c) ss = fmaf(vals[tid + c], vals[tid + c], ss);
    rowss[lr] = ss;
  }
  __syncthreads();
  if (active && normalize) {
    const float norm = tm_round<DT>(sqrtf(rowss[lr]));
    const float eps_dt = tm_round<DT>(eps);
    v = (norm > eps_dt) ? tm_round<DT>(v / fmaxf(norm, eps_dt)) : 0.f;
  }
  if (active) q[row * ld_q + col] = Elem<DT>::from_f(v);
  __syncthreads();
  vals[tid] = v;
  __syncthreads();
  if (active && col == 0 && q_sqnorm != nullptr) {
    float ss = 0.f;
    for (int c = 0; c < dim; ++c) ss = fmaf(vals[tid + c], vals[tid + c], ss);
    q_sqnorm[row] = ss;
  }
}

template <int DT>
int launch_project(const void *x, int64_t n, int hidden, int64_t ld_x, const uint8_t *is_vision,
                   const void *pv, const void *bv, const void *pt, const void *bt, int64_t ps_h,
                   int64_t ps_d, int dim, int normalize, float eps, void *q, int64_t ld_q,
                   float *q_sqnorm, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const T *X = static_cast<const T *>(x);
  const T *PV = static_cast<const T *>(pv), *BV = static_cast<const T *>(bv);
  const T *PT = static_cast<const T *>(pt ? pt : pv), *BT = static_cast<const T *>(pt ? bt : bv);
  T *Q = static_cast<T *>(q);
  const bool pk = (ps_h == 1);
  bool mfma_ok = DT != TM_DT_F32 && (hidden % 8 == 0) && (dim == 16 || dim == 32 || dim == 64 ||
                                                           dim == 128 || dim == 256);
  if (mfma_ok) {
    const int E = Elem<DT>::kBytes;
    mfma_ok = tm_aligned16(x) && ((ld_x * E) % 16 == 0) && tm_aligned16(pv) && tm_aligned16(PT) &&
              (pk ? ((ps_d * E) % 16 == 0) : ((ps_h * E) % 16 == 0));
  }
  if (mfma_ok) {
    dim3 grid((unsigned)tm_cdiv(n, kBM)), block(kThreads);
#define TM_PROJ_LAUNCH(D)                                                                        \
  if (dim == D) {                                                                                \
    if (pk)                                                                                      \
      hipLaunchKernelGGL((project_mfma_kernel<DT, D, true>), grid, block, 0, stream, X, n, hidden, \
                         ld_x, is_vision, PV, BV, PT, BT, ps_h, ps_d, normalize, eps, Q, ld_q,   \
                         q_sqnorm);                                                              \
    else                                                                                         \
      hipLaunchKernelGGL((project_mfma_kernel<DT, D, false>), grid, block, 0, stream, X, n,      \
                         hidden, ld_x, is_vision, PV, BV, PT, BT, ps_h, ps_d, normalize, eps, Q,  \
                         ld_q, q_sqnorm);                                                        \
  }
    TM_PROJ_LAUNCH(16)
    TM_PROJ_LAUNCH(32)
    TM_PROJ_LAUNCH(64)
    TM_PROJ_LAUNCH(128)
    TM_PROJ_LAUNCH(256)
#undef TM_PROJ_LAUNCH
    TM_LAUNCH_CHECK("tm_project");
    return TM_OK;
  }
  const int rows_per_block = kThreads / dim;
  dim3 grid((unsigned)tm_cdiv(n, rows_per_block)), block(kThreads);
  hipLaunchKernelGGL((project_scalar_kernel<DT>), grid, block, 0, stream, X, n, hidden, ld_x,
                     is_vision, PV, BV, PT, BT, ps_h, ps_d, dim, normalize, eps, Q, ld_q, q_sqnorm);
  TM_LAUNCH_CHECK("tm_project");
  return TM_OK;
}

}  // namespace

extern "C" int tm_project(int32_t dtype, const void *x, int64_t n_tokens, int32_t hidden,
                          int64_t ld_x, const uint8_t *is_vision, const void *proj_vis,
                          const void *bias_vis, const void *proj_txt, const void *bias_txt,
                          int64_t ps_h, int64_t ps_d, int32_t dim, int32_t normalize, float eps,
                          void *q_out, int64_t ld_q, float *q_sqnorm, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && hidden > 0 && dim > 0 && dim <= 256, TM_EINVAL_SHAPE,
             "tm_project: bad sizes n=%lld hidden=%d dim=%d", (long long)n_tokens, hidden, dim);
  TM_REQUIRE(ld_x >= hidden && ld_q >= dim, TM_EINVAL_SHAPE, "tm_project: bad row strides");
  TM_REQUIRE(ps_h == 1 || ps_d == 1, TM_EINVAL_SHAPE,
             "tm_project: projection needs a unit stride along hidden or dim");
  TM_REQUIRE(proj_vis && bias_vis && q_out && (n_tokens == 0 || x), TM_EINVAL_ARG,
             "tm_project: null pointer");
  TM_REQUIRE((proj_txt == nullptr) == (bias_txt == nullptr), TM_EINVAL_ARG,
             "tm_project: proj_txt and bias_txt must both be set or both be NULL");
  if (n_tokens == 0) return TM_OK;
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    return launch_project<DT>(x, n_tokens, hidden, ld_x, is_vision, proj_vis, bias_vis, proj_txt,
                              bias_txt, ps_h, ps_d, dim, normalize, eps, q_out, ld_q, q_sqnorm,
                              tm_hip_stream(stream));
  });
}
