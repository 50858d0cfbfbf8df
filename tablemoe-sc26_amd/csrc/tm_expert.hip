// Recompute path: the SwiGLU expert MLP of the slots that are not reused,
// grouped over experts, on bf16/fp16 matrix cores.
//
// Replaces the reference's per-expert loop (models/qwen3_vl_moe/
// cached_layers.py:431-437: index_select the expert's tokens, run the expert,
// scatter into collected[token, slot]) and its CUTLASS expert MLP
// (ops/csrc/fp16_fused_expert/fp16_fused_moe_mlp.cu:107-274 with the SiLU-mul
// epilogue of fp16_epilogue_utils.h:51-125):
//   g = dtype(x W1^T)                      (fp32 accumulation, one rounding)
//   f = dtype(silu(g) * (x W3^T))          (up projection unrounded, silu in fp32)
//   y = dtype(f W2^T)
//
// tm_group_slots (one workgroup) buckets the recomputed (token, slot) pairs
// by expert: per-expert counts in LDS, offsets, one row per pair (token and
// the element offset of its output row in the slot layout), and the list of
// BM-row tiles of every expert.  The order of rows inside an expert is that
// of LDS atomics; every output row is computed the same way wherever its row
// sits in a tile, so results do not depend on it.
//
// grouped_gemm_kernel computes one BM x BN tile C = A B^T of one expert:
// A rows gathered (token rows of x, or the grouped rows of the intermediate),
// B rows k-contiguous (nn.Linear weights [out, in]), K in BK-wide stages.
// Stages move global -> LDS by direct loads, three in flight (16-byte chunks
// XOR-swizzled by row, so the operand reads of 32 rows spread over the
// banks); one barrier per stage.  Four waves own 128 x 64 quadrants (4 x 2
// blocks of v_mfma_f32_32x32x16).  Up mode multiplies W1 and W3 against the same A
// fragments and applies the SiLU-mul epilogue; down mode writes each row to
// its slot of the output.
#include "tm_internal.h"
#include "tm_dma.h"
#include "tm_mfma.h"

namespace {

constexpr int BM = 256, BN = 128, BK = 32, kThreads = 256, kRing = 4;
constexpr int kCPR = BK / 8;                 // 16-byte chunks per tile row
constexpr int kAStage = BM * kCPR;           // A slots (16 bytes) per stage
constexpr int kBStage = BN * kCPR;           // slots of each B per stage
constexpr int kADma = kAStage / 64 / 4;      // A loads per wave per stage (4)
constexpr int kBDma = kBStage / 64 / 4;      // loads of each B per wave per stage (2)
constexpr int kMI = 4, kNI = 2;              // 32 x 32 blocks per wave: 128 rows x 64 columns

enum { kModeUp = 0, kModeDown = 1 };

// Slot of (row, 16-byte chunk kc) in a stage.  A row is 64 bytes, so two
// rows share one 128-byte line of banks; XOR-ing the chunk with (row / 2) % 4
// puts the 8 rows of a line group on 8 distinct 16-byte bank groups, and an
// operand read (one chunk of 32 consecutive rows) is conflict-free.
__device__ __forceinline__ int swz_chunk(int row, int kc) { return kc ^ ((row >> 1) & (kCPR - 1)); }
__device__ __forceinline__ int swz(int row, int kc) { return row * kCPR + swz_chunk(row, kc); }

// Tile source: the grouped tile list (tiles != nullptr: [0] rows, [1] tiles,
// then tile_expert[t_max], tile_row0[t_max]) or one dense expert of `rows`.
struct TileSrc {
  const int32_t *tiles;
  const int32_t *expert_offsets;
  int64_t t_max;
  int32_t rows;
};

// One BM x BN tile, 4 waves in a 2 x 2 grid of 128 x 64 quadrants (one wave
// per SIMD, accumulators in the AGPRs).  Operands move global -> LDS by
// direct loads into a kRing-stage ring, kRing - 1 stages in flight: at step i
// a wave waits for its own loads of stage i, the barrier makes every wave's
// loads of stage i visible (and retires every wave's reads of stage i - 1),
// then the loads of stage i + 3 go into that freed slot and stage i is
// multiplied.  Lane l of a load fills slot p0 + l; it reads the global chunk
// that belongs there (the inverse of the swizzle).
template <int DT, int NB, int MODE>
__global__ __launch_bounds__(kThreads, 1) void grouped_gemm_kernel(
    const typename Elem<DT>::T *__restrict__ A, int64_t lda, const int32_t *__restrict__ a_rows,
    const typename Elem<DT>::T *__restrict__ B0, const typename Elem<DT>::T *__restrict__ B1, int64_t b_expert,
    int K, int n_tiles, TileSrc ts, typename Elem<DT>::T *__restrict__ C, int64_t ldc,
    const int64_t *__restrict__ c_rows, const typename Elem<DT>::T *__restrict__ addend, int64_t ld_add) {
  using T = typename Elem<DT>::T;
  constexpr int kStage = kAStage + NB * kBStage;
  constexpr int kDma = kADma + NB * kBDma;  // loads per wave per stage
  __shared__ uint4 lds[kRing * kStage];

  // Block b runs on XCD b % 8 (the dispatcher's round robin): the n_tiles
  // column tiles of row tile y get ids 8 apart, so they share one XCD and its
  // L2 copy of the tile's A rows.
  const int64_t b = blockIdx.x;
  const int64_t slot = b >> 3;
  const int64_t y = (slot / n_tiles) * 8 + (b & 7);
  const int n0 = (int)(slot % n_tiles) * BN;
  int e, r0, r_end;
  if (ts.tiles != nullptr) {
    if (y >= ts.t_max || y >= ts.tiles[1]) return;  // uniform: past the last tile
    e = ts.tiles[2 + y];
    r0 = ts.tiles[2 + ts.t_max + y];
    r_end = ts.expert_offsets[e + 1];
  } else {
    e = 0;
    r0 = (int)y * BM;
    if (r0 >= ts.rows) return;
    r_end = ts.rows;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Global source of each of this lane's loads (stage 0); stage s adds s * BK.
  const T *a_src[kADma];
  const T *b_src[NB][kBDma];
#pragma unroll
  for (int j = 0; j < kADma; ++j) {
    const int p = (wave * kADma + j) * 64 + lane;
    const int row = p / kCPR, kc = swz_chunk(row, p % kCPR);  // the swizzle is its own inverse
    int gr = r0 + row;
    gr = gr < r_end ? gr : r_end - 1;  // rows past the expert re-read its last row; their results are dropped
    const int64_t ar = a_rows ? (int64_t)a_rows[gr] : (int64_t)gr;
    a_src[j] = A + ar * lda + kc * 8;
  }
#pragma unroll
  for (int j = 0; j < kBDma; ++j) {
    const int p = (wave * kBDma + j) * 64 + lane;
    const int row = p / kCPR, kc = swz_chunk(row, p % kCPR);
    const int64_t br = (int64_t)e * b_expert + (int64_t)(n0 + row) * K + kc * 8;
    b_src[0][j] = B0 + br;
    if constexpr (NB > 1) b_src[1][j] = B1 + br;
  }
  const int KT = K / BK;
  auto issue = [&](int stage) {  // stages past the last re-read it (their slot is never multiplied)
    const int kt = stage < KT ? stage : KT - 1;
    uint4 *s = lds + (stage % kRing) * kStage;
#pragma unroll
    for (int j = 0; j < kADma; ++j) tm_dma16(a_src[j] + (int64_t)kt * BK, s + (wave * kADma + j) * 64);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < kBDma; ++j)
        tm_dma16(b_src[b][j] + (int64_t)kt * BK, s + kAStage + b * kBStage + (wave * kBDma + j) * 64);
  };

  tm_f32x16 acc[NB][kMI][kNI];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
      for (int ni = 0; ni < kNI; ++ni) acc[b][mi][ni] = tm_f32x16{};

  issue(0);
  issue(1);
  issue(2);
  for (int i = 0; i < KT; ++i) {
    tm_wait_vm_lgkm0<2 * kDma>();  // this wave's loads of stage i are done (stages i+1, i+2 may fly)
    __syncthreads();
    issue(i + 3);
    const uint4 *s = lds + (i % kRing) * kStage;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kc = ks * 2 + (lane >> 5);
      uint4 fa[kMI], fb[NB][kNI];
#pragma unroll
      for (int mi = 0; mi < kMI; ++mi) fa[mi] = s[swz(wm * 128 + mi * 32 + (lane & 31), kc)];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) fb[b][ni] = s[kAStage + b * kBStage + swz(wn * 64 + ni * 32 + (lane & 31), kc)];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
          for (int ni = 0; ni < kNI; ++ni) acc[b][mi][ni] = tm_mfma32x32x16<DT>(fa[mi], fb[b][ni], acc[b][mi][ni]);
    }
  }
  tm_wait_vm_lgkm0<0>();  // no load may still target this workgroup's LDS when it exits

  // Epilogue: lane owns column (lane % 32) of each block and its 16 rows.
#pragma unroll
  for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNI; ++ni)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = wm * 128 + mi * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        const int col = n0 + wn * 64 + ni * 32 + (lane & 31);
        const int gr = r0 + row;
        if (gr >= r_end) continue;
        float v;
        if constexpr (MODE == kModeUp) {
          const float g = tm_round<DT>(acc[0][mi][ni][i]);
          const float u = acc[NB - 1][mi][ni][i];
          v = (g / (1.f + __expf(-g))) * u;
        } else {
          v = acc[0][mi][ni][i];
          if (addend != nullptr) v += Elem<DT>::to_f(addend[(int64_t)gr * ld_add + col]);  // dense rows only
        }
        const int64_t dst = c_rows ? c_rows[gr] + col : (int64_t)gr * ldc + col;
        C[dst] = Elem<DT>::from_f(v);
      }
}

// One workgroup of kGroupThreads: bucket the recomputed (token, slot) pairs
// by expert.  mask[b * ms_b + s * ms_s] != 0 selects a pair (ms_s = 0: a
// per-token flag); ids outside [0, n_experts) are skipped.
constexpr int kGroupThreads = 1024;
constexpr int kMaxExperts = 1024;
constexpr int kGroupTok = 4;    // tokens per thread on the register path (n <= 4096)
constexpr int kGroupSlots = 8;  // slots per token on the register path (top_k <= 8)

__global__ __launch_bounds__(kGroupThreads) void group_slots_kernel(
    const int64_t *__restrict__ ids, int64_t n, int top_k, int64_t ld_ids, const uint8_t *__restrict__ mask,
    int64_t ms_b, int64_t ms_s, int n_experts, int64_t so_b, int64_t so_s, int32_t *__restrict__ offsets,
    int32_t *__restrict__ row_token, int64_t *__restrict__ row_out, int32_t *__restrict__ tiles, int64_t t_max) {
  __shared__ int32_t hist[kMaxExperts];
  __shared__ int32_t cursor[kMaxExperts];
  __shared__ int32_t tile_base[kMaxExperts + 1];
  const int tid = threadIdx.x;
  for (int e = tid; e < n_experts; e += kGroupThreads) hist[e] = 0;
  // Each thread keeps the experts of its tokens (b = tid + 1024 j, j < kGroupTok)
  // in registers: all of their loads are issued before the first count.
  int32_t ex[kGroupTok][kGroupSlots];
  // n == 0 takes the loop path, whose loops run no iteration: the register
  // path clamps to token n - 1 and would read below `ids` and `mask`.
  const bool fast = n > 0 && n <= (int64_t)kGroupTok * kGroupThreads && top_k <= kGroupSlots;  // uniform
  if (fast) {
#pragma unroll
    for (int j = 0; j < kGroupTok; ++j) {
      const int64_t b = tid + (int64_t)kGroupThreads * j;
      const int64_t bb = b < n ? b : n - 1;
#pragma unroll
      for (int s = 0; s < kGroupSlots; ++s) {
        const int ss = s < top_k ? s : top_k - 1;
        const int64_t e = ids[bb * ld_ids + ss];
        const bool use = b < n && s < top_k && mask[bb * ms_b + ss * ms_s] && e >= 0 && e < n_experts;
        ex[j][s] = use ? (int32_t)e : -1;
      }
    }
  }
  __syncthreads();
  if (fast) {
#pragma unroll
    for (int j = 0; j < kGroupTok; ++j)
#pragma unroll
      for (int s = 0; s < kGroupSlots; ++s)
        if (ex[j][s] >= 0) atomicAdd(&hist[ex[j][s]], 1);
  } else {
    for (int64_t b = tid; b < n; b += kGroupThreads)  // a token per thread, its slots in order
      for (int s = 0; s < top_k; ++s) {
        const int64_t e = ids[b * ld_ids + s];
        if (mask[b * ms_b + s * ms_s] && e >= 0 && e < n_experts) atomicAdd(&hist[e], 1);
      }
  }
  __syncthreads();
  if (tid == 0) {  // offsets and tile bases (n_experts <= 1024: a short serial scan)
    int32_t run = 0, tr = 0;
    for (int e = 0; e < n_experts; ++e) {
      offsets[e] = run;
      cursor[e] = run;
      tile_base[e] = tr;
      run += hist[e];
      tr += (hist[e] + BM - 1) / BM;
    }
    offsets[n_experts] = run;
    tile_base[n_experts] = tr;
    tiles[0] = run;
    tiles[1] = tr;
  }
  __syncthreads();
  for (int e = tid; e < n_experts; e += kGroupThreads) {
    const int32_t t0 = tile_base[e], t1 = tile_base[e + 1];
    int32_t r = cursor[e];
    for (int32_t t = t0; t < t1; ++t, r += BM) {
      tiles[2 + t] = e;
      tiles[2 + t_max + t] = r;
    }
  }
  __syncthreads();  // cursor[] is read above before the placement below advances it
  if (fast) {
#pragma unroll
    for (int j = 0; j < kGroupTok; ++j)
#pragma unroll
      for (int s = 0; s < kGroupSlots; ++s)
        if (ex[j][s] >= 0) {
          const int64_t b = tid + (int64_t)kGroupThreads * j;
          const int32_t pos = atomicAdd(&cursor[ex[j][s]], 1);
          row_token[pos] = (int32_t)b;
          row_out[pos] = b * so_b + (int64_t)s * so_s;
        }
  } else {
    for (int64_t b = tid; b < n; b += kGroupThreads)
      for (int s = 0; s < top_k; ++s) {
        const int64_t e = ids[b * ld_ids + s];
        if (mask[b * ms_b + s * ms_s] && e >= 0 && e < n_experts) {
          const int32_t pos = atomicAdd(&cursor[e], 1);
          row_token[pos] = (int32_t)b;
          row_out[pos] = b * so_b + (int64_t)s * so_s;
        }
      }
  }
}

template <int DT, int NB, int MODE>
void launch_gemm(const void *A, int64_t lda, const int32_t *a_rows, const void *B0, const void *B1, int64_t b_expert,
                 int K, int N, const TileSrc &ts, int64_t grid_y, void *C, int64_t ldc, const int64_t *c_rows,
                 const void *addend, int64_t ld_add, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const int n_tiles = N / BN;
  const int64_t blocks = tm_cdiv(grid_y, 8) * 8 * n_tiles;
  hipLaunchKernelGGL((grouped_gemm_kernel<DT, NB, MODE>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                     static_cast<const T *>(A), lda, a_rows, static_cast<const T *>(B0), static_cast<const T *>(B1),
                     b_expert, K, n_tiles, ts, static_cast<T *>(C), ldc, c_rows, static_cast<const T *>(addend),
                     ld_add);
}

// The two GEMMs of the MLP over the rows the tile source names; `addend`
// (dense rows only, nullable) is added to the down projection before its
// rounding.
int swiglu_impl(int32_t dtype, const void *x, int64_t ld_x, const int32_t *row_token, int32_t hidden,
                int32_t inter, const void *w1, const void *w3, const void *w2, const TileSrc &ts, int64_t grid_y,
                void *out, int64_t ld_out, const int64_t *row_out, void *fused, const void *addend, int64_t ld_add,
                hipStream_t s) {
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    if constexpr (DT == TM_DT_F32) {
      return tm_fail(TM_EINVAL_DTYPE, "tm_grouped_swiglu: dtype must be F16 or BF16");
    } else {
      launch_gemm<DT, 2, kModeUp>(x, ld_x, row_token, w1, w3, (int64_t)inter * hidden, hidden, inter, ts, grid_y,
                                  fused, inter, nullptr, nullptr, 0, s);
      TM_LAUNCH_CHECK("tm_grouped_swiglu(up)");
      launch_gemm<DT, 1, kModeDown>(fused, inter, nullptr, w2, nullptr, (int64_t)hidden * inter, inter, hidden, ts,
                                    grid_y, out, ld_out, row_out, addend, ld_add, s);
      TM_LAUNCH_CHECK("tm_grouped_swiglu(down)");
      return TM_OK;
    }
  });
}

bool shapes_ok(int32_t hidden, int32_t inter) {
  return hidden > 0 && inter > 0 && hidden % BN == 0 && inter % BN == 0 && hidden % BK == 0 && inter % BK == 0 &&
         hidden / BK >= 1 && inter / BK >= 1;
}

}  // namespace

extern "C" int64_t tm_group_slots_tiles(int64_t max_rows, int32_t n_experts) {
  if (max_rows < 0 || n_experts <= 0) return 0;
  return tm_cdiv(max_rows, BM) + n_experts;
}

extern "C" int tm_group_slots(const int64_t *ids, int64_t n_tokens, int32_t top_k, int64_t ld_ids,
                              const uint8_t *mask, int64_t ms_b, int64_t ms_s, int32_t n_experts, int64_t so_b,
                              int64_t so_s, int32_t *expert_offsets, int32_t *row_token, int64_t *row_out,
                              int32_t *tiles, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && top_k >= 1 && ld_ids >= top_k && n_experts >= 1 && n_experts <= kMaxExperts,
             TM_EINVAL_SHAPE, "tm_group_slots: bad sizes (n_experts must be in [1, %d])", kMaxExperts);
  TM_REQUIRE(n_tokens * top_k < ((int64_t)1 << 31), TM_EINVAL_SHAPE, "tm_group_slots: too many slots");
  TM_REQUIRE(expert_offsets && tiles && (n_tokens == 0 || (ids && mask && row_token && row_out)), TM_EINVAL_ARG,
             "tm_group_slots: null pointer");
  const int64_t t_max = tm_group_slots_tiles(n_tokens * top_k, n_experts);
  hipLaunchKernelGGL(group_slots_kernel, dim3(1), dim3(kGroupThreads), 0, tm_hip_stream(stream), ids, n_tokens,
                     top_k, ld_ids, mask, ms_b, ms_s, n_experts, so_b, so_s, expert_offsets, row_token, row_out,
                     tiles, t_max);
  TM_LAUNCH_CHECK("tm_group_slots");
  return TM_OK;
}

extern "C" size_t tm_swiglu_workspace_size(int64_t max_rows, int32_t inter, int32_t dtype) {
  if (max_rows <= 0 || inter <= 0) return 0;
  return (size_t)max_rows * (size_t)inter * (dtype == TM_DT_F32 ? 4 : 2);
}

extern "C" int tm_grouped_swiglu(int32_t dtype, const void *x, int64_t ld_x, int32_t hidden, int32_t inter,
                                 int32_t n_experts, const void *w1, const void *w3, const void *w2, int64_t max_rows,
                                 const int32_t *expert_offsets, const int32_t *row_token, const int64_t *row_out,
                                 const int32_t *tiles, void *out, void *workspace, size_t workspace_bytes,
                                 tm_stream_t stream) {
  TM_REQUIRE(shapes_ok(hidden, inter), TM_EINVAL_SHAPE,
             "tm_grouped_swiglu: hidden and inter must be positive multiples of %d", BN);
  TM_REQUIRE(n_experts >= 1 && max_rows >= 0 && max_rows < ((int64_t)1 << 31) && ld_x >= hidden, TM_EINVAL_SHAPE,
             "tm_grouped_swiglu: bad sizes");
  if (max_rows == 0) return TM_OK;
  TM_REQUIRE(x && w1 && w3 && w2 && expert_offsets && row_token && row_out && tiles && out, TM_EINVAL_ARG,
             "tm_grouped_swiglu: null pointer");
  TM_REQUIRE(tm_aligned16(x) && (ld_x * 2) % 16 == 0 && tm_aligned16(w1) && tm_aligned16(w3) && tm_aligned16(w2),
             TM_EINVAL_SHAPE, "tm_grouped_swiglu: x rows and weights must be 16-byte aligned");
  const size_t need = tm_swiglu_workspace_size(max_rows, inter, dtype);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need && tm_aligned16(workspace), TM_EWORKSPACE,
             "tm_grouped_swiglu: workspace %zu bytes < %zu", workspace_bytes, need);
  const int64_t t_max = tm_group_slots_tiles(max_rows, n_experts);
  const TileSrc ts{tiles, expert_offsets, t_max, 0};
  return swiglu_impl(dtype, x, ld_x, row_token, hidden, inter, w1, w3, w2, ts, t_max, out, 0, row_out, workspace,
                     nullptr, 0, tm_hip_stream(stream));
}

namespace {

int expert_swiglu_impl(const char *name, int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                       const void *w1, const void *w3, const void *w2, int32_t inter, const void *addend,
                       int64_t ld_add, void *out, int64_t ld_out, void *workspace, size_t workspace_bytes,
                       tm_stream_t stream) {
  TM_REQUIRE(shapes_ok(hidden, inter), TM_EINVAL_SHAPE, "%s: hidden and inter must be positive multiples of %d",
             name, BN);
  TM_REQUIRE(n_rows >= 0 && n_rows < ((int64_t)1 << 31) && ld_x >= hidden && ld_out >= hidden &&
                 (addend == nullptr || ld_add >= hidden),
             TM_EINVAL_SHAPE, "%s: bad sizes", name);
  if (n_rows == 0) return TM_OK;
  TM_REQUIRE(x && w1 && w3 && w2 && out, TM_EINVAL_ARG, "%s: null pointer", name);
  TM_REQUIRE(tm_aligned16(x) && (ld_x * 2) % 16 == 0 && tm_aligned16(w1) && tm_aligned16(w3) && tm_aligned16(w2),
             TM_EINVAL_SHAPE, "%s: x rows and weights must be 16-byte aligned", name);
  const size_t need = tm_swiglu_workspace_size(n_rows, inter, dtype);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need && tm_aligned16(workspace), TM_EWORKSPACE,
             "%s: workspace %zu bytes < %zu", name, workspace_bytes, need);
  const TileSrc ts{nullptr, nullptr, 0, (int32_t)n_rows};
  return swiglu_impl(dtype, x, ld_x, nullptr, hidden, inter, w1, w3, w2, ts, tm_cdiv(n_rows, BM), out, ld_out,
                     nullptr, workspace, addend, ld_add, tm_hip_stream(stream));
}

}  // namespace

extern "C" int tm_expert_swiglu(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                                const void *w1, const void *w3, const void *w2, int32_t inter, void *out,
                                int64_t ld_out, void *workspace, size_t workspace_bytes, tm_stream_t stream) {
  return expert_swiglu_impl("tm_expert_swiglu", dtype, x, n_rows, hidden, ld_x, w1, w3, w2, inter, nullptr, 0, out,
                            ld_out, workspace, workspace_bytes, stream);
}

extern "C" int tm_expert_swiglu_add(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                                    const void *w1, const void *w3, const void *w2, int32_t inter,
                                    const void *addend, int64_t ld_add, void *out, int64_t ld_out, void *workspace,
                                    size_t workspace_bytes, tm_stream_t stream) {
  TM_REQUIRE(addend != nullptr, TM_EINVAL_ARG, "tm_expert_swiglu_add: null addend");
  return expert_swiglu_impl("tm_expert_swiglu_add", dtype, x, n_rows, hidden, ld_x, w1, w3, w2, inter, addend, ld_add,
                            out, ld_out, workspace, workspace_bytes, stream);
}
