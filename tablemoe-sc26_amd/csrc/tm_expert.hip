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
// B rows k-contiguous (nn.Linear weights [out, in]), K in BK-wide stages
// moved global -> LDS by direct loads (16-byte chunks XOR-swizzled by row, so
// the operand reads of 32 rows spread over the banks), three in flight.
// Four waves, one per SIMD, each software-pipelined so that the operand reads
// of one k-step run under the MFMAs of the previous one.  Up mode multiplies
// W1 and W3 against the same A fragments and applies the SiLU-mul epilogue;
// down mode writes each row to its slot of the output.
//
// Packed path (tm_expert_pack_weights, tm_grouped_swiglu_packed,
// tm_expert_swiglu_packed): each weight tile is stored stage by stage in the
// LDS slot order, so a stage's weight tile is one contiguous read; the up
// GEMM then writes the intermediate in the same stage order (whole 256-row
// tiles) and the down GEMM reads its A stages contiguously.  Same arithmetic,
// same bits.
#include "tm_internal.h"
#include "tm_dma.h"
#include "tm_mfma.h"

namespace {

constexpr int BM = 256, BK = 32, kThreads = 256;
constexpr int kMinBN = 128;                  // column tile of the up GEMM (and of narrow down GEMMs)
constexpr int kCPR = BK / 8;                 // 16-byte chunks per tile row and stage
constexpr int kAStage = BM * kCPR;           // A slots (16 bytes) per stage
constexpr int kADma = kAStage / kThreads;    // A loads per thread per stage (4)
constexpr int kMI = 4;                       // 32-row blocks per wave: 128 rows
constexpr int kStageCols = 128;              // epilogue staging width (columns per pass)
constexpr int kStageLd = kStageCols + 8;     // staging row stride in floats
constexpr int kEpiFloats = BM * kStageLd;    // staging tile size in floats (139,264 bytes)

enum { kModeUp = 0, kModeDown = 1 };

// Slot of (row, 16-byte chunk kc) in a stage.  A row is 64 bytes, so four
// rows share one 256-byte line of the 64 banks, which a 16-byte read serves
// 16 lanes at a time; XOR-ing the chunk with (row / 4) % 4 puts 16
// consecutive rows on 16 distinct 16-byte bank groups, and an operand read
// (one chunk of 32 consecutive rows) is conflict-free.
__device__ __forceinline__ int swz_chunk(int row, int kc) { return kc ^ ((row >> 2) & (kCPR - 1)); }

// Tile source: the grouped tile list (tiles != nullptr: [0] rows, [1] tiles,
// then tile_expert[t_max], tile_row0[t_max]) or one dense expert of `rows`.
struct TileSrc {
  const int32_t *tiles;
  const int32_t *expert_offsets;
  int64_t t_max;
  int32_t rows;
};

// One BM x BN tile C = A B^T of one expert (NB = 2: two B matrices against
// the same A, the gate and up projections).  Four waves in a 2 x 2 grid of
// 128 x BN/2 quadrants, one wave per SIMD, 16 accumulator blocks of
// v_mfma_f32_32x32x16 per wave (all 256 AGPRs): 4 x 2 per B for the up GEMM
// (BN = 128), 4 x 4 for the down GEMM (BN = 256), so every k-step reads 8
// operand fragments from LDS for 16 MFMAs (a hidden size that is not a
// multiple of 256 takes 128-column down tiles: 6 reads, 8 MFMAs).
//
// K moves in BK-wide stages through a 4-slot LDS ring filled by direct
// global -> LDS loads (A rows gathered by 64-bit per-lane addresses, B rows
// through a buffer resource whose scalar offset walks K), three stages in
// flight.  Each wave is software-pipelined over half-stages (k-steps): while
// the matrix core runs the 16 MFMAs of one k-step, the wave reads the next
// k-step's 8 fragments into the other register set (sched_group_barrier
// interleaves one read per two MFMAs).  The stage boundary sits between a
// stage's two k-steps: wait for this wave's loads of the next stage, barrier
// (every wave's loads of it are then visible and every wave has finished its
// reads of the current stage's slot), and refill that slot with the stage
// four ahead.  Stages past the last re-read the last one (never multiplied),
// so the wait counts are the same in every iteration.
template <int DT, int NB, int MODE, int BN, bool PB>
__global__ __launch_bounds__(kThreads, 1) void grouped_gemm_kernel(
    const typename Elem<DT>::T *__restrict__ A, int64_t lda, const int32_t *__restrict__ a_rows,
    const typename Elem<DT>::T *__restrict__ B0, const typename Elem<DT>::T *__restrict__ B1, int64_t b_expert,
    int K, int n_tiles, TileSrc ts, typename Elem<DT>::T *__restrict__ C, int64_t ldc,
    const int64_t *__restrict__ c_rows, const typename Elem<DT>::T *__restrict__ addend, int64_t ld_add) {
  using T = typename Elem<DT>::T;
  constexpr int kNI = BN / 64;                   // 32-column blocks per wave and B
  constexpr int kBStage = BN * kCPR;             // slots of each B per stage
  constexpr int kBDma = kBStage / kThreads;      // loads of each B per thread per stage
  constexpr int kStage = kAStage + NB * kBStage;
  constexpr int kDma = kADma + NB * kBDma;       // loads per wave per stage
  constexpr int kFrag = kMI + NB * kNI;          // operand fragments per k-step
  constexpr int kMfma = NB * kMI * kNI;          // MFMAs per k-step (16; 8 for a 128-column down GEMM)
  static_assert(kMfma <= 16, "accumulators fit the AGPRs");
  static_assert(kBStage % kThreads == 0 && 3 * kDma < 64, "stage shape");
  // One LDS array: the 4-slot ring during the K loop, then the fp32 staging
  // tile of the epilogue (kStageCols columns, rows padded to kStageLd floats).
  constexpr int kLdsSlots = 4 * kStage > kEpiFloats / 4 ? 4 * kStage : kEpiFloats / 4;
  __shared__ uint4 lds_all[kLdsSlots];
  uint4 *const ring0 = lds_all, *const ring1 = lds_all + kStage, *const ring2 = lds_all + 2 * kStage,
               *const ring3 = lds_all + 3 * kStage;

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
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // Loads: thread t fills slots t + 256 j of the A part and of each B part;
  // slot p holds row p / kCPR, chunk swz_chunk(row, p % kCPR) (the swizzle is
  // its own inverse).  A: 64-bit address of stage 0 (stage s adds s * BK).
  // The packed down GEMM reads the intermediate tile y as the up GEMM wrote
  // it, stage by stage in slot order: stage s of the tile is the contiguous
  // block s * BM * BK (rows past the expert hold whatever was there; their
  // results are dropped).
  constexpr bool kTiledA = PB && MODE == kModeDown;
  constexpr int64_t kAStep = kTiledA ? BM * BK : BK;  // elements from one stage to the next
  const T *a_src[kADma];
#pragma unroll
  for (int j = 0; j < kADma; ++j) {
    const int p = tid + kThreads * j;
    const int row = p / kCPR, kc = swz_chunk(row, p % kCPR);
    if constexpr (kTiledA) {
      a_src[j] = A + y * (int64_t)BM * lda + (int64_t)p * 8;
    } else {
      int gr = r0 + row;
      gr = gr < r_end ? gr : r_end - 1;  // rows past the expert re-read its last row; their results are dropped
      const int64_t ar = a_rows ? (int64_t)a_rows[gr] : (int64_t)gr;
      a_src[j] = A + ar * lda + kc * 8;
    }
  }
  // B: the expert's BN rows from n0 on, through a buffer; lane offsets fixed,
  // the stage's K offset in the scalar offset.  Packed weights (PB) hold each
  // stage of the tile as one contiguous block in slot order, so slot p is at
  // byte 16 p of the stage's block.
  tm_rsrc_t b_rs[NB];
  b_rs[0] = tm_make_rsrc(B0 + (int64_t)e * b_expert + (int64_t)n0 * K, (uint64_t)BN * K * sizeof(T));
  if constexpr (NB > 1) b_rs[1] = tm_make_rsrc(B1 + (int64_t)e * b_expert + (int64_t)n0 * K, (uint64_t)BN * K * sizeof(T));
  uint32_t b_off[kBDma];
#pragma unroll
  for (int j = 0; j < kBDma; ++j) {
    const int p = tid + kThreads * j;
    const int row = p / kCPR, kc = swz_chunk(row, p % kCPR);
    b_off[j] = PB ? (uint32_t)p * 16u : (uint32_t)row * (uint32_t)K * (uint32_t)sizeof(T) + (uint32_t)kc * 16u;
  }
  const int KT = K / BK;  // a multiple of 4 (the host checks)
  // Load j (0 .. kDma-1) of stage `stage` into `ring`: A loads first, then
  // each B's.  Stages past the last re-read the last one.
  auto issue_one = [&](auto j_c, uint4 *ring, int stage) {
    constexpr int j = decltype(j_c)::value;
    const int kt = stage < KT ? stage : KT - 1;
    const uint32_t lds = (uint32_t)(uintptr_t)ring + (uint32_t)wave * 1024u;  // wave's 64 slots of load 0
    if constexpr (j < kADma) {
      tm_dma16_s(a_src[j] + (int64_t)kt * kAStep, lds + (uint32_t)(j * kThreads * 16));
    } else {
      constexpr int bb = (j - kADma) / kBDma, jb = (j - kADma) % kBDma;
      tm_dma16_buf_so(b_rs[bb], b_off[jb], (uint32_t)kt * (uint32_t)(PB ? kBStage * 16 : BK * sizeof(T)),
                      lds + (uint32_t)((kAStage + bb * kBStage + jb * kThreads) * 16));
    }
  };
  auto issue = [&](uint4 *ring, int stage) { tm_static_for<kDma>([&](auto j_c) { issue_one(j_c, ring, stage); }); };

  // Fragment byte offsets within a slot: row R + (lane % 32) (R a multiple of
  // 32) at chunk 2 ks + lane / 32 sits at R * 64 + off[ks], the same for every
  // block, part and slot; opaque, so the rest stays an immediate offset.
  uint32_t f_off[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int r = lane & 31;
    f_off[ks] = (uint32_t)(r * kCPR + swz_chunk(r, 2 * ks + (lane >> 5))) * 16u;
    asm volatile("" : "+v"(f_off[ks]));
  }
  uint4 fr[2][kFrag];  // two k-steps' operands: [0..kMI) A blocks, then B blocks
  auto read_one = [&](auto g_c, uint4 (&f)[kFrag], const uint4 *ring, int ks) {
    constexpr int g = decltype(g_c)::value;
    const char *base = reinterpret_cast<const char *>(ring) + f_off[ks];
    if constexpr (g < kMI) {
      f[g] = *reinterpret_cast<const uint4 *>(base + (wm * 128 + g * 32) * 64);
    } else {
      constexpr int bb = (g - kMI) / kNI, ni = (g - kMI) % kNI;
      f[g] = *reinterpret_cast<const uint4 *>(base + (kAStage + bb * kBStage) * 16 + (wn * (BN / 2) + ni * 32) * 64);
    }
  };

  tm_f32x16 acc[NB][kMI][kNI];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb)
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
      for (int ni = 0; ni < kNI; ++ni) acc[bb][mi][ni] = tm_f32x16{};
  auto mfma_one = [&](auto m_c, const uint4 (&f)[kFrag]) {
    constexpr int m = decltype(m_c)::value;
    constexpr int bb = m / (kMI * kNI), mi = (m / kNI) % kMI, ni = m % kNI;
    acc[bb][mi][ni] = tm_mfma32x32x16<DT>(f[mi], f[kMI + bb * kNI + ni], acc[bb][mi][ni]);
  };
  // One k-step: its MFMAs on `f`, and between them (in fixed groups, so the
  // waits of neither sit in front of the matrix core) the reads of `next`
  // from `rd` at k-step ks and, with DMA, the kDma loads of stage `st` into
  // `dst` (kDma == kFrag for every shape here).
  static_assert(kDma == kFrag, "one load per operand read");
  constexpr int kPer = kMfma / kFrag;
  auto kstep = [&](auto dma_c, const uint4 (&f)[kFrag], uint4 (&next)[kFrag], const uint4 *rd, int ks, uint4 *dst,
                   int st) {
    tm_static_for<kFrag>([&](auto g_c) {
      constexpr int g = decltype(g_c)::value;
      tm_static_for<kPer>([&](auto q_c) { mfma_one(std::integral_constant<int, g * kPer + decltype(q_c)::value>{}, f); });
      read_one(g_c, next, rd, ks);
      if constexpr (decltype(dma_c)::value) issue_one(g_c, dst, st);
      __builtin_amdgcn_sched_barrier(0);
    });
    tm_static_for<kMfma - kFrag * kPer>(
        [&](auto q_c) { mfma_one(std::integral_constant<int, kFrag * kPer + decltype(q_c)::value>{}, f); });
  };

  issue(ring0, 0);
  issue(ring1, 1);
  issue(ring2, 2);
  issue(ring3, 3);
  tm_wait_vm_lgkm0<3 * kDma>();  // stage 0 of this wave landed
  __builtin_amdgcn_s_barrier();
  tm_static_for<kFrag>([&](auto g_c) { read_one(g_c, fr[0], ring0, 0); });

  // stage i in ring slot `cur`, stage i + 1 in `nxt`
  auto step = [&](uint4 *cur, const uint4 *nxt, int i) {
    kstep(std::false_type{}, fr[0], fr[1], cur, 1, cur, 0);
    tm_wait_vm_lgkm0<2 * kDma>();  // stage i + 1 of this wave landed (i + 2, i + 3 may fly); reads done
    __builtin_amdgcn_s_barrier();  // ... in every wave; no wave reads slot `cur` any more
    kstep(std::true_type{}, fr[1], fr[0], nxt, 0, cur, i + 4);
  };
  for (int i = 0; i < KT; i += 4) {
    step(ring0, ring1, i);
    step(ring1, ring2, i + 1);
    step(ring2, ring3, i + 2);
    step(ring3, ring0, i + 3);
  }
  tm_wait_vm_lgkm0<0>();  // no load may still target this workgroup's LDS when it exits
  __syncthreads();         // ... and every wave is done with the ring

  // Epilogue through LDS, kStageCols columns at a time.  Each wave writes its
  // fp32 results (up mode: silu(dtype(g)) * u, unrounded) to the staging tile
  // [BM][kStageLd]: lane owns column (lane % 32) of each block and its 16 rows
  // 8 (i / 4) + 4 (lane / 32) + i % 4 (the +8 float row padding puts the two
  // row groups of one write on disjoint banks).  Then each thread rounds and
  // stores 8-column chunks: 16 threads per 128-column row, so every store of a
  // wave writes 4 whole rows (down mode adds the addend row chunk first, in
  // fp32, one rounding).
  float *const stage = reinterpret_cast<float *>(lds_all);
  const int lrow = wm * 128 + 4 * (lane >> 5), lcol = wn * (BN / 2) + (lane & 31);
#pragma unroll
  for (int pass = 0; pass < BN / kStageCols; ++pass) {
    if (pass > 0) __syncthreads();  // the previous pass's chunks are read
    if (lcol - (lane & 31) >= pass * kStageCols && lcol - (lane & 31) < (pass + 1) * kStageCols) {  // uniform
      float *w = stage + lrow * kStageLd + (lcol - pass * kStageCols);
#pragma unroll
      for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            float v;
            if constexpr (MODE == kModeUp) {
              const float g = tm_round<DT>(acc[0][mi][ni][i]);
              v = g * __builtin_amdgcn_rcpf(1.f + __expf(-g)) * acc[NB - 1][mi][ni][i];
            } else {
              v = acc[0][mi][ni][i];
            }
            w[(mi * 32 + 8 * (i >> 2) + (i & 3)) * kStageLd + ni * 32] = v;
          }
    }
    __syncthreads();
#pragma unroll 4
    for (int k = 0; k < BM * kStageCols / 8 / kThreads; ++k) {
      const int c = tid + k * kThreads;
      const int row = c / (kStageCols / 8), col8 = (c % (kStageCols / 8)) * 8;
      const int gr = r0 + row;
      if (gr >= r_end) break;  // rows only grow with k
      const int col = n0 + pass * kStageCols + col8;
      float v[8];
      const float4 *src = reinterpret_cast<const float4 *>(stage + row * kStageLd + col8);
      const float4 lo = src[0], hi = src[1];
      v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w; v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
      if constexpr (MODE == kModeDown) {
        if (addend != nullptr) {  // dense rows only
          float a[8];
          tm_load8<DT>(addend + (int64_t)gr * ld_add + col, a);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] += a[j];
        }
      }
      if constexpr (PB && MODE == kModeUp)  // tile y of the intermediate in the down GEMM's stage order
        tm_store8<DT>(C + y * (int64_t)BM * ldc + (col / BK) * (BM * BK) +
                          (row * kCPR + swz_chunk(row, (col % BK) / 8)) * 8,
                      v);
      else
        tm_store8<DT>(C + (c_rows ? c_rows[gr] + col : (int64_t)gr * ldc + col), v);
    }
  }
}

// One workgroup of kGroupThreads: bucket the recomputed (token, slot) pairs
// by expert.  mask[b * ms_b + s * ms_s] != 0 selects a pair (ms_s = 0: a
// per-token flag); ids outside [0, n_experts) are skipped.
constexpr int kGroupThreads = 1024;
constexpr int kMaxExperts = 1024;  // one scanning thread per expert
static_assert(kMaxExperts <= kGroupThreads, "one expert per thread");
constexpr int kGroupTok = 4;    // tokens per thread on the register path (n <= 4096)
constexpr int kGroupSlots = 8;  // slots per token on the register path (top_k <= 8)
static_assert(kGroupTok * kGroupThreads * 8 <= 65536, "a placed row (token << 3 | slot) fits 16 bits");

__global__ __launch_bounds__(kGroupThreads) void group_slots_kernel(
    const int64_t *__restrict__ ids, int64_t n, int top_k, int64_t ld_ids, const uint8_t *__restrict__ mask,
    int64_t ms_b, int64_t ms_s, int n_experts, int64_t so_b, int64_t so_s, int32_t *__restrict__ offsets,
    int32_t *__restrict__ row_token, int64_t *__restrict__ row_out, int32_t *__restrict__ tiles, int64_t t_max) {
  __shared__ int32_t hist[kMaxExperts];
  __shared__ int32_t cursor[kMaxExperts];
  __shared__ int32_t tile_base[kMaxExperts + 1];
  // register path: each placed row as (token << 3 | slot), written out in row
  // order afterwards (scattered 4- and 8-byte stores cost ~10 us; in row
  // order they are a few coalesced passes)
  __shared__ uint16_t placed[kGroupTok * kGroupThreads * kGroupSlots];
  __shared__ int32_t s_rows;
  __shared__ int32_t wave_rows[kGroupThreads / 64], wave_tiles[kGroupThreads / 64];
  const int tid = threadIdx.x;
  for (int e = tid; e < n_experts; e += kGroupThreads) hist[e] = 0;
  // Each thread keeps the experts of its tokens (b = tid + 1024 j, j < kGroupTok)
  // in registers: all of their loads are issued before the first count.
  // (Reading the id array as consecutive elements per wave load instead
  // measured slower: 16.4 / 24.9 us against 15.2 / 21.7 us hot / cold.)
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
  {
    // offsets and tile bases: exclusive scans over the experts, thread e
    // owning expert e (n_experts <= kGroupThreads): wave scans, then the
    // waves' totals in wave order (a serial loop over the experts cost ~4 us)
    const int lane = tid & 63, wave = tid >> 6;
    const int32_t h = tid < n_experts ? hist[tid] : 0;
    const int32_t tc = (h + BM - 1) / BM;
    int32_t ih = h, it = tc;  // inclusive within the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int32_t oh = __shfl_up(ih, d, 64), ot = __shfl_up(it, d, 64);
      if (lane >= d) {
        ih += oh;
        it += ot;
      }
    }
    if (lane == 63) {
      wave_rows[wave] = ih;
      wave_tiles[wave] = it;
    }
    __syncthreads();
    int32_t bh = 0, bt = 0;
    for (int w = 0; w < wave; ++w) {
      bh += wave_rows[w];
      bt += wave_tiles[w];
    }
    const int32_t eh = bh + ih - h, et = bt + it - tc;  // exclusive
    if (tid < n_experts) {
      offsets[tid] = eh;
      cursor[tid] = eh;
      tile_base[tid] = et;
    }
    if (tid == n_experts - 1) {
      offsets[n_experts] = eh + h;
      tile_base[n_experts] = et + tc;
      tiles[0] = eh + h;
      tiles[1] = et + tc;
      s_rows = eh + h;
    }
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
          const int b = tid + kGroupThreads * j;  // < 4096
          const int32_t pos = atomicAdd(&cursor[ex[j][s]], 1);
          placed[pos] = (uint16_t)((b << 3) | s);
        }
    __syncthreads();
    const int32_t rows = s_rows;
    for (int32_t i = tid; i < rows; i += kGroupThreads) {
      const int v = placed[i];
      const int64_t b = v >> 3;
      row_token[i] = (int32_t)b;
      row_out[i] = b * so_b + (int64_t)(v & 7) * so_s;
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

// Multi-workgroup grouping (tm_group_slots_ws): kGrpTok tokens per
// workgroup, in two launches.  group_count_kernel loads its tokens' ids and
// mask bytes and writes the workgroup's per-expert counts to a row of the
// workspace; group_place_kernel loads them again, sums every workgroup's row
// for each expert (and the rows of the workgroups before it), scans the
// experts for the offsets and tile bases (workgroup 0 writes them and the
// tile list) and places its rows at offset + rows of earlier workgroups +
// an LDS cursor.  Each CU then loads 1/G of the ids instead of one CU all
// of them.
constexpr int kGrpThreads = 256;
constexpr int kGrpTok = 64;            // tokens per workgroup: 4 threads per token, 2 slots each
constexpr int kGrpMaxSlots = 8;        // top_k
constexpr int kGrpMaxExperts = 256;    // one expert per thread in the scan
constexpr int kGrpMaxWgs = 128;        // n_tokens <= 8192
constexpr int kGrpBatch = 16;          // count rows loaded per round trip

// The two (token, slot) entries of this thread: expert id, or -1 when the
// pair is not recomputed.  Clamped addresses (no load is conditional).
__device__ __forceinline__ void grp_entries(const int64_t *__restrict__ ids, int64_t n, int top_k, int64_t ld_ids,
                                            const uint8_t *__restrict__ mask, int64_t ms_b, int64_t ms_s,
                                            int n_experts, int64_t b, int s0, int (&ex)[2]) {
  const int64_t bb = b < n ? b : n - 1;
  int64_t e[2];
  uint8_t m[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int s = s0 + u;
    const int ss = s < top_k ? s : top_k - 1;
    e[u] = ids[bb * ld_ids + ss];
    m[u] = mask[bb * ms_b + ss * ms_s];
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const bool use = b < n && s0 + u < top_k && m[u] && e[u] >= 0 && e[u] < n_experts;
    ex[u] = use ? (int)e[u] : -1;
  }
}

__global__ __launch_bounds__(kGrpThreads) void group_count_kernel(const int64_t *__restrict__ ids, int64_t n,
                                                                  int top_k, int64_t ld_ids,
                                                                  const uint8_t *__restrict__ mask, int64_t ms_b,
                                                                  int64_t ms_s, int n_experts,
                                                                  int32_t *__restrict__ counts) {
  __shared__ int32_t h[kGrpMaxExperts];
  const int tid = threadIdx.x;
  int ex[2];
  grp_entries(ids, n, top_k, ld_ids, mask, ms_b, ms_s, n_experts, (int64_t)blockIdx.x * kGrpTok + tid / 4,
              2 * (tid % 4), ex);
  for (int e = tid; e < n_experts; e += kGrpThreads) h[e] = 0;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (ex[u] >= 0) atomicAdd(&h[ex[u]], 1);
  __syncthreads();
  for (int e = tid; e < n_experts; e += kGrpThreads) counts[(int64_t)blockIdx.x * n_experts + e] = h[e];
}

__global__ __launch_bounds__(kGrpThreads) void group_place_kernel(
    const int64_t *__restrict__ ids, int64_t n, int top_k, int64_t ld_ids, const uint8_t *__restrict__ mask,
    int64_t ms_b, int64_t ms_s, int n_experts, int64_t so_b, int64_t so_s, const int32_t *__restrict__ counts,
    int32_t *__restrict__ offsets, int32_t *__restrict__ row_token, int64_t *__restrict__ row_out,
    int32_t *__restrict__ tiles, int64_t t_max) {
  __shared__ int32_t part_tot[kGrpThreads], part_bef[kGrpThreads];
  __shared__ int32_t cur[kGrpMaxExperts];
  __shared__ int32_t wave_rows[kGrpThreads / 64], wave_tiles[kGrpThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = (int)gridDim.x, g0 = (int)blockIdx.x;
  const int64_t b = (int64_t)g0 * kGrpTok + tid / 4;
  const int s0 = 2 * (tid % 4);
  int ex[2];
  grp_entries(ids, n, top_k, ld_ids, mask, ms_b, ms_s, n_experts, b, s0, ex);
  // Thread (e, p) of ep = pow2 >= n_experts columns sums the count rows
  // g = p, p + P, .. (P = 256 / ep) of expert e: kGrpBatch rows per round
  // trip (clamped rows, masked by a select).
  int ep = 1;
  while (ep < n_experts) ep <<= 1;
  const int P = kGrpThreads / ep;
  const int e = tid % ep, p = tid / ep;
  const int ec = e < n_experts ? e : n_experts - 1;
  int32_t tot = 0, bef = 0;
  for (int g = p; g < G; g += P * kGrpBatch) {
    int32_t v[kGrpBatch];
#pragma unroll
    for (int j = 0; j < kGrpBatch; ++j) {
      const int gj = g + P * j;
      v[j] = counts[(int64_t)(gj < G ? gj : G - 1) * n_experts + ec];
    }
#pragma unroll
    for (int j = 0; j < kGrpBatch; ++j) {
      const int gj = g + P * j;
      const int32_t c = (gj < G && e < n_experts) ? v[j] : 0;
      tot += c;
      bef += gj < g0 ? c : 0;
    }
  }
  part_tot[tid] = tot;
  part_bef[tid] = bef;
  __syncthreads();
  // thread x owns expert x: its total and the rows of the earlier workgroups
  int32_t h = 0, hb = 0;
  if (tid < n_experts)
    for (int q = 0; q < P; ++q) {
      h += part_tot[q * ep + tid];
      hb += part_bef[q * ep + tid];
    }
  // exclusive scans over the experts (rows and 256-row tiles): wave scans,
  // then the waves' totals in wave order
  const int32_t tc = (h + BM - 1) / BM;
  int32_t ih = h, it = tc;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t oh = __shfl_up(ih, d, 64), ot = __shfl_up(it, d, 64);
    if (lane >= d) {
      ih += oh;
      it += ot;
    }
  }
  if (lane == 63) {
    wave_rows[wave] = ih;
    wave_tiles[wave] = it;
  }
  __syncthreads();
  int32_t bh = 0, bt = 0;
  for (int w = 0; w < wave; ++w) {
    bh += wave_rows[w];
    bt += wave_tiles[w];
  }
  const int32_t eh = bh + ih - h, et = bt + it - tc;  // exclusive
  if (tid < n_experts) {
    cur[tid] = eh + hb;
    if (g0 == 0) {
      offsets[tid] = eh;
      for (int32_t t = 0; t < tc; ++t) {
        tiles[2 + et + t] = tid;
        tiles[2 + t_max + et + t] = eh + t * BM;
      }
      if (tid == n_experts - 1) {
        offsets[n_experts] = eh + h;
        tiles[0] = eh + h;
        tiles[1] = et + tc;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (ex[u] >= 0) {
      const int32_t pos = atomicAdd(&cur[ex[u]], 1);
      row_token[pos] = (int32_t)b;
      row_out[pos] = b * so_b + (int64_t)(s0 + u) * so_s;
    }
}

template <int DT, int NB, int MODE, int BN, bool PB>
void launch_gemm(const void *A, int64_t lda, const int32_t *a_rows, const void *B0, const void *B1, int64_t b_expert,
                 int K, int N, const TileSrc &ts, int64_t grid_y, void *C, int64_t ldc, const int64_t *c_rows,
                 const void *addend, int64_t ld_add, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const int n_tiles = N / BN;
  const int64_t blocks = tm_cdiv(grid_y, 8) * 8 * n_tiles;
  hipLaunchKernelGGL((grouped_gemm_kernel<DT, NB, MODE, BN, PB>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                     static_cast<const T *>(A), lda, a_rows, static_cast<const T *>(B0), static_cast<const T *>(B1),
                     b_expert, K, n_tiles, ts, static_cast<T *>(C), ldc, c_rows, static_cast<const T *>(addend),
                     ld_add);
}

// Column tile of the down GEMM: 256 columns when hidden allows (half the LDS
// reads per MFMA of 128-column tiles).
inline int down_bn(int32_t hidden) { return hidden % (2 * kMinBN) == 0 ? 2 * kMinBN : kMinBN; }

template <int DT, bool PB>
void swiglu_launch(const void *x, int64_t ld_x, const int32_t *row_token, int32_t hidden, int32_t inter,
                   const void *w1, const void *w3, const void *w2, const TileSrc &ts, int64_t grid_y, void *out,
                   int64_t ld_out, const int64_t *row_out, void *fused, const void *addend, int64_t ld_add,
                   hipStream_t s) {
  launch_gemm<DT, 2, kModeUp, kMinBN, PB>(x, ld_x, row_token, w1, w3, (int64_t)inter * hidden, hidden, inter, ts,
                                          grid_y, fused, inter, nullptr, nullptr, 0, s);
  if (down_bn(hidden) == 2 * kMinBN)
    launch_gemm<DT, 1, kModeDown, 2 * kMinBN, PB>(fused, inter, nullptr, w2, nullptr, (int64_t)hidden * inter, inter,
                                                  hidden, ts, grid_y, out, ld_out, row_out, addend, ld_add, s);
  else
    launch_gemm<DT, 1, kModeDown, kMinBN, PB>(fused, inter, nullptr, w2, nullptr, (int64_t)hidden * inter, inter,
                                              hidden, ts, grid_y, out, ld_out, row_out, addend, ld_add, s);
}

// The two GEMMs of the MLP over the rows the tile source names; `addend`
// (dense rows only, nullable) is added to the down projection before its
// rounding; `packed`: the weights are in tm_expert_pack_weights's layout.
int swiglu_impl(int32_t dtype, const void *x, int64_t ld_x, const int32_t *row_token, int32_t hidden,
                int32_t inter, const void *w1, const void *w3, const void *w2, const TileSrc &ts, int64_t grid_y,
                void *out, int64_t ld_out, const int64_t *row_out, void *fused, const void *addend, int64_t ld_add,
                bool packed, hipStream_t s) {
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    if constexpr (DT == TM_DT_F32) {
      return tm_fail(TM_EINVAL_DTYPE, "tm_grouped_swiglu: dtype must be F16 or BF16");
    } else {
      if (packed)
        swiglu_launch<DT, true>(x, ld_x, row_token, hidden, inter, w1, w3, w2, ts, grid_y, out, ld_out, row_out,
                                fused, addend, ld_add, s);
      else
        swiglu_launch<DT, false>(x, ld_x, row_token, hidden, inter, w1, w3, w2, ts, grid_y, out, ld_out, row_out,
                                 fused, addend, ld_add, s);
      TM_LAUNCH_CHECK("tm_grouped_swiglu");
      return TM_OK;
    }
  });
}

// Packed weights: tile t of BN rows of expert e (rows n0 = t BN ..) keeps
// its place [e][n0 .. n0 + BN) x K of the nn.Linear layout, reordered by
// stage: stage kt (columns kt BK .. + BK) is one contiguous block of BN x BK
// elements holding slot p = 16 bytes (row p / kCPR, chunk swz_chunk(row,
// p % kCPR)) at element 8 p -- the order the GEMM's LDS ring holds a stage
// in, so a stage's weight tile is one contiguous read.  One workgroup per
// stage of one tile.
template <typename T, int BN>
__global__ __launch_bounds__(kThreads) void pack_weights_kernel(const T *__restrict__ w, int64_t K, int64_t KT,
                                                                 T *__restrict__ out) {
  const int64_t b = blockIdx.x;  // (tile of every expert) * KT + kt
  const int64_t tile = b / KT, kt = b % KT;
  const T *src = w + tile * BN * K + kt * BK;
  T *dst = out + tile * BN * K + kt * (BN * BK);
#pragma unroll
  for (int j = 0; j < BN * kCPR / kThreads; ++j) {
    const int p = threadIdx.x + kThreads * j;
    const int row = p / kCPR, kc = swz_chunk(row, p % kCPR);
    *reinterpret_cast<uint4 *>(dst + (int64_t)p * 8) =
        *reinterpret_cast<const uint4 *>(src + (int64_t)row * K + kc * 8);
  }
}

bool shapes_ok(int32_t hidden, int32_t inter) {
  // multiples of 128: whole column tiles, and K in whole rounds of the 4-slot ring (4 stages of BK)
  return hidden > 0 && inter > 0 && hidden % kMinBN == 0 && inter % kMinBN == 0 && (int64_t)inter * hidden <
         ((int64_t)1 << 30);
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
  // tm_grouped_swiglu writes each row in 16-byte pieces from row_out
  TM_REQUIRE(so_b % 8 == 0 && so_s % 8 == 0, TM_EINVAL_SHAPE,
             "tm_group_slots: output strides (%lld, %lld) must be multiples of 8 elements", (long long)so_b,
             (long long)so_s);
  const int64_t t_max = tm_group_slots_tiles(n_tokens * top_k, n_experts);
  hipLaunchKernelGGL(group_slots_kernel, dim3(1), dim3(kGroupThreads), 0, tm_hip_stream(stream), ids, n_tokens,
                     top_k, ld_ids, mask, ms_b, ms_s, n_experts, so_b, so_s, expert_offsets, row_token, row_out,
                     tiles, t_max);
  TM_LAUNCH_CHECK("tm_group_slots");
  return TM_OK;
}

namespace {
bool group_multi_ok(int64_t n_tokens, int32_t top_k, int32_t n_experts) {
  return n_tokens > 0 && n_tokens <= (int64_t)kGrpTok * kGrpMaxWgs && top_k >= 1 && top_k <= kGrpMaxSlots &&
         n_experts >= 1 && n_experts <= kGrpMaxExperts;
}
}  // namespace

extern "C" size_t tm_group_slots_workspace_size(int64_t n_tokens, int32_t top_k, int32_t n_experts) {
  if (!group_multi_ok(n_tokens, top_k, n_experts)) return 0;
  return (size_t)tm_cdiv(n_tokens, kGrpTok) * (size_t)n_experts * sizeof(int32_t);
}

extern "C" int tm_group_slots_ws(const int64_t *ids, int64_t n_tokens, int32_t top_k, int64_t ld_ids,
                                 const uint8_t *mask, int64_t ms_b, int64_t ms_s, int32_t n_experts, int64_t so_b,
                                 int64_t so_s, int32_t *expert_offsets, int32_t *row_token, int64_t *row_out,
                                 int32_t *tiles, void *workspace, size_t workspace_bytes, tm_stream_t stream) {
  const size_t need = tm_group_slots_workspace_size(n_tokens, top_k, n_experts);
  if (need == 0)  // outside the multi-workgroup shapes: the one-workgroup grouping
    return tm_group_slots(ids, n_tokens, top_k, ld_ids, mask, ms_b, ms_s, n_experts, so_b, so_s, expert_offsets,
                          row_token, row_out, tiles, stream);
  TM_REQUIRE(ld_ids >= top_k && top_k >= 1, TM_EINVAL_SHAPE, "tm_group_slots_ws: bad sizes");
  TM_REQUIRE(ids && mask && expert_offsets && row_token && row_out && tiles, TM_EINVAL_ARG,
             "tm_group_slots_ws: null pointer");
  TM_REQUIRE(so_b % 8 == 0 && so_s % 8 == 0, TM_EINVAL_SHAPE,
             "tm_group_slots_ws: output strides (%lld, %lld) must be multiples of 8 elements", (long long)so_b,
             (long long)so_s);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need && tm_aligned16(workspace), TM_EWORKSPACE,
             "tm_group_slots_ws: workspace %zu bytes < %zu", workspace_bytes, need);
  const int64_t t_max = tm_group_slots_tiles(n_tokens * top_k, n_experts);
  const unsigned G = (unsigned)tm_cdiv(n_tokens, kGrpTok);
  hipStream_t s = tm_hip_stream(stream);
  int32_t *counts = static_cast<int32_t *>(workspace);
  hipLaunchKernelGGL(group_count_kernel, dim3(G), dim3(kGrpThreads), 0, s, ids, n_tokens, top_k, ld_ids, mask, ms_b,
                     ms_s, n_experts, counts);
  hipLaunchKernelGGL(group_place_kernel, dim3(G), dim3(kGrpThreads), 0, s, ids, n_tokens, top_k, ld_ids, mask, ms_b,
                     ms_s, n_experts, so_b, so_s, counts, expert_offsets, row_token, row_out, tiles, t_max);
  TM_LAUNCH_CHECK("tm_group_slots_ws");
  return TM_OK;
}

extern "C" size_t tm_swiglu_workspace_size(int64_t max_rows, int32_t inter, int32_t dtype) {
  if (max_rows <= 0 || inter <= 0) return 0;
  return (size_t)max_rows * (size_t)inter * (dtype == TM_DT_F32 ? 4 : 2);
}

// The packed path keeps the intermediate as whole 256-row tiles (one per
// entry of the tile list).
extern "C" size_t tm_grouped_swiglu_packed_workspace_size(int64_t max_rows, int32_t inter, int32_t n_experts,
                                                          int32_t dtype) {
  if (max_rows <= 0 || inter <= 0 || n_experts <= 0) return 0;
  return (size_t)tm_group_slots_tiles(max_rows, n_experts) * BM * (size_t)inter * (dtype == TM_DT_F32 ? 4 : 2);
}

namespace {

int grouped_swiglu_impl(int32_t dtype, const void *x, int64_t ld_x, int32_t hidden, int32_t inter,
                        int32_t n_experts, const void *w1, const void *w3, const void *w2, int64_t max_rows,
                        const int32_t *expert_offsets, const int32_t *row_token, const int64_t *row_out,
                        const int32_t *tiles, void *out, void *workspace, size_t workspace_bytes, bool packed,
                        tm_stream_t stream) {
  TM_REQUIRE(shapes_ok(hidden, inter), TM_EINVAL_SHAPE,
             "tm_grouped_swiglu: hidden and inter must be positive multiples of %d", kMinBN);
  TM_REQUIRE(n_experts >= 1 && max_rows >= 0 && max_rows < ((int64_t)1 << 31) && ld_x >= hidden, TM_EINVAL_SHAPE,
             "tm_grouped_swiglu: bad sizes");
  if (max_rows == 0) return TM_OK;
  TM_REQUIRE(x && w1 && w3 && w2 && expert_offsets && row_token && row_out && tiles && out, TM_EINVAL_ARG,
             "tm_grouped_swiglu: null pointer");
  TM_REQUIRE(tm_aligned16(x) && (ld_x * 2) % 16 == 0 && tm_aligned16(w1) && tm_aligned16(w3) && tm_aligned16(w2) &&
                 tm_aligned16(out),
             TM_EINVAL_SHAPE, "tm_grouped_swiglu: x rows, weights and out must be 16-byte aligned");
  const size_t need = packed ? tm_grouped_swiglu_packed_workspace_size(max_rows, inter, n_experts, dtype)
                              : tm_swiglu_workspace_size(max_rows, inter, dtype);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need && tm_aligned16(workspace), TM_EWORKSPACE,
             "tm_grouped_swiglu: workspace %zu bytes < %zu", workspace_bytes, need);
  const int64_t t_max = tm_group_slots_tiles(max_rows, n_experts);
  const TileSrc ts{tiles, expert_offsets, t_max, 0};
  return swiglu_impl(dtype, x, ld_x, row_token, hidden, inter, w1, w3, w2, ts, t_max, out, 0, row_out, workspace,
                     nullptr, 0, packed, tm_hip_stream(stream));
}

}  // namespace

extern "C" int tm_grouped_swiglu(int32_t dtype, const void *x, int64_t ld_x, int32_t hidden, int32_t inter,
                                 int32_t n_experts, const void *w1, const void *w3, const void *w2, int64_t max_rows,
                                 const int32_t *expert_offsets, const int32_t *row_token, const int64_t *row_out,
                                 const int32_t *tiles, void *out, void *workspace, size_t workspace_bytes,
                                 tm_stream_t stream) {
  return grouped_swiglu_impl(dtype, x, ld_x, hidden, inter, n_experts, w1, w3, w2, max_rows, expert_offsets,
                             row_token, row_out, tiles, out, workspace, workspace_bytes, false, stream);
}

extern "C" int tm_grouped_swiglu_packed(int32_t dtype, const void *x, int64_t ld_x, int32_t hidden, int32_t inter,
                                        int32_t n_experts, const void *w1p, const void *w3p, const void *w2p,
                                        int64_t max_rows, const int32_t *expert_offsets, const int32_t *row_token,
                                        const int64_t *row_out, const int32_t *tiles, void *out, void *workspace,
                                        size_t workspace_bytes, tm_stream_t stream) {
  return grouped_swiglu_impl(dtype, x, ld_x, hidden, inter, n_experts, w1p, w3p, w2p, max_rows, expert_offsets,
                             row_token, row_out, tiles, out, workspace, workspace_bytes, true, stream);
}

extern "C" int tm_expert_pack_weights(int32_t dtype, const void *w, int32_t n_experts, int32_t hidden, int32_t inter,
                                      int32_t role, void *out, tm_stream_t stream) {
  TM_REQUIRE(shapes_ok(hidden, inter) && n_experts >= 1, TM_EINVAL_SHAPE,
             "tm_expert_pack_weights: hidden and inter must be positive multiples of %d", kMinBN);
  TM_REQUIRE(role == TM_PACK_GATE_UP || role == TM_PACK_DOWN, TM_EINVAL_ARG, "tm_expert_pack_weights: bad role");
  TM_REQUIRE(w && out, TM_EINVAL_ARG, "tm_expert_pack_weights: null pointer");
  TM_REQUIRE(tm_aligned16(w) && tm_aligned16(out), TM_EINVAL_SHAPE,
             "tm_expert_pack_weights: weights must be 16-byte aligned");
  // W1 / W3: [n_experts, inter, hidden] in 128-row tiles; W2: [n_experts, hidden, inter] in down_bn rows
  const int64_t rows = role == TM_PACK_GATE_UP ? inter : hidden;
  const int64_t K = role == TM_PACK_GATE_UP ? hidden : inter;
  const int bn = role == TM_PACK_GATE_UP ? kMinBN : down_bn(hidden);
  const int64_t esz = dtype == TM_DT_F32 ? 4 : 2;
  const char *wb = static_cast<const char *>(w);
  char *ob = static_cast<char *>(out);
  const int64_t bytes = (int64_t)n_experts * rows * K * esz;
  TM_REQUIRE(ob + bytes <= wb || wb + bytes <= ob, TM_EINVAL_ARG, "tm_expert_pack_weights: out overlaps the weights");
  const int64_t KT = K / BK;
  const int64_t blocks = (int64_t)n_experts * (rows / bn) * KT;
  hipStream_t s = tm_hip_stream(stream);
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    if constexpr (DT == TM_DT_F32) {
      return tm_fail(TM_EINVAL_DTYPE, "tm_expert_pack_weights: dtype must be F16 or BF16");
    } else {
      using T = typename Elem<DT>::T;
      if (bn == kMinBN)
        hipLaunchKernelGGL((pack_weights_kernel<T, kMinBN>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                           static_cast<const T *>(w), K, KT, static_cast<T *>(out));
      else
        hipLaunchKernelGGL((pack_weights_kernel<T, 2 * kMinBN>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                           static_cast<const T *>(w), K, KT, static_cast<T *>(out));
      TM_LAUNCH_CHECK("tm_expert_pack_weights");
      return TM_OK;
    }
  });
}

namespace {

int expert_swiglu_impl(const char *name, int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                       const void *w1, const void *w3, const void *w2, int32_t inter, const void *addend,
                       int64_t ld_add, void *out, int64_t ld_out, void *workspace, size_t workspace_bytes,
                       bool packed, tm_stream_t stream) {
  TM_REQUIRE(shapes_ok(hidden, inter), TM_EINVAL_SHAPE, "%s: hidden and inter must be positive multiples of %d",
             name, kMinBN);
  TM_REQUIRE(n_rows >= 0 && n_rows < ((int64_t)1 << 31) && ld_x >= hidden && ld_out >= hidden &&
                 (addend == nullptr || ld_add >= hidden),
             TM_EINVAL_SHAPE, "%s: bad sizes", name);
  if (n_rows == 0) return TM_OK;
  TM_REQUIRE(x && w1 && w3 && w2 && out, TM_EINVAL_ARG, "%s: null pointer", name);
  TM_REQUIRE(tm_aligned16(x) && (ld_x * 2) % 16 == 0 && tm_aligned16(w1) && tm_aligned16(w3) && tm_aligned16(w2) &&
                 tm_aligned16(out) && (ld_out * 2) % 16 == 0 &&
                 (addend == nullptr || (tm_aligned16(addend) && (ld_add * 2) % 16 == 0)),
             TM_EINVAL_SHAPE, "%s: x, out and addend rows and the weights must be 16-byte aligned", name);
  const size_t need = packed ? tm_grouped_swiglu_packed_workspace_size(n_rows, inter, 1, dtype)
                              : tm_swiglu_workspace_size(n_rows, inter, dtype);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need && tm_aligned16(workspace), TM_EWORKSPACE,
             "%s: workspace %zu bytes < %zu", name, workspace_bytes, need);
  const TileSrc ts{nullptr, nullptr, 0, (int32_t)n_rows};
  return swiglu_impl(dtype, x, ld_x, nullptr, hidden, inter, w1, w3, w2, ts, tm_cdiv(n_rows, BM), out, ld_out,
                     nullptr, workspace, addend, ld_add, packed, tm_hip_stream(stream));
}

}  // namespace

extern "C" int tm_expert_swiglu(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                                const void *w1, const void *w3, const void *w2, int32_t inter, void *out,
                                int64_t ld_out, void *workspace, size_t workspace_bytes, tm_stream_t stream) {
  return expert_swiglu_impl("tm_expert_swiglu", dtype, x, n_rows, hidden, ld_x, w1, w3, w2, inter, nullptr, 0, out,
                            ld_out, workspace, workspace_bytes, false, stream);
}

extern "C" int tm_expert_swiglu_add(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                                    const void *w1, const void *w3, const void *w2, int32_t inter,
                                    const void *addend, int64_t ld_add, void *out, int64_t ld_out, void *workspace,
                                    size_t workspace_bytes, tm_stream_t stream) {
  TM_REQUIRE(addend != nullptr, TM_EINVAL_ARG, "tm_expert_swiglu_add: null addend");
  return expert_swiglu_impl("tm_expert_swiglu_add", dtype, x, n_rows, hidden, ld_x, w1, w3, w2, inter, addend, ld_add,
                            out, ld_out, workspace, workspace_bytes, false, stream);
}

extern "C" int tm_expert_swiglu_packed(int32_t dtype, const void *x, int64_t n_rows, int32_t hidden, int64_t ld_x,
                                       const void *w1p, const void *w3p, const void *w2p, int32_t inter,
                                       const void *addend, int64_t ld_add, void *out, int64_t ld_out,
                                       void *workspace, size_t workspace_bytes, tm_stream_t stream) {
  return expert_swiglu_impl("tm_expert_swiglu_packed", dtype, x, n_rows, hidden, ld_x, w1p, w3p, w2p, inter, addend,
                            ld_add, out, ld_out, workspace, workspace_bytes, true, stream);
}
