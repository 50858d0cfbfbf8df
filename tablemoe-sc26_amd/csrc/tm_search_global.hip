// Mode G (global table) nearest-centroid search: north-star kernels (1)+(2).
//
// dist(q, c) = ||q||^2 - 2 q.c + ||c||^2 with q.c on bf16/fp16 MFMA (fp32
// accumulation); only d' = ||c||^2 - 2 q.c is ranked (||q||^2 is constant per
// query) and the n x C score matrix is never written.
//
// Layout of the contraction: D^T = C . Q^T with v_mfma_f32_32x32x16.  The A
// operand is a 32-centroid slab, the B operand is one slab of 32 queries held
// in registers for the whole kernel (DIM/16 k-steps).  In the result each
// lane owns ONE query (column l%32) and 16 centroids, so the running top-k is
// a per-lane register list with no cross-lane traffic until the end.
//
// Two launch shapes:
//  - tile kernel (n > 64): a workgroup owns 256 queries (4 waves x 2 slabs of
//    32, so each A fragment read from LDS feeds two MFMAs) and one range of
//    centroids, streamed in 16 KiB stages through a 4-slot LDS ring filled by
//    direct global->LDS loads, three stages in flight;
//  - stream kernel (n <= 64, decode): the workgroup's waves share the queries
//    and each wave streams its own 32-centroid blocks straight from global
//    memory (next block prefetched), so a small batch still reads the table
//    across the whole chip.
// Invalid centroid positions (past the end of the chunk) carry an infinite
// penalty instead of a branch.
//
// Each workgroup writes its top-k per query as packed keys
// (orderable(d') << 32 | c) into the workspace; merge_kernel reduces the
// splits.  Packed keys make the order total: smaller distance first, then
// lower centroid index.
#include "tm_internal.h"
#include "tm_mfma.h"
#include "tm_route_dev.h"
#include "tm_dma.h"
#include "tm_keep_dev.h"

namespace {

constexpr int kThreads = 256;
constexpr int kQS = 2;      // query slabs per wave in the tile kernel
constexpr int kTileRows = 4 * kQS * 32;
constexpr int kDmaMaxChunk = 2048;  // centroids per workgroup of the tile kernels (start values in LDS)
constexpr int kStreamChunk = 128;  // centroids per split of the stream kernel (one 32-block per wave)

struct SplitPlan {
  bool stream;  // small-n shape
  bool wide;    // top-1 wide tile kernel (8-wave workgroups)
  int qs;       // query slabs per wave
  int64_t row_blocks;
  int64_t nsplit;
  int64_t chunk;  // centroids per split
};

// Wide top-1 tile kernel (search_top1_wide_kernel): 256 queries and one
// centroid range per 8-wave workgroup, 32 KiB stages.
constexpr int kWideThreads = 512;
constexpr int kWideQ = 256;  // queries per workgroup
constexpr int kWideStageBytes = 32768;
constexpr int kWideMinGroups = 192;  // fewer leave too many of the 256 CUs idle
// The layer call's ranked plan takes the wide kernel from 128 workgroups on:
// its key decode and the ranked combine save the keep-select launch, which
// outweighs idle CUs (N = 2048 at C = 8192 fills the chip with half-round
// ranges: 8 tiles x 32 ranges of 256 centroids).
constexpr int kWideDecMinGroups = 128;

struct WidePlan {
  int64_t tiles, nsplit, chunk;
};

inline int64_t wide_rows(int dim) { return kWideStageBytes / (dim * 2); }
// Centroids of a half-round range (two stages).
inline int64_t wide_half_rows(int dim) { return 2 * wide_rows(dim); }

// One workgroup per CU where the shape allows: ranges of whole ring rounds
// (4 stages) or of half a round, at most kDmaMaxChunk centroids (the
// start-value array).
WidePlan plan_wide(int64_t n, int64_t c, int dim) {
  WidePlan p;
  p.tiles = tm_cdiv(n, kWideQ);
  const int64_t unit = 4 * wide_rows(dim);
  const int64_t max_split = tm_cdiv(c, unit);
  const int64_t min_split = tm_cdiv(c, kDmaMaxChunk);
  int64_t want = tm_cdiv(256, p.tiles);
  if (want < min_split) want = min_split;
  if (want > max_split) want = max_split;
  if (want < 1) want = 1;
  p.chunk = tm_cdiv(tm_cdiv(c, want), unit) * unit;
  p.nsplit = tm_cdiv(c, p.chunk);
  // One round per range and still at most half the CUs busy: ranges of half
  // a round (two stages, the kernel's HALF form, d = 128) double the
  // workgroups, up to one per CU.
  if (dim == 128 && p.chunk == unit && p.tiles * p.nsplit * 2 <= 256) {
    const int64_t half = wide_half_rows(dim);
    const int64_t ns = tm_cdiv(c, half);
    if (p.tiles * ns <= 256) {
      p.chunk = half;
      p.nsplit = ns;
    }
  }
  return p;
}

// Row strides the wide kernel's 32-bit buffer offsets cover.
inline bool wide_strides_ok(int64_t ld_q, int64_t ld_c, int dim) {
  const int64_t rows = wide_rows(dim);
  return ld_c * 2 * rows < ((int64_t)1 << 31) && ld_q * 2 * rows < ((int64_t)1 << 31);
}

// Centroid rows per pipelined stage of the tile kernel (16 KiB stages).
static inline int64_t dma_rows(int dim) { return 16384 / (dim * 2); }

// Top-1 searches with d <= 128 run search_top1_kernel (or, for very wide
// centroid strides, search_dma_kernel); its loop covers whole rounds of the
// four-stage ring, so their chunks are a multiple of four stages.
static inline bool top1_tile(int dim, int top_k) { return top_k <= 1 && dim <= 128; }

SplitPlan plan_split(int64_t n, int64_t c, int dim, int top_k) {
  SplitPlan p;
  p.stream = n <= 64;
  p.wide = false;
  if (p.stream) {
    p.qs = n <= 32 ? 1 : 2;
    p.row_blocks = 1;
    p.chunk = kStreamChunk;
    p.nsplit = tm_cdiv(c, p.chunk);
    return p;
  }
  p.qs = kQS;
  p.wide = false;
  if (top1_tile(dim, top_k)) {
    const WidePlan w = plan_wide(n, c, dim);
    if (w.tiles * w.nsplit >= kWideMinGroups) {
      p.wide = true;
      p.row_blocks = w.tiles;  // = tm_cdiv(n, kTileRows): the 4-wave kernels can run the same plan
      p.nsplit = w.nsplit;
      p.chunk = w.chunk;
      return p;
    }
  }
  p.row_blocks = tm_cdiv(n, kTileRows);
  const int64_t rows = dma_rows(dim);
  const int64_t max_split = tm_cdiv(c, rows);
  int64_t want = tm_cdiv(512, p.row_blocks);  // ~2 workgroups per CU
  const int64_t min_split = tm_cdiv(c, 2048);  // the penalty array holds 2048 centroids
  if (want < min_split) want = min_split;
  if (want < 1) want = 1;
  if (want > max_split) want = max_split;
  const int64_t unit = top1_tile(dim, top_k) ? 4 * rows : rows;  // 2048 is a multiple of either
  p.chunk = tm_cdiv(tm_cdiv(c, want), unit) * unit;
  p.nsplit = tm_cdiv(c, p.chunk);
  return p;
}

// Register-list length used for a requested top_k (the first top_k entries
// of a longer list are the same top_k).
static inline int list_len(int top_k) { return top_k <= 1 ? 1 : (top_k <= 4 ? 4 : 8); }

__device__ __forceinline__ uint64_t make_key(float dprime, int c) {
  return ((uint64_t)tm_orderable(dprime) << 32) | (uint32_t)c;
}

// Insert `x` into the ascending list `l` of length K (compare-swap chain).
template <int K>
__device__ __forceinline__ void list_insert(uint64_t (&l)[K], uint64_t x) {
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const uint64_t lo = l[j] < x ? l[j] : x;
    x = l[j] < x ? x : l[j];
    l[j] = lo;
  }
}

// Running best of one lane: top-1 as (value, index) registers, top-k as a
// packed-key list.
template <int K>
struct Best {
  float d;
  int i;
  uint64_t l[K];
  __device__ __forceinline__ void init() {
    d = __builtin_huge_valf();
    i = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < K; ++j) l[j] = ~0ull;
  }
  // candidates arrive in increasing centroid order within a lane
  __device__ __forceinline__ void push(float dp, int c) {
    if constexpr (K == 1) {
      if (dp < d) { d = dp; i = c; }
    } else {
      const uint64_t key = make_key(dp, c);
      if (key < l[K - 1]) list_insert<K>(l, key);
    }
  }
  __device__ __forceinline__ void finalize() {
    if constexpr (K == 1) l[0] = (i == 0x7fffffff || d == __builtin_huge_valf()) ? ~0ull : make_key(d, i);
  }
  // merge with the lane `o` lanes away (same query, other centroids)
  __device__ __forceinline__ void merge_xor(int o) {
    uint64_t other[K];
#pragma unroll
    for (int j = 0; j < K; ++j) other[j] = __shfl_xor(l[j], o, 64);
#pragma unroll
    for (int j = 0; j < K; ++j)
      if (other[j] < l[K - 1]) list_insert<K>(l, other[j]);
  }
};

// Epilogue of one 32x32 block: lane owns query (l%32) and the 16 centroids
// m = 8*(i/4) + 4*(l/32) + (i%4) of the block.  pen[i] = ||c||^2 (L2) or
// 0 (dot) for valid centroids, +inf past the end.
template <int K, int METRIC>
__device__ __forceinline__ void block_epilogue(const tm_f32x16 &acc, const float (&pen)[16], int cbase,
                                               int lane, Best<K> &best) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = cbase + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    const float dp = (METRIC == TM_METRIC_L2) ? fmaf(-2.f, acc[i], pen[i]) : (pen[i] - acc[i]);
    best.push(dp, c);
  }
}

// ---------------------------------------------------------------------------
// Pipelined tile kernel: centroid stages arrive through direct global->LDS
// loads (global_load_lds_dwordx4: lane l of a wave writes LDS bytes
// [M0 + 16 l, M0 + 16 l + 16)), kDmaBufs stages in a ring, kDmaBufs - 1 of
// them in flight while one is multiplied.  Each ring slot is its own LDS
// array and the loop is unrolled over the ring, so the compiler can tell the
// loads of one slot from the reads of another and the only waits are the
// explicit ones below (one per stage, before the stage's barrier).
//
// A stage holds kDmaRows centroid rows as 16-byte chunks.  Chunk j of row r
// is stored at slot r*CH + (j ^ (r % CH)) (CH = chunks per row): the
// matrix-core operand reads (32 rows at one chunk) then fall in distinct
// banks.  The lane that fills slot p loads the chunk that belongs there.
// The penalty ||c||^2 of the workgroup's whole centroid range is staged in
// LDS once, +inf past the end of the range (rows past the end are loaded
// from the last valid row and lose on their infinite penalty).
// ---------------------------------------------------------------------------
constexpr int kDmaBufs = 4;
constexpr int kDmaStageBytes = 16384;



template <int DT, int DIM, int K, int METRIC>
__global__ __launch_bounds__(kThreads, 2) void search_dma_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t n, int64_t ld_q,
    const typename Elem<DT>::T *__restrict__ cents, int64_t n_cent, int64_t ld_c,
    const float *__restrict__ c_sqnorm, int64_t chunk, uint64_t *__restrict__ ws) {
  using T = typename Elem<DT>::T;
  constexpr int KS = DIM / 16;                       // k-steps of the 32x32x16 MFMA
  constexpr int CH = DIM / 8;                        // 16-byte chunks per centroid row
  constexpr int ROWS = kDmaStageBytes / (DIM * 2);   // centroid rows per stage
  constexpr int NSUB = ROWS / 32;                    // 32-row MFMA blocks per stage
  constexpr int SLOTS = ROWS * CH;                   // 16-byte chunks per stage
  constexpr int NDMA = SLOTS / kThreads;             // loads per thread (= per wave instruction count) per stage
  static_assert(SLOTS % kThreads == 0 && NSUB >= 1, "stage shape");
  __shared__ uint4 st0[SLOTS], st1[SLOTS], st2[SLOTS], st3[SLOTS];
  __shared__ float pen_s[kDmaMaxChunk];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t split = blockIdx.y;
  const int64_t row_base = (int64_t)blockIdx.x * kTileRows + wave * (kQS * 32);
  const int64_t c_begin = split * chunk;
  const int64_t c_end = (c_begin + chunk < n_cent) ? c_begin + chunk : n_cent;
  const int64_t c_last = c_end - 1;
  const int nstage = (int)((c_end - c_begin + ROWS - 1) / ROWS);
  const T *q_rows[kQS];
#pragma unroll
  for (int sl = 0; sl < kQS; ++sl) {
    const int64_t r = row_base + sl * 32 + (lane & 31);
    q_rows[sl] = (r < n) ? q + r * ld_q : nullptr;
  }

  // ring fill: slot p = tid + 256 u of stage `s` (clamped to the last stage,
  // so every wave issues the same number of loads per step)
  auto issue = [&](uint4 *buf, int s) {
    const int sc = s < nstage - 1 ? s : nstage - 1;
    const int64_t r0 = c_begin + (int64_t)sc * ROWS;
#pragma unroll
    for (int u = 0; u < NDMA; ++u) {
      const int p = tid + u * kThreads;
      const int r = p / CH;
      const int j = (p % CH) ^ (r % CH);
      const int64_t row = (r0 + r < c_last) ? r0 + r : c_last;
      tm_dma16(cents + row * ld_c + j * 8, &buf[p - lane]);
    }
  };
  // Issue order: penalties, the first ring stages, the queries; the penalty
  // stores to LDS then wait only for the penalty loads.
  constexpr int PEN_PER_THREAD = kDmaMaxChunk / kThreads;
  float pen_v[PEN_PER_THREAD];
#pragma unroll
  for (int u = 0; u < PEN_PER_THREAD; ++u) {
    const int64_t c = c_begin + tid + u * kThreads;
    const float v = (METRIC == TM_METRIC_L2) ? c_sqnorm[c < c_last ? c : c_last] : 0.f;
    pen_v[u] = (c < c_end) ? v : __builtin_huge_valf();
  }
  issue(st0, 0);
  issue(st1, 1);
  issue(st2, 2);

  // B operands: kQS slabs of 32 queries, all k-steps, in registers.
  uint4 qf[kQS][KS];
#pragma unroll
  for (int sl = 0; sl < kQS; ++sl)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[sl][ks] = q_rows[sl] ? *reinterpret_cast<const uint4 *>(q_rows[sl] + ks * 16 + 8 * (lane >> 5))
                              : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int u = 0; u < PEN_PER_THREAD; ++u) pen_s[tid + u * kThreads] = pen_v[u];

  Best<K> best[kQS];
#pragma unroll
  for (int sl = 0; sl < kQS; ++sl) best[sl].init();

  auto step = [&](const uint4 *cur, uint4 *refill, int s) {
    tm_wait_vm_lgkm0<2 * NDMA>();  // this stage's loads are done (two younger stages may be in flight)
    __builtin_amdgcn_s_barrier();  // ... and every wave's, and the slot refilled below is free
    issue(refill, s + kDmaBufs - 1);
    const int64_t s0 = c_begin + (int64_t)s * ROWS;
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int row = sub * 32 + (lane & 31);
      tm_f32x16 acc[kQS];
#pragma unroll
      for (int sl = 0; sl < kQS; ++sl) acc[sl] = tm_f32x16{};
      constexpr int AB = KS < 8 ? KS : 8;  // A fragments read ahead of their MFMAs
#pragma unroll
      for (int k0 = 0; k0 < KS; k0 += AB) {
        uint4 a[AB];
#pragma unroll
        for (int u = 0; u < AB; ++u) {
          const int j = 2 * (k0 + u) + (lane >> 5);
          a[u] = cur[row * CH + (j ^ (row % CH))];
        }
#pragma unroll
        for (int u = 0; u < AB; ++u)
#pragma unroll
          for (int sl = 0; sl < kQS; ++sl) acc[sl] = tm_mfma32x32x16<DT>(a[u], qf[sl][k0 + u], acc[sl]);
      }
      float pen[16];
      const int pb = s * ROWS + sub * 32 + 4 * (lane >> 5);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 p4 = *reinterpret_cast<const float4 *>(&pen_s[pb + 8 * g]);
        pen[4 * g + 0] = p4.x; pen[4 * g + 1] = p4.y; pen[4 * g + 2] = p4.z; pen[4 * g + 3] = p4.w;
      }
#pragma unroll
      for (int sl = 0; sl < kQS; ++sl) block_epilogue<K, METRIC>(acc[sl], pen, (int)(s0 + sub * 32), lane, best[sl]);
    }
  };
  for (int s = 0; s < nstage; s += kDmaBufs) {
    step(st0, st3, s);
    if (s + 1 < nstage) step(st1, st0, s + 1);  // uniform
    if (s + 2 < nstage) step(st2, st1, s + 2);
    if (s + 3 < nstage) step(st3, st2, s + 3);
  }
  tm_wait_vm_lgkm0<0>();  // no load may still target this workgroup's LDS when it exits

#pragma unroll
  for (int sl = 0; sl < kQS; ++sl) {
    best[sl].finalize();
    best[sl].merge_xor(32);  // the two half-waves saw disjoint centroids of the same query
    const int64_t r = row_base + sl * 32 + (lane & 31);
    if (lane < 32 && r < n) {
      uint64_t *dst = ws + (split * n + r) * K;
#pragma unroll
      for (int j = 0; j < K; ++j) dst[j] = best[sl].l[j];
    }
  }
}

// ---------------------------------------------------------------------------
// Top-1 tile kernel (the prefill shape): the stage layout of search_dma_kernel
// (256 queries x one centroid range per workgroup, 16 KiB stages of swizzled
// centroid rows in a 4-slot LDS ring), with the work software-pipelined
// inside each wave: while the matrix cores multiply block b (32 centroids x
// 2 query slabs), the same wave runs block b-1's epilogue and reads block
// b+1's operands, so neither sits between two blocks' MFMAs.  Blocks
// alternate between two accumulator sets; sched_group_barrier pins the
// interleave (per k-step: 2 MFMAs, a share of the epilogue, one LDS read).
//
// Epilogue: the accumulator of a block starts from -||c||^2/2 (L2) or 0
// (dot), -inf past the end of the range, and so ends at -d'/2 or -d': the
// nearest centroid holds the LARGEST value.  Per block only the block
// maximum is computed (a max3 tree); where it beats the lane's running
// maximum, the block's 16 values and its first centroid are kept (selects,
// no branch).  At the end the first kept position holding the maximum names
// the centroid.  Strict comparisons keep the earliest block, and within a
// lane position order is centroid order, so ties go to the lower index.
//
// Ring: stages are loaded by buffer loads straight into LDS, two stages
// ahead.  The barrier before the last block of stage t waits for stage t+1
// and refills the slot of stage t-1 (read by no wave any more) with stage
// t+3.  The stage count is padded to whole rounds of the ring so the loop
// body has no branch; padded stages meet -inf start values.
// ---------------------------------------------------------------------------

struct Top1Lane {
  float r;      // running maximum
  int cb;       // first centroid of the block it came from (-1: none)
  float s[16];  // that block's values
};

__device__ __forceinline__ void top1_init(Top1Lane &t) {
  t.r = -__builtin_huge_valf();
  t.cb = -1;
#pragma unroll
  for (int i = 0; i < 16; ++i) t.s[i] = t.r;
}

// ~10 (max tree) + 1 + 18 (selects) VALU ops, no branch.
__device__ __forceinline__ void top1_update(Top1Lane &t, const tm_f32x16 &acc, int cbase) {
  const float m0 = fmaxf(fmaxf(acc[0], acc[1]), acc[2]);
  const float m1 = fmaxf(fmaxf(acc[3], acc[4]), acc[5]);
  const float m2 = fmaxf(fmaxf(acc[6], acc[7]), acc[8]);
  const float m3 = fmaxf(fmaxf(acc[9], acc[10]), acc[11]);
  const float m4 = fmaxf(fmaxf(acc[12], acc[13]), acc[14]);
  const float m = fmaxf(fmaxf(fmaxf(m0, m1), m2), fmaxf(fmaxf(m3, m4), acc[15]));
  const bool gt = m > t.r;
  t.r = gt ? m : t.r;
  t.cb = gt ? cbase : t.cb;
#pragma unroll
  for (int i = 0; i < 16; ++i) t.s[i] = gt ? acc[i] : t.s[i];
}

// The first kept position holding the maximum names the centroid.
template <int METRIC>
__device__ __forceinline__ void top1_to_best(const Top1Lane &t, int lane, Best<1> &b) {
  int pos = 15;
#pragma unroll
  for (int i = 14; i >= 0; --i)
    if (t.s[i] == t.r) pos = i;
  if (t.cb >= 0) {
    b.d = (METRIC == TM_METRIC_L2) ? -2.f * t.r : -t.r;
    b.i = t.cb + 8 * (pos >> 2) + 4 * (lane >> 5) + (pos & 3);
  }
}

template <int DT, int DIM, int METRIC>
__global__ __launch_bounds__(kThreads, 2) void search_top1_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t n, int64_t ld_q,
    const typename Elem<DT>::T *__restrict__ cents, int64_t n_cent, int64_t ld_c,
    const float *__restrict__ c_sqnorm, int64_t chunk, uint64_t *__restrict__ ws, uint64_t *__restrict__ keys) {
  using T = typename Elem<DT>::T;
  constexpr int KS = DIM / 16;
  constexpr int CH = DIM / 8;
  constexpr int ROWS = kDmaStageBytes / (DIM * 2);
  constexpr int NSUB = ROWS / 32;
  constexpr int SLOTS = ROWS * CH;
  constexpr int NDMA = SLOTS / kThreads;
  static_assert(SLOTS % kThreads == 0 && NSUB >= 1, "stage shape");
  __shared__ uint4 st0[SLOTS], st1[SLOTS], st2[SLOTS], st3[SLOTS];
  __shared__ float init_s[kDmaMaxChunk];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t split = blockIdx.y;
  const int64_t row_base = (int64_t)blockIdx.x * kTileRows + wave * (kQS * 32);
  const int64_t c_begin = split * chunk;
  const int64_t c_end = (c_begin + chunk < n_cent) ? c_begin + chunk : n_cent;
  const int64_t c_last = c_end - 1;
  const int nstage = (int)((c_end - c_begin + ROWS - 1) / ROWS);
  const int nstage4 = (nstage + kDmaBufs - 1) / kDmaBufs * kDmaBufs;  // <= kDmaMaxChunk / ROWS
  const T *q_rows[kQS];
#pragma unroll
  for (int sl = 0; sl < kQS; ++sl) {
    const int64_t r = row_base + sl * 32 + (lane & 31);
    q_rows[sl] = (r < n) ? q + r * ld_q : nullptr;
  }

  // Ring fill of stage `s`: a buffer over the table from the stage's first row
  // on, so rows past the end of the table read nothing (the range's rows past
  // c_end are read but carry a -inf start value).  Thread t's chunk u sits at
  // a fixed byte offset from the stage's first row: chunk 0's plus
  // u * (256 / CH) rows (the swizzle repeats every CH rows).  The host keeps
  // ROWS * ld_c * sizeof(T) below 2^31.
  static_assert(CH <= 16, "one swizzle period per 256 chunks");
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint64_t ldb = (uint64_t)ld_c * sizeof(T);
  constexpr int kRowsPerU = kThreads / CH;
  uint32_t voff[NDMA];
#pragma unroll
  for (int u = 0; u < NDMA; ++u) {
    const int r = tid / CH + u * kRowsPerU;
    const int j = (tid % CH) ^ (r % CH);
    voff[u] = (uint32_t)r * (uint32_t)ldb + (uint32_t)j * 16u;
  }
  auto issue = [&](uint4 *buf, int s) {
    const uint32_t lds0 = (uint32_t)(uintptr_t)buf + (uint32_t)wave_u * 1024u;
    // the resource ends with the workgroup's range: rows past it (the stages
    // of the last ring round past the range, a partial last stage) read
    // nothing instead of another range's centroids
    const int64_t row0 = __builtin_elementwise_min(c_begin + (int64_t)s * ROWS, c_end);
    const tm_rsrc_t rs = tm_make_rsrc(cents + row0 * ld_c, (uint64_t)(c_end - row0) * ldb);
#pragma unroll
    for (int u = 0; u < NDMA; ++u) tm_dma16_buf(rs, voff[u], lds0 + (uint32_t)(u * kThreads * 16));
  };
  constexpr int INIT_PER_THREAD = kDmaMaxChunk / kThreads;
  float init_v[INIT_PER_THREAD];
#pragma unroll
  for (int u = 0; u < INIT_PER_THREAD; ++u) {
    const int64_t c = c_begin + tid + u * kThreads;
    const float v = (METRIC == TM_METRIC_L2) ? -0.5f * c_sqnorm[c < c_last ? c : c_last] : 0.f;
    init_v[u] = (c < c_end) ? v : -__builtin_huge_valf();
  }
  issue(st0, 0);
  issue(st1, 1);
  uint4 qf[kQS][KS];
#pragma unroll
  for (int sl = 0; sl < kQS; ++sl)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[sl][ks] = q_rows[sl] ? *reinterpret_cast<const uint4 *>(q_rows[sl] + ks * 16 + 8 * (lane >> 5))
                              : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int u = 0; u < INIT_PER_THREAD; ++u) init_s[tid + u * kThreads] = init_v[u];

  static_assert(NSUB % 2 == 0, "blocks alternate between two accumulator sets");
  Top1Lane top[kQS];
  // Accumulators of even and odd blocks: block b fills set b&1 while the
  // epilogue of block b-1 reads set (b-1)&1 (no copy between them).
  tm_f32x16 accs[2][kQS];
  int cbs[2] = {0, 0};  // first centroid of the block in each set
#pragma unroll
  for (int sl = 0; sl < kQS; ++sl) {
    top1_init(top[sl]);
#pragma unroll
    for (int i = 0; i < 16; ++i) accs[1][sl][i] = -__builtin_huge_valf();
  }

  // Lane byte offsets of A operand k within a 32-row block (the same for
  // every block, slot and stage).  Made opaque to the compiler so that the
  // slot and block offsets stay additive immediates of the LDS reads.
  uint32_t a_off[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int row = lane & 31;
    const int j = 2 * k + (lane >> 5);
    a_off[k] = (uint32_t)(row * CH + (j ^ (row % CH))) * 16u;
    asm volatile("" : "+v"(a_off[k]));
  }
  uint32_t i_off = (uint32_t)(16 * (lane >> 5));
  asm volatile("" : "+v"(i_off));
  // A operands are read kAhead k-steps before their MFMAs (a sliding window
  // that runs into the next block), start values near the end of the block
  // before; only kAhead + 1 operand registers are live at a time.
  constexpr int kAhead = KS >= 8 ? 3 : 2;
  static_assert(KS >= 4 && kAhead < KS, "window shorter than a block");
  uint4 fa[KS];
  float fi[16];
  auto read_a = [&](const uint4 *buf, int sub, int k) {
    fa[k] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const char *>(buf) + sub * 32 * CH * 16 + a_off[k]);
  };
  auto read_start = [&](int s, int sub) {
    const int sc = s < nstage4 ? s : nstage4 - 1;  // the read past the last stage: any in-range values
    const char *ib = reinterpret_cast<const char *>(init_s) + (sc * ROWS + sub * 32) * 4 + i_off;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 p4 = *reinterpret_cast<const float4 *>(ib + 32 * g);
      fi[4 * g + 0] = p4.x; fi[4 * g + 1] = p4.y; fi[4 * g + 2] = p4.z; fi[4 * g + 3] = p4.w;
    }
  };

  // Two stages in flight: the barrier before the last block of stage t waits
  // for stage t+1 (stage t+2 may still be loading) and refills the slot of
  // stage t-1, which every wave has finished reading, with stage t+3.
  tm_wait_vm_lgkm0<0>();  // stages 0, 1 and the query operands landed; init_s written
  __builtin_amdgcn_s_barrier();
  issue(st2, 2);
  read_start(0, 0);
#pragma unroll
  for (int k = 0; k < kAhead; ++k) read_a(st0, 0, k);

  // stage s: slot `cur`; stage s+1: `nxt`; `old` (stage s-1's) is refilled with stage s+3
  auto step = [&](const uint4 *cur, const uint4 *nxt, uint4 *old, int s) {
    const int64_t s0 = c_begin + (int64_t)s * ROWS;
    tm_static_for<NSUB>([&](auto sub_c) {
      constexpr int sub = decltype(sub_c)::value;
      constexpr int PA = sub & 1;  // this block's accumulator set
      if (sub == NSUB - 1) {
        tm_wait_vm_lgkm0<NDMA>();      // stage s+1 landed (stage s+2 may be in flight)
        __builtin_amdgcn_s_barrier();  // ... in every wave; stage s-1's slot is no longer read
        issue(old, s + 3);
      }
      tm_f32x16 (&acc)[kQS] = accs[PA];
      tm_f32x16 start;
#pragma unroll
      for (int i = 0; i < 16; ++i) start[i] = fi[i];
      tm_static_for<KS>([&](auto k_c) {
        constexpr int k = decltype(k_c)::value;
#pragma unroll
        for (int sl = 0; sl < kQS; ++sl) acc[sl] = tm_mfma32x32x16<DT>(fa[k], qf[sl][k], k == 0 ? start : acc[sl]);
        constexpr int kk = k + kAhead;  // operand read this step
        if constexpr (kk < KS)
          read_a(cur, sub, kk);
        else if constexpr (sub + 1 < NSUB)
          read_a(cur, sub + 1, kk - KS);
        else
          read_a(nxt, 0, kk - KS);
        if constexpr (k == KS - 3) {
          if constexpr (sub + 1 < NSUB)
            read_start(s, sub + 1);
          else
            read_start(s + 1, 0);
        }
      });
#pragma unroll
      for (int sl = 0; sl < kQS; ++sl) top1_update(top[sl], accs[PA ^ 1][sl], cbs[PA ^ 1]);
      cbs[PA] = (int)(s0 + sub * 32);
      // per k-step: its MFMAs, a share of the previous block's epilogue, a read
      constexpr int kValu = (30 * kQS + KS - 1) / KS;
      tm_static_for<KS>([&](auto k_c) {
        constexpr int k = decltype(k_c)::value;
        __builtin_amdgcn_sched_group_barrier(0x008, kQS, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x100, k == KS - 3 ? 5 : 1, 0);  // DS read
      });
      __builtin_amdgcn_sched_barrier(0);  // blocks are scheduled one at a time
    });
  };
  // Whole rounds of the ring: stages past the range only meet -inf start
  // values (and rows past the table read nothing), so padding nstage to a
  // multiple of the ring keeps the loop body free of branches.
  for (int s = 0; s < nstage4; s += kDmaBufs) {
    step(st0, st1, st3, s);
    step(st1, st2, st0, s + 1);
    step(st2, st3, st1, s + 2);
    step(st3, st0, st2, s + 3);
  }
#pragma unroll
  for (int sl = 0; sl < kQS; ++sl) top1_update(top[sl], accs[1][sl], cbs[1]);  // the last block is odd
  tm_wait_vm_lgkm0<0>();  // no load may still target this workgroup's LDS when it exits

#pragma unroll
  for (int sl = 0; sl < kQS; ++sl) {
    Best<1> best;
    best.init();
    top1_to_best<METRIC>(top[sl], lane, best);
    best.finalize();
    best.merge_xor(32);  // the two half-waves saw disjoint centroids of the same query
    const int64_t r = row_base + sl * 32 + (lane & 31);
    if (lane < 32 && r < n) {
      if (keys == nullptr)
        ws[split * n + r] = best.l[0];
      else if (best.l[0] != ~0ull)
        atomicMin(reinterpret_cast<unsigned long long *>(keys + r), (unsigned long long)best.l[0]);
    }
  }
}

// ---------------------------------------------------------------------------
// Top-1 tile kernel, wide form (the layer call's fused top-1 plan, large n):
// one 8-wave workgroup per CU owns 256 queries and one range of centroids.
// Waves w and w + 4 hold the same 64 queries (two slabs of 32) and take the
// even and the odd 32-row blocks of each 32 KiB stage, so a CU fetches its
// queries once and every centroid stage once for all 8 waves (per CU:
// 64 KiB of queries + the range's centroids, against 2 x (64 + 64) KiB for
// two 4-wave workgroups).
//
// The query tile travels through the ring: direct global->LDS loads bring
// whole rows (4 rows of 256 bytes per wave instruction, where register loads
// in the operand layout touch 32 rows per instruction) into ring slots 2
// and 3 while stage 0 fills slot 0; the waves read their fragments into
// registers and the slots go back to the ring (stage 2, then 3).  The swizzle
// of a query row is the one of a centroid row, so the fragment offsets are
// those of the A operand.
//
// Blocks: stage s, block i of a wave is the stage's block 2i + half (half =
// wave / 4).  The accumulator sets, the one-block-behind epilogue and the
// stage waits are those of search_top1_kernel.  The two halves' keys of a
// query meet in LDS; then one store per query and workgroup into the
// per-split key array keys[split][n] (DEC false: tm_search_global, merged by
// merge_top1_kernel) or one atomic minimum into keys[n] (DEC true: the layer
// call).
//
// HALF: the range is at most two stages (half a ring round), run as two
// steps without the round loop.
//
// With DEC, the workgroup that finishes a query tile last (one arrival
// counter per tile, zero before the launch and left zero) decodes the
// tile's finished keys into distance, centroid and |q|^2 (device-coherent
// key loads: the other splits' minima were made on other CUs in this launch).
// ---------------------------------------------------------------------------
struct WideDecode {
  const float *qn_part;  // [parts][n] partial |q|^2
  int parts;
  float *out_dist;
  int64_t *out_idx;
  float *out_qn;
  uint32_t *cnt;  // one per query tile
};

template <int DT, int DIM, int METRIC, bool DEC, bool HALF>
__global__ __launch_bounds__(kWideThreads, 1) void search_top1_wide_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t n, int64_t ld_q,
    const typename Elem<DT>::T *__restrict__ cents, int64_t n_cent, int64_t ld_c,
    const float *__restrict__ c_sqnorm, int64_t chunk, uint64_t *__restrict__ keys, WideDecode wd) {
  using T = typename Elem<DT>::T;
  constexpr int KS = DIM / 16;
  constexpr int CH = DIM / 8;
  constexpr int ROWS = kWideStageBytes / (DIM * 2);
  constexpr int NSUB = ROWS / 32;
  constexpr int NBW = NSUB / 2;  // blocks per stage of one wave
  constexpr int SLOTS = ROWS * CH;
  constexpr int NDMA = SLOTS / kWideThreads;
  constexpr int QST = kWideQ / ROWS;  // ring slots of the query tile
  static_assert(SLOTS % kWideThreads == 0 && NBW % 2 == 0 && (QST == 1 || QST == 2), "stage shape");
  static_assert(CH <= 16 && (kWideThreads / CH) % CH == 0, "one swizzle period per load row group");
  __shared__ uint4 ring[4 * SLOTS];
  __shared__ float init_s[kDmaMaxChunk];
  __shared__ uint64_t half_keys[4][64];  // odd-block waves' keys of each query group
  __shared__ uint32_t s_last;
  uint4 *const st0 = ring;
  uint4 *const st1 = ring + SLOTS;
  uint4 *const st2 = ring + 2 * SLOTS;
  uint4 *const st3 = ring + 3 * SLOTS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qg = wave & 3;
  const int half = wave >> 2;
  // x: centroid range (the 8 XCDs each see a few ranges), y: query tile
  const int64_t split = blockIdx.x;
  const int64_t tile0 = (int64_t)blockIdx.y * kWideQ;
  const int64_t row_base = tile0 + qg * 64;
  const int64_t c_begin = split * chunk;
  const int64_t c_end = (c_begin + chunk < n_cent) ? c_begin + chunk : n_cent;
  const int64_t c_last = c_end - 1;
  const int nstage = (int)((c_end - c_begin + ROWS - 1) / ROWS);
  const int nstage4 = (nstage + 3) / 4 * 4;  // <= kDmaMaxChunk / ROWS

  // Ring fills: thread t's chunk u of a stage is row t / CH + u * (512 / CH),
  // global chunk (t % CH) ^ (row % CH), LDS slot u * 512 + t.  Rows past the
  // table (or past n for the query tile) read nothing.  The host keeps
  // ROWS * row stride below 2^31 bytes.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint64_t ldb = (uint64_t)ld_c * sizeof(T);
  const uint64_t ldqb = (uint64_t)ld_q * sizeof(T);
  constexpr int kRowsPerU = kWideThreads / CH;
  uint32_t voff[NDMA];
#pragma unroll
  for (int u = 0; u < NDMA; ++u) {
    const int r = tid / CH + u * kRowsPerU;
    const int j = (tid % CH) ^ (r % CH);
    voff[u] = (uint32_t)r * (uint32_t)ldb + (uint32_t)j * 16u;
  }
  auto issue = [&](uint4 *buf, int s) {
    const uint32_t lds0 = (uint32_t)(uintptr_t)buf + (uint32_t)wave_u * 1024u;
    // the resource ends with the workgroup's range: rows past it (the stages
    // of the last ring round past the range, a partial last stage) read
    // nothing instead of another range's centroids
    const int64_t row0 = __builtin_elementwise_min(c_begin + (int64_t)s * ROWS, c_end);
    const tm_rsrc_t rs = tm_make_rsrc(cents + row0 * ld_c, (uint64_t)(c_end - row0) * ldb);
#pragma unroll
    for (int u = 0; u < NDMA; ++u) tm_dma16_buf(rs, voff[u], lds0 + (uint32_t)(u * kWideThreads * 16));
  };
  auto issue_q = [&](uint4 *buf, int part) {
    const uint32_t lds0 = (uint32_t)(uintptr_t)buf + (uint32_t)wave_u * 1024u;
    const int64_t row0 = __builtin_elementwise_min(tile0 + (int64_t)part * ROWS, n);
    const tm_rsrc_t rs = tm_make_rsrc(q + row0 * ld_q, (uint64_t)(n - row0) * ldqb);
#pragma unroll
    for (int u = 0; u < NDMA; ++u) {
      const int r = tid / CH + u * kRowsPerU;
      const int j = (tid % CH) ^ (r % CH);
      tm_dma16_buf(rs, (uint32_t)r * (uint32_t)ldqb + (uint32_t)j * 16u, lds0 + (uint32_t)(u * kWideThreads * 16));
    }
  };
  constexpr int IPT = kDmaMaxChunk / kWideThreads;
  float sqn[IPT];
#pragma unroll
  for (int u = 0; u < IPT; ++u) {
    const int64_t c = c_begin + tid + u * kWideThreads;
    sqn[u] = (METRIC == TM_METRIC_L2) ? c_sqnorm[c < c_last ? c : c_last] : 0.f;
  }
  issue_q(st2, 0);
  if constexpr (QST == 2) issue_q(st3, 1);
  issue(st0, 0);
  // The start values are formed only now: left to itself the compiler
  // computed them (waiting for the norms) before issuing the ring loads.
#pragma unroll
  for (int u = 0; u < IPT; ++u) asm volatile("" : "+v"(sqn[u]));
  tm_wait_vm_lgkm0<0>();  // norms, the query tile and stage 0 (this thread's loads)
#pragma unroll
  for (int u = 0; u < IPT; ++u) {
    const int64_t c = c_begin + tid + u * kWideThreads;
    init_s[tid + u * kWideThreads] = (c < c_end) ? ((METRIC == TM_METRIC_L2) ? -0.5f * sqn[u] : 0.f)
                                                 : -__builtin_huge_valf();
  }
  issue(st1, 1);
  tm_wait_vm_lgkm0<NDMA>();  // init_s written; stage 1 may still load
  __builtin_amdgcn_s_barrier();

  // Lane byte offsets of operand k within a 32-row block (see
  // search_top1_kernel); the query fragments use them as they are, the
  // centroid blocks of this half one block further.
  uint32_t a_off[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int row = lane & 31;
    const int j = 2 * k + (lane >> 5);
    a_off[k] = (uint32_t)(row * CH + (j ^ (row % CH))) * 16u;
  }
  uint4 qf[2][KS];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    const int t0 = qg * 64 + sl * 32;  // tile row of the slab
    const char *qb = reinterpret_cast<const char *>(t0 < ROWS ? st2 : st3) + (t0 % ROWS) * CH * 16;
#pragma unroll
    for (int k = 0; k < KS; ++k) qf[sl][k] = *reinterpret_cast<const uint4 *>(qb + a_off[k]);
  }
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    a_off[k] += (uint32_t)(half * 32 * CH * 16);
    asm volatile("" : "+v"(a_off[k]));
  }
  uint32_t i_off = (uint32_t)(16 * (lane >> 5) + 128 * half);
  asm volatile("" : "+v"(i_off));

  Top1Lane top[2];
  tm_f32x16 accs[2][2];
  int cbs[2] = {0, 0};
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    top1_init(top[sl]);
#pragma unroll
    for (int i = 0; i < 16; ++i) accs[1][sl][i] = -__builtin_huge_valf();
  }
  constexpr int kAhead = KS >= 8 ? 3 : 2;
  static_assert(KS >= 4 && kAhead < KS, "window shorter than a block");
  uint4 fa[KS];
  float fi[16];
  auto read_a = [&](const uint4 *buf, int i, int k) {
    fa[k] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const char *>(buf) + i * 64 * CH * 16 + a_off[k]);
  };
  auto read_start = [&](int s, int i) {
    const int sc = s < nstage4 ? s : nstage4 - 1;  // the read past the last stage: any in-range values
    const char *ib = reinterpret_cast<const char *>(init_s) + (sc * ROWS + i * 64) * 4 + i_off;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 p4 = *reinterpret_cast<const float4 *>(ib + 32 * g);
      fi[4 * g + 0] = p4.x; fi[4 * g + 1] = p4.y; fi[4 * g + 2] = p4.z; fi[4 * g + 3] = p4.w;
    }
  };
  read_start(0, 0);
#pragma unroll
  for (int k = 0; k < kAhead; ++k) read_a(st0, 0, k);
  tm_wait_vm_lgkm0<NDMA>();  // query fragments in registers
  __builtin_amdgcn_s_barrier();  // ... in every wave: slots 2 and 3 go back to the ring
  issue(st2, 2);

  auto step = [&](const uint4 *cur, const uint4 *nxt, uint4 *old, int s) {
    const int64_t s0 = c_begin + (int64_t)s * ROWS + half * 32;
    tm_static_for<NBW>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      constexpr int PA = i & 1;
      if (i == NBW - 1) {
        tm_wait_vm_lgkm0<NDMA>();      // stage s+1 landed (stage s+2 may be in flight)
        __builtin_amdgcn_s_barrier();  // ... in every wave; stage s-1's slot is no longer read
        issue(old, s + 3);
      }
      tm_f32x16 (&acc)[2] = accs[PA];
      tm_f32x16 start;
#pragma unroll
      for (int e = 0; e < 16; ++e) start[e] = fi[e];
      tm_static_for<KS>([&](auto k_c) {
        constexpr int k = decltype(k_c)::value;
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) acc[sl] = tm_mfma32x32x16<DT>(fa[k], qf[sl][k], k == 0 ? start : acc[sl]);
        constexpr int kk = k + kAhead;
        if constexpr (kk < KS)
          read_a(cur, i, kk);
        else if constexpr (i + 1 < NBW)
          read_a(cur, i + 1, kk - KS);
        else
          read_a(nxt, 0, kk - KS);
        if constexpr (k == KS - 3) {
          if constexpr (i + 1 < NBW)
            read_start(s, i + 1);
          else
            read_start(s + 1, 0);
        }
      });
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) top1_update(top[sl], accs[PA ^ 1][sl], cbs[PA ^ 1]);
      cbs[PA] = (int)(s0 + i * 64);
      constexpr int kValu = (30 * 2 + KS - 1) / KS;
      tm_static_for<KS>([&](auto k_c) {
        constexpr int k = decltype(k_c)::value;
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, k == KS - 3 ? 5 : 1, 0);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  if constexpr (HALF) {
    // Half-round range (at most two stages): the two steps alone; the loads
    // of the stages past the range read nothing, target this workgroup's
    // ring and are waited for below, and the operands read ahead from slot
    // 2 are never used.
    step(st0, st1, st3, 0);
    step(st1, st2, st0, 1);
  } else {
    for (int s = 0; s < nstage4; s += 4) {
      step(st0, st1, st3, s);
      step(st1, st2, st0, s + 1);
      step(st2, st3, st1, s + 2);
      step(st3, st0, st2, s + 3);
    }
  }
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) top1_update(top[sl], accs[1][sl], cbs[1]);  // the last block is odd
  tm_wait_vm_lgkm0<0>();  // no load may still target this workgroup's LDS when it exits

  uint64_t bk[2];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    Best<1> best;
    best.init();
    top1_to_best<METRIC>(top[sl], lane, best);
    best.finalize();
    best.merge_xor(32);  // the two half-waves saw disjoint centroids of the same query
    bk[sl] = best.l[0];
    if (half == 1 && lane < 32) half_keys[qg][sl * 32 + lane] = bk[sl];
  }
  __syncthreads();
  if (half == 0) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const int64_t r = row_base + sl * 32 + (lane & 31);
      const uint64_t o = half_keys[qg][sl * 32 + (lane & 31)];
      const uint64_t key = bk[sl] < o ? bk[sl] : o;
      if (lane < 32 && r < n) {
        if constexpr (!DEC)
          keys[split * n + r] = key;  // per-split keys, merged by merge_top1_kernel
        else if (key != ~0ull)
          atomicMin(reinterpret_cast<unsigned long long *>(keys + r), (unsigned long long)key);
      }
    }
  }
  if constexpr (DEC) {
    // Arrival: every thread's key updates performed, then one ticket per tile.
    // Ordering argument (the same as the decode plan's projection hand-off):
    // the keys are only ever touched by device-scope atomics (atomicMin here,
    // the relaxed agent-scope load below), which the hardware performs at
    // one point of coherence per address for every XCD, bypassing the
    // non-coherent per-XCD L2 for the load (sc1).  On gfx9 vmcnt also counts
    // returnless atomics, so the s_waitcnt vmcnt(0) below returns only after
    // this workgroup's atomicMins are acknowledged, and only then is the
    // ticket taken; the last ticket therefore follows every tile workgroup's
    // updates, and its keys load is issued after it returns.  The HIP memory
    // model proper would ask for agent-scope release/acquire fences around
    // the ticket instead; those write back and invalidate the whole L2
    // (buffer_wbl2 / buffer_inv), measured at several microseconds per
    // launch of this shape, so the kernel relies on the per-address
    // coherence of its atomics and the explicit wait.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    tm_wait_vm_lgkm0<0>();
    __syncthreads();
    if (tid == 0) {
      uint32_t *cnt = wd.cnt + blockIdx.y * kTmCntStride;
      const uint32_t ticket = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = ticket == gridDim.x - 1;
      if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u) return;  // uniform
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const int64_t r = tile0 + tid;
    if (tid < kWideQ && r < n) {
      const uint64_t key = __hip_atomic_load(keys + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      float a[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) a[p] = p < wd.parts ? wd.qn_part[(int64_t)p * n + r] : 0.f;
      const float qn = qn_sum(a[0], a[1], a[2], a[3], wd.parts);
      int64_t ix;
      const float d = tm_key_to_dist(key, qn, METRIC == TM_METRIC_L2, ix);
      wd.out_dist[r] = d;
      wd.out_idx[r] = ix;
      wd.out_qn[r] = qn;
    }
  }
}

// The wide kernel for a plan's range length: the HALF form for half-round
// ranges (d = 128 only: at d = 64 that form spills registers).
template <int DT, int DIM, int METRIC, bool DEC>
auto wide_kernel_for(int64_t chunk) {
  if constexpr (DIM == 128)
    if (chunk == wide_half_rows(DIM)) return search_top1_wide_kernel<DT, DIM, METRIC, DEC, true>;
  return search_top1_wide_kernel<DT, DIM, METRIC, DEC, false>;
}

// The K smallest of two ascending K-lists, ascending: min(a[i], b[K-1-i]) is
// bitonic and holds exactly the K smallest; a half-cleaner cascade sorts it.
template <int K>
__device__ __forceinline__ void merge_min(uint64_t (&a)[K], const uint64_t (&b)[K]) {
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

// Stream kernel (n <= 64): wave w of split s owns the 32-centroid block
// s * kStreamChunk + 32 w and every query (QS slabs of 32).  All operand loads
// are unconditional and issued together: query rows past n re-read row n - 1
// (their lists are never written), centroid rows past the table re-read its
// last row, and positions past the split's range carry an infinite penalty,
// which makes no candidate (key ~0).  The per-lane running lists take every
// candidate through a branch-free compare-swap chain; the two lanes of a
// query (l, l ^ 32) and then the four waves (through LDS, entry-major so the
// reads are conflict-free) are merged with the bitonic min-merge.
template <int DT, int DIM, int K, int QS, int METRIC>
__global__ __launch_bounds__(kThreads) void search_stream_kernel(
    const typename Elem<DT>::T *__restrict__ q, int64_t n, int64_t ld_q,
    const typename Elem<DT>::T *__restrict__ cents, int64_t n_cent, int64_t ld_c,
    const float *__restrict__ c_sqnorm, int64_t chunk, uint64_t *__restrict__ ws, uint64_t *__restrict__ keys,
    int key_rep) {
  constexpr int KS = DIM / 16;
  __shared__ uint64_t merge_buf[4][K][QS * 32];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t split = blockIdx.x;
  const int64_t c_begin = split * chunk;
  const int64_t c_end = (c_begin + chunk < n_cent) ? c_begin + chunk : n_cent;
  const int64_t c0 = c_begin + 32 * wave;

  uint4 qf[QS][KS];
#pragma unroll
  for (int sl = 0; sl < QS; ++sl) {
    const int64_t r = sl * 32 + (lane & 31);
    const int64_t rr = r < n ? r : n - 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[sl][ks] = *reinterpret_cast<const uint4 *>(q + rr * ld_q + ks * 16 + 8 * (lane >> 5));
  }
  uint4 af[KS];
  {
    const int64_t cr = c0 + (lane & 31);
    const int64_t crr = cr < n_cent ? cr : n_cent - 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      af[ks] = *reinterpret_cast<const uint4 *>(cents + crr * ld_c + ks * 16 + 8 * (lane >> 5));
  }
  float pen[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t cm = c0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    pen[i] = (METRIC == TM_METRIC_L2) ? c_sqnorm[cm < n_cent ? cm : n_cent - 1] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t cm = c0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    pen[i] = cm < c_end ? pen[i] : __builtin_huge_valf();
  }

  tm_f32x16 acc[QS];
#pragma unroll
  for (int sl = 0; sl < QS; ++sl) acc[sl] = tm_f32x16{};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int sl = 0; sl < QS; ++sl) acc[sl] = tm_mfma32x32x16<DT>(af[ks], qf[sl][ks], acc[sl]);

#pragma unroll
  for (int sl = 0; sl < QS; ++sl) {
    uint64_t l[K];
#pragma unroll
    for (int j = 0; j < K; ++j) l[j] = ~0ull;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = (int)c0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      const float dp = (METRIC == TM_METRIC_L2) ? fmaf(-2.f, acc[sl][i], pen[i]) : (pen[i] - acc[sl][i]);
      uint64_t x = dp == __builtin_huge_valf() ? ~0ull : make_key(dp, c);
#pragma unroll
      for (int j = 0; j < K; ++j) {  // compare-swap chain (no branch)
        const uint64_t lo = l[j] < x ? l[j] : x;
        x = l[j] < x ? x : l[j];
        l[j] = lo;
      }
    }
    uint64_t o[K];
#pragma unroll
    for (int j = 0; j < K; ++j) o[j] = __shfl_xor(l[j], 32, 64);
    merge_min<K>(l, o);
    if (lane < 32) {
#pragma unroll
      for (int j = 0; j < K; ++j) merge_buf[wave][j][sl * 32 + lane] = l[j];
    }
  }
  __syncthreads();
  // waves saw disjoint centroid blocks of the same queries: merge through LDS
  if (tid < QS * 32) {
    const int r = tid;
    uint64_t l[K];
#pragma unroll
    for (int j = 0; j < K; ++j) l[j] = merge_buf[0][j][r];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      uint64_t o[K];
#pragma unroll
      for (int j = 0; j < K; ++j) o[j] = merge_buf[w][j][r];
      merge_min<K>(l, o);
    }
    if (r < n) {
      uint64_t *dst = ws + (split * n + r) * K;
#pragma unroll
      for (int j = 0; j < K; ++j) dst[j] = l[j];
      // the query's best key over the splits of replica split % key_rep (reset to ~0 before the launch)
      if (keys != nullptr)
        atomicMin(reinterpret_cast<unsigned long long *>(keys + (split % key_rep) * tm_key_stride(n) + r),
                  (unsigned long long)l[0]);
    }
  }
}

// Output of one query: key ~0 (no candidate) -> index -1 and the worst distance.
template <int METRIC>
__device__ __forceinline__ void write_hit(uint64_t key, float qn, float *dist, int64_t *idx) {
  int64_t i;
  *dist = tm_key_to_dist(key, qn, METRIC == TM_METRIC_L2, i);
  *idx = i;
}

// 64-bit value of the lane `x` lanes away within a quad (x = 1 or 2), by DPP.
template <int X>
__device__ __forceinline__ uint64_t quad_xor(uint64_t v) {
  constexpr int ctrl = X == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, ctrl, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), ctrl, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}
template <int X>
__device__ __forceinline__ float quad_xor_f(float v) {
  constexpr int ctrl = X == 1 ? 0xB1 : 0x4E;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
}

// A merge launch may carry the router: workgroups from `first` on route
// kThreads / 8 tokens each (8 lanes per token).
struct MergeRoute {
  tm_route_args a;
  int64_t first;
};

template <int RVPL>
__device__ __forceinline__ bool merge_route_role(const MergeRoute &mr, int64_t n) {
  if constexpr (RVPL > 0) {
    if ((int64_t)blockIdx.x >= mr.first) {  // uniform
      const int64_t tok = ((int64_t)blockIdx.x - mr.first) * (kThreads / 8) + (threadIdx.x >> 3);
      tm_route_token<RVPL, 8>(mr.a.logits, n, mr.a.ld, mr.a.top_k, 0, mr.a.out_w, mr.a.out_ids, tok, threadIdx.x & 7);
      return true;
    }
  }
  return false;
}

// Top-1 merge: a quad of lanes per query; lane j takes splits j, j+4, ... (8
// loads in flight per lane), then two DPP steps give every lane of the quad
// the smallest key.  Every lane of a partial last quad reads a valid query.
template <int DT, int METRIC, int RVPL>
__global__ __launch_bounds__(kThreads) void merge_top1_kernel(
    const uint64_t *__restrict__ ws, int64_t n, int64_t nsplit, const typename Elem<DT>::T *__restrict__ q,
    int64_t ld_q, int dim, const float *__restrict__ q_sqnorm, float *__restrict__ out_dist,
    int64_t *__restrict__ out_idx, MergeRoute mr) {
  if (merge_route_role<RVPL>(mr, n)) return;
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t r = t >> 2;
  const int j = threadIdx.x & 3;
  const int64_t rr = r < n ? r : n - 1;
  float qn = 0.f;
  if (METRIC == TM_METRIC_L2 && q_sqnorm != nullptr) qn = q_sqnorm[rr];
  uint64_t best = ~0ull;
#pragma unroll 8
  for (int64_t s = j; s < nsplit; s += 4) {
    const uint64_t v = ws[s * n + rr];
    best = v < best ? v : best;
  }
  uint64_t o = quad_xor<1>(best);
  best = o < best ? o : best;
  o = quad_xor<2>(best);
  best = o < best ? o : best;
  if (METRIC == TM_METRIC_L2 && q_sqnorm == nullptr) {
    for (int i = j; i < dim; i += 4) {
      const float v = Elem<DT>::to_f(q[rr * ld_q + i]);
      qn = fmaf(v, v, qn);
    }
    qn += quad_xor_f<1>(qn);
    qn += quad_xor_f<2>(qn);
  }
  if (r < n && j == 0) write_hit<METRIC>(best, qn, out_dist + r, out_idx + r);
}

// Top-k merge (k = 4 or 8): one wave per query; lane l merges the sorted lists
// of splits l, l+64, ...; then six xor-shuffle steps merge the lanes' lists.
template <int DT, int K, int METRIC, int RVPL>
__global__ __launch_bounds__(kThreads) void merge_kernel(
    const uint64_t *__restrict__ ws, int64_t n, int64_t nsplit, const typename Elem<DT>::T *__restrict__ q,
    int64_t ld_q, int dim, const float *__restrict__ q_sqnorm, int top_k, float *__restrict__ out_dist,
    int64_t *__restrict__ out_idx, MergeRoute mr) {
  if (merge_route_role<RVPL>(mr, n)) return;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= n) return;  // whole wave exits together
  float qn = 0.f;
  if (METRIC == TM_METRIC_L2 && q_sqnorm != nullptr) qn = q_sqnorm[r];
  uint64_t lst[K];
#pragma unroll
  for (int j = 0; j < K; ++j) lst[j] = ~0ull;
  for (int64_t s = lane; s < nsplit; s += 64) {
    const uint64_t *src = ws + (s * n + r) * K;
    uint64_t b[K];
#pragma unroll
    for (int j = 0; j < K; ++j) b[j] = src[j];
    merge_min<K>(lst, b);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    if (o >= nsplit) continue;  // (uniform) lanes o.. hold no list
    uint64_t other[K];
#pragma unroll
    for (int j = 0; j < K; ++j) other[j] = __shfl_xor(lst[j], o, 64);
    merge_min<K>(lst, other);
  }
  if (METRIC == TM_METRIC_L2 && q_sqnorm == nullptr) {
    for (int j = lane; j < dim; j += 64) {
      const float v = Elem<DT>::to_f(q[r * ld_q + j]);
      qn = fmaf(v, v, qn);
    }
    qn = tm_wave_sum(qn);
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < K; ++j)
      if (j < top_k) write_hit<METRIC>(lst[j], qn, out_dist + r * top_k + j, out_idx + r * top_k + j);
  }
}

template <int DT>
__global__ void sqnorm_kernel(const typename Elem<DT>::T *c, int64_t n, int dim, int64_t ld, float *out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int j = 0; j < dim; ++j) {
    const float v = Elem<DT>::to_f(c[i * ld + j]);
    s = fmaf(v, v, s);
  }
  out[i] = s;
}

template <int DT, int K, int METRIC, int RVPL>
void launch_merge(const SplitPlan &p, int top_k, const typename Elem<DT>::T *Q, int64_t n, int64_t ld_q, int dim,
                  const float *q_sqnorm, float *out_dist, int64_t *out_idx, const uint64_t *ws,
                  const tm_route_args *ra, hipStream_t stream) {
  const int64_t mblocks = K == 1 ? tm_cdiv(n, kThreads / 4) : tm_cdiv(n, kThreads / 64);
  MergeRoute mr{};
  int64_t blocks = mblocks;
  if (RVPL > 0) {
    mr.a = *ra;
    mr.first = mblocks;
    blocks += tm_cdiv(n, kThreads / 8);
  }
  if constexpr (K == 1)
    hipLaunchKernelGGL((merge_top1_kernel<DT, METRIC, RVPL>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, ws,
                       n, p.nsplit, Q, ld_q, dim, q_sqnorm, out_dist, out_idx, mr);
  else
    hipLaunchKernelGGL((merge_kernel<DT, K, METRIC, RVPL>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, ws,
                       n, p.nsplit, Q, ld_q, dim, q_sqnorm, top_k, out_dist, out_idx, mr);
}

template <int DT, int DIM, int K, int METRIC>
int launch_search(int top_k, const void *q, int64_t n, int64_t ld_q, const float *q_sqnorm,
                  const void *cents, int64_t n_cent, int64_t ld_c, const float *c_sqnorm,
                  float *out_dist, int64_t *out_idx, uint64_t *ws, const tm_route_args *ra, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const SplitPlan p = plan_split(n, n_cent, DIM, top_k);
  const T *Q = static_cast<const T *>(q);
  const T *C = static_cast<const T *>(cents);
  dim3 block(kThreads);
  if (p.stream) {
    if (p.qs == 1)
      hipLaunchKernelGGL((search_stream_kernel<DT, DIM, K, 1, METRIC>), dim3((unsigned)p.nsplit), block, 0, stream,
                         Q, n, ld_q, C, n_cent, ld_c, c_sqnorm, p.chunk, ws, nullptr, 1);
    else
      hipLaunchKernelGGL((search_stream_kernel<DT, DIM, K, 2, METRIC>), dim3((unsigned)p.nsplit), block, 0, stream,
                         Q, n, ld_q, C, n_cent, ld_c, c_sqnorm, p.chunk, ws, nullptr, 1);
  } else if (K == 1 && p.wide && wide_strides_ok(ld_q, ld_c, DIM)) {
    hipLaunchKernelGGL((wide_kernel_for<DT, DIM < 256 ? DIM : 128, METRIC, false>(p.chunk)), dim3((unsigned)p.nsplit, (unsigned)p.row_blocks), dim3(kWideThreads), 0, stream, Q, n,
                       ld_q, C, n_cent, ld_c, c_sqnorm, p.chunk, ws, WideDecode{});
  } else if (K == 1 && DIM <= 128 && ld_c * dma_rows(DIM) * (int64_t)sizeof(T) < ((int64_t)1 << 31)) {
    // (d = 256 would not fit two waves per SIMD; the stage byte offsets must fit 31 bits)
    hipLaunchKernelGGL((search_top1_kernel<DT, DIM < 256 ? DIM : 128, METRIC>), dim3((unsigned)p.row_blocks, (unsigned)p.nsplit),
                       block, 0, stream, Q, n, ld_q, C, n_cent, ld_c, c_sqnorm, p.chunk, ws, nullptr);
  } else {
    hipLaunchKernelGGL((search_dma_kernel<DT, DIM, K, METRIC>), dim3((unsigned)p.row_blocks, (unsigned)p.nsplit),
                       block, 0, stream, Q, n, ld_q, C, n_cent, ld_c, c_sqnorm, p.chunk, ws);
  }
  TM_LAUNCH_CHECK("tm_search_global");
  if (ra == nullptr)
    launch_merge<DT, K, METRIC, 0>(p, top_k, Q, n, ld_q, DIM, q_sqnorm, out_dist, out_idx, ws, ra, stream);
  else if (ra->n_experts == 64)
    launch_merge<DT, K, METRIC, 8>(p, top_k, Q, n, ld_q, DIM, q_sqnorm, out_dist, out_idx, ws, ra, stream);
  else
    launch_merge<DT, K, METRIC, 16>(p, top_k, Q, n, ld_q, DIM, q_sqnorm, out_dist, out_idx, ws, ra, stream);
  TM_LAUNCH_CHECK("tm_search_global(merge)");
  return TM_OK;
}

template <int DT, int DIM, int METRIC>
int dispatch_k(int top_k, const void *q, int64_t n, int64_t ld_q, const float *q_sqnorm,
               const void *cents, int64_t n_cent, int64_t ld_c, const float *c_sqnorm,
               float *out_dist, int64_t *out_idx, uint64_t *ws, const tm_route_args *ra, hipStream_t stream) {
  switch (list_len(top_k)) {
    case 1: return launch_search<DT, DIM, 1, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, stream);
    case 4: return launch_search<DT, DIM, 4, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, stream);
    default: return launch_search<DT, DIM, 8, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, stream);
  }
}

template <int DT, int METRIC>
int dispatch_dim(int dim, int top_k, const void *q, int64_t n, int64_t ld_q, const float *q_sqnorm,
                 const void *cents, int64_t n_cent, int64_t ld_c, const float *c_sqnorm,
                 float *out_dist, int64_t *out_idx, uint64_t *ws, const tm_route_args *ra, hipStream_t stream) {
  switch (dim) {
    case 64: return dispatch_k<DT, 64, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, stream);
    case 128: return dispatch_k<DT, 128, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, stream);
    case 256: return dispatch_k<DT, 256, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, stream);
    default: return tm_fail(TM_EINVAL_SHAPE, "tm_search_global: dim %d not in {64, 128, 256}", dim);
  }
}

// ---------------------------------------------------------------------------
// fp32 tables (the CPU-reference configuration): a workgroup owns 64
// queries (lane = query, the query held in registers) and one centroid
// range; the range is staged through LDS kF32Block rows at a time and the
// four waves take every fourth row of it (rows are read as broadcasts: every
// lane of a wave reads the same address).  Each row's dot product is fp32
// FMAs in dimension order; each lane keeps a packed-key list (the 16-bit
// forms' keys and order) and the four waves' lists are merged through LDS.
// Per-split lists are merged by the same merge kernels as the 16-bit forms;
// tm_search_global_workspace_size covers the larger of the two plans.
// ---------------------------------------------------------------------------
constexpr int kF32Block = 32;  // centroid rows per LDS stage
constexpr int kF32Rows = 64;   // queries per workgroup

// About 1024 workgroups (one per 32-row stage at small n), so a small
// batch still spreads over the chip.
SplitPlan plan_f32(int64_t n, int64_t c) {
  SplitPlan p{};
  p.row_blocks = tm_cdiv(n, kF32Rows);
  int64_t want = tm_cdiv(1024, p.row_blocks);
  if (want > tm_cdiv(c, kF32Block)) want = tm_cdiv(c, kF32Block);
  if (want < 1) want = 1;
  p.chunk = tm_cdiv(tm_cdiv(c, want), kF32Block) * kF32Block;
  p.nsplit = tm_cdiv(c, p.chunk);
  return p;
}

// RVPL > 0: rows y >= mr.first of the grid are router workgroups (32 tokens
// each, numbered along x): the router's DPP chain runs beside the search
// instead of in the short merge launch after it.
template <int DIM, int K, int METRIC, int RVPL>
__global__ __launch_bounds__(kThreads) void search_f32_kernel(const float *__restrict__ q, int64_t n, int64_t ld_q,
                                                              const float *__restrict__ cents, int64_t n_cent,
                                                              int64_t ld_c, const float *__restrict__ c_sqnorm,
                                                              int64_t chunk, uint64_t *__restrict__ ws,
                                                              MergeRoute mr) {
  constexpr int V4 = DIM / 4;  // float4 per centroid row
  __shared__ float4 cs[kF32Block * V4];
  __shared__ float pen_s[kF32Block];
  __shared__ uint64_t lists[3][K][kF32Rows];  // waves 1..3 hand their lists to wave 0
  if constexpr (RVPL > 0) {
    if ((int64_t)blockIdx.y >= mr.first) {  // uniform: router workgroup
      const int64_t w = ((int64_t)blockIdx.y - mr.first) * gridDim.x + blockIdx.x;
      const int64_t tok = w * (kThreads / 8) + (threadIdx.x >> 3);
      tm_route_token<RVPL, 8>(mr.a.logits, n, mr.a.ld, mr.a.top_k, 0, mr.a.out_w, mr.a.out_ids, tok, threadIdx.x & 7);
      return;
    }
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t r = (int64_t)blockIdx.x * kF32Rows + lane;
  const float4 *qrow = reinterpret_cast<const float4 *>(q + (r < n ? r : n - 1) * ld_q);
  const int64_t c0 = (int64_t)blockIdx.y * chunk;
  const int64_t c1 = c0 + chunk < n_cent ? c0 + chunk : n_cent;
  float4 qv[V4];
#pragma unroll
  for (int k = 0; k < V4; ++k) qv[k] = qrow[k];
  Best<K> best;
  best.init();
  for (int64_t cb = c0; cb < c1; cb += kF32Block) {
    __syncthreads();  // the previous stage's reads are done
    for (int e = tid; e < kF32Block * V4; e += kThreads) {
      const int64_t c = cb + e / V4;
      cs[e] = c < c1 ? *reinterpret_cast<const float4 *>(cents + c * ld_c + 4 * (e % V4)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (tid < kF32Block) pen_s[tid] = (METRIC == TM_METRIC_L2 && cb + tid < c1) ? c_sqnorm[cb + tid] : 0.f;
    __syncthreads();
    const int valid = (int)(c1 - cb < kF32Block ? c1 - cb : kF32Block);  // uniform
    for (int j = wave; j < valid; j += 4) {  // this wave's rows, ascending
      const float4 *row = cs + j * V4;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < V4; ++k) {
        const float4 cv = row[k];
        acc = fmaf(qv[k].x, cv.x, acc);
        acc = fmaf(qv[k].y, cv.y, acc);
        acc = fmaf(qv[k].z, cv.z, acc);
        acc = fmaf(qv[k].w, cv.w, acc);
      }
      const float dp = (METRIC == TM_METRIC_L2) ? fmaf(-2.f, acc, pen_s[j]) : -acc;
      best.push(dp, (int)(cb + j));
    }
  }
  best.finalize();
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < K; ++i) lists[wave - 1][i][lane] = best.l[i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const uint64_t key = lists[w][i][lane];
        if (key < best.l[K - 1]) list_insert<K>(best.l, key);
      }
    if (r < n) {
#pragma unroll
      for (int i = 0; i < K; ++i) ws[((int64_t)blockIdx.y * n + r) * K + i] = best.l[i];
    }
  }
}

template <int DIM, int K, int METRIC>
int launch_search_f32(int top_k, const void *q, int64_t n, int64_t ld_q, const float *q_sqnorm, const void *cents,
                      int64_t n_cent, int64_t ld_c, const float *c_sqnorm, float *out_dist, int64_t *out_idx,
                      uint64_t *ws, const tm_route_args *ra, hipStream_t stream) {
  const SplitPlan p = plan_f32(n, n_cent);
  const float *Q = static_cast<const float *>(q);
  // the router (when fused) in extra grid rows of the search launch
  MergeRoute mr{};
  int64_t rows = p.nsplit;
  if (ra != nullptr) {
    mr.a = *ra;
    mr.first = p.nsplit;
    rows += tm_cdiv(tm_cdiv(n, kThreads / 8), p.row_blocks);
  }
  auto go = [&](auto rvpl_tag) {
    constexpr int RVPL = decltype(rvpl_tag)::value;
    hipLaunchKernelGGL((search_f32_kernel<DIM, K, METRIC, RVPL>), dim3((unsigned)p.row_blocks, (unsigned)rows),
                       dim3(kThreads), 0, stream, Q, n, ld_q, static_cast<const float *>(cents), n_cent, ld_c,
                       c_sqnorm, p.chunk, ws, mr);
  };
  if (ra == nullptr)
    go(std::integral_constant<int, 0>{});
  else if (ra->n_experts == 64)
    go(std::integral_constant<int, 8>{});
  else
    go(std::integral_constant<int, 16>{});
  TM_LAUNCH_CHECK("tm_search_global(f32)");
  launch_merge<TM_DT_F32, K, METRIC, 0>(p, top_k, Q, n, ld_q, DIM, q_sqnorm, out_dist, out_idx, ws, nullptr, stream);
  TM_LAUNCH_CHECK("tm_search_global(merge)");
  return TM_OK;
}

template <int METRIC>
int dispatch_f32(int dim, int top_k, const void *q, int64_t n, int64_t ld_q, const float *q_sqnorm,
                 const void *cents, int64_t n_cent, int64_t ld_c, const float *c_sqnorm, float *out_dist,
                 int64_t *out_idx, uint64_t *ws, const tm_route_args *ra, hipStream_t s) {
#define TM_F32_K(D)                                                                                                 \
  switch (list_len(top_k)) {                                                                                        \
    case 1: return launch_search_f32<D, 1, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm,      \
                                                   out_dist, out_idx, ws, ra, s);                                   \
    case 4: return launch_search_f32<D, 4, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm,      \
                                                   out_dist, out_idx, ws, ra, s);                                   \
    default: return launch_search_f32<D, 8, METRIC>(top_k, q, n, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm,     \
                                                    out_dist, out_idx, ws, ra, s);                                  \
  }
  switch (dim) {
    case 64: TM_F32_K(64)
    case 128: TM_F32_K(128)
    case 256: TM_F32_K(256)
    default: return tm_fail(TM_EINVAL_SHAPE, "tm_search_global: dim %d not in {64, 128, 256}", dim);
  }
#undef TM_F32_K
}

}  // namespace

extern "C" int tm_centroid_sqnorms(int32_t dtype, const void *cents, int64_t n_cent, int32_t dim,
                                   int64_t ld_c, float *out, tm_stream_t stream) {
  TM_REQUIRE(n_cent >= 0 && dim > 0 && ld_c >= dim, TM_EINVAL_SHAPE, "tm_centroid_sqnorms: bad sizes");
  TM_REQUIRE(n_cent == 0 || (cents && out), TM_EINVAL_ARG, "tm_centroid_sqnorms: null pointer");
  if (n_cent == 0) return TM_OK;
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    hipLaunchKernelGGL((sqnorm_kernel<DT>), dim3((unsigned)tm_cdiv(n_cent, 256)), dim3(256), 0,
                       tm_hip_stream(stream), static_cast<const typename Elem<DT>::T *>(cents),
                       n_cent, dim, ld_c, out);
    TM_LAUNCH_CHECK("tm_centroid_sqnorms");
    return TM_OK;
  });
}

extern "C" size_t tm_search_global_workspace_size(int64_t n_tokens, int64_t n_cent, int32_t dim,
                                                  int32_t top_k) {
  if (n_tokens <= 0 || n_cent <= 0 || top_k <= 0 || (dim != 64 && dim != 128 && dim != 256)) return 0;
  const int64_t s16 = plan_split(n_tokens, n_cent, dim, top_k).nsplit;  // 16-bit tables
  const int64_t s32 = plan_f32(n_tokens, n_cent).nsplit;                // fp32 tables
  return (size_t)(s16 > s32 ? s16 : s32) * (size_t)n_tokens * (size_t)list_len(top_k) * sizeof(uint64_t);
}

static int search_impl(int32_t dtype, const void *q, int64_t n_tokens, int64_t ld_q, const float *q_sqnorm,
                       const void *cents, int64_t n_cent, int64_t ld_c, const float *c_sqnorm, int32_t dim,
                       int32_t top_k, int32_t metric, float *out_dist, int64_t *out_idx, void *workspace,
                       size_t workspace_bytes, const tm_route_args *ra, hipStream_t s) {
  TM_REQUIRE(n_tokens >= 0 && n_tokens < ((int64_t)1 << 31) && n_cent > 0 && n_cent < (int64_t)0x7fffffff, TM_EINVAL_SHAPE,
             "tm_search_global: bad sizes n=%lld C=%lld", (long long)n_tokens, (long long)n_cent);
  TM_REQUIRE(ld_q >= dim && ld_c >= dim, TM_EINVAL_SHAPE, "tm_search_global: bad row strides");
  TM_REQUIRE(top_k >= 1 && top_k <= 8, TM_EINVAL_SHAPE, "tm_search_global: top_k %d not in [1, 8]", top_k);
  TM_REQUIRE(metric == TM_METRIC_L2 || metric == TM_METRIC_DOT, TM_EINVAL_ARG, "tm_search_global: bad metric");
  TM_REQUIRE(dtype == TM_DT_BF16 || dtype == TM_DT_F16 || dtype == TM_DT_F32, TM_EINVAL_DTYPE,
             "tm_search_global: dtype must be F32, F16 or BF16");
  if (n_tokens == 0) return TM_OK;
  TM_REQUIRE(q && cents && out_dist && out_idx, TM_EINVAL_ARG, "tm_search_global: null pointer");
  TM_REQUIRE(metric != TM_METRIC_L2 || c_sqnorm, TM_EINVAL_ARG, "tm_search_global: L2 needs c_sqnorm");
  const int64_t esz = dtype == TM_DT_F32 ? 4 : 2;
  TM_REQUIRE(tm_aligned16(q) && tm_aligned16(cents) && (ld_q * esz) % 16 == 0 && (ld_c * esz) % 16 == 0,
             TM_EINVAL_SHAPE, "tm_search_global: q and centroid rows must be 16-byte aligned");
  const size_t need = tm_search_global_workspace_size(n_tokens, n_cent, dim, top_k);
  TM_REQUIRE(workspace != nullptr && workspace_bytes >= need, TM_EWORKSPACE,
             "tm_search_global: workspace %zu bytes < %zu", workspace_bytes, need);
  uint64_t *ws = static_cast<uint64_t *>(workspace);
  if (dtype == TM_DT_F32) {
    if (metric == TM_METRIC_L2)
      return dispatch_f32<TM_METRIC_L2>(dim, top_k, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, s);
    return dispatch_f32<TM_METRIC_DOT>(dim, top_k, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, s);
  }
  if (dtype == TM_DT_BF16) {
    if (metric == TM_METRIC_L2)
      return dispatch_dim<TM_DT_BF16, TM_METRIC_L2>(dim, top_k, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, s);
    return dispatch_dim<TM_DT_BF16, TM_METRIC_DOT>(dim, top_k, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, s);
  }
  if (metric == TM_METRIC_L2)
    return dispatch_dim<TM_DT_F16, TM_METRIC_L2>(dim, top_k, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, s);
  return dispatch_dim<TM_DT_F16, TM_METRIC_DOT>(dim, top_k, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, out_dist, out_idx, ws, ra, s);
}

bool tm_internal_route_fusable(const tm_route_args *ra) {
  return ra != nullptr && ra->logits != nullptr && ra->out_w != nullptr && ra->out_ids != nullptr &&
         ra->top_k >= 1 && ra->top_k <= 8 && (ra->n_experts == 64 || ra->n_experts == 128) &&
         ra->ld >= ra->n_experts && ra->ld % 4 == 0 && tm_aligned16(ra->logits);
}

int tm_internal_search_route(int32_t dtype, const void *q, int64_t n_tokens, int64_t ld_q, const float *q_sqnorm,
                             const void *cents, int64_t n_cent, int64_t ld_c, const float *c_sqnorm, int32_t dim,
                             int32_t top_k, int32_t metric, float *out_dist, int64_t *out_idx, void *workspace,
                             size_t workspace_bytes, const tm_route_args *ra, hipStream_t stream) {
  TM_REQUIRE(tm_internal_route_fusable(ra), TM_EINVAL_ARG, "tm_table_forward: router shape cannot be fused");
  return search_impl(dtype, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, dim, top_k, metric,
                     out_dist, out_idx, workspace, workspace_bytes, ra, stream);
}

extern "C" int tm_search_global(int32_t dtype, const void *q, int64_t n_tokens, int64_t ld_q,
                                const float *q_sqnorm, const void *cents, int64_t n_cent,
                                int64_t ld_c, const float *c_sqnorm, int32_t dim, int32_t top_k,
                                int32_t metric, float *out_dist, int64_t *out_idx, void *workspace,
                                size_t workspace_bytes, tm_stream_t stream) {
  return search_impl(dtype, q, n_tokens, ld_q, q_sqnorm, cents, n_cent, ld_c, c_sqnorm, dim, top_k, metric,
                     out_dist, out_idx, workspace, workspace_bytes, nullptr, tm_hip_stream(stream));
}

namespace {

template <int DT, int DIM, int METRIC>
void launch_search_keys(const void *q, int64_t n, int64_t ld_q, const void *cents, int64_t n_cent, int64_t ld_c,
                        const float *c_sqnorm, uint64_t *keys, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const SplitPlan p = plan_split(n, n_cent, DIM, 1);
  hipLaunchKernelGGL((search_top1_kernel<DT, DIM, METRIC>), dim3((unsigned)p.row_blocks, (unsigned)p.nsplit),
                     dim3(kThreads), 0, stream, static_cast<const T *>(q), n, ld_q, static_cast<const T *>(cents),
                     n_cent, ld_c, c_sqnorm, p.chunk, nullptr, keys);
}

template <int DT, int METRIC>
void search_keys_dim(int dim, const void *q, int64_t n, int64_t ld_q, const void *cents, int64_t n_cent,
                     int64_t ld_c, const float *c_sqnorm, uint64_t *keys, hipStream_t stream) {
  if (dim == 64)
    launch_search_keys<DT, 64, METRIC>(q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, stream);
  else
    launch_search_keys<DT, 128, METRIC>(q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, stream);
}

}  // namespace

bool tm_internal_search_keys_ok(int32_t dtype, int64_t n, int64_t n_cent, int64_t ld_c, int32_t dim,
                                int32_t top_k) {
  if (!(dtype == TM_DT_BF16 || dtype == TM_DT_F16) || top_k != 1 || !(dim == 64 || dim == 128)) return false;
  if (n <= 0 || n >= ((int64_t)1 << 31) || n_cent <= 0 || n_cent >= (int64_t)0x7fffffff || ld_c < dim) return false;
  if (plan_split(n, n_cent, dim, 1).stream) return false;
  return ld_c * dma_rows(dim) * 2 < ((int64_t)1 << 31);
}

int tm_internal_search_keys(int32_t dtype, const void *q, int64_t n, int64_t ld_q, const void *cents,
                            int64_t n_cent, int64_t ld_c, const float *c_sqnorm, int32_t dim, int32_t metric,
                            uint64_t *keys, hipStream_t stream) {
  TM_REQUIRE(tm_internal_search_keys_ok(dtype, n, n_cent, ld_c, dim, 1), TM_EINVAL_SHAPE,
             "tm_table_forward: search shape not supported by the atomic top-1 path");
  TM_REQUIRE(metric == TM_METRIC_L2 || metric == TM_METRIC_DOT, TM_EINVAL_ARG, "tm_table_forward: bad metric");
  TM_REQUIRE(q && cents && keys && (metric != TM_METRIC_L2 || c_sqnorm), TM_EINVAL_ARG,
             "tm_table_forward: null pointer");
  TM_REQUIRE(ld_q >= dim && tm_aligned16(q) && tm_aligned16(cents) && (ld_q * 2) % 16 == 0 && (ld_c * 2) % 16 == 0,
             TM_EINVAL_SHAPE, "tm_table_forward: q and centroid rows must be 16-byte aligned");
  if (dtype == TM_DT_BF16) {
    if (metric == TM_METRIC_L2)
      search_keys_dim<TM_DT_BF16, TM_METRIC_L2>(dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, stream);
    else
      search_keys_dim<TM_DT_BF16, TM_METRIC_DOT>(dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, stream);
  } else {
    if (metric == TM_METRIC_L2)
      search_keys_dim<TM_DT_F16, TM_METRIC_L2>(dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, stream);
    else
      search_keys_dim<TM_DT_F16, TM_METRIC_DOT>(dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, stream);
  }
  TM_LAUNCH_CHECK("tm_table_forward(search)");
  return TM_OK;
}

// ---------------------------------------------------------------------------
// Fused top-1 plan, large n (internal): the wide search kernel with the keep
// selection in its last workgroup.
// ---------------------------------------------------------------------------
namespace {

template <int DT, int DIM, int METRIC>
void launch_search_decode(const WidePlan &p, const void *q, int64_t n, int64_t ld_q, const void *cents,
                          int64_t n_cent, int64_t ld_c, const float *c_sqnorm, uint64_t *keys, const WideDecode &wd,
                          hipStream_t stream) {
  using T = typename Elem<DT>::T;
  hipLaunchKernelGGL((wide_kernel_for<DT, DIM, METRIC, true>(p.chunk)), dim3((unsigned)p.nsplit, (unsigned)p.tiles),
                     dim3(kWideThreads), 0, stream, static_cast<const T *>(q), n, ld_q, static_cast<const T *>(cents),
                     n_cent, ld_c, c_sqnorm, p.chunk, keys, wd);
}

template <int DT, int METRIC>
void search_decode_dim(const WidePlan &p, int dim, const void *q, int64_t n, int64_t ld_q, const void *cents,
                       int64_t n_cent, int64_t ld_c, const float *c_sqnorm, uint64_t *keys, const WideDecode &wd,
                       hipStream_t stream) {
  if (dim == 64)
    launch_search_decode<DT, 64, METRIC>(p, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, wd, stream);
  else
    launch_search_decode<DT, 128, METRIC>(p, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, wd, stream);
}

}  // namespace

int64_t tm_internal_search_decode_tiles(int32_t dtype, int64_t n, int64_t n_cent, int64_t ld_q, int64_t ld_c,
                                        int32_t dim) {
  if (!tm_internal_search_keys_ok(dtype, n, n_cent, ld_c, dim, 1) || ld_q < dim) return 0;
  const WidePlan p = plan_wide(n, n_cent, dim);
  if (p.tiles * p.nsplit < kWideDecMinGroups || !wide_strides_ok(ld_q, ld_c, dim)) return 0;
  return p.tiles;
}

int tm_internal_search_decode(int32_t dtype, const void *q, int64_t n, int64_t ld_q, const void *cents,
                              int64_t n_cent, int64_t ld_c, const float *c_sqnorm, int32_t dim, int32_t metric,
                              uint64_t *keys, const float *qn_part, int32_t parts, float *out_dist, int64_t *out_idx,
                              float *out_qn, uint32_t *cnt, hipStream_t stream) {
  TM_REQUIRE(tm_internal_search_decode_tiles(dtype, n, n_cent, ld_q, ld_c, dim) > 0, TM_EINVAL_SHAPE,
             "tm_table_forward: search shape not supported by the wide top-1 path");
  TM_REQUIRE(metric == TM_METRIC_L2 || metric == TM_METRIC_DOT, TM_EINVAL_ARG, "tm_table_forward: bad metric");
  TM_REQUIRE(q && cents && keys && (metric != TM_METRIC_L2 || c_sqnorm) && qn_part && out_dist && out_idx &&
                 out_qn && cnt && parts >= 1 && parts <= 4,
             TM_EINVAL_ARG, "tm_table_forward: null pointer");
  TM_REQUIRE(tm_aligned16(q) && tm_aligned16(cents) && (ld_q * 2) % 16 == 0 && (ld_c * 2) % 16 == 0,
             TM_EINVAL_SHAPE, "tm_table_forward: q and centroid rows must be 16-byte aligned");
  const WidePlan p = plan_wide(n, n_cent, dim);
  const WideDecode wd{qn_part, parts, out_dist, out_idx, out_qn, cnt};
  if (dtype == TM_DT_BF16) {
    if (metric == TM_METRIC_L2)
      search_decode_dim<TM_DT_BF16, TM_METRIC_L2>(p, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, wd, stream);
    else
      search_decode_dim<TM_DT_BF16, TM_METRIC_DOT>(p, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, wd, stream);
  } else {
    if (metric == TM_METRIC_L2)
      search_decode_dim<TM_DT_F16, TM_METRIC_L2>(p, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, wd, stream);
    else
      search_decode_dim<TM_DT_F16, TM_METRIC_DOT>(p, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, keys, wd, stream);
  }
  TM_LAUNCH_CHECK("tm_table_forward(search)");
  return TM_OK;
}

// ---------------------------------------------------------------------------
// Decode plan (internal): the stream kernel alone, writing its per-split
// sorted lists into `lists` and each query's best key into keys[n] (reset to
// ~0 beforehand); the consumer merges the lists itself.
// ---------------------------------------------------------------------------
namespace {

template <int DT, int DIM, int K, int METRIC>
void launch_stream_keys(const SplitPlan &p, const void *q, int64_t n, int64_t ld_q, const void *cents,
                        int64_t n_cent, int64_t ld_c, const float *c_sqnorm, uint64_t *lists, uint64_t *keys,
                        int key_rep, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const T *Q = static_cast<const T *>(q);
  const T *C = static_cast<const T *>(cents);
  if (p.qs == 1)
    hipLaunchKernelGGL((search_stream_kernel<DT, DIM, K, 1, METRIC>), dim3((unsigned)p.nsplit), dim3(kThreads), 0,
                       stream, Q, n, ld_q, C, n_cent, ld_c, c_sqnorm, p.chunk, lists, keys, key_rep);
  else
    hipLaunchKernelGGL((search_stream_kernel<DT, DIM, K, 2, METRIC>), dim3((unsigned)p.nsplit), dim3(kThreads), 0,
                       stream, Q, n, ld_q, C, n_cent, ld_c, c_sqnorm, p.chunk, lists, keys, key_rep);
}

template <int DT, int METRIC, int K>
void stream_keys_dim(const SplitPlan &p, int dim, const void *q, int64_t n, int64_t ld_q, const void *cents,
                     int64_t n_cent, int64_t ld_c, const float *c_sqnorm, uint64_t *lists, uint64_t *keys,
                     int key_rep, hipStream_t stream) {
  switch (dim) {
    case 64: launch_stream_keys<DT, 64, K, METRIC>(p, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream); break;
    case 128: launch_stream_keys<DT, 128, K, METRIC>(p, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream); break;
    default: launch_stream_keys<DT, 256, K, METRIC>(p, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream); break;
  }
}

template <int DT, int METRIC>
void stream_keys_k(const SplitPlan &p, int top_k, int dim, const void *q, int64_t n, int64_t ld_q,
                   const void *cents, int64_t n_cent, int64_t ld_c, const float *c_sqnorm, uint64_t *lists,
                   uint64_t *keys, int key_rep, hipStream_t stream) {
  switch (list_len(top_k)) {
    case 1: stream_keys_dim<DT, METRIC, 1>(p, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream); break;
    case 4: stream_keys_dim<DT, METRIC, 4>(p, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream); break;
    default: stream_keys_dim<DT, METRIC, 8>(p, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream); break;
  }
}

}  // namespace

int64_t tm_internal_stream_nsplit(int64_t n, int64_t n_cent, int32_t dim, int32_t top_k) {
  if (n <= 0 || n > 64 || n_cent <= 0 || !(dim == 64 || dim == 128 || dim == 256)) return 0;
  return plan_split(n, n_cent, dim, top_k).nsplit;
}

int tm_internal_search_stream(int32_t dtype, const void *q, int64_t n, int64_t ld_q, const void *cents,
                              int64_t n_cent, int64_t ld_c, const float *c_sqnorm, int32_t dim, int32_t top_k,
                              int32_t metric, uint64_t *lists, uint64_t *keys, int32_t key_rep,
                              hipStream_t stream) {
  TM_REQUIRE(key_rep >= 1, TM_EINVAL_ARG, "tm_table_forward: key_rep < 1");
  TM_REQUIRE(tm_internal_stream_nsplit(n, n_cent, dim, top_k) > 0 && top_k >= 1 && top_k <= 8 &&
                 n_cent < (int64_t)0x7fffffff && ld_c >= dim && ld_q >= dim,
             TM_EINVAL_SHAPE, "tm_table_forward: search shape not supported by the decode plan");
  TM_REQUIRE(metric == TM_METRIC_L2 || metric == TM_METRIC_DOT, TM_EINVAL_ARG, "tm_table_forward: bad metric");
  TM_REQUIRE(dtype == TM_DT_BF16 || dtype == TM_DT_F16, TM_EINVAL_DTYPE, "tm_table_forward: dtype must be F16 or BF16");
  TM_REQUIRE(q && cents && lists && keys && (metric != TM_METRIC_L2 || c_sqnorm), TM_EINVAL_ARG,
             "tm_table_forward: null pointer");
  TM_REQUIRE(tm_aligned16(q) && tm_aligned16(cents) && (ld_q * 2) % 16 == 0 && (ld_c * 2) % 16 == 0,
             TM_EINVAL_SHAPE, "tm_table_forward: q and centroid rows must be 16-byte aligned");
  const SplitPlan p = plan_split(n, n_cent, dim, top_k);
  if (dtype == TM_DT_BF16) {
    if (metric == TM_METRIC_L2)
      stream_keys_k<TM_DT_BF16, TM_METRIC_L2>(p, top_k, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream);
    else
      stream_keys_k<TM_DT_BF16, TM_METRIC_DOT>(p, top_k, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream);
  } else {
    if (metric == TM_METRIC_L2)
      stream_keys_k<TM_DT_F16, TM_METRIC_L2>(p, top_k, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream);
    else
      stream_keys_k<TM_DT_F16, TM_METRIC_DOT>(p, top_k, dim, q, n, ld_q, cents, n_cent, ld_c, c_sqnorm, lists, keys, key_rep, stream);
  }
  TM_LAUNCH_CHECK("tm_table_forward(search)");
  return TM_OK;
}
