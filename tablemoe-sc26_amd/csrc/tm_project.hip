// a4: projection of hidden states into the PCA space (+ optional L2 normalise).
//
// q[b] = dtype(x[b] @ P_m + bias_m), one rounding after fp32 accumulation,
// as torch.addmm in the model dtype (table_moe/cache_engine/search.py:484,492).
// Normalisation follows _normalize_last_dim (search.py:12-21): the norm is
// rounded to dtype, the quotient is an fp32 division rounded to dtype, and
// rows with norm <= eps become zero.
//
// F16/BF16 with P stored k-contiguous (ps_h == 1, the layout the table path
// keeps): project_direct_kernel below, MFMA operands loaded straight from
// global memory, no workspace.
//
// Other P layouts (LDS-staged MFMA path): a workgroup owns 32 token rows, all
// `DIM` output columns and one slice of `hidden` (the k split).  The slice is walked in
// 64-wide stages through double-buffered LDS: the next stage's x and P tiles
// are fetched into registers while the current stage's MFMAs run, so global
// latency overlaps compute and each stage needs one barrier.  The x tile is
// stored row-major, the P tile k-contiguous per output column, so both MFMA
// operands are 16-byte LDS reads.  Tiles that mix modalities run one pass per
// modality and keep each row's own result.
//
// With a k split, workgroups write fp32 partial sums [split][n][DIM] and
// project_epilogue_kernel adds them in split order (deterministic), adds the
// bias, rounds, normalises and stores q.  Without one, the same epilogue runs
// inside the workgroup.
#include "tm_dma.h"
#include "tm_internal.h"
#include "tm_mfma.h"
#include "tm_route_dev.h"

namespace {

constexpr int kBM = 32;
constexpr int kBK = 64;
constexpr int kPad = 8;
constexpr int kThreads = 256;

struct ProjPlan {
  int64_t row_blocks;
  int nsplit;
  int k_chunk;  // multiple of kBK
};

ProjPlan plan_project(int64_t n, int hidden) {
  ProjPlan p;
  p.row_blocks = tm_cdiv(n, kBM);
  const int ksteps = (int)tm_cdiv(hidden, kBK);
  int64_t want = tm_cdiv(512, p.row_blocks);  // fill the chip: ~2 workgroups per CU
  if (want > 8) want = 8;                      // bounds the partial traffic of small batches
  if (want > ksteps) want = ksteps;
  if (want < 1) want = 1;
  p.k_chunk = (int)tm_cdiv(ksteps, want) * kBK;
  p.nsplit = (int)tm_cdiv(hidden, p.k_chunk);
  return p;
}

// Split plan of the fp32 kernel (its vector-unit k loop is slower per
// element than the matrix cores, so small batches split hidden further):
// up to 32 chunks of at least 64, with partials of at most 4 MiB unless the
// 16-bit plan's are larger.
ProjPlan plan_project_f32(int64_t n, int hidden, int dim) {
  ProjPlan p;
  p.row_blocks = tm_cdiv(n, kBM);
  const int ksteps = (int)tm_cdiv(hidden, kBK);
  int64_t want = tm_cdiv(1024, p.row_blocks);
  if (want > 32) want = 32;
  int64_t cap = (int64_t)(4u << 20) / (n * (int64_t)dim * 4);
  const int64_t s16 = plan_project(n, hidden).nsplit;
  if (cap < s16) cap = s16;
  if (want > cap) want = cap;
  if (want > ksteps) want = ksteps;
  if (want < 1) want = 1;
  p.k_chunk = (int)tm_cdiv(ksteps, want) * kBK;
  p.nsplit = (int)tm_cdiv(hidden, p.k_chunk);
  return p;
}

// Row epilogue shared by the fused kernel and the split epilogue: one row is
// handled by TPR consecutive lanes, 8 columns each.  v[] holds the rounded
// pre-normalisation values.
template <int DT, int TPR>
__device__ __forceinline__ void finish_row(float (&v)[8], int normalize, float eps,
                                           typename Elem<DT>::T *dst, float *sq_dst) {
  if (normalize) {  // uniform
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1) ss += __shfl_xor(ss, o, 64);
    const float norm = tm_round<DT>(sqrtf(ss));
    const float eps_dt = tm_round<DT>(eps);
    const bool zero_row = !(norm > eps_dt);
    const float den = fmaxf(norm, eps_dt);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = zero_row ? 0.f : tm_round<DT>(v[i] / den);
  }
  float so = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) so = fmaf(v[i], v[i], so);
#pragma unroll
  for (int o = 1; o < TPR; o <<= 1) so += __shfl_xor(so, o, 64);
  if (dst) tm_store8<DT>(dst, v);
  if (sq_dst) *sq_dst = so;
}

// Packed path (P in the layout of tm_project_pack).
//
// A workgroup owns 16 token rows and all DIM output columns; its KW waves
// split `hidden` into KW contiguous slices.  Every MFMA operand is one 16-byte
// load straight from global memory: A = x[row][k..k+7] and B = one lane's
// chunk of a packed 1 KiB fragment, so each B load of a wave is a contiguous
// 1 KiB and the k loop has no LDS staging and no barrier.  Each wave keeps
// kDepth k-steps of loads in flight in a register ring and issues the MFMAs
// of the oldest.  The KW partial tiles are then added in wave order through
// LDS (deterministic), the bias is added and the row epilogue runs in the
// same workgroup.  A tile whose rows mix modalities runs the k loop once per
// modality present and keeps each row's own result.
template <int DIM>
struct DirectCfg {
  static constexpr int NCB = DIM / 16;             // 16-column MFMA blocks
  static constexpr int kDepthX = 8;                // k-steps of x (HBM) loads in flight per wave
  static constexpr int kDepthP = DIM <= 128 ? 4 : 2;  // k-steps of P (L2-resident) loads in flight
};

template <int DT, int DIM, int KW>
__global__ __launch_bounds__(64 * KW) void project_direct_kernel(
    const typename Elem<DT>::T *__restrict__ x, int64_t n, int hidden, int64_t ld_x,
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ pv,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ pt,
    const typename Elem<DT>::T *__restrict__ bt, int normalize, float eps,
    typename Elem<DT>::T *__restrict__ q, int64_t ld_q, float *__restrict__ q_sqnorm) {
  using T = typename Elem<DT>::T;
  constexpr int NCB = DirectCfg<DIM>::NCB;
  constexpr int DX = DirectCfg<DIM>::kDepthX;
  constexpr int DP = DirectCfg<DIM>::kDepthP;
  static_assert(DX % DP == 0, "x ring must be a multiple of the P ring");
  constexpr int kRowPad = DIM + 4;
  __shared__ float red[KW][16][kRowPad];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  const int64_t arow = row0 + (lane & 15);  // the row this lane loads (lanes l and l+16k share it)
  const bool arow_ok = arow < n;
  const T *xrow = x + (arow_ok ? arow : 0) * ld_x;

  const int nks = (hidden + 31) / 32;
  const int per = (nks + KW - 1) / KW;
  const int ks_begin = wave * per;
  const int ks_end = (ks_begin + per < nks) ? ks_begin + per : nks;
  const int klast = ks_end - 1;  // >= 0: clamp target of every load past this wave's slice
  const int kq = 8 * (lane >> 4);  // this lane's 8-wide k chunk within a 32-wide k-step

  // Loads are unconditional (addresses clamped into the operands) so the
  // compiler can count them and keep both rings in flight; rows past n read
  // row 0 (their results are dropped) and x chunks past `hidden` in a partial
  // last k-step are zeroed when consumed (the packed P is zero there too).
  uint4 ar[DX];
  bool kin[DX];
  uint4 br[DP][NCB];
  auto fetch_x = [&](int slot, int ks) {
    const int kc = ks < klast ? ks : klast;
    const int kraw = kc * 32 + kq;
    kin[slot] = kraw < hidden;
    const int k = kraw < hidden - 8 ? kraw : hidden - 8;  // a valid 16-byte chunk
    ar[slot] = *reinterpret_cast<const uint4 *>(xrow + k);
  };
  // Issue order: the row's modality byte, then the first pass's x ring, then
  // the bias; loads complete in order, so the modality ballot below waits only
  // for the first load while the x loads stay in flight.
  // (unconditional load: without is_vision it reads a byte of x and ignores it)
  const uint8_t *vsrc = is_vision ? is_vision + (arow_ok ? arow : 0) : reinterpret_cast<const uint8_t *>(x);
  const uint8_t vis_byte = *vsrc;
#pragma unroll
  for (int s = 0; s < DX; ++s) fetch_x(s, ks_begin + s);

  const int amod = !arow_ok ? 2 : ((is_vision == nullptr || vis_byte) ? 0 : 1);
  const uint32_t vis_bits = (uint32_t)(__ballot(amod == 0) & 0xFFFFull);  // bit r: row r uses P_vis
  const uint32_t txt_bits = (uint32_t)(__ballot(amod == 1) & 0xFFFFull);

  // Epilogue mapping (TPR threads per row, 8 columns each); both modalities'
  // bias chunks are loaded now so their latency hides behind the k loop.
  constexpr int TPR = DIM / 8;
  constexpr int RPP = 64 * KW / TPR;  // rows per pass
  constexpr int NPASS = (16 + RPP - 1) / RPP;
  const int part = tid % TPR;
  float bias_v[8], bias_t[8];
  tm_load8<DT>(bv + part * 8, bias_v);
  tm_load8<DT>(bt + part * 8, bias_t);

  tm_f32x4 fin[NCB];
#pragma unroll
  for (int c = 0; c < NCB; ++c) fin[c] = tm_f32x4{0.f, 0.f, 0.f, 0.f};

  auto run_pass = [&](const T *P, uint32_t rows_of_pass, bool refetch_x) {
    tm_f32x4 acc[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) acc[c] = tm_f32x4{0.f, 0.f, 0.f, 0.f};
    const uint4 *pf = reinterpret_cast<const uint4 *>(P) + lane;
    auto fetch_p = [&](int slot, int ks) {
      const int kc = ks < klast ? ks : klast;
#pragma unroll
      for (int c = 0; c < NCB; ++c) br[slot][c] = pf[((int64_t)kc * NCB + c) * 64];
    };
    auto consume = [&](int xs, int ps) {
      const uint4 a = kin[xs] ? ar[xs] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int c = 0; c < NCB; ++c) acc[c] = tm_mfma16x16x32<DT>(a, br[ps][c], acc[c]);
    };
    if (refetch_x) {
#pragma unroll
      for (int s = 0; s < DX; ++s) fetch_x(s, ks_begin + s);
    }
#pragma unroll
    for (int s = 0; s < DP; ++s) fetch_p(s, ks_begin + s);
    int ks0 = ks_begin;
    for (; ks0 + DX <= ks_end; ks0 += DX) {  // full rings: no guards
#pragma unroll
      for (int j = 0; j < DX; ++j) {
        consume(j, j % DP);
        fetch_p(j % DP, ks0 + j + DP);
        fetch_x(j, ks0 + j + DX);
      }
    }
    if (ks0 < ks_end) {  // remainder: x already in the ring, P still streamed
#pragma unroll
      for (int j = 0; j < DX; ++j) {
        if (ks0 + j < ks_end) consume(j, j % DP);
        fetch_p(j % DP, ks0 + j + DP);
      }
    }
    // keep the rows of this pass: D row of acc[c][i] is 4*(lane>>4)+i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool mine = (rows_of_pass >> (4 * (lane >> 4) + i)) & 1u;
#pragma unroll
      for (int c = 0; c < NCB; ++c)
        if (mine) fin[c][i] = acc[c][i];
    }
  };
  if (vis_bits) run_pass(pv, vis_bits, false);  // uniform branches
  if (txt_bits) run_pass(pt, txt_bits, vis_bits != 0);

#pragma unroll
  for (int c = 0; c < NCB; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][4 * (lane >> 4) + i][c * 16 + (lane & 15)] = fin[c][i];
  __syncthreads();

  // Row epilogue: the wave partials are added in wave order.
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int row = ps * RPP + tid / TPR;
    const bool in_tile = row < 16;
    const int64_t gr = row0 + row;
    const bool ok = in_tile && gr < n;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.f;
    if (ok) {
#pragma unroll
      for (int w = 0; w < KW; ++w) {
        const float4 a = *reinterpret_cast<const float4 *>(&red[w][row][part * 8]);
        const float4 b = *reinterpret_cast<const float4 *>(&red[w][row][part * 8 + 4]);
        v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
        v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
      }
      const bool vis = (vis_bits >> row) & 1u;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = tm_round<DT>(v[i] + (vis ? bias_v[i] : bias_t[i]));
    }
    finish_row<DT, TPR>(v, normalize, eps, ok ? q + gr * ld_q + part * 8 : nullptr,
                        (ok && part == 0 && q_sqnorm) ? q_sqnorm + gr : nullptr);
  }
}

// Column-split packed path (internal, used by the layer call).
//
// Every CU that owns all DIM columns of its rows streams all of P (hidden *
// DIM * 2 bytes) from L2, and the per-CU fetch rate bounds that.  Here a
// workgroup owns 32 token rows and 64 of the DIM columns, so a CU fetches
// (32 + 64) * hidden * 2 bytes (the smallest sum for 32 * 64 outputs), and
// its 4 waves split `hidden` so no two waves load the same bytes.  Each wave
// computes a 32 x 64 partial tile (2 x 4 MFMA blocks per 32-wide k-step); the
// wave partials are added in wave order through LDS.  The row epilogue adds
// the bias, rounds once and writes the 64 columns and the partial |q|^2 of
// those columns, qn_part[g][row] (the consumer adds the DIM / 64 parts in
// order).  No normalisation (the rows' norm needs all columns).
//
// Operands: B (packed P) fragments are contiguous 1 KiB per wave and are
// loaded straight into a register ring.  A (x) fragments span 16 rows x 64
// bytes, a gather that halves the fetch rate, so x travels in chunks of 4
// k-steps instead: one load covers 4 rows x 256 contiguous bytes (whole cache
// lines), the chunk is written to the wave's own LDS tile and the fragments
// are read back from it.  Slot s (16 bytes) of tile row r holds the row's
// chunk s ^ (r % 16), so the 16 rows of a fragment read fall in distinct
// banks.  The values and the order of every fp32 operation are those of
// project_direct_kernel with 4 waves (same k slices, same MFMA sequence).
//
// Placement: the DIM / 64 column groups of a row tile get block ids 8 apart,
// so the dispatcher's round-robin over the 8 XCDs puts them on one XCD and
// they share its L2 copy of the x rows.  The same launch may carry the
// router (workgroups after the projection ones) and, when `keys` is set,
// resets the tile's packed top-1 search keys to ~0 (no candidate yet).
template <int DIM>
struct ColsCfg {
  static constexpr int G = DIM / 64;    // column groups
  static constexpr int NCB = DIM / 16;  // 16-column blocks of the packed layout
  static constexpr int XC = 1;          // x chunks (4 k-steps each) in flight per wave
  static constexpr int DP = 4;          // k-steps of P in flight per wave (= k-steps per x chunk)
};

struct ColsRoute {
  tm_route_args a;
  int64_t first;  // first router workgroup
};

template <int DT, int DIM, int RVPL>
__global__ __launch_bounds__(256, 2) void project_cols_kernel(
    const typename Elem<DT>::T *__restrict__ x, int64_t n, int hidden, int64_t ld_x,
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ pv,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ pt,
    const typename Elem<DT>::T *__restrict__ bt, typename Elem<DT>::T *__restrict__ q, int64_t ld_q,
    float *__restrict__ qn_part, uint64_t *__restrict__ keys, int64_t n_tiles, ColsRoute cr) {
  using T = typename Elem<DT>::T;
  constexpr int G = ColsCfg<DIM>::G;
  constexpr int NCB = ColsCfg<DIM>::NCB;
  constexpr int XC = ColsCfg<DIM>::XC;
  constexpr int DP = ColsCfg<DIM>::DP;
  static_assert(DP == 4 && G >= 1, "one P ring round per x chunk");
  constexpr int kRowPad = 64 + 4;
  __shared__ float red[4][32][kRowPad];
  __shared__ uint4 xs[4][32 * 16];  // per wave: 32 rows x 16 slots (one 4-k-step chunk)

  const int tid = threadIdx.x;
  if constexpr (RVPL > 0) {
    if ((int64_t)blockIdx.x >= cr.first) {  // uniform: router workgroup, 32 tokens
      const int64_t tok = ((int64_t)blockIdx.x - cr.first) * 32 + (tid >> 3);
      tm_route_token<RVPL, 8>(cr.a.logits, n, cr.a.ld, cr.a.top_k, 0, cr.a.out_w, cr.a.out_ids, tok, tid & 7);
      return;
    }
  }
  const int64_t b = blockIdx.x;
  const int64_t tile = (b / (8 * G)) * 8 + (b % 8);
  const int g = (int)((b / 8) % G);
  if (tile >= n_tiles) return;  // uniform (the grid is padded to whole groups of 8 tiles)

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t row0 = tile * 32;

  const int nks = (hidden + 31) / 32;
  const int per = (nks + 3) / 4;
  const int ks_begin = wave * per;
  const int ks_end = (ks_begin + per < nks) ? ks_begin + per : nks;
  const int klast = ks_end - 1 >= 0 ? ks_end - 1 : 0;  // clamp target of every P load past this wave's slice
  const int nchunk = ks_end > ks_begin ? (ks_end - ks_begin + 3) / 4 : 0;

  // x chunk loads: load i (0..7) of a chunk brings tile rows 4i + lane/16, this
  // lane's 16 bytes being the row's chunk slot (lane % 16) ^ (row % 16).
  // Unconditional with clamped addresses (rows past n read the last row and
  // are dropped; chunks past `hidden` are zeroed when written to LDS).
  // (addresses are recomputed per load: a pointer per load slot would cost
  // more registers than the ring itself)
  const int xslot = lane & 15;
  const int xr0 = lane >> 4;
  const int64_t rows_left = n - 1 - row0;  // rows past n read the last row
  auto x_src = [&](int i, int c) {
    const int r = 4 * i + xr0;
    const int kk = (ks_begin + 4 * c) * 32 + 8 * (xslot ^ (r & 15));
    return x + (row0 + (r < rows_left ? r : rows_left)) * ld_x + (kk < hidden ? kk : hidden - 8);
  };
  uint4 xr[XC][8];
  auto load_x = [&](int u, int c) {  // chunk c of this wave's slice into register set u
#pragma unroll
    for (int i = 0; i < 8; ++i) xr[u][i] = *reinterpret_cast<const uint4 *>(x_src(i, c));
  };
  uint4 *xw = &xs[wave][0];
  auto store_x = [&](int u, int c) {
    if ((ks_begin + 4 * c + 4) * 32 <= hidden) {  // uniform: the whole chunk lies inside `hidden`
#pragma unroll
      for (int i = 0; i < 8; ++i) xw[(4 * i + xr0) * 16 + xslot] = xr[u][i];
    } else {  // (a select per element here made the compiler branch and wait around each one)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 4 * i + xr0;
        const int kk = (ks_begin + 4 * c) * 32 + 8 * (xslot ^ (r & 15));
        xw[r * 16 + xslot] = kk < hidden ? xr[u][i] : make_uint4(0, 0, 0, 0);
      }
    }
  };
  // A fragment of k-step t of the chunk in LDS, rows 16*rb + lane%16
  auto read_a = [&](int rb, int t) {
    const int r = 16 * rb + (lane & 15);
    return xw[r * 16 + ((4 * t + (lane >> 4)) ^ (r & 15))];
  };

  // modality byte of row (lane & 31) first: loads complete in order
  const int64_t vr = row0 + (lane & 31);
  const bool vr_ok = vr < n;
  const uint8_t *vsrc = is_vision ? is_vision + (vr_ok ? vr : 0) : reinterpret_cast<const uint8_t *>(x);
  const uint8_t vis_byte = *vsrc;
#pragma unroll
  for (int u = 0; u < XC; ++u) load_x(u, u);
  const int amod = !vr_ok ? 2 : ((is_vision == nullptr || vis_byte) ? 0 : 1);
  const uint32_t vis_bits = (uint32_t)(__ballot(amod == 0) & 0xFFFFFFFFull);  // bit r: tile row r uses P_vis
  const uint32_t txt_bits = (uint32_t)(__ballot(amod == 1) & 0xFFFFFFFFull);

  // epilogue mapping: 8 threads per row, 8 columns each
  const int erow = tid >> 3;
  const int part = tid & 7;
  const int col = 64 * g + 8 * part;
  const uint4 braw_v = *reinterpret_cast<const uint4 *>(bv + col);  // raw: 4 registers each
  const uint4 braw_t = *reinterpret_cast<const uint4 *>(bt + col);

  uint4 br[DP][4];
  auto run_pass = [&](const T *P, uint32_t rows_of_pass, bool refetch_x) {
    tm_f32x4 acc[2][4];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[rb][c] = tm_f32x4{0.f, 0.f, 0.f, 0.f};
    const uint4 *pf = reinterpret_cast<const uint4 *>(P) + (int64_t)(4 * g) * 64 + lane;
    auto fetch_p = [&](int slot, int ks) {
      const int kc = ks < klast ? ks : klast;
#pragma unroll
      for (int c = 0; c < 4; ++c) br[slot][c] = pf[((int64_t)kc * NCB + c) * 64];
    };
    auto consume = [&](int t) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const uint4 a = read_a(rb, t);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[rb][c] = tm_mfma16x16x32<DT>(a, br[t][c], acc[rb][c]);
      }
    };
    if (refetch_x) {
#pragma unroll
      for (int u = 0; u < XC; ++u) load_x(u, u);
    }
#pragma unroll
    for (int t = 0; t < DP; ++t) fetch_p(t, ks_begin + t);
    int c0 = 0;
    for (; c0 + XC <= nchunk; c0 += XC) {  // whole rounds of the x ring: no guards
#pragma unroll
      for (int u = 0; u < XC; ++u) {
        const int c = c0 + u;
        store_x(u, c);
        load_x(u, c + XC);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int ks = ks_begin + 4 * c + t;
          if (ks < ks_end) consume(t);  // (only a partial last chunk skips)
          fetch_p(t, ks + DP);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < XC; ++u) {  // remainder: fewer than XC chunks, already in registers
      const int c = c0 + u;
      if (c < nchunk) {  // uniform
        store_x(u, c);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int ks = ks_begin + 4 * c + t;
          if (ks < ks_end) consume(t);
          fetch_p(t, ks + DP);
        }
      }
    }
    // this pass's rows go to the wave's LDS tile (D row of acc[rb][c][i] is
    // 16*rb + 4*(lane>>4) + i); the passes own disjoint rows
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rb + 4 * (lane >> 4) + i;
        if ((rows_of_pass >> r) & 1u) {
#pragma unroll
          for (int c = 0; c < 4; ++c) red[wave][r][16 * c + (lane & 15)] = acc[rb][c][i];
        }
      }
  };
  if (vis_bits) run_pass(pv, vis_bits, false);  // uniform branches
  if (txt_bits) run_pass(pt, txt_bits, vis_bits != 0);
  __syncthreads();

  const int64_t gr = row0 + erow;
  const bool ok = gr < n;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {  // wave order: deterministic
    const float4 a = *reinterpret_cast<const float4 *>(&red[w][erow][8 * part]);
    const float4 c = *reinterpret_cast<const float4 *>(&red[w][erow][8 * part + 4]);
    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
    v[4] += c.x; v[5] += c.y; v[6] += c.z; v[7] += c.w;
  }
  const bool vis = (vis_bits >> erow) & 1u;
  const uint4 braw = vis ? braw_v : braw_t;
  const T *be = reinterpret_cast<const T *>(&braw);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = tm_round<DT>(v[i] + Elem<DT>::to_f(be[i]));
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  ss += __shfl_xor(ss, 4, 64);
  if (ok) {
    tm_store8<DT>(q + gr * ld_q + col, v);
    if (part == 0) qn_part[(int64_t)g * n + gr] = ss;
    if (keys != nullptr && g == 0 && part == 1) keys[gr] = ~0ull;
  }
}

// project_cols_pipe_kernel: the column-split projection with every operand
// load issued from inline asm and waited for with an exact count (DIM = 128,
// hidden = 512 * NCH: each wave's slice is NCH whole chunks of 4 k-steps, so
// the pipeline is straight-line code with compile-time wait counts).  Same
// tiles, waves, k slices and MFMA sequence as project_cols_kernel, so the
// same bits.
//
// Loads retire in order.  In the register kernel the P fragments of chunk
// c + 1 are requested after the x of chunk c + 2, so waiting for them waits
// for that x too, and every chunk costs one HBM round trip (~1.5 us under
// load; P is as cold as x when each layer has its own table).  Here each wave
// keeps two chunks of both operands in flight: a 2-slot ring of x chunks in
// LDS (direct global -> LDS loads, 8 KiB a chunk) and two register buffers of
// P chunks (16 KiB each).  While chunk c is multiplied, P(c + 2, t) is issued
// into P(c, t)'s registers as soon as k-step t is done, then x(c + 2) into
// chunk c's slot once its fragment reads are done, so every wait leaves the
// next chunk's loads in flight.  The compiler does not see these loads, so it adds no waits of its own; the
// values are tied to the waits by empty asm statements, which every path
// reaches after the wait that retires them (no register that a load will
// still write is read or reused before).  LDS per workgroup is
// the ring (64 KiB), with the wave partials aliased onto it after the last
// chunk, so two workgroups fit a CU (router workgroups of the same launch
// included).  Tiles that mix modalities run the pipeline once per modality
// (the second pass streams x again) and keep each row's own result.
//
// CB: 16-column blocks per workgroup.  4 (64 columns, two groups at d = 128)
// keeps a CU's bytes smallest once the grid fills the chip; 2 (32 columns,
// four groups) doubles the workgroups for batches whose 64-column grid
// leaves half the CUs idle (a workgroup then streams 256 KiB instead of
// 384 KiB).  The groups' partial |q|^2 are subtrees of the direct kernel's
// lane tree either way (8 or 4 lanes of 8 columns), so qn_sum adds them to
// the same bits.
template <int DT, int DIM, int RVPL, int NCH, int CB, int RB = 2>
__global__ __launch_bounds__(256, 2) void project_cols_pipe_kernel(
    const typename Elem<DT>::T *__restrict__ x, int64_t n, int hidden, int64_t ld_x,
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ pv,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ pt,
    const typename Elem<DT>::T *__restrict__ bt, typename Elem<DT>::T *__restrict__ q, int64_t ld_q,
    float *__restrict__ qn_part, uint64_t *__restrict__ keys, int64_t n_tiles, ColsRoute cr, int normalize,
    float eps, float *__restrict__ q_sqnorm) {
  using T = typename Elem<DT>::T;
  constexpr int G = DIM / (16 * CB);  // column groups
  constexpr int NCB = ColsCfg<DIM>::NCB;
  static_assert(NCH >= 1 && NCH <= 8, "chunks per wave");
  constexpr int kRowPad = 64 + 4;
  static_assert((DIM == 128 && (CB == 4 || CB == 2)) || (DIM == 64 && CB == 4),
                "CB column blocks of 1 KiB per k-step and wave");
  constexpr int TPRW = 2 * CB;  // epilogue threads per row (8 columns each)
  static_assert(RB == 1 || RB == 2, "16 or 32 rows per tile");
  constexpr int TR = 16 * RB;    // rows per tile
  constexpr int XS = TR * 16;    // 16-byte chunks per ring slot (TR rows x 4 k-steps)
  constexpr int NXL = 4 * RB;    // x loads per chunk and wave (4 rows each)
  // per wave: 2 ring slots of up to 32 rows x 16 x 16 bytes; the wave
  // partials (TR x kRowPad floats) reuse the wave's own slots after its last
  // chunk
  __shared__ uint4 ring[4][2 * 512];
  static_assert(32 * kRowPad * 4 <= 2 * 512 * 16, "partials fit the wave's ring");

  const int tid = threadIdx.x;
  if constexpr (RVPL > 0) {
    if ((int64_t)blockIdx.x >= cr.first) {  // uniform: router workgroup, 32 tokens
      const int64_t tok = ((int64_t)blockIdx.x - cr.first) * 32 + (tid >> 3);
      tm_route_token<RVPL, 8>(cr.a.logits, n, cr.a.ld, cr.a.top_k, 0, cr.a.out_w, cr.a.out_ids, tok, tid & 7);
      return;
    }
  }
  const int64_t b = blockIdx.x;
  const int64_t tile = (b / (8 * G)) * 8 + (b % 8);
  const int g = (int)((b / 8) % G);
  if (tile >= n_tiles) return;  // uniform (the grid is padded to whole groups of 8 tiles)

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t row0 = tile * TR;

  const int ks_begin = wave * 4 * NCH;  // hidden == 512 * NCH (checked by the launcher)

  const int xslot = lane & 15;
  const int xr0 = lane >> 4;
  const int64_t rows_left = n - 1 - row0;
  auto x_src = [&](int i, int c) {  // rows past n read the last row
    const int r = 4 * i + xr0;
    const int kk = (ks_begin + 4 * c) * 32 + 8 * (xslot ^ (r & 15));
    return x + (row0 + (r < rows_left ? r : rows_left)) * ld_x + kk;
  };
  const uint32_t lds_w = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&ring[wave][0]);
  auto issue_x = [&](int c) {  // chunk c into slot c & 1: load i brings rows 4i .. 4i + 3
#pragma unroll
    for (int i = 0; i < NXL; ++i) tm_dma16_s(x_src(i, c), lds_w + (uint32_t)(((c & 1) * XS + 64 * i) * 16));
  };
  auto read_a = [&](int c, int rb, int t) {  // A fragment of k-step t of chunk c, rows 16*rb + lane%16
    const int r = 16 * rb + (lane & 15);
    return ring[wave][(c & 1) * XS + r * 16 + ((4 * t + (lane >> 4)) ^ (r & 15))];
  };

  // modality byte of row (lane & 31), then the first two x chunks; the byte
  // is in once at most NXL * X0 loads remain outstanding
  const int64_t vr = row0 + (lane & 31);
  const bool vr_ok = (lane & 31) < TR && vr < n;
  const uint8_t *vsrc = is_vision ? is_vision + (vr_ok ? vr : 0) : reinterpret_cast<const uint8_t *>(x);
  uint32_t vb;
  asm volatile("global_load_ubyte %0, %1, off" : "=v"(vb) : "v"(vsrc) : "memory");
  constexpr int X0 = NCH > 1 ? 2 : 1;  // x chunks issued ahead of the loop
  issue_x(0);
  if constexpr (X0 > 1) issue_x(1);
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(vb) : "n"(NXL * X0) : "memory");
  const int amod = !vr_ok ? 2 : ((is_vision == nullptr || (vb & 0xffu)) ? 0 : 1);
  const uint32_t vis_bits = (uint32_t)(__ballot(amod == 0) & 0xFFFFFFFFull);  // bit r: tile row r uses P_vis
  const uint32_t txt_bits = (uint32_t)(__ballot(amod == 1) & 0xFFFFFFFFull);

  const int erow = tid / TPRW;  // rows past 31 (CB = 2: threads 128 ..) only load
  const int part = tid % TPRW;
  const int col = 16 * CB * g + 8 * part;
  const uint4 braw_v = *reinterpret_cast<const uint4 *>(bv + col);
  const uint4 braw_t = *reinterpret_cast<const uint4 *>(bt + col);

  tm_u32x4 pb[2][4][CB];  // P of two chunks: [c & 1][k-step][column block]
  tm_f32x4 fin[RB][CB];   // each row's result from the pass of its modality
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int c = 0; c < CB; ++c) fin[rb][c] = tm_f32x4{0.f, 0.f, 0.f, 0.f};

  auto run_pass = [&](const T *P, uint32_t rows_of_pass, bool first) {
    const uint4 *pf = reinterpret_cast<const uint4 *>(P) + (int64_t)(CB * g) * 64 + lane;
    auto issue_p = [&](int c, int t) {  // k-step t of chunk c
      const uint4 *src = pf + (int64_t)(ks_begin + 4 * c + t) * NCB * 64;
      if constexpr (CB == 4)
        asm volatile(
            "global_load_dwordx4 %0, %4, off\n\t"
            "global_load_dwordx4 %1, %4, off offset:1024\n\t"
            "global_load_dwordx4 %2, %4, off offset:2048\n\t"
            "global_load_dwordx4 %3, %4, off offset:3072"
            : "=&v"(pb[c & 1][t][0]), "=&v"(pb[c & 1][t][1]), "=&v"(pb[c & 1][t][2]), "=&v"(pb[c & 1][t][3])
            : "v"(src)
            : "memory");
      else
        asm volatile(
            "global_load_dwordx4 %0, %2, off\n\t"
            "global_load_dwordx4 %1, %2, off offset:1024"
            : "=&v"(pb[c & 1][t][0]), "=&v"(pb[c & 1][t][1])
            : "v"(src)
            : "memory");
    };
    if (!first) {  // the first pass's x chunks were issued before the modality wait
      issue_x(0);
      if constexpr (X0 > 1) issue_x(1);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) issue_p(0, t);
    if constexpr (NCH > 1) {
#pragma unroll
      for (int t = 0; t < 4; ++t) issue_p(1, t);
    }
    tm_f32x4 acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int c = 0; c < CB; ++c) acc[rb][c] = tm_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      // x(c) and P(c) are in once only the loads issued after both remain:
      // P(1) for chunk 0 (x(1) precedes P(0)); for chunk c >= 1 the P and x of
      // chunk c + 1, issued while chunk c - 1 was multiplied (4 k-steps of CB
      // P loads, NXL x loads a chunk)
      constexpr int kAfter0 = NCH > 1 ? 4 * CB : 0;
      constexpr int kAfterMid = 4 * CB + NXL;
      if (c == 0)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfter0) : "memory");
      else if (c + 1 < NCH)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfterMid) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < CB; ++u) asm volatile("" : "+v"(pb[c & 1][t][u]));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const uint4 a = read_a(c, rb, t);
#pragma unroll
          for (int u = 0; u < CB; ++u) {
            const tm_u32x4 &bb = pb[c & 1][t][u];
            acc[rb][u] = tm_mfma16x16x32<DT>(a, make_uint4(bb.x, bb.y, bb.z, bb.w), acc[rb][u]);
          }
        }
        if (c + 2 < NCH) issue_p(c + 2, t);
      }
      if (c + 2 < NCH) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // chunk c's fragment reads are done
        issue_x(c + 2);
      }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // nothing of this pass still lands in the ring
    // D row of acc[rb][u][i] is 16*rb + 4*(lane>>4) + i
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool mine = (rows_of_pass >> (16 * rb + 4 * (lane >> 4) + i)) & 1u;
#pragma unroll
        for (int u = 0; u < CB; ++u) fin[rb][u][i] = mine ? acc[rb][u][i] : fin[rb][u][i];
      }
  };
  if (vis_bits) run_pass(pv, vis_bits, true);  // uniform branches
  if (txt_bits) run_pass(pt, txt_bits, vis_bits == 0);
  if (!vis_bits && !txt_bits) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no row: drain the x loads

  float *red = reinterpret_cast<float *>(&ring[0][0]);  // [4][TR][kRowPad], wave w inside its own ring
  auto red_at = [&](int w, int r, int c) { return red + w * (2 * 512 * 4) + r * kRowPad + c; };
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * rb + 4 * (lane >> 4) + i;
#pragma unroll
      for (int u = 0; u < CB; ++u) *red_at(wave, r, 16 * u + (lane & 15)) = fin[rb][u][i];
    }
  __syncthreads();
  if (erow >= TR) return;  // threads past the tile's rows (waves 2 and 3 when TR * TPRW = 128; no barrier follows)

  const int64_t gr = row0 + erow;
  const bool ok = gr < n;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {  // wave order: deterministic
    const float4 a = *reinterpret_cast<const float4 *>(red_at(w, erow, 8 * part));
    const float4 c = *reinterpret_cast<const float4 *>(red_at(w, erow, 8 * part + 4));
    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
    v[4] += c.x; v[5] += c.y; v[6] += c.z; v[7] += c.w;
  }
  const bool vis = (vis_bits >> erow) & 1u;
  const uint4 braw = vis ? braw_v : braw_t;
  const T *be = reinterpret_cast<const T *>(&braw);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = tm_round<DT>(v[i] + Elem<DT>::to_f(be[i]));
  // the row epilogue of project_direct_kernel (normalisation needs the whole
  // row: one column group, which the host ensures); the column group's
  // partial |q|^2 (qn_part) or the row's (q_sqnorm)
  float *sq_dst = nullptr;
  if (ok && part == 0) sq_dst = qn_part != nullptr ? qn_part + (int64_t)g * n + gr : (q_sqnorm ? q_sqnorm + gr : nullptr);
  finish_row<DT, TPRW>(v, normalize, eps, ok ? q + gr * ld_q + col : nullptr, sq_dst);
  if (ok && keys != nullptr && g == 0 && part == 1) keys[gr] = ~0ull;
}

// tm_project_pack: one thread per 16-byte chunk of the packed layout.
template <int DT>
__global__ __launch_bounds__(kThreads) void project_pack_kernel(const typename Elem<DT>::T *__restrict__ src,
                                                                int hidden, int dim, int64_t ps_h, int64_t ps_d,
                                                                int64_t n_chunks, uint4 *__restrict__ out) {
  using T = typename Elem<DT>::T;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n_chunks) return;
  const int ncb = dim / 16;
  const int lane = (int)(i & 63);
  const int64_t frag = i >> 6;
  const int c = (int)(frag % ncb);
  const int64_t t = frag / ncb;
  const int col = 16 * c + (lane & 15);
  const int64_t k0 = 32 * t + 8 * (lane >> 4);
  T e[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t h = k0 + j;
    e[j] = (h < hidden) ? src[h * ps_h + (int64_t)col * ps_d] : Elem<DT>::from_f(0.f);
  }
  uint4 v;
  __builtin_memcpy(&v, e, sizeof(v));
  out[i] = v;
}

template <int DT, int DIM, bool PK, bool SPLIT>
__global__ __launch_bounds__(kThreads) void project_mfma_kernel(
    const typename Elem<DT>::T *__restrict__ x, int64_t n, int hidden, int64_t ld_x,
    const uint8_t *__restrict__ is_vision, const typename Elem<DT>::T *__restrict__ pv,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ pt,
    const typename Elem<DT>::T *__restrict__ bt, int64_t ps_h, int64_t ps_d, int normalize,
    float eps, typename Elem<DT>::T *__restrict__ q, int64_t ld_q, float *__restrict__ q_sqnorm,
    int k_chunk, float *__restrict__ partial) {
  using T = typename Elem<DT>::T;
  constexpr int NBLK = (kBM / 16) * (DIM / 16);  // 16x16 output blocks
  constexpr int PER_WAVE = (NBLK + 3) / 4;
  constexpr int PCH = (DIM * kBK / 8 + kThreads - 1) / kThreads;  // P chunks per thread per stage
  __shared__ __attribute__((aligned(16))) T xs[2][kBM][kBK + kPad];
  __shared__ __attribute__((aligned(16))) T ps[2][DIM][kBK + kPad];
  __shared__ float qs[SPLIT ? 1 : kBM][SPLIT ? 1 : DIM + 1];
  __shared__ uint8_t row_mod[kBM];
  __shared__ int mod_present[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * kBM;
  const int split = blockIdx.y;
  const int k_begin = split * k_chunk;
  const int k_end = (k_begin + k_chunk < hidden) ? k_begin + k_chunk : hidden;
  const int nstage = (k_end - k_begin + kBK - 1) / kBK;

  if (tid < 2) mod_present[tid] = 0;
  __syncthreads();
  if (tid < kBM) {
    const int64_t r = row0 + tid;
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

    tm_f32x4 acc[PER_WAVE];
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) acc[i] = tm_f32x4{0.f, 0.f, 0.f, 0.f};

    uint4 xr;
    uint4 pr[PCH];
    auto fetch = [&](int k0) {
      {
        const int r = tid >> 3, c8 = (tid & 7) * 8;
        const int64_t gr = row0 + r;
        xr = make_uint4(0, 0, 0, 0);
        if (gr < n && k0 + c8 < k_end) xr = *reinterpret_cast<const uint4 *>(x + gr * ld_x + k0 + c8);
      }
#pragma unroll
      for (int u = 0; u < PCH; ++u) {
        const int ci = tid + u * kThreads;
        pr[u] = make_uint4(0, 0, 0, 0);
        if (ci < DIM * (kBK / 8)) {
          if constexpr (PK) {
            const int j = ci / (kBK / 8), h0 = (ci % (kBK / 8)) * 8;
            if (k0 + h0 < k_end) pr[u] = *reinterpret_cast<const uint4 *>(P + (int64_t)j * ps_d + k0 + h0);
          } else {
            const int h = ci / (DIM / 8), j0 = (ci % (DIM / 8)) * 8;
            if (k0 + h < k_end) pr[u] = *reinterpret_cast<const uint4 *>(P + (int64_t)(k0 + h) * ps_h + j0);
          }
        }
      }
    };
    auto stash = [&](int buf) {
      {
        const int r = tid >> 3, c8 = (tid & 7) * 8;
        *reinterpret_cast<uint4 *>(&xs[buf][r][c8]) = xr;
      }
#pragma unroll
      for (int u = 0; u < PCH; ++u) {
        const int ci = tid + u * kThreads;
        if (ci < DIM * (kBK / 8)) {
          if constexpr (PK) {
            const int j = ci / (kBK / 8), h0 = (ci % (kBK / 8)) * 8;
            *reinterpret_cast<uint4 *>(&ps[buf][j][h0]) = pr[u];
          } else {
            const int h = ci / (DIM / 8), j0 = (ci % (DIM / 8)) * 8;
            const T *e = reinterpret_cast<const T *>(&pr[u]);
#pragma unroll
            for (int i = 0; i < 8; ++i) ps[buf][j0 + i][h] = e[i];
          }
        }
      }
    };

    fetch(k_begin);
    for (int st = 0; st < nstage; ++st) {
      const int buf = st & 1;
      stash(buf);
      __syncthreads();
      if (st + 1 < nstage) fetch(k_begin + (st + 1) * kBK);
#pragma unroll
      for (int ks = 0; ks < kBK / 32; ++ks) {
        const int kk = ks * 32 + 8 * (lane >> 4);
#pragma unroll
        for (int i = 0; i < PER_WAVE; ++i) {
          const int b = wave + 4 * i;
          if (b < NBLK) {
            const int rb = b % (kBM / 16), cb = b / (kBM / 16);
            const uint4 a = *reinterpret_cast<const uint4 *>(&xs[buf][rb * 16 + (lane & 15)][kk]);
            const uint4 bb = *reinterpret_cast<const uint4 *>(&ps[buf][cb * 16 + (lane & 15)][kk]);
            acc[i] = tm_mfma16x16x32<DT>(a, bb, acc[i]);
          }
        }
      }
    }
    __syncthreads();  // every wave is done with both LDS buffers before the next pass refills them

#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int b = wave + 4 * i;
      if (b < NBLK) {
        const int rb = b % (kBM / 16), cb = b / (kBM / 16);
        const int col = cb * 16 + (lane & 15);
        if constexpr (SPLIT) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb * 16 + 4 * (lane >> 4) + r;
            const int64_t gr = row0 + row;
            if (gr < n && row_mod[row] == m) partial[((int64_t)split * n + gr) * DIM + col] = acc[i][r];
          }
        } else {
          const float bcol = Elem<DT>::to_f(((m == 0) ? bv : bt)[col]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb * 16 + 4 * (lane >> 4) + r;
            if (row_mod[row] == m) qs[row][col] = tm_round<DT>(acc[i][r] + bcol);
          }
        }
      }
    }
  }
  if constexpr (!SPLIT) {
    __syncthreads();
    // Row epilogue: DIM/8 threads per row, 8 columns each (DIM >= 16 -> 2..32 threads).
    constexpr int TPR = DIM / 8;
    constexpr int RPP = kThreads / TPR;  // rows per pass
    for (int r0 = 0; r0 < kBM; r0 += RPP) {
      const int row = r0 + tid / TPR, part = tid % TPR;
      const int64_t gr = row0 + row;
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (row < kBM) ? qs[row < kBM ? row : 0][part * 8 + i] : 0.f;
      const bool ok = row < kBM && gr < n;
      finish_row<DT, TPR>(v, normalize, eps, ok ? q + gr * ld_q + part * 8 : nullptr,
                          (ok && part == 0 && q_sqnorm) ? q_sqnorm + gr : nullptr);
    }
  }
}

// Split epilogue: q[r] = finish(dtype(sum_s partial[s][r] + bias_m)).  One
// 64-thread workgroup per 64 / (DIM / 8) rows, so the partials (L2-resident:
// the split kernel just wrote them) spread over many CUs.
constexpr int kEpiThreads = 64;
template <int DT, int DIM>
__global__ __launch_bounds__(kEpiThreads) void project_epilogue_kernel(
    const float *__restrict__ partial, int nsplit, int64_t n, const uint8_t *__restrict__ is_vision,
    const typename Elem<DT>::T *__restrict__ bv, const typename Elem<DT>::T *__restrict__ bt, int normalize,
    float eps, typename Elem<DT>::T *__restrict__ q, int64_t ld_q, float *__restrict__ q_sqnorm) {
  constexpr int TPR = DIM / 8;
  constexpr int RPB = kEpiThreads / TPR;
  constexpr int kRound = 16;  // splits whose loads are issued together
  const int tid = threadIdx.x;
  const int64_t r = (int64_t)blockIdx.x * RPB + tid / TPR;
  const int part = tid % TPR;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.f;
  const bool ok = r < n;
  if (ok) {
    // splits summed in order; the loads of kRound splits issued before the adds
    for (int s0 = 0; s0 < nsplit; s0 += kRound) {
      float4 a[kRound], b[kRound];
#pragma unroll
      for (int u = 0; u < kRound; ++u) {
        if (s0 + u < nsplit) {
          const float4 *src = reinterpret_cast<const float4 *>(partial + ((int64_t)(s0 + u) * n + r) * DIM + part * 8);
          a[u] = src[0];
          b[u] = src[1];
        }
      }
#pragma unroll
      for (int u = 0; u < kRound; ++u) {
        if (s0 + u < nsplit) {
          v[0] += a[u].x; v[1] += a[u].y; v[2] += a[u].z; v[3] += a[u].w;
          v[4] += b[u].x; v[5] += b[u].y; v[6] += b[u].z; v[7] += b[u].w;
        }
      }
    }
    const bool vis = is_vision == nullptr || is_vision[r];
    const typename Elem<DT>::T *bias = (vis ? bv : bt) + part * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = tm_round<DT>(v[i] + Elem<DT>::to_f(bias[i]));
  }
  finish_row<DT, TPR>(v, normalize, eps, ok ? q + r * ld_q + part * 8 : nullptr,
                      (ok && part == 0 && q_sqnorm) ? q_sqnorm + r : nullptr);
}

// fp32 path (DIM in {32, 64, 128, 256}): fp32 FMAs on the vector units.  A
// workgroup owns kBM rows and all DIM columns over one k chunk of the split
// plan and writes fp32 partials [split][n][DIM] (summed in split order by
// project_epilogue_kernel, which also adds the bias, rounds and normalises).
// k advances 32 at a time through LDS: the x tile [kBM][32] and the P tile
// [32][DIM] of each modality present in the tile, loaded along whichever of
// P's axes is contiguous.  Thread (row group, column group) accumulates RPT
// rows x 4 columns, each output a sequential sum over its k chunk.
template <int DIM>
__global__ __launch_bounds__(kThreads) void project_f32_kernel(
    const float *__restrict__ x, int64_t n, int hidden, int64_t ld_x, const uint8_t *__restrict__ is_vision,
    const float *__restrict__ pv, const float *__restrict__ pt, int64_t ps_h, int64_t ps_d, int k_chunk,
    float *__restrict__ partial) {
  constexpr int KT = 32;
  constexpr int CG = DIM / 4;           // column groups of 4
  constexpr int RG = kThreads / CG;     // row groups
  constexpr int RPT = kBM / RG;         // rows per thread
  static_assert(RPT >= 1 && RG * RPT == kBM, "tile shape");
  __shared__ float xs[kBM][KT + 1];
  __shared__ float4 ps[2][KT][CG];
  __shared__ int s_mods;
  const int tid = threadIdx.x;
  const int cg = tid % CG, rg = tid / CG;
  const int64_t r0 = (int64_t)blockIdx.x * kBM;
  const int k0 = blockIdx.y * k_chunk;
  const int k1 = k0 + k_chunk < hidden ? k0 + k_chunk : hidden;
  if (tid == 0) s_mods = 0;
  __syncthreads();
  if (tid < kBM) {
    const int64_t r = r0 + tid;
    if (r < n) atomicOr(&s_mods, (is_vision == nullptr || is_vision[r]) ? 1 : 2);
  }
  __syncthreads();
  const int mods = s_mods;  // bit 0: a vision row, bit 1: a text row
  int mrow[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t r = r0 + rg * RPT + i;
    mrow[i] = (r < n && is_vision != nullptr && !is_vision[r]) ? 1 : 0;
  }
  float acc[RPT][4];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[i][c] = 0.f;
  // Tile kb's operands are loaded into registers one tile ahead (the loads
  // of tile kb + KT are in flight while tile kb is multiplied).
  constexpr int XE = kBM * KT / kThreads;  // x elements per thread per tile
  constexpr int PE = KT * DIM / kThreads;  // P elements per thread per tile and modality
  float xr[XE], pr[2][PE];
  auto load = [&](int kb) {
#pragma unroll
    for (int u = 0; u < XE; ++u) {
      const int e = tid + u * kThreads, row = e / KT, kk = e % KT;
      const int64_t r = r0 + row;
      xr[u] = (r < n && kb + kk < k1) ? x[r * ld_x + kb + kk] : 0.f;
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      if (!(mods & (1 << m))) continue;  // uniform
      const float *P = m == 0 ? pv : pt;
#pragma unroll
      for (int u = 0; u < PE; ++u) {
        const int e = tid + u * kThreads;
        int kk, j;
        if (ps_d == 1) { kk = e / DIM; j = e % DIM; }  // row-major [hidden, DIM]: contiguous along j
        else { j = e / KT; kk = e % KT; }              // k-contiguous copy: contiguous along h
        const int h = kb + kk;
        pr[m][u] = h < k1 ? P[(int64_t)h * ps_h + (int64_t)j * ps_d] : 0.f;
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int u = 0; u < XE; ++u) {
      const int e = tid + u * kThreads;
      xs[e / KT][e % KT] = xr[u];
    }
    float *psf = reinterpret_cast<float *>(ps);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      if (!(mods & (1 << m))) continue;
#pragma unroll
      for (int u = 0; u < PE; ++u) {
        const int e = tid + u * kThreads;
        int kk, j;
        if (ps_d == 1) { kk = e / DIM; j = e % DIM; }
        else { j = e / KT; kk = e % KT; }
        psf[(m * KT + kk) * DIM + j] = pr[m][u];
      }
    }
  };
  if (k0 < k1) load(k0);
  for (int kb = k0; kb < k1; kb += KT) {
    __syncthreads();  // the previous tile's reads are done
    stash();
    __syncthreads();
    if (kb + KT < k1) load(kb + KT);
#pragma unroll 8
    for (int kk = 0; kk < KT; ++kk) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float xv = xs[rg * RPT + i][kk];
        const float4 pw = ps[mrow[i]][kk][cg];
        acc[i][0] = fmaf(xv, pw.x, acc[i][0]);
        acc[i][1] = fmaf(xv, pw.y, acc[i][1]);
        acc[i][2] = fmaf(xv, pw.z, acc[i][2]);
        acc[i][3] = fmaf(xv, pw.w, acc[i][3]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t r = r0 + rg * RPT + i;
    if (r < n)
      *reinterpret_cast<float4 *>(partial + ((int64_t)blockIdx.y * n + r) * DIM + 4 * cg) =
          make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
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

template <int DT, int DIM>
int launch_mfma(const ProjPlan &pl, bool split, bool pk, const typename Elem<DT>::T *X, int64_t n, int hidden,
                int64_t ld_x, const uint8_t *is_vision, const typename Elem<DT>::T *PV,
                const typename Elem<DT>::T *BV, const typename Elem<DT>::T *PT, const typename Elem<DT>::T *BT,
                int64_t ps_h, int64_t ps_d, int normalize, float eps, typename Elem<DT>::T *Q, int64_t ld_q,
                float *q_sqnorm, float *partial, hipStream_t stream) {
  const int nsplit = split ? pl.nsplit : 1;
  const int k_chunk = split ? pl.k_chunk : (int)tm_cdiv(hidden, kBK) * kBK;
  dim3 grid((unsigned)pl.row_blocks, (unsigned)nsplit), block(kThreads);
  if (split) {
    if (pk)
      hipLaunchKernelGGL((project_mfma_kernel<DT, DIM, true, true>), grid, block, 0, stream, X, n, hidden, ld_x,
                         is_vision, PV, BV, PT, BT, ps_h, ps_d, normalize, eps, Q, ld_q, q_sqnorm, k_chunk, partial);
    else
      hipLaunchKernelGGL((project_mfma_kernel<DT, DIM, false, true>), grid, block, 0, stream, X, n, hidden, ld_x,
                         is_vision, PV, BV, PT, BT, ps_h, ps_d, normalize, eps, Q, ld_q, q_sqnorm, k_chunk, partial);
    TM_LAUNCH_CHECK("tm_project");
    constexpr int RPB = kEpiThreads / (DIM / 8);
    hipLaunchKernelGGL((project_epilogue_kernel<DT, DIM>), dim3((unsigned)tm_cdiv(n, RPB)), dim3(kEpiThreads), 0,
                       stream, partial, nsplit, n, is_vision, BV, BT, normalize, eps, Q, ld_q, q_sqnorm);
    TM_LAUNCH_CHECK("tm_project(epilogue)");
    return TM_OK;
  }
  if (pk)
    hipLaunchKernelGGL((project_mfma_kernel<DT, DIM, true, false>), grid, block, 0, stream, X, n, hidden, ld_x,
                       is_vision, PV, BV, PT, BT, ps_h, ps_d, normalize, eps, Q, ld_q, q_sqnorm, k_chunk, nullptr);
  else
    hipLaunchKernelGGL((project_mfma_kernel<DT, DIM, false, false>), grid, block, 0, stream, X, n, hidden, ld_x,
                       is_vision, PV, BV, PT, BT, ps_h, ps_d, normalize, eps, Q, ld_q, q_sqnorm, k_chunk, nullptr);
  TM_LAUNCH_CHECK("tm_project");
  return TM_OK;
}

// Rows from which tm_project's packed d = 64 path takes the pipelined kernel.
constexpr int64_t kPipeMinRows64 = 2048;

template <int DT>
int launch_project(const void *x, int64_t n, int hidden, int64_t ld_x, const uint8_t *is_vision,
                   const void *pv, const void *bv, const void *pt, const void *bt, int64_t ps_h,
                   int64_t ps_d, int dim, int normalize, float eps, void *q, int64_t ld_q,
                   float *q_sqnorm, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const T *X = static_cast<const T *>(x);
  const T *PV = static_cast<const T *>(pv), *BV = static_cast<const T *>(bv);
  const T *PT = static_cast<const T *>(pt ? pt : pv), *BT = static_cast<const T *>(pt ? bt : bv);
  T *Q = static_cast<T *>(q);
  const bool packed = ps_h == 0 && ps_d == 0;
  const bool pk = (ps_h == 1);
  const int E = Elem<DT>::kBytes;
  bool mfma_ok = DT != TM_DT_F32 && (hidden % 8 == 0) && (dim == 16 || dim == 32 || dim == 64 ||
                                                           dim == 128 || dim == 256);
  if (mfma_ok)
    mfma_ok = tm_aligned16(x) && ((ld_x * E) % 16 == 0) && tm_aligned16(pv) && tm_aligned16(PT) &&
              (pk ? ((ps_d * E) % 16 == 0) : ((ps_h * E) % 16 == 0)) && tm_aligned16(q) && ((ld_q * E) % 16 == 0);
  if (packed) {
    TM_REQUIRE(mfma_ok && tm_aligned16(BV) && tm_aligned16(BT), TM_EINVAL_ARG,
               "tm_project: the packed layout needs F16/BF16, hidden %% 8 == 0, dim in {16..256} and "
               "16-byte aligned x/q rows and bias");
  }
  if constexpr (DT != TM_DT_F32) {
  if (packed) {
    // d = 64 at the model hidden sizes with many rows: the pipelined column
    // kernel with one 64-column group per 16-row tile (its operand loads in
    // flight two chunks ahead; the direct kernel's tiles, slices, MFMA chains,
    // wave order and row epilogue, so the same bits)
    if (dim == 64 && (hidden == 2048 || hidden == 2560) && n >= kPipeMinRows64 &&
        n < ((int64_t)1 << 31) / 32) {
      const int64_t n_tiles = tm_cdiv(n, 16);
      auto kern = hidden == 2048 ? project_cols_pipe_kernel<DT, 64, 0, 4, 4, 1> : project_cols_pipe_kernel<DT, 64, 0, 5, 4, 1>;
      hipLaunchKernelGGL(kern, dim3((unsigned)(tm_cdiv(n_tiles, 8) * 8)), dim3(256), 0, stream, X, n, hidden, ld_x,
                         is_vision, PV, BV, PT, BT, Q, ld_q, nullptr, nullptr, n_tiles, ColsRoute{}, normalize, eps,
                         q_sqnorm);
      TM_LAUNCH_CHECK("tm_project");
      return TM_OK;
    }
    // 16 rows per workgroup, 4 waves splitting hidden
    const dim3 grid((unsigned)tm_cdiv(n, 16));
    switch (dim) {
#define TM_PROJ_PACKED(D)                                                                                    \
  case D:                                                                                                  \
    hipLaunchKernelGGL((project_direct_kernel<DT, D, 4>), grid, dim3(256), 0, stream, X, n, hidden, ld_x,     \
                       is_vision, PV, BV, PT, BT, normalize, eps, Q, ld_q, q_sqnorm);                       \
    TM_LAUNCH_CHECK("tm_project");                                                                         \
    return TM_OK;
      TM_PROJ_PACKED(16)
      TM_PROJ_PACKED(32)
      TM_PROJ_PACKED(64)
      TM_PROJ_PACKED(128)
      TM_PROJ_PACKED(256)
#undef TM_PROJ_PACKED
      default: break;
    }
  }
  if (mfma_ok) {
    const ProjPlan pl = plan_project(n, hidden);
    const size_t need = (size_t)pl.nsplit * (size_t)n * (size_t)dim * sizeof(float);
    const bool split = pl.nsplit > 1 && workspace != nullptr && workspace_bytes >= need &&
                       tm_aligned16(workspace);
    float *partial = static_cast<float *>(workspace);
    switch (dim) {
#define TM_PROJ_CASE(D)                                                                                     \
  case D:                                                                                                  \
    return launch_mfma<DT, D>(pl, split, pk, X, n, hidden, ld_x, is_vision, PV, BV, PT, BT, ps_h, ps_d,     \
                              normalize, eps, Q, ld_q, q_sqnorm, partial, stream);
      TM_PROJ_CASE(16)
      TM_PROJ_CASE(32)
      TM_PROJ_CASE(64)
      TM_PROJ_CASE(128)
      TM_PROJ_CASE(256)
#undef TM_PROJ_CASE
      default: break;
    }
  }
  }
  if constexpr (DT == TM_DT_F32) {
    const ProjPlan pl = plan_project_f32(n, hidden, dim);
    const size_t need = (size_t)pl.nsplit * (size_t)n * (size_t)dim * sizeof(float);
    const bool tiled = (dim == 32 || dim == 64 || dim == 128 || dim == 256) && !packed && workspace != nullptr &&
                       workspace_bytes >= need && tm_aligned16(workspace) && tm_aligned16(q) && (ld_q % 4) == 0;
    if (tiled) {
      float *partial = static_cast<float *>(workspace);
      const dim3 grid((unsigned)pl.row_blocks, (unsigned)pl.nsplit);
      switch (dim) {
#define TM_PROJ_F32(D)                                                                                         \
  case D:                                                                                                      \
    hipLaunchKernelGGL((project_f32_kernel<D>), grid, dim3(kThreads), 0, stream, X, n, hidden, ld_x, is_vision, \
                       PV, PT, ps_h, ps_d, pl.k_chunk, partial);                                                \
    TM_LAUNCH_CHECK("tm_project");                                                                             \
    hipLaunchKernelGGL((project_epilogue_kernel<DT, D>), dim3((unsigned)tm_cdiv(n, kEpiThreads / (D / 8))),     \
                       dim3(kEpiThreads), 0, stream, partial, pl.nsplit, n, is_vision, BV, BT, normalize, eps, Q, \
                       ld_q, q_sqnorm);                                                                         \
    TM_LAUNCH_CHECK("tm_project(epilogue)");                                                                   \
    return TM_OK;
        TM_PROJ_F32(32)
        TM_PROJ_F32(64)
        TM_PROJ_F32(128)
        TM_PROJ_F32(256)
#undef TM_PROJ_F32
        default: break;
      }
    }
  }
  const int rows_per_block = kThreads / dim;
  dim3 grid((unsigned)tm_cdiv(n, rows_per_block)), block(kThreads);
  hipLaunchKernelGGL((project_scalar_kernel<DT>), grid, block, 0, stream, X, n, hidden, ld_x,
                     is_vision, PV, BV, PT, BT, ps_h, ps_d, dim, normalize, eps, Q, ld_q, q_sqnorm);
  TM_LAUNCH_CHECK("tm_project");
  return TM_OK;
}

}  // namespace

extern "C" size_t tm_project_workspace_size(int64_t n_tokens, int32_t hidden, int32_t dim) {
  if (n_tokens <= 0 || hidden <= 0 || dim <= 0) return 0;
  const int s16 = plan_project(n_tokens, hidden).nsplit;      // 16-bit operands, matrix cores
  const int s32 = plan_project_f32(n_tokens, hidden, dim).nsplit;  // fp32 operands
  const int ns = s16 > s32 ? s16 : s32;
  if (ns <= 1) return 0;
  return (size_t)ns * (size_t)n_tokens * (size_t)dim * sizeof(float);
}

extern "C" int tm_project(int32_t dtype, const void *x, int64_t n_tokens, int32_t hidden,
                          int64_t ld_x, const uint8_t *is_vision, const void *proj_vis,
                          const void *bias_vis, const void *proj_txt, const void *bias_txt,
                          int64_t ps_h, int64_t ps_d, int32_t dim, int32_t normalize, float eps,
                          void *q_out, int64_t ld_q, float *q_sqnorm, void *workspace,
                          size_t workspace_bytes, tm_stream_t stream) {
  TM_REQUIRE(n_tokens >= 0 && hidden > 0 && dim > 0 && dim <= 256, TM_EINVAL_SHAPE,
             "tm_project: bad sizes n=%lld hidden=%d dim=%d", (long long)n_tokens, hidden, dim);
  TM_REQUIRE(ld_x >= hidden && ld_q >= dim, TM_EINVAL_SHAPE, "tm_project: bad row strides");
  TM_REQUIRE(ps_h == 1 || ps_d == 1 || (ps_h == 0 && ps_d == 0), TM_EINVAL_SHAPE,
             "tm_project: projection needs a unit stride along hidden or dim, or the packed layout");
  TM_REQUIRE(proj_vis && bias_vis && q_out && (n_tokens == 0 || x), TM_EINVAL_ARG,
             "tm_project: null pointer");
  TM_REQUIRE((proj_txt == nullptr) == (bias_txt == nullptr), TM_EINVAL_ARG,
             "tm_project: proj_txt and bias_txt must both be set or both be NULL");
  TM_REQUIRE(n_tokens < ((int64_t)1 << 31) / 32, TM_EINVAL_SHAPE, "tm_project: too many tokens");
  if (n_tokens == 0) return TM_OK;
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    return launch_project<DT>(x, n_tokens, hidden, ld_x, is_vision, proj_vis, bias_vis, proj_txt,
                              bias_txt, ps_h, ps_d, dim, normalize, eps, q_out, ld_q, q_sqnorm,
                              workspace, workspace_bytes, tm_hip_stream(stream));
  });
}

extern "C" size_t tm_project_packed_size(int32_t hidden, int32_t dim, int32_t dtype) {
  if (hidden <= 0 || (dim != 16 && dim != 32 && dim != 64 && dim != 128 && dim != 256) ||
      (dtype != TM_DT_BF16 && dtype != TM_DT_F16))
    return 0;
  return (size_t)tm_cdiv(hidden, 32) * 32 * (size_t)dim * 2;
}

extern "C" int tm_project_pack(int32_t dtype, const void *src, int32_t hidden, int32_t dim, int64_t ps_h,
                               int64_t ps_d, void *packed, size_t packed_bytes, tm_stream_t stream) {
  const size_t need = tm_project_packed_size(hidden, dim, dtype);
  TM_REQUIRE(dtype == TM_DT_BF16 || dtype == TM_DT_F16, TM_EINVAL_DTYPE, "tm_project_pack: dtype %d", dtype);
  TM_REQUIRE(need > 0, TM_EINVAL_SHAPE, "tm_project_pack: bad sizes hidden=%d dim=%d", hidden, dim);
  TM_REQUIRE(src && packed && tm_aligned16(packed), TM_EINVAL_ARG, "tm_project_pack: null or unaligned pointer");
  TM_REQUIRE(packed_bytes >= need, TM_EWORKSPACE, "tm_project_pack: %zu bytes given, %zu needed", packed_bytes,
             need);
  const int64_t n_chunks = (int64_t)(need / 16);
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    if constexpr (DT != TM_DT_F32) {
      hipLaunchKernelGGL((project_pack_kernel<DT>), dim3((unsigned)tm_cdiv(n_chunks, kThreads)), dim3(kThreads), 0,
                         tm_hip_stream(stream), static_cast<const typename Elem<DT>::T *>(src), hidden, dim, ps_h,
                         ps_d, n_chunks, static_cast<uint4 *>(packed));
      TM_LAUNCH_CHECK("tm_project_pack");
    }
    return TM_OK;
  });
}

namespace {

template <int DT, int DIM, int RVPL>
void launch_cols(const void *x, int64_t n, int hidden, int64_t ld_x, const uint8_t *is_vision, const void *pv,
                 const void *bv, const void *pt, const void *bt, void *q, int64_t ld_q, float *qn_part,
                 uint64_t *keys, const tm_route_args *ra, hipStream_t stream) {
  using T = typename Elem<DT>::T;
  const int64_t n_tiles = tm_cdiv(n, 32);
  ColsRoute cr{};
  const int64_t groups = (int64_t)tm_internal_project_cols_parts(DIM, n, hidden);
  int64_t blocks = tm_cdiv(n_tiles, 8) * 8 * groups;
  if (RVPL > 0) {
    cr.a = *ra;
    cr.first = blocks;
    blocks += tm_cdiv(n, 32);
  }
  if constexpr (DIM == 128) {
    // hidden 2048 or 2560: every wave's slice is 4 or 5 whole chunks, the pipelined kernel
    if (hidden == 2048 || hidden == 2560) {
      const bool narrow = groups == 4;  // 32-column groups
      auto kern = hidden == 2048 ? (narrow ? project_cols_pipe_kernel<DT, DIM, RVPL, 4, 2>
                                           : project_cols_pipe_kernel<DT, DIM, RVPL, 4, 4>)
                                 : (narrow ? project_cols_pipe_kernel<DT, DIM, RVPL, 5, 2>
                                           : project_cols_pipe_kernel<DT, DIM, RVPL, 5, 4>);
      hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<const T *>(x), n, hidden,
                         ld_x, is_vision, static_cast<const T *>(pv), static_cast<const T *>(bv),
                         static_cast<const T *>(pt ? pt : pv), static_cast<const T *>(pt ? bt : bv),
                         static_cast<T *>(q), ld_q, qn_part, keys, n_tiles, cr, 0, 0.f, nullptr);
      return;
    }
  }
  hipLaunchKernelGGL((project_cols_kernel<DT, DIM, RVPL>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const T *>(x), n, hidden, ld_x, is_vision, static_cast<const T *>(pv),
                     static_cast<const T *>(bv), static_cast<const T *>(pt ? pt : pv),
                     static_cast<const T *>(pt ? bt : bv), static_cast<T *>(q), ld_q, qn_part, keys, n_tiles, cr);
}

template <int DT, int DIM>
void launch_cols_route(const void *x, int64_t n, int hidden, int64_t ld_x, const uint8_t *is_vision,
                       const void *pv, const void *bv, const void *pt, const void *bt, void *q, int64_t ld_q,
                       float *qn_part, uint64_t *keys, const tm_route_args *ra, hipStream_t stream) {
  if (ra == nullptr)
    launch_cols<DT, DIM, 0>(x, n, hidden, ld_x, is_vision, pv, bv, pt, bt, q, ld_q, qn_part, keys, ra, stream);
  else if (ra->n_experts == 64)
    launch_cols<DT, DIM, 8>(x, n, hidden, ld_x, is_vision, pv, bv, pt, bt, q, ld_q, qn_part, keys, ra, stream);
  else
    launch_cols<DT, DIM, 16>(x, n, hidden, ld_x, is_vision, pv, bv, pt, bt, q, ld_q, qn_part, keys, ra, stream);
}

}  // namespace

bool tm_internal_project_cols_ok(int32_t dtype, const void *x, int64_t n, int32_t hidden, int64_t ld_x,
                                 const void *pv, const void *bv, const void *pt, const void *bt, int64_t ps_h,
                                 int64_t ps_d, int32_t dim, const void *q, int64_t ld_q) {
  const bool packed = ps_h == 0 && ps_d == 0;
  return (dtype == TM_DT_BF16 || dtype == TM_DT_F16) && packed && (dim == 64 || dim == 128 || dim == 256) &&
         n > 0 && n < ((int64_t)1 << 31) / 32 && hidden >= 8 && hidden % 8 == 0 && ld_x >= hidden &&
         ld_q >= dim && x && pv && bv && q && (pt == nullptr) == (bt == nullptr) && tm_aligned16(x) &&
         (ld_x * 2) % 16 == 0 && tm_aligned16(pv) && tm_aligned16(bv) && (pt == nullptr || tm_aligned16(pt)) &&
         (bt == nullptr || tm_aligned16(bt)) && tm_aligned16(q) && (ld_q * 2) % 16 == 0;
}

// Column groups of the column-split projection, which is also the number of
// partial |q|^2 per row: 64-column groups, or 32-column groups at d = 128 on
// the pipelined kernel's hidden sizes when the 64-column grid would keep at
// most half of the 256 CUs busy (n <= 2048).
size_t tm_internal_project_cols_parts(int32_t dim, int64_t n, int32_t hidden) {
  if (dim < 64) return 0;
  const bool narrow = dim == 128 && (hidden == 2048 || hidden == 2560) && tm_cdiv(n, 32) * 2 <= 128;
  return narrow ? 4 : (size_t)dim / 64;
}

int tm_internal_project_cols(int32_t dtype, const void *x, int64_t n, int32_t hidden, int64_t ld_x,
                             const uint8_t *is_vision, const void *pv, const void *bv, const void *pt,
                             const void *bt, int64_t ps_h, int64_t ps_d, int32_t dim, void *q, int64_t ld_q,
                             float *qn_part, uint64_t *keys, const tm_route_args *ra, hipStream_t stream) {
  TM_REQUIRE(tm_internal_project_cols_ok(dtype, x, n, hidden, ld_x, pv, bv, pt, bt, ps_h, ps_d, dim, q, ld_q) &&
                 qn_part != nullptr,
             TM_EINVAL_ARG, "tm_table_forward: projection shape not supported by the column-split kernel");
  TM_REQUIRE(ra == nullptr || tm_internal_route_fusable(ra), TM_EINVAL_ARG,
             "tm_table_forward: router shape cannot be fused");
  return TM_DISPATCH_DTYPE(dtype, DT, [&] {
    if constexpr (DT != TM_DT_F32) {
      switch (dim) {
        case 64: launch_cols_route<DT, 64>(x, n, hidden, ld_x, is_vision, pv, bv, pt, bt, q, ld_q, qn_part, keys, ra, stream); break;
        case 128: launch_cols_route<DT, 128>(x, n, hidden, ld_x, is_vision, pv, bv, pt, bt, q, ld_q, qn_part, keys, ra, stream); break;
        default: launch_cols_route<DT, 256>(x, n, hidden, ld_x, is_vision, pv, bv, pt, bt, q, ld_q, qn_part, keys, ra, stream); break;
      }
      TM_LAUNCH_CHECK("tm_table_forward(project)");
    }
    return TM_OK;
  });
}
