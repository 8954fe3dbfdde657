// Full-weight linear layers: per-example gradient norms and the clipped sum
// on CDNA4 MFMA, without materialising per-example gradients.
//
// For y = x W^T the per-example weight gradient is M_i = G_i^T X_i
// (d_out x d_in) over the example's rows.  The reference materialises every
// M_i under vmap(grad) (opaque-engine/.../clipping/_clipped_fun.py:756-762)
// and then squares, scales and sums them.  Here:
//
//   k_lin_outer_norm : ||M_i||_F^2 tile by tile (256 x 256 output tiles,
//                      contraction over the example's tokens), squares
//                      summed in fp64 into one partial slot per tile;
//   k_lin_gram_norm  : sum_{t,s} (x_t . x_s)(g_t . g_s) over the upper
//                      triangle of 128-token blocks (off-diagonal blocks
//                      counted twice), one block against two per workgroup,
//                      the cheaper form when the example is short relative
//                      to the weight;
//   k_lin_prescale   : X' = c_i x_t rounded to bf16, per (X, group, class).
//   k_lin_clip_sum   : out = sum_i c_i M_i as one GEMM over all rows, on X'
//                      or with the clip factor applied to each example's X
//                      fragments in registers (the same c_i x_t in bf16).
//
// All three are bf16 MFMA (16x16x32, fp32 accumulate).  Operand tiles move
// from HBM to LDS by buffer loads straight into LDS (no staging registers)
// through rings of LDS stages, several steps ahead of the compute, with
// explicit vmcnt waits and LDS-only barriers; buffer resources bounded to
// the current segment's rows turn rows outside it into zeros.  Rows are
// token-major in HBM, so the outer-product forms read their operands K-major
// and take them from LDS with the gfx950 transposing read; the Gram form's
// operands are K-contiguous rows.
#include "odp_internal.h"

namespace {

#include "odp_outer.h"

constexpr int LT = 128;         // token block of the Gram form
constexpr int OUTER_GROUP = 8;  // tile rows per group in the outer-norm work order
static_assert(WN == 64 && 2 * WM * WN <= OUTER_STAGE && NW <= 2 * RING,
              "two waves' bf16 blocks fit in each ring stage (outer-norm store)");

// Work decoding of the Gram form.  Workgroups are dispatched round-robin
// over the 8 XCDs (blockIdx % 8), each with its own L2, and every problem's
// block count is a multiple of 8 so that blockIdx % 8 == local % 8.  With 8
// or more segments, XCD j works through segments j, j + 8, ... so that an
// example's rows are cached by one L2 only (the workgroups drift apart in
// the feature loop).  Returns false for padding blocks.
__device__ __forceinline__ bool seg_item(int local, int n_seg, int per_seg, int& seg, int& item) {
  if (n_seg >= 8) {
    const int k = local >> 3;
    seg = (local & 7) + 8 * (k / per_seg);
    item = k % per_seg;
  } else {
    seg = local / per_seg;
    item = local % per_seg;
  }
  return seg < n_seg;
}

// Block-wide fp64 sum; the result is valid in thread 0.
__device__ __forceinline__ double block_sum(double v, double* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < NW; w += 4) t += (red[w] + red[w + 1]) + (red[w + 2] + red[w + 3]);
  }
  return t;
}

// fp32 squares of the finite entries, summed in fp64; `nonfinite` is set
// when an entry was not finite (and counted as 0).
template <int I, int J>
__device__ __forceinline__ double acc_sq(const f32x4_t (&acc)[I][J], bool& nonfinite) {
  double s = 0.0;
  static_for<I * J>([&](auto q) {
    constexpr int i = decltype(q)::value / J, j = decltype(q)::value % J;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = acc[i][j][e];
      const bool fin = isfinite(v);
      nonfinite |= !fin;
      const float vf = fin ? v : 0.f;
      s += (double)__fmul_rn(vf, vf);
    }
    // One tile's accumulators at a time in VGPRs.
    __builtin_amdgcn_sched_barrier(0);
  });
  return s;
}

// ---------------------------------------------------------------------------
// ||M_i||^2 partials, outer form.  Workgroup = (segment, o-tile, n-tile).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(OUTER_THREADS, ODP_LIN_OCC) void k_lin_outer_norm(const int64_t* __restrict__ probs,
                                                        const int32_t* __restrict__ ws, int n_prob,
                                                        const int32_t* __restrict__ sstart,
                                                        const int32_t* __restrict__ slen,
                                                        const int32_t* __restrict__ sex,
                                                        double* __restrict__ part, int64_t part_stride) {
  __shared__ double red[NW];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  const int64_t slot = f[ODP_LN_SLOT];
  const int tn_count = (int)((P.d_in + ON - 1) / ON);
  const int tm_count = (int)((P.d_out + OM - 1) / OM);
  const int tiles = tn_count * tm_count;
  // Work order: XCD j (blockIdx % 8) takes the j-th eighth of the problem's
  // (segment, tile) items, so that the workgroups on one L2 share a
  // segment, and walks its tiles in groups of OUTER_GROUP tile rows, so that
  // the concurrent ones share operand columns (+1.5 % on C4 shapes).
  const int local = bid - ws[p];
  const int nblk = (P.n_seg * tiles + 7) / 8 * 8;  // odp_linear_norm_blocks
  const int pid = (local & 7) * (nblk >> 3) + (local >> 3);
  if (pid >= P.n_seg * tiles) return;
  const int seg = pid / tiles;
  int tile;
  {
    const int t = pid - seg * tiles;
    const int per_group = OUTER_GROUP * tn_count, g = t / per_group, first_m = g * OUTER_GROUP;
    const int gm = min(tm_count - first_m, OUTER_GROUP), rr = t - g * per_group;
    tile = (first_m + rr % gm) * tn_count + rr / gm;
  }
  const int64_t o0 = (int64_t)(tile / tn_count) * OM, n0 = (int64_t)(tile % tn_count) * ON;
  const int gs = P.seg_first + seg;
  const int64_t t_begin = sstart[gs], t_end = t_begin + slen[gs];
  const int ex = sex[gs];

  OuterAcc acc;
  zero_acc(acc);
  const Step first = {(int32_t)t_begin, (int32_t)t_begin, (int32_t)t_end, seg, t_end > t_begin ? 1 : 0, 0};
  auto next = [&](const Step& st) {
    Step n = st;
    n.t0 = st.t0 + OK;
    n.live = n.t0 < st.te ? 1 : 0;
    return n;
  };
  dma_mainloop<false, true, false>(P, o0, n0, first, next, [](const Step&) { return 1.0f; },
                                   [](uint16_t*, const Step&) {}, acc);
  // Columns/rows past the matrix were zero operands, so they add nothing.
  // Non-finite entries of M_s count 0 (nan_to_num before the norm).
  bool nonfinite = false;
  const double tot = block_sum(acc_sq(acc, nonfinite), red);
  if (threadIdx.x == 0) part[(int64_t)ex * part_stride + slot + tile] = tot;
  uint32_t* nfflag = (uint32_t*)f[ODP_LN_NFFLAG];
  // Every writer stores the same value, so a plain store suffices.
  if (nfflag != nullptr && nonfinite) odp_gstore(nfflag, 1u);
  // Optionally keep the tile of M_s itself, rounded to bf16, for a later
  // clipped sum over stored per-example gradients.  Each wave's WM x WN
  // block goes through its own part of the (now idle) LDS ring so that rows
  // leave in 16-byte pieces: 8-column chunk q of block row r sits at chunk
  // q ^ ((r >> 2) & 7), which keeps both the 2-byte writes of the MFMA
  // layout and the 16-byte reads free of bank conflicts.
  uint16_t* pe = (uint16_t*)f[ODP_LN_PE];
  if (pe != nullptr) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint16_t* stg = lin_stage(wave >> 1) + (wave & 1) * (WM * WN);
    static_for<BI * BJ>([&](auto q) {
      constexpr int i = decltype(q)::value / BJ, j = decltype(q)::value % BJ;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 16 * i + 4 * (lane >> 4) + e, c = 16 * j + (lane & 15);
        stg[r * WN + 8 * ((c >> 3) ^ ((r >> 2) & 7)) + (c & 7)] = odp_f2bf(acc[i][j][e]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    uint16_t* dst = pe + (int64_t)seg * P.d_out * P.d_in;
    const int64_t ob = o0 + WM * (wave & 1), nb = n0 + WN * (wave >> 1);
#pragma unroll
    for (int k = 0; k < WM / 8; ++k) {
      const int r = 8 * k + (lane >> 3), qq = lane & 7;
      const u32x4_t v = *(const u32x4_alias_t*)&stg[r * WN + 8 * (qq ^ ((r >> 2) & 7))];
      const int64_t o = ob + r, n = nb + 8 * qq;
      // Non-temporal: the stored gradients are read again only by a later
      // launch, and should not evict this launch's operands from L2.
      if (o < P.d_out && n < P.d_in)
        __builtin_nontemporal_store(v, (ODP_GLOBAL u32x4_t*)(ODP_GLOBAL void*)(dst + o * P.d_in + n));
    }
  }
}

// ---------------------------------------------------------------------------
// ||M_i||^2 partials, outer form, for the segments at risk of float32
// overflow in the Gram form only (see lin_seg_at_risk).  GUARD_SPLIT
// workgroups per (problem, segment) exit at once unless the segment is at
// risk, and otherwise loop over its tiles: cheap when no segment is at risk
// (the usual case), exact (slow) when one is.
// ---------------------------------------------------------------------------
constexpr int GUARD_SPLIT = 8;

__global__ __launch_bounds__(OUTER_THREADS, ODP_LIN_OCC) void k_lin_outer_norm_guarded(
    const int64_t* __restrict__ probs, const int32_t* __restrict__ ws, int n_prob,
    const int32_t* __restrict__ sstart, const int32_t* __restrict__ slen, const int32_t* __restrict__ sex,
    double* __restrict__ part, int64_t part_stride) {
  __shared__ double red[NW];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  const int local = bid - ws[p];
  const int seg = local / GUARD_SPLIT, j = local % GUARD_SPLIT;
  if (seg >= P.n_seg) return;
  const int gs = P.seg_first + seg;
  const int32_t t_begin = sstart[gs], len = slen[gs];
  if (!lin_seg_at_risk(f, seg, len, P.d_in, P.d_out)) return;
  const int ex = sex[gs];
  const int64_t slot = f[ODP_LN_SLOT];
  const int tn_count = (int)((P.d_in + ON - 1) / ON);
  const int tiles = tn_count * (int)((P.d_out + OM - 1) / OM);
  uint32_t* nfflag = (uint32_t*)f[ODP_LN_NFFLAG];
  auto next = [](const Step& st) {
    Step n = st;
    n.t0 = st.t0 + OK;
    n.live = n.t0 < st.te ? 1 : 0;
    return n;
  };
  for (int tile = j; tile < tiles; tile += GUARD_SPLIT) {
    const int64_t o0 = (int64_t)(tile / tn_count) * OM, n0 = (int64_t)(tile % tn_count) * ON;
    OuterAcc acc;
    zero_acc(acc);
    const Step first = {t_begin, t_begin, t_begin + len, seg, 1, 0};
    dma_mainloop<false, true, false>(P, o0, n0, first, next, [](const Step&) { return 1.0f; },
                                     [](uint16_t*, const Step&) {}, acc);
    bool nonfinite = false;
    const double tot = block_sum(acc_sq(acc, nonfinite), red);
    if (threadIdx.x == 0) part[(int64_t)ex * part_stride + slot + tile] = tot;
    if (nfflag != nullptr && nonfinite) odp_gstore(nfflag, 1u);
  }
}

// ---------------------------------------------------------------------------
// ||M_i||^2 partials, token-Gram form, wide tiles.  A workgroup of 8 waves
// covers token block tb (128 rows) against blocks sb0 and sb0 + 1 (256
// rows) of one segment, with both Gram products in registers: waves 0-3
// own (tb, sb0), waves 4-7 (tb, sb0 + 1), each a 64 x 64 block of
// sum_f x_t,f x_s,f (features of X) and of sum_f g_t,f g_s,f (features of
// G).  The 384 rows x 32 features of a step arrive by buffer loads straight
// into a ring of GR_RING LDS stages (GR_RING - 1 steps in flight), the X
// steps then the G steps as one sequence.  Rows past the segment and
// features past d arrive as zeros.  Rows are 64 bytes, swizzled in 16-byte
// slots by gr_swz below.
// ---------------------------------------------------------------------------
constexpr int GR_K = 32;                   // features per step
constexpr int GR_ROWS = 3 * LT;            // t block + two s blocks
constexpr int GR_STAGE = GR_ROWS * GR_K;   // elements
constexpr int GR_RING = 6;
constexpr int GR_LOADS = GR_ROWS * GR_K * 2 / 1024 / 8;  // 1 KB loads per wave per step
static_assert(GR_LOADS == 3, "three loads per wave per step");

// Work items of a segment with nb blocks: for each tb, s-block pairs
// sb0 = tb, tb + 2, ... (the second block may lie past the segment).
__host__ __device__ constexpr int64_t gram_items(int64_t nb) {
  return (nb & 1) ? ((nb + 1) / 2) * ((nb + 1) / 2) : (nb / 2) * (nb / 2 + 1);
}

static_assert(GR_K == 32, "one 32-bit column-mask word per Gram step");

// Rows are 64 bytes (four 16-byte slots); slot k of row r lives at slot
// k ^ gr_swz(r).  An MFMA operand read (ds_read_b128) takes slot kq of 16
// consecutive rows per 16 lanes.  Measured with SQ_LDS_BANK_CONFLICT on
// gfx950: this swizzle reads at full rate, while (r >> 2) & 3, no swizzle,
// and ((r >> 1) ^ (r >> 3)) & 3 all take twice the LDS cycles per read.
__device__ __forceinline__ int gr_swz(int row) { return (row >> 1) & 3; }
__device__ __forceinline__ int gr_at(int row, int slot) { return row * GR_K + 8 * (slot ^ gr_swz(row)); }

__global__ __launch_bounds__(512, 1) void k_lin_gram_norm(const int64_t* __restrict__ probs,
                                                             const int32_t* __restrict__ ws, int n_prob,
                                                             const int32_t* __restrict__ sstart,
                                                             const int32_t* __restrict__ slen,
                                                             const int32_t* __restrict__ sex,
                                                             double* __restrict__ part, int64_t part_stride) {
  __shared__ __attribute__((aligned(16))) uint16_t st0[GR_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st1[GR_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st2[GR_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st3[GR_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st4[GR_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t st5[GR_STAGE];
  __shared__ double red[8];
  auto stage = [&](int k) -> uint16_t* {
    return k == 0 ? st0 : k == 1 ? st1 : k == 2 ? st2 : k == 3 ? st3 : k == 4 ? st4 : st5;
  };
  static_assert(GR_RING == 6, "six ring stages");
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  const int64_t slot = f[ODP_LN_SLOT];
  const int nb = (int)f[ODP_LN_NB];
  const int items = (int)gram_items(nb);
  int seg, item;
  if (!seg_item(bid - ws[p], P.n_seg, items, seg, item)) return;
  int tb = 0, rem = item;
  while (rem >= (nb - tb + 1) / 2) {
    rem -= (nb - tb + 1) / 2;
    ++tb;
  }
  const int sb0 = tb + 2 * rem;
  const int gs = P.seg_first + seg;
  const int32_t t_begin = sstart[gs], len = slen[gs];
  const int ex = sex[gs];
  // A segment at risk of float32 overflow takes the outer form instead
  // (ODP_FORM_OUTER_GUARDED); its Gram partials stay 0.
  if (lin_seg_at_risk(f, seg, len, P.d_in, P.d_out)) return;
  double* dst = part + (int64_t)ex * part_stride + slot + item;
  if ((int64_t)sb0 * LT >= len) {  // item past this segment's length
    if (threadIdx.x == 0) *dst = 0.0;
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // Non-finite columns of this segment (odp_nonfinite_columns): `fix` when
  // any is set, then each step zeroes its masked features in LDS.
  const int xw = (int)((P.d_in + 31) / 32), gw = (int)((P.d_out + 31) / 32);
  const uint32_t* xm = (const uint32_t*)f[ODP_LN_XMASK];
  const uint32_t* gm = (const uint32_t*)f[ODP_LN_GMASK];
  if (xm != nullptr) xm += (int64_t)seg * xw;
  if (gm != nullptr) gm += (int64_t)seg * gw;
  int fix = 0;
  if (xm != nullptr || gm != nullptr) {
    int any = 0;
    for (int w = threadIdx.x; w < xw + gw; w += 512)
      any |= (w < xw ? (xm != nullptr ? xm[w] : 0u) : (gm != nullptr ? gm[w - xw] : 0u)) != 0u;
    fix = __syncthreads_or(any);
  }

  // Rows of the stage: 0..127 block tb, 128..255 block sb0, 256..383 sb0 + 1.
  // Wave w loads stage rows 48 w .. + 47, 16 per load; lane l lands in row
  // 16 i' + (l >> 2), physical slot l & 3, and fetches its logical slot.
  int lrow[GR_LOADS];
  uint32_t lbase[GR_LOADS];  // segment row of the loaded row, times the row pitch later
  int lslot[GR_LOADS];
#pragma unroll
  for (int i = 0; i < GR_LOADS; ++i) {
    const int row = 48 * wave + 16 * i + (lane >> 2);
    lrow[i] = row;
    const int blk = row < LT ? tb : (row < 2 * LT ? sb0 : sb0 + 1);
    lbase[i] = (uint32_t)(blk * LT + (row & (LT - 1)));
    lslot[i] = (lane & 3) ^ gr_swz(row);
  }
  const uint32_t nrow = (uint32_t)len;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.X + (int64_t)t_begin * P.ldx), (short)0, (int)(nrow * (uint32_t)P.ldx * 2u), LIN_BUF_DWORD3);
  const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.G + (int64_t)t_begin * P.ldg), (short)0, (int)(nrow * (uint32_t)P.ldg * 2u), LIN_BUF_DWORD3);
  // X steps then G steps, each phase padded to a multiple of the ring size
  // (the padding steps load nothing) so that every step's stage is fixed.
  const int nx = (int)((P.d_in + GR_K - 1) / GR_K), ng = (int)((P.d_out + GR_K - 1) / GR_K);
  const int px = (nx + GR_RING - 1) / GR_RING * GR_RING;
  const int total = px + (ng + GR_RING - 1) / GR_RING * GR_RING;
  const uint32_t ldx = (uint32_t)P.ldx, ldg = (uint32_t)P.ldg;
  const int32_t din = (int32_t)P.d_in, dout = (int32_t)P.d_out;

  // Step x: features [GR_K x', + GR_K) of X (x' = x) or of G (x' = x - nx);
  // steps past the end load nothing (out of range) but still issue.
  auto issue = [&](uint16_t* st, int x) {
    const bool isx = x < px;
    const int32_t kx = isx ? x : x - px;
    const int32_t k0 = kx * GR_K;
    // A finished phase (or step) gets d = 0: every column is then past the end.
    const int32_t d = x < total && kx < (isx ? nx : ng) ? (isx ? din : dout) : 0;
    const uint32_t ld = isx ? ldx : ldg;
    const __amdgpu_buffer_rsrc_t rs = isx ? xr : gr;
#pragma unroll
    for (int i = 0; i < GR_LOADS; ++i) {
      const int32_t col = k0 + 8 * lslot[i];
      const uint32_t o = (lbase[i] * ld + (uint32_t)col) * 2u;
      const uint32_t off = col < d ? o : LIN_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (ODP_LDS void*)(st + (48 * wave + 16 * i) * GR_K), 16, off, 0,
                                               0, 0);
    }
  };

  // Wave w: t rows 64 (w & 1) .., s rows 128 + 64 (w >> 1) .. of the stage.
  const int wt = 64 * (wave & 1), wsr = LT + 64 * (wave >> 1);
  f32x4_t sx[4][4], sg[4][4];
  zero_acc(sx);
  zero_acc(sg);
  auto compute = [&](const uint16_t* st, f32x4_t (&acc)[4][4]) {
    const int r = lane & 15, kq = lane >> 4;
    bf16x8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)&st[gr_at(wt + 16 * i + r, kq)]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b[j] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)&st[gr_at(wsr + 16 * j + r, kq)]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  };

  // One phase: steps [lo, hi) (a multiple of GR_RING), the first `live`
  // of them holding features.
  // Loads into `nxt` and reads of `cur` as restrict parameters of one
  // inlined call: the alias scopes keep the reads from waiting for the
  // loads in flight.
  auto step = [&](uint16_t* __restrict__ nxt, const uint16_t* __restrict__ cur, int x, bool live,
                  f32x4_t (&acc)[4][4]) {
    issue(nxt, x);
    if (live) compute(cur, acc);
  };
  // Zeroes the features of a landed stage whose bits are set in `word`
  // (the step's 32 features), for all 384 rows.
  auto zero_features = [&](uint16_t* st, uint32_t word) {
    const int fc = threadIdx.x & 31;
    if ((word >> fc) & 1u)
      for (int r = threadIdx.x >> 5; r < GR_ROWS; r += 16) st[gr_at(r, fc >> 3) + (fc & 7)] = 0;
  };
  auto phase = [&](int lo, int hi, int live, const uint32_t* mask, f32x4_t (&acc)[4][4]) {
    for (int g0 = lo; g0 < hi; g0 += GR_RING) {
#pragma unroll
      for (int k = 0; k < GR_RING; ++k) {
        const int g = g0 + k;
        // This step's loads have landed; the later GR_RING - 2 steps' may fly.
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((GR_RING - 2) * GR_LOADS));
        __asm__ volatile("s_barrier" ::: "memory");
        if (fix && mask != nullptr && g - lo < live) {
          const uint32_t word = mask[g - lo];  // features [32 (g - lo), + 32)
          if (word != 0u) {
            zero_features(stage(k), word);
            __syncthreads();
          }
        }
        step(stage((k + GR_RING - 1) % GR_RING), stage(k), g + GR_RING - 1, g - lo < live, acc);
      }
    }
  };
#pragma unroll
  for (int x = 0; x < GR_RING - 1; ++x) issue(stage(x), x);
  phase(0, px, nx, xm, sx);
  phase(px, total, ng, gm, sg);
  __builtin_amdgcn_s_waitcnt(0);  // no load into LDS may outlive the workgroup

  // Off-diagonal blocks count twice (the (s, t) block is not computed);
  // a block past the segment holds zeros.
  const int sb = sb0 + (wave >> 2);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += (double)sx[i][j][e] * (double)sg[i][j][e];
  if (sb != tb) s *= 2.0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < 8; ++w) t += red[w];
    *dst = t;
  }
}

// ---------------------------------------------------------------------------
// Gram form over 256-row blocks (ODP_FORM_GRAM256).  Item (tb, sb), tb <= sb,
// of a segment pairs the t block (rows 256 tb ..) with the s block (rows
// 256 sb ..); eight waves in 2 x 4 each own 128 x 64 of the 256 x 256 block
// pair, as in the outer-form kernels, and a step moves 512 rows x G2_K
// features into LDS: 128 flop per byte loaded against 87 for the 128 x 256
// pairs of k_lin_gram_norm, whose loads into LDS bound it.  With 64
// features per step each row piece is a whole 128-byte line (32 features
// fetched every line twice, doubling the L2 requests per flop), in a ring
// of two 64 KB stages.  The two Gram blocks of a
// 256 x 256 pair do not fit in registers together, so the X block
// P = X_t X_s^T is accumulated first and written to the item's fp32 scratch
// in register order (each lane its own 16-byte pieces, 1 KB per wave and
// block), then G's block Q is accumulated and the item's partial
// sum_{t,s} P Q is formed against the scratch read back by the same lanes.
// A diagonal item (tb == sb) loads its rows once and reads both operands
// from them.  Same non-finite column handling and work order as
// k_lin_gram_norm.
// ---------------------------------------------------------------------------
#ifndef ODP_G2_K
#define ODP_G2_K 64  // features per step: 64 (128-byte rows, two stages) or 32 (64-byte rows, four)
#endif
constexpr int G2_B = 256;                                 // rows per block
constexpr int G2_ROWS = 2 * G2_B;                         // t block + s block
constexpr int G2_K = ODP_G2_K;
constexpr int G2_SLOTS = G2_K / 8;                        // 16-byte slots per row
constexpr int G2_STAGE = G2_ROWS * G2_K;                  // elements (64 or 32 KB)
constexpr int G2_RING = G2_K == 64 ? 2 : 4;               // 128 KB of LDS either way
constexpr int G2_LOADS = G2_ROWS * G2_K * 2 / 1024 / 8;   // 1 KB loads per wave per step
constexpr int G2_RPL = 64 / G2_SLOTS;                     // rows per load
constexpr int G2_WORDS = G2_K / 32;                       // column-mask words per step
constexpr int64_t G2_SCRATCH = (int64_t)G2_B * G2_B;      // floats per (segment, item)
static_assert((G2_K == 32 || G2_K == 64) && G2_LOADS * G2_RPL == 64, "each wave loads 64 rows per step");
// Slot k of row r at k ^ g2_swz(r): 16 rows read at one slot hit the LDS at
// full rate (measured; for 64-byte rows as gr_swz).
__device__ __forceinline__ int g2_swz(int row) { return (row >> 1) & (G2_SLOTS - 1); }
__device__ __forceinline__ int g2_at(int row, int slot) { return row * G2_K + 8 * (slot ^ g2_swz(row)); }

__host__ __device__ constexpr int64_t gram2_items(int64_t nb) { return nb * (nb + 1) / 2; }

__global__ __launch_bounds__(512, 1) void k_lin_gram2_norm(const int64_t* __restrict__ probs,
                                                              const int32_t* __restrict__ ws, int n_prob,
                                                              const int32_t* __restrict__ sstart,
                                                              const int32_t* __restrict__ slen,
                                                              const int32_t* __restrict__ sex,
                                                              double* __restrict__ part, int64_t part_stride) {
  __shared__ __attribute__((aligned(16))) uint16_t q0[G2_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t q1[G2_STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t q2[G2_RING > 2 ? G2_STAGE : 8];
  __shared__ __attribute__((aligned(16))) uint16_t q3[G2_RING > 2 ? G2_STAGE : 8];
  __shared__ double red[8];
  auto stage = [&](int k) -> uint16_t* { return k == 0 ? q0 : k == 1 ? q1 : k == 2 ? q2 : q3; };
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  const int64_t slot = f[ODP_LN_SLOT];
  const int nb = (int)f[ODP_LN_NB];
  const int items = (int)gram2_items(nb);
  int seg, item;
  if (!seg_item(bid - ws[p], P.n_seg, items, seg, item)) return;
  int tb = 0, rem = item;
  while (rem >= nb - tb) {
    rem -= nb - tb;
    ++tb;
  }
  const int sb = tb + rem;
  const bool diag = sb == tb;
  const int gs = P.seg_first + seg;
  const int32_t t_begin = sstart[gs], len = slen[gs];
  const int ex = sex[gs];
  if (lin_seg_at_risk(f, seg, len, P.d_in, P.d_out)) return;  // outer form (guarded) instead
  double* dst = part + (int64_t)ex * part_stride + slot + item;
  if ((int64_t)sb * G2_B >= len) {  // item past this segment's length
    if (threadIdx.x == 0) *dst = 0.0;
    return;
  }
  float* scr = (float*)f[ODP_LN_SCRATCH] + ((int64_t)seg * items + item) * G2_SCRATCH;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const int xw = (int)((P.d_in + 31) / 32), gw = (int)((P.d_out + 31) / 32);
  const uint32_t* xm = (const uint32_t*)f[ODP_LN_XMASK];
  const uint32_t* gm = (const uint32_t*)f[ODP_LN_GMASK];
  if (xm != nullptr) xm += (int64_t)seg * xw;
  if (gm != nullptr) gm += (int64_t)seg * gw;
  int fix = 0;
  if (xm != nullptr || gm != nullptr) {
    int any = 0;
    for (int w = threadIdx.x; w < xw + gw; w += 512)
      any |= (w < xw ? (xm != nullptr ? xm[w] : 0u) : (gm != nullptr ? gm[w - xw] : 0u)) != 0u;
    fix = __syncthreads_or(any);
  }

  // Stage rows 0..255: block tb; 256..511: block sb (not loaded for a
  // diagonal item).  Wave w loads rows 64 w .. + 63, G2_RPL per load.
  uint32_t lbase[G2_LOADS];
  int lslot[G2_LOADS];
  bool lload[G2_LOADS];
#pragma unroll
  for (int i = 0; i < G2_LOADS; ++i) {
    const int row = 64 * wave + G2_RPL * i + lane / G2_SLOTS;
    lbase[i] = (uint32_t)((row < G2_B ? tb : sb) * G2_B + (row & (G2_B - 1)));
    lslot[i] = (lane % G2_SLOTS) ^ g2_swz(row);
    lload[i] = row < G2_B || !diag;
  }
  const uint32_t nrow = (uint32_t)len;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.X + (int64_t)t_begin * P.ldx), (short)0, (int)(nrow * (uint32_t)P.ldx * 2u), LIN_BUF_DWORD3);
  const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P.G + (int64_t)t_begin * P.ldg), (short)0, (int)(nrow * (uint32_t)P.ldg * 2u), LIN_BUF_DWORD3);
  const int nx = (int)((P.d_in + G2_K - 1) / G2_K), ng = (int)((P.d_out + G2_K - 1) / G2_K);
  const int px = (nx + G2_RING - 1) / G2_RING * G2_RING;
  const int total = px + (ng + G2_RING - 1) / G2_RING * G2_RING;
  const uint32_t ldx = (uint32_t)P.ldx, ldg = (uint32_t)P.ldg;
  const int32_t din = (int32_t)P.d_in, dout = (int32_t)P.d_out;

  auto issue = [&](uint16_t* st, int x) __attribute__((always_inline)) {
    const bool isx = x < px;
    const int32_t kx = isx ? x : x - px;
    const int32_t k0 = kx * G2_K;
    const int32_t d = x < total && kx < (isx ? nx : ng) ? (isx ? din : dout) : 0;
    const uint32_t ld = isx ? ldx : ldg;
    const __amdgpu_buffer_rsrc_t rs = isx ? xr : gr;
#pragma unroll
    for (int i = 0; i < G2_LOADS; ++i) {
      const int32_t col = k0 + 8 * lslot[i];
      const uint32_t o = (lbase[i] * ld + (uint32_t)col) * 2u;
      const uint32_t off = col < d && lload[i] ? o : LIN_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (ODP_LDS void*)(st + (64 * wave + G2_RPL * i) * G2_K), 16, off,
                                               0, 0, 0);
    }
  };

  // Wave w: t rows 128 (w & 1) .., s rows 64 (w >> 1) .. of the s half (the
  // t half itself for a diagonal item).
  const int wt = 128 * (wave & 1), wsr = (diag ? 0 : G2_B) + 64 * (wave >> 1);
  f32x4_t acc[8][4];
  zero_acc(acc);
  // One step: G2_K / 32 MFMA K blocks in feature order (the same order of
  // 32-feature blocks whatever G2_K, so results do not depend on it).
  auto compute = [&](const uint16_t* st, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
    const int r = lane & 15;
#pragma unroll
    for (int h = 0; h < G2_K / 32; ++h) {
      const int kq = 4 * h + (lane >> 4);
      bf16x8_t b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)&st[g2_at(wsr + 16 * j + r, kq)]);
      // A fragments stream one ahead of the MFMAs that consume them.
      bf16x8_t a[2];
      a[0] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)&st[g2_at(wt + r, kq)]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i + 1 < 8)
          a[(i + 1) & 1] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)&st[g2_at(wt + 16 * (i + 1) + r, kq)]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i & 1], b[j], acc[i][j], 0, 0, 0);
      }
    }
  };
  auto step = [&](uint16_t* __restrict__ nxt, const uint16_t* __restrict__ cur, int x, bool live,
                  f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
    issue(nxt, x);
    if (live) compute(cur, acc);
  };
  // Zeroes the step's masked features (bit f of word w: feature 32 w + f).
  auto zero_features = [&](uint16_t* st, const uint32_t (&word)[G2_WORDS]) __attribute__((always_inline)) {
    const int fc = threadIdx.x % G2_K;
    if ((word[fc >> 5] >> (fc & 31)) & 1u)
      for (int r = threadIdx.x / G2_K; r < G2_ROWS; r += 512 / G2_K) st[g2_at(r, fc >> 3) + (fc & 7)] = 0;
  };
  auto phase = [&](int lo, int hi, int live, const uint32_t* mask, int mwords, f32x4_t(&acc)[8][4])
      __attribute__((always_inline)) {
    for (int g0 = lo; g0 < hi; g0 += G2_RING) {
#pragma unroll
      for (int k = 0; k < G2_RING; ++k) {
        const int g = g0 + k;
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((G2_RING - 2) * G2_LOADS));
        __asm__ volatile("s_barrier" ::: "memory");
        if (fix && mask != nullptr && g - lo < live) {
          uint32_t word[G2_WORDS];
          uint32_t any = 0u;
#pragma unroll
          for (int w = 0; w < G2_WORDS; ++w) {
            const int wi = G2_WORDS * (g - lo) + w;
            word[w] = wi < mwords ? mask[wi] : 0u;
            any |= word[w];
          }
          if (any != 0u) {
            zero_features(stage(k), word);
            __syncthreads();
          }
        }
        step(stage((k + G2_RING - 1) % G2_RING), stage(k), g + G2_RING - 1, g - lo < live, acc);
      }
    }
  };
#pragma unroll
  for (int x = 0; x < G2_RING - 1; ++x) issue(stage(x), x);
  phase(0, px, nx, xm, xw, acc);
  // P leaves in register order; lane l of wave w holds block (i, j) at
  // ((w * 8 + i) * 4 + j) * 64 + l (16 bytes each).
  f32x4_t ODP_GLOBAL* sp = (f32x4_t ODP_GLOBAL*)(ODP_GLOBAL void*)scr + wave * 8 * 4 * 64 + lane;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sp[(i * 4 + j) * 64] = acc[i][j];
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  __asm__ volatile("" ::: "memory");  // P is read back from memory, not kept live
  phase(px, total, ng, gm, gw, acc);
  __builtin_amdgcn_s_waitcnt(0);  // no load into LDS may outlive the workgroup

  // P comes back four pieces at a time (the fence keeps the compiler from
  // issuing all 32 loads while the 128 accumulator registers are live).
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f32x4_t pv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pv[j] = sp[(i * 4 + j) * 64];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += (double)pv[j][e] * (double)acc[i][j][e];
    __asm__ volatile("" ::: "memory");
  }
  if (!diag) s *= 2.0;  // the (s, t) pair is not computed
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < 8; ++w) t += red[w];
    *dst = t;
  }
}

// ---------------------------------------------------------------------------
// Prescale for the clipped sum: X'[t] = c_i x_t (fp32 product rounded to
// bf16, as the clipped sum would form it in registers) for the rows t of
// example i's segments, 0 for rows in no segment.  With X' the clipped sum
// is a plain GEMM; the in-register scaling costs it more than this pass.
// Workgroup = PS_ROWS rows of one problem; rows are found in the sorted
// segment list by binary search.
// ---------------------------------------------------------------------------
constexpr int PS_ROWS = 16;

__global__ __launch_bounds__(256) void k_lin_prescale(const int64_t* __restrict__ probs,
                                                      const int32_t* __restrict__ ws, int n_prob,
                                                      const int32_t* __restrict__ sstart,
                                                      const int32_t* __restrict__ slen,
                                                      const int32_t* __restrict__ sex,
                                                      const double* __restrict__ scales, int n_ex,
                                                      int n_groups) {
  __shared__ float rowc[PS_ROWS];
  __shared__ int rowin[PS_ROWS];
  __shared__ int rowseg[PS_ROWS];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const uint16_t* X = (const uint16_t*)f[ODP_LN_X];
  const int64_t ldx = f[ODP_LN_LDX], d = f[ODP_LN_DIN], n_rows = f[ODP_LN_NROWS];
  uint16_t* out = (uint16_t*)f[ODP_LN_OUT];
  const uint32_t* xm = (const uint32_t*)f[ODP_LN_XMASK];
  const int64_t xw = (d + 31) / 32;
  const int seg_first = (int)f[ODP_LN_SEG_FIRST], n_seg = (int)f[ODP_LN_NSEG];
  const int64_t flags = f[ODP_LN_FLAGS];
  const int grp = (int)((flags >> 8) & 0xffff), cls = (int)((flags >> 24) & 0xffff);
  const double* sc = scales + ((int64_t)cls * n_groups + grp) * n_ex;
  const int64_t row0 = (int64_t)(bid - ws[p]) * PS_ROWS;
  const int tid = threadIdx.x;
  if (tid < PS_ROWS) {
    const int64_t t = row0 + tid;
    // Last segment starting at or before t.
    int lo = 0, hi = n_seg;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sstart[seg_first + mid] <= t)
        lo = mid + 1;
      else
        hi = mid;
    }
    const int s = lo - 1;
    const bool in = t < n_rows && s >= 0 && t < (int64_t)sstart[seg_first + s] + slen[seg_first + s];
    const float c = in ? (float)sc[sex[seg_first + s]] : 0.f;  // exact: a bf16 class scale
    // A zero factor writes zeros (by select: 0 * Inf would be NaN).
    rowin[tid] = in && c != 0.f ? 1 : 0;
    rowc[tid] = c;
    rowseg[tid] = in ? s : 0;
  }
  __syncthreads();
  const int64_t pieces = d / 8;
  for (int64_t i = tid; i < PS_ROWS * pieces; i += 256) {
    const int r = (int)(i / pieces);
    const int64_t pc = i - (int64_t)r * pieces, t = row0 + r;
    if (t >= n_rows) break;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (rowin[r]) {
      v = scale_bf16x8(*(const ODP_GLOBAL u32x4_t*)(const ODP_GLOBAL void*)(X + t * ldx + 8 * pc), rowc[r]);
      if (xm != nullptr) {
        // Columns holding a non-finite value in this segment become 0.
        const uint32_t bits = (xm[rowseg[r] * xw + (8 * pc >> 5)] >> (8 * pc & 31)) & 0xffu;
        if (bits != 0u) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t m = (((bits >> (2 * k)) & 1u) ? 0x0000ffffu : 0u) |
                               (((bits >> (2 * k + 1)) & 1u) ? 0xffff0000u : 0u);
            v[k] &= ~m;
          }
        }
      }
    }
    odp_gstore((u32x4_t*)(out + t * d + 8 * pc), v);
  }
}

// ---------------------------------------------------------------------------
// Clipped sum.  Workgroup = (o-tile, n-tile) of one weight; the contraction
// runs over every segment's rows in order, and a pipeline step never spans
// two segments.  The X fragments of a step are multiplied by their
// example's clip factor (in fp32, rounded back to bf16) after the LDS read,
// so one accumulator holds sum_i c_i M_i.
// ---------------------------------------------------------------------------
template <bool PRESCALED>
__global__ __launch_bounds__(OUTER_THREADS, ODP_LIN_OCC) void k_lin_clip_sum(const int64_t* __restrict__ probs,
                                                      const int32_t* __restrict__ ws, int n_prob,
                                                      const int32_t* __restrict__ sstart,
                                                      const int32_t* __restrict__ slen,
                                                      const int32_t* __restrict__ sex,
                                                      const double* __restrict__ scales, int n_ex,
                                                      int n_groups, float normalize_by) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  void* out = (void*)f[ODP_LN_OUT];
  const int64_t flags = f[ODP_LN_FLAGS];
  const int odt = (int)(flags & 0xff);
  const int grp = (int)((flags >> 8) & 0xffff);
  const int cls = (int)((flags >> 24) & 0xffff);
  const double* sc = scales + ((int64_t)cls * n_groups + grp) * n_ex;
  const int tn_count = (int)((P.d_in + ON - 1) / ON);
  const int tm_count = (int)((P.d_out + OM - 1) / OM);
  const int tile = bid - ws[p];
  if (tile >= tm_count * tn_count) return;  // padding block
  // A problem with a segment at risk of float32 overflow is written by the
  // guarded moments kernel instead.
  if (lin_problem_at_risk(f, slen, P.seg_first, P.n_seg, P.d_in, P.d_out)) return;
  const int64_t o0 = (int64_t)(tile / tn_count) * OM, n0 = (int64_t)(tile % tn_count) * ON;

  OuterAcc acc;
  zero_acc(acc);

  // Steps walk every live segment in order, OK rows at a time.
  // Segment bounds through the scalar (constant) path: uniform loads that
  // must not wait behind the vector loads in flight.
  const ODP_CONST int32_t* cstart = (const ODP_CONST int32_t*)(sstart + P.seg_first);
  const ODP_CONST int32_t* clen = (const ODP_CONST int32_t*)(slen + P.seg_first);
  // Column masks of non-finite inputs (odp_nonfinite_columns), if any.
  const int xw = (int)((P.d_in + 31) / 32), gw = (int)((P.d_out + 31) / 32);
  const ODP_CONST uint32_t* xm = (const ODP_CONST uint32_t*)f[ODP_LN_XMASK];
  const ODP_CONST uint32_t* gm = (const ODP_CONST uint32_t*)f[ODP_LN_GMASK];
  // Whether segment sg masks a column of this tile.
  auto tile_masked = [&](int sg) -> int32_t {
    uint32_t any = 0u;
    if (xm != nullptr) {
      const int w0 = (int)(n0 >> 5);
#pragma unroll
      for (int w = 0; w < ON / 32; ++w)
        if (w0 + w < xw) any |= xm[(int64_t)sg * xw + w0 + w];
    }
    if (gm != nullptr) {
      const int w0 = (int)(o0 >> 5);
#pragma unroll
      for (int w = 0; w < OM / 32; ++w)
        if (w0 + w < gw) any |= gm[(int64_t)sg * gw + w0 + w];
    }
    return any != 0u ? 1 : 0;
  };
  auto at_segment = [&](int sg) {
    while (sg < P.n_seg && clen[sg] <= 0) ++sg;
    Step st;
    st.seg = sg;
    st.live = sg < P.n_seg ? 1 : 0;
    st.tb = st.live ? cstart[sg] : 0;
    st.te = st.live ? st.tb + clen[sg] : 0;
    st.t0 = st.tb;
    st.fix = st.live && (xm != nullptr || gm != nullptr) ? tile_masked(sg) : 0;
    return st;
  };
  // Zeroes the masked G columns (tile rows o) and X columns (tile columns n)
  // of a landed stage, so that the step adds nothing to those entries.
  auto fixup = [&](uint16_t* st, const Step& s) {
    const int c = threadIdx.x & 255;
    const int64_t o = o0 + c, n = n0 + c;
    if (gm != nullptr && o < P.d_out && mask_bit((const uint32_t*)(gm + (int64_t)s.seg * gw), o))
      for (int r = threadIdx.x >> 8; r < OK; r += OUTER_THREADS / 256) st[tile_at(r, c, OM)] = 0;
    if (xm != nullptr && c < ON && n < P.d_in && mask_bit((const uint32_t*)(xm + (int64_t)s.seg * xw), n))
      for (int r = threadIdx.x >> 8; r < OK; r += OUTER_THREADS / 256) st[A_TILE + tile_at(r, c, ON)] = 0;
  };
  // Also valid on a finished step (which stays finished).
  auto next = [&](const Step& st) {
    if (st.t0 + OK < st.te) {
      Step n = st;
      n.t0 = st.t0 + OK;
      return n;
    }
    return at_segment(st.seg + 1 < P.n_seg ? st.seg + 1 : P.n_seg);
  };
  const ODP_CONST int32_t* cex = (const ODP_CONST int32_t*)(sex + P.seg_first);
  const ODP_CONST double* csc = (const ODP_CONST double*)sc;
  auto scale = [&](const Step& st) { return (float)csc[cex[st.seg]]; };
  // PRESCALED: X already holds c_i x_t (odp_linear_prescale).
  dma_mainloop<!PRESCALED, true, true>(P, o0, n0, at_segment(0), next, scale, fixup, acc);

  // Lane holds D[4 (lane >> 4) + e][lane & 15] of each 16 x 16 block.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = WM * (wave & 1), wn = WN * (wave >> 1);
  static_for<BI * BJ>([&](auto q) {
    constexpr int i = decltype(q)::value / BJ, j = decltype(q)::value % BJ;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t o = o0 + wm + 16 * i + 4 * (lane >> 4) + e;
      const int64_t n = n0 + wn + 16 * j + (lane & 15);
      if (o < P.d_out && n < P.d_in) {
        float x = odp_round_to(acc[i][j][e], odt);
        if (normalize_by != 1.0f) x = odp_round_to(__fdiv_rn(x, normalize_by), odt);
        odp_store_from_float(out, o * P.d_in + n, odt, x);
      }
    }
    // One tile's accumulators at a time in VGPRs.
    __builtin_amdgcn_sched_barrier(0);
  });
}

// ---------------------------------------------------------------------------
// Column masks of non-finite values per segment.  Workgroup = (segment,
// strip of 256 columns): 32 lanes cover a strip row in 16-byte pieces, 8 row
// groups walk the segment's rows, and the per-lane 8-bit masks are OR-ed
// over the row groups and packed into the strip's 8 words.  HBM-bound: one
// read of the segment's rows.
// ---------------------------------------------------------------------------
constexpr int NF_THREADS = 256;
constexpr int NF_STRIP = 256;  // columns per workgroup

// Bit k set when bf16 element k of the 8 is NaN or Inf (exponent all ones).
__device__ __forceinline__ uint32_t nonfinite8(u32x4_t v) {
  uint32_t b = 0u;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    b |= ((v[k] & 0x00007f80u) == 0x00007f80u ? 1u : 0u) << (2 * k);
    b |= ((v[k] & 0x7f800000u) == 0x7f800000u ? 1u : 0u) << (2 * k + 1);
  }
  return b;
}

// Largest magnitude among the finite bf16 elements of the 8, as bf16 bits.
__device__ __forceinline__ uint32_t finite_amax8(u32x4_t v) {
  uint32_t m = 0u;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = v[k] & 0xffffu, hi = v[k] >> 16;
    if ((lo & 0x7f80u) != 0x7f80u) m = max(m, lo & 0x7fffu);
    if ((hi & 0x7f80u) != 0x7f80u) m = max(m, hi & 0x7fffu);
  }
  return m;
}

__global__ __launch_bounds__(NF_THREADS) void k_nonfinite_cols(const int64_t* __restrict__ probs,
                                                               const int32_t* __restrict__ ws, int n_prob,
                                                               const int32_t* __restrict__ sstart,
                                                               const int32_t* __restrict__ slen) {
  __shared__ uint32_t red[NF_THREADS / 32][32];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_NF_FIELDS;
  const uint16_t* P = (const uint16_t*)f[ODP_NF_P];
  const int64_t ldp = f[ODP_NF_LDP], d = f[ODP_NF_D];
  const int seg_first = (int)f[ODP_NF_SEG_FIRST];
  uint32_t* mask = (uint32_t*)f[ODP_NF_MASK];
  const int strips = (int)((d + NF_STRIP - 1) / NF_STRIP);
  const int64_t words = (d + 31) / 32;
  const int local = bid - ws[p];
  const int seg = local / strips, strip = local - seg * strips;
  const int64_t t0 = sstart[seg_first + seg];
  const int len = slen[seg_first + seg];
  const int lane = threadIdx.x & 31, rg = threadIdx.x >> 5;
  const int64_t col = (int64_t)strip * NF_STRIP + 8 * lane;
  uint32_t* amax = (uint32_t*)f[ODP_NF_AMAX];
  uint32_t bits = 0u, am = 0u;
  if (col < d) {
    const uint16_t* base = P + t0 * ldp + col;
    auto row = [&](int r) { return *(const ODP_GLOBAL u32x4_t*)(const ODP_GLOBAL void*)(base + (int64_t)r * ldp); };
    int r = rg;
    // Four rows in flight per lane.
    if (amax != nullptr) {
      for (; r + 24 < len; r += 32) {
        const u32x4_t a = row(r), b = row(r + 8), c = row(r + 16), e = row(r + 24);
        bits |= nonfinite8(a) | nonfinite8(b) | nonfinite8(c) | nonfinite8(e);
        am = max(max(am, max(finite_amax8(a), finite_amax8(b))), max(finite_amax8(c), finite_amax8(e)));
      }
      for (; r < len; r += 8) {
        const u32x4_t a = row(r);
        bits |= nonfinite8(a);
        am = max(am, finite_amax8(a));
      }
    } else {
      for (; r + 24 < len; r += 32) {
        const u32x4_t a = row(r), b = row(r + 8), c = row(r + 16), e = row(r + 24);
        bits |= nonfinite8(a) | nonfinite8(b) | nonfinite8(c) | nonfinite8(e);
      }
      for (; r < len; r += 8) bits |= nonfinite8(row(r));
    }
  }
  if (amax != nullptr) {
    // The workgroup's largest finite magnitude, as float bits (monotonic
    // for non-negative values), raised into the segment's word.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) am = max(am, (uint32_t)__shfl_xor((int)am, off));
    if ((threadIdx.x & 63) == 0 && am != 0u) atomicMax(amax + seg, am << 16);
  }
  red[rg][lane] = bits;
  __syncthreads();
  if (threadIdx.x < 32) {
    uint32_t b = 0u;
#pragma unroll
    for (int k = 0; k < NF_THREADS / 32; ++k) b |= red[k][lane];
    // Lanes 4w .. 4w + 3 hold the four bytes of the strip's word w.
    uint32_t w = b << (8 * (lane & 3));
    w |= __shfl_xor(w, 1, 32);
    w |= __shfl_xor(w, 2, 32);
    const int64_t wi = (int64_t)strip * (NF_STRIP / 32) + (lane >> 2);
    if ((lane & 3) == 0 && wi < words) odp_gstore(mask + (int64_t)seg * words + wi, w);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" int64_t odp_nonfinite_blocks(int64_t d, int64_t n_seg) {
  if (d <= 0 || n_seg <= 0) return 0;
  return n_seg * ((d + NF_STRIP - 1) / NF_STRIP);
}

extern "C" int odp_nonfinite_columns(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                                     int32_t n_prob, int32_t total_blocks, const int32_t* seg_row_start,
                                     const int32_t* seg_row_len) {
  int rc = odp_check_table("odp_nonfinite_columns", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr) {
    odp_set_error("odp_nonfinite_columns: null segment arrays");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_nonfinite_cols, dim3(total_blocks), dim3(NF_THREADS), 0, odp_hip_stream(stream),
                     problems, work_start, n_prob, seg_row_start, seg_row_len);
  return odp_check_launch("odp_nonfinite_columns");
}

extern "C" int64_t odp_linear_tiles(int form, int64_t d_in, int64_t d_out, int64_t max_seg_len) {
  if (d_in <= 0 || d_out <= 0) return 0;
  // ODP_FORM_OUTER_GUARDED: the outer tiles.
  if (form == ODP_FORM_GRAM) {
    const int64_t nb = max_seg_len > 0 ? (max_seg_len + LT - 1) / LT : 0;
    return gram_items(nb);
  }
  if (form == ODP_FORM_GRAM256) {
    const int64_t nb = max_seg_len > 0 ? (max_seg_len + G2_B - 1) / G2_B : 0;
    return gram2_items(nb);
  }
  return ((d_out + OM - 1) / OM) * ((d_in + ON - 1) / ON);
}

extern "C" int64_t odp_linear_norm_blocks(int form, int64_t d_in, int64_t d_out, int64_t max_seg_len,
                                          int64_t n_seg) {
  const int64_t per = odp_linear_tiles(form, d_in, d_out, max_seg_len);
  if (per <= 0 || n_seg <= 0) return 0;
  if (form == ODP_FORM_OUTER_GUARDED) return n_seg * GUARD_SPLIT;
  if ((form == ODP_FORM_GRAM || form == ODP_FORM_GRAM256) && n_seg >= 8) return 8 * ((n_seg + 7) / 8) * per;
  return (n_seg * per + 7) / 8 * 8;
}

extern "C" int64_t odp_linear_sum_blocks(int64_t d_in, int64_t d_out) {
  if (d_in <= 0 || d_out <= 0) return 0;
  const int64_t tiles = ((d_out + OM - 1) / OM) * ((d_in + ON - 1) / ON);
  return (tiles + 7) / 8 * 8;
}

extern "C" int odp_linear_sqnorm(odp_stream_t stream, int form, const int64_t* problems,
                                 const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                                 const int32_t* seg_row_start, const int32_t* seg_row_len,
                                 const int32_t* seg_example, double* part, int64_t part_stride) {
  int rc = odp_check_table("odp_linear_sqnorm", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (form != ODP_FORM_OUTER && form != ODP_FORM_GRAM && form != ODP_FORM_GRAM256 &&
      form != ODP_FORM_OUTER_GUARDED) {
    odp_set_error("odp_linear_sqnorm: unknown form %d", form);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr ||
      part == nullptr || part_stride <= 0) {
    odp_set_error("odp_linear_sqnorm: null segment/partial arrays or part_stride <= 0");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = odp_hip_stream(stream);
  const dim3 grid(total_blocks), block(OUTER_THREADS);
  if (form == ODP_FORM_GRAM)
    hipLaunchKernelGGL(k_lin_gram_norm, grid, dim3(512), 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len, seg_example, part, part_stride);
  else if (form == ODP_FORM_GRAM256)
    hipLaunchKernelGGL(k_lin_gram2_norm, grid, dim3(512), 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len, seg_example, part, part_stride);
  else if (form == ODP_FORM_OUTER_GUARDED)
    hipLaunchKernelGGL(k_lin_outer_norm_guarded, grid, block, 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len, seg_example, part, part_stride);
  else
    hipLaunchKernelGGL(k_lin_outer_norm, grid, block, 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len, seg_example, part, part_stride);
  return odp_check_launch("odp_linear_sqnorm");
}

extern "C" int64_t odp_linear_prescale_blocks(int64_t n_rows) {
  return n_rows <= 0 ? 0 : (n_rows + PS_ROWS - 1) / PS_ROWS;
}

extern "C" int odp_linear_prescale(odp_stream_t stream, const int64_t* problems,
                                   const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                                   const int32_t* seg_row_start, const int32_t* seg_row_len,
                                   const int32_t* seg_example, const double* scales, int32_t n_ex,
                                   int32_t n_groups) {
  int rc = odp_check_table("odp_linear_prescale", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr ||
      scales == nullptr || n_ex <= 0 || n_groups <= 0) {
    odp_set_error("odp_linear_prescale: null segment/scale arrays or empty batch");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_lin_prescale, dim3(total_blocks), dim3(256), 0, odp_hip_stream(stream), problems,
                     work_start, n_prob, seg_row_start, seg_row_len, seg_example, scales, n_ex, n_groups);
  return odp_check_launch("odp_linear_prescale");
}

extern "C" int odp_linear_clipped_sum(odp_stream_t stream, const int64_t* problems,
                                      const int32_t* work_start, int32_t n_prob,
                                      int32_t total_blocks, const int32_t* seg_row_start,
                                      const int32_t* seg_row_len, const int32_t* seg_example,
                                      const double* scales, int32_t n_ex, int32_t n_groups,
                                      float normalize_by, int32_t prescaled) {
  int rc = odp_check_table("odp_linear_clipped_sum", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (!(normalize_by > 0.0f)) {
    odp_set_error("odp_linear_clipped_sum: normalize_by must be > 0, got %g", (double)normalize_by);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr ||
      scales == nullptr || n_ex <= 0 || n_groups <= 0) {
    odp_set_error("odp_linear_clipped_sum: null segment/scale arrays or empty batch");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = odp_hip_stream(stream);
  hipLaunchKernelGGL(prescaled ? k_lin_clip_sum<true> : k_lin_clip_sum<false>, dim3(total_blocks), dim3(OUTER_THREADS), 0, s, problems, work_start,
                     n_prob, seg_row_start, seg_row_len, seg_example, scales, n_ex, n_groups,
                     normalize_by);
  return odp_check_launch("odp_linear_clipped_sum");
}
