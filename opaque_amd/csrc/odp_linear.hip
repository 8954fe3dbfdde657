// Full-weight linear layers: per-example gradient norms and the clipped sum
// on CDNA4 MFMA, without materialising per-example gradients.
//
// For y = x W^T the per-example weight gradient is M_i = G_i^T X_i
// (d_out x d_in) over the example's rows.  The reference materialises every
// M_i under vmap(grad) (opaque-engine/.../clipping/_clipped_fun.py:756-762)
// and then squares, scales and sums them.  Here:
//
//   k_lin_outer_norm : ||M_i||_F^2 tile by tile (128 x 128 output tiles,
//                      contraction over the example's tokens), squares
//                      summed in fp64 into one partial slot per tile;
//   k_lin_gram_norm  : sum_{t,s} (x_t . x_s)(g_t . g_s) over 128 x 128 token
//                      tiles of the upper triangle (off-diagonal tiles
//                      counted twice), the cheaper form when the example is
//                      short relative to the weight;
//   k_lin_clip_sum   : out = sum_i c_i M_i as one GEMM over all rows,
//                      accumulating each example in its own fp32 registers
//                      and folding it in with its clip factor (non-finite
//                      entries dropped, as nan_to_num does in the reference).
//
// All three are bf16 MFMA (16x16x32, fp32 accumulate) on 128 x 128
// workgroup tiles with 4 waves of 64 x 64, operands staged through LDS with
// one pipeline step of global loads in flight.  Rows are token-major in HBM,
// so the outer-product forms read their operands K-major and take them from
// LDS with the gfx950 transposing read; the Gram form's operands are
// K-contiguous rows.
#include "odp_internal.h"

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short v4i16_t __attribute__((ext_vector_type(4)));

namespace {

constexpr int LT = 128;      // output tile edge (rows and columns)
constexpr int LK = 64;       // tokens (outer forms) or features (Gram) per pipeline step
constexpr int OP = LT + 8;   // LDS pitch of a [LK][LT] token-major tile (elements)
constexpr int GP = LK + 8;   // LDS pitch of a [LT][LK] feature-major tile (elements)

#define ODP_GLOBAL __attribute__((address_space(1)))
#define ODP_LDS __attribute__((address_space(3)))
__device__ __forceinline__ u32x4_t ldg16(const uint16_t* p) {
  return *(const ODP_GLOBAL u32x4_t*)(const ODP_GLOBAL void*)p;
}
__device__ __forceinline__ v4i16_t lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((ODP_LDS v4i16_t*)(ODP_LDS void*)p);
}

struct LinProblem {
  const uint16_t* X;
  const uint16_t* G;
  int64_t ldx, ldg, d_in, d_out;
  int seg_first, n_seg;
};

__device__ __forceinline__ LinProblem read_problem(const int64_t* f) {
  LinProblem P;
  P.X = (const uint16_t*)f[ODP_LN_X];
  P.ldx = f[ODP_LN_LDX];
  P.G = (const uint16_t*)f[ODP_LN_G];
  P.ldg = f[ODP_LN_LDG];
  P.d_in = f[ODP_LN_DIN];
  P.d_out = f[ODP_LN_DOUT];
  P.seg_first = (int)f[ODP_LN_SEG_FIRST];
  P.n_seg = (int)f[ODP_LN_NSEG];
  return P;
}

// ---------------------------------------------------------------------------
// Outer-product main loop.  acc[i][j] (wave tile 64 x 64 as 4 x 4 MFMA
// blocks) += sum over tokens t in [t_begin, t_end) of G[t][o] X[t][n] for
// o in [o0, o0 + 128), n in [n0, n0 + 128).  Each step stages 64 tokens of
// both operands as token-major [64][128] LDS tiles; token rows outside the
// range and columns past the matrix are zeroed at the LDS store.
// ---------------------------------------------------------------------------
struct OuterStage {
  u32x4_t a[4];  // G pieces
  u32x4_t b[4];  // X pieces
};

__device__ __forceinline__ void outer_load(const LinProblem& P, int64_t o0, int64_t n0, int64_t t0,
                                           int64_t t_begin, int64_t t_end, OuterStage& S) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int id = tid + 256 * q;          // 1024 pieces: 64 rows x 16 pieces of 8
    int64_t t = t0 + (id >> 4);
    t = t < t_begin ? t_begin : (t >= t_end ? t_end - 1 : t);
    const int64_t c = 8 * (id & 15);
    const int64_t co = o0 + c, cn = n0 + c;
    S.a[q] = ldg16(P.G + t * P.ldg + (co < P.d_out ? co : P.d_out - 8));
    S.b[q] = ldg16(P.X + t * P.ldx + (cn < P.d_in ? cn : P.d_in - 8));
  }
}

__device__ __forceinline__ void outer_store(const LinProblem& P, int64_t o0, int64_t n0, int64_t t0,
                                            int64_t t_begin, int64_t t_end, const OuterStage& S,
                                            uint16_t* ta, uint16_t* tb) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int id = tid + 256 * q;
    const int row = id >> 4, c = 8 * (id & 15);
    const int64_t t = t0 + row;
    const bool tok = t >= t_begin && t < t_end;
    const u32x4_t z = {0u, 0u, 0u, 0u};
    *(u32x4_t*)&ta[row * OP + c] = (tok && o0 + c < P.d_out) ? S.a[q] : z;
    *(u32x4_t*)&tb[row * OP + c] = (tok && n0 + c < P.d_in) ? S.b[q] : z;
  }
}

// 16 columns col0.. of a token-major tile, tokens 32u + 8 (lane >> 4) + 0..7:
// the MFMA operand layout (lane & 15 = row of A / column of B).
__device__ __forceinline__ bf16x8_t outer_frag(const uint16_t* tile, int u, int col0) {
  const int lane = threadIdx.x & 63, c = lane & 15;
  const uint16_t* src = tile + (32 * u + 8 * (lane >> 4) + (c >> 2)) * OP + col0 + 4 * (c & 3);
  const v4i16_t t0 = lds_tr16(src), t1 = lds_tr16(src + 4 * OP);
  const v4i16_t tt[2] = {t0, t1};
  return __builtin_bit_cast(bf16x8_t, tt);
}

__device__ __forceinline__ void outer_compute(const uint16_t* ta, const uint16_t* tb,
                                              f32x4_t (&acc)[4][4]) {
  const int wave = threadIdx.x >> 6;
  const int wm = 64 * (wave & 1), wn = 64 * (wave >> 1);
#pragma unroll
  for (int u = 0; u < LK / 32; ++u) {
    bf16x8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = outer_frag(ta, u, wm + 16 * i);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = outer_frag(tb, u, wn + 16 * j);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// LDS: two stages of (G tile, X tile), each [LK][OP] bf16.
constexpr int OUTER_TILE = LK * OP;
constexpr int OUTER_LDS = 2 * 2 * OUTER_TILE;

__device__ __forceinline__ void zero_acc(f32x4_t (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
}

// Block-wide fp64 sum; the result is valid in thread 0.
__device__ __forceinline__ double block_sum(double v, double* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0) t = (red[0] + red[1]) + (red[2] + red[3]);
  return t;
}

// fp32 squares of the finite entries, summed in fp64.
__device__ __forceinline__ double acc_sq(const f32x4_t (&acc)[4][4]) {
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = acc[i][j][e];
        const float vf = isfinite(v) ? v : 0.f;
        s += (double)__fmul_rn(vf, vf);
      }
  return s;
}

// ---------------------------------------------------------------------------
// ||M_i||^2 partials, outer form.  Workgroup = (segment, o-tile, n-tile).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_lin_outer_norm(const int64_t* __restrict__ probs,
                                                        const int32_t* __restrict__ ws, int n_prob,
                                                        const int32_t* __restrict__ sstart,
                                                        const int32_t* __restrict__ slen,
                                                        const int32_t* __restrict__ sex,
                                                        double* __restrict__ part, int64_t part_stride) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[OUTER_LDS];
  __shared__ double red[4];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  const int64_t slot = f[ODP_LN_SLOT];
  const int tn_count = (int)((P.d_in + LT - 1) / LT);
  const int tm_count = (int)((P.d_out + LT - 1) / LT);
  const int tiles = tn_count * tm_count;
  const int local = bid - ws[p];
  const int seg = local / tiles, tile = local % tiles;
  const int64_t o0 = (int64_t)(tile / tn_count) * LT, n0 = (int64_t)(tile % tn_count) * LT;
  const int gs = P.seg_first + seg;
  const int64_t t_begin = sstart[gs], t_end = t_begin + slen[gs];
  const int ex = sex[gs];

  f32x4_t acc[4][4];
  zero_acc(acc);
  const int64_t nsteps = t_end > t_begin ? (t_end - t_begin + LK - 1) / LK : 0;
  OuterStage S;
  if (nsteps > 0) {
    outer_load(P, o0, n0, t_begin, t_begin, t_end, S);
    outer_store(P, o0, n0, t_begin, t_begin, t_end, S, lds, lds + OUTER_TILE);
  }
  __syncthreads();
  for (int64_t s = 0; s < nsteps; ++s) {
    const int b = (int)(s & 1);
    const bool more = s + 1 < nsteps;
    const int64_t tn = t_begin + (s + 1) * LK;
    if (more) outer_load(P, o0, n0, tn, t_begin, t_end, S);
    outer_compute(lds + b * 2 * OUTER_TILE, lds + b * 2 * OUTER_TILE + OUTER_TILE, acc);
    if (more) outer_store(P, o0, n0, tn, t_begin, t_end, S, lds + (b ^ 1) * 2 * OUTER_TILE,
                          lds + (b ^ 1) * 2 * OUTER_TILE + OUTER_TILE);
    __syncthreads();
  }
  // Columns/rows past the matrix were zero operands, so they add nothing.
  const double tot = block_sum(acc_sq(acc), red);
  if (threadIdx.x == 0) part[(int64_t)ex * part_stride + slot + tile] = tot;
}

// ---------------------------------------------------------------------------
// ||M_i||^2 partials, Gram form.  Workgroup = (segment, token-tile pair
// tb <= sb).  Sx = X_tb X_sb^T over d_in and Sg = G_tb G_sb^T over d_out
// (operands are K-contiguous rows), then sum Sx * Sg.
// ---------------------------------------------------------------------------
constexpr int GRAM_TILE = LT * GP;          // [128 rows][LK + 8]
constexpr int GRAM_LDS = 2 * 2 * GRAM_TILE;  // two stages x (t rows, s rows)

struct GramStage {
  u32x4_t a[4];
  u32x4_t b[4];
};

__device__ __forceinline__ void gram_load(const uint16_t* M, int64_t ld, int64_t d, int64_t ta0,
                                          int64_t sb0, int64_t t_end, int64_t k0, GramStage& S) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int id = tid + 256 * q;  // 1024 pieces: 128 rows x 8 pieces of 8
    const int row = id >> 3;
    const int64_t k = k0 + 8 * (id & 7);
    const int64_t kc = k < d ? k : d - 8;
    int64_t ra = ta0 + row, rb = sb0 + row;
    ra = ra < t_end ? ra : t_end - 1;
    rb = rb < t_end ? rb : t_end - 1;
    S.a[q] = ldg16(M + ra * ld + kc);
    S.b[q] = ldg16(M + rb * ld + kc);
  }
}

__device__ __forceinline__ void gram_store(int64_t d, int64_t ta0, int64_t sb0, int64_t t_end,
                                           int64_t k0, const GramStage& S, uint16_t* la,
                                           uint16_t* lb) {
  const int tid = threadIdx.x;
  const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int id = tid + 256 * q;
    const int row = id >> 3, c = 8 * (id & 7);
    const bool kin = k0 + c < d;
    *(u32x4_t*)&la[row * GP + c] = (kin && ta0 + row < t_end) ? S.a[q] : z;
    *(u32x4_t*)&lb[row * GP + c] = (kin && sb0 + row < t_end) ? S.b[q] : z;
  }
}

__device__ __forceinline__ void gram_compute(const uint16_t* la, const uint16_t* lb,
                                             f32x4_t (&acc)[4][4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = 64 * (wave & 1), wn = 64 * (wave >> 1);
  const int r = lane & 15, kq = 8 * (lane >> 4);
#pragma unroll
  for (int u = 0; u < LK / 32; ++u) {
    bf16x8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)&la[(wm + 16 * i + r) * GP + 32 * u + kq]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b[j] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)&lb[(wn + 16 * j + r) * GP + 32 * u + kq]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// acc += (rows ta0.. of M)(rows sb0.. of M)^T over the d features of M.
__device__ __forceinline__ void gram_pass(const uint16_t* M, int64_t ld, int64_t d, int64_t ta0,
                                          int64_t sb0, int64_t t_end, uint16_t* lds,
                                          f32x4_t (&acc)[4][4]) {
  const int64_t nsteps = (d + LK - 1) / LK;
  GramStage S;
  gram_load(M, ld, d, ta0, sb0, t_end, 0, S);
  gram_store(d, ta0, sb0, t_end, 0, S, lds, lds + GRAM_TILE);
  __syncthreads();
  for (int64_t s = 0; s < nsteps; ++s) {
    const int b = (int)(s & 1);
    const bool more = s + 1 < nsteps;
    const int64_t k1 = (s + 1) * LK;
    if (more) gram_load(M, ld, d, ta0, sb0, t_end, k1, S);
    gram_compute(lds + b * 2 * GRAM_TILE, lds + b * 2 * GRAM_TILE + GRAM_TILE, acc);
    if (more) gram_store(d, ta0, sb0, t_end, k1, S, lds + (b ^ 1) * 2 * GRAM_TILE,
                         lds + (b ^ 1) * 2 * GRAM_TILE + GRAM_TILE);
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void k_lin_gram_norm(const int64_t* __restrict__ probs,
                                                       const int32_t* __restrict__ ws, int n_prob,
                                                       const int32_t* __restrict__ sstart,
                                                       const int32_t* __restrict__ slen,
                                                       const int32_t* __restrict__ sex,
                                                       double* __restrict__ part, int64_t part_stride) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[GRAM_LDS];
  __shared__ double red[4];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  const int64_t slot = f[ODP_LN_SLOT];
  const int nb = (int)f[ODP_LN_NB];
  const int pairs = nb * (nb + 1) / 2;
  const int local = bid - ws[p];
  const int seg = local / pairs, pair = local % pairs;
  // pair -> (tb, sb), tb <= sb, row-major over the upper triangle.
  int tb = 0, rem = pair;
  while (rem >= nb - tb) {
    rem -= nb - tb;
    ++tb;
  }
  const int sb = tb + rem;
  const int gs = P.seg_first + seg;
  const int64_t t_begin = sstart[gs], t_end = t_begin + slen[gs];
  const int ex = sex[gs];
  const int64_t ta0 = t_begin + (int64_t)tb * LT, sb0 = t_begin + (int64_t)sb * LT;
  double* dst = part + (int64_t)ex * part_stride + slot + pair;
  if (sb0 >= t_end) {  // tile past this segment's length
    if (threadIdx.x == 0) *dst = 0.0;
    return;
  }
  f32x4_t sx[4][4], sg[4][4];
  zero_acc(sx);
  zero_acc(sg);
  gram_pass(P.X, P.ldx, P.d_in, ta0, sb0, t_end, lds, sx);
  gram_pass(P.G, P.ldg, P.d_out, ta0, sb0, t_end, lds, sg);
  // Rows past the segment were zero operands, so their products vanish.
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += (double)sx[i][j][e] * (double)sg[i][j][e];
  const double tot = block_sum(s, red);
  if (threadIdx.x == 0) *dst = tb == sb ? tot : 2.0 * tot;
}

// ---------------------------------------------------------------------------
// Clipped sum.  Workgroup = (o-tile, n-tile) of one weight; the contraction
// runs over every segment's rows in order.  Each segment accumulates into
// its own registers (M_i exactly as fp32), which are folded in with the
// example's clip factor when the next segment starts.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_lin_clip_sum(const int64_t* __restrict__ probs,
                                                      const int32_t* __restrict__ ws, int n_prob,
                                                      const int32_t* __restrict__ sstart,
                                                      const int32_t* __restrict__ slen,
                                                      const int32_t* __restrict__ sex,
                                                      const float* __restrict__ scales, int n_ex,
                                                      int n_groups, float normalize_by) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[OUTER_LDS];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  void* out = (void*)f[ODP_LN_OUT];
  const int64_t flags = f[ODP_LN_FLAGS];
  const int odt = (int)(flags & 0xff);
  const int grp = (int)((flags >> 8) & 0xffff);
  const int cls = (int)((flags >> 24) & 0xffff);
  const float* sc = scales + ((int64_t)cls * n_groups + grp) * n_ex;
  const int tn_count = (int)((P.d_in + LT - 1) / LT);
  const int tile = bid - ws[p];
  const int64_t o0 = (int64_t)(tile / tn_count) * LT, n0 = (int64_t)(tile % tn_count) * LT;

  f32x4_t acc[4][4], tot[4][4];
  zero_acc(acc);
  zero_acc(tot);

  // Step cursor over (segment, first token) pairs; empty segments are skipped.
  int cs = 0;
  int64_t ct = 0;
  auto seek = [&](int s) {
    while (s < P.n_seg && slen[P.seg_first + s] <= 0) ++s;
    cs = s;
    ct = s < P.n_seg ? (int64_t)sstart[P.seg_first + s] : 0;
  };
  auto seg_end = [&](int s) {
    return (int64_t)sstart[P.seg_first + s] + slen[P.seg_first + s];
  };
  seek(0);
  if (cs >= P.n_seg) {  // no rows at all: the sum is zero
    // fall through with zero accumulators
  }
  OuterStage S;
  int cur_s = cs;
  int64_t cur_t = ct;
  if (cs < P.n_seg) {
    const int64_t tb = sstart[P.seg_first + cs], te = seg_end(cs);
    outer_load(P, o0, n0, ct, tb, te, S);
    outer_store(P, o0, n0, ct, tb, te, S, lds, lds + OUTER_TILE);
  }
  __syncthreads();
  int b = 0;
  while (cur_s < P.n_seg) {
    // Cursor of the following step.
    int nx_s = cur_s;
    int64_t nx_t = cur_t + LK;
    if (nx_t >= seg_end(cur_s)) {
      seek(cur_s + 1);
      nx_s = cs;
      nx_t = ct;
    }
    const bool more = nx_s < P.n_seg;
    int64_t ntb = 0, nte = 0;
    if (more) {
      ntb = sstart[P.seg_first + nx_s];
      nte = seg_end(nx_s);
      outer_load(P, o0, n0, nx_t, ntb, nte, S);
    }
    outer_compute(lds + b * 2 * OUTER_TILE, lds + b * 2 * OUTER_TILE + OUTER_TILE, acc);
    if (nx_s != cur_s) {
      // Segment cur_s is complete: fold it in with its clip factor.
      const float c = sc[sex[P.seg_first + cur_s]];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc[i][j][e];
            tot[i][j][e] = __fadd_rn(tot[i][j][e], __fmul_rn(c, isfinite(v) ? v : 0.f));
          }
      zero_acc(acc);
    }
    if (more) outer_store(P, o0, n0, nx_t, ntb, nte, S, lds + (b ^ 1) * 2 * OUTER_TILE,
                          lds + (b ^ 1) * 2 * OUTER_TILE + OUTER_TILE);
    __syncthreads();
    b ^= 1;
    cur_s = nx_s;
    cur_t = nx_t;
  }

  // Lane holds D[4 (lane >> 4) + e][lane & 15] of each 16 x 16 block.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = 64 * (wave & 1), wn = 64 * (wave >> 1);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t o = o0 + wm + 16 * i + 4 * (lane >> 4) + e;
        const int64_t n = n0 + wn + 16 * j + (lane & 15);
        if (o < P.d_out && n < P.d_in) {
          float x = odp_round_to(tot[i][j][e], odt);
          if (normalize_by != 1.0f) x = odp_round_to(__fdiv_rn(x, normalize_by), odt);
          odp_store_from_float(out, o * P.d_in + n, odt, x);
        }
      }
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" int64_t odp_linear_tiles(int form, int64_t d_in, int64_t d_out, int64_t max_seg_len) {
  if (d_in <= 0 || d_out <= 0) return 0;
  if (form == ODP_FORM_GRAM) {
    const int64_t nb = max_seg_len > 0 ? (max_seg_len + LT - 1) / LT : 0;
    return nb * (nb + 1) / 2;
  }
  return ((d_out + LT - 1) / LT) * ((d_in + LT - 1) / LT);
}

extern "C" int64_t odp_linear_sum_blocks(int64_t d_in, int64_t d_out) {
  if (d_in <= 0 || d_out <= 0) return 0;
  return ((d_out + LT - 1) / LT) * ((d_in + LT - 1) / LT);
}

extern "C" int odp_linear_sqnorm(odp_stream_t stream, int form, const int64_t* problems,
                                 const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                                 const int32_t* seg_row_start, const int32_t* seg_row_len,
                                 const int32_t* seg_example, double* part, int64_t part_stride) {
  int rc = odp_check_table("odp_linear_sqnorm", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (form != ODP_FORM_OUTER && form != ODP_FORM_GRAM) {
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
  const dim3 grid(total_blocks), block(256);
  if (form == ODP_FORM_GRAM)
    hipLaunchKernelGGL(k_lin_gram_norm, grid, block, 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len, seg_example, part, part_stride);
  else
    hipLaunchKernelGGL(k_lin_outer_norm, grid, block, 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len, seg_example, part, part_stride);
  return odp_check_launch("odp_linear_sqnorm");
}

extern "C" int odp_linear_clipped_sum(odp_stream_t stream, const int64_t* problems,
                                      const int32_t* work_start, int32_t n_prob,
                                      int32_t total_blocks, const int32_t* seg_row_start,
                                      const int32_t* seg_row_len, const int32_t* seg_example,
                                      const float* scales, int32_t n_ex, int32_t n_groups,
                                      float normalize_by) {
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
  hipLaunchKernelGGL(k_lin_clip_sum, dim3(total_blocks), dim3(256), 0, s, problems, work_start,
                     n_prob, seg_row_start, seg_row_len, seg_example, scales, n_ex, n_groups,
                     normalize_by);
  return odp_check_launch("odp_linear_clipped_sum");
}
