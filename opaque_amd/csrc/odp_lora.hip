// LoRA per-example factor gradients and their squared norms on CDNA4 MFMA.
//
// A LoRA adapter y = x W^T + s (x A) B has per-example factor gradients
//   dA_i = s X_i^T U_i,  U = G B^T        (d_in x r)
//   dB_i = s V_i^T G_i,  V = X A          (r x d_out)
// (reference: opaque-patches/.../kernels/lora.py:164-176, where they are
// materialised with torch.bmm under vmap).  Both are skinny products whose
// long dimension is a row of X or G, so the work is HBM-bound: each kernel
// streams X or G and keeps the rank-r side (U, V, the r x M output tile) on
// chip.  The bf16 kernels are instantiated per rank block count NKB =
// ceil(r / 16) so that registers match the rank, and keep two pipeline steps
// of loads in flight per wave so that enough bytes are outstanding per CU to
// approach HBM bandwidth.
//
//   k_project_*  : Q^T = (P W^T)^T for every row of a segment      (U, V)
//   k_factor_*   : pe[s] = s * Q_s^T P_s per segment, plus fp64 sums of
//                  squares per leaf and M-tile                   (dA, dB)
#include <type_traits>

#include "odp_internal.h"

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

namespace {

#ifndef ODP_FT_T
#define ODP_FT_T 32  // tokens per bf16 factor step (a multiple of the MFMA K, 32)
#endif
constexpr int PJ_ROWS = 64;   // rows per fp32 project workgroup (4 waves x 16)
// Workgroups per CU the compiler must fit registers for in k_factor_bf16:
// each fits its LDS tiles that many times in 160 KB without spilling, and
// the extra loads in flight measured 1-5 % faster (one rank block: no
// difference, left to the compiler; three rank blocks: two workgroups, the
// registers of a 256-wide tile without spills).
__host__ __device__ constexpr int ft_min_blocks(int nkb) { return nkb == 2 ? 3 : nkb == 3 ? 2 : 1; }
constexpr int FT_T = ODP_FT_T;
constexpr int FT_M_F32 = 128; // M columns per fp32 factor workgroup

// bf16 factor: 16-wide m blocks per wave (M-tile = 64 NJ).  256-wide tiles
// (512-byte contiguous runs of each P row) measured fastest for every rank
// (three rank blocks: 11 % faster than 128-wide tiles at two workgroups per
// CU; 512-wide tiles slower).
#ifndef ODP_FT_NJ
#define ODP_FT_NJ 4
#endif
__host__ __device__ constexpr int ft_nj(int) { return ODP_FT_NJ; }

// Table pointers arrive as integers (generic address space); loads through
// them are issued as global (not flat) loads so that they only count in
// vmcnt and the compiler can keep a prefetch in flight across LDS traffic.
#define ODP_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ u32x4_t ld16(const void* p) {
  return *(const ODP_GLOBAL u32x4_t*)(const ODP_GLOBAL void*)p;
}
// The same load marked non-temporal, for streams read once.
__device__ __forceinline__ u32x4_t ld16_nt(const void* p) {
  return __builtin_nontemporal_load((const ODP_GLOBAL u32x4_t*)(const ODP_GLOBAL void*)p);
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16).  Within each group of 16
// lanes, lane i receives v[j] = (4 x b16 chunk addressed by lane (i >> 2) + 4j)
// element (i & 3).  If lane c of the group addresses row (c >> 2), columns
// 4 (c & 3) .. +3 of a row-major [t][m] tile, lane i therefore receives
// column i of 4 consecutive rows: the K-contiguous MFMA operand layout.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
#define ODP_LDS __attribute__((address_space(3)))

// LDS row pitch, in bf16 elements, for tiles whose MFMA operands are read
// as 16-byte pieces of 16 consecutive rows at one column (ds_read_b128):
// measured on gfx950 (SQ_LDS_BANK_CONFLICT), such a read runs at full rate
// when the pitch is an odd multiple of 32 bytes and at half rate otherwise
// (e.g. 80, 144 or 272 bytes).  The smallest such pitch >= `cols`.
__host__ __device__ constexpr int lds_pitch(int cols) { return ((cols + 15) / 32) * 32 + 16; }
__device__ __forceinline__ v4i16_t lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((ODP_LDS v4i16_t*)(ODP_LDS void*)p);
}

// ---------------------------------------------------------------------------
// Projection, fp32 inputs: MFMA 16x16x4 f32.  Each wave owns 16 rows; each
// lane loads 4 consecutive contraction elements and feeds them to 4 MFMAs
// (MFMA q uses element q).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_project_f32(const int64_t* __restrict__ probs,
                                                     const int32_t* __restrict__ ws, int n_prob,
                                                     const int32_t* __restrict__ sstart,
                                                     const int32_t* __restrict__ slen) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_PJ_FIELDS;
  const float* P = (const float*)f[ODP_PJ_P];
  const int64_t ldp = f[ODP_PJ_LDP], d = f[ODP_PJ_D];
  const float* W = (const float*)f[ODP_PJ_W];
  const int r = (int)f[ODP_PJ_R];
  float* Q = (float*)f[ODP_PJ_Q];
  const int64_t ldq = f[ODP_PJ_LDQ], n_rows = f[ODP_PJ_NROWS];
  const int seg_first = (int)f[ODP_PJ_SEG_FIRST], n_seg = (int)f[ODP_PJ_NSEG];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row0 = (int64_t)(bid - ws[p]) * PJ_ROWS + 16 * wave;
  const int64_t my_row = row0 + (lane & 15);
  const bool valid = my_row < n_rows &&
                     odp_row_in_segments(my_row, sstart + seg_first, slen + seg_first, n_seg);
  // A block without segment rows reads nothing and stores its zeros.
  const bool live = __syncthreads_or(valid ? 1 : 0) != 0;
  const int nkb = (r + 15) >> 4;
  const int kq = (lane >> 4) * 4;
  const float* prow = P + (valid ? my_row : 0) * ldp;
  const int64_t dl = live ? d : 0;

  f32x4_t acc[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) acc[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = kq; k0 < dl; k0 += 16) {
    const f32x4_t a = valid ? *(const f32x4_t*)(prow + k0) : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if (kb < nkb) {
        const int wr = kb * 16 + (lane & 15);
        f32x4_t b = {0.f, 0.f, 0.f, 0.f};
        if (wr < r) b = *(const f32x4_t*)(W + (int64_t)wr * d + k0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], b[q], acc[kb], 0, 0, 0);
      }
    }
  }
  // 4 consecutive rows of one rank column: one 16-byte piece of the plane
  // row (rb is a multiple of 4; ldq, a multiple of 8, exceeds n_rows by at
  // least 32, and plane entries of rows outside segments are never read).
  const int64_t rb = row0 + 4 * (lane >> 4);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int col = kb * 16 + (lane & 15);
    if (kb < nkb && col < r && rb < n_rows) odp_gstore((f32x4_t*)(Q + (int64_t)col * ldq + rb), acc[kb]);
  }
}

// Shared epilogue of the factor kernels: scale, store per-leaf rows, and
// reduce the squared values per leaf in a fixed order.  Wave w owns the
// 16-wide m blocks w*NJ .. w*NJ + NJ - 1 of the workgroup's M-tile.
struct FactorLeaves {
  int n;
  float* pe[4];  // f32 rows, or bf16 rows where pe16 is set
  int col0[4];
  int rank[4];
  int pe16[4];
  int64_t slot[4];
};

__device__ __forceinline__ FactorLeaves read_leaves(const int64_t* f) {
  FactorLeaves L;
  L.n = (int)f[ODP_FT_NLEAF];
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const int64_t* g = f + ODP_FT_LEAF0 + 3 * l;
    const bool on = l < L.n;
    L.pe[l] = on ? (float*)g[0] : nullptr;
    L.col0[l] = on ? (int)(g[1] & 0xffff) : 1 << 20;
    L.rank[l] = on ? (int)((g[1] >> 16) & 0xffff) : 0;
    L.pe16[l] = on ? (int)((g[1] >> 32) & 1) : 0;
    L.slot[l] = on ? g[2] : 0;
  }
  return L;
}

// Value of the lane t ^ 1 (X1) or t ^ 2 (X2) of the same quad, by DPP.
__device__ __forceinline__ uint32_t quad_x1(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
}
__device__ __forceinline__ uint32_t quad_x2(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
}

// 4 x 4 transpose within each quad of lanes: lane t of the quad holds
// x[i] = B[i][t] on entry and x[c] = B[t][c] on return (two exchanges).
__device__ __forceinline__ void quad_transpose4(uint32_t (&x)[4]) {
  const int t = threadIdx.x & 3, tl = t & 1, th = t >> 1;
  const uint32_t r0 = quad_x1(tl ? x[0] : x[1]);
  const uint32_t r1 = quad_x1(tl ? x[2] : x[3]);
  // e_ab = B[2a + tl][2 th + b]
  const uint32_t e00 = tl ? r0 : x[0], e01 = tl ? x[1] : r0;
  const uint32_t e10 = tl ? r1 : x[2], e11 = tl ? x[3] : r1;
  const uint32_t ra = quad_x2(th ? e00 : e10);
  const uint32_t rb = quad_x2(th ? e01 : e11);
  const uint32_t ka = th ? e10 : e00, kb = th ? e11 : e01;
  x[0] = th ? ra : ka;
  x[1] = th ? rb : kb;
  x[2] = th ? ka : ra;
  x[3] = th ? kb : rb;
}

template <int NJ, int NKB>
__device__ __forceinline__ void factor_epilogue(const f32x4_t (&acc)[NJ][NKB], int r, float scale,
                                                int64_t M, int64_t m_base, int seg, int tile,
                                                int ex, int64_t part_stride,
                                                const FactorLeaves& L, double* __restrict__ part) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  double wsum[4] = {0.0, 0.0, 0.0, 0.0};  // this wave's sum of squares per leaf
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    double cs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cs[i] = 0.0;
      const int k = kb * 16 + 4 * (lane >> 4) + i;
      if (k >= r) continue;
      // Leaf owning column k (leaves are sorted by col0); selected without
      // dynamic indexing so the descriptor stays in registers.
      float* lpe = L.pe[0];
      int lc0 = L.col0[0], lrk = L.rank[0], l16 = L.pe16[0];
#pragma unroll
      for (int q = 1; q < 4; ++q)
        if (q < L.n && k >= L.col0[q]) {
          lpe = L.pe[q];
          lc0 = L.col0[q];
          lrk = L.rank[q];
          l16 = L.pe16[q];
        }
      // Columns of frozen factors between leaves belong to no leaf.
      if (k < lc0 || k - lc0 >= lrk) continue;
      (void)lpe;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t m = m_base + (NJ * wave + j) * 16 + (lane & 15);
        if (m < M) {
          // The value as stored in the leaf's dtype (the reference squares
          // its per-example gradient as stored, _pytree.py:224-265);
          // non-finite entries count as 0 (nan_to_num); squares are taken
          // in fp32 like the reference's float32 accumulation dtype.
          float v = scale * acc[j][kb][i];
          if (l16) v = odp_bf2f(odp_f2bf(v));
          const float vf = isfinite(v) ? v : 0.f;
          cs[i] += (double)__fmul_rn(vf, vf);
        }
      }
    }
    // The stored copy (summed after clipping) is in the leaf's dtype, as the
    // reference's per-example gradients are (the norm above squares the same
    // rounded values).  After a quad transpose each lane holds 4 consecutive
    // columns of one row: 8-byte (bf16) or 16-byte (f32) stores.
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      uint32_t x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = __float_as_uint(scale * acc[j][kb][i]);
      quad_transpose4(x);
      const int k = kb * 16 + 4 * (lane >> 4) + (lane & 3);
      const int64_t mq = m_base + (NJ * wave + j) * 16 + 4 * ((lane & 15) >> 2);
      if (k >= r || mq >= M) continue;
      float* lpe = L.pe[0];
      int lc0 = L.col0[0], lrk = L.rank[0], l16 = L.pe16[0];
#pragma unroll
      for (int q = 1; q < 4; ++q)
        if (q < L.n && k >= L.col0[q]) {
          lpe = L.pe[q];
          lc0 = L.col0[q];
          lrk = L.rank[q];
          l16 = L.pe16[q];
        }
      if (k < lc0 || k - lc0 >= lrk) continue;
      const int64_t at = ((int64_t)seg * lrk + (k - lc0)) * M + mq;
      if (l16) {
        const uint32_t lo = (uint32_t)odp_f2bf(__uint_as_float(x[0])) | ((uint32_t)odp_f2bf(__uint_as_float(x[1])) << 16);
        const uint32_t hi = (uint32_t)odp_f2bf(__uint_as_float(x[2])) | ((uint32_t)odp_f2bf(__uint_as_float(x[3])) << 16);
        odp_gstore((u32x2_t*)((uint16_t*)lpe + at), u32x2_t{lo, hi});
      } else {
        odp_gstore((u32x4_t*)(lpe + at), u32x4_t{x[0], x[1], x[2], x[3]});
      }
    }
    // Sum over the 16 lanes that share a column (same lane >> 4), then add
    // the column to its leaf's sum.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const double v = row_sum16(cs[i]);
      const int k = kb * 16 + 4 * (lane >> 4) + i;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q < L.n && k >= L.col0[q] && k < L.col0[q] + L.rank[q]) wsum[q] += v;
    }
  }
  // The four column groups of the wave, then one slot per (tile, wave): no
  // workgroup barrier, and a fixed order, so runs stay bitwise reproducible.
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (q < L.n) {
      const double v = rows_sum4(wsum[q]);
      if (lane == 0) odp_gstore(part + (int64_t)ex * part_stride + L.slot[q] + ODP_FT_WAVE_SLOTS * tile + wave, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Factor gradients, bf16 P: MFMA 16x16x32 with K = 32 tokens per step.  Per
// step the workgroup stages the P tile [32 tokens x 128 m] and the Q^T tile
// ([16*NKB x 32 tokens]) through LDS; each lane gathers its
// 8 consecutive tokens of one column for the B operand.  Loads run two steps
// ahead of the compute; the token mask is applied when a stage is written to
// LDS (never right after its load, which would stall the prefetch).
// ---------------------------------------------------------------------------
// P tiles of the factor kernel are unpadded [token][MT] rows, XOR-swizzled
// in 4-element chunks (chunk k of row r at k ^ ft_swz(r)): the 16 rows x 4
// chunks of one transposing operand read then hit every LDS bank twice and
// a stage is written with 16-byte stores.
__device__ __forceinline__ int ft_swz(int row) { return ((row & 3) | ((row >> 1) & 4)) << 2; }

template <int NKB>
__global__ __launch_bounds__(256, ft_min_blocks(NKB)) void k_factor_bf16(const int64_t* __restrict__ probs,
                                                     const int32_t* __restrict__ ws, int n_prob,
                                                     const int32_t* __restrict__ sstart,
                                                     const int32_t* __restrict__ slen,
                                                     const int32_t* __restrict__ sex,
                                                     double* __restrict__ part, int64_t part_stride) {
  constexpr int NJ = ft_nj(NKB), MT = 64 * NJ, PP = MT;  // unpadded, XOR-swizzled rows
  constexpr int QP = lds_pitch(FT_T), QROWS = 16 * NKB;
  constexpr int PTILE = FT_T * PP, STAGE = PTILE + QROWS * QP;
  constexpr int NPP = NJ * FT_T / 32;             // P pieces per thread per step
  constexpr int QPC = FT_T / 8;                   // Q pieces per row per step
  constexpr int NQP = (QPC * QROWS + 255) / 256;  // Q pieces per thread per step
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_FT_FIELDS;
  const uint16_t* P = (const uint16_t*)f[ODP_FT_P];
  const int64_t ldp = f[ODP_FT_LDP], M = f[ODP_FT_M];
  const uint16_t* Q = (const uint16_t*)f[ODP_FT_Q];
  const int64_t ldq = f[ODP_FT_LDQ];
  const int r = (int)f[ODP_FT_R];
  const int seg_first = (int)f[ODP_FT_SEG_FIRST];
  const float scale = (float)__longlong_as_double(f[ODP_FT_SCALING]);

  const int ntile = (int)((M + MT - 1) / MT);
  const int local = bid - ws[p];
  const int seg = local / ntile, tile = local % ntile;
  const int gs = seg_first + seg;
  const int64_t rs = sstart[gs], t_hi = rs + slen[gs];
  const int ex = sex[gs];
  const int64_t m_base = (int64_t)tile * MT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t_lo = rs & ~(int64_t)7;
  const int64_t nchunk = t_hi > rs ? (t_hi - t_lo + FT_T - 1) / FT_T : 0;

  struct Stage {
    u32x4_t p[NPP];
    u32x4_t q[NQP];
  };
  // Loads are branch-free (addresses clamped in bounds); rows outside the
  // segment and columns past M are zeroed when the stage is written to LDS.
  auto load = [&](int64_t c, Stage& S) {
    const int64_t t0 = t_lo + c * FT_T;
#pragma unroll
    for (int ps = 0; ps < NPP; ++ps) {
      const int id = tid + 256 * ps;
      int64_t t = t0 + id / (MT / 8);
      t = t < rs ? rs : (t >= t_hi ? t_hi - 1 : t);
      const int64_t m = m_base + (id % (MT / 8)) * 8;
      S.p[ps] = ld16(P + t * ldp + (m < M ? m : M - 8));
    }
#pragma unroll
    for (int ps = 0; ps < NQP; ++ps) {
      const int id = (tid + 256 * ps) % (QPC * QROWS);
      const int row = id / QPC, pc = id % QPC;
      S.q[ps] = ld16(Q + (int64_t)row * ldq + t0 + 8 * pc);
    }
  };
  auto store = [&](int b, int64_t c, const Stage& S) {
    uint16_t* st = lds + b * STAGE;
    const int64_t t0 = t_lo + c * FT_T;
#pragma unroll
    for (int ps = 0; ps < NPP; ++ps) {
      const int id = tid + 256 * ps;
      const int64_t t = t0 + id / (MT / 8);
      const bool ok = t >= rs && t < t_hi && m_base + (id % (MT / 8)) * 8 < M;
      const u32x4_t v = ok ? S.p[ps] : u32x4_t{0u, 0u, 0u, 0u};
      const int row = id / (MT / 8), chunk = 2 * (id % (MT / 8));
      *(u32x4_t*)&st[row * PP + 4 * (chunk ^ ft_swz(row))] = v;
    }
#pragma unroll
    for (int ps = 0; ps < NQP; ++ps) {
      const int id = tid + 256 * ps;
      if (id < QPC * QROWS) {
        const int row = id / QPC, pc = id % QPC;
        const int64_t tq = t0 + 8 * pc;
        u32x4_t v = S.q[ps];
        // Tokens outside [rs, t_hi) contribute nothing.
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int64_t ta = tq + 2 * w;
          v[w] &= ((ta >= rs && ta < t_hi) ? 0x0000ffffu : 0u) |
                  ((ta + 1 >= rs && ta + 1 < t_hi) ? 0xffff0000u : 0u);
        }
        *(u32x4_t*)&st[PTILE + row * QP + 8 * pc] = v;
      }
    }
  };

  f32x4_t acc[NJ][NKB];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc[j][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int b) {
    const uint16_t* st = lds + b * STAGE;
#pragma unroll
    for (int u = 0; u < FT_T / 32; ++u)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      // B operand: lane gets tokens 32u + 8*(lane>>4) + 0..7 of column m0 + (lane&15),
      // as two transposing reads of 4 tokens each.
      const int m0 = (NJ * wave + j) * 16, c = lane & 15;
      const int row = 32 * u + 8 * (lane >> 4) + (c >> 2);
      // Rows r and r + 4 share ft_swz(), so the second read is 4 rows on.
      const uint16_t* src = st + row * PP + 4 * (((m0 >> 2) + (c & 3)) ^ ft_swz(row));
      const v4i16_t t0 = lds_tr16(src), t1 = lds_tr16(src + 4 * PP);
      const v4i16_t tt[2] = {t0, t1};
      const bf16x8_t bop = __builtin_bit_cast(bf16x8_t, tt);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const int row = kb * 16 + (lane & 15);
        const int tc = 32 * u + 8 * (lane >> 4);
        const u32x4_t qv = *(const u32x4_t*)&st[PTILE + row * QP + tc];
        acc[j][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qv), bop,
                                                             acc[j][kb], 0, 0, 0);
      }
    }
  };

  // Prefetch indices are clamped to the last chunk instead of branching.
  Stage SA, SB;
  const int64_t last = nchunk - 1;
  if (nchunk > 0) {
    load(0, SA);
    load(1 < last ? 1 : last, SB);
  }
  for (int64_t c = 0; c < nchunk; c += 2) {
    store(0, c, SA);
    __syncthreads();
    load(c + 2 < last ? c + 2 : last, SA);
    // Keep the prefetch issued here: left alone, the scheduler sinks these
    // loads past the compute to shorten live ranges, which leaves only one
    // stage in flight.
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    if (c + 1 >= nchunk) break;
    store(1, c + 1, SB);
    __syncthreads();
    load(c + 3 < last ? c + 3 : last, SB);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
  }

  const FactorLeaves L = read_leaves(f);
  factor_epilogue<NJ, NKB>(acc, r, scale, M, m_base, seg, tile, ex, part_stride, L, part);
}

// ---------------------------------------------------------------------------
// G side of one LoRA site in a single pass over G, bf16, r <= 16.  For one
// segment the workgroup walks G in 256-column chunks; within a chunk it
// streams the segment's tokens 64 at a time and forms both
//   pe[k][m]  = scaling * sum_t V[k][t] G[t][m]   (dB rows, as k_factor_bf16)
//   U[t][k]  += sum_{m in chunk} G[t][m] B[k][m]  (the projection U = G B^T)
// so that G is read from HBM once instead of once per stage.  U of every
// token of the segment stays in registers across the chunks (wave w owns
// tokens 16w .. 16w + 15 of each step), which bounds the segment to
// FP_STEPS steps: lengths up to FP_STEPS * 64 - 7 tokens.  One step of
// loads is in flight (the LDS stage parity then does not depend on the
// step count); B's 256-column chunk is held in registers as MFMA operands.
// ---------------------------------------------------------------------------
constexpr int FP_T = 64, FP_MT = 256, FP_STEPS = 17;
constexpr uint32_t ODP_BUFFER_DWORD3 = 0x00020000;  // raw 32-bit dwords (CDNA buffer resource)
// G's loads are marked non-temporal (cache policy bit NT): G streams
// through once, and the hint keeps it from evicting the segment's V plane,
// which every chunk reads again (4.5 % faster on C3 shapes).
constexpr int FP_G_NT = 2;

// Default column chunks per workgroup of the streamed factor pass (PROJ =
// false below; the table row gives the group count): a segment's chunks are
// split into groups of at most this many, so that the widest rows do not
// leave a tail of long workgroups.
#ifndef ODP_FS_GROUP
#define ODP_FS_GROUP 4  // C3: 4 best for three rank blocks (6 % over 8), 4-12 alike for one, 16+ slower
#endif
__host__ __device__ constexpr int fs_groups(int nchunks) {
  return nchunks <= 0 ? 1 : (nchunks + ODP_FS_GROUP - 1) / ODP_FS_GROUP;
}

// One pass over P = G of a segment in 256-column chunks.  PROJ: the fused
// G side above (dB rows and U = G B^T, one workgroup per segment, all
// chunks).  !PROJ: the planes are given, so the pass forms only the
// per-example factor rows pe[k][m] = scaling * sum_t Q[k][t] P[t][m] (dB
// from G and V, or dA from X and U) of a problem with NKB 16-row blocks of
// Q, each holding at most one leaf that starts at the block (rank <= 16):
// the pipeline of the fused kernel without B, U and its registers.  A
// workgroup then takes one of the row's ODP_FT_GROUPS groups of
// consecutive chunks of its segment.  Both compute each chunk's rows,
// squares and partial slots exactly as k_factor_bf16<NKB> does for its
// 256-column tile (same token blocks, same order).
template <bool PROJ, int NKB>
__device__ __forceinline__ void factor_pass_bf16(const int64_t* __restrict__ probs, const int32_t* __restrict__ ws,
                                                 int n_prob, const int32_t* __restrict__ sstart,
                                                 const int32_t* __restrict__ slen, const int32_t* __restrict__ sex,
                                                 double* __restrict__ part, int64_t part_stride) {
  static_assert(NKB >= 1 && NKB <= 3 && (!PROJ || NKB == 1), "one to three rank blocks; the fused G side has one");
  constexpr int NJ = FP_MT / 64, PP = FP_MT;  // unpadded, XOR-swizzled G rows
  constexpr int QP = lds_pitch(FP_T), QROWS = 16 * NKB;
  constexpr int PTILE = FP_T * PP, STAGE = PTILE + QROWS * QP;
  constexpr int QPC = FP_T / 8;                  // V pieces per row per step
  constexpr int NQP = QPC * QROWS;               // V pieces per step: 128 per rank block
  constexpr int NQ = (NQP + 255) / 256;          // per thread (waves past NQP issue none)
  static_assert(NQP % 128 == 0, "V pieces cover whole waves");
  // Stores a chunk's flush issues (every one unconditional): NJ rows and a
  // partial per rank block.  The step-1 wait below encodes it in 4 bits.
  constexpr int NFLUSH = NKB * (NJ + 1);
  static_assert(NFLUSH <= 15, "vmcnt immediate");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_FT_FIELDS;
  const uint16_t* P = (const uint16_t*)f[ODP_FT_P];
  const int32_t ldp = (int32_t)f[ODP_FT_LDP], M = (int32_t)f[ODP_FT_M];
  const int32_t ldq = (int32_t)f[ODP_FT_LDQ];
  const int r = (int)f[ODP_FT_R];
  const float scale = (float)__longlong_as_double(f[ODP_FT_SCALING]);
  const uint16_t* W = PROJ ? (const uint16_t*)f[ODP_FP_W] : nullptr;

  const int nchunks = (M + FP_MT - 1) / FP_MT;
  const int local = bid - ws[p];
  int seg, c_begin, c_end;
  if constexpr (PROJ) {
    seg = local;
    c_begin = 0;
    c_end = nchunks;
  } else {
    const int64_t ng = f[ODP_FT_GROUPS] > 0 ? f[ODP_FT_GROUPS] : 1;
    seg = (int)(local / ng);
    const int64_t grp = local - seg * ng;
    c_begin = (int)(grp * nchunks / ng);
    c_end = (int)((grp + 1) * nchunks / ng);
    // Workgroups past the row's segments (a table whose work_start counts
    // more than n_seg * groups) have nothing to do.
    if (seg >= (int)f[ODP_FT_NSEG]) return;
  }
  const int gs = (int)f[ODP_FT_SEG_FIRST] + seg;
  const int32_t rs = sstart[gs], len = slen[gs], t_hi = rs + len;
  const int ex = sex[gs];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t t_lo = rs & ~7;
  int nsteps = len > 0 ? (t_hi - t_lo + FP_T - 1) / FP_T : 0;
  nsteps = nsteps < FP_STEPS ? nsteps : FP_STEPS;  // the host keeps segments within bounds

  // G through a buffer resource over the segment's rows, loaded straight
  // into LDS: rows outside the segment (offsets below it wrap past the end)
  // and columns past M (given an offset past the end) arrive as zeros.
  const __amdgpu_buffer_rsrc_t grsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(P + (int64_t)rs * ldp), (short)0, (int)((uint32_t)len * (uint32_t)ldp * 2u), ODP_BUFFER_DWORD3);
  // Each wave fills tile rows 16 wave .. + 15, two rows (1 KB) per
  // instruction; lane l lands in physical 16-byte slot l & 31 of row
  // 16 wave + 2 i + (l >> 5), so it fetches the logical slot that the XOR
  // swizzle maps there.
  const int gh = lane >> 5, gslot = lane & 31;
  // V pieces (a rank row and 8 tokens of a step) go to threads in order,
  // 128 per rank block: with one block waves 0 and 1 load them.  `vown` is
  // wave-uniform, so the V loads and stores are scalar branches.
  const int qpc = tid % QPC;
  bool vown[NQ];
  const uint16_t* qsrc[NQ];
  uint16_t* qdst_base[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    vown[i] = __builtin_amdgcn_readfirstlane(wave) * 64 + 256 * i < NQP;
    const int qrow = ((tid + 256 * i) % NQP) / QPC;
    qsrc[i] = (const uint16_t*)f[ODP_FT_Q] + (int64_t)qrow * ldq;
    qdst_base[i] = lds + PTILE + qrow * QP + 8 * qpc;
  }

  auto load = [&](uint16_t* stage, int32_t t0, int32_t m_base, u32x4_t (&qv)[NQ]) {
    uint16_t* dst = stage + 16 * wave * PP;
#pragma unroll
    for (int i = 0; i < FP_T / 4 / 2; ++i) {
      const int row = 16 * wave + 2 * i + gh;
      const int32_t col = m_base + 8 * (gslot ^ (ft_swz(row) >> 1));
      const uint32_t off = col < M ? ((uint32_t)(t0 - rs + row) * (uint32_t)ldp + (uint32_t)col) * 2u
                                   : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(grsrc, (ODP_LDS void*)(dst + 2 * i * PP), 16, off, 0, 0, FP_G_NT);
    }
    const int32_t tq = t0 + 8 * qpc;
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      if (vown[i]) qv[i] = ld16(qsrc[i] + (tq < t_hi ? tq : t_lo));
  };
  // V's tokens outside [rs, t_hi) are zeroed when its piece is written.
  auto store_q = [&](int b, int32_t t0, const u32x4_t (&qv)[NQ]) {
    const int32_t tq = t0 + 8 * qpc;
    uint32_t mask[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int32_t ta = tq + 2 * w;
      mask[w] = ((ta >= rs && ta < t_hi) ? 0x0000ffffu : 0u) | ((ta + 1 >= rs && ta + 1 < t_hi) ? 0xffff0000u : 0u);
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      if (!vown[i]) continue;
      u32x4_t v = qv[i];
#pragma unroll
      for (int w = 0; w < 4; ++w) v[w] &= mask[w];
      *(u32x4_t*)(qdst_base[i] + b * STAGE) = v;
    }
  };

  f32x4_t acc_u[PROJ ? FP_STEPS : 1];
#pragma unroll
  for (int st = 0; st < (PROJ ? FP_STEPS : 1); ++st) acc_u[st] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // The leaf of each rank block (bf16 rows): the one that starts at column
  // 16 kb of Q, if any (rank 0 otherwise: nothing stored, no partial).
  const FactorLeaves L = read_leaves(f);
  uint16_t* lpe[NKB];
  int lrank[NKB];
  int64_t lslot[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    lpe[kb] = nullptr;
    lrank[kb] = 0;
    lslot[kb] = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q < L.n && L.col0[q] == 16 * kb) {
        lpe[kb] = (uint16_t*)L.pe[q];
        lrank[kb] = L.rank[q] < 16 ? L.rank[q] : 16;
        lslot[kb] = L.slot[q];
      }
  }
  // A segment longer than FP_STEPS steps does not fit this pass (the host
  // keeps segments within odp_factor_project_max_len()): its partial slots
  // become NaN, so that its norm and clip factor show it, and nothing else
  // is written.
  if (len > 0 && (t_hi - t_lo + FP_T - 1) / FP_T > FP_STEPS) {
    if (lane == 0)
      for (int kb = 0; kb < NKB; ++kb)
        if (lrank[kb] > 0)
          for (int c = c_begin; c < c_end; ++c)
            odp_gstore(part + (int64_t)ex * part_stride + lslot[kb] + ODP_FT_WAVE_SLOTS * c + wave,
                       __builtin_nan(""));
    return;
  }

  // A chunk's rows (bf16) and this wave's norm partials wait in registers
  // and are stored after the next step's barrier: a barrier waits for every
  // memory operation in flight, so stores issued just before one would
  // stall it for their whole latency.  The arithmetic is factor_epilogue's
  // for one leaf per rank block, in the same order.
  uint32_t pend[NKB][NJ * 2];
  double pend_sq[NKB];
  int32_t pend_m0 = -1, pend_tile = 0;  // pend_m0 < 0: nothing pending
  auto hold = [&](const f32x4_t (&acc)[NJ][NKB], int32_t m_base, int tile) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int rk = lrank[kb];
      double wsum = 0.0, cs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cs[i] = 0.0;
        const int k = 4 * (lane >> 4) + i;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int32_t m = m_base + (NJ * wave + j) * 16 + (lane & 15);
          const float v = scale * acc[j][kb][i];
          const uint32_t h = odp_f2bf(v);
          if (i & 1)
            pend[kb][2 * j + (i >> 1)] |= h << 16;
          else
            pend[kb][2 * j + (i >> 1)] = h;
          if (k < rk && m < M) {
            const float vq = odp_bf2f((uint16_t)h);  // the value as stored
            const float vf = isfinite(vq) ? vq : 0.f;
            cs[i] += (double)__fmul_rn(vf, vf);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double v = row_sum16(cs[i]);
        if (4 * (lane >> 4) + i < rk) wsum += v;
      }
      pend_sq[kb] = rows_sum4(wsum);
    }
    pend_m0 = m_base;
    pend_tile = tile;
  };
  // Each 16 x 16 block of rows leaves as 8-byte pieces: a 4 x 4 transpose
  // within each quad of lanes (two exchanges) turns lane (g, 4q + t)'s
  // column of rows 4g .. 4g + 3 into row 4g + t, columns 4q .. 4q + 3.  The
  // stores are buffer stores issued unconditionally (an offset past the end
  // drops a store with nothing to write): the compiler then knows that
  // exactly NFLUSH of them follow B's loads, and the MFMAs that wait for B
  // do not wait for the stores.
  __amdgpu_buffer_rsrc_t pe_rsrc[NKB], part_rsrc[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    pe_rsrc[kb] = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(lpe[kb] + (int64_t)seg * lrank[kb] * M), (short)0,
        (int)((uint32_t)lrank[kb] * (uint32_t)M * 2u), ODP_BUFFER_DWORD3);
    part_rsrc[kb] = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(part + (int64_t)ex * part_stride + lslot[kb]), (short)0,
        lrank[kb] > 0 ? (int)(ODP_FT_WAVE_SLOTS * (uint32_t)nchunks * 8u) : 0, ODP_BUFFER_DWORD3);
  }
  auto flush = [&]() {
    const bool live = pend_m0 >= 0;
    const int t = lane & 3, tl = t & 1, th = t >> 1;
    const int k = 4 * (lane >> 4) + t;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint32_t h0 = pend[kb][2 * j] & 0xffffu, h1 = pend[kb][2 * j] >> 16;
        const uint32_t h2 = pend[kb][2 * j + 1] & 0xffffu, h3 = pend[kb][2 * j + 1] >> 16;
        // Rows of the other parity to the odd/even neighbour.
        const uint32_t r1 = quad_x1(tl ? (h0 | (h2 << 16)) : (h1 | (h3 << 16)));
        // Rows 4g + 2a + tl, columns of this lane pair (low half: even column).
        const uint32_t p0 = tl ? ((r1 & 0xffffu) | (h1 << 16)) : (h0 | (r1 << 16));
        const uint32_t p1 = tl ? ((r1 >> 16) | (h3 << 16)) : (h2 | (r1 & 0xffff0000u));
        // Row pairs across the two lane pairs of the quad.
        const uint32_t r2 = quad_x2(th ? p0 : p1);
        const uint32_t keep = th ? p1 : p0;
        const int32_t m = pend_m0 + (NJ * wave + j) * 16 + 4 * ((lane & 15) >> 2);
        const uint32_t off =
            live && k < lrank[kb] && m < M ? ((uint32_t)k * (uint32_t)M + (uint32_t)m) * 2u : 0x80000000u;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{th ? r2 : keep, th ? keep : r2}, pe_rsrc[kb], (int)off, 0, 0);
      }
      const uint32_t poff =
          live && lane == 0 ? (uint32_t)(ODP_FT_WAVE_SLOTS * pend_tile + wave) * 8u : 0x80000000u;
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, pend_sq[kb]), part_rsrc[kb], (int)poff, 0,
                                            0);
    }
    pend_m0 = -1;
  };
  // B's chunk as MFMA B operands: k-step ks covers columns 32 ks .. + 31,
  // lane holds B[lane & 15][32 ks + 8 (lane >> 4) .. + 7].  Loaded after the
  // chunk's first barrier, like the stores above, through a buffer resource
  // over B's r rows: columns past M and rows past r arrive as zeros, with
  // no select that would make the wave wait for the loads at once.
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)W, (short)0, (int)((uint32_t)r * (uint32_t)M * 2u), ODP_BUFFER_DWORD3);
  const uint32_t wrow = (lane & 15) < r ? (uint32_t)(lane & 15) * (uint32_t)M : 0x40000000u;

  u32x4_t qv[NQ];
  int buf = 0;
  if (nsteps > 0 && c_begin < c_end) load(lds, t_lo, c_begin * FP_MT, qv);
  for (int c = c_begin; c < c_end; ++c) {
    const int32_t m_base = c * FP_MT;
    // The first token of the steps, re-read per chunk: address arithmetic
    // of the unrolled steps then stays inside the loop instead of being
    // hoisted out of it for every step (which exhausts registers).
    int32_t tc0 = t_lo;
    __asm__ volatile("" : "+s"(tc0));
    bf16x8_t wf[FP_MT / 32];
    f32x4_t acc[NJ][NKB];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) acc[j][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // One step: the next stage's loads go into `nxt` while the step reads
    // `sp`.  The two are restrict-qualified, so the compiler's scoped alias
    // information tells them apart and the transposing reads of `sp` do
    // not wait for the loads just issued into `nxt` (a barrier at the top
    // of each step already waits for the stage's own loads).
    auto step = [&](uint16_t* __restrict__ nxt, const uint16_t* __restrict__ sp,
                    int st) __attribute__((always_inline)) {
      if (st + 1 < nsteps)
        load(nxt, tc0 + (st + 1) * FP_T, m_base, qv);
      else if (c + 1 < c_end)
        load(nxt, tc0, m_base + FP_MT, qv);
      if (st == 0) {
        if constexpr (PROJ) {
          // B's loads before the stores: the MFMAs that wait for B then do
          // not wait for the stores too (memory operations complete in
          // issue order as far as s_waitcnt counts them).
#pragma unroll
          for (int ks = 0; ks < FP_MT / 32; ++ks) {
            const int32_t m = m_base + 32 * ks + 8 * (lane >> 4);
            const uint32_t off = m < M ? (wrow + (uint32_t)m) * 2u : 0x80000000u;
            wf[ks] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)off, 0, 0));
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        flush();
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
      // Factor rows: B operand = P columns by transposing reads, A = Q.
#pragma unroll
      for (int u = 0; u < FP_T / 32; ++u) {
        const int tc = 32 * u + 8 * (lane >> 4);
        u32x4_t vv[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) vv[kb] = *(const u32x4_t*)&sp[PTILE + (16 * kb + (lane & 15)) * QP + tc];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int m0 = (NJ * wave + j) * 16, cc = lane & 15;
          const int row = 32 * u + 8 * (lane >> 4) + (cc >> 2);
          const uint16_t* src = sp + row * PP + 4 * (((m0 >> 2) + (cc & 3)) ^ ft_swz(row));
          const v4i16_t t0 = lds_tr16(src), t1 = lds_tr16(src + 4 * PP);
          const v4i16_t tt[2] = {t0, t1};
          const bf16x8_t bop = __builtin_bit_cast(bf16x8_t, tt);
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
            acc[j][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, vv[kb]), bop,
                                                                 acc[j][kb], 0, 0, 0);
        }
      }
      // U rows 16 wave .. + 15 of the step: A = G rows (8 consecutive
      // columns per lane; a swizzled chunk pair stays contiguous).
      if constexpr (PROJ) {
        const int row = 16 * wave + (lane & 15);
#pragma unroll
        for (int ks = 0; ks < FP_MT / 32; ++ks) {
          const int chunk = 8 * ks + 2 * (lane >> 4);
          const u32x4_t av = *(const u32x4_t*)&sp[row * PP + 4 * (chunk ^ ft_swz(row))];
          acc_u[st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), wf[ks],
                                                              acc_u[st], 0, 0, 0);
        }
      }
    };
    // Steps as nested conditionals (step st + 1 inside step st): each step
    // is then reached only from the one before it, and the compiler counts
    // the memory operations in flight exactly across them.
    auto steps = [&](auto self, auto I) __attribute__((always_inline)) {
      constexpr int st = decltype(I)::value;
      if constexpr (st < FP_STEPS) {
        if (st < nsteps) {
          store_q(buf, tc0 + st * FP_T, qv);
          // The stage's loads (this wave's) must have landed and its V pieces
          // be written before the barrier.  Vector memory operations complete
          // in issue order as s_waitcnt counts them, and step 0 issues the
          // stage's loads before B's loads and the NFLUSH stores of the
          // previous chunk: at step 1, vmcnt <= NFLUSH covers the stage while
          // the stores drain.  Other steps wait for everything.
          if (st == 1)
            __builtin_amdgcn_s_waitcnt(0x0070 | NFLUSH);  // vmcnt(NFLUSH) lgkmcnt(0)
          else
            __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
          __asm__ volatile("s_barrier" ::: "memory");
          step(lds + (buf ^ 1) * STAGE, lds + buf * STAGE, st);
          buf ^= 1;
          self(self, std::integral_constant<int, st + 1>{});
        }
      }
    };
    steps(steps, std::integral_constant<int, 0>{});
    hold(acc, m_base, c);
    if (nsteps == 0) flush();  // no step of the next chunk will
  }
  flush();

  // U: lane holds rows 4 (lane >> 4) + i, column lane & 15 of each step's
  // 16 x 16 block: 4 consecutive entries of the column's plane row (tb is a
  // multiple of 4), stored as one 8-byte piece when all four tokens are the
  // segment's; tokens outside the segment belong to other workgroups, so a
  // group that straddles a segment end is stored entry by entry.
  if constexpr (PROJ) {
    const int col = lane & 15;
    if (col < r) {
      uint16_t* uq = (uint16_t*)f[ODP_FP_U] + (int64_t)col * ldq;
#pragma unroll
      for (int st = 0; st < FP_STEPS; ++st) {
        if (st < nsteps) {
          const int32_t tb = t_lo + st * FP_T + 16 * wave + 4 * (lane >> 4);
          uint32_t h[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) h[i] = odp_f2bf(acc_u[st][i]);
          if (tb >= rs && tb + 3 < t_hi) {
            odp_gstore((u32x2_t*)(uq + tb), u32x2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)});
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int32_t t = tb + i;
              if (t >= rs && t < t_hi) odp_gstore(uq + t, (uint16_t)h[i]);
            }
          }
        }
      }
    }
  }
}

__global__ __launch_bounds__(256, 2) void k_factor_project_bf16(const int64_t* __restrict__ probs,
                                                                const int32_t* __restrict__ ws, int n_prob,
                                                                const int32_t* __restrict__ sstart,
                                                                const int32_t* __restrict__ slen,
                                                                const int32_t* __restrict__ sex,
                                                                double* __restrict__ part,
                                                                int64_t part_stride) {
  factor_pass_bf16<true, 1>(probs, ws, n_prob, sstart, slen, sex, part, part_stride);
}

template <int NKB>
__global__ __launch_bounds__(256, 2) void k_factor_stream_bf16(const int64_t* __restrict__ probs,
                                                               const int32_t* __restrict__ ws, int n_prob,
                                                               const int32_t* __restrict__ sstart,
                                                               const int32_t* __restrict__ slen,
                                                               const int32_t* __restrict__ sex,
                                                               double* __restrict__ part,
                                                               int64_t part_stride) {
  factor_pass_bf16<false, NKB>(probs, ws, n_prob, sstart, slen, sex, part, part_stride);
}

// ---------------------------------------------------------------------------
// Projection, bf16: MFMA 16x16x32 bf16 with fp32 accumulation, the
// contraction 32 columns at a time in order, with P and W moved by buffer
// loads straight into a ring of LDS stages, PS_RING - 1 steps ahead of the
// compute.  A workgroup owns
// PS_ROWS = 256 rows, each wave 64 of them (four 16-row MFMA blocks), and
// walks the contraction PS_KC = 64 columns per step.  Each wave loads, and
// reads, only its own rows of P (1 KB = 8 rows per load); the step's W tile
// (16 NKB rank rows) is loaded a quarter per wave, 4 bytes per lane.  Rows
// outside the segments or past n_rows, rank rows past r and columns past d
// get offsets past the buffers' ends, so they arrive as zeros and cost no
// HBM traffic.  LDS rows are 128 bytes, unpadded, with 16-byte slot q of
// row t at slot q ^ (t & 7): the operand reads (16 rows at one slot) then
// run without bank conflicts.
// ---------------------------------------------------------------------------
constexpr int PS_ROWS = 256, PS_KC = 64;
// Ring stages per rank block count: as many 32 KB steps of P in flight as
// the 160 KB of LDS hold (one workgroup per CU).
#ifndef ODP_PS_RING
#define ODP_PS_RING 4
#endif
__host__ __device__ constexpr int ps_ring(int nkb) { return nkb <= 3 ? ODP_PS_RING : 3; }

// One step: loads for a later step into `nxt`, then this step's MFMAs from
// `cur`.  Both are restrict parameters of one inlined call, so that the
// compiler's alias scopes keep the reads of `cur` from waiting for the loads
// into `nxt`.
template <int NKB, typename Issue>
__device__ __forceinline__ void ps_step(uint16_t* __restrict__ nxt, const uint16_t* __restrict__ cur, Issue issue,
                                        f32x4_t (&acc)[4][NKB]) {
  constexpr int XT = PS_ROWS * PS_KC;
  issue(nxt);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sw = lane & 7;  // t & 7 of every row this lane reads
#pragma unroll
  for (int h = 0; h < PS_KC / 32; ++h) {
    const int q = 4 * h + (lane >> 4);
    u32x4_t bv[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      bv[kb] = *(const u32x4_t*)&cur[XT + (16 * kb + (lane & 15)) * PS_KC + 8 * (q ^ sw)];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const u32x4_t av = *(const u32x4_t*)&cur[(64 * wave + 16 * rb + (lane & 15)) * PS_KC + 8 * (q ^ sw)];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        acc[rb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av),
                                                              __builtin_bit_cast(bf16x8_t, bv[kb]), acc[rb][kb], 0,
                                                              0, 0);
    }
  }
}

template <int NKB>
__global__ __launch_bounds__(256, ps_ring(NKB) == 2 ? 2 : 1) void k_project_stream_bf16(
    const int64_t* __restrict__ probs, const int32_t* __restrict__ ws, int n_prob,
    const int32_t* __restrict__ sstart, const int32_t* __restrict__ slen) {
  static_assert(NKB >= 1 && NKB <= 4, "one to four rank blocks");
  constexpr int PS_RING = ps_ring(NKB);
  static_assert(PS_RING >= 2 && PS_RING <= 4, "two to four ring stages");
  constexpr int XT = PS_ROWS * PS_KC, STAGE = XT + 16 * NKB * PS_KC;
  static_assert(PS_RING * STAGE * 2 <= 156 * 1024, "the ring fits in LDS");
  constexpr int XD = PS_ROWS / 4 / 8;  // 1 KB loads of P per wave per step
  constexpr int WD = 2 * NKB;          // 256-byte loads of W per wave per step
  constexpr int NDMA = XD + WD;
  static_assert(NDMA < 64, "vmcnt range");
  constexpr uint32_t OOB = 0x80000000u;
  __shared__ __attribute__((aligned(16))) uint16_t ps0[STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t ps1[STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t ps2[PS_RING > 2 ? STAGE : 8];
  __shared__ __attribute__((aligned(16))) uint16_t ps3[PS_RING > 3 ? STAGE : 8];
  auto stage = [&](int k) -> uint16_t* { return k == 0 ? ps0 : k == 1 ? ps1 : k == 2 ? ps2 : ps3; };

  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_PJ_FIELDS;
  const uint16_t* P = (const uint16_t*)f[ODP_PJ_P];
  const int64_t ldp = f[ODP_PJ_LDP], d = f[ODP_PJ_D];
  const uint16_t* W = (const uint16_t*)f[ODP_PJ_W];
  const int r = (int)f[ODP_PJ_R];
  uint16_t* Q = (uint16_t*)f[ODP_PJ_Q];
  const int64_t ldq = f[ODP_PJ_LDQ], n_rows = f[ODP_PJ_NROWS];
  const int seg_first = (int)f[ODP_PJ_SEG_FIRST], n_seg = (int)f[ODP_PJ_NSEG];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Rows: the problem's covered rows (each segment widened to whole 8-row
  // groups, [start & ~7, ceil8(start + len)), concatenated in segment
  // order) in blocks of PS_ROWS, so that padding between segments costs no
  // workgroups.  Wave w takes groups 8 w .. 8 w + 7 of its block; lane j < 8
  // finds the first row of group 8 w + j (-1 past the covered rows).  The
  // walk over the segments is the same for every lane.
  const int64_t v0 = (int64_t)(bid - ws[p]) * PS_ROWS;
  int32_t gfirst = -1;
  {
    const int64_t v = v0 + 64 * wave + 8 * (lane & 7);
    int64_t cum = 0;
    for (int sg = 0; sg < n_seg && cum < v0 + PS_ROWS; ++sg) {
      const int64_t st = sstart[seg_first + sg], ln = slen[seg_first + sg];
      if (ln <= 0) continue;
      const int64_t a = st & ~(int64_t)7, cov = ((st + ln + 7) & ~(int64_t)7) - a;
      if (v >= cum && v < cum + cov) gfirst = (int32_t)(a + (v - cum));
      cum += cov;
    }
  }
  int32_t gb[XD];
  bool any = false;
#pragma unroll
  for (int i = 0; i < XD; ++i) {
    gb[i] = __builtin_amdgcn_readlane(gfirst, i);
    any |= gb[i] >= 0;
  }
  // A block past the covered rows loads and stores nothing.
  const bool live = __syncthreads_or(any ? 1 : 0) != 0;

  // P: load i fills group i of the wave (8 rows of 128 bytes) through a
  // buffer resource over the group's rows; lane l fills physical slot l & 7
  // of row l / 8, which holds logical slot (l & 7) ^ (l / 8).
  __amdgpu_buffer_rsrc_t prs[XD];
#pragma unroll
  for (int i = 0; i < XD; ++i) {
    const int64_t rows = gb[i] < 0 ? 0 : (n_rows - gb[i] < 8 ? n_rows - gb[i] : 8);
    prs[i] = __builtin_amdgcn_make_buffer_rsrc((void*)(P + (gb[i] < 0 ? 0 : (int64_t)gb[i]) * ldp), (short)0,
                                               rows > 0 ? (int)((uint32_t)rows * (uint32_t)ldp * 2u) : 0,
                                               ODP_BUFFER_DWORD3);
  }
  const uint32_t xrow = (uint32_t)(lane >> 3) * (uint32_t)ldp * 2u;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)W, (short)0, (int)((uint32_t)r * (uint32_t)d * 2u), ODP_BUFFER_DWORD3);
  const int xcol = 8 * ((lane & 7) ^ ((lane >> 3) & 7));
  // W: load j covers rank rows 4 NKB wave + 2 j + lane / 32, 4 bytes per
  // lane: word lane & 3 of physical slot (lane & 31) / 4.
  uint32_t wrow[WD];
  int wcol[WD];
#pragma unroll
  for (int j = 0; j < WD; ++j) {
    const int k = 4 * NKB * wave + 2 * j + (lane >> 5);
    wcol[j] = 8 * (((lane & 31) >> 2) ^ (k & 7));
    wrow[j] = k < r ? (uint32_t)k * (uint32_t)d * 2u + 4u * (uint32_t)(lane & 3) : OOB;
  }
  // Loads of the step at column c0 (c0 >= d: none, every offset past the end).
  auto issue = [&](uint16_t* st, int64_t c0) {
#pragma unroll
    for (int i = 0; i < XD; ++i) {
      const int64_t c = c0 + xcol;
      const uint32_t off = c < d ? xrow + (uint32_t)c * 2u : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(prs[i], (ODP_LDS void*)(st + (64 * wave + 8 * i) * PS_KC), 16, off,
                                               0, 0, FP_G_NT);
    }
#pragma unroll
    for (int j = 0; j < WD; ++j) {
      const int64_t c = c0 + wcol[j];
      const uint32_t off = wrow[j] != OOB && c < d ? wrow[j] + (uint32_t)c * 2u : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (ODP_LDS void*)(st + XT + (4 * NKB * wave + 2 * j) * PS_KC), 4,
                                               off, 0, 0, 0);
    }
  };

  f32x4_t acc[4][NKB];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc[b][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int64_t nsteps = live ? (d + PS_KC - 1) / PS_KC : 0;
#pragma unroll
  for (int q = 0; q < PS_RING - 1; ++q)
    if (live) issue(stage(q), q < nsteps ? q * PS_KC : d);
  for (int64_t s = 0; s < nsteps;) {
#pragma unroll
    for (int k = 0; k < PS_RING; ++k) {
      if (s >= nsteps) break;
      // This step's loads (this wave's) have landed; the later ones may fly.
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((PS_RING - 2) * NDMA));
      __asm__ volatile("s_barrier" ::: "memory");
      const int64_t nx = s + PS_RING - 1;
      const int64_t c0 = nx < nsteps ? nx * PS_KC : d;
      ps_step<NKB>(stage((k + PS_RING - 1) % PS_RING), stage(k), [&](uint16_t* st) { issue(st, c0); }, acc);
      ++s;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no load into LDS may outlive the workgroup

  // 4 consecutive rows of one rank column per lane (rows 4 (lane / 16) ..
  // + 3 of block b: half of group 2 b + lane / 32), which are 4 consecutive
  // entries of that column's plane row, rounded to bf16 (the rank-space
  // products of the reference's per-sample rule, X A and G B^T, are bf16
  // tensors) and stored as one 8-byte piece.  ldq exceeds n_rows by at
  // least 32, so a piece that starts below n_rows stays inside the plane.
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int32_t g0 = (lane >> 5) ? gb[2 * b + 1] : gb[2 * b];
    const int64_t rb = g0 < 0 ? n_rows : (int64_t)g0 + 4 * ((lane >> 4) & 1);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int col = kb * 16 + (lane & 15);
      if (col < r && rb < n_rows) {
        uint32_t h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i] = odp_f2bf(acc[b][kb][i]);
        odp_gstore((u32x2_t*)(Q + (int64_t)col * ldq + rb), u32x2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)});
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Factor gradients, fp32 P: MFMA 16x16x4 f32 with K = 16 tokens per step in
// four MFMAs; operands come straight from global memory (P rows are read
// 64 bytes per 16 lanes, which coalesces).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_factor_f32(const int64_t* __restrict__ probs,
                                                    const int32_t* __restrict__ ws, int n_prob,
                                                    const int32_t* __restrict__ sstart,
                                                    const int32_t* __restrict__ slen,
                                                    const int32_t* __restrict__ sex,
                                                    double* __restrict__ part, int64_t part_stride) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_FT_FIELDS;
  const float* P = (const float*)f[ODP_FT_P];
  const int64_t ldp = f[ODP_FT_LDP], M = f[ODP_FT_M];
  const float* Q = (const float*)f[ODP_FT_Q];
  const int64_t ldq = f[ODP_FT_LDQ];
  const int r = (int)f[ODP_FT_R];
  const int seg_first = (int)f[ODP_FT_SEG_FIRST];
  const float scale = (float)__longlong_as_double(f[ODP_FT_SCALING]);

  const int ntile = (int)((M + FT_M_F32 - 1) / FT_M_F32);
  const int local = bid - ws[p];
  const int seg = local / ntile, tile = local % ntile;
  const int gs = seg_first + seg;
  const int64_t rs = sstart[gs], t_hi = rs + slen[gs];
  const int ex = sex[gs];
  const int64_t m_base = (int64_t)tile * FT_M_F32;
  const int nkb = (r + 15) >> 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4;

  f32x4_t acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) acc[j][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t t_lo = rs & ~(int64_t)3;
  for (int64_t t0 = t_lo; t0 < t_hi; t0 += 16) {
    const int64_t tb = t0 + 4 * g;
    float bv[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t m = m_base + (2 * wave + j) * 16 + (lane & 15);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t t = tb + q;
        bv[j][q] = (t >= rs && t < t_hi && m < M) ? P[t * ldp + m] : 0.f;
      }
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if (kb < nkb) {
        const int k = kb * 16 + (lane & 15);
        f32x4_t a = *(const f32x4_t*)(Q + (int64_t)k * ldq + tb);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t t = tb + q;
          if (!(t >= rs && t < t_hi)) a[q] = 0.f;
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            acc[j][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], bv[j][q], acc[j][kb], 0, 0, 0);
      }
    }
  }

  const FactorLeaves L = read_leaves(f);
  factor_epilogue<2, 4>(acc, r, scale, M, m_base, seg, tile, ex, part_stride, L, part);
}


}  // namespace

// ---------------------------------------------------------------------------
// A^T operands of the projection: one thread per row k of A, writing
// column k of W row by row (coalesced across the workgroup's threads).
// ---------------------------------------------------------------------------
constexpr int PF_THREADS = 256;

__global__ __launch_bounds__(PF_THREADS) void k_pack_factors(const int64_t* __restrict__ probs,
                                                             const int32_t* __restrict__ ws, int n_prob) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_PF_FIELDS;
  const void* src = (const void*)f[ODP_PF_SRC];
  const int64_t ld0 = f[ODP_PF_LD0], ld1 = f[ODP_PF_LD1], din = f[ODP_PF_DIN];
  const int sdt = (int)(f[ODP_PF_DTYPES] & 0xff), ddt = (int)((f[ODP_PF_DTYPES] >> 8) & 0xff);
  const int r = (int)f[ODP_PF_R];
  void* dst = (void*)f[ODP_PF_DST];
  const int64_t k = (int64_t)(bid - ws[p]) * PF_THREADS + threadIdx.x;
  if (k >= din) return;
  for (int j = 0; j < r; ++j)
    odp_store_from_float(dst, (int64_t)j * din + k, ddt, odp_load_as_float(src, k * ld0 + (int64_t)j * ld1, sdt));
}

extern "C" int64_t odp_pack_factors_blocks(int64_t d_in) {
  return d_in <= 0 ? 0 : (d_in + PF_THREADS - 1) / PF_THREADS;
}

extern "C" int odp_pack_factors(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                                int32_t n_prob, int32_t total_blocks) {
  int rc = odp_check_table("odp_pack_factors", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (total_blocks == 0) return ODP_OK;
  hipLaunchKernelGGL(k_pack_factors, dim3(total_blocks), dim3(PF_THREADS), 0, odp_hip_stream(stream), problems,
                     work_start, n_prob);
  return odp_check_launch("odp_pack_factors");
}

// ---------------------------------------------------------------------------
// Rank-space products from the seam laid out as planes.  A workgroup takes
// PL_THREADS consecutive rows, PL_K columns at a time: each thread reads its
// row's columns (16-byte loads where rows are aligned), the block is
// transposed through LDS, and each plane row leaves as 16-byte pieces of
// consecutive rows.  Rows outside the segments get 0.
// ---------------------------------------------------------------------------
constexpr int PL_THREADS = 256;
constexpr int PL_K = 16;  // plane rows per pass

template <typename T>
__device__ __forceinline__ void pack_planes_tile(const T* __restrict__ src, int64_t lds, T* __restrict__ dst,
                                                 int64_t ldq, int r, int64_t row0, int64_t n_rows, bool in,
                                                 T* __restrict__ tile) {
  constexpr int V = 16 / sizeof(T);       // elements per 16-byte piece
  constexpr int TP = PL_THREADS + V;       // LDS pitch of a plane row
  constexpr int PIECES = PL_THREADS / V;   // 16-byte pieces per plane row
  const int t = threadIdx.x;
  const T* s = src + (row0 + t) * lds;
  const bool vec = (((uintptr_t)src | (uintptr_t)(lds * (int64_t)sizeof(T))) & 15) == 0;
  const bool dvec = (((uintptr_t)dst | (uintptr_t)(ldq * (int64_t)sizeof(T))) & 15) == 0;
  for (int k0 = 0; k0 < r; k0 += PL_K) {
    T e[PL_K];
    if (in && vec && k0 + PL_K <= r) {
#pragma unroll
      for (int q = 0; q < PL_K / V; ++q) {
        const u32x4_t w = ld16(s + k0 + q * V);
        __builtin_memcpy(e + q * V, &w, 16);
      }
    } else {
#pragma unroll
      for (int c = 0; c < PL_K; ++c) e[c] = in && k0 + c < r ? s[k0 + c] : (T)0;
    }
    if (k0 > 0) __syncthreads();  // the previous pass has read the tile
#pragma unroll
    for (int c = 0; c < PL_K; ++c) tile[c * TP + t] = e[c];
    __syncthreads();
#pragma unroll
    for (int i = t; i < PL_K * PIECES; i += PL_THREADS) {
      const int c = i / PIECES, pc = i % PIECES;
      const int64_t r0 = row0 + (int64_t)pc * V;
      if (k0 + c >= r || r0 >= n_rows) continue;
      T* d = dst + (int64_t)(k0 + c) * ldq + r0;
      const T* sp = tile + c * TP + pc * V;
      if (dvec && r0 + V <= n_rows) {
        u32x4_t w;
        __builtin_memcpy(&w, sp, 16);
        odp_gstore((u32x4_t*)d, w);
      } else {
        for (int q = 0; q < V && r0 + q < n_rows; ++q) odp_gstore(d + q, sp[q]);
      }
    }
  }
}

__global__ __launch_bounds__(PL_THREADS) void k_pack_planes(const int64_t* __restrict__ probs,
                                                            const int32_t* __restrict__ ws, int n_prob,
                                                            const int32_t* __restrict__ sstart,
                                                            const int32_t* __restrict__ slen) {
  __shared__ __attribute__((aligned(16))) uint32_t tile[PL_K * (PL_THREADS + 4)];  // f32: pitch 260
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_PL_FIELDS;
  const int64_t n_rows = f[ODP_PL_NROWS];
  const int64_t row0 = (int64_t)(bid - ws[p]) * PL_THREADS, row = row0 + threadIdx.x;
  const int seg_first = (int)f[ODP_PL_SEG_FIRST];
  const bool in = row < n_rows &&
                  odp_row_in_segments(row, sstart + seg_first, slen + seg_first, (int)f[ODP_PL_NSEG]);
  const int64_t lds = f[ODP_PL_LDS], ldq = f[ODP_PL_LDQ];
  const int r = (int)f[ODP_PL_R];
  if (f[ODP_PL_DTYPE] == ODP_DTYPE_BF16)
    pack_planes_tile((const uint16_t*)f[ODP_PL_SRC], lds, (uint16_t*)f[ODP_PL_DST], ldq, r, row0, n_rows, in,
                     (uint16_t*)tile);
  else
    pack_planes_tile((const float*)f[ODP_PL_SRC], lds, (float*)f[ODP_PL_DST], ldq, r, row0, n_rows, in,
                     (float*)tile);
}

extern "C" int64_t odp_pack_planes_blocks(int64_t n_rows) {
  return n_rows <= 0 ? 0 : (n_rows + PL_THREADS - 1) / PL_THREADS;
}

extern "C" int odp_pack_planes(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                               int32_t n_prob, int32_t total_blocks, const int32_t* seg_row_start,
                               const int32_t* seg_row_len) {
  int rc = odp_check_table("odp_pack_planes", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr) {
    odp_set_error("odp_pack_planes: null segment arrays");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_pack_planes, dim3(total_blocks), dim3(PL_THREADS), 0, odp_hip_stream(stream), problems,
                     work_start, n_prob, seg_row_start, seg_row_len);
  return odp_check_launch("odp_pack_planes");
}

extern "C" int64_t odp_project_covered_rows(const int32_t* seg_row_start, const int32_t* seg_row_len,
                                            int32_t n_seg) {
  if (n_seg > 0 && (seg_row_start == nullptr || seg_row_len == nullptr)) {
    odp_set_error("odp_project_covered_rows: null segment arrays");
    return -1;
  }
  int64_t cov = 0;
  for (int32_t s = 0; s < n_seg; ++s) {
    const int64_t st = seg_row_start[s], ln = seg_row_len[s];
    if (ln > 0) cov += ((st + ln + 7) & ~(int64_t)7) - (st & ~(int64_t)7);
  }
  return cov;
}

extern "C" int64_t odp_project_blocks(int dtype, int64_t n_rows, int32_t r) {
  (void)r;
  const int64_t rows = dtype == ODP_DTYPE_BF16 ? PS_ROWS : PJ_ROWS;
  return n_rows <= 0 ? 0 : (n_rows + rows - 1) / rows;
}

extern "C" int64_t odp_seg_factor_tiles(int dtype, int64_t M, int32_t r) {
  if (M <= 0 || r <= 0) return 0;
  const int64_t mt = dtype == ODP_DTYPE_BF16 ? 64 * ft_nj((r + 15) / 16) : FT_M_F32;
  return (M + mt - 1) / mt;
}

extern "C" int odp_project(odp_stream_t stream, int dtype, const int64_t* problems,
                           const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                           const int32_t* seg_row_start, const int32_t* seg_row_len, int32_t nkb) {
  int rc = odp_check_table("odp_project", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (dtype != ODP_DTYPE_BF16 && dtype != ODP_DTYPE_F32) {
    odp_set_error("odp_project: unsupported dtype %d", dtype);
    return ODP_ERR_UNSUPPORTED;
  }
  if (nkb < 1 || nkb > 4) {
    odp_set_error("odp_project: nkb=%d outside [1, 4] (rank must be <= 64)", nkb);
    return ODP_ERR_UNSUPPORTED;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr) {
    odp_set_error("odp_project: null segment arrays");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = odp_hip_stream(stream);
  const dim3 grid(total_blocks), block(256);
  if (dtype == ODP_DTYPE_BF16) {
    switch (nkb) {
      case 1: hipLaunchKernelGGL(k_project_stream_bf16<1>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len); break;
      case 2: hipLaunchKernelGGL(k_project_stream_bf16<2>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len); break;
      case 3: hipLaunchKernelGGL(k_project_stream_bf16<3>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len); break;
      default: hipLaunchKernelGGL(k_project_stream_bf16<4>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len); break;
    }
  } else {
    hipLaunchKernelGGL(k_project_f32, grid, block, 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len);
  }
  return odp_check_launch("odp_project");
}

extern "C" int64_t odp_factor_project_max_len(void) { return (int64_t)FP_STEPS * FP_T - 7; }

extern "C" int odp_seg_factor_project(odp_stream_t stream, const int64_t* problems,
                                      const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                                      const int32_t* seg_row_start, const int32_t* seg_row_len,
                                      const int32_t* seg_example, double* part, int64_t part_stride) {
  int rc = odp_check_table("odp_seg_factor_project", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr ||
      part == nullptr || part_stride <= 0) {
    odp_set_error("odp_seg_factor_project: null segment/partial arrays or part_stride <= 0");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  static_assert(FP_MT == 64 * ODP_FT_NJ, "chunks must match the bf16 factor tiles (partial slots)");
  hipLaunchKernelGGL(k_factor_project_bf16, dim3(total_blocks), dim3(256), 0, odp_hip_stream(stream),
                     problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part,
                     part_stride);
  return odp_check_launch("odp_seg_factor_project");
}

extern "C" int64_t odp_seg_factor_stream_groups(int64_t M) {
  return M <= 0 ? 0 : fs_groups((int)((M + FP_MT - 1) / FP_MT));
}

extern "C" int odp_seg_factor_stream(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                                     int32_t n_prob, int32_t total_blocks, const int32_t* seg_row_start,
                                     const int32_t* seg_row_len, const int32_t* seg_example, double* part,
                                     int64_t part_stride, int32_t nkb) {
  int rc = odp_check_table("odp_seg_factor_stream", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (nkb < 1 || nkb > 3) {
    odp_set_error("odp_seg_factor_stream: nkb=%d outside [1, 3]", nkb);
    return ODP_ERR_UNSUPPORTED;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr ||
      part == nullptr || part_stride <= 0) {
    odp_set_error("odp_seg_factor_stream: null segment/partial arrays or part_stride <= 0");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = odp_hip_stream(stream);
  const dim3 grid(total_blocks), block(256);
  switch (nkb) {
    case 1: hipLaunchKernelGGL(k_factor_stream_bf16<1>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride); break;
    case 2: hipLaunchKernelGGL(k_factor_stream_bf16<2>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride); break;
    default: hipLaunchKernelGGL(k_factor_stream_bf16<3>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride); break;
  }
  return odp_check_launch("odp_seg_factor_stream");
}

extern "C" int odp_seg_factor(odp_stream_t stream, int dtype, const int64_t* problems,
                              const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                              const int32_t* seg_row_start, const int32_t* seg_row_len,
                              const int32_t* seg_example, double* part, int64_t part_stride,
                              int32_t nkb) {
  int rc = odp_check_table("odp_seg_factor", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (dtype != ODP_DTYPE_BF16 && dtype != ODP_DTYPE_F32) {
    odp_set_error("odp_seg_factor: unsupported dtype %d", dtype);
    return ODP_ERR_UNSUPPORTED;
  }
  if (nkb < 1 || nkb > 4) {
    odp_set_error("odp_seg_factor: nkb=%d outside [1, 4] (rank must be <= 64)", nkb);
    return ODP_ERR_UNSUPPORTED;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr ||
      part == nullptr || part_stride <= 0) {
    odp_set_error("odp_seg_factor: null segment/partial arrays or part_stride <= 0");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = odp_hip_stream(stream);
  const dim3 grid(total_blocks), block(256);
  if (dtype == ODP_DTYPE_BF16) {
    switch (nkb) {
      case 1: hipLaunchKernelGGL(k_factor_bf16<1>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride); break;
      case 2: hipLaunchKernelGGL(k_factor_bf16<2>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride); break;
      case 3: hipLaunchKernelGGL(k_factor_bf16<3>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride); break;
      default: hipLaunchKernelGGL(k_factor_bf16<4>, grid, block, 0, s, problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride); break;
    }
  } else {
    hipLaunchKernelGGL(k_factor_f32, grid, block, 0, s, problems, work_start, n_prob,
                       seg_row_start, seg_row_len, seg_example, part, part_stride);
  }
  return odp_check_launch("odp_seg_factor");
}
