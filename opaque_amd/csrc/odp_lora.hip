// LoRA per-example factor gradients and their squared norms on CDNA4 MFMA.
//
// A LoRA adapter y = x W^T + s (x A) B has per-example factor gradients
//   dA_i = s X_i^T U_i,  U = G B^T        (d_in x r)
//   dB_i = s V_i^T G_i,  V = X A          (r x d_out)
// (reference: opaque-patches/.../kernels/lora.py:164-176, where they are
// materialised with torch.bmm under vmap).  Both are skinny products whose
// long dimension is a row of X or G, so the work is HBM-bound: each kernel
// streams X or G and keeps the rank-r side (U, V, the r x M output tile) on
// chip.  Both kernels keep two pipeline steps of loads in flight per wave so
// that enough bytes are outstanding per CU to approach HBM bandwidth.
//
//   k_project_*  : Q^T = (P W^T)^T for every row of a segment      (U, V)
//   k_factor_*   : pe[s] = s * Q_s^T P_s per segment, plus fp64 sums of
//                  squares per leaf and M-tile                   (dA, dB)
#include "odp_internal.h"

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

namespace {

constexpr int PJ_ROWS = 64;             // rows per project workgroup (4 waves x 16)
constexpr int PJ_KS = 128;              // contraction elements per bf16 pipeline step
constexpr int PJ_WPITCH = PJ_KS + 8;    // u16 per staged W row
constexpr int FT_M = 128;               // M columns per factor workgroup
constexpr int FT_T = 32;                // tokens per bf16 factor step (MFMA K)
constexpr int FT_PP = FT_M + 4;         // u16 pitch of the staged P tile [t][m]
constexpr int FT_QP = FT_T + 8;         // u16 pitch of the staged Q tile [k][t]
constexpr int FT_QROWS = 64;            // staged Q rows per plane (r <= 64)
constexpr int FT_PTILE = FT_T * FT_PP;  // u16 per staged P tile
constexpr int FT_STAGE = FT_PTILE + 2 * FT_QROWS * FT_QP;

__device__ __forceinline__ u32x4_t ld16(const void* p) { return *(const u32x4_t*)p; }

// ---------------------------------------------------------------------------
// Projection, bf16: MFMA 16x16x32 bf16 with fp32 accumulation.  Each wave
// owns 16 rows and the full contraction; P rows feed the MFMA A operand
// straight from global memory (row-major P already has the K-contiguous
// layout the operand needs), W is staged through LDS once per workgroup per
// 128-wide step.  Loads of step s+1 are issued before step s is computed.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_project_bf16(const int64_t* __restrict__ probs,
                                                      const int32_t* __restrict__ ws, int n_prob,
                                                      const int32_t* __restrict__ sstart,
                                                      const int32_t* __restrict__ slen) {
  extern __shared__ __attribute__((aligned(16))) uint16_t wlds[];  // [2][rp][PJ_WPITCH]
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_PJ_FIELDS;
  const uint16_t* P = (const uint16_t*)f[ODP_PJ_P];
  const int64_t ldp = f[ODP_PJ_LDP], d = f[ODP_PJ_D];
  const uint16_t* W = (const uint16_t*)f[ODP_PJ_W];
  const int r = (int)f[ODP_PJ_R];
  uint16_t* Q = (uint16_t*)f[ODP_PJ_Q];
  uint16_t* Qlo = (uint16_t*)f[ODP_PJ_QLO];
  const int64_t ldq = f[ODP_PJ_LDQ], n_rows = f[ODP_PJ_NROWS];
  const int seg_first = (int)f[ODP_PJ_SEG_FIRST], n_seg = (int)f[ODP_PJ_NSEG];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = (int64_t)(bid - ws[p]) * PJ_ROWS + 16 * wave;
  const int64_t my_row = row0 + (lane & 15);
  const bool valid = my_row < n_rows &&
                     odp_row_in_segments(my_row, sstart + seg_first, slen + seg_first, n_seg);
  if (!__syncthreads_or(valid ? 1 : 0)) return;  // whole block is padding

  const int nkb = (r + 15) >> 4, rp = nkb * 16;
  const int kq = (lane >> 4) * 8;
  const uint16_t* prow = P + (valid ? my_row : 0) * ldp;
  const int64_t nsteps = (d + PJ_KS - 1) / PJ_KS;

  f32x4_t acc[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) acc[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto load_p = [&](int64_t s, u32x4_t(&pa)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = s * PJ_KS + 32 * i + kq;
      pa[i] = (valid && k < d) ? ld16(prow + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto load_w = [&](int64_t s, u32x4_t(&wr)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int id = tid + 256 * q;
      const int row = id >> 4, col = (id & 15) * 8;
      const int64_t k = s * PJ_KS + col;
      wr[q] = (row < r && k < d) ? ld16(W + (int64_t)row * d + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store_w = [&](int b, const u32x4_t(&wr)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int id = tid + 256 * q;
      if (id < rp * 16) {
        const int row = id >> 4, col = (id & 15) * 8;
        *(u32x4_t*)&wlds[(b * rp + row) * PJ_WPITCH + col] = wr[q];
      }
    }
  };
  auto compute = [&](int b, const u32x4_t(&pa)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x8_t a = __builtin_bit_cast(bf16x8_t, pa[i]);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        if (kb < nkb) {
          const u32x4_t bv = *(const u32x4_t*)&wlds[(b * rp + kb * 16 + (lane & 15)) * PJ_WPITCH + 32 * i + kq];
          acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, bv),
                                                            acc[kb], 0, 0, 0);
        }
      }
    }
  };

  u32x4_t pa0[4], pa1[4], wr[4];
  load_p(0, pa0);
  load_w(0, wr);
  for (int64_t s = 0; s < nsteps; s += 2) {
    store_w(0, wr);
    __syncthreads();
    if (s + 1 < nsteps) {
      load_p(s + 1, pa1);
      load_w(s + 1, wr);
    }
    compute(0, pa0);
    if (s + 1 >= nsteps) break;
    store_w(1, wr);
    __syncthreads();
    if (s + 2 < nsteps) {
      load_p(s + 2, pa0);
      load_w(s + 2, wr);
    }
    compute(1, pa1);
  }

  // lane holds D[4*(lane>>4) + i][lane & 15] of each 16x16 block
  const int64_t rb = row0 + 4 * (lane >> 4);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int col = kb * 16 + (lane & 15);
    if (kb < nkb && col < r) {
      uint16_t* qhi = Q + (int64_t)col * ldq;
      uint16_t* qlo = Qlo + (int64_t)col * ldq;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (rb + i < n_rows) {
          const uint16_t h = odp_f2bf(acc[kb][i]);
          qhi[rb + i] = h;
          qlo[rb + i] = odp_f2bf(acc[kb][i] - odp_bf2f(h));
        }
      }
    }
  }
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
  if (!__syncthreads_or(valid ? 1 : 0)) return;
  const int nkb = (r + 15) >> 4;
  const int kq = (lane >> 4) * 4;
  const float* prow = P + (valid ? my_row : 0) * ldp;

  f32x4_t acc[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) acc[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = kq; k0 < d; k0 += 16) {
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
  const int64_t rb = row0 + 4 * (lane >> 4);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int col = kb * 16 + (lane & 15);
    if (kb < nkb && col < r) {
      float* q = Q + (int64_t)col * ldq;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (rb + i < n_rows) q[rb + i] = acc[kb][i];
    }
  }
}

// Shared epilogue of the factor kernels: scale, store per-leaf rows, and
// reduce the squared values per leaf in a fixed order.
struct FactorLeaves {
  int n;
  float* pe[4];
  int col0[4];
  int rank[4];
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
    L.slot[l] = on ? g[2] : 0;
  }
  return L;
}

__device__ __forceinline__ void factor_epilogue(const f32x4_t (&acc)[2][4], int nkb, int r,
                                                float scale, int64_t M, int64_t m_base,
                                                int seg, int tile, int ex, int64_t part_stride,
                                                const FactorLeaves& L, double* __restrict__ part) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __shared__ double colsq[4][64];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    if (kb >= nkb) continue;
    double cs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cs[i] = 0.0;
      const int k = kb * 16 + 4 * (lane >> 4) + i;
      if (k >= r) continue;
      int l = 0;
#pragma unroll
      for (int q = 1; q < 4; ++q)
        if (q < L.n && k >= L.col0[q]) l = q;
      // Columns of frozen factors between leaves belong to no leaf.
      if (k < L.col0[l] || k - L.col0[l] >= L.rank[l]) continue;
      float* dst = L.pe[l] + ((int64_t)seg * L.rank[l] + (k - L.col0[l])) * M;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t m = m_base + (2 * wave + j) * 16 + (lane & 15);
        if (m < M) {
          const float v = scale * acc[j][kb][i];
          dst[m] = v;
          // Non-finite entries count as 0 (nan_to_num); squares are taken
          // in fp32 like the reference's float32 accumulation dtype.
          const float vf = isfinite(v) ? v : 0.f;
          cs[i] += (double)__fmul_rn(vf, vf);
        }
      }
    }
    // Sum over the 16 lanes that share a column (same lane >> 4).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      double v = cs[i];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      v += __shfl_xor(v, 8);
      if ((lane & 15) == 0) colsq[wave][kb * 16 + 4 * (lane >> 4) + i] = v;
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < L.n) {
    double total = 0.0;
    for (int k = L.col0[t]; k < L.col0[t] + L.rank[t]; ++k)
      for (int w = 0; w < 4; ++w) total += colsq[w][k];
    part[(int64_t)ex * part_stride + L.slot[t] + tile] = total;
  }
}

// ---------------------------------------------------------------------------
// Factor gradients, bf16 P: MFMA 16x16x32 with K = 32 tokens.  Per step the
// workgroup stages the P tile [32 tokens x 128 m] and the Q^T tile (hi and
// lo planes, [rp x 32 tokens]) through LDS; each lane then gathers its 8
// consecutive tokens of one column for the B operand.  Two steps of loads
// are in flight while a third is computed.
// ---------------------------------------------------------------------------
struct FactorStage {
  u32x4_t p[2];
  u32x4_t q[2];
};

__global__ __launch_bounds__(256, 4) void k_factor_bf16(const int64_t* __restrict__ probs,
                                                     const int32_t* __restrict__ ws, int n_prob,
                                                     const int32_t* __restrict__ sstart,
                                                     const int32_t* __restrict__ slen,
                                                     const int32_t* __restrict__ sex,
                                                     double* __restrict__ part, int64_t part_stride) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * FT_STAGE];
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_FT_FIELDS;
  const uint16_t* P = (const uint16_t*)f[ODP_FT_P];
  const int64_t ldp = f[ODP_FT_LDP], M = f[ODP_FT_M];
  const uint16_t* Q = (const uint16_t*)f[ODP_FT_Q];
  const uint16_t* Qlo = (const uint16_t*)f[ODP_FT_QLO];
  const int64_t ldq = f[ODP_FT_LDQ];
  const int r = (int)f[ODP_FT_R];
  const int seg_first = (int)f[ODP_FT_SEG_FIRST];
  const float scale = (float)__longlong_as_double(f[ODP_FT_SCALING]);

  const int ntile = (int)((M + FT_M - 1) / FT_M);
  const int local = bid - ws[p];
  const int seg = local / ntile, tile = local % ntile;
  const int gs = seg_first + seg;
  const int64_t rs = sstart[gs], t_hi = rs + slen[gs];
  const int ex = sex[gs];
  const int64_t m_base = (int64_t)tile * FT_M;
  const int nkb = (r + 15) >> 4, rp = nkb * 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t_lo = rs & ~(int64_t)7;
  const int64_t nchunk = t_hi > rs ? (t_hi - t_lo + FT_T - 1) / FT_T : 0;

  auto load = [&](int64_t c, FactorStage& S) {
    const int64_t t0 = t_lo + c * FT_T;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int id = tid + 256 * ps;
      const int64_t t = t0 + (id >> 4);
      const int64_t m = m_base + (id & 15) * 8;
      S.p[ps] = (t >= rs && t < t_hi && m < M) ? ld16(P + t * ldp + m) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int id = tid + 256 * ps;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (id < 8 * rp) {
        const int plane = id / (4 * rp), rem = id - plane * 4 * rp;
        const int row = rem >> 2, pc = rem & 3;
        const int64_t tq = t0 + 8 * pc;
        v = ld16((plane ? Qlo : Q) + (int64_t)row * ldq + tq);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int64_t ta = tq + 2 * w;
          const uint32_t lo_ok = (ta >= rs && ta < t_hi) ? 0x0000ffffu : 0u;
          const uint32_t hi_ok = (ta + 1 >= rs && ta + 1 < t_hi) ? 0xffff0000u : 0u;
          v[w] &= lo_ok | hi_ok;
        }
      }
      S.q[ps] = v;
    }
  };
  auto store = [&](int b, const FactorStage& S) {
    uint16_t* st = lds + b * FT_STAGE;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int id = tid + 256 * ps;
      u32x2_t* dst = (u32x2_t*)&st[(id >> 4) * FT_PP + (id & 15) * 8];
      dst[0] = u32x2_t{S.p[ps][0], S.p[ps][1]};
      dst[1] = u32x2_t{S.p[ps][2], S.p[ps][3]};
    }
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const int id = tid + 256 * ps;
      if (id < 8 * rp) {
        const int plane = id / (4 * rp), rem = id - plane * 4 * rp;
        const int row = rem >> 2, pc = rem & 3;
        *(u32x4_t*)&st[FT_PTILE + (plane * FT_QROWS + row) * FT_QP + 8 * pc] = S.q[ps];
      }
    }
  };

  f32x4_t acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) acc[j][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int b) {
    const uint16_t* st = lds + b * FT_STAGE;
    bf16x8_t bop[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = (2 * wave + j) * 16 + (lane & 15);
      const uint16_t* col = st + (8 * (lane >> 4)) * FT_PP + m;
      u32x4_t v;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        v[w] = (uint32_t)col[(2 * w) * FT_PP] | ((uint32_t)col[(2 * w + 1) * FT_PP] << 16);
      bop[j] = __builtin_bit_cast(bf16x8_t, v);
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if (kb < nkb) {
        const int row = kb * 16 + (lane & 15);
        const u32x4_t hv = *(const u32x4_t*)&st[FT_PTILE + row * FT_QP + 8 * (lane >> 4)];
        const u32x4_t lv = *(const u32x4_t*)&st[FT_PTILE + (FT_QROWS + row) * FT_QP + 8 * (lane >> 4)];
        const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, hv);
        const bf16x8_t al = __builtin_bit_cast(bf16x8_t, lv);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[j][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bop[j], acc[j][kb], 0, 0, 0);
          acc[j][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bop[j], acc[j][kb], 0, 0, 0);
        }
      }
    }
  };

  FactorStage SA, SB;
  if (nchunk > 0) load(0, SA);
  if (nchunk > 1) load(1, SB);
  for (int64_t c = 0; c < nchunk; c += 2) {
    store(0, SA);
    __syncthreads();
    if (c + 2 < nchunk) load(c + 2, SA);
    compute(0);
    if (c + 1 >= nchunk) break;
    store(1, SB);
    __syncthreads();
    if (c + 3 < nchunk) load(c + 3, SB);
    compute(1);
  }

  const FactorLeaves L = read_leaves(f);
  factor_epilogue(acc, nkb, r, scale, M, m_base, seg, tile, ex, part_stride, L, part);
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

  const int ntile = (int)((M + FT_M - 1) / FT_M);
  const int local = bid - ws[p];
  const int seg = local / ntile, tile = local % ntile;
  const int gs = seg_first + seg;
  const int64_t rs = sstart[gs], t_hi = rs + slen[gs];
  const int ex = sex[gs];
  const int64_t m_base = (int64_t)tile * FT_M;
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
  factor_epilogue(acc, nkb, r, scale, M, m_base, seg, tile, ex, part_stride, L, part);
}

}  // namespace

extern "C" int64_t odp_project_blocks(int64_t n_rows) {
  return n_rows <= 0 ? 0 : (n_rows + PJ_ROWS - 1) / PJ_ROWS;
}

extern "C" int64_t odp_seg_factor_tiles(int64_t M) {
  return M <= 0 ? 0 : (M + FT_M - 1) / FT_M;
}

extern "C" int odp_project(odp_stream_t stream, int dtype, const int64_t* problems,
                           const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                           const int32_t* seg_row_start, const int32_t* seg_row_len,
                           int32_t max_rank) {
  int rc = odp_check_table("odp_project", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (dtype != ODP_DTYPE_BF16 && dtype != ODP_DTYPE_F32) {
    odp_set_error("odp_project: unsupported dtype %d", dtype);
    return ODP_ERR_UNSUPPORTED;
  }
  if (max_rank < 1 || max_rank > 64) {
    odp_set_error("odp_project: max_rank=%d outside [1, 64]", max_rank);
    return ODP_ERR_UNSUPPORTED;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr) {
    odp_set_error("odp_project: null segment arrays");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = odp_hip_stream(stream);
  if (dtype == ODP_DTYPE_BF16) {
    const size_t lds = (size_t)2 * ((max_rank + 15) / 16 * 16) * PJ_WPITCH * sizeof(uint16_t);
    hipLaunchKernelGGL(k_project_bf16, dim3(total_blocks), dim3(256), lds, s, problems, work_start,
                       n_prob, seg_row_start, seg_row_len);
  } else {
    hipLaunchKernelGGL(k_project_f32, dim3(total_blocks), dim3(256), 0, s, problems, work_start,
                       n_prob, seg_row_start, seg_row_len);
  }
  return odp_check_launch("odp_project");
}

extern "C" int odp_seg_factor(odp_stream_t stream, int dtype, const int64_t* problems,
                              const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                              const int32_t* seg_row_start, const int32_t* seg_row_len,
                              const int32_t* seg_example, double* part, int64_t part_stride) {
  int rc = odp_check_table("odp_seg_factor", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (dtype != ODP_DTYPE_BF16 && dtype != ODP_DTYPE_F32) {
    odp_set_error("odp_seg_factor: unsupported dtype %d", dtype);
    return ODP_ERR_UNSUPPORTED;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr ||
      part == nullptr || part_stride <= 0) {
    odp_set_error("odp_seg_factor: null segment/partial arrays or part_stride <= 0");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = odp_hip_stream(stream);
  if (dtype == ODP_DTYPE_BF16)
    hipLaunchKernelGGL(k_factor_bf16, dim3(total_blocks), dim3(256), 0, s, problems, work_start,
                       n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride);
  else
    hipLaunchKernelGGL(k_factor_f32, dim3(total_blocks), dim3(256), 0, s, problems, work_start,
                       n_prob, seg_row_start, seg_row_len, seg_example, part, part_stride);
  return odp_check_launch("odp_seg_factor");
}
