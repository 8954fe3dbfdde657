// The outer-product MFMA pipeline shared by the full-weight kernels: operand
// tiles of G and X staged by buffer loads straight into a ring of LDS stages,
// consumed by bf16 MFMA 16x16x32 into per-wave accumulator blocks.
//
// Included inside an anonymous namespace by each kernel source, after
// odp_internal.h.  The tile shape comes from macros a source may set before
// the include: ODP_LIN_OM x ODP_LIN_ON output tile (default 256 x 256),
// ODP_LIN_WAVES waves (default 8), ODP_LIN_RING stages (default 4),
// ODP_LIN_OCC waves per SIMD (default 2).  Each source thereby compiles its
// own copy of the pipeline for its own tile.
#pragma once

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// The same 16 bytes read from memory last written as other types (a tile
// staged element by element in LDS): may_alias keeps the compiler from
// moving the read above those writes.
typedef u32x4_t u32x4_alias_t __attribute__((may_alias));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short v4i16_t __attribute__((ext_vector_type(4)));

#ifndef ODP_LIN_OCC
#define ODP_LIN_OCC 2  // waves per SIMD the outer-product kernels are compiled for
#endif

#define ODP_GLOBAL __attribute__((address_space(1)))
#define ODP_LDS __attribute__((address_space(3)))
#define ODP_CONST __attribute__((address_space(4)))
__device__ __forceinline__ v4i16_t lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((ODP_LDS v4i16_t*)(ODP_LDS void*)p);
}

// Whether local segment sg (len rows) of problem f may overflow float32 in
// the Gram or clipped-sum forms: with a = max|x| and b = max|g| over the
// segment's finite entries (odp_nonfinite_columns), a b max(L, sqrt(d_in
// d_out)) >= 2^60, d_in a^2 >= 2^124 or d_out b^2 >= 2^124.  False without
// the per-segment maxima (no check requested).
__device__ __forceinline__ bool lin_seg_at_risk(const int64_t* f, int sg, int32_t len, int64_t d_in,
                                                int64_t d_out) {
  const uint32_t* xa = (const uint32_t*)f[ODP_LN_XAMAX];
  const uint32_t* ga = (const uint32_t*)f[ODP_LN_GAMAX];
  if (xa == nullptr || ga == nullptr || len <= 0) return false;
  const double a = (double)__uint_as_float(xa[sg]), b = (double)__uint_as_float(ga[sg]);
  const double din = (double)d_in, dout = (double)d_out;
  const double w = fmax((double)len, sqrt(din * dout));
  return a * b * w >= 0x1p60 || din * a * a >= 0x1p124 || dout * b * b >= 0x1p124;
}

// Whether any segment of the problem is at risk.
__device__ __forceinline__ bool lin_problem_at_risk(const int64_t* f, const int32_t* slen, int seg_first,
                                                    int n_seg, int64_t d_in, int64_t d_out) {
  if (f[ODP_LN_XAMAX] == 0 || f[ODP_LN_GAMAX] == 0) return false;
  for (int sg = 0; sg < n_seg; ++sg)
    if (lin_seg_at_risk(f, sg, slen[seg_first + sg], d_in, d_out)) return true;
  return false;
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
// Outer-product main loop.  The workgroup's tile covers OM output rows (o,
// columns of G) by ON output columns (n, columns of X); NW waves in a
// 2 x (NW / 2) arrangement each own a WM x WN block as BI x BJ MFMA 16 x 16
// blocks.  A pipeline step stages OK tokens of both operands as token-major
// LDS tiles.  256 x 256 tiles of eight 128 x 64 waves (one workgroup and two
// waves per SIMD per CU) move a third less data from L2 into LDS per flop
// than 256 x 128 tiles of four, at the same registers per wave; the loads
// into LDS, not the MFMAs or the LDS reads, bound these kernels.
// ---------------------------------------------------------------------------
#ifndef ODP_LIN_OM
#define ODP_LIN_OM 256
#endif
#ifndef ODP_LIN_ON
#define ODP_LIN_ON 256
#endif
#ifndef ODP_LIN_WAVES
#define ODP_LIN_WAVES 8  // waves per workgroup, 2 x (NW / 2) over the tile
#endif
constexpr int OM = ODP_LIN_OM, ON = ODP_LIN_ON, OK = 32, NW = ODP_LIN_WAVES, OUTER_THREADS = 64 * NW;
constexpr int WM = OM / 2, WN = ON / (NW / 2), BI = WM / 16, BJ = WN / 16;
constexpr int A_TILE = OK * OM, B_TILE = OK * ON;  // elements
constexpr int OUTER_STAGE = A_TILE + B_TILE;


// Token-major tiles are unpadded and XOR-swizzled in 4-element (8-byte)
// chunks: chunk k of row r lives at chunk k ^ swz(r).  The 16 rows x 4
// chunks that one transposing operand read touches (rows 8g + j, j < 4,
// g < 4) then land on every LDS bank exactly twice, and a 16-byte piece
// (an aligned chunk pair) stays contiguous.
__device__ __forceinline__ int swz(int row) { return ((row & 3) | ((row >> 1) & 4)) << 2; }


// 16 columns col0.. of a token-major tile of row pitch `pitch`, tokens
// 8 (lane >> 4) + 0..7: the MFMA operand layout (lane & 15 = row of A /
// column of B).  Rows r and r + 4 share swz(), so the second read is
// 4 rows further on.
__device__ __forceinline__ bf16x8_t outer_frag(const uint16_t* tile, int pitch, int col0) {
  const int lane = threadIdx.x & 63, c = lane & 15;
  const int row = 8 * (lane >> 4) + (c >> 2);
  const int k = (col0 >> 2) + (c & 3);
  const uint16_t* src = tile + row * pitch + 4 * (k ^ swz(row));
  const v4i16_t t0 = lds_tr16(src), t1 = lds_tr16(src + 4 * pitch);
  const v4i16_t tt[2] = {t0, t1};
  return __builtin_bit_cast(bf16x8_t, tt);
}

typedef f32x4_t OuterAcc[BI][BJ];

__device__ __forceinline__ void outer_compute(const uint16_t* ta, const uint16_t* tb, OuterAcc& acc) {
  const int wave = threadIdx.x >> 6;
  const int wm = WM * (wave & 1), wn = WN * (wave >> 1);
  // Operand reads run two A fragments ahead of the MFMAs that consume them.
  bf16x8_t b[BJ], a[3];
#pragma unroll
  for (int j = 0; j < BJ; ++j) b[j] = outer_frag(tb, ON, wn + 16 * j);
  a[0] = outer_frag(ta, OM, wm);
  a[1] = outer_frag(ta, OM, wm + 16);
#pragma unroll
  for (int i = 0; i < BI; ++i) {
    if (i + 2 < BI) a[(i + 2) % 3] = outer_frag(ta, OM, wm + 16 * (i + 2));
#pragma unroll
    for (int j = 0; j < BJ; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i % 3], b[j], acc[i][j], 0, 0, 0);
  }
}

// One pipeline step: rows [t0, t0 + OK) clipped to its segment [tb, te).
// `fix`: the segment has non-finite columns inside the tile, which the step
// zeroes in LDS before its MFMAs.  Plain 32-bit fields (row counts stay
// below 2^31): a struct of mixed widths and a bool was kept in memory by
// the compiler when copied conditionally.
struct Step {
  int32_t t0, tb, te, seg, live, fix;
};

// Element (r, c) of a token-major tile of row pitch `pitch` (the XOR swizzle
// above).
__device__ __forceinline__ int tile_at(int r, int c, int pitch) {
  return r * pitch + 4 * ((c >> 2) ^ swz(r)) + (c & 3);
}

// Bit `c` of a segment's column mask (uint32 words, bit j of word w =
// column 32 w + j).
__device__ __forceinline__ bool mask_bit(const uint32_t* m, int64_t c) {
  return (m[c >> 5] >> (c & 31)) & 1u;
}

typedef float f32x8_t __attribute__((ext_vector_type(8)));

// c * v for 8 bf16 values: widened exactly, multiplied in fp32 and rounded
// to nearest-even bf16 (v_cvt_pk_bf16_f32).
__device__ __forceinline__ u32x4_t scale_bf16x8(u32x4_t v, float c) {
  f32x8_t f = __builtin_convertvector(__builtin_bit_cast(bf16x8_t, v), f32x8_t);
  f = f * c;
  return __builtin_bit_cast(u32x4_t, __builtin_convertvector(f, bf16x8_t));
}


// ---------------------------------------------------------------------------
// Outer-product main loop, buffer loads straight into LDS.  The step's G and
// X tiles (token-major rows, the XOR swizzle above) are fetched by
// buffer_load ... lds into a ring of RING LDS stages, RING - 1 steps ahead of
// the compute, with no staging registers; each step waits for its own loads
// with an explicit vmcnt and an LDS-only barrier.  The buffer resources
// cover only the rows of the step's segment, so rows outside it (and
// columns past the matrix, sent past the end) arrive as zeros.  A step never
// crosses a segment, so the clip factor is one scalar per step; it scales
// X's fragments after the LDS read (c * x rounded to bf16).
// ---------------------------------------------------------------------------
constexpr uint32_t LIN_BUF_DWORD3 = 0x00020000;  // raw 32-bit dwords (CDNA buffer resource)
constexpr uint32_t LIN_OOB = 0x80000000u;        // an offset past every buffer's end
constexpr int A_DMA = A_TILE * 2 / 1024 / NW;     // 1 KB loads per wave per step (G tile)
constexpr int B_DMA = B_TILE * 2 / 1024 / NW;     // (X tile)
constexpr int RPW = OK / NW;                      // tile rows each wave loads per step
#ifndef ODP_LIN_RING
#define ODP_LIN_RING 4  // LDS stages of the outer-form ring (RING - 1 steps in flight)
#endif
constexpr int RING = ODP_LIN_RING;
static_assert((RING == 3 || RING == 4) && (RING - 2) * (A_DMA + B_DMA) < 64, "ring depth");
constexpr int DMA_PER_STEP = A_DMA + B_DMA;
constexpr int B_LPR = ON / 8, B_RPI = 64 / B_LPR;  // X tile: lanes per row, rows per load
static_assert(OM == 256 && (ON == 128 || ON == 256), "G tile rows take 32 lanes; X tile rows 16 or 32");
static_assert((NW == 4 || NW == 8) && A_DMA * 2 == RPW && B_DMA * B_RPI == RPW && WN % 16 == 0,
              "each wave loads whole rows of both tiles");
static_assert(DMA_PER_STEP < 16, "the step wait encodes vmcnt in 4 bits");

// Column-major over the wave's blocks: X fragment j + 1 is scaled (VALU)
// while the MFMAs of fragment j run, instead of all scaling up front.
__device__ __forceinline__ void outer_compute_scaled(const uint16_t* ta, const uint16_t* tb, float c,
                                                     OuterAcc& acc) {
  const int wave = threadIdx.x >> 6;
  const int wm = WM * (wave & 1), wn = WN * (wave >> 1);
  bf16x8_t a[BI], b[BJ];
#pragma unroll
  for (int j = 0; j < BJ; ++j) b[j] = outer_frag(tb, ON, wn + 16 * j);
#pragma unroll
  for (int i = 0; i < BI; ++i) a[i] = outer_frag(ta, OM, wm + 16 * i);
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    const bf16x8_t bs = __builtin_bit_cast(bf16x8_t, scale_bf16x8(__builtin_bit_cast(u32x4_t, b[j]), c));
#pragma unroll
    for (int i = 0; i < BI; ++i)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bs, acc[i][j], 0, 0, 0);
  }
}

// One ring step: loads into stage `nxt`, then the MFMAs from stage `cur`.
// Both pointers are restrict parameters of one inlined call, which gives
// the compiler the alias scopes that keep the reads of `cur` from waiting
// for the loads into `nxt` (without them every LDS read waits for all
// loads into LDS in flight).
template <bool SCALE, typename Issue>
__device__ __forceinline__ void ring_step(uint16_t* __restrict__ nxt, const uint16_t* __restrict__ cur,
                                          Issue issue, float c, OuterAcc& acc) {
  issue(nxt);
  if (SCALE)
    outer_compute_scaled(cur, cur + A_TILE, c, acc);
  else
    outer_compute(cur, cur + A_TILE, acc);
}

// The ring: one array per stage, so that reads of one stage are not made to
// wait for the loads into the others.  Kernels may reuse it once the main
// loop has returned.
__shared__ __attribute__((aligned(16))) uint16_t lin_ring0[OUTER_STAGE];
__shared__ __attribute__((aligned(16))) uint16_t lin_ring1[OUTER_STAGE];
__shared__ __attribute__((aligned(16))) uint16_t lin_ring2[OUTER_STAGE];
__shared__ __attribute__((aligned(16))) uint16_t lin_ring3[RING > 3 ? OUTER_STAGE : 8];
__device__ __forceinline__ uint16_t* lin_stage(int k) {
  return k == 0 ? lin_ring0 : k == 1 ? lin_ring1 : k == 2 ? lin_ring2 : lin_ring3;
}

// DEEP: the step's reads carry alias scopes (ring_step), so they do not
// wait for the next stage's loads and RING - 1 steps stay in flight.
// Without it the compiler makes the reads wait for all but the newest
// loads, one step fewer (every kernel here measured faster with DEEP; the
// clipped sum by 2 % on C4).
// FIX: a step whose `fix` is set calls fixup(stage, step) once its loads
// have landed, then waits for every wave before the MFMAs (segments with
// non-finite columns only).
template <bool SCALE, bool DEEP, bool FIX, typename Next, typename Scale, typename Fixup>
__device__ __forceinline__ void dma_mainloop(const LinProblem& P, int64_t o0, int64_t n0, Step first,
                                             Next next, Scale scale, Fixup fixup, OuterAcc& acc) {
  auto stage = [&](int k) -> uint16_t* { return lin_stage(k); };
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Per lane: tile row and column of each of its loads (row within the
  // step, column within the tile after undoing the swizzle).
  int arow[A_DMA], acol[A_DMA], brow[B_DMA], bcol[B_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    arow[i] = RPW * wave + 2 * i + (lane >> 5);
    acol[i] = 8 * ((lane & 31) ^ (swz(arow[i]) >> 1));
  }
#pragma unroll
  for (int i = 0; i < B_DMA; ++i) {
    brow[i] = RPW * wave + B_RPI * i + (lane / B_LPR);
    bcol[i] = 8 * ((lane % B_LPR) ^ (swz(brow[i]) >> 1));
  }
  const int32_t dout = (int32_t)P.d_out, din = (int32_t)P.d_in;
  const uint32_t ldg = (uint32_t)P.ldg, ldx = (uint32_t)P.ldx;

  auto issue = [&](uint16_t* st, const Step& x) {
    const uint32_t rows = x.live ? (uint32_t)(x.te - x.tb) : 0u;
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(P.G + x.tb * P.ldg), (short)0, (int)(rows * ldg * 2u), LIN_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(P.X + x.tb * P.ldx), (short)0, (int)(rows * ldx * 2u), LIN_BUF_DWORD3);
    const uint32_t r0 = (uint32_t)(x.t0 - x.tb);
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const int32_t col = (int32_t)o0 + acol[i];
      const uint32_t off = col < dout ? ((r0 + arow[i]) * ldg + (uint32_t)col) * 2u : LIN_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (ODP_LDS void*)(st + (RPW * wave + 2 * i) * OM), 16, off, 0,
                                               0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int32_t col = (int32_t)n0 + bcol[i];
      const uint32_t off = col < din ? ((r0 + brow[i]) * ldx + (uint32_t)col) * 2u : LIN_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (ODP_LDS void*)(st + A_TILE + (RPW * wave + B_RPI * i) * ON),
                                               16, off, 0, 0, 0);
    }
  };

  // Prologue: steps 0 .. RING - 2 in flight.  Steps past the last one
  // still issue (zero rows, so out of range) to keep the wait counts
  // constant.
  Step cur = first;
  Step ld = first;
  float cs[RING];
#pragma unroll
  for (int q = 0; q < RING - 1; ++q) {
    issue(stage(q), ld);
    cs[q] = SCALE && ld.live ? scale(ld) : 1.0f;
    ld = next(ld);
  }
  while (cur.live) {
#pragma unroll
    for (int k = 0; k < RING; ++k) {
      if (!cur.live) break;
      // This step's loads have landed; the later RING - 2 steps' may fly.
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((RING - 2) * DMA_PER_STEP));
      __asm__ volatile("s_barrier" ::: "memory");
      if (FIX && cur.fix) {
        fixup(stage(k), cur);
        __syncthreads();
      }
      // Loads of step ld go into the stage computed at the previous step.
      const Step x = ld;
      const int kn = (k + RING - 1) % RING;
      if (DEEP) {
        ring_step<SCALE>(stage(kn), stage(k), [&](uint16_t* st) { issue(st, x); }, cs[k], acc);
      } else {
        issue(stage(kn), x);
        if (SCALE)
          outer_compute_scaled(stage(k), stage(k) + A_TILE, cs[k], acc);
        else
          outer_compute(stage(k), stage(k) + A_TILE, acc);
      }
      cs[kn] = SCALE && ld.live ? scale(ld) : 1.0f;
      ld = next(ld);
      cur = next(cur);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no load into LDS may outlive the workgroup
  __asm__ volatile("s_barrier" ::: "memory");
}

// Compile-time loop: f(Idx<0>{}), ..., f(Idx<N - 1>{}).  Accumulator
// arrays indexed only through it stay in registers whatever their size
// (a plain loop the unroller declines leaves them in scratch memory).
template <int V>
struct Idx {
  static constexpr int value = V;
};
template <int N, int K = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (K < N) {
    f(Idx<K>{});
    static_for<N, K + 1>(f);
  }
}

template <int I, int J>
__device__ __forceinline__ void zero_acc(f32x4_t (&acc)[I][J]) {
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
}
