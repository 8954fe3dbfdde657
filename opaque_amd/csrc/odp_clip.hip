// Clip factors (fixed / AUTO-S, global or per group) and the clipped batch
// sum of stored per-segment gradients.
//
// The scale arithmetic follows clip_pytree / auto_scale_pytree
// (opaque-engine/.../clipping/_pytree.py:106-142, 345-431, 475-564): fp64
// norms, ratio C/||g|| (or R/(||g||+gamma)), the storage guard
// ratio*rel - abs evaluated as two separately rounded fp64 operations,
// min(1, .) for fixed clipping with NaN propagating as in torch.minimum,
// non-finite -> 0, clamp at 0, then rounded to the leaf dtype the way
// torch casts a float64 tensor (to float32, then to bfloat16).
#include <mutex>

#include "odp_internal.h"

namespace {

constexpr int CL_THREADS = 1024;  // one workgroup per example
constexpr int CL_DEPTH = 8;      // loads in flight per thread (a power of two)
constexpr int CL_MAX_GROUPS = 1024;
static_assert(CL_MAX_GROUPS <= CL_THREADS, "thread g finishes group g");
constexpr int SS_THREADS = 256;
constexpr int SS_ELEMS = 8;  // elements per thread

// Workgroup sum in a fixed order (a fixed tree within each wave by DPP and
// lane reads, then the wave sums in wave order), so that runs are bitwise
// reproducible.  The result is valid in every thread.
__device__ __forceinline__ double block_sum_fixed(double v, double* red) {
  v = rows_sum4(row_sum16(v));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < CL_THREADS / 64; ++w) t += red[w];
  __syncthreads();
  return t;
}

// The scale as the leaf dtype holds it (float64 leaves keep every bit).
__device__ __forceinline__ double finalize_scale(double ratio, double rel, double abs_, int clamp_one,
                                                 int dtype) {
  double s = __dsub_rn(__dmul_rn(ratio, rel), abs_);
  if (clamp_one && !(s < 1.0) && !isnan(s)) s = 1.0;
  if (!isfinite(s)) s = 0.0;
  if (s < 0.0) s = 0.0;
  if (dtype == ODP_DTYPE_F64) return s;
  return (double)odp_round_to((float)s, dtype);
}

// One workgroup per example.  Group g owns slots [gstart[g], gstart[g+1]).
// The sum of an example's partials (a few hundred KB on Llama-shaped
// models) is bound by what one CU can have in flight, so each thread issues
// CL_DEPTH 16-byte loads at once; the order of additions is fixed (it does
// not depend on which loads are masked), so runs are bitwise reproducible.
// `status` (optional): a word that k_sqnorm sets when it dropped a write
// outside the partials; every example then gets a NaN norm, zero scales and
// clear masks, since the partials are incomplete.
__global__ __launch_bounds__(CL_THREADS) void k_clip_factors(
    const double* __restrict__ part, int64_t n_slots, int n_ex, const int64_t* __restrict__ gstart, int n_groups,
    const double* __restrict__ thr, double eff_thr, int mode, double gamma, int n_cls,
    const double* __restrict__ guard, const int32_t* __restrict__ cls_dtype,
    double* __restrict__ scale_out, float* __restrict__ norm_out, float* __restrict__ gnorm_out,
    uint8_t* __restrict__ clip_out, uint8_t* __restrict__ clip_total_out, const uint32_t* __restrict__ status) {
  const int ex = blockIdx.x;
  const int t = threadIdx.x;
  if (status != nullptr && *status != 0u) {
    if (t == 0) {
      norm_out[ex] = __builtin_nanf("");
      if (clip_total_out) clip_total_out[ex] = 0;
    }
    if (t < n_groups) {
      if (gnorm_out) gnorm_out[(int64_t)t * n_ex + ex] = __builtin_nanf("");
      if (clip_out) clip_out[(int64_t)t * n_ex + ex] = 0;
      for (int k = 0; k < n_cls; ++k) scale_out[((int64_t)k * n_groups + t) * n_ex + ex] = 0.0;
    }
    return;
  }
  __shared__ double red[CL_THREADS / 64];
  __shared__ double gsq[CL_MAX_GROUPS];
  __shared__ double sguard[16];
  __shared__ int scls[8];
  const double* row = part + (int64_t)ex * n_slots;
  // The inputs of the scale arithmetic are read now, so that their load
  // latency overlaps the partials' instead of following the reduction
  // (n_groups <= CL_THREADS: thread g finishes group g; the barriers of the
  // reduction publish sguard and scls).
  const double thr_t = t < n_groups ? thr[t] : 0.0;
  if (t < 2 * n_cls) sguard[t] = guard[t];
  if (t < n_cls) scls[t] = cls_dtype[t];

  for (int g = 0; g < n_groups; ++g) {
    const int64_t hi = gstart[g + 1];
    double a[CL_DEPTH];
#pragma unroll
    for (int q = 0; q < CL_DEPTH; ++q) a[q] = 0.0;
    // Slots are read in 16-byte pairs from the first 16-byte aligned one
    // (by address, so any 8-byte aligned partials buffer works; a leading
    // and a trailing odd slot go to thread 0), and every load of a round is
    // issued before the first add (masked past the group's end).
    const int64_t lo = gstart[g];
    int64_t la = lo + (int64_t)((((uintptr_t)(row + lo)) >> 3) & 1u);
    la = la < hi ? la : hi;
    const int64_t npair = (hi - la) >> 1;
    if (t == 0) {
      if (lo < la) a[0] += row[lo];
      if (la + 2 * npair < hi) a[1] += row[hi - 1];
    }
    const double2* pr = (const double2*)(row + la);
    for (int64_t q0 = t; q0 < npair; q0 += CL_DEPTH * CL_THREADS) {
      double2 v[CL_DEPTH];
#pragma unroll
      for (int q = 0; q < CL_DEPTH; ++q)
        v[q] = q0 + q * CL_THREADS < npair ? pr[q0 + q * CL_THREADS] : double2{0.0, 0.0};
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < CL_DEPTH; ++q) a[q] = (a[q] + v[q].x) + v[q].y;
    }
    // Pairwise over the accumulators, in a fixed order.
#pragma unroll
    for (int w = CL_DEPTH / 2; w > 0; w >>= 1)
#pragma unroll
      for (int q = 0; q < w; ++q) a[q] = a[2 * q] + a[2 * q + 1];
    const double tot = block_sum_fixed(a[0], red);
    if (t == 0) gsq[g] = tot;
  }
  __syncthreads();

  if (t == 0) {
    double total = 0.0;
    for (int g = 0; g < n_groups; ++g) total += gsq[g];
    const double norm = sqrt(total);
    const float normf = (float)norm;
    norm_out[ex] = normf;
    if (clip_total_out) clip_total_out[ex] = normf > (float)eff_thr ? 1 : 0;
  }
  if (t < n_groups) {
    const int g = t;
    const double gn = sqrt(gsq[g]);
    if (gnorm_out) gnorm_out[(int64_t)g * n_ex + ex] = (float)gn;
    if (clip_out) clip_out[(int64_t)g * n_ex + ex] = (float)gn > (float)thr_t ? 1 : 0;
    const double c = thr_t > 0.0 ? thr_t : 0.0;
    const double ratio = mode == ODP_CLIP_AUTOS ? c / (gn + gamma) : c / gn;
    for (int k = 0; k < n_cls; ++k)
      scale_out[((int64_t)k * n_groups + g) * n_ex + ex] =
          finalize_scale(ratio, sguard[2 * k], sguard[2 * k + 1], mode == ODP_CLIP_FIXED, scls[k]);
  }
}

// Clipped sum of one leaf per problem: 8 consecutive elements per thread
// (one 16-byte load per segment for bf16), summed over the leaf's segments
// in segment order.  Each term is scale * value rounded to the value's dtype
// (clip_pytree's `scale.to(dtype) * leaf`), accumulated in float32, or in
// float64 (Acc = double) for float64 values or a float64 compute dtype.
// This element-wise form serves float16/float64, the float64 sums and raw
// sums; the kernel below vectorises float32/bfloat16.  `raw`: the values
// are already scaled (a caller's scale function): each is summed as it is,
// with scale 1 and no nan_to_num, as the reference sums a scale function's
// output (_clipped_fun.py:673-700, 777-782).
template <typename Acc>
__device__ __forceinline__ void scale_sum_generic(const void* pe, int pdt, int64_t E, int64_t e0, int n_seg,
                                                  int seg_first, const int32_t* __restrict__ sex,
                                                  const double* __restrict__ sc, float normalize_by, void* out,
                                                  void* out2, int odt, int transpose, int64_t M, int rank,
                                                  bool raw) {
  Acc acc[SS_ELEMS], acc2[SS_ELEMS];
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i) acc[i] = acc2[i] = (Acc)0;
  for (int s = 0; s < n_seg; ++s) {
    const double c = raw ? 1.0 : sc[sex[seg_first + s]];
#pragma unroll
    for (int i = 0; i < SS_ELEMS; ++i) {
      if (e0 + i >= E) break;
      const double v = odp_load_as_double(pe, (int64_t)s * E + e0 + i, pdt);
      double y = 0.0, yy = 0.0;
      if (raw || isfinite(v)) {  // nan_to_num of the per-example value
        if (pdt == ODP_DTYPE_F64) {
          y = c * v;
          yy = y * y;
        } else {
          y = (double)odp_round_to(__fmul_rn((float)c, (float)v), pdt);
          yy = (double)odp_round_to(__fmul_rn((float)y, (float)y), pdt);
        }
      }
      acc[i] += (Acc)y;
      acc2[i] += (Acc)yy;
    }
  }
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i) {
    const int64_t e = e0 + i;
    if (e >= E) break;
    const int64_t k = e / M, m = e - k * M;
    const int64_t o = transpose ? m * rank + k : e;
    // Cast to the output dtype, then divide in it (the reference's order).
    if (odt == ODP_DTYPE_F64) {
      const double x = (double)acc[i], x2 = (double)acc2[i];
      odp_store_from_double(out, o, odt, normalize_by != 1.0f ? x / (double)normalize_by : x);
      if (out2) odp_store_from_double(out2, o, odt, normalize_by != 1.0f ? x2 / (double)normalize_by : x2);
    } else {
      float x = odp_round_to((float)acc[i], odt), x2 = odp_round_to((float)acc2[i], odt);
      if (normalize_by != 1.0f) {
        x = odp_round_to(__fdiv_rn(x, normalize_by), odt);
        x2 = odp_round_to(__fdiv_rn(x2, normalize_by), odt);
      }
      odp_store_from_float(out, o, odt, x);
      if (out2) odp_store_from_float(out2, o, odt, x2);
    }
  }
}

// One clipped-sum term per element: the per-example value with non-finite
// entries zeroed (nan_to_num), times the scale, rounded to bf16 when the
// values are bf16 (scale.to(dtype) * leaf); accumulated in float32.
template <bool SECOND, bool BF>
__device__ __forceinline__ void ss_term(float v, float c, float& acc, float& acc2) {
  if (!isfinite(v)) v = 0.f;
  float y = __fmul_rn(c, v);
  if (BF) y = odp_round_bf16(y);
  acc = __fadd_rn(acc, y);
  if (SECOND) {
    float yy = __fmul_rn(y, y);
    if (BF) yy = odp_round_bf16(yy);
    acc2 = __fadd_rn(acc2, yy);
  }
}

// The sum cast to the output dtype, then divided in it (the reference's order).
__device__ __forceinline__ float ss_finish(float acc, float normalize_by, int odt) {
  float x = odp_round_to(acc, odt);
  if (normalize_by != 1.0f) x = odp_round_to(__fdiv_rn(x, normalize_by), odt);
  return x;
}

// 8 consecutive outputs: one 16-byte store (bf16) or two (f32).
__device__ __forceinline__ void ss_put8(void* dst, int64_t o, int odt, const float (&y)[SS_ELEMS]) {
  if (odt == ODP_DTYPE_BF16) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 w;
    w.x = (uint32_t)odp_f2bf(y[0]) | ((uint32_t)odp_f2bf(y[1]) << 16);
    w.y = (uint32_t)odp_f2bf(y[2]) | ((uint32_t)odp_f2bf(y[3]) << 16);
    w.z = (uint32_t)odp_f2bf(y[4]) | ((uint32_t)odp_f2bf(y[5]) << 16);
    w.w = (uint32_t)odp_f2bf(y[6]) | ((uint32_t)odp_f2bf(y[7]) << 16);
    odp_gstore((u32x4*)((uint16_t*)dst + o), w);
  } else {
    odp_gstore((f32x4_t*)((float*)dst + o), f32x4_t{y[0], y[1], y[2], y[3]});
    odp_gstore((f32x4_t*)((float*)dst + o + 4), f32x4_t{y[4], y[5], y[6], y[7]});
  }
}

// The sums take segments SS_SG at a time: the scales and values of a group
// are all loaded before the first of them is accumulated, so several loads
// are in flight per thread, and the accumulation order (and so every sum)
// is that of one segment at a time.  Stored per-example values are read
// once, non-temporally.
constexpr int SS_SG = 4;
typedef uint32_t ss_u32x4 __attribute__((ext_vector_type(4)));

// Eight consecutive values at element `at` (bf16: one 16-byte load).
template <bool BF>
__device__ __forceinline__ void ss_load8_row(const void* pe, int64_t at, float (&v)[SS_ELEMS]) {
  if (BF) {
    const ss_u32x4 w = __builtin_nontemporal_load((const ss_u32x4*)((const uint16_t*)pe + at));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const f32x4_t a = __builtin_nontemporal_load((const f32x4_t*)((const float*)pe + at));
    const f32x4_t b = __builtin_nontemporal_load((const f32x4_t*)((const float*)pe + at + 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
}

// Eight values M elements apart from element `base` (ranks k0.. of a column).
template <bool BF>
__device__ __forceinline__ void ss_load8_col(const void* pe, int64_t base, int64_t M, float (&v)[SS_ELEMS]) {
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i)
    v[i] = BF ? odp_bf2f(__builtin_nontemporal_load((const uint16_t*)pe + base + i * M))
              : __builtin_nontemporal_load((const float*)pe + base + i * M);
}

// bf16/f32 values and outputs, E a multiple of 8: a thread sums the 8
// consecutive elements e0.. over the segments (16-byte loads for bf16).
template <bool SECOND, bool BF>
__device__ __forceinline__ void scale_sum_rows(const void* pe, int64_t E, int64_t M, int rank, int64_t e0, int n_seg,
                                               int seg_first, const int32_t* __restrict__ sex,
                                               const double* __restrict__ sc, float normalize_by, void* out,
                                               void* out2, int odt, int transpose) {
  float acc[SS_ELEMS], acc2[SS_ELEMS];
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i) acc[i] = acc2[i] = 0.f;
  int s = 0;
  for (; s + SS_SG <= n_seg; s += SS_SG) {
    float c[SS_SG], v[SS_SG][SS_ELEMS];
#pragma unroll
    for (int q = 0; q < SS_SG; ++q) {
      c[q] = (float)sc[sex[seg_first + s + q]];
      ss_load8_row<BF>(pe, (int64_t)(s + q) * E + e0, v[q]);
    }
#pragma unroll
    for (int q = 0; q < SS_SG; ++q)
#pragma unroll
      for (int i = 0; i < SS_ELEMS; ++i) ss_term<SECOND, BF>(v[q][i], c[q], acc[i], acc2[i]);
  }
  for (; s < n_seg; ++s) {
    const float c = (float)sc[sex[seg_first + s]];
    float v[SS_ELEMS];
    ss_load8_row<BF>(pe, (int64_t)s * E + e0, v);
#pragma unroll
    for (int i = 0; i < SS_ELEMS; ++i) ss_term<SECOND, BF>(v[i], c, acc[i], acc2[i]);
  }
  float x[SS_ELEMS], x2[SS_ELEMS];
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i) {
    x[i] = ss_finish(acc[i], normalize_by, odt);
    if (SECOND) x2[i] = ss_finish(acc2[i], normalize_by, odt);
  }
  if (!transpose) {
    ss_put8(out, e0, odt, x);
    if (SECOND) ss_put8(out2, e0, odt, x2);
    return;
  }
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i) {
    const int64_t e = e0 + i;
    const int64_t k = e / M, m = e - k * M;
    odp_store_from_float(out, m * rank + k, odt, x[i]);
    if (SECOND) odp_store_from_float(out2, m * rank + k, odt, x2[i]);
  }
}

// Transposed outputs: a thread sums ranks k0..k0+7 of column m (e_first is
// element (k0, m), rows M apart) and stores them at o = m * rank + k0.
template <bool SECOND, bool BF>
__device__ __forceinline__ void scale_sum_cols(const void* pe, int64_t E, int64_t M, int64_t e_first, int n_seg,
                                               int seg_first, const int32_t* __restrict__ sex,
                                               const double* __restrict__ sc, float normalize_by, void* out,
                                               void* out2, int odt, int64_t o) {
  float acc[SS_ELEMS], acc2[SS_ELEMS];
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i) acc[i] = acc2[i] = 0.f;
  int s = 0;
  for (; s + SS_SG <= n_seg; s += SS_SG) {
    float c[SS_SG], v[SS_SG][SS_ELEMS];
#pragma unroll
    for (int q = 0; q < SS_SG; ++q) {
      c[q] = (float)sc[sex[seg_first + s + q]];
      ss_load8_col<BF>(pe, (int64_t)(s + q) * E + e_first, M, v[q]);
    }
#pragma unroll
    for (int q = 0; q < SS_SG; ++q)
#pragma unroll
      for (int i = 0; i < SS_ELEMS; ++i) ss_term<SECOND, BF>(v[q][i], c[q], acc[i], acc2[i]);
  }
  for (; s < n_seg; ++s) {
    const float c = (float)sc[sex[seg_first + s]];
    float v[SS_ELEMS];
    ss_load8_col<BF>(pe, (int64_t)s * E + e_first, M, v);
#pragma unroll
    for (int i = 0; i < SS_ELEMS; ++i) ss_term<SECOND, BF>(v[i], c, acc[i], acc2[i]);
  }
  float x[SS_ELEMS], x2[SS_ELEMS];
#pragma unroll
  for (int i = 0; i < SS_ELEMS; ++i) {
    x[i] = ss_finish(acc[i], normalize_by, odt);
    if (SECOND) x2[i] = ss_finish(acc2[i], normalize_by, odt);
  }
  ss_put8(out, o, odt, x);
  if (SECOND) ss_put8(out2, o, odt, x2);
}

__global__ __launch_bounds__(SS_THREADS) void k_scale_sum(
    const int64_t* __restrict__ probs, const int32_t* __restrict__ ws, int n_prob,
    const int32_t* __restrict__ sex, const double* __restrict__ scales, int n_ex, int n_groups,
    float normalize_by) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_SS_FIELDS;
  const float* pe = (const float*)f[ODP_SS_PE];
  const int64_t M = f[ODP_SS_M];
  const int rank = (int)f[ODP_SS_RANK];
  const int seg_first = (int)f[ODP_SS_SEG_FIRST], n_seg = (int)f[ODP_SS_NSEG];
  void* out = (void*)f[ODP_SS_OUT];
  void* out2 = (void*)f[ODP_SS_OUT2];
  const int64_t flags = f[ODP_SS_FLAGS];
  const int odt = (int)(flags & 0xff);
  const int transpose = (int)((flags >> 8) & 0xff);
  const int grp = (int)((flags >> 16) & 0xffffff);
  const int cls = (int)((flags >> 40) & 0xff);
  const int wide = (int)((flags >> 48) & 1);
  const bool raw = ((flags >> 52) & 1) != 0;
  const int pdt = (int)((flags >> 56) & 0xff);
  const int64_t E = M * rank;
  const double* sc = scales + ((int64_t)cls * n_groups + grp) * n_ex;
  const bool generic = wide || raw || pdt == ODP_DTYPE_F64 || pdt == ODP_DTYPE_F16 || odt == ODP_DTYPE_F16 ||
                       odt == ODP_DTYPE_F64 || (E & 7) != 0;
  if (generic) {
    const int64_t e0 = ((int64_t)(bid - ws[p]) * SS_THREADS + threadIdx.x) * SS_ELEMS;
    if (e0 >= E) return;
    if (wide || pdt == ODP_DTYPE_F64)
      scale_sum_generic<double>(pe, pdt, E, e0, n_seg, seg_first, sex, sc, normalize_by, out, out2, odt, transpose,
                                M, rank, raw);
    else
      scale_sum_generic<float>(pe, pdt, E, e0, n_seg, seg_first, sex, sc, normalize_by, out, out2, odt, transpose,
                               M, rank, raw);
    return;
  }
  const bool bf_in = pdt == ODP_DTYPE_BF16;
  const int b = bid - ws[p];
  // Transposed leaves ([M][rank] out of [rank][M] sums) with rank in
  // {8, 16, 32, 64}: each thread sums 8 consecutive ranks of one column, so
  // that its outputs are one 16-byte store; lanes take consecutive columns,
  // so every load instruction reads consecutive elements of a row.
  const int k8 = rank >> 3;
  if (transpose && (rank & 7) == 0 && rank <= 64 && SS_THREADS % k8 == 0) {
    const int cols = SS_THREADS / k8;  // columns per workgroup
    const int64_t m = (int64_t)b * cols + threadIdx.x % cols;
    if (m >= M) return;
    const int64_t e_first = (int64_t)(threadIdx.x / cols) * 8 * M + m;  // element (k0, m)
    if (out2) {
      if (bf_in) scale_sum_cols<true, true>(pe, E, M, e_first, n_seg, seg_first, sex, sc, normalize_by, out, out2,
                                            odt, m * rank + (threadIdx.x / cols) * 8);
      else scale_sum_cols<true, false>(pe, E, M, e_first, n_seg, seg_first, sex, sc, normalize_by, out, out2, odt,
                                       m * rank + (threadIdx.x / cols) * 8);
    } else {
      if (bf_in) scale_sum_cols<false, true>(pe, E, M, e_first, n_seg, seg_first, sex, sc, normalize_by, out,
                                             nullptr, odt, m * rank + (threadIdx.x / cols) * 8);
      else scale_sum_cols<false, false>(pe, E, M, e_first, n_seg, seg_first, sex, sc, normalize_by, out, nullptr,
                                        odt, m * rank + (threadIdx.x / cols) * 8);
    }
    return;
  }
  const int64_t e0 = ((int64_t)b * SS_THREADS + threadIdx.x) * SS_ELEMS;
  if (e0 >= E) return;
  if (out2) {
    if (bf_in) scale_sum_rows<true, true>(pe, E, M, rank, e0, n_seg, seg_first, sex, sc, normalize_by, out, out2,
                                          odt, transpose);
    else scale_sum_rows<true, false>(pe, E, M, rank, e0, n_seg, seg_first, sex, sc, normalize_by, out, out2, odt,
                                     transpose);
  } else {
    if (bf_in) scale_sum_rows<false, true>(pe, E, M, rank, e0, n_seg, seg_first, sex, sc, normalize_by, out,
                                           nullptr, odt, transpose);
    else scale_sum_rows<false, false>(pe, E, M, rank, e0, n_seg, seg_first, sex, sc, normalize_by, out, nullptr,
                                      odt, transpose);
  }
}

// Per-segment sums of squares of materialised per-example tensors: x^2 in
// clip_pytree's accumulation dtype (float32, or float64 with the flag bit 8
// of ODP_SQ_DTYPE, as for float64 leaves), summed in fp64.  Each workgroup
// reduces SQ_CHUNK elements of one segment and writes one slot.
constexpr int SQ_THREADS = 256;
constexpr int64_t SQ_CHUNK = 8192;

// Writes outside the partials ([0, n_ex) x [0, part_stride)) are dropped;
// `status` (optional) is then set to 1.
__global__ __launch_bounds__(SQ_THREADS) void k_sqnorm(const int64_t* __restrict__ probs,
                                                       const int32_t* __restrict__ ws, int n_prob,
                                                       const int32_t* __restrict__ sex,
                                                       double* __restrict__ part,
                                                       int64_t part_stride, int n_ex, uint32_t* status) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_SQ_FIELDS;
  const void* X = (const void*)f[ODP_SQ_X];
  const int64_t n = f[ODP_SQ_N];
  const int seg_first = (int)f[ODP_SQ_SEG_FIRST];
  const int64_t slot = f[ODP_SQ_SLOT];
  const int dt = (int)(f[ODP_SQ_DTYPE] & 0xff);
  const bool sq64 = ((f[ODP_SQ_DTYPE] >> 8) & 1) != 0;
  const bool raw = ((f[ODP_SQ_DTYPE] >> 9) & 1) != 0;  // no nan_to_num
  const int64_t nchunk = (n + SQ_CHUNK - 1) / SQ_CHUNK;
  const int64_t local = bid - ws[p];
  const int64_t seg = local / nchunk, chunk = local % nchunk;
  const int64_t lo = chunk * SQ_CHUNK, hi = lo + SQ_CHUNK < n ? lo + SQ_CHUNK : n;
  double acc = 0.0;
  if (sq64) {
    for (int64_t i = lo + threadIdx.x; i < hi; i += SQ_THREADS) {
      double x = odp_load_as_double(X, seg * n + i, dt);
      if (!raw && !isfinite(x)) x = 0.0;  // nan_to_num before the norm
      acc += x * x;
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += SQ_THREADS) {
      float x = odp_load_as_float(X, seg * n + i, dt);
      if (!raw && !isfinite(x)) x = 0.f;
      acc += (double)__fmul_rn(x, x);
    }
  }
  __shared__ double red[SQ_THREADS];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = SQ_THREADS / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int ex = sex[seg_first + seg];
    if (ex >= 0 && ex < n_ex && slot >= 0 && slot + chunk < part_stride)
      part[(int64_t)ex * part_stride + slot + chunk] = red[0];
    else if (status != nullptr)
      odp_gstore(status, 1u);  // every such writer stores the same value
  }
}

}  // namespace

extern "C" int64_t odp_sqnorm_blocks(int64_t n) {
  return n <= 0 ? 0 : (n + SQ_CHUNK - 1) / SQ_CHUNK;
}

extern "C" int odp_sqnorm(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                          int32_t n_prob, int32_t total_blocks, const int32_t* seg_example,
                          double* part, int64_t part_stride) {
  int rc = odp_check_table("odp_sqnorm", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (total_blocks == 0) return ODP_OK;
  if (seg_example == nullptr || part == nullptr || part_stride <= 0) {
    odp_set_error("odp_sqnorm: null seg_example/part or part_stride <= 0");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_sqnorm, dim3(total_blocks), dim3(SQ_THREADS), 0, odp_hip_stream(stream),
                     problems, work_start, n_prob, seg_example, part, part_stride, INT32_MAX, nullptr);
  return odp_check_launch("odp_sqnorm");
}

// Argument checks shared by odp_clip_factors and its allocation-free
// variant (everything but the partials pointer).
static int check_clip_args(const char* what, int64_t n_slots, int32_t n_ex, const int64_t* group_slot_start,
                           int32_t n_groups, const double* thresholds, int32_t mode, double gamma, int32_t n_cls,
                           const double* guard, const int32_t* cls_dtype, const double* scale_out,
                           const float* norm_out) {
  if (n_ex < 0 || n_slots < 0) {
    odp_set_error("%s: negative n_ex or n_slots", what);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (n_groups < 1 || n_groups > CL_MAX_GROUPS) {
    odp_set_error("%s: n_groups=%d outside [1, %d]", what, n_groups, CL_MAX_GROUPS);
    return ODP_ERR_UNSUPPORTED;
  }
  if (n_cls < 1 || n_cls > 8) {
    odp_set_error("%s: n_cls=%d outside [1, 8]", what, n_cls);
    return ODP_ERR_UNSUPPORTED;
  }
  if (mode != ODP_CLIP_FIXED && mode != ODP_CLIP_AUTOS) {
    odp_set_error("%s: unknown mode %d", what, mode);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (mode == ODP_CLIP_AUTOS && !(gamma > 0.0)) {
    odp_set_error("%s: gamma must be positive, got %g", what, gamma);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (n_ex > 0 && (group_slot_start == nullptr || thresholds == nullptr || guard == nullptr ||
                   cls_dtype == nullptr || scale_out == nullptr || norm_out == nullptr)) {
    odp_set_error("%s: null required pointer", what);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  return ODP_OK;
}

extern "C" int odp_clip_factors(odp_stream_t stream, const double* part, int64_t n_slots,
                                int32_t n_ex, const int64_t* group_slot_start, int32_t n_groups,
                                const double* thresholds, double effective_threshold, int32_t mode,
                                double gamma, int32_t n_cls, const double* guard,
                                const int32_t* cls_dtype, double* scale_out, float* norm_out,
                                float* group_norm_out, uint8_t* clipped_out,
                                uint8_t* clipped_total_out) {
  int rc = check_clip_args("odp_clip_factors", n_slots, n_ex, group_slot_start, n_groups, thresholds, mode,
                           gamma, n_cls, guard, cls_dtype, scale_out, norm_out);
  if (rc != ODP_OK) return rc;
  if (n_ex == 0) return ODP_OK;
  if (n_slots > 0 && part == nullptr) {
    odp_set_error("odp_clip_factors: null required pointer");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_clip_factors, dim3(n_ex), dim3(CL_THREADS), 0, odp_hip_stream(stream), part,
                     n_slots, n_ex, group_slot_start, n_groups, thresholds, effective_threshold, mode,
                     gamma, n_cls, guard, cls_dtype, scale_out, norm_out, group_norm_out,
                     clipped_out, clipped_total_out, nullptr);
  return odp_check_launch("odp_clip_factors");
}

extern "C" int64_t odp_scale_sum_blocks(int64_t n_elems) {
  const int64_t per = (int64_t)SS_THREADS * SS_ELEMS;
  return n_elems <= 0 ? 0 : (n_elems + per - 1) / per;
}

extern "C" int odp_scale_sum(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                             int32_t n_prob, int32_t total_blocks, const int32_t* seg_example,
                             const double* scales, int32_t n_ex, int32_t n_groups,
                             float normalize_by) {
  int rc = odp_check_table("odp_scale_sum", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (!(normalize_by > 0.0f)) {
    odp_set_error("odp_scale_sum: normalize_by must be > 0, got %g", (double)normalize_by);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_example == nullptr || scales == nullptr || n_ex <= 0 || n_groups <= 0) {
    odp_set_error("odp_scale_sum: null seg_example/scales or non-positive n_ex/n_groups");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_scale_sum, dim3(total_blocks), dim3(SS_THREADS), 0, odp_hip_stream(stream),
                     problems, work_start, n_prob, seg_example, scales, n_ex, n_groups,
                     normalize_by);
  return odp_check_launch("odp_scale_sum");
}

// ---------------------------------------------------------------------------
// Allocation-free clipping of materialised per-example gradients.
//
// odp_sqnorm fills caller-provided fp64 partials that odp_clip_factors then
// reads.  Callers that cannot allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc) call
// odp_clip_materialized_noalloc instead: the partials live in `scratch`, a
// file-scope device array each GPU holds until the process ends.  The array
// is found by its address per device (hipGetSymbolAddress on the first call
// made with that device current); host code never passes the array's name
// itself to a kernel.  Every call on a GPU shares that GPU's array, so calls
// that overlap on one GPU race.
// ---------------------------------------------------------------------------
// The partials, then one status word (k_sqnorm's dropped writes).
static __device__ __align__(256) double scratch[ODP_NOALLOC_MAX_PARTIALS + 32];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
double* g_scratch_ptr[kMaxDevices] = {};

// The address of this device's `scratch`, looked up once per device.
int scratch_on_current_device(double** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    odp_set_error("odp_clip_materialized_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return ODP_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    odp_set_error("odp_clip_materialized_noalloc: device %d outside [0, %d)", dev, kMaxDevices);
    return ODP_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      odp_set_error("odp_clip_materialized_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                    hipGetErrorString(e));
      return ODP_ERR_HIP;
    }
    g_scratch_ptr[dev] = (double*)ptr;
  }
  *out = g_scratch_ptr[dev];
  return ODP_OK;
}

// Clears n partials and the status word (a kernel, not a memset: the call
// may be captured into a graph).
__global__ __launch_bounds__(256) void k_zero_partials(double* __restrict__ p, int64_t n, uint32_t* status) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0;
  if (i == 0) *status = 0u;
}

}  // namespace

extern "C" int64_t odp_noalloc_max_partials(void) { return ODP_NOALLOC_MAX_PARTIALS; }

extern "C" int odp_clip_materialized_noalloc(
    odp_stream_t stream, const int64_t* sq_problems, const int32_t* sq_work_start, int32_t sq_n_prob,
    int32_t sq_total_blocks, const int32_t* seg_example, int64_t n_slots, int32_t n_ex,
    const int64_t* group_slot_start, int32_t n_groups, const double* thresholds, double effective_threshold,
    int32_t mode, double gamma, int32_t n_cls, const double* guard, const int32_t* cls_dtype, double* scale_out,
    float* norm_out, float* group_norm_out, uint8_t* clipped_out, uint8_t* clipped_total_out) {
  const char* what = "odp_clip_materialized_noalloc";
  int rc = odp_check_table(what, sq_problems, sq_work_start, sq_n_prob, sq_total_blocks);
  if (rc != ODP_OK) return rc;
  rc = check_clip_args(what, n_slots, n_ex, group_slot_start, n_groups, thresholds, mode, gamma, n_cls, guard,
                       cls_dtype, scale_out, norm_out);
  if (rc != ODP_OK) return rc;
  if (n_ex == 0) return ODP_OK;
  if (n_slots > ODP_NOALLOC_MAX_PARTIALS / n_ex) {
    odp_set_error("%s: %d examples x %lld slots exceed the %lld partials of the static scratch", what, n_ex,
                  (long long)n_slots, (long long)ODP_NOALLOC_MAX_PARTIALS);
    return ODP_ERR_UNSUPPORTED;
  }
  if (sq_total_blocks > 0 && seg_example == nullptr) {
    odp_set_error("%s: null seg_example", what);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  double* part = nullptr;
  rc = scratch_on_current_device(&part);
  if (rc != ODP_OK) return rc;
  uint32_t* status = (uint32_t*)(part + ODP_NOALLOC_MAX_PARTIALS);
  hipStream_t s = odp_hip_stream(stream);
  const int64_t n = (int64_t)n_ex * n_slots;
  hipLaunchKernelGGL(k_zero_partials, dim3((unsigned)((n + 255) / 256 > 0 ? (n + 255) / 256 : 1)), dim3(256), 0, s,
                     part, n, status);
  rc = odp_check_launch(what);
  if (rc != ODP_OK) return rc;
  if (sq_total_blocks > 0) {
    // The kernel's bounds checks keep every write inside the n_ex x n_slots
    // partials (a malformed table cannot write past the static array).
    hipLaunchKernelGGL(k_sqnorm, dim3(sq_total_blocks), dim3(SQ_THREADS), 0, s, sq_problems, sq_work_start,
                       sq_n_prob, seg_example, part, n_slots, n_ex, status);
    rc = odp_check_launch(what);
    if (rc != ODP_OK) return rc;
  }
  hipLaunchKernelGGL(k_clip_factors, dim3(n_ex), dim3(CL_THREADS), 0, s, part, n_slots, n_ex, group_slot_start,
                     n_groups, thresholds, effective_threshold, mode, gamma, n_cls, guard, cls_dtype, scale_out,
                     norm_out, group_norm_out, clipped_out, clipped_total_out, status);
  return odp_check_launch(what);
}
