// Clipped first and second moments of full-weight per-example gradients
// without storing them.
//
// With second moments the reference squares every clipped per-example
// gradient and sums the squares beside the clipped values
// (opaque-engine/.../clipping/_clipped_fun.py:675-683, 777-782): per example
// i the gradient M_i = G_i^T X_i in the parameter dtype, y_i = scale_i * M_i
// rounded to it, y_i^2 rounded to it, and both summed over the batch in
// float32.  That is not one GEMM: the square is taken per example.  Here one
// workgroup owns an output tile and walks the examples' segments in order;
// per segment it forms the tile of M_s on the matrix cores (the same
// pipeline and accumulation order as the outer-form norm kernel), rounds it
// to bf16 as that kernel stores it, zeroes non-finite entries (nan_to_num),
// and adds y and round(y^2) into fp32 registers.  The sums are therefore
// those of the stored-gradient path (outer norm with its bf16 store, then
// the scale-sum) bit for bit, without the d_out x d_in bytes per example.
//
// Three register arrays per output element (the segment's accumulator and
// the two sums) fit at two waves per SIMD only with a smaller tile than the
// norm kernels': 256 x 128 (8 waves of 128 x 32).
#include "odp_internal.h"

#define ODP_LIN_ON 128

namespace {

#include "odp_outer.h"

// One term of both sums for the four entries of an MFMA block row, as the
// scale-sum over stored bf16 values adds it.
__device__ __forceinline__ void moment_terms(const f32x4_t& m, float c, f32x4_t& s1, f32x4_t& s2) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = odp_bf2f(odp_f2bf(m[e]));  // the entry as stored in bf16
    if (!isfinite(v)) v = 0.f;            // nan_to_num of the per-example value
    const float y = odp_round_bf16(__fmul_rn(c, v));
    s1[e] = __fadd_rn(s1[e], y);
    s2[e] = __fadd_rn(s2[e], odp_round_bf16(__fmul_rn(y, y)));
  }
}

// Stores a sum cast to the output dtype, then divided in it (the reference's
// order: sum, cast, / normalize_by).
__device__ __forceinline__ void moment_store(void* dst, int64_t at, int odt, float s, float normalize_by) {
  if (odt == ODP_DTYPE_F64) {
    odp_store_from_double(dst, at, odt, normalize_by != 1.0f ? (double)s / (double)normalize_by : (double)s);
    return;
  }
  float x = odp_round_to(s, odt);
  if (normalize_by != 1.0f) x = odp_round_to(__fdiv_rn(x, normalize_by), odt);
  odp_store_from_float(dst, at, odt, x);
}

// One OM x ON output tile of problem f: the segments in order.
__device__ __forceinline__ void moments_tile(const int64_t* __restrict__ f, const LinProblem& P, int tile,
                                             const int32_t* __restrict__ sstart, const int32_t* __restrict__ slen,
                                             const int32_t* __restrict__ sex, const double* __restrict__ scales,
                                             int n_ex, int n_groups, float normalize_by) {
  void* out = (void*)f[ODP_LN_OUT];
  void* out2 = (void*)f[ODP_LN_OUT2];
  const int64_t flags = f[ODP_LN_FLAGS];
  const int odt = (int)(flags & 0xff);
  const int grp = (int)((flags >> 8) & 0xffff);
  const int cls = (int)((flags >> 24) & 0xffff);
  const int tn_count = (int)((P.d_in + ON - 1) / ON);
  const int64_t o0 = (int64_t)(tile / tn_count) * OM, n0 = (int64_t)(tile % tn_count) * ON;
  // Uniform values through the scalar path.
  const ODP_CONST int32_t* cstart = (const ODP_CONST int32_t*)(sstart + P.seg_first);
  const ODP_CONST int32_t* clen = (const ODP_CONST int32_t*)(slen + P.seg_first);
  const ODP_CONST int32_t* cex = (const ODP_CONST int32_t*)(sex + P.seg_first);
  const ODP_CONST double* csc = (const ODP_CONST double*)(scales + ((int64_t)cls * n_groups + grp) * n_ex);

  OuterAcc acc, s1, s2;
  zero_acc(s1);
  zero_acc(s2);
  auto next = [](const Step& st) {
    Step n = st;
    n.t0 = st.t0 + OK;
    n.live = n.t0 < st.te ? 1 : 0;
    return n;
  };
  for (int sg = 0; sg < P.n_seg; ++sg) {
    const int32_t tb = cstart[sg], len = clen[sg];
    if (len <= 0) continue;  // M_s = 0 adds nothing
    zero_acc(acc);
    const Step first = {tb, tb, tb + len, sg, 1, 0};
    dma_mainloop<false, true, false>(P, o0, n0, first, next, [](const Step&) { return 1.0f; },
                                     [](uint16_t*, const Step&) {}, acc);
    const float c = (float)csc[cex[sg]];  // exact: a value of the class dtype
    static_for<BI * BJ>([&](auto q) {
      constexpr int i = decltype(q)::value / BJ, j = decltype(q)::value % BJ;
      moment_terms(acc[i][j], c, s1[i][j], s2[i][j]);
    });
  }

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
        moment_store(out, o * P.d_in + n, odt, s1[i][j][e], normalize_by);
        if (out2 != nullptr) moment_store(out2, o * P.d_in + n, odt, s2[i][j][e], normalize_by);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  });
}

// Workgroup = one output tile of one weight.
__global__ __launch_bounds__(OUTER_THREADS, ODP_LIN_OCC) void k_lin_moments(
    const int64_t* __restrict__ probs, const int32_t* __restrict__ ws, int n_prob,
    const int32_t* __restrict__ sstart, const int32_t* __restrict__ slen, const int32_t* __restrict__ sex,
    const double* __restrict__ scales, int n_ex, int n_groups, float normalize_by) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  const int tile = bid - ws[p];
  if (tile >= (int)((P.d_out + OM - 1) / OM) * (int)((P.d_in + ON - 1) / ON)) return;  // padding block
  moments_tile(f, P, tile, sstart, slen, sex, scales, n_ex, n_groups, normalize_by);
}

// The same sums for the problems with a segment at risk of float32
// overflow only (the clipped-sum GEMM skips exactly those): MOM_SPLIT
// workgroups per problem exit at once unless it is at risk, and otherwise
// loop over its tiles.
constexpr int MOM_SPLIT = 32;

__global__ __launch_bounds__(OUTER_THREADS, ODP_LIN_OCC) void k_lin_moments_guarded(
    const int64_t* __restrict__ probs, const int32_t* __restrict__ ws, int n_prob,
    const int32_t* __restrict__ sstart, const int32_t* __restrict__ slen, const int32_t* __restrict__ sex,
    const double* __restrict__ scales, int n_ex, int n_groups, float normalize_by) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_LN_FIELDS;
  const LinProblem P = read_problem(f);
  if (!lin_problem_at_risk(f, slen, P.seg_first, P.n_seg, P.d_in, P.d_out)) return;
  const int tiles = (int)((P.d_out + OM - 1) / OM) * (int)((P.d_in + ON - 1) / ON);
  for (int tile = bid - ws[p]; tile < tiles; tile += MOM_SPLIT)
    moments_tile(f, P, tile, sstart, slen, sex, scales, n_ex, n_groups, normalize_by);
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" int64_t odp_linear_moments_blocks(int64_t d_in, int64_t d_out, int32_t guarded) {
  if (d_in <= 0 || d_out <= 0) return 0;
  if (guarded) return MOM_SPLIT;
  const int64_t tiles = ((d_out + OM - 1) / OM) * ((d_in + ON - 1) / ON);
  return (tiles + 7) / 8 * 8;
}

extern "C" int odp_linear_moments(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                                  int32_t n_prob, int32_t total_blocks, const int32_t* seg_row_start,
                                  const int32_t* seg_row_len, const int32_t* seg_example, const double* scales,
                                  int32_t n_ex, int32_t n_groups, float normalize_by, int32_t guarded) {
  int rc = odp_check_table("odp_linear_moments", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (!(normalize_by > 0.0f)) {
    odp_set_error("odp_linear_moments: normalize_by must be > 0, got %g", (double)normalize_by);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (total_blocks == 0) return ODP_OK;
  if (seg_row_start == nullptr || seg_row_len == nullptr || seg_example == nullptr || scales == nullptr ||
      n_ex <= 0 || n_groups <= 0) {
    odp_set_error("odp_linear_moments: null segment/scale arrays or empty batch");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(guarded ? k_lin_moments_guarded : k_lin_moments, dim3(total_blocks), dim3(OUTER_THREADS), 0,
                     odp_hip_stream(stream), problems, work_start, n_prob, seg_row_start, seg_row_len, seg_example,
                     scales, n_ex, n_groups, normalize_by);
  return odp_check_launch("odp_linear_moments");
}
