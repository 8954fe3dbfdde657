/*
 * opaque_dp.h — C ABI of the MI355X (gfx950) DP-SGD clip + noise core.
 *
 * Every entry point is asynchronous on the caller's HIP stream, takes plain
 * device pointers and sizes, allocates nothing, never throws, and returns an
 * odp_status (0 = success).  On failure odp_last_error() returns a
 * human-readable message for the calling thread.
 *
 * Work is described by "problem tables": device arrays of int64_t rows whose
 * field indices are listed below.  One launch processes every problem of its
 * table, so a whole model's DP step is a handful of launches regardless of
 * depth.
 * Each table comes with a device int32 array work_start[n_prob + 1] holding
 * the cumulative number of workgroups per problem (work_start[0] == 0);
 * the *_blocks() helpers give the per-problem workgroup counts.
 *
 * The reference (JetBrains-Research/opaque) is Python; these entry points
 * replace the following internals of its DP-SGD hot path
 * (paths relative to packages/):
 *   odp_project or odp_pack_planes, odp_seg_factor_project, odp_seg_factor,
 *   odp_seg_factor_stream         -> per-sample LoRA factor gradients,
 *       opaque-patches/src/opaque/api/patches/kernels/lora.py:164-176
 *       (dA[i] = s X[i]^T (G[i] B^T), dB[i] = s (X[i] A)^T G[i]) and the
 *       per-example squared norms of clip_pytree,
 *       opaque-engine/src/opaque/api/engine/clipping/_pytree.py:224-265,520-540
 *   odp_linear_sqnorm             -> per-example squared norm of a full
 *       weight gradient G[i]^T X[i] without materialising it, outer or
 *       token-Gram form (the reference materialises it under vmap(grad),
 *       clipping/_clipped_fun.py:756-762)
 *   odp_clip_factors              -> clip_pytree / auto_scale_pytree ratio,
 *       guard and finalisation, clipping/_pytree.py:106-142,345-431,475-564
 *       and the clipped counts of clipping/_clipped_fun.py:472-523
 *   odp_scale_sum                 -> per-leaf scale, batch sum and
 *       normalize_by, clipping/_pytree.py:553 and
 *       clipping/_clipped_fun.py:115-134,777-782,821-824
 *   odp_linear_clipped_sum        -> the same sum for a full weight,
 *       sum_i c_i G[i]^T X[i] as one GEMM
 *   odp_gaussian_noise            -> the sampler of
 *       opaque-dpsgd/src/opaque/api/dpsgd/noise/_gaussian.py:235-301
 *       (inverse-CDF Gaussian; uniforms from a counter-based Philox4x32-10
 *       stream keyed by the 64-bit RngKey seed instead of a CPU mt19937)
 */
#ifndef OPAQUE_DP_H_
#define OPAQUE_DP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* odp_stream_t; /* == hipStream_t */

typedef enum odp_status {
  ODP_OK = 0,
  ODP_ERR_INVALID_ARGUMENT = 1,
  ODP_ERR_UNSUPPORTED = 2,
  ODP_ERR_HIP = 3
} odp_status;

typedef enum odp_dtype {
  ODP_DTYPE_F32 = 0,
  ODP_DTYPE_BF16 = 1,
  ODP_DTYPE_F16 = 2, /* noise, sqnorm, clip factors and scale-sum only */
  ODP_DTYPE_F64 = 3  /* noise, sqnorm, clip factors and scale-sum only */
} odp_dtype;

typedef enum odp_clip_mode {
  ODP_CLIP_FIXED = 0, /* ratio = C / ||g||, clamped to 1 (clip_pytree) */
  ODP_CLIP_AUTOS = 1  /* ratio = R / (||g|| + gamma), no clamp (auto_scale_pytree) */
} odp_clip_mode;

typedef enum odp_norm_form {
  ODP_FORM_OUTER = 0, /* ||sum_t g_t a_t^T||_F^2 */
  ODP_FORM_GRAM = 1,  /* sum_{t,s} (g_t . g_s)(a_t . a_s), 128-row blocks */
  ODP_FORM_GRAM256 = 2, /* the same sum over 256-row blocks, with scratch */
  ODP_FORM_OUTER_GUARDED = 3 /* OUTER for the segments at risk of float32
                                overflow only (see odp_linear_sqnorm)       */
} odp_norm_form;

/* ---- segments -----------------------------------------------------------
 * Rows of a layer's activations a [n_rows, d_in] and output gradients
 * g [n_rows, d_out] are grouped into segments: seg_row_start[s],
 * seg_row_len[s] (rows of one example, or of one (example, expert) pair),
 * sorted by start and non-overlapping, and seg_example[s] names the example
 * whose norm and clip factor the segment contributes to.  A problem refers
 * to the slice [seg_first, seg_first + n_seg) of these device arrays.      */

/* ---- odp_pack_factors: W[j][k] = A[k][j] ---------------------------------
 * Copies LoRA factors A [d_in][r] (any strides and dtype) into the row-major
 * A^T operand [r][d_in] that odp_project reads (ODP_PJ_W), converting to the
 * activation dtype; one problem per seam.  Replaces the transpose of A that
 * the reference's per-sample gradient forms in torch
 * (opaque-patches/src/opaque/api/patches/kernels/lora.py:164-176), done here
 * on the device so that a call's host work does not touch every factor.    */
enum {
  ODP_PF_SRC = 0,     /* address of A: element (k, j) at SRC + k LD0 + j LD1 elements */
  ODP_PF_LD0 = 1,
  ODP_PF_LD1 = 2,
  ODP_PF_DTYPES = 3,  /* odp_dtype of A | odp_dtype of W << 8 (W: bf16 or f32)        */
  ODP_PF_DIN = 4,
  ODP_PF_R = 5,       /* r <= 64                                                    */
  ODP_PF_DST = 6,     /* address of W rows: element (j, k) at DST + j DIN + k         */
  ODP_PF_FIELDS = 8
};
int64_t odp_pack_factors_blocks(int64_t d_in);
int odp_pack_factors(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                     int32_t n_prob, int32_t total_blocks);

/* ---- odp_pack_planes: Q^T[k][row] = S[row][k] ----------------------------
 * Lays a rank-space product that the seam already computed (V = X A from
 * the LoRA forward, U = G B^T from its input-gradient backward) out as the
 * plane odp_project would have written: rows [0, n_rows), rows outside the
 * problem's segments 0, one plane [k][ldq] at ODP_PL_DST in the activation
 * dtype.  With it the factor kernels read each activation and output
 * gradient once.  The reference computes both products a second time in its
 * per-sample rule (opaque-patches/src/opaque/api/patches/kernels/lora.py:
 * 157-176: grad_out @ B.t() for dX and again per sample, X @ A); here the
 * seam's own are reused.  One workgroup per 256 rows
 * (odp_pack_planes_blocks).                                                 */
enum {
  ODP_PL_SRC = 0,     /* address of S, row-major [n_rows][r], ld = ODP_PL_LDS  */
  ODP_PL_LDS = 1,     /* elements                                             */
  ODP_PL_R = 2,       /* r <= 64                                              */
  ODP_PL_DST = 3,     /* address of the plane                                 */
  ODP_PL_LDQ = 4,     /* row pitch of the plane (elements)                    */
  ODP_PL_NROWS = 5,
  ODP_PL_SEG_FIRST = 6,
  ODP_PL_NSEG = 7,
  ODP_PL_DTYPE = 8,   /* odp_dtype of S and the plane: bf16 or f32            */
  ODP_PL_FIELDS = 12
};
int64_t odp_pack_planes_blocks(int64_t n_rows);
int odp_pack_planes(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                    int32_t n_prob, int32_t total_blocks, const int32_t* seg_row_start,
                    const int32_t* seg_row_len);

/* ---- odp_project: Q^T[k][row] = sum_j P[row][j] * W[k][j] --------------
 * The LoRA rank-space projections U = G B^T and V = X A for the rows of
 * the problem's segments.  Only columns k < r are written, as one plane
 * [k][ldq] at ODP_PJ_Q in P's dtype (bf16 P: the fp32 sums rounded to
 * bf16, as the reference's bf16 X A and G B^T are).
 * bf16 P: the workgroups walk the problem's covered rows (each segment
 *   widened to whole 8-row groups, [start & ~7, ceil8(start + len)),
 *   concatenated in segment order), odp_project_blocks(dtype, covered, r)
 *   of them, covered = odp_project_covered_rows of the problem's segments
 *   (n_rows also works: the surplus workgroups exit).  Rows of a covered
 *   group outside the segments get their products too; other rows are not
 *   written.
 * f32 P: rows [0, n_rows) (pass n_rows); rows outside the segments get 0. */
enum {
  ODP_PJ_P = 0,      /* address of P, row-major, ld = ODP_PJ_LDP elements     */
  ODP_PJ_LDP = 1,
  ODP_PJ_D = 2,      /* contraction length (multiple of 8 for bf16, 4 for f32) */
  ODP_PJ_W = 3,      /* address of W [r][d] row-major, same dtype as P         */
  ODP_PJ_R = 4,      /* r <= 64                                               */
  ODP_PJ_Q = 5,      /* address of the output planes                          */
  ODP_PJ_LDQ = 6,    /* row pitch of Q planes, multiple of 8, >= n_rows + 32   */
  ODP_PJ_NROWS = 7,
  ODP_PJ_SEG_FIRST = 8,
  ODP_PJ_NSEG = 9,
  ODP_PJ_FIELDS = 12
};
int64_t odp_project_blocks(int dtype, int64_t n_rows, int32_t r);
/* Host arrays of one problem's segments (no device access); -1 (and the
 * error text) for null arrays with n_seg > 0. */
int64_t odp_project_covered_rows(const int32_t* seg_row_start, const int32_t* seg_row_len, int32_t n_seg);
/* Every problem of one table must have ceil(ODP_PJ_R / 16) == nkb (1..4). */
int odp_project(odp_stream_t stream, int dtype, const int64_t* problems,
                const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                const int32_t* seg_row_start, const int32_t* seg_row_len, int32_t nkb);

/* ---- odp_seg_factor: per-segment factor gradients and norm partials -----
 * For every segment s and column k < r of Q (up to 4 leaves laid side by
 * side in Q's columns):  pe_leaf[s][k - col0][m] = scaling * sum_{t in s}
 * Q[k][t] * P[t][m],  m < M.  Each workgroup covers FACTOR_MTILE values of
 * m and writes, per leaf, the fp64 sum of squares of each of its four
 * waves to part[seg_example[s] * part_stride + slot_base +
 * ODP_FT_WAVE_SLOTS * tile + wave] (a leaf uses ODP_FT_WAVE_SLOTS slots per
 * tile, so no workgroup barrier is needed).  Requirements: M
 * and the P row pitch are multiples of 8 (bf16) or 4 (f32); Q is the output
 * of odp_project (ldq a multiple of 8 and >= n_rows + 32), readable for
 * 16*ceil(r/16) rows; rows k >= r may hold anything (they are discarded). */
enum {
  ODP_FT_P = 0, ODP_FT_LDP = 1, ODP_FT_M = 2,
  ODP_FT_Q = 3, ODP_FT_LDQ = 4, ODP_FT_R = 5,
  ODP_FT_SEG_FIRST = 6, ODP_FT_NSEG = 7,
  ODP_FT_SCALING = 8, /* double bit pattern                                  */
  ODP_FT_NLEAF = 9,   /* 1..4                                                */
  ODP_FT_LEAF0 = 10,  /* per leaf l: [10+3l] pe address ([n_seg][rank][M], f32,
                         or bf16 when bit 32 of [11+3l] is set; norms square
                         the values as stored), [11+3l] col0 | rank << 16 |
                         pe_bf16 << 32, [12+3l] slot_base;
                         leaves sorted by col0                               */
  ODP_FT_FIELDS = 24,
  ODP_FT_WAVE_SLOTS = 4 /* partial slots per leaf and tile                   */
};
/* M-tiles of a problem (a leaf uses ODP_FT_WAVE_SLOTS partial slots per
 * tile); the bf16 tile width
 * depends on the rank.  Every problem of one table must have
 * ceil(ODP_FT_R / 16) == nkb (1..4).                                       */
int64_t odp_seg_factor_tiles(int dtype, int64_t M, int32_t r);
int odp_seg_factor(odp_stream_t stream, int dtype, const int64_t* problems,
                   const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                   const int32_t* seg_row_start, const int32_t* seg_row_len,
                   const int32_t* seg_example, double* part, int64_t part_stride, int32_t nkb);

/* ---- odp_seg_factor_project: the G side of a LoRA site in one pass ------
 * Replaces the per-sample G-side products of _LoRAWBackward.vmap
 * (opaque-patches/src/opaque/api/patches/kernels/lora.py:164-176):
 * grad_out_Bt = grad_out @ B^T and dB[i] = s * (X[i] A)^T grad_out[i].
 * One bf16 pass over P = G computes, per segment, what odp_project (U =
 * G B^T into the plane at ODP_FP_U) and odp_seg_factor (pe rows and norm
 * partials of the dB leaf, Q = the V plane) would, reading G once.
 * A problem is an odp_seg_factor row with NLEAF == 1 and r <= 16 plus the
 * fields below; one workgroup per segment (total blocks = sum of n_seg).
 * U is written for the rows of the segments only, as odp_project's planes
 * (same ldq as Q).  Segments may be at most odp_factor_project_max_len()
 * rows long (longer segments use odp_project + odp_seg_factor); a longer
 * one that does not fit gets NaN partials and nothing else written.
 * Partial slots and pe layout are odp_seg_factor's.                       */
enum {
  ODP_FP_W = 13,    /* address of B [r][M] bf16 row-major                      */
  ODP_FP_U = 14     /* plane of U [k][ldq], bf16                              */
};
int64_t odp_factor_project_max_len(void);
int odp_seg_factor_project(odp_stream_t stream, const int64_t* problems,
                           const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                           const int32_t* seg_row_start, const int32_t* seg_row_len,
                           const int32_t* seg_example, double* part, int64_t part_stride);

/* ---- odp_seg_factor_stream: factor rows from given planes, streamed ----
 * Replaces the same per-sample products as odp_seg_factor
 * (opaque-patches/src/opaque/api/patches/kernels/lora.py:164-176: dB[i] =
 * s (X[i] A)^T G[i] with Q = the V plane, or dA[i]^T = s (G[i] B^T)^T X[i]
 * with Q = the U plane) for bf16 problems whose leaves each start at a
 * column of Q that is a multiple of 16, with rank <= 16 (at most one leaf
 * per 16-row block of Q), bf16 pe rows, and ceil(ODP_FT_R / 16) == nkb
 * (1..3): the same rows, squares and partial slots as odp_seg_factor with
 * the same nkb, bit for bit, with P streamed through LDS by buffer loads
 * marked non-temporal.  The row's ODP_FT_GROUPS field splits each
 * segment's 256-column tiles into that many groups of consecutive tiles,
 * one workgroup each (1 <= groups <= tiles; odp_seg_factor_stream_groups(M)
 * is the default): workgroups per problem = n_seg * groups.  Segments may
 * be at most odp_factor_project_max_len() rows long; a longer one that
 * does not fit gets NaN partials and nothing else written.               */
enum { ODP_FT_GROUPS = 23 };
int64_t odp_seg_factor_stream_groups(int64_t M);
int odp_seg_factor_stream(odp_stream_t stream, const int64_t* problems,
                          const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                          const int32_t* seg_row_start, const int32_t* seg_row_len,
                          const int32_t* seg_example, double* part, int64_t part_stride, int32_t nkb);

/* ---- odp_sqnorm: squared norms of materialised per-example tensors -------
 * For leaves that are not behind a captured linear op, the per-example
 * gradients X[n_seg][n] are materialised; each workgroup sums x^2
 * (non-finite x counted as 0 unless bit 9 of ODP_SQ_DTYPE is set; squared
 * in float32, or in float64 with bit 8, as clip_pytree's accumulation dtype
 * does) over a chunk
 * of one segment in fp64 and writes part[seg_example[s] * part_stride +
 * slot + chunk]; a problem uses odp_sqnorm_blocks(n) slots.               */
enum {
  ODP_SQ_X = 0, ODP_SQ_N = 1, ODP_SQ_NSEG = 2, ODP_SQ_SEG_FIRST = 3,
  ODP_SQ_SLOT = 4, ODP_SQ_DTYPE = 5, /* x dtype | square in float64 << 8
                                        | keep non-finite x << 9           */
  ODP_SQ_FIELDS = 8
};
int64_t odp_sqnorm_blocks(int64_t n);
int odp_sqnorm(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
               int32_t n_prob, int32_t total_blocks, const int32_t* seg_example,
               double* part, int64_t part_stride);

/* ---- odp_clip_factors ----------------------------------------------------
 * part[n_ex][n_slots] (fp64 squared-norm partials; every slot must have
 * been written or zeroed), group_slot_start[n_groups + 1] (int64, device:
 * group g owns slots [start[g], start[g+1])), thresholds[n_groups] (C_g or
 * R_g, device), guard[2 * n_cls] and cls_dtype[n_cls] (device).  Per example:
 * group squared norms in fp64, ratio per group (mode), then per dtype class
 * c: scale = ratio * guard[2c] - guard[2c+1]; min(1, .) for FIXED;
 * non-finite -> 0; max(0, .); rounded to cls_dtype[c] (any odp_dtype).
 * Outputs: scale_out[c][g][ex] (float64 holding the value as the class
 * dtype stores it),
 * norm_out[ex] = f32(sqrt(total)), group_norm_out[g][ex] (may be null),
 * clipped_out[g][ex] = f32(group norm) > f32(threshold) (uint8, may be
 * null), clipped_total_out[ex] = norm_out > f32(effective threshold).       */
int odp_clip_factors(odp_stream_t stream, const double* part, int64_t n_slots, int32_t n_ex,
                     const int64_t* group_slot_start, int32_t n_groups, const double* thresholds,
                     double effective_threshold, int32_t mode, double gamma,
                     int32_t n_cls, const double* guard, const int32_t* cls_dtype,
                     double* scale_out, float* norm_out, float* group_norm_out,
                     uint8_t* clipped_out, uint8_t* clipped_total_out);

/* ---- odp_clip_materialized_noalloc: the above without caller scratch ------
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Computes what odp_sqnorm (on the table sq_problems /
 * sq_work_start, partial stride n_slots) followed by odp_clip_factors
 * (same remaining arguments and outputs) compute, with the fp64 partials in
 * a static device array of odp_noalloc_max_partials() doubles (8 MiB) that
 * each GPU holds until the process ends, cleared at every call: it returns
 * ODP_ERR_UNSUPPORTED when n_ex * n_slots exceeds that.  Allocates nothing.
 * A table entry whose example index or slot falls outside the n_ex x
 * n_slots partials has its write dropped on the device (nothing is written
 * past the array); the call then reports every example's norm as NaN with
 * zero scales and clear masks, since its partials are incomplete (the
 * launch is asynchronous, so no status code can say so).  Calls that
 * overlap on one GPU share the array and race; the stream must belong to
 * the current device.                                                     */
int64_t odp_noalloc_max_partials(void);
int odp_clip_materialized_noalloc(odp_stream_t stream, const int64_t* sq_problems,
                                  const int32_t* sq_work_start, int32_t sq_n_prob,
                                  int32_t sq_total_blocks, const int32_t* seg_example,
                                  int64_t n_slots, int32_t n_ex, const int64_t* group_slot_start,
                                  int32_t n_groups, const double* thresholds,
                                  double effective_threshold, int32_t mode, double gamma,
                                  int32_t n_cls, const double* guard, const int32_t* cls_dtype,
                                  double* scale_out, float* norm_out, float* group_norm_out,
                                  uint8_t* clipped_out, uint8_t* clipped_total_out);

/* ---- odp_scale_sum: clipped batch sum of stored per-segment gradients ----
 * out = round_out(sum_s t_s) with t_s = round_pe(scale[cls][grp]
 * [seg_example[s]] * pe[s]) (clip_pytree's `scale.to(dtype) * leaf`), the
 * sum in float32, or in float64 for float64 pe or the wide flag; then, if
 * normalize_by != 1, round_out(out / normalize_by).  Optional second
 * output out2 = the same for round_pe(t_s^2).                              */
enum {
  ODP_SS_PE = 0,        /* address of [n_seg][rank][M] in the pe dtype      */
  ODP_SS_M = 1, ODP_SS_RANK = 2,
  ODP_SS_SEG_FIRST = 3, ODP_SS_NSEG = 4,
  ODP_SS_OUT = 5,       /* address of the output leaf                       */
  ODP_SS_FLAGS = 6,     /* out dtype | transpose << 8 | group << 16 | cls << 40
                           | wide << 48 | raw << 52 | pe dtype << 56;
                           transpose 0 writes [rank][M], 1 writes [M][rank];
                           non-finite pe values count 0; raw: the values are
                           already scaled (a caller's scale function) and
                           are summed as they are, scale 1, non-finite kept */
  ODP_SS_OUT2 = 7,      /* address of the second-moment output or 0         */
  ODP_SS_FIELDS = 8
};
int64_t odp_scale_sum_blocks(int64_t n_elems);
int odp_scale_sum(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                  int32_t n_prob, int32_t total_blocks, const int32_t* seg_example,
                  const double* scales, int32_t n_ex, int32_t n_groups, float normalize_by);

/* ---- full-weight linears: per-example norms and the clipped sum ---------
 * A linear y = x W^T over rows of X [n_rows][d_in] and output gradients
 * G [n_rows][d_out] (bf16, row pitches and d_in, d_out multiples of 8) has
 * per-example weight gradients M_s = sum_{t in s} g_t x_t^T ([d_out][d_in]).
 *
 * odp_linear_sqnorm writes fp64 partials of ||M_s||_F^2 to
 * part[seg_example[s] * part_stride + ODP_LN_SLOT + tile], in one of two
 * forms (f32 squares of M's entries, non-finite entries counted as 0, for
 * OUTER; the token-Gram identity sum_{t,u}(x_t.x_u)(g_t.g_u) for GRAM);
 * odp_linear_tiles(form, ...) is the number of slots (and workgroups per
 * segment) a problem uses; GRAM needs ODP_LN_NB = ceil(max_len / 128) of
 * the problem's longest segment.  GRAM256 computes the GRAM sum over pairs
 * of 256-row blocks (nb (nb + 1) / 2 slots per segment, ODP_LN_NB =
 * ceil(max_len / 256)), fewer loads per flop than GRAM; it writes each
 * pair's X block to ODP_LN_SCRATCH, which must hold 65536 floats per
 * (segment, slot) of the problem: n_seg * nb (nb + 1) / 2 * 256 KB.  Replaces the per-example weight
 * gradients that the reference materialises under vmap(grad)
 * (opaque-engine/src/opaque/api/engine/clipping/_clipped_fun.py:756-762)
 * and their squared norms (clipping/_pytree.py:224-265).
 *
 * odp_linear_clipped_sum writes out[o][i] = round_out(sum_s sum_{t in s}
 * g_t[o] bf16(c_s x_t[i])) and then round_out(out / normalize_by) if
 * normalize_by != 1, with c_s = scales[cls][group][seg_example[s]] (the
 * clip factor folded into X's rows, in registers or, with prescaled != 0,
 * by odp_linear_prescale beforehand); one workgroup per 256 x 256 output
 * tile (odp_linear_sum_blocks, padded to a multiple of 8).  Replaces
 * clip_pytree's scale and the batch sum (clipping/_pytree.py:553,
 * clipping/_clipped_fun.py:115-134,821-824).
 *
 * Non-finite inputs.  The reference replaces every non-finite entry of each
 * per-example gradient by 0 before the norm and the scale
 * (clipping/_pytree.py:520-527).  An entry M_s[o][i] is non-finite exactly
 * when column i of X or column o of G holds a NaN/Inf in one of the
 * segment's rows, so zeroing those columns within the segment turns M_s
 * into nan_to_num(M_s).  odp_nonfinite_columns finds the columns; the Gram
 * norm, the prescale and the clipped sum zero them wherever ODP_LN_XMASK /
 * ODP_LN_GMASK are set (the outer norm zeroes non-finite entries of M_s by
 * itself).
 *
 * Overflow.  Where the products of finite inputs may exceed float32 (an
 * entry of M_s itself, or its square in the norm, or an intermediate Gram
 * product), the reference's result is that of the materialised M_s (inf
 * entries zeroed, an inf norm giving scale 0).  odp_nonfinite_columns also
 * records each segment's largest finite |x| and |g| (ODP_NF_AMAX); a
 * segment is at risk when, with a = max|x|, b = max|g| and L its length,
 *   a b max(L, sqrt(d_in d_out)) >= 2^60, d_in a^2 >= 2^124 or d_out b^2 >= 2^124.
 * With ODP_LN_XAMAX / ODP_LN_GAMAX set, the Gram norms skip such segments
 * and ODP_FORM_OUTER_GUARDED computes their outer-form partials (which form
 * M_s tile by tile, as the reference does) into ODP_LN_SLOT + tile; the
 * clipped sum skips a problem with such a segment and odp_linear_moments
 * with guarded != 0 writes it instead.  Below the bound no form can
 * overflow (|M_s| < 2^60, squares and Gram products < 2^124, clipped-sum
 * terms < 2^60 times the clip factor).                                      */
enum {
  ODP_LN_X = 0, ODP_LN_LDX = 1, ODP_LN_G = 2, ODP_LN_LDG = 3,
  ODP_LN_DIN = 4, ODP_LN_DOUT = 5, ODP_LN_SEG_FIRST = 6, ODP_LN_NSEG = 7,
  ODP_LN_SLOT = 8,   /* sqnorm: first partial slot of the weight            */
  ODP_LN_OUT = 9,    /* clipped sum: address of out [d_out][d_in]           */
  ODP_LN_FLAGS = 10, /* clipped sum: out dtype | group << 8 | cls << 24     */
  ODP_LN_NB = 11,    /* GRAM (GRAM256): 128- (256-) row blocks of the longest
                        segment                                             */
  ODP_LN_NROWS = 12, /* prescale: rows of X (the output X' is [n_rows][d_in]) */
  ODP_LN_PE = 13,    /* OUTER sqnorm: address of bf16 [n_seg][d_out][d_in]
                        that receives each M_s (RNE), or 0                  */
  ODP_LN_XMASK = 14, /* GRAM sqnorm, prescale, clipped sum: address of the
                        uint32 column masks of X ([n_seg][ceil(d_in / 32)],
                        odp_nonfinite_columns) or 0 for none                */
  ODP_LN_GMASK = 15, /* GRAM sqnorm, clipped sum: the masks of G
                        ([n_seg][ceil(d_out / 32)]) or 0                    */
  ODP_LN_NFFLAG = 16,/* OUTER sqnorm: address of a uint32 that is OR-ed with
                        1 when an entry of some M_s is non-finite, or 0     */
  ODP_LN_SCRATCH = 17,/* GRAM256 sqnorm: address of the fp32 scratch of the
                        problem ([n_seg][slots][65536], 16-byte aligned)    */
  ODP_LN_OUT2 = 18,  /* moments: address of the second moment [d_out][d_in]
                        (output dtype of ODP_LN_FLAGS) or 0                 */
  ODP_LN_XAMAX = 19, /* GRAM sqnorm, OUTER_GUARDED sqnorm, clipped sum,
                        guarded moments: address of the float bits (uint32)
                        of max |x| per segment of X (ODP_NF_AMAX), or 0 for
                        no overflow check                                   */
  ODP_LN_GAMAX = 20, /* the same for G                                      */
  ODP_LN_FIELDS = 24
};

/* ---- odp_nonfinite_columns: per-segment masks of non-finite columns ------
 * For a bf16 row tensor P [n_rows][d] (row pitch ODP_NF_LDP, d a multiple of
 * 8) and each segment s of the problem, writes mask[s][w] (uint32,
 * w < ceil(d / 32)) whose bit j is set when column 32 w + j holds a NaN or
 * Inf in one of the segment's rows.  Every word is written, so the masks
 * need no clearing.  One workgroup per (segment, 256 columns)
 * (odp_nonfinite_blocks).  Feeds ODP_LN_XMASK / ODP_LN_GMASK.  With
 * ODP_NF_AMAX set it also raises amax[s] (the float bits of a non-negative
 * value, as uint32; the caller zeroes them first) to the largest |value| of
 * a finite entry in the segment's rows.                                     */
enum {
  ODP_NF_P = 0, ODP_NF_LDP = 1, ODP_NF_D = 2, ODP_NF_SEG_FIRST = 3, ODP_NF_NSEG = 4,
  ODP_NF_MASK = 5,   /* address of the uint32 masks [n_seg][ceil(d / 32)]   */
  ODP_NF_AMAX = 6,   /* address of uint32 [n_seg] (zeroed by the caller) or 0 */
  ODP_NF_FIELDS = 8
};
int64_t odp_nonfinite_blocks(int64_t d, int64_t n_seg);
int odp_nonfinite_columns(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                          int32_t n_prob, int32_t total_blocks, const int32_t* seg_row_start,
                          const int32_t* seg_row_len);
int64_t odp_linear_tiles(int form, int64_t d_in, int64_t d_out, int64_t max_seg_len);
/* Workgroups of one sqnorm problem (n_seg segments; padded to a multiple of
 * 8 so that work maps onto the 8 XCDs predictably).                        */
int64_t odp_linear_norm_blocks(int form, int64_t d_in, int64_t d_out, int64_t max_seg_len,
                               int64_t n_seg);
int odp_linear_sqnorm(odp_stream_t stream, int form, const int64_t* problems,
                      const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                      const int32_t* seg_row_start, const int32_t* seg_row_len,
                      const int32_t* seg_example, double* part, int64_t part_stride);
int64_t odp_linear_sum_blocks(int64_t d_in, int64_t d_out);
/* ---- odp_linear_prescale: X' = c_i x_t for the clipped sum ------------
 * The per-example scaling of clip_pytree (scale * leaf, clipping/_pytree.py:
 * 553) moved onto the activations: for every row t of a segment of example
 * i, X'[t] = bf16(c_i * x_t) with c_i the clip factor of the problem's
 * (class, group) (ODP_LN_FLAGS as for the clipped sum); rows in no segment,
 * rows of an example whose factor is 0 and columns set in ODP_LN_XMASK get
 * 0.  odp_linear_clipped_sum with prescaled != 0 reads such an X' in
 * every problem (ODP_LN_X = X', ODP_LN_LDX = d_in) and skips its own
 * scaling; the result is bit-identical.  Problem rows: ODP_LN_X, LDX, DIN,
 * SEG_FIRST, NSEG, NROWS, FLAGS, XMASK, OUT = X' (bf16); one workgroup per
 * 16 rows (odp_linear_prescale_blocks).                                    */
int64_t odp_linear_prescale_blocks(int64_t n_rows);
int odp_linear_prescale(odp_stream_t stream, const int64_t* problems,
                        const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                        const int32_t* seg_row_start, const int32_t* seg_row_len,
                        const int32_t* seg_example, const double* scales, int32_t n_ex,
                        int32_t n_groups);
int odp_linear_clipped_sum(odp_stream_t stream, const int64_t* problems,
                           const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                           const int32_t* seg_row_start, const int32_t* seg_row_len,
                           const int32_t* seg_example, const double* scales, int32_t n_ex,
                           int32_t n_groups, float normalize_by, int32_t prescaled);
/* ---- odp_linear_moments: clipped first and second moments ---------------
 * For each problem (rows as for the clipped sum, plus ODP_LN_OUT2) and each
 * element of the weight: with m = bf16(M_s[o][i]) (0 where non-finite),
 * y_s = bf16(c_s m) and
 *   out[o][i]  = round_out(sum_s y_s),  out2[o][i] = round_out(sum_s bf16(y_s^2)),
 * each sum in fp32 over the segments in order and then divided by
 * normalize_by in the output dtype when it is not 1.  These are the
 * reference's clipped gradient and clipped squared gradient with
 * second_moment=True (clipping/_clipped_fun.py:675-683,777-782,821-824),
 * bit-identical to odp_linear_sqnorm's bf16 store of each M_s followed by
 * odp_scale_sum, without storing M_s.  ODP_LN_OUT2 = 0 writes the first
 * moment only.  One workgroup per 256 x 128 output tile
 * (odp_linear_moments_blocks, padded to a multiple of 8).  With guarded
 * != 0 a problem is written only when one of its segments is at risk of
 * float32 overflow (ODP_LN_XAMAX / GAMAX, the bound above; the clipped sum
 * skips exactly those problems), by a few workgroups that loop over its
 * tiles (odp_linear_moments_blocks with guarded != 0).                      */
int64_t odp_linear_moments_blocks(int64_t d_in, int64_t d_out, int32_t guarded);
int odp_linear_moments(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                       int32_t n_prob, int32_t total_blocks, const int32_t* seg_row_start,
                       const int32_t* seg_row_len, const int32_t* seg_example, const double* scales,
                       int32_t n_ex, int32_t n_groups, float normalize_by, int32_t guarded);

/* ---- odp_gaussian_noise --------------------------------------------------
 * out[i] = round_out(in[i] + sigma * sqrt(2) * erfinv(2u - 1)) for element
 * e = flat_offset + i of the flattened pytree: the inverse-CDF sampler of
 * _gaussian.py:252-266, with u = clamp(u, eps, 1 - eps) of the compute
 * dtype.  Float32 compute (the default) takes the 24-bit uniform u = k 2^-24
 * of a float32 torch.rand, with k = bits [24 (e mod 16), + 24) of the
 * 384-bit string made of the Philox4x32-10 outputs (words in order, bit 0
 * first) for counters 3 (e >> 4) + b, b = 0, 1, 2; erfinv is evaluated as
 * x P(log2(1 - x^2)) (max relative error 4e-7).  Float64 compute
 * (compute_dtype ODP_DTYPE_F64) takes u = (w >> 11) 2^-53 with w = words
 * 2 (e & 1) + 1 : 2 (e & 1) of the block for counter e >> 1, in float64
 * (library erfinv), and casts the result to the output dtype.  A Philox
 * counter is {c (64-bit), stream_tag, 0} and the key the 64-bit seed, so the
 * stream is a pure function of (seed, stream_tag, e).  Inputs are converted
 * to the compute dtype and results rounded to nearest-even in the output
 * dtype.  sigma == 0 copies the input.  With bounded != 0 the Gaussian is
 * renormalised over [low, high] (u -> Phi(za) + u (Phi(zb) - Phi(za)),
 * za = (low - in) / sigma) and the result clamped, as the reference's
 * bounded mode does (low <= 0 <= high).  in and out may alias.  One
 * workgroup covers 4096 consecutive elements (odp_gaussian_noise_blocks).   */
enum {
  ODP_NZ_IN = 0, ODP_NZ_OUT = 1, ODP_NZ_N = 2, ODP_NZ_FLAT_OFFSET = 3,
  ODP_NZ_SIGMA = 4,     /* double bit pattern                               */
  ODP_NZ_DTYPES = 5,    /* in dtype | out dtype << 8 (odp_dtype)            */
  ODP_NZ_FIELDS = 8
};
int64_t odp_gaussian_noise_blocks(int64_t flat_offset, int64_t n);
int odp_gaussian_noise(odp_stream_t stream, const int64_t* problems, const int32_t* work_start,
                       int32_t n_prob, int32_t total_blocks, uint64_t seed, uint32_t stream_tag,
                       int32_t compute_dtype, int32_t bounded, double low, double high);

/* Raw Philox4x32-10 words for counters [ctr0, ctr0 + n), key = seed: for
 * known-answer and determinism tests of the device stream.               */
int odp_philox_words(odp_stream_t stream, uint64_t ctr0, uint32_t ctr2, uint32_t ctr3,
                     uint64_t seed, int64_t n, uint32_t* out /* [n][4] */);

/* The float32 inverse-CDF transform of the noise kernel on its own:
 * out[i] = sqrt(2) * erfinv(2u - 1) for the 24-bit uniform k = k0 + i
 * (u = clamp(k 2^-24, eps, 1 - eps)), k0 + n <= 2^24: for exhaustive
 * accuracy tests against a float64 erfinv.                               */
int odp_noise_icdf(odp_stream_t stream, uint32_t k0, int64_t n, float* out);

/* ---- measurement aid (no counterpart in the reference) --------------------
 * The dense bf16 MFMA rate the GPU sustains with no memory traffic: each of
 * `workgroups` workgroups of 4 waves runs 16 independent chains of
 * v_mfma_f32_16x16x32_bf16 for `iters` rounds on operands that change from
 * one MFMA to the next, and writes one float per thread to sink
 * [workgroups * 256].  odp_calibrate_mfma_flops gives the launch's flops.
 * Used by bench.py to read the full-weight kernels' rates against what the
 * chip holds under a full MFMA load, beside the published peak.           */
int odp_calibrate_mfma(odp_stream_t stream, int32_t workgroups, int32_t iters, float* sink);
int64_t odp_calibrate_mfma_flops(int32_t workgroups, int32_t iters);

/* ---- library -------------------------------------------------------------- */
int odp_abi_version(void);
const char* odp_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* OPAQUE_DP_H_ */
