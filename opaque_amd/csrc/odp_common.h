// Shared device helpers for the DP-SGD clip/noise kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/opaque_dp.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Round-to-nearest-even float -> bf16 bit pattern (NaN stays NaN).
__device__ __forceinline__ uint16_t odp_f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float odp_bf2f(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// A finite float rounded to nearest-even bfloat16, by the hardware
// conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ float odp_round_bf16(float f) {
  return odp_bf2f(__builtin_bit_cast(uint16_t, (__bf16)f));
}

// s_waitcnt immediate: vmcnt <= n (0..63), lgkmcnt and expcnt not waited on.
__host__ __device__ constexpr uint32_t vmcnt_imm(int n) {
  return (uint32_t)(n & 15) | ((uint32_t)(n >> 4) << 14) | 0x0F70u;
}

// Largest p in [0, n) with start[p] <= x. `start` is non-decreasing with
// start[0] == 0 and x < start[n].
__device__ __forceinline__ int odp_find_problem(const int32_t* __restrict__ start, int n, int x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (start[mid] <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Whether `row` lies inside one of the n segments [start[s], start[s]+len[s]).
// Segment starts must be sorted ascending and segments must not overlap.
__device__ __forceinline__ bool odp_row_in_segments(int64_t row, const int32_t* __restrict__ start,
                                                    const int32_t* __restrict__ len, int n) {
  if (n <= 0 || row < start[0]) return false;
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)start[mid] <= row) lo = mid; else hi = mid - 1;
  }
  return row < (int64_t)start[lo] + (int64_t)len[lo];
}

// Stores to global memory through the global address space.  A store
// through a generic pointer becomes a flat store, which also counts in the
// LDS counter: every later wait for an LDS read or lane exchange would then
// wait for the store to complete as well.
#define ODP_GMEM __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ void odp_gstore(T* p, T v) {
  *(ODP_GMEM T*)(ODP_GMEM void*)p = v;
}

// Element i of a tensor of `dtype` as float (float64 rounds to nearest).
__device__ __forceinline__ float odp_load_as_float(const void* p, int64_t i, int dtype) {
  if (dtype == ODP_DTYPE_BF16) return odp_bf2f(((const uint16_t*)p)[i]);
  if (dtype == ODP_DTYPE_F16) return (float)((const _Float16*)p)[i];
  if (dtype == ODP_DTYPE_F64) return (float)((const double*)p)[i];
  return ((const float*)p)[i];
}

// Stores v rounded to nearest-even in `dtype`.
__device__ __forceinline__ void odp_store_from_float(void* p, int64_t i, int dtype, float v) {
  if (dtype == ODP_DTYPE_BF16) odp_gstore((uint16_t*)p + i, odp_f2bf(v));
  else if (dtype == ODP_DTYPE_F16) odp_gstore((_Float16*)p + i, (_Float16)v);
  else if (dtype == ODP_DTYPE_F64) odp_gstore((double*)p + i, (double)v);
  else odp_gstore((float*)p + i, v);
}

// Element i as double (exact for every dtype).
__device__ __forceinline__ double odp_load_as_double(const void* p, int64_t i, int dtype) {
  if (dtype == ODP_DTYPE_F64) return ((const double*)p)[i];
  return (double)odp_load_as_float(p, i, dtype);
}

// Stores a double rounded to nearest-even in `dtype` (float first for the
// 16-bit types, as torch casts float64 tensors).
__device__ __forceinline__ void odp_store_from_double(void* p, int64_t i, int dtype, double v) {
  if (dtype == ODP_DTYPE_F64) odp_gstore((double*)p + i, v);
  else odp_store_from_float(p, i, dtype, (float)v);
}

// Rounds a float to the value it takes when stored in `dtype`.
__device__ __forceinline__ float odp_round_to(float v, int dtype) {
  if (dtype == ODP_DTYPE_BF16) return odp_bf2f(odp_f2bf(v));
  if (dtype == ODP_DTYPE_F16) return (float)(_Float16)v;
  return v;
}

// Bytes per element of `dtype`.
__host__ __device__ __forceinline__ int odp_dtype_size(int dtype) {
  return dtype == ODP_DTYPE_F64 ? 8 : dtype == ODP_DTYPE_F32 ? 4 : 2;
}

// fp64 sums across lanes on the VALU (DPP and readlane instead of LDS lane
// permutes, which would compete with the kernels' LDS reads).  row_sum16
// adds exactly what an xor 1, 2, 4, 8 butterfly adds, in the same order
// (quad pairs, quads, half rows by half-row mirror, rows by row mirror), so
// every lane of a row gets the same value; rows_sum4 returns
// (R0 + R1) + (R2 + R3) of the four rows' values (lanes 0, 16, 32, 48), as
// an xor 16, 32 butterfly does in lane 0.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double row_sum16(double v) {
  v += dpp_f64<0xB1>(v);   // quad_perm 1,0,3,2
  v += dpp_f64<0x4E>(v);   // quad_perm 2,3,0,1
  v += dpp_f64<0x141>(v);  // row_half_mirror
  v += dpp_f64<0x140>(v);  // row_mirror
  return v;
}
__device__ __forceinline__ double lane_f64(double v, int l) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double rows_sum4(double v) {
  return (lane_f64(v, 0) + lane_f64(v, 16)) + (lane_f64(v, 32) + lane_f64(v, 48));
}
