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

__device__ __forceinline__ float odp_load_as_float(const void* p, int64_t i, int dtype) {
  if (dtype == ODP_DTYPE_BF16) return odp_bf2f(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

__device__ __forceinline__ void odp_store_from_float(void* p, int64_t i, int dtype, float v) {
  if (dtype == ODP_DTYPE_BF16) odp_gstore((uint16_t*)p + i, odp_f2bf(v));
  else odp_gstore((float*)p + i, v);
}

// Rounds a float to the value it takes when stored in `dtype`.
__device__ __forceinline__ float odp_round_to(float v, int dtype) {
  if (dtype == ODP_DTYPE_BF16) return odp_bf2f(odp_f2bf(v));
  return v;
}
