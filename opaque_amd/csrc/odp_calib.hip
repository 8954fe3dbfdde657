// Measurement aid: the dense bf16 MFMA rate the chip sustains with no
// memory traffic, the ceiling against which the full-weight kernels' rates
// are read (the published 2.5 PFLOP/s assumes the peak clock, which the
// chip does not hold under a full MFMA load).
#include "odp_internal.h"

// Each wave runs CAL_ACC independent accumulator chains of
// v_mfma_f32_16x16x32_bf16 over four operand pairs drawn per lane from a
// xorshift stream: operands that change from one MFMA to the next draw the
// power of real data (constant operands let the clock rise well above what
// a GEMM sees).  The sums go to `sink`, so that no MFMA is dead code.
constexpr int CAL_ACC = 16, CAL_THREADS = 256;

__global__ __launch_bounds__(CAL_THREADS) void k_mfma_calibrate(float* __restrict__ sink, int iters) {
  f32x4_t acc[CAL_ACC];
#pragma unroll
  for (int i = 0; i < CAL_ACC; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  bf16x8_t a[4], b[4];
  uint32_t h = threadIdx.x * 2654435761u + blockIdx.x * 40503u + 12345u;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      h ^= h << 13;
      h ^= h >> 17;
      h ^= h << 5;
      a[q][i] = (__bf16)((float)(h & 0xffffu) * (1.f / 65536.f) - 0.5f);
      h ^= h << 13;
      h ^= h >> 17;
      h ^= h << 5;
      b[q][i] = (__bf16)((float)(h & 0xffffu) * (1.f / 65536.f) - 0.5f);
    }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < CAL_ACC; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i & 3], b[(i >> 2) & 3], acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CAL_ACC; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  sink[(int64_t)blockIdx.x * CAL_THREADS + threadIdx.x] = s;
}

extern "C" int odp_calibrate_mfma(odp_stream_t stream, int32_t workgroups, int32_t iters, float* sink) {
  if (workgroups < 1 || workgroups > (1 << 20) || iters < 1 || iters > (1 << 24)) {
    odp_set_error("odp_calibrate_mfma: workgroups (%d) must be in [1, 2^20] and iters (%d) in [1, 2^24]",
                  workgroups, iters);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (sink == nullptr) {
    odp_set_error("odp_calibrate_mfma: null sink");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  hipLaunchKernelGGL(k_mfma_calibrate, dim3(workgroups), dim3(CAL_THREADS), 0, odp_hip_stream(stream), sink, iters);
  return odp_check_launch("odp_calibrate_mfma");
}

extern "C" int64_t odp_calibrate_mfma_flops(int32_t workgroups, int32_t iters) {
  return (int64_t)workgroups * (CAL_THREADS / 64) * iters * CAL_ACC * (2 * 16 * 16 * 32);
}
