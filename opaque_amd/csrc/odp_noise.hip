// Gaussian noise for the clipped sum: counter-based Philox4x32-10 uniforms
// (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2,
// 3", SC 2011) mapped through the inverse normal CDF exactly as the
// reference sampler does with its CPU uniforms
// (opaque-dpsgd/.../noise/_gaussian.py:252-278):
//   u = clamp(u, eps, 1 - eps);  x = c + f32(sigma * sqrt 2) * erfinv(2u - 1)
// Element e of the flattened pytree takes word (e & 3) of the Philox block
// with counter e >> 2, so the stream is a pure function of (seed, e) and any
// shard of the pytree reproduces the single-GPU values.
#include "odp_internal.h"

namespace {

constexpr int NZ_THREADS = 256;

struct u32x4s {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ u32x4s philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return u32x4s{c0, c1, c2, c3};
}

__global__ __launch_bounds__(NZ_THREADS) void k_gaussian_noise(const int64_t* __restrict__ probs,
                                                               const int32_t* __restrict__ ws,
                                                               int n_prob, uint32_t k0, uint32_t k1,
                                                               uint32_t tag) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const int64_t* f = probs + (int64_t)p * ODP_NZ_FIELDS;
  const void* in = (const void*)f[ODP_NZ_IN];
  void* out = (void*)f[ODP_NZ_OUT];
  const int64_t n = f[ODP_NZ_N], off = f[ODP_NZ_FLAT_OFFSET];
  const double sigma = __longlong_as_double(f[ODP_NZ_SIGMA]);
  const int idt = (int)(f[ODP_NZ_DTYPES] & 0xff), odt = (int)((f[ODP_NZ_DTYPES] >> 8) & 0xff);

  const int64_t q = (off >> 2) + (int64_t)(bid - ws[p]) * NZ_THREADS + threadIdx.x;
  const int64_t e_lo = q * 4;
  if (e_lo >= off + n) return;

  if (sigma == 0.0) {
    const bool bnd = ((f[ODP_NZ_DTYPES] >> 16) & 1) != 0;
    const float lo0 = (float)__longlong_as_double(f[ODP_NZ_LOW]);
    const float hi0 = (float)__longlong_as_double(f[ODP_NZ_HIGH]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t e = e_lo + j;
      if (e < off || e >= off + n) continue;
      float v = odp_load_as_float(in, e - off, idt);
      if (bnd) v = fminf(fmaxf(v, lo0), hi0);
      odp_store_from_float(out, e - off, odt, v);
    }
    return;
  }

  const bool bounded = ((f[ODP_NZ_DTYPES] >> 16) & 1) != 0;
  const float lo_b = (float)__longlong_as_double(f[ODP_NZ_LOW]);
  const float hi_b = (float)__longlong_as_double(f[ODP_NZ_HIGH]);
  const float sd = (float)sigma;
  const float s2 = (float)(sigma * 1.4142135623730951);
  const u32x4s r = philox4x32_10((uint32_t)q, (uint32_t)((uint64_t)q >> 32), tag, 0u, k0, k1);
  const uint32_t words[4] = {r.x, r.y, r.z, r.w};
  const float eps = 1.1920928955078125e-07f;  // float32 machine epsilon, 2^-23
  const float inv_sqrt2 = 0.70710678118654752f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t e = e_lo + j;
    if (e < off || e >= off + n) continue;
    float u = (float)(words[j] >> 8) * 5.9604644775390625e-08f;  // 2^-24
    const float c = odp_load_as_float(in, e - off, idt);
    if (bounded) {
      // Gaussian renormalised over [lo, hi] by inverse CDF, then clamped
      // (bounded Gaussian mechanism, _gaussian.py:268-276).
      const float za = __fdiv_rn(__fsub_rn(lo_b, c), sd), zb = __fdiv_rn(__fsub_rn(hi_b, c), sd);
      const float a = 0.5f * (1.0f + erff(za * inv_sqrt2));
      const float b = 0.5f * (1.0f + erff(zb * inv_sqrt2));
      u = __fadd_rn(a, __fmul_rn(u, __fsub_rn(b, a)));
    }
    u = fminf(fmaxf(u, eps), 1.0f - eps);
    const float z = erfinvf(__fsub_rn(__fmul_rn(2.0f, u), 1.0f));
    float y = __fadd_rn(c, __fmul_rn(s2, z));
    if (bounded) y = fminf(fmaxf(y, lo_b), hi_b);
    odp_store_from_float(out, e - off, odt, y);
  }
}

__global__ void k_philox_words(uint64_t ctr0, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1,
                               int64_t n, uint32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t c = ctr0 + (uint64_t)i;
  const u32x4s r = philox4x32_10((uint32_t)c, (uint32_t)(c >> 32), c2, c3, k0, k1);
  out[4 * i + 0] = r.x;
  out[4 * i + 1] = r.y;
  out[4 * i + 2] = r.z;
  out[4 * i + 3] = r.w;
}

}  // namespace

extern "C" int64_t odp_gaussian_noise_blocks(int64_t flat_offset, int64_t n) {
  if (n <= 0 || flat_offset < 0) return 0;
  const int64_t quads = ((flat_offset + n + 3) >> 2) - (flat_offset >> 2);
  return (quads + NZ_THREADS - 1) / NZ_THREADS;
}

extern "C" int odp_gaussian_noise(odp_stream_t stream, const int64_t* problems,
                                  const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                                  uint64_t seed, uint32_t stream_tag) {
  int rc = odp_check_table("odp_gaussian_noise", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (total_blocks == 0) return ODP_OK;
  hipLaunchKernelGGL(k_gaussian_noise, dim3(total_blocks), dim3(NZ_THREADS), 0,
                     odp_hip_stream(stream), problems, work_start, n_prob, (uint32_t)seed,
                     (uint32_t)(seed >> 32), stream_tag);
  return odp_check_launch("odp_gaussian_noise");
}

extern "C" int odp_philox_words(odp_stream_t stream, uint64_t ctr0, uint32_t ctr2, uint32_t ctr3,
                                uint64_t seed, int64_t n, uint32_t* out) {
  if (n < 0 || (n > 0 && out == nullptr)) {
    odp_set_error("odp_philox_words: bad n or null out");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (n == 0) return ODP_OK;
  if (n > (int64_t)1 << 30) {
    odp_set_error("odp_philox_words: n too large");
    return ODP_ERR_UNSUPPORTED;
  }
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_philox_words, dim3((unsigned)blocks), dim3(256), 0, odp_hip_stream(stream),
                     ctr0, ctr2, ctr3, (uint32_t)seed, (uint32_t)(seed >> 32), n, out);
  return odp_check_launch("odp_philox_words");
}
