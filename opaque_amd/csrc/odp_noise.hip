// Gaussian noise for the clipped sum: counter-based Philox4x32-10 uniforms
// (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2,
// 3", SC 2011) mapped through the inverse normal CDF as the reference
// sampler does with its CPU uniforms (opaque-dpsgd/.../noise/_gaussian.py:
// 252-278):
//   u = clamp(u, eps, 1 - eps);  x = c + sigma * sqrt 2 * erfinv(2u - 1)
//
// Float32 compute draws 24-bit uniforms, the grid of a float32 torch.rand:
// thread G covers elements [16 G, 16 G + 16) of the flattened pytree and
// element e takes bits [24 (e mod 16), + 24) of the 384-bit string of the
// Philox outputs for counters 3 G, 3 G + 1, 3 G + 2 (16 uniforms per three
// blocks).  Float64 compute takes 53 bits from two words per element (block
// e >> 1).  Either way the stream is a pure function of (seed, e), so any
// shard of the pytree reproduces the single-GPU values.
//
// The kernel is bound by its VALU work, not by HBM: Philox takes two
// 32 x 32 -> 64 multiplies per round (v_mad_u64_u32) and the inverse CDF a
// log2 and a short polynomial; loads and stores move 16 bytes per lane.
#include "odp_internal.h"

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

namespace {

constexpr int NZ_THREADS = 256;
constexpr int NZ_GROUP = 16;  // elements per thread

// sqrt(2) erfinv(x) = x P(L), L = log2(1 - x^2): the variable of M. Giles,
// "Approximating the erfinv function" (GPU Computing Gems Jade, 2011), with
// this project's own coefficients (opaque_amd/csrc/fit_icdf.py): centre
// L >= -8, max relative error 2.9e-7; tail in sqrt(-L) - mid, 1.4e-7.  The
// coefficients carry 2^-23, the scale of xf = x * 2^23.
constexpr float ICDF_L_SPLIT = -8.0f;
constexpr float ICDF_TAIL_MID = 3.759421349e+00f;
constexpr float ICDF_CENTRE[9] = {1.494066595e-07f, -2.711282043e-08f, 9.330247686e-10f,
                                  1.276801165e-10f, -7.310619991e-12f, -2.111257133e-12f,
                                  -1.305657242e-13f, -1.177457959e-15f, 1.061969808e-16f};
constexpr float ICDF_TAIL[8] = {4.995686709e-07f, 1.408896537e-07f, 8.136734619e-10f,
                                -5.061340236e-10f, 3.071515264e-10f, -1.753577006e-10f,
                                6.185213453e-11f, -5.496441410e-12f};

struct u32x4s {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ u32x4s philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    // Three-input XORs in one gfx950 v_bitop3_b32 each (truth table 0x96).
    const uint32_t n0 = __builtin_amdgcn_bitop3_b32((uint32_t)(p1 >> 32), c1, k0, 0x96);
    const uint32_t n2 = __builtin_amdgcn_bitop3_b32((uint32_t)(p0 >> 32), c3, k1, 0x96);
    c0 = n0;
    c1 = (uint32_t)p1;
    c2 = n2;
    c3 = (uint32_t)p0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return u32x4s{c0, c1, c2, c3};
}

// Constants the inverse CDF needs in vector registers.  A gfx9 VALU
// instruction takes at most one literal, so left to itself the compiler
// re-materialises these with a move for every element; made opaque here,
// they are moved once per thread (the noise kernel is bound by its VALU
// instruction count).
struct IcdfRegs {
  float c8;       // leading coefficient of the centre polynomial
  uint32_t kmax;  // largest 24-bit uniform after the clamp
};
__device__ __forceinline__ IcdfRegs icdf_regs() {
  IcdfRegs R{ICDF_CENTRE[8], 0xFFFFFEu};
  __asm__ volatile("" : "+v"(R.c8), "+v"(R.kmax));
  return R;
}

// sqrt(2) erfinv(x) from xf = x 2^23 and L = log2(1 - x^2).
__device__ __forceinline__ float icdf_poly(float xf, float L, const IcdfRegs& R) {
  float p;
  if (L >= ICDF_L_SPLIT) {
    p = __builtin_fmaf(R.c8, L, ICDF_CENTRE[7]);
#pragma unroll
    for (int i = 6; i >= 0; --i) p = __builtin_fmaf(p, L, ICDF_CENTRE[i]);
  } else {
    const float t = __builtin_amdgcn_sqrtf(-L) - ICDF_TAIL_MID;
    p = ICDF_TAIL[7];
#pragma unroll
    for (int i = 6; i >= 0; --i) p = __builtin_fmaf(p, t, ICDF_TAIL[i]);
  }
  return xf * p;
}

// sqrt(2) erfinv(2u - 1) for u = k 2^-24 clamped to [eps, 1 - eps] (eps =
// 2^-23, float32's machine epsilon), i.e. k clamped to [2, 2^24 - 2].  x =
// (k - 2^23) 2^-23 and 1 - x^2 (one rounding, by FMA) are exact inputs to
// the log.
__device__ __forceinline__ float icdf24(uint32_t k, const IcdfRegs& R) {
  // k = min(max(k, 2), kmax) in one instruction (the compiler splits the
  // clamp in two once kmax is a register).
  __asm__("v_med3_u32 %0, %1, 2, %2" : "=v"(k) : "v"(k), "v"(R.kmax));
  const float xf = (float)((int32_t)k - (1 << 23));
  const float r = __builtin_fmaf(-xf, xf * 0x1p-46f, 1.0f);
  return icdf_poly(xf, __builtin_amdgcn_logf(r), R);
}

// Same for a float32 u already clamped to [eps, 1 - eps] (bounded mode).
__device__ __forceinline__ float icdf_u(float u, const IcdfRegs& R) {
  const float x = __builtin_fmaf(2.0f, u, -1.0f);
  const float r = __builtin_fmaf(-x, x, 1.0f);
  return icdf_poly(x * 0x1p23f, __builtin_amdgcn_logf(r), R);
}

// The 16 24-bit uniforms of thread G from its 12 Philox words: element j
// takes bits [24 j, 24 j + 24) (every 3 words hold 4 uniforms).
__device__ __forceinline__ void uniforms24(int64_t G, uint32_t tag, uint32_t k0, uint32_t k1,
                                           uint32_t (&k)[NZ_GROUP]) {
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const uint64_t ctr = (uint64_t)G * 3u + (uint64_t)b;
    const u32x4s r = philox4x32_10((uint32_t)ctr, (uint32_t)(ctr >> 32), tag, 0u, k0, k1);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    // Words 4b .. 4b + 3 of the string; uniforms j with 24 j in [128 b, 128 b + 128).
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int wi = 4 * b + q;  // word index
      // Uniforms whose first bit lies in word wi.
#pragma unroll
      for (int j = 0; j < NZ_GROUP; ++j) {
        const int bit = 24 * j;
        if ((bit >> 5) != wi) continue;
        const int sh = bit & 31;
        if (sh <= 8) {
          k[j] = (w[q] >> sh) & 0xFFFFFFu;
        } else {
          // Straddles into the next word, which may belong to the next block.
          k[j] = w[q] >> sh;  // low 32 - sh bits; the rest is added below
        }
      }
    }
    // Bits of straddling uniforms that lie in this block's words.
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int wi = 4 * b + q;
#pragma unroll
      for (int j = 0; j < NZ_GROUP; ++j) {
        const int bit = 24 * j;
        const int sh = bit & 31;
        if (sh > 8 && (bit >> 5) + 1 == wi) k[j] = (k[j] | (w[q] << (32 - sh))) & 0xFFFFFFu;
      }
    }
  }
}

// ---- 16-element loads and stores ------------------------------------------
// vec: the 16 elements are in range and 16-byte aligned.
__device__ __forceinline__ void load16(const void* p, int64_t i0, int64_t n, int dt, bool vec,
                                       float (&c)[NZ_GROUP]) {
  if (vec) {
    // Plain loads: the input was usually just written by the scale-sum and
    // may still be cached.
    const ODP_GMEM u32x4_t* v = (const ODP_GMEM u32x4_t*)(const ODP_GMEM void*)((const char*)p + i0 * odp_dtype_size(dt));
    if (dt == ODP_DTYPE_BF16) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4_t w = v[h];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          c[8 * h + 2 * q] = __uint_as_float(w[q] << 16);
          c[8 * h + 2 * q + 1] = __uint_as_float(w[q] & 0xFFFF0000u);
        }
      }
      return;
    }
    if (dt == ODP_DTYPE_F32) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const u32x4_t w = v[h];
#pragma unroll
        for (int q = 0; q < 4; ++q) c[4 * h + q] = __uint_as_float(w[q]);
      }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < NZ_GROUP; ++j) {
    const int64_t i = i0 + j;
    c[j] = (i >= 0 && i < n) ? odp_load_as_float(p, i, dt) : 0.0f;
  }
}

__device__ __forceinline__ void store16(void* p, int64_t i0, int64_t n, int dt, bool vec,
                                        const float (&y)[NZ_GROUP]) {
  if (vec) {
    u32x4_t* v = (u32x4_t*)((char*)p + i0 * odp_dtype_size(dt));
    if (dt == ODP_DTYPE_BF16) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4_t w;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          w[q] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                  (f32x2_t){y[8 * h + 2 * q], y[8 * h + 2 * q + 1]}, bf16x2_t));
        __builtin_nontemporal_store(w, (ODP_GMEM u32x4_t*)(ODP_GMEM void*)(v + h));
      }
      return;
    }
    if (dt == ODP_DTYPE_F32) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const u32x4_t w = {__float_as_uint(y[4 * h]), __float_as_uint(y[4 * h + 1]),
                           __float_as_uint(y[4 * h + 2]), __float_as_uint(y[4 * h + 3])};
        __builtin_nontemporal_store(w, (ODP_GMEM u32x4_t*)(ODP_GMEM void*)(v + h));
      }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < NZ_GROUP; ++j) {
    const int64_t i = i0 + j;
    if (i >= 0 && i < n) odp_store_from_float(p, i, dt, y[j]);
  }
}

struct NoiseProblem {
  const void* in;
  void* out;
  int64_t n, off;
  double sigma;
  int idt, odt;
};

__device__ __forceinline__ NoiseProblem read_noise_problem(const int64_t* f) {
  NoiseProblem P;
  P.in = (const void*)f[ODP_NZ_IN];
  P.out = (void*)f[ODP_NZ_OUT];
  P.n = f[ODP_NZ_N];
  P.off = f[ODP_NZ_FLAT_OFFSET];
  P.sigma = __longlong_as_double(f[ODP_NZ_SIGMA]);
  const int64_t d = f[ODP_NZ_DTYPES];
  P.idt = (int)(d & 0xff);
  P.odt = (int)((d >> 8) & 0xff);
  return P;
}

// Float64 compute (compute_dtype=torch.float64): u = k 2^-53 from the top 53
// bits of words 2 (e & 1) + 1 : 2 (e & 1) of block e >> 1, the device math
// library's double erfinv, and the reference's float64 arithmetic.  Its own
// kernel: the double-precision library calls need far more registers than
// the float32 path.
template <bool BOUNDED>
__global__ __launch_bounds__(NZ_THREADS) void k_gaussian_noise_f64(const int64_t* __restrict__ probs,
                                                                   const int32_t* __restrict__ ws, int n_prob,
                                                                   uint32_t k0, uint32_t k1, uint32_t tag,
                                                                   double low, double high) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const NoiseProblem P = read_noise_problem(probs + (int64_t)p * ODP_NZ_FIELDS);
  const int64_t G = (P.off / NZ_GROUP) + (int64_t)(bid - ws[p]) * NZ_THREADS + threadIdx.x;
  const int64_t i0 = G * NZ_GROUP - P.off;
  if (i0 >= P.n) return;
  const double eps = 2.220446049250313e-16;  // 2^-52
  const double s2 = P.sigma * 1.4142135623730951;
#pragma unroll 1
  for (int b = 0; b < NZ_GROUP / 2; ++b) {
    uint64_t bits[2] = {0, 0};
    if (P.sigma != 0.0) {
      const uint64_t ctr = (uint64_t)G * (NZ_GROUP / 2) + (uint64_t)b;
      const u32x4s r = philox4x32_10((uint32_t)ctr, (uint32_t)(ctr >> 32), tag, 0u, k0, k1);
      bits[0] = ((uint64_t)r.y << 32) | r.x;
      bits[1] = ((uint64_t)r.w << 32) | r.z;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t i = i0 + 2 * b + h;
      if (i < 0 || i >= P.n) continue;
      const double c = odp_load_as_double(P.in, i, P.idt);
      double y = c;
      if (P.sigma != 0.0) {
        double u = (double)(bits[h] >> 11) * 1.1102230246251565e-16;  // 2^-53
        if (BOUNDED) {
          const double za = (low - c) / P.sigma, zb = (high - c) / P.sigma;
          const double a = 0.5 * (1.0 + erf(za / 1.4142135623730951));
          const double bb = 0.5 * (1.0 + erf(zb / 1.4142135623730951));
          u = a + u * (bb - a);
        }
        u = fmin(fmax(u, eps), 1.0 - eps);
        y = c + s2 * erfinv(2.0 * u - 1.0);
      }
      if (BOUNDED) y = fmin(fmax(y, low), high);
      odp_store_from_double(P.out, i, P.odt, y);
    }
  }
}

template <bool BOUNDED>
__global__ __launch_bounds__(NZ_THREADS) void k_gaussian_noise(const int64_t* __restrict__ probs,
                                                               const int32_t* __restrict__ ws,
                                                               int n_prob, uint32_t k0, uint32_t k1,
                                                               uint32_t tag, double low, double high) {
  const int bid = blockIdx.x;
  const int p = odp_find_problem(ws, n_prob, bid);
  const NoiseProblem P = read_noise_problem(probs + (int64_t)p * ODP_NZ_FIELDS);
  const int64_t G = (P.off / NZ_GROUP) + (int64_t)(bid - ws[p]) * NZ_THREADS + threadIdx.x;
  const int64_t i0 = G * NZ_GROUP - P.off;  // leaf index of the thread's first element
  if (i0 >= P.n) return;
  const bool whole = i0 >= 0 && i0 + NZ_GROUP <= P.n;
  const bool vin = whole && (((uintptr_t)P.in + (uint64_t)i0 * odp_dtype_size(P.idt)) & 15) == 0;
  const bool vout = whole && (((uintptr_t)P.out + (uint64_t)i0 * odp_dtype_size(P.odt)) & 15) == 0;
  const float lo = (float)low, hi = (float)high;
  float v[NZ_GROUP];
  load16(P.in, i0, P.n, P.idt, vin, v);
  if (P.sigma == 0.0) {
    // Copy (clamped to the bound): the reference returns its input unchanged.
    if (BOUNDED) {
#pragma unroll
      for (int j = 0; j < NZ_GROUP; ++j) v[j] = fminf(fmaxf(v[j], lo), hi);
    }
    store16(P.out, i0, P.n, P.odt, vout, v);
    return;
  }
  uint32_t k[NZ_GROUP];
  uniforms24(G, tag, k0, k1, k);
  const float sd = (float)P.sigma;
  const IcdfRegs R = icdf_regs();
  if (!BOUNDED) {
#pragma unroll
    for (int j = 0; j < NZ_GROUP; ++j) v[j] = __builtin_fmaf(sd, icdf24(k[j], R), v[j]);
  } else {
    // Gaussian renormalised over [lo, hi] by the inverse CDF, then clamped
    // (bounded Gaussian mechanism, _gaussian.py:268-276).
    const float eps = 1.1920928955078125e-07f;  // float32 machine epsilon, 2^-23
    const float sqrt2 = 1.41421356237309515f;
#pragma unroll 1
    for (int j = 0; j < NZ_GROUP; ++j) {
      const float c = v[j];
      const float za = __fdiv_rn(__fsub_rn(lo, c), sd), zb = __fdiv_rn(__fsub_rn(hi, c), sd);
      const float a = 0.5f * (1.0f + erff(__fdiv_rn(za, sqrt2)));
      const float b = 0.5f * (1.0f + erff(__fdiv_rn(zb, sqrt2)));
      float u = __fadd_rn(a, __fmul_rn((float)k[j] * 0x1p-24f, __fsub_rn(b, a)));
      u = fminf(fmaxf(u, eps), 1.0f - eps);
      v[j] = fminf(fmaxf(__builtin_fmaf(sd, icdf_u(u, R), c), lo), hi);
    }
  }
  store16(P.out, i0, P.n, P.odt, vout, v);
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

__global__ void k_noise_icdf(uint32_t k0, int64_t n, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = icdf24((k0 + (uint32_t)i) & 0xFFFFFFu, icdf_regs());
}

}  // namespace

extern "C" int64_t odp_gaussian_noise_blocks(int64_t flat_offset, int64_t n) {
  if (n <= 0 || flat_offset < 0) return 0;
  const int64_t groups = (flat_offset + n + NZ_GROUP - 1) / NZ_GROUP - flat_offset / NZ_GROUP;
  return (groups + NZ_THREADS - 1) / NZ_THREADS;
}

extern "C" int odp_gaussian_noise(odp_stream_t stream, const int64_t* problems,
                                  const int32_t* work_start, int32_t n_prob, int32_t total_blocks,
                                  uint64_t seed, uint32_t stream_tag, int32_t compute_dtype,
                                  int32_t bounded, double low, double high) {
  int rc = odp_check_table("odp_gaussian_noise", problems, work_start, n_prob, total_blocks);
  if (rc != ODP_OK) return rc;
  if (compute_dtype != ODP_DTYPE_F32 && compute_dtype != ODP_DTYPE_F64) {
    odp_set_error("odp_gaussian_noise: compute_dtype %d is neither float32 nor float64", compute_dtype);
    return ODP_ERR_UNSUPPORTED;
  }
  if (bounded && !(low <= 0.0 && 0.0 <= high && low < high)) {
    odp_set_error("odp_gaussian_noise: bound (%g, %g) must satisfy low <= 0 <= high, low < high", low, high);
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (total_blocks == 0) return ODP_OK;
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const dim3 grid(total_blocks), block(NZ_THREADS);
  hipStream_t s = odp_hip_stream(stream);
  if (compute_dtype == ODP_DTYPE_F64) {
    if (bounded)
      hipLaunchKernelGGL(k_gaussian_noise_f64<true>, grid, block, 0, s, problems, work_start, n_prob, k0, k1,
                         stream_tag, low, high);
    else
      hipLaunchKernelGGL(k_gaussian_noise_f64<false>, grid, block, 0, s, problems, work_start, n_prob, k0, k1,
                         stream_tag, low, high);
  } else if (bounded) {
    hipLaunchKernelGGL(k_gaussian_noise<true>, grid, block, 0, s, problems, work_start, n_prob, k0, k1,
                       stream_tag, low, high);
  } else {
    hipLaunchKernelGGL(k_gaussian_noise<false>, grid, block, 0, s, problems, work_start, n_prob, k0, k1,
                       stream_tag, low, high);
  }
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

extern "C" int odp_noise_icdf(odp_stream_t stream, uint32_t k0, int64_t n, float* out) {
  if (n < 0 || n > ((int64_t)1 << 24) || (n > 0 && out == nullptr) || k0 >= (1u << 24)) {
    odp_set_error("odp_noise_icdf: need 0 <= n <= 2^24, k0 < 2^24 and a non-null out");
    return ODP_ERR_INVALID_ARGUMENT;
  }
  if (n == 0) return ODP_OK;
  hipLaunchKernelGGL(k_noise_icdf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     odp_hip_stream(stream), k0, n, out);
  return odp_check_launch("odp_noise_icdf");
}
