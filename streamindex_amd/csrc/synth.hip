// Counter-based N(0,1) draws for the benchmarks' and tests' synthetic
// inputs.  Element i of stream `stream` under `seed` depends on (seed,
// stream, i) only, so a tensor is the same on every box, ROCm version and
// launch shape, and any slice of it can be recomputed on the CPU (the oracle
// restates this generator in C and the tests compare the two bit for bit).
//
//   * bits: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
//     numbers: as easy as 1, 2, 3", SC 2011), key (seed lo, seed hi), counter
//     (i/4 lo, i/4 hi, stream, 0); the four words of a counter feed elements
//     4q .. 4q+3;
//   * N(0,1): Box-Muller on word pairs (x0, x1) and (x2, x3):
//     u1 = ((x >> 8) + 1) 2^-24 in (0, 1], u2 = (y >> 8) 2^-24,
//     r = sqrt(-2 ln u1), even element r cos(2 pi u2), odd element r sin(2 pi u2);
//   * ln, sin, cos, the reciprocal and the square root are built from
//     additions, multiplies and explicit fused multiply-adds only (no library
//     transcendental, division or square root), so every step is an exactly
//     specified IEEE operation that the CPU restatement reproduces bit for bit.
//   * out = round-to-nearest-even(n * scale) in fp32 or bf16.
#include <stdint.h>

#include "si_status.h"

namespace si {

#pragma clang fp contract(off)

__device__ __forceinline__ void philox_round(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c[0];
  const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c[2];
  const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
  const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
  c[0] = hi1 ^ c[1] ^ k0;
  c[1] = lo1;
  c[2] = hi0 ^ c[3] ^ k1;
  c[3] = lo0;
}

__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    philox_round(c, k0, k1);
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// 1/d for d in [1.70, 2.42]: a linear seed (within 3 %) and three
// Newton-Raphson steps, multiplies and fused multiply-adds only (so the CPU
// restatement rounds every step identically; a library division need not).
__device__ __forceinline__ float synth_recip(float d) {
  float y = __builtin_fmaf(-0.225f, d, 0.96f);
#pragma unroll
  for (int i = 0; i < 3; ++i) y = __builtin_fmaf(y, __builtin_fmaf(-d, y, 1.0f), y);
  return y;
}

// sqrt(t) for t in [0, 34]: t / sqrt(t) from the bit-pattern seed of
// 1/sqrt(t) (Lomont, "Fast inverse square root", 2003) and three Newton steps
// y <- y (3/2 - t/2 y^2), multiplies and fused multiply-adds only.
__device__ __forceinline__ float synth_sqrt(float t) {
  if (!(t > 0.0f)) return 0.0f;
  float y = __uint_as_float(0x5F3759DFu - (__float_as_uint(t) >> 1));
  const float h = 0.5f * t;
#pragma unroll
  for (int i = 0; i < 3; ++i) y = y * __builtin_fmaf(-(h * y), y, 1.5f);
  return t * y;
}

// ln(u) for u in [2^-24, 1]: u = m 2^e with m in (sqrt(1/2), sqrt(2)],
// ln m = 2 atanh(s), s = (m - 1)/(m + 1), |s| <= 0.1716 (odd series to s^11).
__device__ __forceinline__ float synth_log(float u) {
  uint32_t b = __float_as_uint(u);
  int e = static_cast<int>(b >> 23) - 127;
  float m = __uint_as_float((b & 0x7FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) * synth_recip(m + 1.0f);
  const float s2 = s * s;
  float p = __builtin_fmaf(s2, 0.18181818f, 0.22222222f);
  p = __builtin_fmaf(s2, p, 0.28571429f);
  p = __builtin_fmaf(s2, p, 0.4f);
  p = __builtin_fmaf(s2, p, 0.66666667f);
  const float lnm = __builtin_fmaf(s * s2, p, 2.0f * s);
  const float ef = static_cast<float>(e);
  return __builtin_fmaf(ef, 0.693145752f, __builtin_fmaf(ef, 1.42860677e-06f, lnm));
}

// cos and sin of phi in [0, pi/2) (Taylor to phi^12 / phi^11).
__device__ __forceinline__ void synth_sincos(float phi, float& c, float& s) {
  const float x2 = phi * phi;
  float pc = __builtin_fmaf(x2, 2.08767570e-09f, -2.75573192e-07f);
  pc = __builtin_fmaf(x2, pc, 2.48015873e-05f);
  pc = __builtin_fmaf(x2, pc, -1.38888889e-03f);
  pc = __builtin_fmaf(x2, pc, 4.16666667e-02f);
  pc = __builtin_fmaf(x2, pc, -0.5f);
  c = __builtin_fmaf(x2, pc, 1.0f);
  float ps = __builtin_fmaf(x2, -2.50521084e-08f, 2.75573192e-06f);
  ps = __builtin_fmaf(x2, ps, -1.98412698e-04f);
  ps = __builtin_fmaf(x2, ps, 8.33333333e-03f);
  ps = __builtin_fmaf(x2, ps, -0.166666667f);
  s = __builtin_fmaf(phi * x2, ps, phi);
}

// The two normals of one Box-Muller pair.
__device__ __forceinline__ void synth_box_muller(uint32_t x, uint32_t y, float& n0, float& n1) {
  const float u1 = static_cast<float>((x >> 8) + 1u) * 5.9604644775390625e-08f;  // 2^-24
  const float r = synth_sqrt(-2.0f * synth_log(u1));
  const uint32_t y24 = y >> 8;
  const uint32_t quad = y24 >> 22;
  const float phi = static_cast<float>(y24 & 0x3FFFFFu) * 2.384185791015625e-07f * 1.57079637f;  // f 2^-22 pi/2
  float c, s;
  synth_sincos(phi, c, s);
  float cs, sn;
  if (quad == 0) {
    cs = c; sn = s;
  } else if (quad == 1) {
    cs = -s; sn = c;
  } else if (quad == 2) {
    cs = -c; sn = -s;
  } else {
    cs = s; sn = -c;
  }
  n0 = r * cs;
  n1 = r * sn;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// One thread per group of four consecutive elements (one Philox counter).
template <bool BF16>
__global__ void fill_normal_kernel(void* out, int64_t n, uint32_t k0, uint32_t k1, uint32_t stream, float scale) {
  const int64_t nq = (n + 3) / 4;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < nq;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    uint32_t c[4] = {static_cast<uint32_t>(q), static_cast<uint32_t>(static_cast<uint64_t>(q) >> 32), stream, 0u};
    philox4x32_10(c, k0, k1);
    float v[4];
    synth_box_muller(c[0], c[1], v[0], v[1]);
    synth_box_muller(c[2], c[3], v[2], v[3]);
    const int64_t i0 = q * 4;
    if (BF16) {
      uint16_t* o = static_cast<uint16_t*>(out);
      if (i0 + 4 <= n && (reinterpret_cast<uintptr_t>(o + i0) & 7) == 0) {
        const uint64_t w = static_cast<uint64_t>(f32_to_bf16_rne(v[0] * scale)) |
                           (static_cast<uint64_t>(f32_to_bf16_rne(v[1] * scale)) << 16) |
                           (static_cast<uint64_t>(f32_to_bf16_rne(v[2] * scale)) << 32) |
                           (static_cast<uint64_t>(f32_to_bf16_rne(v[3] * scale)) << 48);
        *reinterpret_cast<uint64_t*>(o + i0) = w;
      } else {
        for (int j = 0; j < 4 && i0 + j < n; ++j) o[i0 + j] = f32_to_bf16_rne(v[j] * scale);
      }
    } else {
      float* o = static_cast<float*>(out);
      for (int j = 0; j < 4 && i0 + j < n; ++j) o[i0 + j] = v[j] * scale;
    }
  }
}

#pragma clang fp contract(on)

}  // namespace si

using namespace si;

extern "C" int si_fill_normal(void* out, int dtype, int64_t n, uint64_t seed, uint32_t stream, float scale,
                              void* hip_stream) {
  if (n < 0) return set_error(SI_ERR_INVALID, "negative element count");
  if (dtype != 0 && dtype != 1) return set_error(SI_ERR_INVALID, "dtype must be 0 (fp32) or 1 (bf16)");
  if (n == 0) return SI_OK;
  if (!out) return set_error(SI_ERR_INVALID, "null output");
  if (reinterpret_cast<uintptr_t>(out) & (dtype ? 1 : 3)) return set_error(SI_ERR_INVALID, "misaligned output");
  const int64_t nq = (n + 3) / 4;
  const int64_t blocks64 = (nq + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(blocks64 < 65536 * 16 ? blocks64 : 65536 * 16);
  const uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  if (dtype) {
    hipLaunchKernelGGL(fill_normal_kernel<true>, dim3(blocks), dim3(256), 0, st, out, n, k0, k1, stream, scale);
  } else {
    hipLaunchKernelGGL(fill_normal_kernel<false>, dim3(blocks), dim3(256), 0, st, out, n, k0, k1, stream, scale);
  }
  return check_launch("fill_normal_kernel");
}
