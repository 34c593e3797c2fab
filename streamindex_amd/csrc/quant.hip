// FP8 / FP4 activation quantisation and the token compressor for gfx950.
//
// Reference behaviour being replaced:
//   * flash_sparse/utils/quantization.py:19-37  (act_quant_simulate: per-block
//     fp8 e4m3 quantise-dequantise, scale = amax / 448)
//   * flash_sparse/utils/quantization.py:40-65  (fp4_act_quant_simulate: per-block
//     e2m1 grid snap, scale = amax / 6)
//   * flash_sparse/reference.py:176-272          (reference_token_compressor,
//     eq. 11-12 with overlap, eq. 22-23 without)
//   * flash_sparse/utils/compression.py:13-24    (softmax_gated_pool)
//
// The simulate kernels reproduce the reference's torch arithmetic step by
// step, including the rounding to the input dtype after every elementwise op
// (bf16 / fp16 results are rounded to nearest even, as torch's CPU and GPU
// kernels do), so their outputs are bit-identical to the reference formulas.
// The packing kernels write the production formats the quantised indexer
// reads: fp8 e4m3 values with one fp32 scale per block, and fp4 e2m1 values
// packed two per byte (element 2i in the low nibble) with power-of-two
// (UE8M0) scales.  All are bandwidth-bound: one thread handles 8 elements, a
// block of `bs` elements is reduced across bs/8 adjacent lanes.
#include <hip/hip_fp16.h>

#include <string>

#include "si_common.h"
#include "si_status.h"

namespace si {

// ---- rounding helpers --------------------------------------------------------
// dtype codes: 0 = fp32, 1 = bf16, 2 = fp16
template <int DT>
struct Elt;
template <>
struct Elt<0> {
  using T = float;
  static __device__ __forceinline__ float load(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  static __device__ __forceinline__ float round(float x) { return x; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) { static_cast<float*>(p)[i] = x; }
};
__device__ __forceinline__ float bf16_round(float x) {
  // round to nearest even (NaN kept quiet)
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(u | 0x00400000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}
template <>
struct Elt<1> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
  }
  static __device__ __forceinline__ float round(float x) { return bf16_round(x); }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(__float_as_uint(bf16_round(x)) >> 16);
  }
};
template <>
struct Elt<2> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return __half2float(static_cast<const __half*>(p)[i]);
  }
  static __device__ __forceinline__ float round(float x) { return __half2float(__float2half_rn(x)); }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) {
    static_cast<__half*>(p)[i] = __float2half_rn(x);
  }
};

// Nearest fp8 e4m3 (OCP "fn": bias 7, no infinities, max 448) value to x,
// ties to even; |x| <= 448 here (callers clamp).  Returns the value as float.
__device__ __forceinline__ float e4m3_round(float x) {
  const float a = __builtin_fabsf(x);
  if (!(a > 0.f)) return x;  // +-0 (and NaN) unchanged
  int e;
  __builtin_frexpf(a, &e);        // a = f 2^e, f in [0.5, 1)
  int ex = e - 1;                 // a = g 2^ex, g in [1, 2)
  if (ex < -6) ex = -6;           // subnormals share the 2^-6 binade's quantum
  const float q = __builtin_ldexpf(1.0f, ex - 3);  // spacing: 3 mantissa bits
  const float r = __builtin_rintf(a / q) * q;      // a / q exact (power of two); rint = ties to even
  return __builtin_copysignf(r > 448.f ? 448.f : r, x);
}
// Byte encoding of an e4m3 value produced by e4m3_round.
__device__ __forceinline__ uint8_t e4m3_bits(float v) {
  const uint32_t sign = __float_as_uint(v) >> 31;
  const float a = __builtin_fabsf(v);
  uint32_t code;
  if (a < 0.015625f) {  // subnormal: m 2^-9
    code = static_cast<uint32_t>(a * 512.f);
  } else {
    int e;
    const float f = __builtin_frexpf(a, &e);  // a = f 2^e
    const uint32_t m = static_cast<uint32_t>((f * 2.f - 1.f) * 8.f);
    code = (static_cast<uint32_t>(e - 1 + 7) << 3) | m;
  }
  return static_cast<uint8_t>((sign << 7) | code);
}

// e2m1 grid as the reference lists it (ascending), used by the simulation's
// argmin; and the encoding of |value| for the packed format.
__constant__ float kFp4Grid[15] = {-6.f, -4.f, -3.f, -2.f, -1.5f, -1.f, -0.5f, 0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};

// Nearest e2m1 value, ties to the even code (0, 1, 2, 4 have even codes).
__device__ __forceinline__ uint32_t e2m1_code(float x) {
  const float a = __builtin_fabsf(x);
  uint32_t c;
  if (a <= 0.25f) c = 0;            // 0.25: tie between 0 (code 0) and 0.5 (code 1) -> 0
  else if (a < 0.75f) c = 1;        // 0.5
  else if (a <= 1.25f) c = 2;       // 1.0 (0.75 -> 1.0, 1.25 -> 1.0)
  else if (a < 1.75f) c = 3;        // 1.5
  else if (a <= 2.5f) c = 4;        // 2.0 (1.75 -> 2.0, 2.5 -> 2.0)
  else if (a < 3.5f) c = 5;         // 3.0
  else if (a <= 5.f) c = 6;         // 4.0 (3.5 -> 4.0, 5 -> 4.0)
  else c = 7;                       // 6.0
  return (c != 0 && __builtin_signbitf(x)) ? (c | 8u) : c;
}

// ---- simulate kernels (bit-identical to the reference formulas) --------------
struct QuantArgs {
  const void* x;
  void* y;          // simulate: dequantised values (same dtype); pack: values
  float* scale;     // pack: one scale per block
  int64_t nblocks;
  int bs;           // block size (multiple of 8, bs / 8 a power of two <= 64)
  int mode;         // pack: 0 = fp32 scale (amax / max), 1 = power-of-two (UE8M0) scale
};

template <int DT>
__device__ __forceinline__ float block_amax(const QuantArgs& q, int64_t blk, int sub, int g, float (&v)[8]) {
  const int64_t base = blk * q.bs + sub * 8;
  float m = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v[e] = Elt<DT>::load(q.x, base + e);
    m = __builtin_fmaxf(m, __builtin_fabsf(v[e]));
  }
  for (int w = 1; w < g; w <<= 1) m = __builtin_fmaxf(m, __shfl_xor(m, w, 64));
  return m;
}

// act_quant_simulate: amax -> clamp_min(1e-4) -> scale = amax / 448 ->
// clamp(x / scale, +-448) -> e4m3 -> float * scale -> dtype (each op rounded to
// the dtype as torch does).
template <int DT>
__global__ __launch_bounds__(256) void fp8_simulate_kernel(QuantArgs q) {
  const int g = q.bs / 8;  // lanes per block
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t blk = t / g;
  const int sub = static_cast<int>(t % g);
  if (blk >= q.nblocks) return;  // whole lane groups leave together (g divides 64)
  float v[8];
  float amax = block_amax<DT>(q, blk, sub, g, v);
  amax = Elt<DT>::round(__builtin_fmaxf(amax, 1e-4f));
  const float scale = Elt<DT>::round(amax / 448.f);
  const int64_t base = blk * q.bs + sub * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float y = Elt<DT>::round(v[e] / scale);
    y = __builtin_fminf(__builtin_fmaxf(y, -448.f), 448.f);
    Elt<DT>::store(q.y, base + e, e4m3_round(y) * scale);
  }
}

// fp4_act_quant_simulate: amax -> clamp_min(6 * 2^-126) -> scale = amax / 6 ->
// clamp(x / scale, +-6) -> argmin |scaled - grid| (first minimum, diffs in the
// dtype) -> grid value * scale.
template <int DT>
__global__ __launch_bounds__(256) void fp4_simulate_kernel(QuantArgs q) {
  const int g = q.bs / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t blk = t / g;
  const int sub = static_cast<int>(t % g);
  if (blk >= q.nblocks) return;
  float v[8];
  float amax = block_amax<DT>(q, blk, sub, g, v);
  amax = Elt<DT>::round(__builtin_fmaxf(amax, 6.f * 0x1p-126f));
  const float scale = Elt<DT>::round(amax / 6.f);
  const int64_t base = blk * q.bs + sub * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float y = Elt<DT>::round(v[e] / scale);
    y = __builtin_fminf(__builtin_fmaxf(y, -6.f), 6.f);
    float best = __builtin_fabsf(Elt<DT>::round(y - kFp4Grid[0]));
    int bi = 0;
#pragma unroll
    for (int i = 1; i < 15; ++i) {
      const float d = __builtin_fabsf(Elt<DT>::round(y - kFp4Grid[i]));
      if (d < best) {
        best = d;
        bi = i;
      }
    }
    Elt<DT>::store(q.y, base + e, kFp4Grid[bi] * scale);
  }
}

// ---- packing kernels (production formats) ------------------------------------
__device__ __forceinline__ float pow2_ceil(float x) {  // smallest 2^k >= x (x > 0, normal)
  int e;
  const float f = __builtin_frexpf(x, &e);  // x = f 2^e, f in [0.5, 1)
  return f == 0.5f ? x : __builtin_ldexpf(1.0f, e);
}

// fp8 e4m3 + one fp32 scale per block: scale = max(amax, 1e-4) / 448 (mode 0)
// or its power-of-two ceiling (mode 1); value = e4m3(clamp(x / scale, +-448)).
template <int DT>
__global__ __launch_bounds__(256) void fp8_pack_kernel(QuantArgs q) {
  const int g = q.bs / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t blk = t / g;
  const int sub = static_cast<int>(t % g);
  if (blk >= q.nblocks) return;
  float v[8];
  const float amax = __builtin_fmaxf(block_amax<DT>(q, blk, sub, g, v), 1e-4f);
  float scale = amax / 448.f;
  if (q.mode == 1) scale = pow2_ceil(scale);
  if (sub == 0) q.scale[blk] = scale;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float y = v[e] / scale;
    y = __builtin_fminf(__builtin_fmaxf(y, -448.f), 448.f);
    w[e >> 2] |= static_cast<uint32_t>(e4m3_bits(e4m3_round(y))) << (8 * (e & 3));
  }
  *reinterpret_cast<uint2*>(static_cast<uint8_t*>(q.y) + blk * q.bs + sub * 8) = uint2{w[0], w[1]};
}

// fp4 e2m1 packed two per byte (element 2i low nibble) + power-of-two scale
// per block: scale = 2^ceil(log2(max(amax, 6 * 2^-126) / 6)), so |x / scale| <= 6.
template <int DT>
__global__ __launch_bounds__(256) void fp4_pack_kernel(QuantArgs q) {
  const int g = q.bs / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t blk = t / g;
  const int sub = static_cast<int>(t % g);
  if (blk >= q.nblocks) return;
  float v[8];
  const float amax = __builtin_fmaxf(block_amax<DT>(q, blk, sub, g, v), 6.f * 0x1p-126f);
  const float scale = pow2_ceil(amax / 6.f);
  if (sub == 0) q.scale[blk] = scale;
  uint32_t w = 0u;
#pragma unroll
  for (int e = 0; e < 8; ++e) w |= e2m1_code(v[e] / scale) << (4 * e);
  *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(q.y) + (blk * q.bs + sub * 8) / 2) = w;
}

// ---- token compressor / softmax-gated pool ----------------------------------
struct PoolArgs {
  const void* ca;  // [B, S, C] content, stream a
  const void* za;  // [B, S, C] scores, stream a
  const void* cb;  // stream b (overlap) or null
  const void* zb;
  const float* ba;  // [m, C] bias of stream a (fp32)
  const float* bb;  // [m, C] bias of stream b or null
  void* out;        // [B, S / m, C]
  int64_t B, S, C, m, nblk;
  int overlap;
};

// One thread per (batch, compressed entry, channel).  Overlap (CSA, eq. 11-12):
// softmax over the 2m scores [z_a + b_a of block i ; z_b + b_b of block i-1]
// (block 0: the b half is -inf / 0); no overlap (HCA, eq. 22-23): softmax over
// the m scores of block i.  fp32 arithmetic, output rounded to the dtype.
template <int DT>
__global__ __launch_bounds__(256) void token_compress_kernel(PoolArgs p) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = p.B * p.nblk * p.C;
  if (t >= total) return;
  const int64_t c = t % p.C;
  const int64_t i = (t / p.C) % p.nblk;
  const int64_t b = t / (p.C * p.nblk);
  const int64_t row0 = (b * p.S + i * p.m) * p.C + c;
  float mx = -__builtin_inff();
  for (int64_t j = 0; j < p.m; ++j) mx = __builtin_fmaxf(mx, Elt<DT>::load(p.za, row0 + j * p.C) + p.ba[j * p.C + c]);
  const bool has_b = p.overlap && i > 0;
  const int64_t rowb = row0 - p.m * p.C;  // block i-1
  if (has_b)
    for (int64_t j = 0; j < p.m; ++j) mx = __builtin_fmaxf(mx, Elt<DT>::load(p.zb, rowb + j * p.C) + p.bb[j * p.C + c]);
  float den = 0.f, num = 0.f;
  for (int64_t j = 0; j < p.m; ++j) {
    const float w = __expf(Elt<DT>::load(p.za, row0 + j * p.C) + p.ba[j * p.C + c] - mx);
    den += w;
    num += w * Elt<DT>::load(p.ca, row0 + j * p.C);
  }
  if (has_b)
    for (int64_t j = 0; j < p.m; ++j) {
      const float w = __expf(Elt<DT>::load(p.zb, rowb + j * p.C) + p.bb[j * p.C + c] - mx);
      den += w;
      num += w * Elt<DT>::load(p.cb, rowb + j * p.C);
    }
  Elt<DT>::store(p.out, t, num / den);
}

// softmax_gated_pool over the middle axis of [outer, L, inner] tensors.
template <int DT>
__global__ __launch_bounds__(256) void gated_pool_kernel(const void* kv, const void* score, void* out, int64_t outer,
                                                          int64_t L, int64_t inner) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, in = t % inner;
  const int64_t base = o * L * inner + in;
  float mx = -__builtin_inff();
  for (int64_t l = 0; l < L; ++l) mx = __builtin_fmaxf(mx, Elt<DT>::load(score, base + l * inner));
  float den = 0.f, num = 0.f;
  for (int64_t l = 0; l < L; ++l) {
    const float w = __expf(Elt<DT>::load(score, base + l * inner) - mx);
    den += w;
    num += w * Elt<DT>::load(kv, base + l * inner);
  }
  Elt<DT>::store(out, t, num / den);
}

template <template <int> class K, typename A>
static int launch_dt(int dt, int64_t threads, const A& args, const char* name, hipStream_t st) {
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "tensor too large");
  if (blocks == 0) return SI_OK;
  switch (dt) {
    case 0: hipLaunchKernelGGL(K<0>::fn, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, args); break;
    case 1: hipLaunchKernelGGL(K<1>::fn, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, args); break;
    case 2: hipLaunchKernelGGL(K<2>::fn, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, args); break;
    default: return set_error(SI_ERR_UNSUPPORTED, "dtype must be fp32, bf16 or fp16");
  }
  return check_launch(name);
}
template <int DT> struct Fp8Sim { static constexpr auto fn = fp8_simulate_kernel<DT>; };
template <int DT> struct Fp4Sim { static constexpr auto fn = fp4_simulate_kernel<DT>; };
template <int DT> struct Fp8Pack { static constexpr auto fn = fp8_pack_kernel<DT>; };
template <int DT> struct Fp4Pack { static constexpr auto fn = fp4_pack_kernel<DT>; };
template <int DT> struct Compress { static constexpr auto fn = token_compress_kernel<DT>; };

static int check_block(int64_t n, int64_t bs) {
  if (bs < 8 || bs > 512 || bs % 8 || ((bs / 8) & (bs / 8 - 1)))
    return set_error(SI_ERR_UNSUPPORTED, "block_size must be 8 * 2^j <= 512, got " + std::to_string(bs));
  if (n < 0 || n % bs) return set_error(SI_ERR_INVALID, "element count must be a multiple of block_size");
  return SI_OK;
}

}  // namespace si

using namespace si;

extern "C" int si_quant_simulate(const void* x, void* y, int dtype, int64_t n, int64_t block_size, int fp4,
                                 void* stream) {
  int rc = check_block(n, block_size);
  if (rc) return rc;
  if (n > 0 && (!x || !y)) return set_error(SI_ERR_INVALID, "null pointer argument");
  QuantArgs q{x, y, nullptr, n / block_size, static_cast<int>(block_size), 0};
  const int64_t threads = n / 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return fp4 ? launch_dt<Fp4Sim>(dtype, threads, q, "fp4_simulate_kernel", st)
             : launch_dt<Fp8Sim>(dtype, threads, q, "fp8_simulate_kernel", st);
}

extern "C" int si_quant_pack(const void* x, void* y, float* scale, int dtype, int64_t n, int64_t block_size, int fp4,
                             int pow2_scale, void* stream) {
  int rc = check_block(n, block_size);
  if (rc) return rc;
  if (n > 0 && (!x || !y || !scale)) return set_error(SI_ERR_INVALID, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(y) & 7) || (fp4 && (reinterpret_cast<uintptr_t>(y) & 3)))
    return set_error(SI_ERR_INVALID, "output must be 8-byte aligned");
  QuantArgs q{x, y, scale, n / block_size, static_cast<int>(block_size), pow2_scale ? 1 : 0};
  const int64_t threads = n / 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return fp4 ? launch_dt<Fp4Pack>(dtype, threads, q, "fp4_pack_kernel", st)
             : launch_dt<Fp8Pack>(dtype, threads, q, "fp8_pack_kernel", st);
}

extern "C" int si_token_compress(const void* c_a, const void* z_a, const float* b_a, const void* c_b, const void* z_b,
                                 const float* b_b, int dtype, int64_t B, int64_t S, int64_t C, int64_t m, int overlap,
                                 void* out, void* stream) {
  if (B < 0 || S < 0 || C <= 0 || m <= 0) return set_error(SI_ERR_INVALID, "bad dimension");
  const int64_t nblk = S / m;
  if (B * nblk > 0 && (!c_a || !z_a || !b_a || !out || (overlap && (!c_b || !z_b || !b_b))))
    return set_error(SI_ERR_INVALID, "null pointer argument");
  PoolArgs p{c_a, z_a, c_b, z_b, b_a, b_b, out, B, S, C, m, nblk, overlap ? 1 : 0};
  return launch_dt<Compress>(dtype, B * nblk * C, p, "token_compress_kernel", static_cast<hipStream_t>(stream));
}

extern "C" int si_gated_pool(const void* kv, const void* score, void* out, int dtype, int64_t outer, int64_t L,
                             int64_t inner, void* stream) {
  if (outer < 0 || L <= 0 || inner < 0) return set_error(SI_ERR_INVALID, "bad dimension");
  if (outer * inner > 0 && (!kv || !score || !out)) return set_error(SI_ERR_INVALID, "null pointer argument");
  const int64_t threads = outer * inner;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks == 0) return SI_OK;
  if (blocks > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "tensor too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(blocks));
  switch (dtype) {
    case 0: hipLaunchKernelGGL(gated_pool_kernel<0>, grid, dim3(256), 0, st, kv, score, out, outer, L, inner); break;
    case 1: hipLaunchKernelGGL(gated_pool_kernel<1>, grid, dim3(256), 0, st, kv, score, out, outer, L, inner); break;
    case 2: hipLaunchKernelGGL(gated_pool_kernel<2>, grid, dim3(256), 0, st, kv, score, out, outer, L, inner); break;
    default: return set_error(SI_ERR_UNSUPPORTED, "dtype must be fp32, bf16 or fp16");
  }
  return check_launch("gated_pool_kernel");
}
