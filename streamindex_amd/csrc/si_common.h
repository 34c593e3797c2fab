// Shared device helpers for the StreamIndex gfx950 kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts,
// v_mfma_f32_{32x32x16,16x16x32}_bf16 matrix cores and 160 KiB of LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Order-preserving float <-> uint32 map.  ord(a) > ord(b) as unsigned integers
// iff a > b as floats (for all non-NaN values; -0.0 is folded onto +0.0 first
// so that the two zeros tie, as they do under IEEE comparison).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_to_ord(float x) {
  x = x + 0.0f;  // -0.0 + 0.0 == +0.0 under round-to-nearest
  const uint32_t b = __float_as_uint(x);
  // negative: ~b; otherwise b with the sign bit set
  const uint32_t neg = static_cast<uint32_t>(static_cast<int32_t>(b) >> 31);
  return b ^ (neg | 0x80000000u);
}

__device__ __forceinline__ float ord_to_f32(uint32_t o) {
  const uint32_t b = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(b);
}

// A selection key packs (score, index) so that a larger unsigned 64-bit key
// means "ranks higher" under the total order used by the indexer top-k:
// higher score first, and on equal score the smaller index first.  The key 0
// is the empty-slot sentinel; every real key is larger because ord() of a
// finite float is at least 0x00800000.
__device__ __forceinline__ uint64_t make_key(float score, uint32_t idx) {
  return (static_cast<uint64_t>(f32_to_ord(score)) << 32) | static_cast<uint64_t>(~idx);
}
// make_key with the index already complemented (inv_idx = ~idx).
__device__ __forceinline__ uint64_t make_key_inv(float score, uint32_t inv_idx) {
  return (static_cast<uint64_t>(f32_to_ord(score)) << 32) | static_cast<uint64_t>(inv_idx);
}
__device__ __forceinline__ uint32_t key_hi(uint64_t k) { return static_cast<uint32_t>(k >> 32); }
__device__ __forceinline__ uint32_t key_idx(uint64_t k) { return ~static_cast<uint32_t>(k); }

// ---------------------------------------------------------------------------
// Cross-lane helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

// Value of lane (this lane ^ LX) for LX in {1, 2, 4, 8, 16, 32}, without LDS:
// DPP quad permutes for 1 and 2, two bank-masked row shifts for 4, a row
// rotation by 8 for 8, and v_permlane{16,32}_swap (plus a select by the lane's
// half) for 16 and 32.  A swap(x, x) returns {vdst', src'}: lanes of the upper
// row / half find their partner in vdst', the others in src'.
template <int LX>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t x) {
  const int xi = static_cast<int>(x);
  // (mov_dpp leaves the lanes it does not write undefined, so the compiler
  // needs no copy of the old value; every lane is written here.)
  if constexpr (LX == 1) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(xi, 0xB1, 0xf, 0xf, false));  // quad_perm 1,0,3,2
  } else if constexpr (LX == 2) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(xi, 0x4E, 0xf, 0xf, false));  // quad_perm 2,3,0,1
  } else if constexpr (LX == 4) {
    const int t = __builtin_amdgcn_mov_dpp(xi, 0x114, 0xf, 0xA, false);  // row_shr:4 into banks 1,3
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(t, xi, 0x104, 0xf, 0x5, false));  // row_shl:4 into 0,2
  } else if constexpr (LX == 8) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(xi, 0x128, 0xf, 0xf, false));  // row_ror:8
  } else if constexpr (LX == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return __builtin_amdgcn_inverse_ballot_w64(0xFFFF0000FFFF0000ull) ? static_cast<uint32_t>(r[0])
                                                                       : static_cast<uint32_t>(r[1]);
  } else {
    static_assert(LX == 32, "lane xor distance");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return __builtin_amdgcn_inverse_ballot_w64(0xFFFFFFFF00000000ull) ? static_cast<uint32_t>(r[0])
                                                                       : static_cast<uint32_t>(r[1]);
  }
}

template <int LX>
__device__ __forceinline__ uint64_t lane_xor_u64(uint64_t v) {
  const uint32_t lo = lane_xor_u32<LX>(static_cast<uint32_t>(v));
  const uint32_t hi = lane_xor_u32<LX>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Half-wave exchange (v_permlane32_swap): returns {a', b'} where a' and b'
// together hold a's and b's 32-lane halves regrouped so that, in every lane,
// a' and b' come from the same source register (a or b) and from the two
// different halves.  Which of a/b a lane ends up with is reported by
// swapping an id vector the same way.
struct SwapPair {
  uint32_t x, y;
};
__device__ __forceinline__ SwapPair permlane32_swap(uint32_t a, uint32_t b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  return SwapPair{static_cast<uint32_t>(r[0]), static_cast<uint32_t>(r[1])};
}

// Wave-wide maximum of an unsigned value, returned uniformly.  Within each
// 16-lane row: xor-1 and xor-2 (quad_perm), then the half-row and row
// mirrors; across rows: v_permlane16_swap and v_permlane32_swap.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  x = mx(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xf, 0xf, false)));
  x = mx(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xf, 0xf, false)));
  x = mx(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x141, 0xf, 0xf, false)));
  x = mx(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x140, 0xf, 0xf, false)));
  const auto r16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = mx(static_cast<uint32_t>(r16[0]), static_cast<uint32_t>(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  x = mx(static_cast<uint32_t>(r32[0]), static_cast<uint32_t>(r32[1]));
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
}

// Number of set bits of `m` in lanes strictly below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
}

// Orders this wave's LDS traffic: every LDS write issued before the call is
// visible to every lane of the same wave after it.  A wave's LDS operations
// execute in issue order, so wavefront-scope fences (compiler ordering, no
// s_waitcnt) suffice; workgroup scope would also wait for every outstanding
// global load, including LDS-DMA tile copies still in flight.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

}  // namespace si
