// Building blocks shared by the sparse-attention forward and backward
// kernels for gfx950: the KV tile shape and its LDS swizzle, inline-asm LDS
// reads with exact waits, and the fence-free tile barrier.
#pragma once
#include <type_traits>

#include "si_common.h"

namespace si {

constexpr int kAttnTK = 32;      // keys per tile
constexpr int kAttnWaves = 4;    // waves per workgroup; 16 heads each in S^T
constexpr int kAttnRing = 4;     // KV tiles resident in LDS
template <int D>
struct AttnShape {
  static constexpr int CPR = D / 8;                  // 16-byte chunks per KV row
  static constexpr int ROW = D * 2;                  // bytes per KV row
  static constexpr int TILE = kAttnTK * ROW;         // bytes per KV tile
  static constexpr int CH = kAttnTK * CPR;           // chunks per tile
  static constexpr int NT = kAttnWaves * 64;
  static constexpr int LPT = (CH + NT - 1) / NT;     // tile copies per thread
  static constexpr int KS = D / 32;                  // S^T k-steps
  static constexpr int MBT = D / 16;                 // 16-dim output blocks
  static constexpr int MBW = (MBT + kAttnWaves - 1) / kAttnWaves;  // per wave
  static constexpr int OROW = ROW + 16;              // staged output row (padded)
  static constexpr int OUT = 64 * OROW;              // staged output bytes
  static constexpr int LDS_KV = (kAttnRing * TILE > OUT) ? kAttnRing * TILE : OUT;
  static constexpr int FMASK = CPR >= 8 ? 7 : 0;     // chunk swizzle width
};

// Chunk swizzle of key row k: chunk c is stored at c ^ (k & 7).  Measured on
// gfx950 (SQ_LDS_BANK_CONFLICT), this makes both read patterns below
// conflict-free: the S^T A-fragment ds_read_b128 (16 keys at one chunk per
// quarter-wave) and the V^T ds_read_b64_tr_b16 (4 keys x 32 bytes per
// 16-lane group).  The row stride alone (1152 bytes) gives 4-way conflicts.
template <int D>
__device__ __forceinline__ int kv_swz(int k) {
  return k & AttnShape<D>::FMASK;
}
template <int D>
__device__ __forceinline__ int kv_off(int k, int c) {
  return k * (D * 2) + ((c ^ kv_swz<D>(k)) << 4);
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const char lds_cchar;

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cchar*)p));
}

// ds_read_b64_tr_b16 issued from inline asm at LDS byte address addr + OFF.
// Through the builtin, the compiler makes every such read wait for all
// outstanding LDS-DMA copies (vmcnt(0)), which would serialise the gather of
// later tiles with this tile's P.V; issued this way the read is ordered only
// by lds_wait below.
template <int OFF>
__device__ __forceinline__ v4i16 tr_read(uint32_t addr) {
  v4i16 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}

// ds_read_b128 at LDS byte address addr + OFF, issued in program order (the
// compiler would otherwise move each read next to its use and serialise the
// S^T MFMAs behind the LDS latency).
template <int OFF>
__device__ __forceinline__ bf16x8 ld128(uint32_t addr) {
  bf16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
  return r;
}

// Waits until at most N of this wave's LDS operations are outstanding.  The
// two registers are tied to the wait so that their uses stay after it.  LDS
// operations complete in order, so the compiler's own lgkmcnt waits stay
// correct (they only become stricter) with these reads in flight.
template <int N>
__device__ __forceinline__ void lds_wait(v4i16& x, v4i16& y) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}
template <int N>
__device__ __forceinline__ void lds_wait(bf16x8& x, bf16x8& y) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// A VALU instruction may read the result of a v_mfma only after the MFMA's
// wait states (11 for an 8-pass XDL op).  The compiler does not count them
// when the first read lands in a successor block (here: after the rescale
// branch), so accumulators that VALU reads go through this fence: 20 wait
// states, tied to the registers so that every read stays behind it.
__device__ __forceinline__ void mfma_result_fence(f32x4& x, f32x4& y) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(x), "+v"(y));
}

// Two floats to packed bf16, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// ---------------------------------------------------------------------------
// The 16-bit element type of q / kv / o (and of the backward's dO, dq, dkv and
// its bf16 coefficient tiles): F16 = false is bf16, true is fp16.  Operands
// travel as raw 16-bit lanes (bf16x8 / uint32 pairs) and are reinterpreted at
// the MFMA and at the conversions.
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// D += A * B over 16x16x32 tiles in the element type (fp32 accumulate).
template <bool F16>
__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  if constexpr (F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
}

// Two floats to two packed elements, round-to-nearest-even.
template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (F16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  } else {
    return f32x2_to_bf16x2(a, b);
  }
}

// The low / high element of a packed pair, widened to fp32 (exact).
template <bool F16>
__device__ __forceinline__ float elem_lo(uint32_t w) {
  if constexpr (F16) {
    return static_cast<float>(__builtin_bit_cast(f16x2, w)[0]);
  } else {
    return __uint_as_float(w << 16);
  }
}
template <bool F16>
__device__ __forceinline__ float elem_hi(uint32_t w) {
  if constexpr (F16) {
    return static_cast<float>(__builtin_bit_cast(f16x2, w)[1]);
  } else {
    return __uint_as_float(w & 0xffff0000u);
  }
}

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1.
template <int I, int N, typename F>
__device__ __forceinline__ void attn_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    attn_static_for<I + 1, N>(f);
  }
}

// s_waitcnt immediate: vmcnt <= n (6-bit field: bits 3:0 and 15:14),
// lgkmcnt = 0, expcnt not waited (gfx9 encoding).
constexpr int vm_lgkm0(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | (0x7 << 4); }

// Waits until at most N LDS operations of this wave are outstanding (no
// registers tied; follow with reg_tie on the registers the wait covers).
template <int N>
__device__ __forceinline__ void lds_wait_n() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
}
// Keeps every use of x after the preceding inline-asm wait.
template <typename T>
__device__ __forceinline__ void reg_tie(T& x) {
  asm volatile("" : "+v"(x));
}

// Block order of the forward's row groups.  Workgroups go to the 8 XCDs
// round-robin, so consecutive blocks run on different L2s.  Within every full
// chunk of 256 blocks this returns, for XCD x, 32 consecutive block numbers
// instead, so
// that queries sharing KV rows (HCA / CSA windows and compressed rows) gather
// them through one L2, while every XCD still gets a share of each chunk (the
// order of the chunks themselves is unchanged).  A bijection on
// [0, gridDim.x); the partial last chunk keeps the plain order.  (The
// backward's row kernel measured the same with it: its time is its row and
// reduction traffic, not gather locality.)
__device__ __forceinline__ int xcd_block_order() {
  constexpr int kXcds = 8, kPerXcd = 32;
  int lb = static_cast<int>(blockIdx.x);
  const int chunk = lb / (kXcds * kPerXcd);
  if ((chunk + 1) * (kXcds * kPerXcd) <= static_cast<int>(gridDim.x))
    lb = chunk * (kXcds * kPerXcd) + (lb % kXcds) * kPerXcd + (lb / kXcds) % kPerXcd;
  return lb;
}

// Tile barrier of the main loops.  __syncthreads() carries a workgroup
// release fence, for which the compiler waits on every outstanding LDS-DMA
// copy (vmcnt(0)) -- including the gathers just issued for later tiles, which
// would leave no gather latency hidden.  Here each wave first waits for
// exactly what the other waves read after the barrier (its LDS stores:
// lgkmcnt(0); the copies of the next tile: an explicit vmcnt), and the empty
// asm statements keep the compiler from moving memory accesses across the
// barrier.
__device__ __forceinline__ void attn_tile_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace si
