// Wave-level exact top-k selection over 64-bit (score, index) keys.
//
// One wave owns the selection state of one query row.  The state is
//   * `top`  : the best `top_k` keys seen so far, sorted descending, in LDS;
//   * `cand` : an append buffer of keys that beat the current threshold;
//   * `tau`  : the high word (ordered score) of the top_k-th best key in
//              `top`, or 0 while `top` holds fewer than top_k keys.
// Keys arrive in increasing index order, so a new key whose ordered score
// equals `tau` always loses the tie (its index is larger than every index
// already held) and the filter is a strict `ord(score) > tau`.  Because
// `tau` only rises when buffered candidates are merged, it is a lower bound
// of the true running threshold: the filter never drops a key that belongs
// to the final top-k, so the result is exact (the partition-merge argument:
// top-k of a multiset equals top-k of the union of per-part top-ks).
//
// KCAP keys are held per wave, E = KCAP / 64 per lane.  A lane's register
// element j is global rank e = lane * E + j.  In LDS, rank e lives at
// slot (e % E) * 64 + e / E so that lane-parallel accesses are conflict-free.
#pragma once

#include "si_common.h"

namespace si {

template <int E>
__device__ __forceinline__ int sel_slot(int e) {
  return (e % E) * kWave + e / E;
}

// One bitonic compare-exchange stage; rank e = lane*E+j.  SIZE and STRIDE are
// compile-time so that every register index below is static.
template <int E, int N, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_stage(uint64_t (&v)[E], int lane) {
  if constexpr (STRIDE >= E) {
    constexpr int LX = STRIDE / E;
    const bool lower = (lane & LX) == 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int e = lane * E + j;
      const bool desc = (SIZE >= N) || ((e & SIZE) == 0);
      const uint64_t o = shfl_xor_u64(v[j], lane, LX);
      const bool keep_max = (lower == desc);
      const bool take = keep_max ? (o > v[j]) : (o < v[j]);
      v[j] = take ? o : v[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if ((j ^ STRIDE) > j) {
        const int p = j ^ STRIDE;
        const int e = lane * E + j;
        const bool desc = (SIZE >= N) || ((e & SIZE) == 0);
        const uint64_t a = v[j], b = v[p];
        const bool sw = desc ? (a < b) : (a > b);
        v[j] = sw ? b : a;
        v[p] = sw ? a : b;
      }
    }
  }
}

// Strides STRIDE, STRIDE/2, ..., 1 of one bitonic level.
template <int E, int N, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_level(uint64_t (&v)[E], int lane) {
  if constexpr (STRIDE > 0) {
    bitonic_stage<E, N, SIZE, STRIDE>(v, lane);
    bitonic_level<E, N, SIZE, STRIDE / 2>(v, lane);
  }
}

template <int E, int N, int SIZE>
__device__ __forceinline__ void bitonic_levels(uint64_t (&v)[E], int lane) {
  if constexpr (SIZE <= N) {
    bitonic_level<E, N, SIZE, SIZE / 2>(v, lane);
    bitonic_levels<E, N, SIZE * 2>(v, lane);
  }
}

// Full bitonic sort of 64*E keys, descending.
template <int E>
__device__ __forceinline__ void wave_sort_desc(uint64_t (&v)[E], int lane) {
  bitonic_levels<E, kWave * E, 2>(v, lane);
}

// Sorts a bitonic sequence of 64*E keys descending (final merge level only).
template <int E>
__device__ __forceinline__ void wave_merge_desc(uint64_t (&v)[E], int lane) {
  constexpr int N = kWave * E;
  bitonic_level<E, N, N, N / 2>(v, lane);
}

template <int KCAP>
struct WaveSelect {
  static constexpr int E = KCAP / kWave;
  static_assert(E >= 1 && (E & (E - 1)) == 0, "KCAP must be 64 * 2^n");

  uint64_t* top;   // KCAP keys in LDS (this wave's private region)
  uint64_t* cand;  // KCAP keys in LDS (this wave's private region)
  int n;           // buffered candidates, wave-uniform
  uint32_t tau;    // threshold ordered score, wave-uniform
  int top_k;

  __device__ __forceinline__ void init(uint64_t* top_lds, uint64_t* cand_lds, int k, int lane) {
    top = top_lds;
    cand = cand_lds;
    n = 0;
    tau = 0;
    top_k = k;
#pragma unroll
    for (int j = 0; j < E; ++j) top[j * kWave + lane] = 0ull;
  }

  // Offers one key per lane (only lanes with `pass`), appending in lane order.
  // Returns after merging if the buffer can no longer take a full wave.
  __device__ __forceinline__ void offer(bool pass, uint64_t key, int lane) {
    const uint64_t bal = ballot64(pass);
    if (bal == 0) return;
    if (pass) cand[sel_slot<E>(n + lanes_below(bal))] = key;
    n += __builtin_popcountll(bal);
    if (n > KCAP - kWave) flush(lane);
  }

  // Merges the buffered candidates into `top`; leaves the sorted result in `v`.
  __device__ __forceinline__ void merge(uint64_t (&v)[E], int lane) {
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int e = lane * E + j;
      v[j] = (e < n) ? cand[j * kWave + lane] : 0ull;
    }
    wave_sort_desc<E>(v, lane);
    // Reverse-pair with the held top list: max(cand[e], top[N-1-e]) is bitonic.
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const uint64_t t = top[(E - 1 - j) * kWave + (kWave - 1 - lane)];
      v[j] = t > v[j] ? t : v[j];
    }
    wave_merge_desc<E>(v, lane);
    uint64_t kth = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int e = lane * E + j;
      if (e >= top_k) v[j] = 0ull;
      if (e == top_k - 1) kth = v[j];
    }
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < E; ++j) top[j * kWave + lane] = v[j];
    const int holder = (top_k - 1) / E;
    tau = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key_hi(kth)), holder));
    n = 0;
  }

  __device__ __forceinline__ void flush(int lane) {
    uint64_t v[E];
    merge(v, lane);
  }

  // Final merge and write-out of one row: indices (int64, -1 pad) and scores
  // (fp32, -inf pad), best first.
  __device__ __forceinline__ void finish(int64_t* out_idx, float* out_score, int lane) {
    uint64_t v[E];
    if (n > 0) {
      merge(v, lane);
    } else {
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < E; ++j) v[j] = top[j * kWave + lane];
    }
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int e = lane * E + j;
      if (e < top_k) {
        const uint64_t k = v[j];
        out_idx[e] = k ? static_cast<int64_t>(key_idx(k)) : int64_t(-1);
        out_score[e] = k ? ord_to_f32(key_hi(k)) : -__builtin_inff();
      }
    }
  }
};

}  // namespace si
