// Wave-level exact top-k selection over 64-bit (score, index) keys.
//
// One wave owns the selection state of one query row:
//   * `buf`   : an unsorted LDS buffer of capacity C holding every key seen so
//               far that is >= the floor key P (and nothing below it);
//   * `floor` : P, raised only when the buffer fills; count(buf) >= top_k
//               always holds once P > 0, so no key below P can be in the top-k;
//   * `tau`   : the high word (ordered score) of P.
// A new key arrives with an index larger than every index already seen, so
// if its ordered score equals tau it ranks below every buffered key >= P and
// the arrival filter is the strict test `ord(score) > tau` (exact).
//
// When the buffer cannot take another 32 keys it is compacted: a new floor P'
// is chosen so that top_k <= count(keys >= P') <= C - 64, using 64 evenly
// spaced samples (bitonic-sorted across the wave) and, if needed, bisection
// over the 64-bit key space.  Keys are distinct, so the count drops by at most
// one per key value and bisection always lands in the window.  Counting is a
// ballot per 64-key row, so a compaction costs ~C/64 compares, not a sort.
// The exact sorted top-k is produced once, at the end of the row.
#pragma once

#include "si_common.h"

namespace si {

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

// Full bitonic sort of 64*E keys across the wave, descending; rank e = lane*E+j.
template <int E>
__device__ __forceinline__ void wave_sort_desc(uint64_t (&v)[E], int lane) {
  bitonic_levels<E, kWave * E, 2>(v, lane);
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), l));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), l));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <int C>
struct WaveSelect {
  static constexpr int E = C / kWave;   // 64-key rows in the buffer
  static constexpr int CMAX = C - 64;   // most keys kept by a compaction
  static_assert(E >= 4 && (E & (E - 1)) == 0, "capacity must be 64 * 2^n, n >= 2");

  uint64_t* buf;        // this wave's private LDS buffer, key at position p = buf[p]
  int n;                // keys held (wave-uniform)
  uint32_t tau;         // ordered score of the floor key
  uint64_t floor_key;   // P
  int top_k;

  __device__ __forceinline__ void init(uint64_t* lds, int k) {
    buf = lds;
    n = 0;
    tau = 0;
    floor_key = 0;
    top_k = k;
  }

  // Offers this lane's key if `pass`; appends in lane order.
  __device__ __forceinline__ void offer(bool pass, uint64_t key, int lane) {
    const uint64_t bal = ballot64(pass);
    if (bal == 0) return;
    if (pass) buf[n + lanes_below(bal)] = key;
    n += __builtin_popcountll(bal);
    if (n > C - 32) compact(lane);
  }

  // Number of buffered keys >= p (one ballot per 64-key row).
  __device__ __forceinline__ int count_ge(uint64_t p, int lane) const {
    int c = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int pos = j * kWave + lane;
      if (j * kWave < n) {
        const uint64_t key = pos < n ? buf[pos] : 0ull;
        c += __builtin_popcountll(ballot64(pos < n && key >= p));
      }
    }
    return c;
  }

  __device__ __forceinline__ void compact(int lane) {
    wave_lds_sync();
    // 64 keys at evenly spaced buffer positions, sorted descending across lanes.
    uint64_t smp[1];
    smp[0] = buf[(lane * n) >> 6];
    wave_sort_desc<1>(smp, lane);
    const int kk = top_k;
    const int target = kk + (CMAX - kk) / 3;
    int il = -1, ih = 64;  // count(sample[il]) < kk, count(sample[ih]) > CMAX
    int i = (target * 64) / n;
    i = i < 0 ? 0 : (i > 63 ? 63 : i);
    uint64_t p = 0;
    int c = 0;
    bool found = false;
    for (int it = 0; it < 7 && !found; ++it) {
      p = readlane_u64(smp[0], i);
      c = count_ge(p, lane);
      if (c >= kk && c <= CMAX) {
        found = true;
      } else {
        if (c < kk) il = i; else ih = i;
        if (ih - il <= 1) break;
        i = (il + ih) >> 1;
      }
    }
    if (!found) {
      // Bisection over the key space between a floor with too many keys and a
      // ceiling with too few; terminates because keys are distinct.
      uint64_t lo = ih < 64 ? readlane_u64(smp[0], ih) : floor_key;
      uint64_t hi = il >= 0 ? readlane_u64(smp[0], il) : ~0ull;
      for (int it = 0; it < 66; ++it) {
        p = lo + ((hi - lo) >> 1);
        c = count_ge(p, lane);
        if (c >= kk && c <= CMAX) break;
        if (c < kk) hi = p; else lo = p;
      }
    }
    // In-place compaction: the write position never passes the read position.
    int base = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if (j * kWave < n) {
        const int pos = j * kWave + lane;
        const uint64_t key = pos < n ? buf[pos] : 0ull;
        const bool keep = pos < n && key >= p;
        const uint64_t bal = ballot64(keep);
        wave_lds_sync();
        if (keep) buf[base + lanes_below(bal)] = key;
        base += __builtin_popcountll(bal);
      }
    }
    n = base;
    floor_key = p;
    tau = key_hi(p);
    wave_lds_sync();
  }

  // Sorted top_k of the row: indices (int64, -1 pad) and scores (fp32, -inf pad).
  __device__ __forceinline__ void finish(int64_t* out_idx, float* out_score, int lane) {
    wave_lds_sync();
    if constexpr (E <= 32) {
      uint64_t v[E];
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const int pos = j * kWave + lane;
        v[j] = pos < n ? buf[pos] : 0ull;
      }
      wave_sort_desc<E>(v, lane);
      write_out<E>(v, out_idx, out_score, lane);
    } else {
      // Wider buffers are sorted as two halves of 32 keys per lane: the first
      // half is parked in LDS in rank order, then one half-cleaner + bitonic
      // merge yields the top C/2 >= top_k.  (A single 64-key-per-lane
      // register sort is avoided: it does not fit this kernel's registers.)
      constexpr int HE = E / 2;
      constexpr int HALF = C / 2;
      uint64_t v[HE];
#pragma unroll
      for (int j = 0; j < HE; ++j) {
        const int pos = j * kWave + lane;
        v[j] = pos < n ? buf[pos] : 0ull;
      }
      wave_sort_desc<HE>(v, lane);
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < HE; ++j) buf[lane * HE + j] = v[j];
#pragma unroll
      for (int j = 0; j < HE; ++j) {
        const int pos = HALF + j * kWave + lane;
        v[j] = pos < n ? buf[pos] : 0ull;
      }
      wave_sort_desc<HE>(v, lane);
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < HE; ++j) {
        const uint64_t a = buf[HALF - 1 - (lane * HE + j)];
        v[j] = a > v[j] ? a : v[j];
      }
      bitonic_level<HE, kWave * HE, kWave * HE, kWave * HE / 2>(v, lane);
      write_out<HE>(v, out_idx, out_score, lane);
    }
  }

  template <int EE>
  __device__ __forceinline__ void write_out(const uint64_t (&v)[EE], int64_t* out_idx, float* out_score,
                                            int lane) const {
#pragma unroll
    for (int j = 0; j < EE; ++j) {
      const int e = lane * EE + j;
      if (e < top_k) {
        const uint64_t k = v[j];
        out_idx[e] = k ? static_cast<int64_t>(key_idx(k)) : int64_t(-1);
        out_score[e] = k ? ord_to_f32(key_hi(k)) : -__builtin_inff();
      }
    }
  }
};

}  // namespace si
