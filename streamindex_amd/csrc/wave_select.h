// Wave-level exact top-k selection over 64-bit (score, index) keys.
//
// One wave owns the selection state of one query row:
//   * `buf`   : an unsorted LDS buffer of capacity C holding every key seen so
//               far that is >= the floor key P (and nothing below it);
//   * `floor` : P, raised only when the buffer nears capacity; once P > 0,
//               count(buf) >= top_k always holds, so no key below P can be in
//               the top-k;
//   * `tau`   : the high word (ordered score) of P.
// Keys arrive in increasing index order, so an arriving key whose ordered
// score equals tau ranks below every buffered key with that score (ties rank
// the smaller index first) and the arrival filter is the strict test
// `ord(score) > tau` (exact).
//
// Offers append up to 64 keys at a time without branches.  When the buffer
// holds more than C - 128 keys it is compacted: the keys are pulled into
// registers (C/64 per lane), a new floor P' with
// top_k <= count(keys >= P') <= C - 192 is found by safeguarded interpolation
// over the ordered-score word (each probe is one ballot per 64 keys), with a
// bisection over the full 64-bit key when many keys share one score, and the
// survivors are written back densely.  Keys are distinct, so a count changes
// by at most one per key value and the 64-bit bisection always lands in the
// window.  The exact sorted top-k is produced once, at the end of the row.
#pragma once

#include "si_common.h"

namespace si {

// Bitonic network over 64*E keys held E per lane, rank e = lane*E + j; a
// block of SIZE ranks is sorted descending when (e & SIZE) == 0 (or when it
// is the whole sequence).  Each stage's direction pattern is a compile-time
// lane mask, so a compare-exchange is one 64-bit compare into a lane mask,
// one scalar XOR with the constant and the selects.

// Lanes whose keys of a SIZE-block run descending (SIZE >= E: depends on the lane only).
template <int E, int N, int SIZE>
constexpr uint64_t desc_lane_mask() {
  uint64_t m = 0;
  for (int l = 0; l < kWave; ++l)
    if (SIZE >= N || ((l * E) & SIZE) == 0) m |= 1ull << l;
  return m;
}

// Cross-lane stage, partner lane = lane ^ LX: lanes that keep the larger key.
template <int E, int N, int SIZE, int LX>
constexpr uint64_t keep_max_lane_mask() {
  uint64_t m = 0;
  for (int l = 0; l < kWave; ++l) {
    const bool lower = (l & LX) == 0;
    const bool desc = SIZE >= N || ((l * E) & SIZE) == 0;
    if (lower == desc) m |= 1ull << l;
  }
  return m;
}

// Half-row (LX = 16) or half-wave (LX = 32) exchange of two registers:
// v_permlane{16,32}_swap trades the upper LX-lane groups of `a` with the
// lower ones of `b`, so afterwards every lane holds one partner pair
// (lane p, lane p + LX): that of `a` in lanes whose LX bit is clear, that of
// `b` in the others, with the lower lane's value in `a`.  Applying it again
// restores both registers.
template <int LX>
__device__ __forceinline__ void lane_pair_swap(uint32_t& a, uint32_t& b) {
  if constexpr (LX == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = static_cast<uint32_t>(r[0]);
    b = static_cast<uint32_t>(r[1]);
  } else {
    static_assert(LX == 32, "lane pair distance");
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = static_cast<uint32_t>(r[0]);
    b = static_cast<uint32_t>(r[1]);
  }
}

// After lane_pair_swap<LX>, lanes holding a pair whose block runs descending:
// the pair's lower lane is l, or l - LX when l's LX bit is set.
template <int E, int N, int SIZE, int LX>
constexpr uint64_t pair_desc_lane_mask() {
  uint64_t m = 0;
  for (int l = 0; l < kWave; ++l) {
    const int p = l & ~LX;
    if (SIZE >= N || ((p * E) & SIZE) == 0) m |= 1ull << l;
  }
  return m;
}

template <int E, int N, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_stage(uint64_t (&v)[E], int lane) {
  if constexpr (STRIDE >= E && (STRIDE / E == 16 || STRIDE / E == 32) && E % 2 == 0) {
    // Registers j and j+1 are exchanged pairwise so that both keys of every
    // compare-exchange sit in one lane (lower lane's key in x), compared
    // in-lane, and exchanged back: four swaps per two keys instead of a
    // copy, a swap and a select per 32-bit half of each key.
    constexpr int LX = STRIDE / E;
    constexpr uint64_t DM = pair_desc_lane_mask<E, N, SIZE, LX>();
#pragma unroll
    for (int j = 0; j < E; j += 2) {
      uint32_t xlo = static_cast<uint32_t>(v[j]), xhi = static_cast<uint32_t>(v[j] >> 32);
      uint32_t ylo = static_cast<uint32_t>(v[j + 1]), yhi = static_cast<uint32_t>(v[j + 1] >> 32);
      lane_pair_swap<LX>(xlo, ylo);
      lane_pair_swap<LX>(xhi, yhi);
      const uint64_t x = (static_cast<uint64_t>(xhi) << 32) | xlo;
      const uint64_t y = (static_cast<uint64_t>(yhi) << 32) | ylo;
      // descending pair: the lower lane keeps the larger key (swap when x < y)
      const uint64_t lt = __builtin_amdgcn_ballot_w64(x < y);
      const bool sw = __builtin_amdgcn_inverse_ballot_w64(~(lt ^ DM));
      const uint64_t nx = sw ? y : x, ny = sw ? x : y;
      xlo = static_cast<uint32_t>(nx);
      xhi = static_cast<uint32_t>(nx >> 32);
      ylo = static_cast<uint32_t>(ny);
      yhi = static_cast<uint32_t>(ny >> 32);
      lane_pair_swap<LX>(xlo, ylo);
      lane_pair_swap<LX>(xhi, yhi);
      v[j] = (static_cast<uint64_t>(xhi) << 32) | xlo;
      v[j + 1] = (static_cast<uint64_t>(yhi) << 32) | ylo;
    }
  } else if constexpr (STRIDE >= E) {
    constexpr int LX = STRIDE / E;
    constexpr uint64_t KM = keep_max_lane_mask<E, N, SIZE, LX>();
    uint64_t o[E];
#pragma unroll
    for (int j = 0; j < E; ++j) o[j] = lane_xor_u64<LX>(v[j]);
#pragma unroll
    for (int j = 0; j < E; ++j) {
      // take the partner's key iff it is larger and this lane keeps the max, or
      // smaller and this lane keeps the min (equal keys: either choice)
      const uint64_t gt = __builtin_amdgcn_ballot_w64(o[j] > v[j]);
      const bool take = __builtin_amdgcn_inverse_ballot_w64(~(gt ^ KM));
      v[j] = take ? o[j] : v[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if ((j ^ STRIDE) > j) {
        const int p = j ^ STRIDE;
        // descending pair: swap when v[j] < v[p]; ascending: when v[j] > v[p]
        const uint64_t DM = (SIZE >= N) ? ~0ull
                            : (SIZE >= E ? desc_lane_mask<E, N, SIZE>() : (((j & SIZE) == 0) ? ~0ull : 0ull));
        const uint64_t a = v[j], b = v[p];
        const uint64_t lt = __builtin_amdgcn_ballot_w64(a < b);
        const bool sw = __builtin_amdgcn_inverse_ballot_w64(~(lt ^ DM));
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

// Where finish() writes one row's sorted top-k.  Each pointer may be null.
//   idx64 : int64 key indices, -1 past the held count;
//   score : fp32 scores, -inf past the held count;
//   idx32 : int32 key indices plus off32, -1 past the held count (the
//           compressed-KV columns of a CSA attention index row).
struct TopkRowOut {
  int64_t* idx64;
  float* score;
  int32_t* idx32;
  int32_t off32;
};

template <int C>
struct WaveSelect {
  static constexpr int E = C / kWave;   // 64-key rows in the buffer
  static constexpr int CMAX = C - 192;  // most keys a compaction keeps
  // A compaction holds E keys per lane in registers (2E VGPRs).
  static_assert(C % kWave == 0 && E >= 4 && E <= 72, "capacity must be 64 * E, 4 <= E <= 72");

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

  // Appends the keys of the lanes with `pass` set, in lane order, at
  // positions n, n+1, ...  The other lanes store to positions past the new
  // end, which are never read, so the append has no branch.  Needs n <= C-64.
  __device__ __forceinline__ void offer64(bool pass, uint64_t key, int lane) {
    const uint64_t bal = ballot64(pass);
    const int below = lanes_below(bal);
    const int tot = __builtin_popcountll(bal);
    const int pos = pass ? n + below : n + tot + (lane - below);
    buf[pos] = key;
    n = __builtin_amdgcn_readfirstlane(n + tot);
  }

  // offer64 with the passing lanes given as a lane mask (see offer64_masked
  // for why a mask): the branch-free append, for offers interleaved with MFMA
  // work.  Needs n <= C-64.
  __device__ __forceinline__ void offer64_bal(uint64_t bal, uint64_t key, int lane) {
    const int below = lanes_below(bal);
    const int tot = __builtin_popcountll(bal);
    const int pos = __builtin_amdgcn_inverse_ballot_w64(bal) ? n + below : n + tot + (lane - below);
    buf[pos] = key;
    n = __builtin_amdgcn_readfirstlane(n + tot);
  }

  // As offer64 for the lanes set in the lane mask `bal`, but only those lanes
  // store (an EXEC-masked store), so the other lanes' positions need no
  // arithmetic.  For callers whose offer is not interleaved with MFMA work
  // (the branch splits the instruction schedule).  The caller forms `bal` as
  // an AND of ballots of single compares: a ballot of a combined condition
  // makes the compiler rebuild the mask from a 0/1 register.  Needs n <= C-64.
  __device__ __forceinline__ void offer64_masked(uint64_t bal, uint64_t key) {
    if (__builtin_amdgcn_inverse_ballot_w64(bal)) buf[n + lanes_below(bal)] = key;
    n = __builtin_amdgcn_readfirstlane(n + __builtin_popcountll(bal));
  }

  // Compacting whenever more than C - 128 keys are held leaves room for two
  // 64-key offers before the next check.
  __device__ __forceinline__ bool needs_compaction() const { return n > C - 2 * kWave; }
  // Most keys compact() keeps.
  __device__ __forceinline__ int compact_cmax() const { return top_k + kWave < CMAX ? top_k + kWave : CMAX; }
  // Close enough to needing a compaction that joining one that another row
  // of the workgroup needs is worthwhile: more than halfway from what a
  // compaction keeps to the compaction threshold.
  __device__ __forceinline__ bool wants_compaction() const { return n > (compact_cmax() + C - 2 * kWave) / 2; }

  // Lower bounds of the held count at a compaction: needs_compaction() holds
  // n > NEEDS_MIN, and wants_compaction() n > WANTS_MIN for every top_k >= 1.
  static constexpr int NEEDS_MIN = C - 2 * kWave;
  static constexpr int WANTS_MIN = ((kWave + 1 < CMAX ? kWave + 1 : CMAX) + C - 2 * kWave) / 2;

  // Keys counted one 64-key row at a time: a compare into a lane mask and a
  // scalar popcount (one VALU instruction per row).
  __device__ __forceinline__ static int count_hi_ge(const uint64_t (&v)[E], uint32_t h) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key_hi(v[j]) >= h));
    return c;
  }

  __device__ __forceinline__ static int count_ge(const uint64_t (&v)[E], uint64_t p) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(v[j] >= p));
    return c;
  }

  // Raises the floor so that kk <= n <= cmax (needs n > cmax and kk <= cmax).
  // MINN is a lower bound of n known at the call: the rows below it are
  // loaded without the per-slot check against n.
  template <int MINN>
  __device__ __forceinline__ void compact_to(int lane, int kk, int cmax) {
    constexpr int FULL = (MINN + 1) / kWave < E ? (MINN + 1) / kWave : E;  // rows wholly below n
    wave_lds_sync();
    uint64_t v[E];
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int pos = j * kWave + lane;
      const uint64_t x = buf[pos];
      v[j] = (j < FULL || pos < n) ? x : 0ull;
      mx = key_hi(v[j]) > mx ? key_hi(v[j]) : mx;
    }
    mx = wave_max_u32(mx);
    const int target = kk + (cmax - kk) / 4;
    uint64_t lo = tau, hi_ = static_cast<uint64_t>(mx) + 1;
    int c_lo = n, c_hi = 0;
    uint64_t P = 0;
    int c = 0;
    bool found = false;
    for (int it = 0; it < 48 && hi_ - lo > 1; ++it) {
      const uint64_t span = hi_ - lo;
      uint64_t step;
      if (it & 1) {
        step = span >> 1;
      } else {
        const float f = static_cast<float>(c_lo - target) * __builtin_amdgcn_rcpf(static_cast<float>(c_lo - c_hi));
        const float half_span = static_cast<float>(static_cast<uint32_t>(span >> 1));
        step = static_cast<uint64_t>(static_cast<uint32_t>(half_span * __builtin_fminf(f, 1.0f))) << 1;
      }
      step = step < 1 ? 1 : (step > span - 1 ? span - 1 : step);
      const uint32_t mid = static_cast<uint32_t>(lo + step);
      c = count_hi_ge(v, mid);
      if (c >= kk && c <= cmax) {
        P = static_cast<uint64_t>(mid) << 32;
        found = true;
        break;
      }
      if (c > cmax) {
        lo = mid;
        c_lo = c;
      } else {
        hi_ = mid;
        c_hi = c;
      }
    }
    if (!found) {
      uint64_t plo = lo << 32;
      uint64_t phi = hi_ >= (1ull << 32) ? ~0ull : (hi_ << 32);
      for (int it = 0; it < 64 && phi - plo > 1; ++it) {
        const uint64_t mid = plo + ((phi - plo) >> 1);
        c = count_ge(v, mid);
        if (c >= kk && c <= cmax) {
          P = mid;
          found = true;
          break;
        }
        if (c > cmax) plo = mid; else phi = mid;
      }
      if (!found) {
        P = phi;
        c = count_ge(v, P);
      }
    }
    wave_lds_sync();
    // The kept keys (every key >= P; P > 0, so no empty slot) are written
    // densely, row by row in lane order; the others are not written.  r ends
    // equal to c.
    int r = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const bool keep = v[j] >= P;
      const uint64_t m = __builtin_amdgcn_ballot_w64(keep);
      if (keep) buf[r + lanes_below(m)] = v[j];
      r += __builtin_popcountll(m);
    }
    n = __builtin_amdgcn_readfirstlane(c);
    floor_key = P;
    tau = __builtin_amdgcn_readfirstlane(key_hi(P));
    wave_lds_sync();
  }

  // Keeping close to top_k keys leaves the most room and the highest floor.
  // MINN: a lower bound of n at the call (WANTS_MIN covers every caller;
  // NEEDS_MIN those that compact only when needs_compaction() holds).
  template <int MINN = WANTS_MIN>
  __device__ __forceinline__ void compact(int lane) { compact_to<MINN>(lane, top_k, compact_cmax()); }

  // Sorted top_k of the row, written through `out` (see TopkRowOut).  The
  // held keys are cut to exactly top_k when more are held than the sort
  // width, then the smallest power-of-two number of keys per lane that holds
  // top_k (at most E) is bitonic-sorted in registers.
  // Widest sort this capacity needs: keys per lane for the largest top_k it
  // serves (C - 192), rounded up to a power of two.  It may exceed E (slots
  // past the held count load as zero keys).
  static constexpr int SE_CAP = (C - 192) <= 1 * kWave ? 1 : (C - 192) <= 2 * kWave ? 2
                              : (C - 192) <= 4 * kWave ? 4 : (C - 192) <= 8 * kWave ? 8
                              : (C - 192) <= 16 * kWave ? 16 : 32;
  // Above 2048 keys (32 per lane) finish() sorts two 2048-key runs and merges
  // them, which needs room for 4096 keys in the buffer.
  static constexpr bool MERGED = C >= 4096 + 192;
  // Largest top_k this capacity serves: what a compaction may keep, and what
  // the final sort writes.  Launchers reject anything larger.
  static constexpr int MAX_TOPK = MERGED ? (CMAX < 4096 ? CMAX : 4096) : (CMAX < SE_CAP * kWave ? CMAX : SE_CAP * kWave);

  __device__ __forceinline__ void finish(const TopkRowOut& out, int lane) {
    if (top_k > 32 * kWave) {
      if constexpr (MERGED) finish_merged(out, lane);
    } else if (top_k <= 1 * kWave) {
      finish_sorted<1>(out, lane);
    } else if (top_k <= 2 * kWave) {
      if constexpr (SE_CAP >= 2) finish_sorted<2>(out, lane);
    } else if (top_k <= 4 * kWave) {
      if constexpr (SE_CAP >= 4) finish_sorted<4>(out, lane);
    } else if (top_k <= 8 * kWave) {
      if constexpr (SE_CAP >= 8) finish_sorted<8>(out, lane);
    } else if (top_k <= 16 * kWave) {
      if constexpr (SE_CAP >= 16) finish_sorted<16>(out, lane);
    } else {
      if constexpr (SE_CAP >= 32) finish_sorted<32>(out, lane);
    }
  }

  template <int SE>
  __device__ __forceinline__ void finish_sorted(const TopkRowOut& out, int lane) {
    if (n > SE * kWave) compact_to<SE * kWave>(lane, top_k, top_k);
    wave_lds_sync();
    uint64_t v[SE];
#pragma unroll
    for (int j = 0; j < SE; ++j) {
      const int pos = j * kWave + lane;
      if (j < E) {
        v[j] = pos < n ? buf[pos] : 0ull;
      } else {
        v[j] = 0ull;  // past the buffer (SE > E): never held
      }
    }
    wave_sort_desc<SE>(v, lane);
    write_out<SE>(v, out, lane);
  }

  // 2048 < top_k <= 4096: the held keys (cut to exactly top_k) are split into
  // two runs of up to 2048 keys, each bitonic-sorted in registers and written
  // back in rank order; then each lane merges 64 consecutive output ranks,
  // its start in both runs found by a merge-path binary search.
  __device__ __forceinline__ void sort_run(int base, int lane) {
    uint64_t v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int pos = base + j * kWave + lane;
      v[j] = pos < n ? buf[pos] : 0ull;
    }
    wave_sort_desc<32>(v, lane);
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < 32; ++j) buf[base + lane * 32 + j] = v[j];
    wave_lds_sync();
  }

  __device__ __forceinline__ void finish_merged(const TopkRowOut& out, int lane) {
    constexpr int L = 32 * kWave;  // run length
    if (n > top_k) compact_to<32 * kWave>(lane, top_k, top_k);  // (top_k > 2048 here)
    wave_lds_sync();
    sort_run(0, lane);
    sort_run(L, lane);
    const uint64_t* A = buf;
    const uint64_t* Bv = buf + L;
    // Output ranks [d, d + 64) of this lane: i of them come from run A.
    const int d = lane * kWave;
    int lo = d > L ? d - L : 0, hi = d < L ? d : L;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (A[mid] >= Bv[d - 1 - mid]) lo = mid + 1; else hi = mid;
    }
    int i = lo, j = d - lo;
    for (int e = 0; e < kWave; ++e) {
      const int o = d + e;
      if (o >= top_k) break;
      const uint64_t x = i < L ? A[i] : 0ull;
      const uint64_t y = j < L ? Bv[j] : 0ull;
      const bool ta = x >= y;
      const uint64_t k = ta ? x : y;
      i += ta ? 1 : 0;
      j += ta ? 0 : 1;
      if (out.idx64) out.idx64[o] = k ? static_cast<int64_t>(key_idx(k)) : int64_t(-1);
      if (out.score) out.score[o] = k ? ord_to_f32(key_hi(k)) : -__builtin_inff();
      if (out.idx32) out.idx32[o] = k ? static_cast<int32_t>(key_idx(k)) + out.off32 : int32_t(-1);
    }
  }

  // Keys of rank lane*EE+j are staged through LDS in rank order so that the
  // global stores are contiguous across the wave.
  template <int EE>
  __device__ __forceinline__ void write_out(const uint64_t (&v)[EE], const TopkRowOut& out, int lane) const {
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < EE; ++j) {
      // Ranks past the buffer (EE * 64 > C) are never written out (top_k < C)
      // and must not reach the next wave's buffer.
      const int r = lane * EE + j;
      if (EE * kWave <= C || r < C) buf[r] = v[j];
    }
    wave_lds_sync();
    for (int e = lane; e < top_k; e += kWave) {
      const uint64_t k = buf[e];
      if (out.idx64) out.idx64[e] = k ? static_cast<int64_t>(key_idx(k)) : int64_t(-1);
      if (out.score) out.score[e] = k ? ord_to_f32(key_hi(k)) : -__builtin_inff();
      if (out.idx32) out.idx32[e] = k ? static_cast<int32_t>(key_idx(k)) + out.off32 : int32_t(-1);
    }
  }
};

}  // namespace si
