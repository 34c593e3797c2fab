// Lightning-indexer kernels for gfx950 (templates; instantiated per head dim
// in indexer_inst_d*.hip).
//
//   I(s, t) = sum_h w[s, h] * relu(q[s, h, :] . k[t, :])        (bf16 in, fp32 acc)
//
// Reference behaviour being replaced:
//   * flash_sparse/triton/indexer_score.py:41-120   (_indexer_score_kernel)
//   * flash_sparse/triton/indexer_score.py:123-179  (indexer_score wrapper)
//   * flash_sparse/triton/chunked_indexer.py:47-160 (chunked partition-merge top-k)
//
// Design (one query row per wavefront, NW rows per workgroup):
//   * The row's Q block [H, D] lives in VGPRs as MFMA A-fragments (heads on
//     the M axis), loaded once.  K tiles of TILE_N keys are streamed through
//     a double-buffered, XOR-swizzled LDS ring shared by the workgroup; the
//     global loads of tile i+1 are in flight while tile i is consumed.
//   * Per 32-key block, v_mfma_f32_32x32x16_bf16 produces [32 heads x 32 keys]
//     per M-block; lane l holds key l%32 for 16 heads, so ReLU (v_med3) and
//     the fp32 weighted head sum are in-lane, finished by one xor-32 exchange.
//     B-fragments of block nb+1 are read from LDS while block nb's MFMAs run.
//   * The causal bound t < (s+1)//ratio is evaluated per lane in registers;
//     tiles past the workgroup's last legal key are never loaded or computed.
//   * The top-k kernel never writes scores: each lane offers its key to the
//     wave's selection buffer (wave_select.h); the score kernel stores the
//     fp32 row instead.
//   * Workgroups are issued heaviest-first (the last query block first) so the
//     triangular causal workload drains evenly over the 256 CUs.
#pragma once

#include "indexer.h"
#include "si_common.h"
#include "si_status.h"
#include "wave_select.h"

namespace si {

// Byte offset of 16-byte chunk c of key row r inside a swizzled K tile.
// The XOR spreads the 16 rows read by one ds_read_b128 quarter-wave over
// distinct bank groups.
template <int D>
__device__ __forceinline__ int kt_off(int r, int c) {
  constexpr int CPR = D / 8;                          // 16-byte chunks per row
  constexpr int RPG = (16 / CPR) > 0 ? 16 / CPR : 1;  // rows per 256-byte bank sweep
  constexpr int SW = CPR < 16 ? CPR : 16;
  return r * (D * 2) + ((c ^ ((r / RPG) % SW)) << 4);
}

typedef __attribute__((address_space(3))) void lds_void;

// Copies one K tile straight from HBM/L2 into the swizzled LDS layout with
// global_load_lds_dwordx4 (no staging registers).  One wave instruction
// fills 64 consecutive 16-byte LDS slots (slot = base + lane); each lane
// fetches the global chunk that belongs in its slot under the swizzle.
// Rows past T re-read row T-1; those keys are never legal.
template <int D, int TILE_N, int NTHREADS>
struct KTileLoader {
  static constexpr int CPR = D / 8;
  static constexpr int CHUNKS = TILE_N * CPR;
  static constexpr int LPT = CHUNKS / NTHREADS;
  static_assert(CHUNKS % NTHREADS == 0, "tile must split evenly over the workgroup");

  __device__ __forceinline__ void issue(const uint16_t* kb, int64_t kst, int t0, int T, char* tile) const {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int slot0 = i * NTHREADS + wave * 64;
      const int slot = slot0 + lane;
      const int row = slot / CPR;
      const int c = (slot % CPR) ^ ((kt_off<D>(row, 0) >> 4) - row * CPR);
      int t = t0 + row;
      t = t < T ? t : T - 1;
      __builtin_amdgcn_global_load_lds(kb + static_cast<int64_t>(t) * kst + c * 8,
                                       (lds_void*)(tile + slot0 * 16), 16, 0, 0);
    }
  }
};

// Waits for this thread's tile copies, then makes the tile visible to the workgroup.
__device__ __forceinline__ void tile_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Per-wave query state: A-fragments of Q and the matching head weights.
template <int HB, int D>
struct QueryFrags {
  static constexpr int KS = D / 16;
  bf16x8 qf[HB][KS];
  float wf[HB][16];

  __device__ __forceinline__ void load(const IndexerArgs& a, int b, int s, int lane) {
    const uint16_t* qrow = a.q + b * a.qsb + static_cast<int64_t>(s) * a.qss;
#pragma unroll
    for (int mb = 0; mb < HB; ++mb) {
      const int h = mb * 32 + (lane & 31);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d = ks * 16 + (lane >> 5) * 8;
        if (h < a.H) {
          qf[mb][ks] = *reinterpret_cast<const bf16x8*>(qrow + h * a.qsh + d);
        } else {
          qf[mb][ks] = bf16x8{};
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int hh = mb * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        float wv = 0.f;
        if (hh < a.H) {
          const int64_t off = b * a.wsb + static_cast<int64_t>(s) * a.wss + hh * a.wsh;
          wv = a.w_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.w)[off])
                        : reinterpret_cast<const float*>(a.w)[off];
        }
        wf[mb][v] = wv;
      }
    }
  }

  __device__ __forceinline__ void load_b(const char* tile, int nb, int lane, bf16x8 (&kb)[KS]) const {
    const int row = nb * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kb[ks] = *reinterpret_cast<const bf16x8*>(tile + kt_off<D>(row, ks * 2 + (lane >> 5)));
  }

  // Score of key (block base + lane%32) for this row; identical in lanes l and l+32.
  __device__ __forceinline__ float score(const bf16x8 (&kb)[KS], int lane) const {
    f32x16 acc[HB];
#pragma unroll
    for (int mb = 0; mb < HB; ++mb) acc[mb] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int mb = 0; mb < HB; ++mb) {
        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[mb][ks], kb[ks], acc[mb], 0, 0, 0);
      }
    }
    float sum = 0.f;
#pragma unroll
    for (int mb = 0; mb < HB; ++mb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        // relu as a single v_med3_f32 (clamp to [0, FLT_MAX])
        sum = __builtin_fmaf(wf[mb][v], __builtin_amdgcn_fmed3f(acc[mb][v], 0.f, __FLT_MAX__), sum);
      }
    }
    return sum + shfl_xor_f32(sum, lane, 32);
  }

  // Scores of the first `nblk` 32-key blocks of a tile (all NB when FULL);
  // block nb+1's B-fragments are read while block nb's MFMAs execute.
  template <int NB, bool FULL>
  __device__ __forceinline__ void tile_scores(const char* tile, int nblk, int lane, float (&sc)[NB]) const {
    bf16x8 kb[2][KS];
    load_b(tile, 0, lane, kb[0]);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (FULL || nb < nblk) {
        if (nb + 1 < NB && (FULL || nb + 1 < nblk)) load_b(tile, nb + 1, lane, kb[(nb + 1) & 1]);
        sc[nb] = score(kb[nb & 1], lane);
      } else {
        sc[nb] = 0.f;
      }
    }
  }
};

__device__ __forceinline__ int legal_limit(const IndexerArgs& a, int s) {
  if (a.ratio > 0) {
    const int l = (s + 1) / a.ratio;
    return l < a.T ? l : a.T;
  }
  return a.T;
}

// ---------------------------------------------------------------------------
// Fused score + streaming exact top-k.
// ---------------------------------------------------------------------------
template <int HB, int D, int C, int NW, int TILE_N>
__global__ __launch_bounds__(NW * 64, 1) void indexer_topk_kernel(IndexerArgs a) {
  constexpr int NT = NW * 64;
  constexpr int NB = TILE_N / 32;
  constexpr int TILE_BYTES = TILE_N * D * 2;
  // One LDS arena: the DMA-filled K ring first (offsets below 64 KiB, the
  // range global_load_lds destinations are kept in), then the per-wave
  // selection buffers.
  __shared__ __attribute__((aligned(16))) char lds[2 * TILE_BYTES + NW * C * 8];
  uint64_t* const sel_base = reinterpret_cast<uint64_t*>(lds + 2 * TILE_BYTES);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nqb = (a.S + NW - 1) / NW;
  const int b = blockIdx.x % a.B;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x / a.B);  // heaviest first
  const int s0 = qb * NW;
  const int s = s0 + wave;
  const bool active = s < a.S;
  const int s_last = (s0 + NW < a.S ? s0 + NW : a.S) - 1;
  const int my_lim = active ? legal_limit(a, s) : 0;
  const int wg_lim = legal_limit(a, s_last);

  QueryFrags<HB, D> qfr;
  if (active) qfr.load(a, b, s, lane);

  WaveSelect<C> sel;
  sel.init(sel_base + wave * C, a.top_k);

  const uint16_t* kb = a.k + b * a.ksb;
  const uint8_t* mrow =
      a.mask ? a.mask + b * a.msb + static_cast<int64_t>(active ? s : 0) * a.mss : nullptr;

  const KTileLoader<D, TILE_N, NT> ld;
  const int ntiles = (wg_lim + TILE_N - 1) / TILE_N;
  if (ntiles > 0) ld.issue(kb, a.kst, 0, a.T, lds);
  tile_barrier();

  for (int it = 0; it < ntiles; ++it) {
    const bool more = it + 1 < ntiles;
    if (more) ld.issue(kb, a.kst, (it + 1) * TILE_N, a.T, lds + ((it + 1) & 1) * TILE_BYTES);
    const char* tile = lds + (it & 1) * TILE_BYTES;
    const int tbase = it * TILE_N;
    int nblk = (my_lim - tbase + 31) / 32;
    nblk = nblk > NB ? NB : (nblk < 0 ? 0 : nblk);
    float sc[NB];
    if (nblk == NB) {
      qfr.template tile_scores<NB, true>(tile, NB, lane, sc);
    } else if (nblk > 0) {
      qfr.template tile_scores<NB, false>(tile, nblk, lane, sc);
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (nb < nblk) {
        const int t = tbase + nb * 32 + (lane & 31);
        bool legal = (lane < 32) && (t < my_lim);
        if (mrow != nullptr && legal) legal = mrow[static_cast<int64_t>(t) * a.mst] != 0;
        const uint64_t key = make_key(sc[nb], static_cast<uint32_t>(t));
        sel.offer(legal && key_hi(key) > sel.tau, key, lane);
      }
    }
    tile_barrier();
  }

  if (active) {
    const int64_t row = static_cast<int64_t>(b) * a.S + s;
    sel.finish(a.out_idx + row * a.top_k, a.out_scores + row * a.top_k, lane);
  }
}

// ---------------------------------------------------------------------------
// Materialised score matrix [B, S, T] fp32 (no mask, as the reference kernel).
// ---------------------------------------------------------------------------
template <int HB, int D, int NW, int TILE_N>
__global__ __launch_bounds__(NW * 64, 1) void indexer_score_kernel(IndexerArgs a) {
  constexpr int NT = NW * 64;
  constexpr int NB = TILE_N / 32;
  constexpr int TILE_BYTES = TILE_N * D * 2;
  __shared__ __attribute__((aligned(16))) char lds[2 * TILE_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int b = blockIdx.x % a.B;
  const int qb = static_cast<int>(blockIdx.x / a.B);
  const int s = qb * NW + wave;
  const bool active = s < a.S;

  QueryFrags<HB, D> qfr;
  if (active) qfr.load(a, b, s, lane);

  const uint16_t* kb = a.k + b * a.ksb;
  float* orow = a.scores + b * a.ssb + static_cast<int64_t>(active ? s : 0) * a.sss;

  const KTileLoader<D, TILE_N, NT> ld;
  const int ntiles = (a.T + TILE_N - 1) / TILE_N;
  if (ntiles > 0) ld.issue(kb, a.kst, 0, a.T, lds);
  tile_barrier();
  for (int it = 0; it < ntiles; ++it) {
    const bool more = it + 1 < ntiles;
    if (more) ld.issue(kb, a.kst, (it + 1) * TILE_N, a.T, lds + ((it + 1) & 1) * TILE_BYTES);
    const char* tile = lds + (it & 1) * TILE_BYTES;
    if (active) {
      const int tbase = it * TILE_N;
      int nblk = (a.T - tbase + 31) / 32;
      nblk = nblk > NB ? NB : nblk;
      float sc[NB];
      if (nblk == NB) {
        qfr.template tile_scores<NB, true>(tile, NB, lane, sc);
      } else {
        qfr.template tile_scores<NB, false>(tile, nblk, lane, sc);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int t = tbase + nb * 32 + (lane & 31);
        if (nb < nblk && lane < 32 && t < a.T) orow[static_cast<int64_t>(t) * a.sst] = sc[nb];
      }
    }
    tile_barrier();
  }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
template <int C>
struct TopkLaunchShape {
  // (waves per workgroup, keys per LDS tile) so that NW*C*8 + 2*TILE_N*D*2 <= 160 KiB
  // and the K ring (2*TILE_N*D*2 <= 64 KiB) stays where the tile DMA can address it
  static constexpr int NW = C <= 1024 ? 8 : 4;
  static constexpr int TILE_N = C <= 2048 ? 128 : 64;
};

template <int HB, int D, int C>
int launch_topk(const IndexerArgs& a, hipStream_t st) {
  constexpr int NW = TopkLaunchShape<C>::NW;
  constexpr int TILE_N = TopkLaunchShape<C>::TILE_N;
  const int nqb = (a.S + NW - 1) / NW;
  const int64_t nblk = static_cast<int64_t>(nqb) * a.B;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((indexer_topk_kernel<HB, D, C, NW, TILE_N>), dim3(static_cast<unsigned>(nblk)),
                     dim3(NW * 64), 0, st, a);
  return check_launch("indexer_topk_kernel");
}

template <int HB, int D>
int launch_score(const IndexerArgs& a, hipStream_t st) {
  constexpr int NW = 8;
  constexpr int TILE_N = 128;
  const int nqb = (a.S + NW - 1) / NW;
  const int64_t nblk = static_cast<int64_t>(nqb) * a.B;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((indexer_score_kernel<HB, D, NW, TILE_N>), dim3(static_cast<unsigned>(nblk)),
                     dim3(NW * 64), 0, st, a);
  return check_launch("indexer_score_kernel");
}

#define SI_INSTANTIATE_INDEXER(HB, D)                                   \
  template int launch_score<HB, D>(const IndexerArgs&, hipStream_t);    \
  template int launch_topk<HB, D, 256>(const IndexerArgs&, hipStream_t);  \
  template int launch_topk<HB, D, 512>(const IndexerArgs&, hipStream_t);  \
  template int launch_topk<HB, D, 1024>(const IndexerArgs&, hipStream_t); \
  template int launch_topk<HB, D, 2048>(const IndexerArgs&, hipStream_t); \
  template int launch_topk<HB, D, 4096>(const IndexerArgs&, hipStream_t);

}  // namespace si
