// Fused score + streaming exact top-k with each query row's heads split over
// HS waves: the shapes one wave cannot hold.
//
//   I(s, t) = sum_h w[s, h] * relu(q[s, h, :] . k[t, :])        (bf16 in, fp32 acc)
//
// Reference behaviour being replaced: flash_sparse/triton/indexer_score.py:41-179
// (scores, any power-of-two H_I >= 16 and D_I, indexer_score.py:145-150) and
// flash_sparse/triton/chunked_indexer.py:47-160 (chunked top-k, no bound on
// top_k).  indexer_topk_kernel keeps a whole query row (its Q fragments, head
// weights and accumulators) in one wave and four rows' selection buffers in
// LDS, which bounds it at 128 heads (64 at D_I = 256) and top_k = 2048.  This
// kernel serves the shapes past those bounds, up to H_I = 256 and
// top_k = 4096:
//   * A workgroup of four waves takes ROWS = 4 / HS query rows; the HS waves
//     of a row hold HBH 32-head blocks each (heads part * 32 HBH onwards) as
//     v_mfma_f32_32x32x16_bf16 A-fragments, loaded once.
//   * 64-key tiles are copied by global_load_lds into a two-slot swizzled
//     ring shared by the workgroup (tile i+1 in flight during tile i).
//   * Per tile every wave computes its heads' part of the 64 scores (ReLU and
//     fp32 weighted head sum in-lane, the two half-waves' partial sums paired
//     by one v_permlane32_swap) and posts them to LDS; after a barrier the
//     row's first wave adds the HS parts in part order (a fixed order, so the
//     result is deterministic) and offers the 64 keys to the row's selection
//     buffer (wave_select.h); a second barrier per tile ends it.
//   * Only ROWS selection buffers share the LDS, so they can hold 4608 keys
//     (top_k up to 4096; the final sort merges two sorted 2048-key runs).
// Scores agree with the other indexer kernels to fp32 rounding (the head sum
// is associated per part), not bit for bit.
#pragma once

#include "indexer_kernels.h"

namespace si {

template <int HS, int HBH, int D, int C>
struct SplitShape {
  static constexpr int ROWS = 4 / HS;
  static constexpr int TILE_N = 64;
  static constexpr int TILE_BYTES = TILE_N * D * 2;
  static constexpr int SEL_OFF = 2 * TILE_BYTES;  // the DMA ring first (destinations below 64 KiB)
  static constexpr int X_OFF = SEL_OFF + ROWS * C * 8;
  static constexpr int LDS = X_OFF + ROWS * HS * 64 * 4;
};

template <int HS, int HBH, int D, int C>
constexpr bool topk_split_fits() {
  using SS = SplitShape<HS, HBH, D, C>;
  return (HS == 2 || HS == 4) && HBH >= 1 && HBH <= 4 && SS::SEL_OFF <= 65536 && SS::LDS <= 160 * 1024;
}

template <int HS, int HBH, int D, int C>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void indexer_topk_split_kernel(IndexerArgs a) {
  using SS = SplitShape<HS, HBH, D, C>;
  constexpr int NT = 256;
  constexpr int ROWS = SS::ROWS;
  constexpr int TILE_N = SS::TILE_N;
  constexpr int KS = D / 16;  // MFMA k-steps per 32-key block
  constexpr int TILE_BYTES = SS::TILE_BYTES;
  constexpr int BLK_BYTES = 32 * D * 2;
  static_assert(topk_split_fits<HS, HBH, D, C>(), "ring + selection buffers exceed LDS");
  __shared__ __attribute__((aligned(16))) char lds[SS::LDS];
  uint64_t* const sel_base = reinterpret_cast<uint64_t*>(lds + SS::SEL_OFF);
  float* const xch = reinterpret_cast<float*>(lds + SS::X_OFF);  // [ROWS][HS][64] partial scores

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = wave / HS;     // row of the workgroup
  const int part = wave % HS;  // head part of the row
  const int nqb = (a.S + ROWS - 1) / ROWS;
  const int b = blockIdx.x % a.B;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x / a.B);  // heaviest first
  const int s0 = qb * ROWS;
  const int s = s0 + r;
  const bool active = s < a.S;
  const int s_last = (s0 + ROWS < a.S ? s0 + ROWS : a.S) - 1;
  const int my_lim = active ? legal_limit(a, s) : 0;
  const int wg_lim = legal_limit(a, s_last);
  const int h0 = part * HBH * 32;

  // Q A-fragments (heads on M) and head weights of this wave's HBH blocks.
  bf16x8 qf[HBH][KS];
  float wf[HBH][16];
  {
    const int sq = active ? s : 0;
    const uint16_t* qrow = a.q + b * a.qsb + static_cast<int64_t>(sq) * a.qss;
#pragma unroll
    for (int mb = 0; mb < HBH; ++mb) {
      const int h = h0 + mb * 32 + (lane & 31);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d = ks * 16 + (lane >> 5) * 8;
        qf[mb][ks] = (active && h < a.H) ? *reinterpret_cast<const bf16x8*>(qrow + h * a.qsh + d) : bf16x8{};
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int hh = h0 + mb * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        float wv = 0.f;
        if (active && hh < a.H) {
          const int64_t off = b * a.wsb + static_cast<int64_t>(sq) * a.wss + hh * a.wsh;
          wv = a.w_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.w)[off])
                        : reinterpret_cast<const float*>(a.w)[off];
        }
        wf[mb][v] = wv;
      }
    }
  }

  // Per-lane B-fragment offsets of block 0 (block 1 is BLK_BYTES further on).
  int boff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) boff[ks] = kt_off<D>(lane & 31, ks * 2 + (lane >> 5));
  // Which 32-key block of a tile this lane carries after the half-wave swap.
  const int oblk = static_cast<int>(permlane32_swap(0u, 1u).x);
  const int okey = oblk * 32 + (lane & 31);

  const bool owner = part == 0;  // wave-uniform: keeps the row's selection
  WaveSelect<C> sel;
  sel.init(sel_base + r * C, a.top_k);
  const uint16_t* kb = a.k + b * a.ksb;
  const uint8_t* mrow = a.mask ? a.mask + b * a.msb + static_cast<int64_t>(active ? s : 0) * a.mss : nullptr;

  KTileLoader<D, TILE_N, NT> ld;
  ld.init(a.kst);
  const int ntiles = (wg_lim + TILE_N - 1) / TILE_N;
  if (ntiles > 0) ld.issue(kb, a.kst, 0, a.T, lds);
  wait_vm_lgkm0<0>();
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int slot = it & 1;
    const char* tile = lds + slot * TILE_BYTES;
    // The other slot held tile it-1, which every wave finished before the
    // barrier that ended the previous tile.
    if (it + 1 < ntiles) ld.issue(kb, a.kst, (it + 1) * TILE_N, a.T, lds + (slot ^ 1) * TILE_BYTES);
    const int tbase = it * TILE_N;
    int nblk = (my_lim - tbase + 31) / 32;
    nblk = nblk > 2 ? 2 : (nblk < 0 ? 0 : nblk);
    float p[2] = {0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      if (nb < nblk) {
        bf16x8 kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const bf16x8*>(tile + boff[ks] + nb * BLK_BYTES);
        f32x16 acc[HBH];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
          for (int mb = 0; mb < HBH; ++mb)
            acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[mb][ks], kf[ks], ks == 0 ? f32x16{} : acc[mb], 0, 0,
                                                              0);
        }
#pragma unroll
        for (int mb = 0; mb < HBH; ++mb) {
          // ReLU as v_med3_f32, then the fp32 weighted sum over this lane's 16 heads
          float s0v = 0.f, s1v = 0.f;
#pragma unroll
          for (int v = 0; v < 16; v += 2) {
            s0v = __builtin_fmaf(wf[mb][v], __builtin_amdgcn_fmed3f(acc[mb][v], 0.f, __FLT_MAX__), s0v);
            s1v = __builtin_fmaf(wf[mb][v + 1], __builtin_amdgcn_fmed3f(acc[mb][v + 1], 0.f, __FLT_MAX__), s1v);
          }
          p[nb] += s0v + s1v;
        }
      }
    }
    // Lanes 0..31 get block 0's two half-wave sums, lanes 32..63 block 1's.
    const SwapPair sp = permlane32_swap(__float_as_uint(p[0]), __float_as_uint(p[1]));
    xch[(r * HS + part) * kWave + lane] = __uint_as_float(sp.x) + __uint_as_float(sp.y);
    __syncthreads();  // partial scores posted
    if (owner) {
      float tot = xch[(r * HS) * kWave + lane];
#pragma unroll
      for (int q = 1; q < HS; ++q) tot += xch[(r * HS + q) * kWave + lane];
      const int t = tbase + okey;
      bool legal = t < my_lim;
      if (mrow) legal = legal && mrow[static_cast<int64_t>(t < my_lim ? t : 0) * a.mst] != 0;
      const uint64_t key = make_key(tot, static_cast<uint32_t>(t));
      sel.offer64(legal && key_hi(key) > sel.tau, key, lane);
      // one offer per tile: compact before the next one can overflow
      if (sel.needs_compaction()) sel.template compact<WaveSelect<C>::NEEDS_MIN>(lane);
    }
    // Tile it+1 landed; the partial scores of this tile have been read.
    wait_vm_lgkm0<0>();
    __syncthreads();
  }

  if (owner && active) {
    const int64_t row = static_cast<int64_t>(b) * a.S + s;
    TopkRowOut out{nullptr, a.out_scores ? a.out_scores + row * a.top_k : nullptr, nullptr, 0};
    if (a.out_idx32) {
      int32_t* orow = a.out_idx32 + b * a.o32sb + static_cast<int64_t>(s) * a.o32ss;
      write_window_cols(orow, s, a.n_win, lane);
      out.idx32 = orow + a.n_win;
      out.off32 = a.idx_offset;
    } else {
      out.idx64 = a.out_idx + row * a.top_k;
    }
    sel.finish(out, lane);
  }
}

template <int HS, int HBH, int D, int C>
int launch_topk_split(const IndexerArgs& a, hipStream_t st) {
  if constexpr (!topk_split_fits<HS, HBH, D, C>()) {
    return set_error(SI_ERR_UNSUPPORTED, "shape not served by the head-split top-k kernel");
  } else {
    if (a.top_k > WaveSelect<C>::MAX_TOPK) return set_error(SI_ERR_UNSUPPORTED, "top_k exceeds the selection capacity");
    if ((a.H + 32 * HBH - 1) / (32 * HBH) > HS) return set_error(SI_ERR_UNSUPPORTED, "H_I exceeds the head split");
    constexpr int ROWS = SplitShape<HS, HBH, D, C>::ROWS;
    const int nqb = (a.S + ROWS - 1) / ROWS;
    const int64_t nblk = static_cast<int64_t>(nqb) * a.B;
    if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
    hipLaunchKernelGGL((indexer_topk_split_kernel<HS, HBH, D, C>), dim3(static_cast<unsigned>(nblk)), dim3(256), 0,
                       st, a);
    return check_launch("indexer_topk_split_kernel");
  }
}

}  // namespace si
