// Launchers of the lightning-indexer kernels and the per-shape instantiation
// macro used by indexer_inst_d*.hip: launch_topk (indexer_topk_kernel,
// indexer_kernels.h), launch_topk_wide (four 32-head blocks per wave,
// indexer_topk_wide.h; the C-ABI dispatch picks it for long rows) and
// launch_score.  Both top-k kernels return the same results.
#pragma once

#include "indexer_kernels.h"
#include "indexer_topk_wide.h"

namespace si {

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
template <int HB, int D, int C>
int launch_topk(const IndexerArgs& a, hipStream_t st) {
  if constexpr (!topk_fits_lds<HB, D, C>()) {
    return set_error(SI_ERR_UNSUPPORTED, "top_k too large for this head dim (the selection buffers exceed LDS)");
  } else {
  if (a.top_k > WaveSelect<C>::MAX_TOPK) return set_error(SI_ERR_UNSUPPORTED, "top_k exceeds the selection capacity");
  constexpr int NW = TopkShape<C>::NW;
  const int nqb = (a.S + NW - 1) / NW;
  const int64_t nblk = static_cast<int64_t>(nqb) * a.B;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  if (a.mask) {
    hipLaunchKernelGGL((indexer_topk_kernel<HB, D, C, true>), dim3(static_cast<unsigned>(nblk)), dim3(NW * 64),
                       0, st, a);
  } else {
    hipLaunchKernelGGL((indexer_topk_kernel<HB, D, C, false>), dim3(static_cast<unsigned>(nblk)), dim3(NW * 64),
                       0, st, a);
  }
  return check_launch("indexer_topk_kernel");
  }
}

template <int HB, int D>
int launch_score(const IndexerArgs& a, hipStream_t st) {
  // 8 rows per workgroup (two waves per SIMD) up to two head blocks at
  // D <= 128; wider rows need a SIMD's registers for one wave.
  constexpr int NW = (HB <= 2 && D <= 128) ? 8 : 4;
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
  template int launch_topk<HB, D, 1536>(const IndexerArgs&, hipStream_t); \
  template int launch_topk<HB, D, 2048>(const IndexerArgs&, hipStream_t); \
  template int launch_topk<HB, D, 4096>(const IndexerArgs&, hipStream_t);    \
  template int launch_topk_wide<HB, D, 1024>(const IndexerArgs&, hipStream_t); \
  template int launch_topk_wide<HB, D, 1536>(const IndexerArgs&, hipStream_t); \
  template int launch_topk_wide<HB, D, 2048>(const IndexerArgs&, hipStream_t);

}  // namespace si
