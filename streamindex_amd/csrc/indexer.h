// Lightning-indexer kernel interface shared by the C-ABI entry (indexer.hip)
// and the per-shape instantiation units (indexer_inst_d*.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

struct IndexerArgs {
  const uint16_t* q;  // [B,S,H,D] bf16, d contiguous
  int64_t qsb, qss, qsh;
  const uint16_t* k;  // [B,T,D] bf16, d contiguous
  int64_t ksb, kst;
  const void* w;      // [B,S,H] fp32 or bf16
  int64_t wsb, wss, wsh;
  int w_bf16;
  const uint8_t* mask;  // optional [B,S,T] bool (nonzero = legal)
  int64_t msb, mss, mst;
  int B, S, T, H;
  int top_k;
  int ratio;  // > 0: legal iff t < (s+1)/ratio; 0: no causal bound
  int64_t* out_idx;     // [B,S,top_k] contiguous, or null when out_idx32 is set
  float* out_scores;    // [B,S,top_k] contiguous, or null
  // CSA index rows instead of out_idx: [B,S,n_win+top_k] int32 with batch /
  // row strides o32sb / o32ss (columns contiguous).  Columns [0, n_win) hold
  // the sliding window s-n_win+1 .. s (-1 below 0); columns n_win.. hold the
  // selected keys plus idx_offset (-1 past the legal count).
  int32_t* out_idx32;
  int64_t o32sb, o32ss;
  int n_win;
  int idx_offset;
  float* scores;        // score kernel: [B,S,T]
  int64_t ssb, sss, sst;
  int accumulate;       // score kernel: add to the scores already stored (a later head group)
};

// Selection-buffer capacities the top-k kernel is instantiated for: 256,
// 512, 1024, 1536, 2048 and 4096 keys per query row (capacity C serves
// top_k <= C - 192; up to C = 1536 two workgroups share a CU).

template <int HB, int D, int C>
int launch_topk(const IndexerArgs& a, hipStream_t st);

// Shapes served by the four-M-block top-k kernel (indexer_topk_wide.h):
// HB = 2 (two rows per wave, 8 rows per workgroup) or HB = 4 (one row per
// wave), D = 128, and LDS for its 3-slot K ring (64-key tiles) plus the
// workgroup's selection buffers and compaction requests.
template <int HB, int D, int C>
constexpr bool topk_wide_fits() {
  return (HB == 2 || HB == 4) && D == 128 && 3 * 64 * D * 2 + 4 * (4 / HB) * C * 8 + 3 * 4 * 4 <= 160 * 1024;
}

template <int HB, int D, int C>
int launch_topk_wide(const IndexerArgs& a, hipStream_t st);

// Top-k kernel choice (SI_TOPK_KERNEL_AUTO / _NARROW / _WIDE, set through
// si_indexer_set_topk_kernel).
extern int g_topk_kernel_mode;

// Whether the four-M-block kernel is the faster one (measured): always for
// one 128-head row per wave (the other kernel then runs one wave per SIMD
// too), and for two 64-head rows per wave when rows reach 64K legal keys
// (its single wave per SIMD pays per-row costs -- final sort, compactions,
// workgroup tail -- that the two-workgroup-per-CU indexer_topk_kernel
// hides, and wins in the MFMA loop that long rows spend their time in).
// It needs T >= 64: the copies of a tile past the last one re-read rows 0..63
// of k_idx (at any mode; SI_TOPK_KERNEL_WIDE then falls back to the other
// kernel).
inline bool topk_wide_preferred(const IndexerArgs& a) {
  if (a.T < 64) return false;
  if (g_topk_kernel_mode == 1) return false;
  if (g_topk_kernel_mode == 2) return true;
  if (a.H > 96) return true;
  const int64_t tmax = a.ratio > 0 ? (a.S / a.ratio < a.T ? a.S / a.ratio : a.T) : a.T;
  return tmax >= 65536;
}

template <int HB, int D>
int launch_score(const IndexerArgs& a, hipStream_t st);

// Head-split top-k kernel (indexer_topk_split.h): HS waves per query row,
// HBH 32-head blocks per wave, selection capacity C.
template <int HS, int HBH, int D, int C>
int launch_topk_split(const IndexerArgs& a, hipStream_t st);

// Which top-k kernel serves a shape, and with which selection capacity
// (the C-ABI dispatch and si_indexer_topk_plan both read it).
enum TopkKernel { TOPK_NARROW = 1, TOPK_WIDE = 2, TOPK_SPLIT = 3 };
struct TopkPlan {
  int kernel;  // TopkKernel
  int cap;     // selection capacity (keys per row)
  int hb;      // 32-head blocks per wave (narrow / wide: of the whole row)
  int hs;      // waves per query row (split kernel), else 1
};

}  // namespace si
