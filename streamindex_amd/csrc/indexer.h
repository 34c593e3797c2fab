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
};

// Selection-buffer capacities the top-k kernel is instantiated for: 256,
// 512, 1024, 1536, 2048 and 4096 keys per query row (capacity C serves
// top_k <= C - 192; up to C = 1536 two workgroups share a CU).

template <int HB, int D, int C>
int launch_topk(const IndexerArgs& a, hipStream_t st);

template <int HB, int D>
int launch_score(const IndexerArgs& a, hipStream_t st);

}  // namespace si
