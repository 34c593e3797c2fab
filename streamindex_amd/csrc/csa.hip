// CSA / HCA attention-index builders for gfx950.
//
// The sparse-attention kernel reads one int32 index row per query: n_win
// sliding-window columns (keys s-n_win+1 .. s of the uncompressed KV, -1 below
// 0) followed by the compressed-KV columns, offset by the uncompressed length
// S.  Reference behaviour being replaced:
//   * flash_sparse/csa.py:30-83    build_csa_topk_idxs (mask, topk, -1, +S, concat)
//   * flash_sparse/hca.py:24-51    build_hca_topk_idxs (every causally legal block)
//   * flash_sparse/reference.py:460-475  _build_sliding_window_idxs
// The fused indexer writes the same rows straight from its selection
// (si_csa_indexer_topk in indexer.hip); the kernels here serve callers that
// hold a materialised [B,S,T] score matrix, and HCA, which selects nothing.
#include <string>

#include "si_common.h"
#include "si_status.h"
#include "wave_select.h"

namespace si {

struct ScoreTopkArgs {
  const float* scores;  // [B,S,T] fp32
  int64_t ssb, sss, sst;
  int B, S, T;
  int top_k;
  int ratio;       // > 0: key t legal for row s iff t < (s+1)/ratio
  int n_win;
  int idx_offset;  // added to every selected index
  int32_t* out;    // [B,S,n_win+top_k] int32, columns contiguous
  int64_t osb, oss;
};

// Window columns of query s (shared by both builders).
__device__ __forceinline__ void window_cols(int32_t* orow, int s, int n_win, int j0, int step) {
  for (int j = j0; j < n_win; j += step) {
    const int t = s - n_win + 1 + j;
    orow[j] = t >= 0 ? t : -1;
  }
}

// Top-k over a materialised score row, one wave per query row, four rows per
// workgroup.  The row is read in U coalesced 64-key loads per step (one fp32
// per lane each) and offered in index order, which the selection's strict
// arrival filter needs to be exact.  A -inf score is never selected (the
// reference turns a selected -inf into -1, csa.py:68-69).  Waves are
// independent: no workgroup barrier, so a wave past the last row returns.
template <int C>
__global__ __launch_bounds__(256) void score_topk_kernel(ScoreTopkArgs a) {
  constexpr int NW = 4;
  constexpr int U = 8;
  __shared__ __attribute__((aligned(16))) uint64_t sel_lds[NW * C];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * NW + wave;
  if (row >= static_cast<int64_t>(a.B) * a.S) return;
  const int b = static_cast<int>(row / a.S);
  const int s = static_cast<int>(row - static_cast<int64_t>(b) * a.S);
  int lim = a.ratio > 0 ? (s + 1) / a.ratio : a.T;
  lim = lim < a.T ? lim : a.T;
  const float* srow = a.scores + b * a.ssb + static_cast<int64_t>(s) * a.sss;

  WaveSelect<C> sel;
  sel.init(sel_lds + wave * C, a.top_k);
  for (int base = 0; base < lim; base += U * kWave) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = base + u * kWave + lane;
      v[u] = t < lim ? srow[static_cast<int64_t>(t) * a.sst] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + u * kWave < lim) {
        if (sel.needs_compaction()) sel.template compact<WaveSelect<C>::NEEDS_MIN>(lane);
        const int t = base + u * kWave + lane;
        const uint64_t key = make_key(v[u], static_cast<uint32_t>(t));
        const bool pass = t < lim && v[u] != -__builtin_inff() && key_hi(key) > sel.tau;
        sel.offer64(pass, key, lane);
      }
    }
  }
  int32_t* orow = a.out + b * a.osb + static_cast<int64_t>(s) * a.oss;
  window_cols(orow, s, a.n_win, lane, kWave);
  sel.finish(TopkRowOut{nullptr, nullptr, orow + a.n_win, a.idx_offset}, lane);
}

struct HcaIdxArgs {
  int32_t* out;  // [B,S,n_win+n_comp] int32, columns contiguous
  int64_t osb, oss;
  int S, n_win, n_comp, m_prime, idx_offset;
};

// One workgroup per query row: window columns, then compressed block i with
// index i + idx_offset where m'(i+1)-1 <= s, else -1 (hca.py:42-49).
__global__ __launch_bounds__(256) void hca_idx_kernel(HcaIdxArgs a) {
  const int64_t row = blockIdx.x;
  const int b = static_cast<int>(row / a.S);
  const int s = static_cast<int>(row - static_cast<int64_t>(b) * a.S);
  int32_t* orow = a.out + b * a.osb + static_cast<int64_t>(s) * a.oss;
  window_cols(orow, s, a.n_win, threadIdx.x, blockDim.x);
  const int nlegal = (s + 1) / a.m_prime;
  for (int i = threadIdx.x; i < a.n_comp; i += blockDim.x) orow[a.n_win + i] = i < nlegal ? i + a.idx_offset : -1;
}

template <int C>
static int launch_score_topk(const ScoreTopkArgs& a, hipStream_t st) {
  if (a.top_k > WaveSelect<C>::MAX_TOPK) return set_error(SI_ERR_UNSUPPORTED, "top_k exceeds the selection capacity");
  const int64_t rows = static_cast<int64_t>(a.B) * a.S;
  const int64_t nblk = (rows + 3) / 4;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL(score_topk_kernel<C>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, st, a);
  return check_launch("score_topk_kernel");
}

}  // namespace si

using namespace si;

extern "C" int si_csa_scores_topk(const float* scores, const int64_t* score_strides, int64_t B, int64_t S,
                                  int64_t T, int64_t top_k, int64_t causal_ratio, int64_t n_win,
                                  int64_t idx_offset, int32_t* out_idx, const int64_t* out_strides,
                                  void* stream) {
  if (!score_strides || !out_strides) return set_error(SI_ERR_INVALID, "null stride argument");
  if (B < 0 || S < 0 || T < 0) return set_error(SI_ERR_INVALID, "negative dimension");
  if (B > 0x7fffffff || S > 0x7fffffff || T > 0x7fffffff) return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (top_k <= 0) return set_error(SI_ERR_INVALID, "top_k must be positive");
  if (top_k > 4096) return set_error(SI_ERR_UNSUPPORTED, "top_k > 4096 is not supported");
  if (causal_ratio < 0 || causal_ratio > 0x7fffffff) return set_error(SI_ERR_INVALID, "bad causal_ratio");
  if (n_win < 0 || n_win > 0x7fffffff) return set_error(SI_ERR_INVALID, "n_win must be non-negative");
  if (idx_offset < 0 || idx_offset + T > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "idx_offset + T must fit in int32");
  if (out_strides[2] != 1) return set_error(SI_ERR_INVALID, "index rows must be contiguous");
  const bool rows = B > 0 && S > 0;
  if (rows && (!out_idx || (T > 0 && !scores))) return set_error(SI_ERR_INVALID, "null pointer argument");
  ScoreTopkArgs a{};
  a.scores = scores;
  a.ssb = score_strides[0]; a.sss = score_strides[1]; a.sst = score_strides[2];
  a.B = static_cast<int>(B); a.S = static_cast<int>(S); a.T = static_cast<int>(T);
  a.top_k = static_cast<int>(top_k);
  a.ratio = static_cast<int>(causal_ratio);
  a.n_win = static_cast<int>(n_win);
  a.idx_offset = static_cast<int>(idx_offset);
  a.out = out_idx;
  a.osb = out_strides[0]; a.oss = out_strides[1];
  if (!rows) return SI_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a.top_k <= 32) return launch_score_topk<256>(a, st);
  if (a.top_k <= 192) return launch_score_topk<512>(a, st);
  if (a.top_k <= 640) return launch_score_topk<1024>(a, st);
  if (a.top_k <= 1536) return launch_score_topk<2048>(a, st);
  if (a.top_k <= 2048) return launch_score_topk<4096>(a, st);
  return launch_score_topk<4608>(a, st);
}

extern "C" int si_hca_topk_idxs(int64_t B, int64_t S, int64_t n_win, int64_t n_compressed, int64_t m_prime,
                                int64_t idx_offset, int32_t* out_idx, const int64_t* out_strides, void* stream) {
  if (!out_strides) return set_error(SI_ERR_INVALID, "null stride argument");
  if (B < 0 || S < 0 || n_win < 0 || n_compressed < 0) return set_error(SI_ERR_INVALID, "negative dimension");
  if (m_prime <= 0) return set_error(SI_ERR_INVALID, "m_prime must be positive");
  if (S > 0x7fffffff || n_win > 0x7fffffff || m_prime > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (idx_offset < 0 || idx_offset + n_compressed > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "idx_offset + n_compressed must fit in int32");
  if (out_strides[2] != 1) return set_error(SI_ERR_INVALID, "index rows must be contiguous");
  const int64_t rows = B * S;
  if (rows == 0 || n_win + n_compressed == 0) return SI_OK;
  if (!out_idx) return set_error(SI_ERR_INVALID, "null output pointer");
  if (rows > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  HcaIdxArgs a{};
  a.out = out_idx;
  a.osb = out_strides[0]; a.oss = out_strides[1];
  a.S = static_cast<int>(S);
  a.n_win = static_cast<int>(n_win);
  a.n_comp = static_cast<int>(n_compressed);
  a.m_prime = static_cast<int>(m_prime);
  a.idx_offset = static_cast<int>(idx_offset);
  hipLaunchKernelGGL(hca_idx_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("hca_idx_kernel");
}
