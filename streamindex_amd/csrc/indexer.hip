// Lightning-indexer C-ABI entries: argument validation and shape dispatch.
// Kernels: indexer_kernels.h (instantiated per head dim in indexer_inst_d*.hip).
#include <string>

#include "indexer.h"
#include "si_status.h"

namespace si {

int g_topk_kernel_mode = 0;

template <int HB, int D>
static int dispatch_kcap(const IndexerArgs& a, hipStream_t st) {
  // A compaction keeps between top_k and C - 192 keys; the capacity is
  // chosen so that this window leaves room for several 64-key offers.  The
  // four-M-block kernel (HB 2 and 4, D = 128, long rows) runs one workgroup
  // per CU and stalls the CU while a row compacts, so it takes the largest
  // capacity its LDS holds: compactions become rarer.
  if constexpr (topk_wide_fits<HB, D, 1024>()) {
    if (topk_wide_preferred(a)) {
      if (a.top_k <= 192) return launch_topk_wide<HB, D, 1024>(a, st);
      if (a.top_k <= 1152 && topk_wide_fits<HB, D, 2048>()) return launch_topk_wide<HB, D, 2048>(a, st);
      if (a.top_k <= 1152) return launch_topk_wide<HB, D, 1536>(a, st);
    }
  }
  // (Capacity 1536 rather than 1024 above top_k = 192: fewer compactions,
  // still two workgroups per CU; measured 1.4 % faster at S = 64K, k = 512.)
  if (a.top_k <= 32) return launch_topk<HB, D, 256>(a, st);
  if (a.top_k <= 192) return launch_topk<HB, D, 512>(a, st);
  if (a.top_k <= 1152) return launch_topk<HB, D, 1536>(a, st);
  if (a.top_k <= 1536) return launch_topk<HB, D, 2048>(a, st);
  if (a.top_k <= 2048) return launch_topk<HB, D, 4096>(a, st);
  return set_error(SI_ERR_UNSUPPORTED, "top_k > 2048 is not supported");
}

template <bool TOPK>
static int dispatch_shape(const IndexerArgs& a, int D, hipStream_t st) {
  const int HB = (a.H + 31) / 32;
#define SI_CASE(hb, d)                                                            \
  if (HB == hb && D == d) {                                                       \
    return TOPK ? dispatch_kcap<hb, d>(a, st) : launch_score<hb, d>(a, st);       \
  }
  SI_CASE(1, 32)
  SI_CASE(1, 64)
  SI_CASE(1, 128)
  SI_CASE(1, 256)
  SI_CASE(2, 32)
  SI_CASE(2, 64)
  SI_CASE(2, 128)
  SI_CASE(2, 256)
  SI_CASE(3, 32)
  SI_CASE(3, 64)
  SI_CASE(3, 128)
  SI_CASE(4, 32)
  SI_CASE(4, 64)
  SI_CASE(4, 128)
#undef SI_CASE
  return set_error(SI_ERR_UNSUPPORTED,
                   "unsupported indexer shape: H_I=" + std::to_string(a.H) + " D_I=" + std::to_string(D) +
                       " (supported: D_I in {32,64,128} with H_I<=128, D_I=256 with H_I<=64)");
}

static int fill_common(IndexerArgs& a, const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                       const void* w, int w_dtype, const int64_t* ws, int64_t B, int64_t S, int64_t T,
                       int64_t H, int64_t D) {
  if (!qs || !ks || !ws) return set_error(SI_ERR_INVALID, "null stride argument");
  if (B < 0 || S < 0 || T < 0 || H <= 0 || D <= 0) return set_error(SI_ERR_INVALID, "negative or zero dimension");
  // Empty tensors may carry a null data pointer; only non-empty ones are dereferenced.
  const bool rows = B > 0 && S > 0;
  if ((rows && (!q || !w)) || (B > 0 && T > 0 && !k)) return set_error(SI_ERR_INVALID, "null pointer argument");
  if (B > 0x7fffffff || S > 0x7fffffff || T > 0x7fffffff) return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (qs[3] != 1 || ks[2] != 1) return set_error(SI_ERR_INVALID, "q and k_idx need a contiguous last dimension");
  if ((qs[2] % 8) || (qs[1] % 8) || (qs[0] % 8) || (ks[1] % 8) || (ks[0] % 8))
    return set_error(SI_ERR_INVALID, "q/k_idx strides must be multiples of 8 elements (16-byte rows)");
  if (ks[1] < 0 || ks[1] >= (int64_t(1) << 23))  // tile loads address 128 rows with 32-bit byte offsets
    return set_error(SI_ERR_UNSUPPORTED, "k_idx row stride must be below 2^23 elements");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) & 15)  // null is aligned
    return set_error(SI_ERR_INVALID, "q/k_idx must be 16-byte aligned");
  if (w_dtype != 0 && w_dtype != 1) return set_error(SI_ERR_INVALID, "weights dtype must be fp32 (0) or bf16 (1)");
  a.q = static_cast<const uint16_t*>(q);
  a.qsb = qs[0]; a.qss = qs[1]; a.qsh = qs[2];
  a.k = static_cast<const uint16_t*>(k);
  a.ksb = ks[0]; a.kst = ks[1];
  a.w = w; a.wsb = ws[0]; a.wss = ws[1]; a.wsh = ws[2];
  a.w_bf16 = w_dtype;
  a.B = static_cast<int>(B); a.S = static_cast<int>(S); a.T = static_cast<int>(T); a.H = static_cast<int>(H);
  return SI_OK;
}

}  // namespace si

using namespace si;

extern "C" int si_indexer_set_topk_kernel(int mode) {
  if (mode < 0 || mode > 2) return set_error(SI_ERR_INVALID, "top-k kernel mode must be 0 (auto), 1 or 2"), -1;
  const int prev = g_topk_kernel_mode;
  g_topk_kernel_mode = mode;
  return prev;
}

extern "C" int si_indexer_topk(const void* q, const int64_t* q_strides, const void* k_idx,
                               const int64_t* k_strides, const void* weights, int w_dtype,
                               const int64_t* w_strides, const uint8_t* mask, const int64_t* mask_strides,
                               int64_t B, int64_t S, int64_t T, int64_t H, int64_t D, int64_t top_k,
                               int64_t causal_ratio, int64_t* out_idx, float* out_scores, void* stream) {
  IndexerArgs a{};
  int rc = fill_common(a, q, q_strides, k_idx, k_strides, weights, w_dtype, w_strides, B, S, T, H, D);
  if (rc) return rc;
  if (top_k <= 0) return set_error(SI_ERR_INVALID, "top_k must be positive");
  if (causal_ratio < 0) return set_error(SI_ERR_INVALID, "causal_ratio must be positive");
  if (mask && causal_ratio > 0) return set_error(SI_ERR_INVALID, "specify either causal_mask or causal_ratio, not both");
  if (mask && !mask_strides) return set_error(SI_ERR_INVALID, "mask strides missing");
  if ((!out_idx || !out_scores) && B > 0 && S > 0) return set_error(SI_ERR_INVALID, "null output pointer");
  if (causal_ratio > 0x7fffffff) return set_error(SI_ERR_INVALID, "causal_ratio too large");
  a.top_k = static_cast<int>(top_k);
  a.ratio = static_cast<int>(causal_ratio);
  a.mask = mask;
  if (mask) { a.msb = mask_strides[0]; a.mss = mask_strides[1]; a.mst = mask_strides[2]; }
  a.out_idx = out_idx;
  a.out_scores = out_scores;
  if (a.B == 0 || a.S == 0) return SI_OK;
  return dispatch_shape<true>(a, static_cast<int>(D), static_cast<hipStream_t>(stream));
}

extern "C" int si_csa_indexer_topk(const void* q, const int64_t* q_strides, const void* k_idx,
                                   const int64_t* k_strides, const void* weights, int w_dtype,
                                   const int64_t* w_strides, int64_t B, int64_t S, int64_t T, int64_t H,
                                   int64_t D, int64_t top_k, int64_t causal_ratio, int64_t n_win,
                                   int64_t idx_offset, int32_t* out_idx, const int64_t* out_strides,
                                   float* out_scores, void* stream) {
  IndexerArgs a{};
  int rc = fill_common(a, q, q_strides, k_idx, k_strides, weights, w_dtype, w_strides, B, S, T, H, D);
  if (rc) return rc;
  if (top_k <= 0) return set_error(SI_ERR_INVALID, "top_k must be positive");
  if (causal_ratio < 0 || causal_ratio > 0x7fffffff) return set_error(SI_ERR_INVALID, "bad causal_ratio");
  if (n_win < 0 || n_win > 0x7fffffff) return set_error(SI_ERR_INVALID, "n_win must be non-negative");
  if (idx_offset < 0 || idx_offset + T > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "idx_offset + T must fit in int32");
  if (!out_strides) return set_error(SI_ERR_INVALID, "null output strides");
  if (!out_idx && B > 0 && S > 0) return set_error(SI_ERR_INVALID, "null output pointer");
  if (out_strides[2] != 1) return set_error(SI_ERR_INVALID, "index rows must be contiguous");
  a.top_k = static_cast<int>(top_k);
  a.ratio = static_cast<int>(causal_ratio);
  a.out_idx = nullptr;
  a.out_scores = out_scores;
  a.out_idx32 = out_idx;
  a.o32sb = out_strides[0];
  a.o32ss = out_strides[1];
  a.n_win = static_cast<int>(n_win);
  a.idx_offset = static_cast<int>(idx_offset);
  if (a.B == 0 || a.S == 0) return SI_OK;
  return dispatch_shape<true>(a, static_cast<int>(D), static_cast<hipStream_t>(stream));
}

extern "C" int si_indexer_score(const void* q, const int64_t* q_strides, const void* k_idx,
                                const int64_t* k_strides, const void* weights, int w_dtype,
                                const int64_t* w_strides, int64_t B, int64_t S, int64_t T, int64_t H,
                                int64_t D, float* scores, const int64_t* score_strides, void* stream) {
  IndexerArgs a{};
  int rc = fill_common(a, q, q_strides, k_idx, k_strides, weights, w_dtype, w_strides, B, S, T, H, D);
  if (rc) return rc;
  if (!score_strides || (!scores && B > 0 && S > 0 && T > 0)) return set_error(SI_ERR_INVALID, "null score output");
  a.scores = scores;
  a.ssb = score_strides[0]; a.sss = score_strides[1]; a.sst = score_strides[2];
  if (a.B == 0 || a.S == 0 || a.T == 0) return SI_OK;
  return dispatch_shape<false>(a, static_cast<int>(D), static_cast<hipStream_t>(stream));
}
