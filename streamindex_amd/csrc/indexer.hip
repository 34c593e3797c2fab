// Lightning-indexer C-ABI entries: argument validation and shape dispatch.
// Kernels: indexer_kernels.h (instantiated per head dim in indexer_inst_d*.hip).
#include <string>

#include "indexer.h"
#include "si_status.h"

namespace si {

int g_topk_kernel_mode = 0;

// Kernel and selection capacity for a top-k shape.  A compaction keeps
// between top_k and C - 192 keys; the capacity leaves room for several
// 64-key offers.  The four-M-block kernel (HB 2 and 4, D = 128, long rows)
// runs one workgroup per CU and stalls the CU while a row compacts, so it
// takes the largest capacity its LDS holds: compactions become rarer.
// Capacity 1536 rather than 1024 above top_k = 192 in the two-workgroup
// kernel: fewer compactions, still two workgroups per CU (measured 1.4 %
// faster at S = 64K, k = 512).  Shapes past what one wave holds (more than
// 128 heads, or 64 at D = 256) or past the four-row LDS budget (top_k above
// 2048, or 1536 at D = 256) run the head-split kernel.
static int plan_topk(const IndexerArgs& a, int D, TopkPlan* p) {
  if (D != 32 && D != 64 && D != 128 && D != 256)
    return set_error(SI_ERR_UNSUPPORTED, "unsupported indexer head dim D_I=" + std::to_string(D) +
                                             " (supported: 32, 64, 128, 256)");
  const int HB = (a.H + 31) / 32;
  if (HB > 8) return set_error(SI_ERR_UNSUPPORTED, "H_I > 256 is not supported");
  if (a.top_k > 4096) return set_error(SI_ERR_UNSUPPORTED, "top_k > 4096 is not supported");
  const int hb_one_wave = D == 256 ? 2 : 4;
  const int k_four_rows = D == 256 ? 1536 : 2048;
  if (HB <= hb_one_wave && a.top_k <= k_four_rows) {
    p->hb = HB;
    p->hs = 1;
    if (D == 128 && (HB == 2 || HB == 4) && a.top_k <= 1152 && topk_wide_preferred(a)) {
      p->kernel = TOPK_WIDE;
      p->cap = a.top_k <= 192 ? 1024 : (HB == 4 ? 2048 : 1536);
      return SI_OK;
    }
    p->kernel = TOPK_NARROW;
    p->cap = a.top_k <= 32 ? 256 : a.top_k <= 192 ? 512 : a.top_k <= 1152 ? 1536 : a.top_k <= 1536 ? 2048 : 4096;
    return SI_OK;
  }
  p->kernel = TOPK_SPLIT;
  if (D == 256) {
    p->hs = HB <= 4 ? 2 : 4;
    p->hb = HB <= 2 ? 1 : 2;
  } else {
    p->hs = 2;
    p->hb = HB <= 2 ? 1 : (HB <= 4 ? 2 : 4);
  }
  p->cap = a.top_k <= 1152 ? 1536 : 4608;
  return SI_OK;
}

template <int HB, int D>
static int launch_planned(const IndexerArgs& a, const TopkPlan& p, hipStream_t st) {
  if (p.kernel == TOPK_WIDE) {
    if constexpr (topk_wide_fits<HB, D, 1024>()) {
      if (p.cap == 1024) return launch_topk_wide<HB, D, 1024>(a, st);
      if (p.cap == 1536) return launch_topk_wide<HB, D, 1536>(a, st);
      if (p.cap == 2048) return launch_topk_wide<HB, D, 2048>(a, st);
    }
    return set_error(SI_ERR_UNSUPPORTED, "no four-M-block kernel for this plan");
  }
  switch (p.cap) {
    case 256: return launch_topk<HB, D, 256>(a, st);
    case 512: return launch_topk<HB, D, 512>(a, st);
    case 1536: return launch_topk<HB, D, 1536>(a, st);
    case 2048: return launch_topk<HB, D, 2048>(a, st);
    case 4096: return launch_topk<HB, D, 4096>(a, st);
    default: return set_error(SI_ERR_UNSUPPORTED, "no top-k kernel for this capacity");
  }
}

template <int D>
static int launch_split_planned(const IndexerArgs& a, const TopkPlan& p, hipStream_t st) {
#define SI_SPLIT(HS_, HBH_, C_) \
  if (p.hs == HS_ && p.hb == HBH_ && p.cap == C_) return launch_topk_split<HS_, HBH_, D, C_>(a, st);
  if constexpr (D == 256) {
    SI_SPLIT(2, 1, 4608)
    SI_SPLIT(2, 2, 1536)
    SI_SPLIT(2, 2, 4608)
    SI_SPLIT(4, 2, 1536)
    SI_SPLIT(4, 2, 4608)
  } else {
    SI_SPLIT(2, 1, 4608)
    SI_SPLIT(2, 2, 4608)
    SI_SPLIT(2, 4, 1536)
    SI_SPLIT(2, 4, 4608)
  }
#undef SI_SPLIT
  return set_error(SI_ERR_UNSUPPORTED, "no head-split kernel for this plan");
}

static int dispatch_topk(const IndexerArgs& a, int D, hipStream_t st) {
  TopkPlan p{};
  const int rc = plan_topk(a, D, &p);
  if (rc) return rc;
  if (p.kernel == TOPK_SPLIT) {
    switch (D) {
      case 32: return launch_split_planned<32>(a, p, st);
      case 64: return launch_split_planned<64>(a, p, st);
      case 128: return launch_split_planned<128>(a, p, st);
      default: return launch_split_planned<256>(a, p, st);
    }
  }
#define SI_CASE(HB_, D_) \
  if (p.hb == HB_ && D == D_) return launch_planned<HB_, D_>(a, p, st);
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
  return set_error(SI_ERR_UNSUPPORTED, "no top-k kernel for this plan");
}

// Materialised scores.  A launch covers up to four 32-head blocks (two at
// D = 256); wider rows run one launch per head group, each after the first
// adding its part to the scores already written (the same stream orders them).
static int dispatch_score(const IndexerArgs& a0, int D, hipStream_t st) {
  if (D != 32 && D != 64 && D != 128 && D != 256)
    return set_error(SI_ERR_UNSUPPORTED, "unsupported indexer head dim D_I=" + std::to_string(D) +
                                             " (supported: 32, 64, 128, 256)");
  if (a0.H > 256) return set_error(SI_ERR_UNSUPPORTED, "H_I > 256 is not supported");
  const int group = D == 256 ? 64 : 128;
  for (int h0 = 0; h0 < a0.H; h0 += group) {
    IndexerArgs a = a0;
    a.q = a0.q + static_cast<int64_t>(h0) * a0.qsh;
    a.w = a0.w_bf16 ? static_cast<const void*>(reinterpret_cast<const uint16_t*>(a0.w) + h0 * a0.wsh)
                    : static_cast<const void*>(reinterpret_cast<const float*>(a0.w) + h0 * a0.wsh);
    a.H = a0.H - h0 < group ? a0.H - h0 : group;
    a.accumulate = h0 > 0;
    const int HB = (a.H + 31) / 32;
    int rc = -1;
#define SI_CASE(hb, d) \
  if (HB == hb && D == d) rc = launch_score<hb, d>(a, st);
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
    if (rc < 0) return set_error(SI_ERR_UNSUPPORTED, "no score kernel for this shape");
    if (rc) return rc;
  }
  return SI_OK;
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

extern "C" int si_indexer_topk_plan(int64_t S, int64_t T, int64_t H, int64_t D, int64_t top_k,
                                    int64_t causal_ratio, int32_t* kernel, int32_t* capacity) {
  if (S < 0 || T < 0 || H <= 0 || D <= 0 || top_k <= 0 || causal_ratio < 0) return set_error(SI_ERR_INVALID, "bad dimension");
  if (S > 0x7fffffff || T > 0x7fffffff || H > 0x7fffffff || top_k > 0x7fffffff || causal_ratio > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  IndexerArgs a{};
  a.B = 1;
  a.S = static_cast<int>(S);
  a.T = static_cast<int>(T);
  a.H = static_cast<int>(H);
  a.top_k = static_cast<int>(top_k);
  a.ratio = static_cast<int>(causal_ratio);
  TopkPlan p{};
  const int rc = plan_topk(a, static_cast<int>(D), &p);
  if (rc) return rc;
  if (kernel) *kernel = p.kernel;
  if (capacity) *capacity = p.cap;
  return SI_OK;
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
  return dispatch_topk(a, static_cast<int>(D), static_cast<hipStream_t>(stream));
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
  return dispatch_topk(a, static_cast<int>(D), static_cast<hipStream_t>(stream));
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
  return dispatch_score(a, static_cast<int>(D), static_cast<hipStream_t>(stream));
}
