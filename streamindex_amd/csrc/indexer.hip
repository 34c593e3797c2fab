// Lightning-indexer kernels for gfx950.
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
//     a double-buffered, XOR-swizzled LDS ring shared by the workgroup and
//     read as B-fragments with ds_read_b128.
//   * v_mfma_f32_32x32x16_bf16 produces a [32 heads x 32 keys] fp32 block per
//     M-block; lane l holds key l%32 and 16 heads, so ReLU and the fp32
//     weighted head sum happen in-lane, finished by one xor-32 exchange.
//   * The causal bound t < (s+1)//ratio is evaluated per lane in registers;
//     tiles past the workgroup's last legal key are never loaded or computed.
//   * The top-k kernel never writes scores: each lane offers its key to the
//     wave's streaming selection (wave_select.h); the score kernel stores the
//     fp32 row instead.
//   * Workgroups are issued heaviest-first (the last query block first) so the
//     triangular causal workload drains evenly over the 256 CUs.
#include <string>

#include "si_common.h"
#include "si_status.h"
#include "wave_select.h"

namespace si {

struct IndexerArgs {
  const uint16_t* q;  // [B,S,H,D] bf16, d contiguous
  int64_t qsb, qss, qsh;
  const uint16_t* k;  // [B,T,D] bf16, d contiguous
  int64_t ksb, kst;
  const void* w;      // [B,S,H] fp32 or bf16
  int64_t wsb, wss, wsh;
  int w_bf16;
  const uint8_t* mask;  // optional [B,S,T] bool (1 = legal)
  int64_t msb, mss, mst;
  int B, S, T, H;
  int top_k;
  int ratio;  // > 0: legal iff t < (s+1)/ratio; 0: no causal bound
  int64_t* out_idx;     // [B,S,top_k] contiguous
  float* out_scores;    // [B,S,top_k] contiguous
  float* scores;        // score kernel: [B,S,T]
  int64_t ssb, sss, sst;
};

// Byte offset of 16-byte chunk c of key row r inside a swizzled K tile.
// The XOR spreads the 16 rows read by one ds_read_b128 quarter-wave over
// distinct bank groups.
template <int D>
__device__ __forceinline__ int kt_off(int r, int c) {
  constexpr int CPR = D / 8;                      // 16-byte chunks per row
  constexpr int RPG = (16 / CPR) > 0 ? 16 / CPR : 1;  // rows per 256-byte bank sweep
  constexpr int SW = CPR < 16 ? CPR : 16;
  return r * (D * 2) + ((c ^ ((r / RPG) % SW)) << 4);
}

template <int D, int TILE_N, int NTHREADS>
struct KTileLoader {
  static constexpr int CPR = D / 8;
  static constexpr int CHUNKS = TILE_N * CPR;
  static constexpr int LPT = CHUNKS / NTHREADS;
  static_assert(CHUNKS % NTHREADS == 0, "tile must split evenly over the workgroup");
  u32x4 r[LPT];

  __device__ __forceinline__ void load(const uint16_t* kb, int64_t kst, int t0, int T) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int L = threadIdx.x + i * NTHREADS;
      const int row = L / CPR, c = L % CPR;
      const int t = t0 + row;
      if (t < T) {
        r[i] = *reinterpret_cast<const u32x4*>(kb + static_cast<int64_t>(t) * kst + c * 8);
      } else {
        r[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  __device__ __forceinline__ void store(char* tile) const {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int L = threadIdx.x + i * NTHREADS;
      const int row = L / CPR, c = L % CPR;
      *reinterpret_cast<u32x4*>(tile + kt_off<D>(row, c)) = r[i];
    }
  }
};

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

  // Score of key (t0 + lane%32) for this row; identical in lanes l and l+32.
  __device__ __forceinline__ float block_score(const char* tile, int nb, int lane) const {
    f32x16 acc[HB];
#pragma unroll
    for (int mb = 0; mb < HB; ++mb) acc[mb] = f32x16{};
    const int row = nb * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 kb =
          *reinterpret_cast<const bf16x8*>(tile + kt_off<D>(row, ks * 2 + (lane >> 5)));
#pragma unroll
      for (int mb = 0; mb < HB; ++mb) {
        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[mb][ks], kb, acc[mb], 0, 0, 0);
      }
    }
    float sum = 0.f;
#pragma unroll
    for (int mb = 0; mb < HB; ++mb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sum = __builtin_fmaf(wf[mb][v], __builtin_fmaxf(acc[mb][v], 0.f), sum);
    }
    return sum + shfl_xor_f32(sum, lane, 32);
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
// Fused score + streaming top-k.
// ---------------------------------------------------------------------------
template <int HB, int D, int KCAP, int NW, int TILE_N>
__global__ __launch_bounds__(NW * 64, 1) void indexer_topk_kernel(IndexerArgs a) {
  constexpr int NT = NW * 64;
  __shared__ __attribute__((aligned(16))) char ktile[2][TILE_N * D * 2];
  __shared__ uint64_t top_lds[NW][KCAP];
  __shared__ uint64_t cand_lds[NW][KCAP];

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

  WaveSelect<KCAP> sel;
  sel.init(top_lds[wave], cand_lds[wave], a.top_k, lane);

  const uint16_t* kb = a.k + b * a.ksb;
  const uint8_t* mrow =
      a.mask ? a.mask + b * a.msb + static_cast<int64_t>(active ? s : 0) * a.mss : nullptr;

  KTileLoader<D, TILE_N, NT> ld;
  const int ntiles = (wg_lim + TILE_N - 1) / TILE_N;
  if (ntiles > 0) {
    ld.load(kb, a.kst, 0, a.T);
    ld.store(ktile[0]);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const bool more = it + 1 < ntiles;
    if (more) ld.load(kb, a.kst, (it + 1) * TILE_N, a.T);
    const char* tile = ktile[it & 1];
    const int tbase = it * TILE_N;
#pragma unroll 1
    for (int nb = 0; nb < TILE_N / 32; ++nb) {
      const int t0 = tbase + nb * 32;
      if (t0 >= my_lim) break;
      const float score = qfr.block_score(tile, nb, lane);
      const int t = t0 + (lane & 31);
      bool legal = (lane < 32) && (t < my_lim);
      if (mrow != nullptr && legal) legal = mrow[static_cast<int64_t>(t) * a.mst] != 0;
      const uint64_t key = make_key(score, static_cast<uint32_t>(t));
      sel.offer(legal && key_hi(key) > sel.tau, key, lane);
    }
    if (more) ld.store(ktile[(it + 1) & 1]);
    __syncthreads();
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
  __shared__ __attribute__((aligned(16))) char ktile[2][TILE_N * D * 2];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nqb = (a.S + NW - 1) / NW;
  const int b = blockIdx.x % a.B;
  const int qb = static_cast<int>(blockIdx.x / a.B);
  const int s = qb * NW + wave;
  const bool active = s < a.S;

  QueryFrags<HB, D> qfr;
  if (active) qfr.load(a, b, s, lane);
  (void)nqb;

  const uint16_t* kb = a.k + b * a.ksb;
  float* orow = a.scores + b * a.ssb + static_cast<int64_t>(active ? s : 0) * a.sss;

  KTileLoader<D, TILE_N, NT> ld;
  const int ntiles = (a.T + TILE_N - 1) / TILE_N;
  if (ntiles > 0) {
    ld.load(kb, a.kst, 0, a.T);
    ld.store(ktile[0]);
  }
  __syncthreads();
  for (int it = 0; it < ntiles; ++it) {
    const bool more = it + 1 < ntiles;
    if (more) ld.load(kb, a.kst, (it + 1) * TILE_N, a.T);
    const char* tile = ktile[it & 1];
    if (active) {
#pragma unroll 1
      for (int nb = 0; nb < TILE_N / 32; ++nb) {
        const int t0 = it * TILE_N + nb * 32;
        if (t0 >= a.T) break;
        const float score = qfr.block_score(tile, nb, lane);
        const int t = t0 + (lane & 31);
        if (lane < 32 && t < a.T) orow[static_cast<int64_t>(t) * a.sst] = score;
      }
    }
    if (more) ld.store(ktile[(it + 1) & 1]);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------
template <int HB, int D, int KCAP>
static int launch_topk(const IndexerArgs& a, hipStream_t st) {
  constexpr int NW = KCAP <= 512 ? 8 : (KCAP <= 1024 ? 4 : 4);
  constexpr int TILE_N = KCAP <= 1024 ? 128 : 64;
  const int nqb = (a.S + NW - 1) / NW;
  const int64_t nblk = static_cast<int64_t>(nqb) * a.B;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((indexer_topk_kernel<HB, D, KCAP, NW, TILE_N>), dim3(static_cast<unsigned>(nblk)),
                     dim3(NW * 64), 0, st, a);
  return check_launch("indexer_topk_kernel");
}

template <int HB, int D>
static int dispatch_kcap(const IndexerArgs& a, hipStream_t st) {
  if (a.top_k <= 128) return launch_topk<HB, D, 128>(a, st);
  if (a.top_k <= 512) return launch_topk<HB, D, 512>(a, st);
  if (a.top_k <= 1024) return launch_topk<HB, D, 1024>(a, st);
  if (a.top_k <= 2048) return launch_topk<HB, D, 2048>(a, st);
  return set_error(SI_ERR_UNSUPPORTED, "top_k > 2048 is not supported");
}

template <int HB, int D>
static int launch_score(const IndexerArgs& a, hipStream_t st) {
  constexpr int NW = 8;
  constexpr int TILE_N = 128;
  const int nqb = (a.S + NW - 1) / NW;
  const int64_t nblk = static_cast<int64_t>(nqb) * a.B;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((indexer_score_kernel<HB, D, NW, TILE_N>), dim3(static_cast<unsigned>(nblk)),
                     dim3(NW * 64), 0, st, a);
  return check_launch("indexer_score_kernel");
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
  SI_CASE(2, 32)
  SI_CASE(2, 64)
  SI_CASE(2, 128)
#undef SI_CASE
  return set_error(SI_ERR_UNSUPPORTED,
                   "unsupported indexer shape: H_I=" + std::to_string(a.H) + " D_I=" + std::to_string(D) +
                       " (supported: H_I<=64, D_I in {32,64,128})");
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
