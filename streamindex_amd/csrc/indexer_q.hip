// Lightning indexer with quantised inputs for gfx950: fp4 (e2m1) queries with
// power-of-two (UE8M0) scales per 32 dims, fp8 (e4m3) keys with one fp32
// scale per key row, fused with the exact streaming top-k.
//
// The production V4 dtype policy (indexer queries fp4, compressed indexer
// keys fp8; docs/hyperparameters.yaml:38-44, docs/ir_analysis.md:36-43 of the
// reference) applied to the operator the reference implements in bf16:
//   * flash_sparse/triton/chunked_indexer.py:47-160 (chunked_indexer_topk),
//   * flash_sparse/reference.py:138-168             (score semantics).
// The scores are those of the dequantised inputs,
//   I(s, t) = sum_h w[s, h] relu(q[s, h, :] . k[t, :]),
//   q = e2m1 value * 2^e(s, h, d / 32),  k = e4m3 value * scale(t),
// and since scale(t) > 0, I(s, t) = scale(t) sum_h w relu(q . k_e4m3): the key
// scale multiplies the finished score.
//
// Design: one query row per wavefront, four or eight rows per workgroup
// (TopkQShape), 64-key tiles of fp8 rows (D bytes each) copied HBM/L2 -> LDS
// by global_load_lds into a double-buffered swizzled ring (the bf16 kernel's
// loader, a fp8 row of D bytes being laid out like a bf16 row of D/2
// elements).  One
// v_mfma_scale_f32_32x32x64_f8f6f4 per 32 heads x 32 keys x 64 dims: the A
// operand is the row's fp4 Q (16 bytes per lane, 32 consecutive dims) with
// its E8M0 block scale per lane, the B operand two 16-byte chunks of a key
// row per lane (dims 16 (l / 32) + 0..15 and 32 + 16 (l / 32) + 0..15 of the
// 64-dim step), which is the operand layout of that instruction on gfx950.
// Accumulators have the bf16 kernel's 32x32 layout, so its ReLU / weighted
// head-sum epilogue and the wave-level selection (wave_select.h) are reused.
#include <string>

#include "indexer.h"
#include "indexer_kernels.h"
#include "si_common.h"
#include "si_status.h"
#include "wave_select.h"

namespace si {

struct IndexerQArgs {
  const uint8_t* q;     // [B,S,H,D/2] packed e2m1, byte strides (last 1)
  int64_t qsb, qss, qsh;
  const float* qsc;     // [B,S,H,D/32] power-of-two scales
  int64_t qcsb, qcss, qcsh;
  const uint8_t* k;     // [B,T,D] e4m3, byte strides (last 1)
  int64_t ksb, kst;
  const float* ksc;     // [B,T] scale per key row
  int64_t kcsb, kcst;
  const void* w;        // [B,S,H] fp32 or bf16
  int64_t wsb, wss, wsh;
  int w_bf16;
  const uint8_t* mask;  // optional [B,S,T] bool
  int64_t msb, mss, mst;
  int B, S, T, H;
  int top_k;
  int ratio;
  int64_t* out_idx;     // [B,S,top_k], or null when out_idx32 is set
  float* out_scores;    // [B,S,top_k] or null
  // CSA index rows instead of out_idx (as IndexerArgs::out_idx32)
  int32_t* out_idx32;
  int64_t o32sb, o32ss;
  int n_win;
  int idx_offset;
};

typedef int v8i __attribute__((ext_vector_type(8)));

template <int HB, int D>
struct QuantQuery {
  static constexpr int KS = D / 64;  // 64-dim MFMA steps
  v8i qa[HB][KS];                    // fp4 A-fragments (upper 4 dwords unused)
  int qe[HB][KS];                    // E8M0 scale byte of the lane's 32-dim block
  float wf[HB][16];

  __device__ __forceinline__ void load(const IndexerQArgs& a, int b, int s, int lane) {
#pragma unroll
    for (int mb = 0; mb < HB; ++mb) {
      const int h = mb * 32 + (lane & 31);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        v8i v = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        int e = 127;
        if (h < a.H) {
          const uint8_t* qr = a.q + b * a.qsb + static_cast<int64_t>(s) * a.qss + static_cast<int64_t>(h) * a.qsh;
          const u32x4 d = *reinterpret_cast<const u32x4*>(qr + ks * 32 + (lane >> 5) * 16);
          v[0] = static_cast<int>(d[0]);
          v[1] = static_cast<int>(d[1]);
          v[2] = static_cast<int>(d[2]);
          v[3] = static_cast<int>(d[3]);
          const float sc = a.qsc[b * a.qcsb + static_cast<int64_t>(s) * a.qcss + static_cast<int64_t>(h) * a.qcsh +
                                 ks * 2 + (lane >> 5)];
          e = static_cast<int>((__float_as_uint(sc) >> 23) & 0xFFu);
        }
        qa[mb][ks] = v;
        qe[mb][ks] = e;
      }
#pragma unroll
      for (int vv = 0; vv < 16; ++vv) {
        const int hh = mb * 32 + 8 * (vv >> 2) + 4 * (lane >> 5) + (vv & 3);
        float wv = 0.f;
        if (hh < a.H) {
          const int64_t off = b * a.wsb + static_cast<int64_t>(s) * a.wss + hh * a.wsh;
          wv = a.w_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.w)[off])
                        : reinterpret_cast<const float*>(a.w)[off];
        }
        wf[mb][vv] = wv;
      }
    }
  }

  // Sum over this lane's 16 heads of every head block of one key block,
  // sum_h w_h relu(acc_h) (ReLU as one v_med3_f32), as two fma chains.
  __device__ __forceinline__ float epilogue2(const f32x16 (&acc)[HB]) const {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int mb = 0; mb < HB; ++mb)
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        s0 = __builtin_fmaf(wf[mb][v], __builtin_amdgcn_fmed3f(acc[mb][v], 0.f, __FLT_MAX__), s0);
        s1 = __builtin_fmaf(wf[mb][v + 1], __builtin_amdgcn_fmed3f(acc[mb][v + 1], 0.f, __FLT_MAX__), s1);
      }
    return s0 + s1;
  }

  __device__ __forceinline__ void load_b(const char* tile, int nb, int lane, v8i (&kb)[KS]) const {
    const int row = nb * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(tile + kt_off<D / 2>(row, ks * 4 + (lane >> 5)));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(tile + kt_off<D / 2>(row, ks * 4 + 2 + (lane >> 5)));
      kb[ks] = v8i{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                   static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
    }
  }

  // Partial scores (this lane's 16 heads per head block) of keys lane%32 of
  // blocks 0 and 1: the NB x HB accumulator chains are independent, so all
  // their MFMAs issue back to back before the first epilogue reads a result.
  template <int NBLK>
  __device__ __forceinline__ void tile_scores(const char* tile, int lane, float& p0, float& p1) const {
    v8i kb[NBLK][KS];
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) load_b(tile, nb, lane, kb[nb]);
    f32x16 acc[NBLK][HB];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
        for (int mb = 0; mb < HB; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa[mb][ks], kb[nb][ks],
                                                                         ks == 0 ? f32x16{} : acc[nb][mb], 4, 0, 0,
                                                                         qe[mb][ks], 0, 127);
    // Two fma chains per key block run through all head blocks and are added
    // once (one add per key block instead of one per head block and one per
    // combination).
    p0 = epilogue2(acc[0]);
    p1 = 0.f;
    if constexpr (NBLK > 1) p1 = epilogue2(acc[1]);
  }
};

// Launch shape: as the bf16 kernel (64-key tiles, one query row per wave)
// with more waves per SIMD, which the fp8 ring (half the bf16 one) and the
// smaller fragments allow.  Up to C = 960 (top_k <= 512) a workgroup takes
// eight rows that share one K ring, and two such workgroups fill a CU: four
// waves per SIMD at 128 VGPRs, at most 2 x 76.5 KiB of LDS (960 keys is the
// largest selection buffer that leaves two).  Above, four rows per workgroup
// and three workgroups per CU while the selection buffers leave room in LDS.
template <int C>
struct TopkQShape {
  static constexpr int NW = C <= 960 ? 8 : 4;
  static constexpr int WAVES_PER_EU = NW == 8 ? 4 : (C <= 1152 ? 3 : 1);
};

template <int HB, int D, int C, bool MASKED>
__global__ __launch_bounds__(TopkQShape<C>::NW * 64)
__attribute__((amdgpu_waves_per_eu(TopkQShape<C>::WAVES_PER_EU, TopkQShape<C>::WAVES_PER_EU)))
void indexer_topk_q_kernel(IndexerQArgs a) {
  constexpr int NW = TopkQShape<C>::NW;
  constexpr int NT = NW * 64;
  constexpr int TILE_N = TopkShape<C>::TILE_N;
  constexpr int NB = TILE_N / 32;
  static_assert(NB == 2, "one 64-key offer per tile");
  constexpr int TILE_BYTES = TILE_N * D;  // fp8 rows
  constexpr int RING = 2;
  // K ring, selection buffers, then the key scales of the ring's tiles.
  __shared__ __attribute__((aligned(16))) char lds[RING * TILE_BYTES + NW * C * 8 + RING * TILE_N * 4];
  uint64_t* const sel_base = reinterpret_cast<uint64_t*>(lds + RING * TILE_BYTES);
  float* const ksc_lds = reinterpret_cast<float*>(lds + RING * TILE_BYTES + NW * C * 8);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nqb = (a.S + NW - 1) / NW;
  const int b = blockIdx.x % a.B;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x / a.B);  // heaviest first
  const int s0 = qb * NW;
  const int s = s0 + wave;
  const bool active = s < a.S;
  const int s_last = (s0 + NW < a.S ? s0 + NW : a.S) - 1;
  auto limit = [&](int r) {
    if (a.ratio > 0) {
      const int l = (r + 1) / a.ratio;
      return l < a.T ? l : a.T;
    }
    return a.T;
  };
  const int my_lim = active ? limit(s) : 0;
  const int wg_lim = limit(s_last);

  QuantQuery<HB, D> qry;
  if (active) qry.load(a, b, s, lane);

  const int oblk = static_cast<int>(permlane32_swap(0u, 1u).x);
  const int okey = oblk * 32 + (lane & 31);
  const int lim_o = my_lim - okey;                        // the key of a tile is legal iff tbase < lim_o
  const uint32_t nokey = ~static_cast<uint32_t>(okey);    // ~(tbase + okey) == nokey - tbase

  WaveSelect<C> sel;
  sel.init(sel_base + wave * C, a.top_k);

  const uint16_t* kb16 = reinterpret_cast<const uint16_t*>(a.k + b * a.ksb);
  const float* kscb = a.ksc + b * a.kcsb;
  const uint8_t* mrow =
      MASKED ? a.mask + b * a.msb + static_cast<int64_t>(active ? s : 0) * a.mss : nullptr;
  // the loader addresses fp8 rows as bf16 rows of D/2 elements (byte stride / 2)
  const int64_t kst16 = a.kst / 2;
  KTileLoader<D / 2, TILE_N, NT> ld;
  ld.init(kst16);
  const int ntiles = (wg_lim + TILE_N - 1) / TILE_N;
  // The 64 key scales of tile t go to ksc_lds[t % 2] with one 4-byte
  // global_load_lds by wave t % NW (every row of the workgroup reads the same
  // scales, and the issuing wave rotates so no SIMD does all the address
  // work); keys past T (only in the tile that crosses T) read the last key's.
  // Per-lane element offsets from the tile's first key: lane for a tile
  // inside [0, T), clamped to T - 1 for the one tile that crosses T.
  const int tcross = a.T / TILE_N;
  const int64_t koff_l = static_cast<int64_t>(lane) * a.kcst;
  const int64_t koff_c =
      static_cast<int64_t>(tcross * TILE_N + lane < a.T ? lane : a.T - 1 - tcross * TILE_N) * a.kcst;
  auto issue_scales = [&](int t) {
    if (wave != (t & (NW - 1))) return;
    const float* base = kscb + static_cast<int64_t>(t) * TILE_N * a.kcst;
    const int64_t off = t == tcross ? koff_c : koff_l;
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(base + off),
                                     (lds_void*)(ksc_lds + (t & 1) * TILE_N), 4, 0, 0);
  };
  if (ntiles > 0) {
    ld.issue(kb16, kst16, 0, a.T, lds);
    issue_scales(0);
  }
  wait_vm_lgkm0<0>();
  __syncthreads();
  // One tile; SLOT (the ring slot of tile it) is a compile-time constant, so
  // every LDS address of the tile is a per-lane base plus an immediate.
  auto tile_step = [&](const int it, auto SLOTC) {
    constexpr int slot = decltype(SLOTC)::value;
    const int tbase = it * TILE_N;
    const int t = tbase + okey;  // (t < my_lim is tbase < lim_o; ~t is nokey - tbase)
    // the key's scale (LDS, before the copies below so it does not wait for
    // them) and mask byte first
    const float kscale = ksc_lds[slot * TILE_N + okey];
    bool mok = true;
    if constexpr (MASKED) mok = t < my_lim ? mrow[static_cast<int64_t>(t) * a.mst] != 0 : false;
    const bool more = it + 1 < ntiles;
    if (more) {
      ld.issue(kb16, kst16, (it + 1) * TILE_N, a.T, lds + (1 - slot) * TILE_BYTES);
      issue_scales(it + 1);
    }
    const char* tile = lds + slot * TILE_BYTES;
    int nblk = (my_lim - tbase + 31) / 32;
    nblk = nblk > NB ? NB : (nblk < 0 ? 0 : nblk);
    if (nblk > 0) {
      float p0, p1;
      if (nblk == NB) qry.template tile_scores<2>(tile, lane, p0, p1);
      else qry.template tile_scores<1>(tile, lane, p0, p1);
      const SwapPair r = permlane32_swap(__float_as_uint(p0), __float_as_uint(p1));
      const float sum = (__uint_as_float(r.x) + __uint_as_float(r.y)) * kscale;
      const uint64_t key = make_key_inv(sum, nokey - static_cast<uint32_t>(tbase));
      uint64_t bal = __builtin_amdgcn_ballot_w64(tbase < lim_o) & __builtin_amdgcn_ballot_w64(key_hi(key) > sel.tau);
      if constexpr (MASKED) bal &= __builtin_amdgcn_ballot_w64(mok);
      sel.offer64_masked(bal, key);
      if (sel.needs_compaction()) sel.template compact<WaveSelect<C>::NEEDS_MIN>(lane);
    }
    if (more) wait_vm_lgkm0<0>();
    __syncthreads();
  };
  static_assert(RING == 2, "the tile loop is unrolled over the two ring slots");
  int it = 0;
  for (; it + 1 < ntiles; it += 2) {
    tile_step(it, std::integral_constant<int, 0>{});
    tile_step(it + 1, std::integral_constant<int, 1>{});
  }
  if (it < ntiles) tile_step(it, std::integral_constant<int, 0>{});

  if (active) {
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

template <int HB, int D, int C>
static int launch_q(const IndexerQArgs& a, hipStream_t st) {
  if (a.top_k > WaveSelect<C>::MAX_TOPK) return set_error(SI_ERR_UNSUPPORTED, "top_k exceeds the selection capacity");
  constexpr int NW = TopkQShape<C>::NW;
  const int64_t nqb = (static_cast<int64_t>(a.S) + NW - 1) / NW;
  const int64_t grid = nqb * a.B;
  if (grid > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  if (grid == 0) return SI_OK;
  if (a.mask)
    hipLaunchKernelGGL((indexer_topk_q_kernel<HB, D, C, true>), dim3(static_cast<unsigned>(grid)), dim3(NW * 64), 0,
                       st, a);
  else
    hipLaunchKernelGGL((indexer_topk_q_kernel<HB, D, C, false>), dim3(static_cast<unsigned>(grid)), dim3(NW * 64), 0,
                       st, a);
  return check_launch("indexer_topk_q_kernel");
}

template <int HB, int D>
static int dispatch_q(const IndexerQArgs& a, hipStream_t st) {
  // (eight rows per workgroup, four waves per SIMD, against four rows and three
  // workgroups per CU: top_k 32 -4.5 % at 64K; 128 -3.8 % at 64K, -4.3 % at
  // S = 1M; 512 (C = 960 against C = 1152) -3.8 % at 1M and even at 64K,
  // where C = 896 cost 1 % in compactions)
  if (a.top_k <= 32) return launch_q<HB, D, 256>(a, st);
  if (a.top_k <= 192) return launch_q<HB, D, 512>(a, st);
  if (a.top_k <= 512) return launch_q<HB, D, 960>(a, st);
  // (1152 = the most that leaves three workgroups per CU: 52 KiB of LDS each;
  // fewer compactions than 1024, measured -1.3 % at S = 64K)
  if (a.top_k <= 640) return launch_q<HB, D, 1152>(a, st);
  if (a.top_k <= 1536) return launch_q<HB, D, 2048>(a, st);
  if (a.top_k <= 2048) return launch_q<HB, D, 4096>(a, st);
  return set_error(SI_ERR_UNSUPPORTED, "top_k > 2048 is not supported");
}

// Argument checks and the packed-argument fill shared by both entries.
static int fill_q(IndexerQArgs& a, const void* q_fp4, const int64_t* q_strides, const float* q_scale,
                  const int64_t* q_scale_strides, const void* k_fp8, const int64_t* k_strides, const float* k_scale,
                  const int64_t* k_scale_strides, const void* weights, int w_dtype, const int64_t* w_strides,
                  int64_t B, int64_t S, int64_t T, int64_t H, int64_t D, int64_t top_k, int64_t causal_ratio) {
  if (!q_strides || !q_scale_strides || !k_strides || !k_scale_strides || !w_strides)
    return set_error(SI_ERR_INVALID, "null stride argument");
  if (B < 0 || S < 0 || T < 0 || H <= 0 || D <= 0) return set_error(SI_ERR_INVALID, "negative or zero dimension");
  if (top_k <= 0) return set_error(SI_ERR_INVALID, "top_k must be positive");
  if (top_k > 2048) return set_error(SI_ERR_UNSUPPORTED, "top_k > 2048 is not supported");
  if (causal_ratio < 0 || causal_ratio > 0x7fffffff) return set_error(SI_ERR_INVALID, "bad causal_ratio");
  if (B > 0x7fffffff || S > 0x7fffffff || T > 0x7fffffff) return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (H > 64 || D != 128)
    return set_error(SI_ERR_UNSUPPORTED, "quantised indexer supports H_I <= 64 and D_I = 128 (the V4 indexer)");
  const bool rows = B > 0 && S > 0;
  if (rows && (!q_fp4 || !q_scale || !weights)) return set_error(SI_ERR_INVALID, "null pointer argument");
  if (B > 0 && T > 0 && (!k_fp8 || !k_scale)) return set_error(SI_ERR_INVALID, "null pointer argument");
  if (q_strides[3] != 1 || k_strides[2] != 1 || q_scale_strides[3] != 1)
    return set_error(SI_ERR_INVALID, "q, q_scale and k need a contiguous last dimension");
  if ((q_strides[0] | q_strides[1] | q_strides[2] | k_strides[0] | k_strides[1]) % 16)
    return set_error(SI_ERR_INVALID, "q / k byte strides must be multiples of 16");
  if ((reinterpret_cast<uintptr_t>(q_fp4) | reinterpret_cast<uintptr_t>(k_fp8)) & 15)
    return set_error(SI_ERR_INVALID, "q / k must be 16-byte aligned");
  if (k_strides[1] >= (int64_t{1} << 24)) return set_error(SI_ERR_UNSUPPORTED, "k row stride too large");
  if (w_dtype != 0 && w_dtype != 1) return set_error(SI_ERR_INVALID, "weights dtype must be fp32 (0) or bf16 (1)");
  a.q = static_cast<const uint8_t*>(q_fp4);
  a.qsb = q_strides[0]; a.qss = q_strides[1]; a.qsh = q_strides[2];
  a.qsc = q_scale;
  a.qcsb = q_scale_strides[0]; a.qcss = q_scale_strides[1]; a.qcsh = q_scale_strides[2];
  a.k = static_cast<const uint8_t*>(k_fp8);
  a.ksb = k_strides[0]; a.kst = k_strides[1];
  a.ksc = k_scale;
  a.kcsb = k_scale_strides[0]; a.kcst = k_scale_strides[1];
  a.w = weights;
  a.wsb = w_strides[0]; a.wss = w_strides[1]; a.wsh = w_strides[2];
  a.w_bf16 = w_dtype;
  a.B = static_cast<int>(B); a.S = static_cast<int>(S); a.T = static_cast<int>(T); a.H = static_cast<int>(H);
  a.top_k = static_cast<int>(top_k);
  a.ratio = static_cast<int>(causal_ratio);
  return SI_OK;
}

static int run_q(const IndexerQArgs& a, void* stream) {
  if (a.B == 0 || a.S == 0) return SI_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return a.H <= 32 ? dispatch_q<1, 128>(a, st) : dispatch_q<2, 128>(a, st);
}

}  // namespace si

using namespace si;

extern "C" int si_indexer_topk_q(const void* q_fp4, const int64_t* q_strides, const float* q_scale,
                                 const int64_t* q_scale_strides, const void* k_fp8, const int64_t* k_strides,
                                 const float* k_scale, const int64_t* k_scale_strides, const void* weights,
                                 int w_dtype, const int64_t* w_strides, const uint8_t* causal_mask,
                                 const int64_t* mask_strides, int64_t B, int64_t S, int64_t T, int64_t H, int64_t D,
                                 int64_t top_k, int64_t causal_ratio, int64_t* out_idx, float* out_scores,
                                 void* stream) {
  IndexerQArgs a{};
  int rc = fill_q(a, q_fp4, q_strides, q_scale, q_scale_strides, k_fp8, k_strides, k_scale, k_scale_strides, weights,
                  w_dtype, w_strides, B, S, T, H, D, top_k, causal_ratio);
  if (rc) return rc;
  if (causal_mask && causal_ratio > 0) return set_error(SI_ERR_INVALID, "causal_mask and causal_ratio are exclusive");
  if (causal_mask && !mask_strides) return set_error(SI_ERR_INVALID, "null mask strides");
  if (B > 0 && S > 0 && !out_idx) return set_error(SI_ERR_INVALID, "null output pointer");
  a.mask = causal_mask;
  if (causal_mask) {
    a.msb = mask_strides[0]; a.mss = mask_strides[1]; a.mst = mask_strides[2];
  }
  a.out_idx = out_idx;
  a.out_scores = out_scores;
  return run_q(a, stream);
}

extern "C" int si_csa_indexer_topk_q(const void* q_fp4, const int64_t* q_strides, const float* q_scale,
                                     const int64_t* q_scale_strides, const void* k_fp8, const int64_t* k_strides,
                                     const float* k_scale, const int64_t* k_scale_strides, const void* weights,
                                     int w_dtype, const int64_t* w_strides, int64_t B, int64_t S, int64_t T,
                                     int64_t H, int64_t D, int64_t top_k, int64_t causal_ratio, int64_t n_win,
                                     int64_t idx_offset, int32_t* out_idx, const int64_t* out_strides,
                                     float* out_scores, void* stream) {
  IndexerQArgs a{};
  int rc = fill_q(a, q_fp4, q_strides, q_scale, q_scale_strides, k_fp8, k_strides, k_scale, k_scale_strides, weights,
                  w_dtype, w_strides, B, S, T, H, D, top_k, causal_ratio);
  if (rc) return rc;
  if (n_win < 0 || n_win > 0x7fffffff) return set_error(SI_ERR_INVALID, "n_win must be non-negative");
  if (idx_offset < 0 || idx_offset + T > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "idx_offset + T must fit in int32");
  if (!out_strides) return set_error(SI_ERR_INVALID, "null output strides");
  if (!out_idx && B > 0 && S > 0) return set_error(SI_ERR_INVALID, "null output pointer");
  if (out_strides[2] != 1) return set_error(SI_ERR_INVALID, "index rows must be contiguous");
  a.out_scores = out_scores;
  a.out_idx32 = out_idx;
  a.o32sb = out_strides[0];
  a.o32ss = out_strides[1];
  a.n_win = static_cast<int>(n_win);
  a.idx_offset = static_cast<int>(idx_offset);
  return run_q(a, stream);
}
