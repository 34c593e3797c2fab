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
//     the M axis), loaded once.  K tiles are copied HBM/L2 -> LDS by
//     global_load_lds into a double-buffered, XOR-swizzled ring shared by the
//     workgroup; tile i+1 is in flight while tile i is consumed.
//   * v_mfma_f32_32x32x16_bf16 produces [32 heads x 32 keys] per M-block
//     ("group"); lane l holds key l%32 for 16 heads, so ReLU (v_med3) and the
//     fp32 weighted head sum are in-lane.
//   * Top-k kernel: the groups of a tile are software-pipelined.  Group g's
//     MFMAs accumulate into one of two accumulator sets while the epilogue of
//     group g-1 (ReLU + weighted sum) reads the other, and the next 32-key
//     block's B-fragments are read from LDS behind the MFMAs that consume the
//     current ones.  The two half-wave partial sums of a 64-key tile are
//     combined with one v_permlane32_swap and the tile's 64 keys are offered
//     to the wave's selection buffer (wave_select.h) in one branch-free
//     append, overlapped with the next tile's first MFMAs.
//   * The causal bound t < (s+1)//ratio is evaluated per lane in registers;
//     32-key blocks past a row's bound are skipped and tiles past the
//     workgroup's last legal key are never loaded.
//   * Workgroups are issued heaviest-first (the last query block first) so the
//     triangular causal workload drains evenly; two workgroups share a CU so
//     one's barriers, compactions and final sort overlap the other's MFMAs.
#pragma once

#include "indexer.h"
#include "si_common.h"
#include "si_status.h"
#include "wave_select.h"

#include <type_traits>

namespace si {

// Byte offset of 16-byte chunk c of key row r inside a swizzled K tile.
// The XOR spreads the 16 rows read by one ds_read_b128 quarter-wave over
// distinct bank groups.  The pattern repeats every 16 rows.
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
// fetches the global chunk that belongs in its slot under the swizzle.  The
// lane's byte offsets from the tile's first key row are computed once, so a
// tile inside [0, T) costs one scalar base per tile; a tile that crosses T
// re-reads row T-1 for its missing rows (those keys are never legal).
// Needs TILE_N * k_row_stride * 2 < 2^31 (checked on the host).
template <int D, int TILE_N, int NTHREADS>
struct KTileLoader {
  static constexpr int CPR = D / 8;
  static constexpr int CHUNKS = TILE_N * CPR;
  static constexpr int LPT = CHUNKS / NTHREADS;
  static_assert(CHUNKS % NTHREADS == 0, "tile must split evenly over the workgroup");
  uint32_t voff[LPT];

  __device__ __forceinline__ static void slot_of(int i, int& slot0, int& row, int& c) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    slot0 = i * NTHREADS + wave * 64;
    const int slot = slot0 + lane;
    row = slot / CPR;
    c = (slot % CPR) ^ ((kt_off<D>(row, 0) >> 4) - row * CPR);
  }

  __device__ __forceinline__ void init(int64_t kst) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      int slot0, row, c;
      slot_of(i, slot0, row, c);
      voff[i] = static_cast<uint32_t>(row * kst * 2 + c * 16);
    }
  }

  // Copy i (0 <= i < LPT) of a tile that lies inside [0, T), whose first
  // key row starts at `src`.
  __device__ __forceinline__ void issue_at(const char* src, char* tile, int i) const {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot0 = i * NTHREADS + wave * 64;
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint16_t*>(src + voff[i]), (lds_void*)(tile + slot0 * 16),
                                     16, 0, 0);
  }

  __device__ __forceinline__ void issue(const uint16_t* kb, int64_t kst, int t0, int T, char* tile) const {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (t0 + TILE_N <= T) {
      // (The source pointer is passed as uint16_t*: a char* argument to this
      // builtin makes clang drop the host launch stubs of later instantiations.)
      const char* base = reinterpret_cast<const char*>(kb + static_cast<int64_t>(t0) * kst);
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const int slot0 = i * NTHREADS + wave * 64;
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint16_t*>(base + voff[i]),
                                         (lds_void*)(tile + slot0 * 16), 16, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        int slot0, row, c;
        slot_of(i, slot0, row, c);
        int t = t0 + row;
        t = t < T ? t : T - 1;
        __builtin_amdgcn_global_load_lds(kb + static_cast<int64_t>(t) * kst + c * 8,
                                         (lds_void*)(tile + slot0 * 16), 16, 0, 0);
      }
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

  // Sum over this lane's 16 heads of M-block mb: sum_v w_v * relu(acc_v).
  __device__ __forceinline__ float epilogue(const f32x16& acc, int mb) const {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      // relu as a single v_med3_f32 (clamp to [0, FLT_MAX])
      s0 = __builtin_fmaf(wf[mb][v], __builtin_amdgcn_fmed3f(acc[v], 0.f, __FLT_MAX__), s0);
      s1 = __builtin_fmaf(wf[mb][v + 1], __builtin_amdgcn_fmed3f(acc[v + 1], 0.f, __FLT_MAX__), s1);
    }
    return s0 + s1;
  }

  // This lane's half of the head sum of one 32-key block (key lane % 32,
  // the lane's 16 heads per head block); the two halves are added across the
  // half-waves by the caller.
  __device__ __forceinline__ float partial(const bf16x8 (&kb)[KS]) const {
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
    for (int mb = 0; mb < HB; ++mb) sum += epilogue(acc[mb], mb);
    return sum;
  }

  // Partial head sums (partial()) of the first `nblk` 32-key blocks of a tile
  // (all NB when FULL, 0 for the others).  One set of B-fragments at a time:
  // a second set (reads of block nb+1 behind block nb's MFMAs) needs the 32
  // registers whose spills, reloaded from scratch every tile, made each tile
  // wait for the next tile's copy (vector memory completes in order); the
  // other wave of the SIMD covers the LDS latency instead.
  template <int NB, bool FULL>
  __device__ __forceinline__ void tile_partials(const char* tile, int nblk, int lane, float (&p)[NB]) const {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (FULL || nb < nblk) {
        bf16x8 kb[KS];
        load_b(tile, nb, lane, kb);
        p[nb] = partial(kb);
      } else {
        p[nb] = 0.f;
      }
    }
  }
};

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1 (compile-time loop).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_impl(F& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_impl<I + 1, N>(f);
  }
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<0, N>(f);
}

// Sliding-window columns of query s: column j holds key s - n_win + 1 + j,
// or -1 where that is negative (flash_sparse/reference.py:460-475).
__device__ __forceinline__ void write_window_cols(int32_t* orow, int s, int n_win, int lane) {
  for (int j = lane; j < n_win; j += kWave) {
    const int t = s - n_win + 1 + j;
    orow[j] = t >= 0 ? t : -1;
  }
}

__device__ __forceinline__ int legal_limit(const IndexerArgs& a, int s) {
  if (a.ratio > 0) {
    const int l = (s + 1) / a.ratio;
    return l < a.T ? l : a.T;
  }
  return a.T;
}

// Launch shape of the top-k kernel per selection capacity C: four rows per
// workgroup and 64-key tiles.  Up to C = 1536 a workgroup needs at most
// 2*16 KiB (ring) + 4*12 KiB (selection) = 80 KiB of LDS and 256 VGPRs per
// wave, so two workgroups share a CU; wider capacities run one per CU.
template <int C>
struct TopkShape {
  static constexpr int NW = 4;
  static constexpr int TILE_N = 64;
  static constexpr int WAVES_PER_EU = C <= 1536 ? 2 : 1;  // for one or two 32-head blocks at D <= 128
  // K tiles in the LDS ring: tile i+1 is copied while tile i is consumed (a
  // third buffer measured no faster at S = 64K).
  static constexpr int RING = 2;
};

// Workgroups per CU of the bf16 top-k kernel.  Up to two 32-head blocks at
// D <= 128 a row's Q fragments, head weights and pipelined accumulators fit
// 256 VGPRs, so two workgroups share a CU (up to C = 1536); wider query rows
// (H > 64 or D = 256) hold twice the registers and run one workgroup per CU.
template <int HB, int D, int C>
constexpr int topk_waves_per_eu() {
  return (HB <= 2 && D <= 128) ? TopkShape<C>::WAVES_PER_EU : 1;
}

// Whether the K ring and the selection buffers of a (D, C) instance fit the
// LDS share of one workgroup.
template <int HB, int D, int C>
constexpr bool topk_fits_lds() {
  return TopkShape<C>::RING * TopkShape<C>::TILE_N * D * 2 + TopkShape<C>::NW * C * 8 <=
         160 * 1024 / topk_waves_per_eu<HB, D, C>();
}

// s_waitcnt with vmcnt = n (0..15), lgkmcnt = 0, expcnt not waited (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4));
}

// ---------------------------------------------------------------------------
// Fused score + streaming exact top-k.
// ---------------------------------------------------------------------------
template <int HB, int D, int C, bool MASKED>
__global__ __launch_bounds__(TopkShape<C>::NW * 64)
__attribute__((amdgpu_waves_per_eu(topk_waves_per_eu<HB, D, C>(), topk_waves_per_eu<HB, D, C>())))
void indexer_topk_kernel(IndexerArgs a) {
  constexpr int NW = TopkShape<C>::NW;
  constexpr int NT = NW * 64;
  constexpr int TILE_N = TopkShape<C>::TILE_N;
  constexpr int NB = TILE_N / 32;  // 32-key blocks per tile
  static_assert(NB == 2, "one 64-key offer per tile");
  constexpr int KS = D / 16;       // MFMA k-steps per 32-key block
  constexpr int G = NB * HB;       // MFMA groups per tile (even)
  constexpr int TILE_BYTES = TILE_N * D * 2;
  constexpr int BLK_BYTES = 32 * D * 2;
  constexpr int RING = TopkShape<C>::RING;
  // The DMA-filled K ring sits first (global_load_lds destinations stay
  // below 64 KiB), then the per-wave selection buffers.
  // Compaction requests of the waves (double-buffered by tile parity) are
  // posted before each tile barrier, where LDS has room for them.
  constexpr int SEL_END = RING * TILE_BYTES + NW * C * 8;
  // LDS per workgroup so that WAVES_PER_EU workgroups share a CU's 160 KiB.
  constexpr int LDS_BUDGET = 160 * 1024 / topk_waves_per_eu<HB, D, C>();
  constexpr bool SHARE_COMP = SEL_END + 2 * NW * 4 <= LDS_BUDGET;
  static_assert(SEL_END <= LDS_BUDGET, "ring + selection buffers exceed the LDS share");
  __shared__ __attribute__((aligned(16))) char lds[SEL_END + (SHARE_COMP ? 2 * NW * 4 : 0)];
  uint64_t* const sel_base = reinterpret_cast<uint64_t*>(lds + RING * TILE_BYTES);
  int* const comp_req = reinterpret_cast<int*>(lds + SEL_END);
  static_assert(NW == 4, "the requests of a tile are read as one int4");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

  // Per-lane B-fragment offsets of block 0 (block 1 is BLK_BYTES further on:
  // the swizzle repeats every 16 rows).
  int boff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) boff[ks] = kt_off<D>(lane & 31, ks * 2 + (lane >> 5));

  // Which 32-key block of a tile this lane offers after the half-wave swap.
  const int oblk = static_cast<int>(permlane32_swap(0u, 1u).x);
  const int okey = oblk * 32 + (lane & 31);

  WaveSelect<C> sel;
  sel.init(sel_base + wave * C, a.top_k);

  const uint16_t* kb = a.k + b * a.ksb;
  const uint8_t* mrow =
      MASKED ? a.mask + b * a.msb + static_cast<int64_t>(active ? s : 0) * a.mss : nullptr;

  KTileLoader<D, TILE_N, NT> ld;
  ld.init(a.kst);
  const int ntiles = (wg_lim + TILE_N - 1) / TILE_N;
  if (ntiles > 0) ld.issue(kb, a.kst, 0, a.T, lds);

  // Pipeline state carried across tiles.  Each of the G groups of a tile has
  // its own accumulator; the epilogue runs LAG = HB groups behind the MFMAs,
  // so it never waits on the chain that was just issued.  At a tile boundary
  // the previous tile's block-1 groups (acc[HB..G-1]) are still pending,
  // together with the half-wave partial sum of its block 0.
  constexpr int LAG = HB;
  f32x16 acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = f32x16{};
  float prev_p0 = 0.f;
  int prev_tbase = 0;
  bool pend = false;
  bool prev_mask = true, cur_mask = true;

  auto offer_tile = [&](float p0, float p1, int tbase, bool valid, bool mok) {
    const SwapPair r = permlane32_swap(__float_as_uint(p0), __float_as_uint(p1));
    const float sum = __uint_as_float(r.x) + __uint_as_float(r.y);
    const int t = tbase + okey;
    const uint64_t key = make_key(sum, static_cast<uint32_t>(t));
    uint64_t bal = __builtin_amdgcn_ballot_w64(t < my_lim) & __builtin_amdgcn_ballot_w64(key_hi(key) > sel.tau);
    if constexpr (MASKED) bal &= __builtin_amdgcn_ballot_w64(mok);
    sel.offer64_bal(valid ? bal : 0ull, key, lane);
  };
  // Epilogues of the pending block-1 groups of the previous tile, then its offer.
  auto drain = [&]() {
    float p1 = 0.f;
#pragma unroll
    for (int mb = 0; mb < HB; ++mb) p1 += qfr.epilogue(acc[HB + mb], mb);
    offer_tile(prev_p0, p1, prev_tbase, true, prev_mask);
  };

  // Tile 0 landed.
  wait_vm_lgkm0<0>();
  __syncthreads();

  static_assert(RING == 2, "the tile loop is unrolled over the two ring slots");
  // One tile; SLOT (the ring slot of tile `it`, it % 2) is a compile-time
  // constant, so every LDS address of the tile is a per-lane base plus an
  // immediate offset.
  auto tile_step = [&](const int it, auto SLOTC) {
    constexpr int slot = decltype(SLOTC)::value;
    constexpr int fill = 1 - slot;
    const int tbase = it * TILE_N;
    if constexpr (MASKED) {  // issued before the tile copies so the waits below cover only the copies
      const int t = tbase + okey;
      cur_mask = t < my_lim ? mrow[static_cast<int64_t>(t) * a.mst] != 0 : false;
    }
    const bool more = it + 1 < ntiles;
    const char* tile = lds + slot * TILE_BYTES;
    int nblk = (my_lim - tbase + 31) / 32;
    nblk = nblk > NB ? NB : (nblk < 0 ? 0 : nblk);
    // The B-fragment reads of a full tile's first block go out first: the
    // compaction-request read and the next tile's copies overlap them, so the
    // tile waits for one LDS round trip before its MFMAs.
    bf16x8 kf[KS];
    if (nblk == NB) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const bf16x8*>(tile + boff[ks]);
    }
    int4 rq = int4{0, 0, 0, 0};
    if (SHARE_COMP && it > 0) rq = *reinterpret_cast<const int4*>(comp_req + ((it - 1) & 1) * NW);
    // The slot of tile it+1 last held tile it-1, which every wave finished
    // before the barrier that ended the previous tile.
    if (more) ld.issue(kb, a.kst, (it + 1) * TILE_N, a.T, lds + fill * TILE_BYTES);
    // A compaction that some row asked for at the previous barrier runs now
    // in every row that is close to needing one, so that the workgroup waits
    // once for all of them instead of once per row.
    if (SHARE_COMP && (rq.x | rq.y | rq.z | rq.w) && sel.wants_compaction()) sel.compact(lane);

    if (nblk == NB) {
      // ---- full tile: software-pipelined groups ---------------------------
      __builtin_amdgcn_sched_barrier(0);  // all block-0 reads in flight before the first MFMA
      float p0 = 0.f, p1 = 0.f;
      auto phase = [&](auto PHC) {
        constexpr int ph = decltype(PHC)::value;
        constexpr int mb = ph % HB;
        constexpr bool last_use = (ph == HB - 1);     // block-0 fragments retire in this group
        constexpr int eg = (ph + G - LAG) % G;        // group whose epilogue runs now
        constexpr int emb = eg % HB;
        // The wave's priority rises with its progress through the tile's MFMA
        // groups: when both waves of a SIMD are in their MFMA sections, the
        // one further along issues first, so the two drift apart instead of
        // interleaving and reaching their loop tops together.
        __builtin_amdgcn_s_setprio(ph < 3 ? ph : 3);  // (the priority field is 2 bits wide)
        const float e = qfr.epilogue(acc[eg], emb);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          acc[ph] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qfr.qf[mb][ks], kf[ks], ks == 0 ? f32x16{} : acc[ph],
                                                            0, 0, 0);
          if constexpr (last_use) kf[ks] = *reinterpret_cast<const bf16x8*>(tile + boff[ks] + BLK_BYTES);
        }
        // (the first group of each block starts its sum instead of adding to
        // 0: an epilogue sum starts from +0 and is never -0, so 0 + e == e)
        if constexpr (ph < LAG) {
          if constexpr (ph == 0) p1 = e; else p1 += e;  // previous tile, block 1
          if constexpr (ph == LAG - 1) offer_tile(prev_p0, p1, prev_tbase, pend, prev_mask);
        } else {
          if constexpr (ph == LAG) p0 = e; else p0 += e;  // this tile, block 0
        }
        // Interleave: one MFMA, then a share of the epilogue / offer VALU work.
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if constexpr (last_use) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, ph == LAG - 1 ? 7 : 4, 0);
        }
      };
      static_for<G>(phase);
      __builtin_amdgcn_s_setprio(0);
      (void)p1;
      prev_p0 = p0;
      prev_tbase = tbase;
      prev_mask = cur_mask;
      pend = true;
    } else {
      // ---- partial tile (the row's causal edge): drain, then one block ------
      if (pend) {
        drain();
        pend = false;
      }
      if (nblk == 1) {
        bf16x8 kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const bf16x8*>(tile + boff[ks]);
        float p0 = 0.f;
#pragma unroll
        for (int mb = 0; mb < HB; ++mb) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qfr.qf[mb][ks], kf[ks], ks == 0 ? f32x16{} : acc[0],
                                                             0, 0, 0);
          p0 += qfr.epilogue(acc[0], mb);
        }
        offer_tile(p0, 0.f, tbase, true, cur_mask);
      }
    }
    // Every offer needs room for 64 keys and a tile makes at most two
    // (a partial tile drains the pending one first): a row holding more than
    // C - 128 keys compacts before its next offer.
    if constexpr (SHARE_COMP) {
      comp_req[(it & 1) * NW + wave] = sel.needs_compaction();
    } else {
      if (sel.needs_compaction()) sel.template compact<WaveSelect<C>::NEEDS_MIN>(lane);
    }
    // Tile it+1 must have landed.
    wait_vm_lgkm0<0>();
    __syncthreads();
  };
  {
    int it = 0;
    for (; it + 1 < ntiles; it += 2) {
      tile_step(it, std::integral_constant<int, 0>{});
      tile_step(it + 1, std::integral_constant<int, 1>{});
    }
    if (it < ntiles) tile_step(it, std::integral_constant<int, 0>{});
  }

  if (sel.needs_compaction()) sel.template compact<WaveSelect<C>::NEEDS_MIN>(lane);  // room for the pending offer
  if (pend) drain();

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

  KTileLoader<D, TILE_N, NT> ld;
  ld.init(a.kst);
  const int ntiles = (a.T + TILE_N - 1) / TILE_N;
  if (ntiles > 0) ld.issue(kb, a.kst, 0, a.T, lds);
  tile_barrier();
  static_assert(NB % 2 == 0, "32-key blocks are stored in pairs");
  for (int it = 0; it < ntiles; ++it) {
    const bool more = it + 1 < ntiles;
    if (more) ld.issue(kb, a.kst, (it + 1) * TILE_N, a.T, lds + ((it + 1) & 1) * TILE_BYTES);
    const char* tile = lds + (it & 1) * TILE_BYTES;
    const int tbase = it * TILE_N;
    // Full tiles of a row that overwrites its scores issue exactly NB / 2
    // stores after the copy of tile it+1, so the wait before the barrier
    // leaves them in flight and covers only that copy (vector memory
    // operations -- global loads, LDS-DMA copies, stores -- report completion
    // to the wave in execution order on this GFX9-family part, which is what
    // vmcnt counts); every other case waits for all.
    const bool lean = active && !a.accumulate && tbase + TILE_N <= a.T;
    if (active) {
      int nblk = (a.T - tbase + 31) / 32;
      nblk = nblk > NB ? NB : nblk;
      float p[NB];
      if (nblk == NB) {
        qfr.template tile_partials<NB, true>(tile, NB, lane, p);
      } else {
        qfr.template tile_partials<NB, false>(tile, nblk, lane, p);
      }
      // Blocks 2j and 2j+1: one half-wave swap leaves key 64j + lane's sum in
      // lane `lane` (block 2j's in lanes 0-31, block 2j+1's in 32-63), so each
      // pair is one coalesced 64-lane store.
#pragma unroll
      for (int j = 0; j < NB / 2; ++j) {
        const SwapPair r = permlane32_swap(__float_as_uint(p[2 * j]), __float_as_uint(p[2 * j + 1]));
        const float v = __uint_as_float(r.x) + __uint_as_float(r.y);
        const int t = tbase + 64 * j + lane;
        float* o = orow + static_cast<int64_t>(t) * a.sst;
        if (lean) {
          *o = v;
        } else if (t < a.T) {
          *o = a.accumulate ? *o + v : v;
        }
      }
    }
    asm volatile("" ::: "memory");
    if (lean) wait_vm_lgkm0<NB / 2>();
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
}

}  // namespace si
