// Fused score + streaming exact top-k with four 32-head M-blocks per wave:
// two query rows of up to 64 heads (HB = 2) or one row of up to 128 heads
// (HB = 4).
//
//   I(s, t) = sum_h w[s, h] * relu(q[s, h, :] . k[t, :])        (bf16 in, fp32 acc)
//
// Reference behaviour being replaced: flash_sparse/triton/indexer_score.py:41-179
// (scores) and flash_sparse/triton/chunked_indexer.py:47-160 (chunked top-k);
// results are those of indexer_topk_kernel (indexer_kernels.h), which this
// kernel replaces for the shapes it serves.
//
// Why four M-blocks per wave: every 32-key B-fragment read from LDS feeds
// four v_mfma_f32_32x32x16_bf16 instead of two, halving LDS read traffic
// per FLOP; on gfx950 those reads cost a large share of the power that caps
// the shader clock.  The Q fragments of four M-blocks take 128 registers, so
// a wave owns its SIMD (512 registers, the Q fragments in AGPRs as MFMA
// A-operands) and hides its own latencies:
//   * a 3-slot K ring: tile i+2 is copied (global_load_lds) while tile i is
//     consumed, so tile i+1 is resident and visible during tile i and its
//     first block's B-fragments are read behind tile i's MFMAs;
//   * two B-fragment register sets (block 0, block 1), each read at least a
//     full MFMA group before its first use;
//   * four accumulator sets: group g's MFMAs run while the epilogue (ReLU +
//     fp32 weighted head sum) of group g-2 reads its accumulator;
//   * one workgroup barrier per 64-key tile, in the middle of the tile,
//     where the copy issued one tile earlier has long landed.
// Each 64-key tile runs 8 groups (2 key blocks x 4 M-blocks) of 8 dependent
// MFMAs over D.  A row's 64 keys are offered to its selection buffer
// (wave_select.h) once its four (or eight) group epilogues are summed.
// Tiles are always computed whole: the rows of a workgroup (8 or 4
// consecutive queries) share their last legal tile up to a few keys, and the
// causal bound is applied per key when offering.
#pragma once

#include "indexer_kernels.h"

namespace si {

// Sum over this lane's 16 heads of one M-block: sum_v w_v * relu(acc_v), in
// the order of QueryFrags::epilogue (two interleaved chains), so that scores
// are bit-identical to the other indexer kernels.
__device__ __forceinline__ float weighted_relu_sum(const f32x16& acc, const float (&w)[16]) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int v = 0; v < 16; v += 2) {
    s0 = __builtin_fmaf(w[v], __builtin_amdgcn_fmed3f(acc[v], 0.f, __FLT_MAX__), s0);
    s1 = __builtin_fmaf(w[v + 1], __builtin_amdgcn_fmed3f(acc[v + 1], 0.f, __FLT_MAX__), s1);
  }
  return s0 + s1;
}

// Keeps the computation of x inside the stretch of code between the
// sched_barrier fences around it: an empty volatile asm that reads and
// writes x, so that IR passes do not sink or hoist its producers.
template <typename T>
__device__ __forceinline__ void pin_vgpr(T& x) {
  asm volatile("" : "+v"(x));
}

// Compaction of one row's selection buffer, as a call: it runs rarely, and
// inlined copies (per row and per unrolled tile) would keep their
// precomputed LDS addresses in registers across the whole tile loop.
// Returns the new key count (high word) and floor score word (low word).
template <int C>
__device__ __noinline__ uint64_t wide_compact(__attribute__((address_space(3))) uint64_t* buf, int n, uint32_t tau,
                                              int top_k, int lane) {
  WaveSelect<C> s;
  s.buf = (uint64_t*)(buf);
  s.n = n;
  s.tau = tau;
  s.floor_key = 0;
  s.top_k = top_k;
  s.compact(lane);
  return (static_cast<uint64_t>(static_cast<uint32_t>(s.n)) << 32) | s.tau;
}

template <int HB, int D, int C, bool MASKED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void indexer_topk_wide_kernel(IndexerArgs a) {
  constexpr int NW = 4;
  constexpr int NT = NW * 64;
  constexpr int RPW = 4 / HB;       // query rows per wave
  constexpr int MB = RPW * HB;      // M-blocks per wave (4)
  constexpr int ROWS = NW * RPW;    // query rows per workgroup
  constexpr int KS = D / 16;        // MFMA k-steps per 32-key block
  constexpr int TILE_N = 64;
  constexpr int NB = 2;             // 32-key blocks per tile
  constexpr int G = NB * MB;        // MFMA groups per tile
  constexpr int LAG = 2;            // the epilogue of group g runs during group g + LAG
  constexpr int NACC = 4;           // accumulator sets (G % NACC == 0, NACC > LAG)
  // Group (counted from a tile's first group) at which the offer of row 0 /
  // row RPW-1 for that tile runs: one group after the epilogue of the row's
  // last M-block of block 1.
  constexpr int OFFER_G0 = (NB - 1) * MB + HB - 1 + LAG + 1;
  constexpr int OFFER_G1 = (NB - 1) * MB + (RPW - 1) * HB + HB - 1 + LAG + 1;
  constexpr int RING = 3;
  constexpr int TILE_BYTES = TILE_N * D * 2;
  constexpr int BLK_BYTES = 32 * D * 2;
  constexpr int SEL_OFF = RING * TILE_BYTES;
  constexpr int LPT = KTileLoader<D, TILE_N, NT>::LPT;  // tile copies issued per thread
  static_assert(LPT <= MB, "one copy per group of the tile's second half");
  constexpr int REQ_OFF = SEL_OFF + ROWS * C * 8;
  static_assert(MB == 4 && G % NACC == 0 && NACC > LAG, "group pipeline shape");
  static_assert(OFFER_G0 >= G && OFFER_G1 < G + MB, "offers run in the next tile's first half");
  static_assert(RPW == 1 || OFFER_G1 - OFFER_G0 >= 1, "one offer per group");
  static_assert(KS % 2 == 0, "a block's B-fragment reads are split over two groups");
  static_assert(KS % 4 == 0, "the four offer steps are spread evenly over a group's chunks");
  static_assert(SEL_OFF <= 65536, "global_load_lds destinations stay below 64 KiB");
  static_assert(topk_wide_fits<HB, D, C>(), "ring + selection buffers exceed LDS");
  __shared__ __attribute__((aligned(16))) char lds[REQ_OFF + RING * NW * 4];
  uint64_t* const sel_base = reinterpret_cast<uint64_t*>(lds + SEL_OFF);
  int* const comp_req = reinterpret_cast<int*>(lds + REQ_OFF);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nqb = (a.S + ROWS - 1) / ROWS;
  const int b = blockIdx.x % a.B;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x / a.B);  // heaviest first
  const int s0 = qb * ROWS;
  const int s_last = (s0 + ROWS < a.S ? s0 + ROWS : a.S) - 1;
  const int wg_lim = legal_limit(a, s_last);

  // Per-row state lives in arrays indexed only by compile-time row numbers
  // (static_for), so that it stays in registers.
  int srow[RPW], lim[RPW];
  static_for<RPW>([&](auto RC) {
    constexpr int r = decltype(RC)::value;
    srow[r] = s0 + wave * RPW + r;
    lim[r] = srow[r] < a.S ? legal_limit(a, srow[r]) : 0;
  });

  // Q A-fragments and head weights of the wave's four M-blocks: M-block mb
  // is head block mb % HB of row mb / HB.
  bf16x8 qf[MB][KS];
  float wf[MB][16];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = mb / HB;
    const bool act = srow[r] < a.S;
    const int s = act ? srow[r] : 0;
    const uint16_t* qrow = a.q + b * a.qsb + static_cast<int64_t>(s) * a.qss;
    const int h = (mb % HB) * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d = ks * 16 + (lane >> 5) * 8;
      qf[mb][ks] = (act && h < a.H) ? *reinterpret_cast<const bf16x8*>(qrow + h * a.qsh + d) : bf16x8{};
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int hh = (mb % HB) * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      float wv = 0.f;
      if (act && hh < a.H) {
        const int64_t off = b * a.wsb + static_cast<int64_t>(s) * a.wss + hh * a.wsh;
        wv = a.w_bf16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.w)[off])
                      : reinterpret_cast<const float*>(a.w)[off];
      }
      wf[mb][v] = wv;
    }
  }

  // Per-lane B-fragment offsets of block 0 (block 1 is BLK_BYTES further on).
  int boff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) boff[ks] = kt_off<D>(lane & 31, ks * 2 + (lane >> 5));

  // Which 32-key block of a tile this lane offers after the half-wave swap.
  const int oblk = static_cast<int>(permlane32_swap(0u, 1u).x);
  const int okey = oblk * 32 + (lane & 31);

  WaveSelect<C> sel[RPW];
  static_for<RPW>([&](auto RC) {
    constexpr int r = decltype(RC)::value;
    sel[r].init(sel_base + (wave * RPW + r) * C, a.top_k);
  });

  const uint16_t* kb = a.k + b * a.ksb;
  const uint8_t* mrow[RPW];
  static_for<RPW>([&](auto RC) {
    constexpr int r = decltype(RC)::value;
    mrow[r] = MASKED ? a.mask + b * a.msb + static_cast<int64_t>(srow[r] < a.S ? srow[r] : 0) * a.mss : nullptr;
  });

  KTileLoader<D, TILE_N, NT> ld;
  ld.init(a.kst);
  const int ntiles = (wg_lim + TILE_N - 1) / TILE_N;
  if (ntiles > 0) ld.issue(kb, a.kst, 0, a.T, lds);
  if (ntiles > 1) ld.issue(kb, a.kst, TILE_N, a.T, lds + TILE_BYTES);

  f32x16 acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = f32x16{};
  bf16x8 kf[NB][KS];  // B-fragments of block 0 / block 1
  float ps[RPW][NB];  // per-lane partial sums of the tile being epilogued
  bool mask_cur[RPW], mask_prev[RPW];
  static_for<RPW>([&](auto RC) {
    constexpr int r = decltype(RC)::value;
    ps[r][0] = ps[r][1] = 0.f;
    mask_cur[r] = mask_prev[r] = true;
  });

  // Tiles 0 and 1 landed; block 0 of tile 0 into registers.
  wait_vm_lgkm0<0>();
  __syncthreads();
  if (ntiles > 0) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[0][ks] = *reinterpret_cast<const bf16x8*>(lds + boff[ks]);
  }

  auto compact_row = [&](auto RC) {
    constexpr int r = decltype(RC)::value;
    const uint64_t st = wide_compact<C>((__attribute__((address_space(3))) uint64_t*)(sel[r].buf),
                                        sel[r].n, sel[r].tau, sel[r].top_k, lane);
    sel[r].n = __builtin_amdgcn_readfirstlane(static_cast<int>(st >> 32));
    sel[r].tau = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(st));
  };

  // A row's 64-key offer (WaveSelect::offer64, restated in four steps so
  // that it interleaves with MFMAs): the half-wave swap that adds the two
  // head halves of each key, the key and its filter, the ballot and
  // positions, the append.
  constexpr int OFFER_PARTS = 4;
  float osum = 0.f;     // the score of the key this lane offers
  uint64_t okey64 = 0;  // the key itself
  uint64_t obal = 0;    // the lanes whose keys pass the row's floor
  int opos = 0, otot = 0;
  auto offer_part = [&](auto RC, auto PC, int tbase, bool valid, bool mok) {
    constexpr int r = decltype(RC)::value;
    constexpr int part = decltype(PC)::value;
    if constexpr (part == 0) {
      const SwapPair sp = permlane32_swap(__float_as_uint(ps[r][0]), __float_as_uint(ps[r][1]));
      osum = __uint_as_float(sp.x) + __uint_as_float(sp.y);
      pin_vgpr(osum);
    } else if constexpr (part == 1) {
      const int t = tbase + okey;
      okey64 = make_key(osum, static_cast<uint32_t>(t));
      // (kept as a lane mask, not a per-lane bool, so that no 0/1 register
      // is made and compared back)
      obal = __builtin_amdgcn_ballot_w64(valid && t < lim[r] && mok && key_hi(okey64) > sel[r].tau);
      pin_vgpr(okey64);
    } else if constexpr (part == 2) {
      const int below = lanes_below(obal);
      otot = __builtin_popcountll(obal);
      opos = __builtin_amdgcn_inverse_ballot_w64(obal) ? sel[r].n + below : sel[r].n + otot + (lane - below);
      pin_vgpr(opos);
    } else {
      sel[r].buf[opos] = okey64;
      sel[r].n = __builtin_amdgcn_readfirstlane(sel[r].n + otot);
    }
  };

  int4 rq_prev = int4{0, 0, 0, 0};  // compaction requests posted at the previous mid-tile point

  // One tile.  SLOT (= it % RING) is a compile-time constant so every LDS
  // address is a per-lane base plus an immediate.  Each group is written as
  // KS chunks (one MFMA, its share of B-fragment reads, epilogue VALU and
  // offer steps) fenced by sched_barrier, which fixes the interleaving.
  auto tile_step = [&](const int it, auto SLOTC) {
    constexpr int slot = decltype(SLOTC)::value;
    constexpr int nslot = (slot + 1) % RING;
    constexpr int fslot = (slot + 2) % RING;
    const int tbase = it * TILE_N;
    const char* tile = lds + slot * TILE_BYTES;
    const char* ntile = lds + nslot * TILE_BYTES;
    if constexpr (MASKED) {
      static_for<RPW>([&](auto RC) {
        constexpr int r = decltype(RC)::value;
        mask_prev[r] = mask_cur[r];
        const int t = tbase + okey;
        mask_cur[r] = t < lim[r] ? mrow[r][static_cast<int64_t>(t) * a.mst] != 0 : false;
      });
    }
    __builtin_amdgcn_sched_barrier(0);

    // Copy of tile it+2, issued one load per group in the tile's second half
    // (source and slot set at the mid-tile point).  When there is no such
    // tile, or it crosses T (then the mid-tile point issues it whole,
    // row-clamped), the loads re-copy tile 0 into this tile's own slot, which
    // no wave reads any more and whose next copy is issued after the next
    // mid-tile barrier: the issue needs no branch.
    const char* dma_src = reinterpret_cast<const char*>(kb);
    char* dma_dst = lds + slot * TILE_BYTES;

    auto group = [&](auto GC) {
      constexpr int g = decltype(GC)::value;
      constexpr int nb = g / MB;
      constexpr int mb = g % MB;
      constexpr int set = g % NACC;
      // Epilogue of group g - LAG (of the previous tile when g < LAG).
      constexpr int eg = (g + G - LAG) % G;
      constexpr int emb = eg % MB;
      constexpr int enb = eg / MB;
      constexpr int erow = emb / HB;
      constexpr int eset = eg % NACC;
      // A row's offer for a tile runs one group after the epilogue of its
      // last M-block of block 1, i.e. in the next tile's first half.
      constexpr int orow = (g == OFFER_G0 - G) ? 0 : ((RPW > 1 && g == OFFER_G1 - G) ? RPW - 1 : -1);
      // B-fragment reads issued behind this group's MFMAs: this tile's block 1
      // in groups 0 and 1, the next tile's block 0 in groups MB and MB + 1.
      constexpr bool rd1 = g < 2;
      constexpr bool rd0 = g >= MB && g < MB + 2;
      constexpr int rks0 = (g % 2) * (KS / 2);
      constexpr int PPK = 8 / KS;  // epilogue element pairs per chunk

      float s0 = 0.f, s1 = 0.f;
      auto chunk = [&](auto KC) {
        constexpr int ks = decltype(KC)::value;
        acc[set] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[mb][ks], kf[nb][ks], ks == 0 ? f32x16{} : acc[set],
                                                           0, 0, 0);
        if constexpr (rd1 && ks >= rks0 && ks < rks0 + KS / 2)
          kf[1][ks] = *reinterpret_cast<const bf16x8*>(tile + boff[ks] + BLK_BYTES);
        // (after the last tile this reads a stale slot that is never used)
        if constexpr (rd0 && ks >= rks0 && ks < rks0 + KS / 2)
          kf[0][ks] = *reinterpret_cast<const bf16x8*>(ntile + boff[ks]);
        if constexpr (g >= MB && g < MB + LPT && ks == 1) ld.issue_at(dma_src, dma_dst, g - MB);
#pragma unroll
        for (int j = ks * PPK; j < (ks + 1) * PPK; ++j) {
          const int v = 2 * j;
          s0 = __builtin_fmaf(wf[emb][v], __builtin_amdgcn_fmed3f(acc[eset][v], 0.f, __FLT_MAX__), s0);
          s1 = __builtin_fmaf(wf[emb][v + 1], __builtin_amdgcn_fmed3f(acc[eset][v + 1], 0.f, __FLT_MAX__), s1);
        }
        pin_vgpr(s0);
        pin_vgpr(s1);
        // The offer's steps run every KS / OFFER_PARTS chunks from chunk 0, so
        // that their VALU work hides behind as many MFMAs as possible.
        static_for<OFFER_PARTS>([&](auto PC) {
          constexpr int part = decltype(PC)::value;
          if constexpr (orow >= 0 && part * (KS / OFFER_PARTS) == ks)
            offer_part(std::integral_constant<int, (orow < 0 ? 0 : orow)>{}, PC, tbase - TILE_N, it > 0,
                       mask_prev[orow < 0 ? 0 : orow]);
        });
        __builtin_amdgcn_sched_barrier(0);
      };
      static_for<KS>(chunk);
      // Same association as weighted_relu_sum and QueryFrags::epilogue.  A
      // row's first M-block of a key block starts the partial sum (the row's
      // offer has read the previous tile's by then; an epilogue sum starts
      // from +0 and is never -0, so this equals adding it to zero).
      if constexpr (emb % HB == 0) ps[erow][enb] = s0 + s1; else ps[erow][enb] += s0 + s1;
      pin_vgpr(ps[erow][enb]);

      if constexpr (g == MB - 1) {
        // Mid-tile barrier: the copy of tile it+1 (issued one tile ago) has
        // landed and every wave is past its reads of tile it-1's slot, which
        // then takes the copy of tile it+2.  No copy is in flight between
        // the barrier and that issue, which is where the compactions run.
        // Between two mid-tile points every row receives exactly one 64-key
        // offer, so a row must compact when it holds more than C - 64 keys.
        // A row that will need to at the next mid-tile point (more than
        // C - 128 now) posts a request; the requests are read one tile later
        // (no wait on the read), and then every row that is close to needing
        // a compaction joins in, so the workgroup waits once for all of them.
        int pred = 0;
        static_for<RPW>([&](auto RC) { pred |= sel[decltype(RC)::value].needs_compaction() ? 1 : 0; });
        comp_req[slot * NW + wave] = pred;
        wait_vm_lgkm0<0>();
        __syncthreads();
        const bool any = (rq_prev.x | rq_prev.y | rq_prev.z | rq_prev.w) != 0;
        rq_prev = *reinterpret_cast<const int4*>(comp_req + slot * NW);
        static_for<RPW>([&](auto RC) {
          constexpr int r = decltype(RC)::value;
          if (sel[r].n > C - kWave || (any && sel[r].wants_compaction())) compact_row(RC);
        });
        if (it + 2 < ntiles && (it + 3) * TILE_N <= a.T) {
          dma_src = reinterpret_cast<const char*>(kb + static_cast<int64_t>(it + 2) * TILE_N * a.kst);
          dma_dst = lds + fslot * TILE_BYTES;
        } else if (it + 2 < ntiles) {
          ld.issue(kb, a.kst, (it + 2) * TILE_N, a.T, lds + fslot * TILE_BYTES);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    static_for<G>(group);
  };

  for (int it = 0; it < ntiles; it += RING) {
    tile_step(it, std::integral_constant<int, 0>{});
    if (it + 1 < ntiles) tile_step(it + 1, std::integral_constant<int, 1>{});
    if (it + 2 < ntiles) tile_step(it + 2, std::integral_constant<int, 2>{});
  }

  // Epilogues of the last tile's groups G-LAG .. G-1, then every row's offer
  // for that tile.
  if (ntiles > 0) {
    static_for<LAG>([&](auto GC) {
      constexpr int eg = G - LAG + decltype(GC)::value;
      constexpr int emb = eg % MB;
      const float e = weighted_relu_sum(acc[eg % NACC], wf[emb]);
      if constexpr (emb % HB == 0) ps[emb / HB][eg / MB] = e; else ps[emb / HB][eg / MB] += e;
    });
    static_for<RPW>([&](auto RC) {
      constexpr int r = decltype(RC)::value;
      if (sel[r].n > C - kWave) compact_row(RC);
    });
    const int tlast = (ntiles - 1) * TILE_N;
    static_for<RPW>([&](auto RC) {
      constexpr int r = decltype(RC)::value;
      static_for<OFFER_PARTS>([&](auto PC) { offer_part(RC, PC, tlast, true, mask_cur[r]); });
    });
  }

  static_for<RPW>([&](auto RC) {
    constexpr int r = decltype(RC)::value;
    if (srow[r] < a.S) {
      const int s = srow[r];
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
      sel[r].finish(out, lane);
    }
  });
}

template <int HB, int D, int C>
int launch_topk_wide(const IndexerArgs& a, hipStream_t st) {
  if constexpr (!topk_wide_fits<HB, D, C>()) {
    return set_error(SI_ERR_UNSUPPORTED, "shape not served by the four-M-block top-k kernel");
  } else {
  if (a.top_k > WaveSelect<C>::MAX_TOPK) return set_error(SI_ERR_UNSUPPORTED, "top_k exceeds the selection capacity");
  if (a.T < 64) return set_error(SI_ERR_UNSUPPORTED, "the four-M-block kernel needs T >= 64");
  constexpr int ROWS = 4 * (4 / HB);
  const int nqb = (a.S + ROWS - 1) / ROWS;
  const int64_t nblk = static_cast<int64_t>(nqb) * a.B;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  if (a.mask) {
    hipLaunchKernelGGL((indexer_topk_wide_kernel<HB, D, C, true>), dim3(static_cast<unsigned>(nblk)), dim3(256), 0,
                       st, a);
  } else {
    hipLaunchKernelGGL((indexer_topk_wide_kernel<HB, D, C, false>), dim3(static_cast<unsigned>(nblk)), dim3(256), 0,
                       st, a);
  }
  return check_launch("indexer_topk_wide_kernel");
  }
}

}  // namespace si
