// Sparse-attention backward (MQA, attention sink) for gfx950.
//
// Reference behaviour being replaced:
//   * flash_sparse/triton/sparse_attn_bwd.py:1-26    (the gradients)
//   * flash_sparse/triton/sparse_attn_bwd.py:49-97   (_delta_kernel: delta = sum_d o do)
//   * flash_sparse/triton/sparse_attn_bwd.py:100-283 (_sparse_attn_bwd_kernel)
//   * flash_sparse/triton/sparse_attn_bwd.py:286-416 (sparse_attn_bwd wrapper)
//
// From the forward's saved o (bf16) and lse (fp32, sink included):
//   p[s,h,j]  = e^{scale q.k_j - lse},   delta[s,h] = sum_d o do,
//   ds[s,h,j] = p (do.k_j - delta) scale,
//   dq[s,h]   = sum_j ds k_j,
//   dkv[t]    = sum over (s,j) with idx[s,j] = t of  sum_h ds q[s,h] + p do[s,h],
//   dsink[h]  = -sum_s e^{sink_h - lse[s,h]} delta[s,h].
//
// The reference scatters dkv with fp32 atomics, S*K*D of them.  On MI355X
// those run at ~1.3 TB/s of payload (one dword per L2 channel per clock),
// ~57 ms at S=64K, K=512, D=576, several times the arithmetic.  This build
// instead materialises the per-(query, slot) dkv rows once and reduces them
// key-major, deterministically:
//   1. bwd_rows: one workgroup per query row and 64 heads, shaped like the
//      forward kernel: four producer waves compute S^T = K Q^T and
//      dP^T = K dO^T for their 16 heads from the same K fragments, then
//      P and dS in registers; four consumer waves gather the KV tiles into
//      an LDS ring (global_load_lds) and accumulate dQ^T = K^T dS^T.  The
//      producers also write P and dS (bf16, in their register layout, 8 KiB
//      per tile) for step 2 and the row's dsink terms.
//   2. bwd_dkv_rows: one workgroup per (query row, 64 heads): the row's Q and
//      dO stay in LDS; per tile, dkv rows^T = [Q^T | dO^T] [dS; P] with both
//      operands read through transposing LDS reads; bf16 rows go to a
//      workspace, one per (query, slot).
//   3. The (key, pair) list is sorted by key (rocPRIM radix sort, stable, so
//      the order is deterministic), segments are marked, and bwd_dkv_reduce
//      sums each key's rows in fp32 (one workgroup per key).
//   4. dsink is a fixed-order sum of the per-row terms.
// Long sequences are processed in chunks of query rows sized to the
// workspace the caller provides; dkv accumulates across chunks in fp32.
#include <rocprim/device/device_radix_sort.hpp>

#include <string>
#include <type_traits>

#include "attn_common.h"
#include "si_common.h"
#include "si_status.h"

namespace si {

struct AttnBwdArgs {
  const uint16_t* q;  // [B,S,H,D] bf16 or fp16 (f16); kv, o, dout, dq, coef and prow share the type
  int64_t qsb, qss, qsh;
  const uint16_t* kv;  // [B,N,D]
  int64_t kvsb, kvsn;
  const float* sink;   // [H]
  const void* idx;     // [B,S,K] int32 / int64
  int idx64;
  int64_t isb, iss, isk;
  const uint16_t* o;   // [B,S,H,D], forward output
  int64_t osb, oss, osh;
  const uint16_t* dout;  // [B,S,H,D], gradient of o
  int64_t gsb, gss, gsh;
  const float* lse;    // [B,S,H]
  int64_t lsb, lss, lsh;
  uint16_t* dq;        // [B,S,H,D]
  int64_t dqsb, dqss, dqsh;
  float* dsink_rows;   // [B*S, 64*HG]: -e^{sink-lse} delta per (row, head)
  uint16_t* coef;      // [nrows, HG, ntiles, 2, 4, 64, 8]: P, dS fragments
  uint16_t* prow;      // [nrows, HG, 32 ntiles, D]: per-(query, slot) dkv rows
  int B, S, H, N, K, HG, ntiles;  // ntiles: key tiles of a full row (the workspace layout)
  const int32_t* row_len;  // optional [B,S]: columns at or past row_len[b,s] are masked, their tiles skipped
  int64_t rlsb, rlss;
  int64_t row0;        // first global row (b*S + s) of this chunk
  int nrows;           // rows in this chunk
  float scale, scale_log2;
  int f16;             // element type: 0 bf16, 1 fp16
};

constexpr int kBwdThreads = 2 * kAttnWaves * 64;

// Columns of row (b, s): K, or fewer when row lengths are given.
__device__ __forceinline__ int bwd_row_len(const AttnBwdArgs& a, int b, int s) {
  if (!a.row_len) return a.K;
  const int rl = a.row_len[b * a.rlsb + static_cast<int64_t>(s) * a.rlss];
  return rl < 0 ? 0 : (rl < a.K ? rl : a.K);
}
// bf16 elements of one tile's coefficient block: [P, dS][wave][lane][8 keys]
constexpr int kCoefTile = 2 * kAttnWaves * 64 * 8;
constexpr float kLog2e = 1.4426950408889634f;


// ---------------------------------------------------------------------------
// 1. dQ, P / dS coefficients and dsink terms per query row
// ---------------------------------------------------------------------------
template <int D, bool IDX64, bool F16>
__global__ __launch_bounds__(kBwdThreads) void sparse_attn_bwd_rows_kernel(AttnBwdArgs a) {
  using SH = AttnShape<D>;
  constexpr int KS = SH::KS;
  constexpr int MBW = SH::MBW;
  constexpr int ROW = SH::ROW;
  __shared__ __attribute__((aligned(16))) char kv_lds[SH::LDS_KV];
  __shared__ __attribute__((aligned(16))) char p_lds[2][kAttnWaves * 64 * 16];  // dS^T B-fragments per head block
  __shared__ __attribute__((aligned(16))) float bias_lds[kAttnRing][kAttnTK];  // 0: key used, -inf: masked
  __shared__ uint32_t rowoff_lds[kAttnRing][kAttnTK];    // offset of the key's KV row, 16-byte units
  __shared__ __attribute__((aligned(16))) uint32_t idxraw_lds[2 * kAttnRing][2 * kAttnTK];  // raw index words

  const int lane = threadIdx.x & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  __builtin_assume(wave_all >= 0 && wave_all < 2 * kAttnWaves);
  const bool producer = wave_all < kAttnWaves;
  const int wave = producer ? wave_all : wave_all - kAttnWaves;
  __builtin_assume(wave >= 0 && wave < kAttnWaves);
  const int g = lane >> 4;
  const int i16 = lane & 15;
  const int lrow = static_cast<int>(blockIdx.x % static_cast<unsigned>(a.nrows));
  const int hg = static_cast<int>(blockIdx.x / static_cast<unsigned>(a.nrows));
  const int64_t grow = a.row0 + lrow;
  const int b = static_cast<int>(grow / a.S);
  const int s = static_cast<int>(grow % a.S);
  const int hbase = hg * 64;
  const int klen = bwd_row_len(a, b, s);
  const int ntiles = a.ntiles > 0 ? (klen + kAttnTK - 1) / kAttnTK : 0;  // tiles of this row

  // Tile protocol (one barrier per tile), as in the forward kernel: in
  // iteration `it` the consumers accumulate dQ of tile it while the
  // producers compute P and dS of tile it+1 and publish its dS^T; tile t
  // lives in ring slot t % 4 and its dS^T in p_lds[t % 2].  The consumers
  // issue the copies of tile it+3 at the start of iteration it into the slot
  // of tile it-1 and wait for those of tile it+2 before the barrier.

  if (producer) {
    // ===================== S^T, dP^T, P, dS ===============================
    const int hq = hbase + wave * 16 + i16;
    const bool hvalid = hq < a.H;
    bf16x8 qf[KS], gf[KS];
    float delta = 0.f;
    {
      const int64_t rq = b * a.qsb + static_cast<int64_t>(s) * a.qss + static_cast<int64_t>(hq) * a.qsh;
      const int64_t rg = b * a.gsb + static_cast<int64_t>(s) * a.gss + static_cast<int64_t>(hq) * a.gsh;
      const int64_t ro = b * a.osb + static_cast<int64_t>(s) * a.oss + static_cast<int64_t>(hq) * a.osh;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = hvalid ? *reinterpret_cast<const bf16x8*>(a.q + rq + ks * 32 + g * 8) : bf16x8{};
        gf[ks] = hvalid ? *reinterpret_cast<const bf16x8*>(a.dout + rg + ks * 32 + g * 8) : bf16x8{};
      }
      // delta = sum_d o do over this lane's 8-dim slices, then the 4 lane groups
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 ov = hvalid ? *reinterpret_cast<const u32x4*>(a.o + ro + ks * 32 + g * 8) : u32x4{0u, 0u, 0u, 0u};
        const u32x4 gv = __builtin_bit_cast(u32x4, gf[ks]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          delta = __builtin_fmaf(elem_lo<F16>(ov[c]), elem_lo<F16>(gv[c]), delta);
          delta = __builtin_fmaf(elem_hi<F16>(ov[c]), elem_hi<F16>(gv[c]), delta);
        }
      }
      const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(delta), __float_as_uint(delta), false, false);
      delta = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
      const SwapPair r32 = permlane32_swap(__float_as_uint(delta), __float_as_uint(delta));
      delta = __uint_as_float(r32.x) + __uint_as_float(r32.y);
    }
    float lse2 = __builtin_inff();  // padding heads: p = 2^(x - inf) = 0
    if (hvalid) {
      const float lse = a.lse[b * a.lsb + static_cast<int64_t>(s) * a.lss + static_cast<int64_t>(hq) * a.lsh];
      lse2 = lse * kLog2e;
      if (g == 0)
        a.dsink_rows[grow * (64 * a.HG) + hq] = -__builtin_amdgcn_exp2f((a.sink[hq] - lse) * kLog2e) * delta;
    }
    const float dscale = a.scale;

    // S^T / dP^T A-fragment addresses (keys 16mb + i16, chunk 4ks + g), as in
    // the forward kernel.
    const int qf_swz = kv_swz<D>(i16);
    const int qbase = i16 * ROW + 16 * (g ^ (qf_swz & 3));
    const int qadj = 64 * (qf_swz >> 2);
    constexpr int QPD = KS < 2 ? KS : 2;
    auto qk = [&](int t, f32x4 (&st)[2], f32x4 (&dp)[2]) {
      const uint32_t tile = lds_addr(kv_lds + (t % kAttnRing) * SH::TILE);
      const uint32_t qa_e = tile + qbase + qadj;
      const uint32_t qa_o = tile + qbase - qadj;
      bf16x8 kq[QPD][2];
      auto qk_issue = [&](auto KC) {
        constexpr int ks = decltype(KC)::value;
        const uint32_t base = (ks & 1) ? qa_o : qa_e;
        kq[ks % QPD][0] = ld128<64 * ks>(base);
        kq[ks % QPD][1] = ld128<64 * ks + 16 * ROW>(base);
      };
      attn_static_for<0, QPD>(qk_issue);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        st[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      auto qk_step = [&](auto KC) {
        constexpr int ks = decltype(KC)::value;
        constexpr int later = (KS - 1 - ks) < (QPD - 1) ? (KS - 1 - ks) : (QPD - 1);
        lds_wait<2 * later>(kq[ks % QPD][0], kq[ks % QPD][1]);
        st[0] = mfma16x16x32<F16>(kq[ks % QPD][0], qf[ks], st[0]);
        dp[0] = mfma16x16x32<F16>(kq[ks % QPD][0], gf[ks], dp[0]);
        st[1] = mfma16x16x32<F16>(kq[ks % QPD][1], qf[ks], st[1]);
        dp[1] = mfma16x16x32<F16>(kq[ks % QPD][1], gf[ks], dp[1]);
        if constexpr (ks + QPD < KS) qk_issue(std::integral_constant<int, ks + QPD>{});
      };
      attn_static_for<0, KS>(qk_step);
      mfma_result_fence(st[0], st[1]);
      mfma_result_fence(dp[0], dp[1]);
    };

    uint16_t* coef_row = a.coef + (static_cast<int64_t>(lrow) * a.HG + hg) * a.ntiles * kCoefTile;
    // P and dS of tile t for head hq: dS^T goes to LDS for the dQ waves, both
    // to the coefficient workspace, as bf16 B-fragments whose k-slots
    // 8g+0..3 / 8g+4..7 hold keys 4g+0..3 / 16+4g+0..3.
    auto grad_store = [&](int t, const f32x4 (&st)[2], const f32x4 (&dp)[2], const f32x4 (&bias)[2]) {
      float p[2][4], d[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = __builtin_fmaf(st[mb][r], a.scale_log2, bias[mb][r]);
          p[mb][r] = __builtin_amdgcn_exp2f(x - lse2);
          d[mb][r] = p[mb][r] * (dp[mb][r] - delta) * dscale;
        }
      u32x4 wp, wd;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        wp[c] = pack2<F16>(p[c >> 1][2 * (c & 1)], p[c >> 1][2 * (c & 1) + 1]);
        wd[c] = pack2<F16>(d[c >> 1][2 * (c & 1)], d[c >> 1][2 * (c & 1) + 1]);
      }
      const uint32_t pa = lds_addr(&p_lds[t & 1][(wave * 64 + lane) * 16]);
      asm volatile("ds_write_b128 %0, %1" ::"v"(pa), "v"(wd) : "memory");
      uint16_t* ct = coef_row + static_cast<int64_t>(t) * kCoefTile + (wave * 64 + lane) * 8;
      *reinterpret_cast<u32x4*>(ct) = wp;
      *reinterpret_cast<u32x4*>(ct + kAttnWaves * 64 * 8) = wd;
    };
    auto read_bias = [&](int t, f32x4 (&bias)[2]) {
      bias[0] = *reinterpret_cast<const f32x4*>(&bias_lds[t % kAttnRing][4 * g]);
      bias[1] = *reinterpret_cast<const f32x4*>(&bias_lds[t % kAttnRing][16 + 4 * g]);
    };

    if (ntiles > 0) {
      __syncthreads();      // indices of tiles 0..3 published
      attn_tile_barrier();  // tile 0 landed
      f32x4 bias_cur[2];
      {
        f32x4 bias[2], st[2], dp[2];
        read_bias(0, bias);
        read_bias(1, bias_cur);
        qk(0, st, dp);
        grad_store(0, st, dp, bias);
      }
      attn_tile_barrier();  // tile 1 landed; dS^T of tile 0 published; tile 0's biases read
      attn_tile_barrier();  // indices of tile 4 published
      for (int it = 0; it < ntiles; ++it) {
        f32x4 bias_nx[2];
        read_bias(it + 2, bias_nx);  // the slot read is always inside the array
        if (it + 1 < ntiles) {
          f32x4 st[2], dp[2];
          qk(it + 1, st, dp);
          grad_store(it + 1, st, dp, bias_cur);
        }
        bias_cur[0] = bias_nx[0];
        bias_cur[1] = bias_nx[1];
        attn_tile_barrier();
      }
    }
    __syncthreads();  // every gather landed
    __syncthreads();  // dQ staged
  } else {
    // ================ dQ, KV gather and the index pipeline ==================
    const int ctid = static_cast<int>(threadIdx.x) - kAttnWaves * 64;  // 0 .. SH::NT-1
    const bool idx_wave = wave == 0;
    const char* idx_row = static_cast<const char*>(a.idx) +
                          (b * a.isb + static_cast<int64_t>(s) * a.iss) * (IDX64 ? 8 : 4);
    const char* kvb = reinterpret_cast<const char*>(a.kv + b * a.kvsb);

    // Key indices of tile t: copied raw into idxraw_lds[t % 8] by the index
    // wave (global_load_lds), validated after its next wait and published to
    // ring slot t % 4.
    auto load_idx = [&](int t) {
      int j = t * kAttnTK + (IDX64 ? (lane >> 1) : (lane & 31));
      j = j < klen ? j : klen - 1;  // klen > 0 whenever a tile exists
      const int64_t byte = static_cast<int64_t>(j) * a.isk * (IDX64 ? 8 : 4) + (IDX64 ? (lane & 1) * 4 : 0);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(idx_row + byte),
                                       (lds_void_t*)(&idxraw_lds[t % (2 * kAttnRing)][0]), 4, 0, 0);
    };
    auto store_idx = [&](int t) {
      const int slot = t % kAttnRing;
      const int rslot = t % (2 * kAttnRing);
      if (lane < kAttnTK) {
        const int64_t raw = IDX64 ? static_cast<int64_t>((static_cast<uint64_t>(idxraw_lds[rslot][2 * lane + 1]) << 32) |
                                                         idxraw_lds[rslot][2 * lane])
                                  : static_cast<int64_t>(static_cast<int32_t>(idxraw_lds[rslot][lane]));
        const int j = t * kAttnTK + lane;
        const bool ok = j < klen && raw >= 0 && raw < a.N;
        bias_lds[slot][lane] = ok ? 0.f : -__builtin_inff();
        rowoff_lds[slot][lane] = static_cast<uint32_t>((ok ? raw : 0) * (a.kvsn / 8));
      }
    };
    // Gather of tile t: LDS slot e (16 bytes) holds chunk (e % CPR) ^ f(key)
    // of key e / CPR; this thread's keys and chunks are fixed per copy.
    int dkey[SH::LPT], dcoff[SH::LPT];
#pragma unroll
    for (int i = 0; i < SH::LPT; ++i) {
      const int e = i * SH::NT + ctid;
      dkey[i] = e / SH::CPR;
      dcoff[i] = (e % SH::CPR) ^ kv_swz<D>(dkey[i]);
    }
    uint32_t roff[SH::LPT];
    auto read_roff = [&](int t, uint32_t (&dst)[SH::LPT]) {
      const int slot = t % kAttnRing;
#pragma unroll
      for (int i = 0; i < SH::LPT; ++i)
        dst[i] = (i * SH::NT + wave * 64 < SH::CH) ? rowoff_lds[slot][dkey[i]] + dcoff[i] : 0u;
    };
    // Copy i of tile t (one 64-lane group of 16-byte slots); every 64-slot
    // group lies wholly inside or wholly outside the tile (CH % 64 == 0), so a
    // wave issues either LPT or no copies per tile for every supported D.
    auto dma = [&](int t, auto IC) {
      constexpr int i = decltype(IC)::value;
      const int e0 = i * SH::NT + wave * 64;
      char* dst = kv_lds + (t % kAttnRing) * SH::TILE + e0 * 16;
      const uint16_t* src = reinterpret_cast<const uint16_t*>(kvb + (static_cast<uint64_t>(roff[i]) << 4));
      if constexpr (SH::CH % SH::NT == 0 || i + 1 < SH::LPT) {
        __builtin_amdgcn_global_load_lds(src, (lds_void_t*)dst, 16, 0, 0);
      } else if (e0 < SH::CH) {
        __builtin_amdgcn_global_load_lds(src, (lds_void_t*)dst, 16, 0, 0);
      }
    };
    auto issue_tile = [&](int t) {
      read_roff(t, roff);
      attn_static_for<0, SH::LPT>([&](auto IC) { dma(t, IC); });
    };

    // K^T transposing-read address (the forward kernel's V^T read).
    const int tkey = 4 * g + (i16 >> 2);
    const int tx = 2 * wave + ((i16 & 3) >> 1);
    const int tbase = tkey * ROW + 16 * ((tx ^ kv_swz<D>(tkey)) & (SH::CPR - 1)) + 8 * (i16 & 1);

    f32x4 qacc[MBW][4];
#pragma unroll
    for (int j = 0; j < MBW; ++j)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) qacc[j][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    // dQ^T += K^T dS^T of tile it for this wave's 16-dim blocks, all 64 heads.
    auto dq_tile = [&](int it) {
      const uint32_t pa = lds_addr(&p_lds[it & 1][0]) + lane * 16;
      bf16x8 pbr[4];
      pbr[0] = ld128<0>(pa);
      pbr[1] = ld128<1024>(pa);
      pbr[2] = ld128<2048>(pa);
      pbr[3] = ld128<3072>(pa);
      const uint32_t ta = lds_addr(kv_lds + (it % kAttnRing) * SH::TILE) + tbase;
      v4i16 lo[2], hi[2];
      lo[0] = tr_read<0>(ta);
      hi[0] = tr_read<16 * ROW>(ta);
      if constexpr (MBW > 1) {
        lo[1] = tr_read<128>(ta);
        hi[1] = tr_read<16 * ROW + 128>(ta);
      }
      auto block = [&](auto JC) {
        constexpr int j = decltype(JC)::value;
        if constexpr (j + 1 < MBW) lds_wait<2>(lo[j & 1], hi[j & 1]); else lds_wait<0>(lo[j & 1], hi[j & 1]);
        if constexpr (j == 0) {
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) reg_tie(pbr[nb]);
        }
        const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo[j & 1], hi[j & 1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) qacc[j][nb] = mfma16x16x32<F16>(vf, pbr[nb], qacc[j][nb]);
        if constexpr (j + 2 < MBW) {
          lo[j & 1] = tr_read<128 * (j + 2)>(ta);
          hi[j & 1] = tr_read<16 * ROW + 128 * (j + 2)>(ta);
        }
      };
      attn_static_for<0, MBW>(block);
    };

    uint32_t roff_nx[SH::LPT];  // copy sources of tile it+4
    auto iteration = [&](int it) {
      const bool issue = it + 3 < ntiles;
      const bool idx_load = idx_wave && it + 6 < ntiles;
      // tracked LDS reads before the copies (the compiler would make a tracked
      // LDS access that follows LDS-DMA copies wait for them)
      read_roff(it + 4, roff_nx);  // the slot read is always inside the array
      if (idx_load) load_idx(it + 6);
      if (issue) attn_static_for<0, SH::LPT>([&](auto IC) { dma(it + 3, IC); });
      dq_tile(it);
#pragma unroll
      for (int i = 0; i < SH::LPT; ++i) roff[i] = roff_nx[i];
      // the copies of tile it+2 and the indices of tile it+5 (issued one
      // iteration ago) landed; this iteration's stay in flight
      if (issue) {
        if (idx_load) __builtin_amdgcn_s_waitcnt(vm_lgkm0(SH::LPT + 1));
        else __builtin_amdgcn_s_waitcnt(vm_lgkm0(SH::LPT));
      } else {
        __builtin_amdgcn_s_waitcnt(vm_lgkm0(0));
      }
      if (idx_wave && it + 5 < ntiles) store_idx(it + 5);
    };

    if (ntiles > 0) {
      if (idx_wave) {
        const int np = ntiles < 6 ? ntiles : 6;
        for (int t = 0; t < np; ++t) load_idx(t);
        __builtin_amdgcn_s_waitcnt(0x7 << 4);
        for (int t = 0; t < np && t < 4; ++t) store_idx(t);
      }
      __syncthreads();  // indices of tiles 0..3 published
      issue_tile(0);
      if (ntiles > 1) issue_tile(1);
      if (ntiles > 2) issue_tile(2);
      if (ntiles > 2) __builtin_amdgcn_s_waitcnt(vm_lgkm0(2 * SH::LPT));
      else if (ntiles > 1) __builtin_amdgcn_s_waitcnt(vm_lgkm0(SH::LPT));
      else __builtin_amdgcn_s_waitcnt(vm_lgkm0(0));
      attn_tile_barrier();  // tile 0 landed
      read_roff(3, roff);
      if (ntiles > 2) __builtin_amdgcn_s_waitcnt(vm_lgkm0(SH::LPT));
      else __builtin_amdgcn_s_waitcnt(vm_lgkm0(0));
      attn_tile_barrier();  // tile 1 landed; every wave has read tile 0's row offsets and biases
      if (idx_wave && ntiles > 4) store_idx(4);
      attn_tile_barrier();  // indices of tile 4 published
      for (int it = 0; it < ntiles; ++it) {
        iteration(it);
        attn_tile_barrier();
      }
    }
    __builtin_amdgcn_s_waitcnt(0x7 << 4);  // no gather may still target the ring
    __syncthreads();  // every gather landed
    // dQ (bf16) staged head-major in LDS: [64 heads][OROW bytes]
#pragma unroll
    for (int j = 0; j < MBW; ++j) {
      const int mbi = j * kAttnWaves + wave;
      if (SH::MBT % kAttnWaves == 0 || mbi < SH::MBT) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          uint2 w;
          w.x = pack2<F16>(qacc[j][nb][0], qacc[j][nb][1]);
          w.y = pack2<F16>(qacc[j][nb][2], qacc[j][nb][3]);
          *reinterpret_cast<uint2*>(kv_lds + (nb * 16 + i16) * SH::OROW + (mbi * 16 + 4 * g) * 2) = w;
        }
      }
    }
    __syncthreads();  // dQ staged
  }

  // ---- coalesced 16-byte stores of the staged dQ (all threads) -------------
  const int hcount = (a.H - hbase) < 64 ? (a.H - hbase) : 64;
  uint16_t* qbase_out = a.dq + b * a.dqsb + static_cast<int64_t>(s) * a.dqss + static_cast<int64_t>(hbase) * a.dqsh;
  for (int e = threadIdx.x; e < hcount * SH::CPR; e += kBwdThreads) {
    const int h = e / SH::CPR, c = e % SH::CPR;
    *reinterpret_cast<u32x4*>(qbase_out + static_cast<int64_t>(h) * a.dqsh + c * 8) =
        *reinterpret_cast<const u32x4*>(kv_lds + h * SH::OROW + c * 16);
  }
}

// ---------------------------------------------------------------------------
// 2. per-(query, slot) dkv rows
// ---------------------------------------------------------------------------
constexpr int kRowsThreads = 256;

template <int D>
struct DkvShape {
  static constexpr int QROW = D * 2 + 32;  // padded LDS row of Q / dO (bytes): conflict-free transposing reads
  static constexpr int MBT = D / 16;       // 16-dim blocks
  static constexpr int MBW = (MBT + 3) / 4;
  static constexpr int QD = 64 * QROW;     // bytes of one of Q, dO
  static constexpr int COEF = kCoefTile * 2;  // bytes of one tile's coefficients
};

// dkv rows^T [D x 32 keys] of tile t = A [D x 128] . B [128 x 32 keys], with
// k = (dS heads 0..63 | P heads 0..63) against (Q | dO).  A lane of a
// 16x16x32 A-fragment holds 8 heads of one dimension and a B-fragment lane 8
// heads of one key: both come from two ds_read_b64_tr_b16 (a 16-lane group
// reads a 4 x 16 block and each lane receives one column of 4).
template <int D, bool F16>
__global__ __launch_bounds__(kRowsThreads) void sparse_attn_bwd_dkv_rows_kernel(AttnBwdArgs a) {
  using DS = DkvShape<D>;
  constexpr int MBW = DS::MBW;
  __shared__ __attribute__((aligned(16))) char qd_lds[2 * DS::QD];  // Q then dO, [64 heads][QROW]
  __shared__ __attribute__((aligned(16))) char coef_lds[DS::COEF];  // [P, dS][wave][lane][8 keys]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  __builtin_assume(wave >= 0 && wave < 4);
  const int g = lane >> 4;
  const int i16 = lane & 15;
  const int lrow = static_cast<int>(blockIdx.x % static_cast<unsigned>(a.nrows));
  const int hg = static_cast<int>(blockIdx.x / static_cast<unsigned>(a.nrows));
  const int64_t grow = a.row0 + lrow;
  const int b = static_cast<int>(grow / a.S);
  const int s = static_cast<int>(grow % a.S);
  const int hbase = hg * 64;
  const int klen = bwd_row_len(a, b, s);
  const int ntiles = a.ntiles > 0 ? (klen + kAttnTK - 1) / kAttnTK : 0;  // tiles of this row
  constexpr int CPR = D / 8;

  // Q and dO of the row's 64 heads into LDS (zero past H).  Every load of a
  // thread is issued before its first LDS store (one wave per SIMD leaves the
  // registers), so the row's 2 x 64 x D elements arrive in one round trip.
  {
    constexpr int PER = 2 * 64 * CPR / kRowsThreads;  // 16-byte chunks per thread (CPR is even)
    static_assert(2 * 64 * CPR % kRowsThreads == 0, "chunks must divide over the threads");
    u32x4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = i * kRowsThreads + static_cast<int>(threadIdx.x);
      const int m = e / (64 * CPR);
      const int h = (e / CPR) % 64;
      const int c = e % CPR;
      const int hq = hbase + h;
      const uint16_t* src = m == 0 ? a.q + b * a.qsb + static_cast<int64_t>(s) * a.qss + static_cast<int64_t>(hq) * a.qsh
                                   : a.dout + b * a.gsb + static_cast<int64_t>(s) * a.gss + static_cast<int64_t>(hq) * a.gsh;
      v[i] = hq < a.H ? *reinterpret_cast<const u32x4*>(src + c * 8) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = i * kRowsThreads + static_cast<int>(threadIdx.x);
      const int m = e / (64 * CPR);
      const int h = (e / CPR) % 64;
      const int c = e % CPR;
      *reinterpret_cast<u32x4*>(qd_lds + m * DS::QD + h * DS::QROW + c * 16) = v[i];
    }
  }
  const uint16_t* coef_row = a.coef + (static_cast<int64_t>(lrow) * a.HG + hg) * a.ntiles * kCoefTile;
  // Each thread moves 2 x 16 bytes of a tile's coefficient block.  The blocks
  // are fetched two tiles ahead into two alternating register sets, so the
  // wait before a block's LDS store leaves the previous and the current
  // tile's row stores (10 + 10 per thread at D = 576) in flight.
  u32x4 c0[2], c1[2];
  auto coef_load = [&](int t, u32x4 (&dst)[2]) {
    const u32x4* src = reinterpret_cast<const u32x4*>(coef_row + static_cast<int64_t>(t) * kCoefTile);
    dst[0] = src[threadIdx.x];
    dst[1] = src[threadIdx.x + kRowsThreads];
  };
  auto coef_store = [&](const u32x4 (&v)[2]) {
    reinterpret_cast<u32x4*>(coef_lds)[threadIdx.x] = v[0];
    reinterpret_cast<u32x4*>(coef_lds)[threadIdx.x + kRowsThreads] = v[1];
  };
  if (ntiles > 0) {
    coef_load(0, c0);
    coef_store(c0);
  }
  if (ntiles > 1) coef_load(1, c0);
  __syncthreads();

  // A-fragment source (Q or dO; 8 heads of one dimension per lane after two
  // reads): group g reads heads 8g + (i16 >> 2) (+4 for the second read),
  // dimensions 16 mbi + 4 (i16 & 3) + 0..3.  This wave's dimension blocks are
  // mbi = MBW wave + j.
  const uint32_t qd0 = lds_addr(qd_lds) + (8 * g + (i16 >> 2)) * DS::QROW + 8 * (i16 & 3) + wave * MBW * 32;
  // B-fragment source (P or dS; 8 heads of one key per lane after two reads):
  // heads h = 8g + (i16 >> 2) (+4) of a 32-head k-step and keys 16nb +
  // 4 (i16 & 3) + 0..3, which producer wave h >> 4, lane 16 (i16 & 3) +
  // (h & 15) holds at bytes 8nb..8nb+7 of its 16-byte fragment (the +4 heads
  // of the second read are 4 lanes further, in the same producer wave).
  const int bh = 8 * g + (i16 >> 2);
  const uint32_t cf0 = lds_addr(coef_lds) + ((bh >> 4) * 64 + (i16 & 3) * 16 + (bh & 15)) * 16;

  const int64_t prow_base = (static_cast<int64_t>(lrow) * a.HG + hg) * (static_cast<int64_t>(a.ntiles) * kAttnTK);

  // Tile t: fetch the block of tile t+2 into `ahead`, compute, then publish
  // the block of tile t+1 held in `held`.
  auto tile = [&](int t, u32x4 (&ahead)[2], const u32x4 (&held)[2]) {
    if (t + 2 < ntiles) coef_load(t + 2, ahead);
    // k-steps 0, 1: dS of heads 0..31, 32..63 against Q; 2, 3: P against dO
    bf16x8 bfr[4][2];
    auto b_read = [&](auto KC, auto NC) {
      constexpr int kst = decltype(KC)::value;
      constexpr int nb = decltype(NC)::value;
      constexpr int off = ((kst < 2 ? 1 : 0) * 4 + 2 * (kst & 1)) * 64 * 16 + 8 * nb;
      const v4i16 lo = tr_read<off>(cf0);
      const v4i16 hi = tr_read<off + 64>(cf0);
      bfr[kst][nb] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    attn_static_for<0, 4>([&](auto KC) { attn_static_for<0, 2>([&](auto NC) { b_read(KC, NC); }); });
    lds_wait_n<0>();
#pragma unroll
    for (int kst = 0; kst < 4; ++kst)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) reg_tie(bfr[kst][nb]);

    // A fragments of block j, double-buffered: block j+1's reads run under
    // block j's MFMAs
    v4i16 alo[2][4], ahi[2][4];
    auto a_read = [&](auto JC) {
      constexpr int j = decltype(JC)::value;
#pragma unroll
      for (int kst = 0; kst < 4; ++kst) {
        const uint32_t base = qd0 + (kst >> 1) * DS::QD + (kst & 1) * 32 * DS::QROW;
        alo[j & 1][kst] = tr_read<j * 32>(base);
        ahi[j & 1][kst] = tr_read<j * 32 + 4 * DS::QROW>(base);
      }
    };
    if (DS::MBT % 4 == 0 || wave * MBW < DS::MBT) a_read(std::integral_constant<int, 0>{});
    uint2 pend[2];  // packed rows of an even block, stored with the next block
    static_assert(DS::MBT % 4 == 0 || MBW == 1, "both blocks of a stored pair are inside the row");
    auto block = [&](auto JC) {
      constexpr int j = decltype(JC)::value;
      lds_wait_n<0>();
#pragma unroll
      for (int kst = 0; kst < 4; ++kst) {
        reg_tie(alo[j & 1][kst]);
        reg_tie(ahi[j & 1][kst]);
      }
      if constexpr (j + 1 < MBW) {
        if (DS::MBT % 4 == 0 || wave * MBW + j + 1 < DS::MBT) a_read(std::integral_constant<int, j + 1>{});
      }
      const int mbi = wave * MBW + j;
      if (DS::MBT % 4 == 0 || mbi < DS::MBT) {
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int kst = 0; kst < 4; ++kst) {
          const bf16x8 af =
              __builtin_bit_cast(bf16x8, __builtin_shufflevector(alo[j & 1][kst], ahi[j & 1][kst], 0, 1, 2, 3, 4, 5, 6, 7));
          acc[0] = mfma16x16x32<F16>(af, bfr[kst][0], acc[0]);
          acc[1] = mfma16x16x32<F16>(af, bfr[kst][1], acc[1]);
        }
        // lane (key 16nb + i16, g) holds dimensions 16 mbi + 4g + 0..3.  Every
        // slot of the padded tile is written: a masked or padding slot has
        // P = dS = 0 and no key, so the reduction never reads its row, and
        // unconditional stores keep the prefetch waits exact.
        uint2 w[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          w[nb].x = pack2<F16>(acc[nb][0], acc[nb][1]);
          w[nb].y = pack2<F16>(acc[nb][2], acc[nb][3]);
        }
        if constexpr (j % 2 == 0 && j + 1 < MBW) {
          // held until block j+1 (the next 16 dimensions of the same keys)
          pend[0] = w[0];
          pend[1] = w[1];
        } else if constexpr (j % 2 == 1) {
          // Blocks j-1 and j regrouped so that lane group g holds 16 bytes:
          // dimensions 16 mbi(j-1) + 8g + 0..7 of its key (a permlane32 swap
          // pairs the blocks' lane halves, a permlane16 swap the lane groups);
          // each store then writes 64 contiguous bytes of 16 keys.
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const auto sx = __builtin_amdgcn_permlane32_swap(pend[nb].x, w[nb].x, false, false);
            const auto sy = __builtin_amdgcn_permlane32_swap(pend[nb].y, w[nb].y, false, false);
            const auto tx = __builtin_amdgcn_permlane16_swap(sx[0], sx[1], false, false);
            const auto ty = __builtin_amdgcn_permlane16_swap(sy[0], sy[1], false, false);
            u32x4 v;
            v[0] = tx[0];
            v[1] = ty[0];
            v[2] = tx[1];
            v[3] = ty[1];
            *reinterpret_cast<u32x4*>(a.prow + (prow_base + t * kAttnTK + nb * 16 + i16) * D + (mbi - 1) * 16 + 8 * g) = v;
          }
        } else {
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
            *reinterpret_cast<uint2*>(a.prow + (prow_base + t * kAttnTK + nb * 16 + i16) * D + mbi * 16 + 4 * g) = w[nb];
        }
      }
    };
    attn_static_for<0, MBW>(block);
    // Barriers without a release fence: they order only LDS (the row stores
    // need no ordering), so the stores of this tile stay in flight.
    attn_tile_barrier();  // every wave is done with this tile's coefficients
    if (t + 1 < ntiles) coef_store(held);
    attn_tile_barrier();
  };
  for (int t = 0; t < ntiles; t += 2) {
    tile(t, c1, c0);
    if (t + 1 < ntiles) tile(t + 1, c0, c1);
  }
}

// ---------------------------------------------------------------------------
// 3. key-major reduction of the dkv rows
// ---------------------------------------------------------------------------
struct DkvReduceArgs {
  const uint32_t* pair;   // pair ids of the sort group (lrow K + j, lrow counted from the group's first row)
  const int32_t* seg_lo;  // per key id b N + t: its pairs in this chunk are pair[seg_lo, seg_hi)
  const int32_t* seg_hi;
  const uint16_t* prow;   // [nrows, HG, KP, D]
  float* acc;             // [B N, D] running fp32 sum across chunks
  uint16_t* dkv;          // [B, N, D] bf16
  int64_t dsb, dsn;
  int64_t prow0;          // the chunk's first row, counted from the group's first row
  int K, KP, HG, N;      // KP: slots per (row, head group), K rounded up to whole tiles
  int first, last;        // first / last chunk of query rows
};

// Reduction workgroup per key: 256 threads, G = 256 / CPR groups of CPR
// threads (one 16-byte chunk of a row each); each group keeps 8 rows in
// flight, so a long segment (a key picked by many queries, such as a
// compressed KV row, collects as many rows as the chunk has queries) streams
// 8 G rows at a time.
template <int D>
struct ReduceShape {
  static constexpr int CPR = D / 8;
  static constexpr int G = 256 / CPR;
  static constexpr int NT = 256;
};

template <int D, bool F16>
__global__ __launch_bounds__(ReduceShape<D>::NT) void sparse_attn_bwd_dkv_reduce_kernel(DkvReduceArgs r) {
  constexpr int CPR = ReduceShape<D>::CPR;    // 16-byte chunks per row
  constexpr int G = ReduceShape<D>::G;        // pair groups
  __shared__ float red[G * D];
  // Keys in reverse: in [kv ; kv_compressed] layouts the compressed rows,
  // each selected by many queries, are the last keys, and their long
  // segments start first instead of forming the grid's tail.
  const int kid = static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x);
  const int grp = threadIdx.x / CPR;
  const int c = threadIdx.x % CPR;
  float* accp = r.acc + static_cast<int64_t>(kid) * D + c * 8;
  const int lo = r.seg_lo[kid], hi = r.seg_hi[kid];
  // A key that no query of this chunk selects keeps its running sum where it
  // is (the first chunk still writes its zeros, the last its dkv row): with
  // window and compressed keys, most of the keys of a chunk of queries are
  // such keys, and rewriting their sums would move 2 x 4 x D bytes each.
  if (lo == hi && !r.first && !r.last) return;
  // The running sum of the earlier chunks is read before the rows, so that
  // its load overlaps the segment's row loads instead of following them.
  float prev[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (!r.first && threadIdx.x < CPR) {
    const f32x4 a0 = *reinterpret_cast<const f32x4*>(accp);
    const f32x4 a1 = *reinterpret_cast<const f32x4*>(accp + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      prev[e] = a0[e];
      prev[4 + e] = a1[e];
    }
  }
  float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  {
    auto add_row = [&](int p) {
      const uint32_t pid = r.pair[p];
      const int64_t lrow = pid / static_cast<uint32_t>(r.K) - r.prow0;
      const int64_t j = pid % static_cast<uint32_t>(r.K);
      for (int h = 0; h < r.HG; ++h) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(r.prow + ((lrow * r.HG + h) * r.KP + j) * D + c * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sum[2 * e] += elem_lo<F16>(v[e]);
          sum[2 * e + 1] += elem_hi<F16>(v[e]);
        }
      }
    };
    int p = lo + grp;
    if (grp < G) {
      if (r.HG == 1) {
        // one head group: 8 independent row loads in flight, and the next 8
        // pair ids loaded behind them, so that a long segment waits for one
        // memory round trip per 8 rows instead of two
        uint32_t pid[8];
        if (p + 7 * G < hi) {
#pragma unroll
          for (int u = 0; u < 8; ++u) pid[u] = r.pair[p + u * G];
        }
        for (; p + 7 * G < hi; p += 8 * G) {
          u32x4 v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int64_t lrow = pid[u] / static_cast<uint32_t>(r.K) - r.prow0;
            const int64_t j = pid[u] % static_cast<uint32_t>(r.K);
            v[u] = *reinterpret_cast<const u32x4*>(r.prow + (lrow * r.KP + j) * D + c * 8);
          }
          if (p + 15 * G < hi) {
#pragma unroll
            for (int u = 0; u < 8; ++u) pid[u] = r.pair[p + 8 * G + u * G];
          }
#pragma unroll
          for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              sum[2 * e] += elem_lo<F16>(v[u][e]);
              sum[2 * e + 1] += elem_hi<F16>(v[u][e]);
            }
        }
        // The group's last (at most 7) rows as one round rather than one
        // round trip pair each: the same rows, added in the same order.  The
        // loads are unconditional (a slot past the segment reads the round's
        // first row again) and a select keeps those slots out of the sums, so
        // no branch splits the loads apart.
        if (p < hi) {
          const int n = (hi - p + G - 1) / G;
          uint32_t pr[7];
          u32x4 vr[7];
#pragma unroll
          for (int u = 0; u < 7; ++u) pr[u] = r.pair[u < n ? p + u * G : p];
#pragma unroll
          for (int u = 0; u < 7; ++u) {
            const int64_t lrow = pr[u] / static_cast<uint32_t>(r.K) - r.prow0;
            const int64_t j = pr[u] % static_cast<uint32_t>(r.K);
            vr[u] = *reinterpret_cast<const u32x4*>(r.prow + (lrow * r.KP + j) * D + c * 8);
          }
#pragma unroll
          for (int u = 0; u < 7; ++u) {
            const bool in = u < n;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float lo_v = sum[2 * e] + elem_lo<F16>(vr[u][e]);
              const float hi_v = sum[2 * e + 1] + elem_hi<F16>(vr[u][e]);
              sum[2 * e] = in ? lo_v : sum[2 * e];
              sum[2 * e + 1] = in ? hi_v : sum[2 * e + 1];
            }
          }
          p = hi;
        }
      } else {
        for (; p + 7 * G < hi; p += 8 * G) {
#pragma unroll
          for (int u = 0; u < 8; ++u) add_row(p + u * G);
        }
      }
      for (; p < hi; p += G) add_row(p);
    }
    if (grp < G) {
#pragma unroll
      for (int e = 0; e < 8; ++e) red[grp * D + c * 8 + e] = sum[e];
    }
  }
  __syncthreads();
  if (threadIdx.x < CPR) {
    float tot[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = 0.f;
      for (int q = 0; q < G; ++q) v += red[q * D + c * 8 + e];
      tot[e] = v;
    }
    if (!r.first) {
#pragma unroll
      for (int e = 0; e < 8; ++e) tot[e] += prev[e];
    }
    if (!r.last) {
#pragma unroll
      for (int e = 0; e < 8; ++e) accp[e] = tot[e];
    } else {
      const int b = kid / r.N, t = kid % r.N;
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = pack2<F16>(tot[2 * e], tot[2 * e + 1]);
      *reinterpret_cast<u32x4*>(r.dkv + b * r.dsb + static_cast<int64_t>(t) * r.dsn + c * 8) = w;
    }
  }
}

// Sort keys and payloads of a sort group's (query, slot) pairs, the group
// being consecutive chunks of chunk_rows query rows from row0: the key of the
// pair in chunk c is c (nkeys + 1) + (b N + t) for a valid index t, and
// c (nkeys + 1) + nkeys (sorted after the chunk's keys, never reduced)
// otherwise.  One sort then orders the pairs by chunk, then key, then pair id.
__global__ void sparse_attn_bwd_pairs_kernel(const void* idx, int idx64, int64_t isb, int64_t iss, int64_t isk,
                                             int S, int N, int K, int64_t row0, int64_t n, uint32_t nkeys,
                                             int64_t chunk_rows, const int32_t* row_len, int64_t rlsb, int64_t rlss,
                                             uint32_t* keys, uint32_t* vals) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const int64_t lrow = p / K;
  const int j = static_cast<int>(p % K);
  const int64_t grow = row0 + lrow;
  const int64_t b = grow / S, s = grow % S;
  const int64_t off = b * isb + s * iss + j * isk;
  const int64_t raw = idx64 ? static_cast<const int64_t*>(idx)[off] : static_cast<int64_t>(static_cast<const int32_t*>(idx)[off]);
  const bool in_row = !row_len || j < row_len[b * rlsb + s * rlss];
  const uint32_t key = (in_row && raw >= 0 && raw < N) ? static_cast<uint32_t>(b * N + raw) : nkeys;
  keys[p] = static_cast<uint32_t>(lrow / chunk_rows) * (nkeys + 1u) + key;
  vals[p] = static_cast<uint32_t>(p);
}

__global__ void sparse_attn_bwd_fill_kernel(int32_t* dst, int64_t n, int32_t v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dst[i] = v;
}

// Each (chunk c, key k) run [seg_lo, seg_hi) in the sorted pair list, stored
// at c nkeys + k (keys without pairs keep the empty run 0, 0 from the fill).
__global__ void sparse_attn_bwd_segments_kernel(const uint32_t* sk, int64_t n, uint32_t nkeys, int32_t* lo, int32_t* hi) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint32_t key = sk[p];
  const uint32_t c = key / (nkeys + 1u), k = key % (nkeys + 1u);
  if (k >= nkeys) return;
  const int64_t at = static_cast<int64_t>(c) * nkeys + k;
  if (p == 0 || sk[p - 1] != key) lo[at] = static_cast<int32_t>(p);
  if (p == n - 1 || sk[p + 1] != key) hi[at] = static_cast<int32_t>(p + 1);
}

// dsink[h] = sum over rows of the per-row terms, in a fixed order.
__global__ __launch_bounds__(256) void sparse_attn_bwd_dsink_kernel(const float* rows, int64_t nrows, int stride,
                                                                     float* dsink) {
  __shared__ float red[256];
  const int h = blockIdx.x;
  float v = 0.f;
  for (int64_t r = threadIdx.x; r < nrows; r += 256) v += rows[r * stride + h];
  red[threadIdx.x] = v;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) dsink[h] = red[0];
}

// bf16 zeros for dkv when no key can be selected (K = 0 or N = 0).
__global__ void sparse_attn_bwd_zero_dkv_kernel(uint16_t* dkv, int64_t dsb, int64_t dsn, int N, int D, int64_t total) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t d = i % D, t = (i / D) % N, b = i / (static_cast<int64_t>(D) * N);
    dkv[b * dsb + t * dsn + d] = 0;
  }
}

// ---------------------------------------------------------------------------
// host side: workspace plan and launches
// ---------------------------------------------------------------------------
static size_t bwd_align(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct BwdPlan {
  int64_t rows;   // query rows per chunk
  int64_t group;  // chunks per sort group (their pairs are sorted by one radix sort)
  unsigned end_bit;
  size_t dsink_rows, acc, seg_lo, seg_hi, coef, prow, kin, kout, vin, vout, tmp, tmp_bytes, total;
};

static unsigned bwd_end_bit(int64_t max_key) {
  unsigned bits = 1;
  while ((int64_t{1} << bits) <= max_key) ++bits;  // keys 0 .. max_key
  return bits;
}

// Workspace layout for chunks of `rows` query rows sorted `group` chunks at a
// time.  The sort's inputs and its temporary storage share one region with
// the chunk's coefficient tiles and dkv rows: a group is sorted before its
// first chunk runs, after the previous group's last chunk has finished.
static int bwd_plan(int64_t B, int64_t S, int64_t H, int64_t D, int64_t N, int64_t K, int64_t rows, int64_t group,
                    BwdPlan* p) {
  const int64_t HG = (H + 63) / 64;
  const int64_t ntiles = N > 0 ? (K + kAttnTK - 1) / kAttnTK : 0;
  const int64_t nkeys = B * N;
  const int64_t total_rows = B * S;
  const bool chunked = rows < total_rows;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = bwd_align(off + bytes);
    return at;
  };
  p->rows = rows;
  p->group = group;
  p->end_bit = bwd_end_bit(group * (nkeys + 1) - 1);
  p->dsink_rows = take(static_cast<size_t>(total_rows) * 64 * HG * 4);
  p->acc = take(chunked ? static_cast<size_t>(nkeys) * D * 4 : 0);
  const size_t npairs = ntiles > 0 ? static_cast<size_t>(rows) * group * K : 0;
  p->seg_lo = take(static_cast<size_t>(nkeys) * group * 4);
  p->seg_hi = take(static_cast<size_t>(nkeys) * group * 4);
  p->kout = take(npairs * 4);
  p->vout = take(npairs * 4);
  const size_t shared = off;
  p->coef = take(static_cast<size_t>(rows) * HG * ntiles * kCoefTile * 2);
  p->prow = take(static_cast<size_t>(rows) * HG * ntiles * kAttnTK * D * 2);
  const size_t chunk_end = off;
  off = shared;
  p->kin = take(npairs * 4);
  p->vin = take(npairs * 4);
  size_t tmp = 0;
  if (npairs > 0) {
    const hipError_t e = rocprim::radix_sort_pairs(nullptr, tmp, static_cast<uint32_t*>(nullptr),
                                                   static_cast<uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
                                                   static_cast<uint32_t*>(nullptr), npairs, 0u, p->end_bit,
                                                   static_cast<hipStream_t>(0));
    if (e != hipSuccess) return set_error(SI_ERR_LAUNCH, std::string("radix sort size query: ") + hipGetErrorString(e));
  }
  p->tmp_bytes = tmp;
  p->tmp = take(tmp);
  p->total = off > chunk_end ? off : chunk_end;
  return SI_OK;
}

// Largest chunk (query rows) whose plan fits `bytes`; 0 when even one row does
// not.  A chunk and a sort group keep their (query, slot) pairs and a chunk its
// grid (rows x head groups) inside int32, and a group's sort keys inside 32
// bits.  The sort groups take up to a quarter of the budget (pairs and segment
// bounds), so that a small workspace is not paid for with one radix sort (a
// few kernels of fixed cost) per chunk.
static int bwd_rows_for(int64_t B, int64_t S, int64_t H, int64_t D, int64_t N, int64_t K, size_t bytes, BwdPlan* out) {
  const int64_t HG = (H + 63) / 64;
  const int64_t nkeys = B * N;
  int64_t total = B * S;
  BwdPlan p{};
  if (total <= 0) return bwd_plan(B, S, H, D, N, K, 0, 1, out);
  const int64_t kLim = 0x7fffffff;
  const int64_t kpairs = K > 0 ? K : 1;
  int64_t cap = kLim / kpairs;
  if (kLim / HG < cap) cap = kLim / HG;
  if (total > cap) total = cap;
  int rc = bwd_plan(B, S, H, D, N, K, total, 1, &p);
  if (rc) return rc;
  if (p.total <= bytes && total == B * S) {
    *out = p;
    return SI_OK;
  }
  auto group_for = [&](int64_t rows) {
    const int64_t chunks = (B * S + rows - 1) / rows;
    int64_t g = static_cast<int64_t>(bytes / 4) / (rows * kpairs * 8 + nkeys * 8 + 1);
    if (g > chunks) g = chunks;
    if (g > kLim / (rows * kpairs)) g = kLim / (rows * kpairs);
    if (g > (int64_t{1} << 32) / (nkeys + 1)) g = (int64_t{1} << 32) / (nkeys + 1);
    return g < 1 ? int64_t{1} : g;
  };
  int64_t lo = 0, hi = total + 1;  // plan(lo) fits (lo = 0: nothing fits yet), plan(hi) does not
  while (hi - lo > 1) {
    const int64_t mid = lo + (hi - lo) / 2;
    rc = bwd_plan(B, S, H, D, N, K, mid, group_for(mid), &p);
    if (rc) return rc;
    if (p.total <= bytes) lo = mid; else hi = mid;
  }
  return bwd_plan(B, S, H, D, N, K, lo, lo > 0 ? group_for(lo) : 1, out);
}

template <int D, bool F16>
static int launch_bwd(AttnBwdArgs a, const BwdPlan& pl, char* ws, int64_t total_rows, uint16_t* dkv, int64_t dkvsb,
                      int64_t dkvsn, float* dsink, hipStream_t st) {
  const int64_t nkeys = static_cast<int64_t>(a.B) * a.N;
  a.dsink_rows = reinterpret_cast<float*>(ws + pl.dsink_rows);
  a.coef = reinterpret_cast<uint16_t*>(ws + pl.coef);
  a.prow = reinterpret_cast<uint16_t*>(ws + pl.prow);
  uint32_t* kin = reinterpret_cast<uint32_t*>(ws + pl.kin);
  uint32_t* kout = reinterpret_cast<uint32_t*>(ws + pl.kout);
  uint32_t* vin = reinterpret_cast<uint32_t*>(ws + pl.vin);
  uint32_t* vout = reinterpret_cast<uint32_t*>(ws + pl.vout);
  int32_t* seg_lo = reinterpret_cast<int32_t*>(ws + pl.seg_lo);
  int32_t* seg_hi = reinterpret_cast<int32_t*>(ws + pl.seg_hi);
  int rc;
  // No (row, key) pair contributes when there are no key tiles or no query
  // rows: dkv is all zeros and the chunk loop below never writes it.
  if ((a.ntiles == 0 || total_rows == 0) && nkeys > 0) {
    const int64_t tot = nkeys * D;
    const int64_t blocks = (tot + 255) / 256 < 65536 ? (tot + 255) / 256 : 65536;
    hipLaunchKernelGGL(sparse_attn_bwd_zero_dkv_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, dkv,
                       dkvsb, dkvsn, a.N, D, tot);
    if ((rc = check_launch("sparse_attn_bwd_zero_dkv_kernel"))) return rc;
  }
  const int64_t grows_max = pl.rows * pl.group;
  for (int64_t g0 = 0; g0 < total_rows; g0 += grows_max) {
    const int64_t grows = total_rows - g0 < grows_max ? total_rows - g0 : grows_max;
    const int64_t gchunks = (grows + pl.rows - 1) / pl.rows;
    if (a.ntiles > 0) {
      // the group's pairs, sorted by (chunk, key, pair id), and each
      // (chunk, key)'s run in that order
      const int64_t npairs = grows * a.K;
      const unsigned pblocks = static_cast<unsigned>((npairs + 255) / 256);
      hipLaunchKernelGGL(sparse_attn_bwd_pairs_kernel, dim3(pblocks), dim3(256), 0, st, a.idx, a.idx64, a.isb, a.iss,
                         a.isk, a.S, a.N, a.K, g0, npairs, static_cast<uint32_t>(nkeys), pl.rows, a.row_len, a.rlsb,
                         a.rlss, kin, vin);
      if ((rc = check_launch("sparse_attn_bwd_pairs_kernel"))) return rc;
      size_t tmp_bytes = pl.tmp_bytes;
      const hipError_t e = rocprim::radix_sort_pairs(ws + pl.tmp, tmp_bytes, kin, kout, vin, vout,
                                                     static_cast<size_t>(npairs), 0u, pl.end_bit, st);
      if (e != hipSuccess) return set_error(SI_ERR_LAUNCH, std::string("radix sort: ") + hipGetErrorString(e));
      const int64_t nseg = gchunks * nkeys;
      const int64_t fblocks = (nseg + 255) / 256 < 65536 ? (nseg + 255) / 256 : 65536;
      hipLaunchKernelGGL(sparse_attn_bwd_fill_kernel, dim3(static_cast<unsigned>(fblocks)), dim3(256), 0, st, seg_lo,
                         nseg, 0);
      hipLaunchKernelGGL(sparse_attn_bwd_fill_kernel, dim3(static_cast<unsigned>(fblocks)), dim3(256), 0, st, seg_hi,
                         nseg, 0);
      if ((rc = check_launch("sparse_attn_bwd_fill_kernel"))) return rc;
      hipLaunchKernelGGL(sparse_attn_bwd_segments_kernel, dim3(pblocks), dim3(256), 0, st, kout, npairs,
                         static_cast<uint32_t>(nkeys), seg_lo, seg_hi);
      if ((rc = check_launch("sparse_attn_bwd_segments_kernel"))) return rc;
    }
    for (int64_t c = 0; c < gchunks; ++c) {
      const int64_t row0 = g0 + c * pl.rows;
      const int64_t nr = total_rows - row0 < pl.rows ? total_rows - row0 : pl.rows;
      a.row0 = row0;
      a.nrows = static_cast<int>(nr);
      const unsigned grid = static_cast<unsigned>(nr * a.HG);
      if (a.idx64)
        hipLaunchKernelGGL((sparse_attn_bwd_rows_kernel<D, true, F16>), dim3(grid), dim3(kBwdThreads), 0, st, a);
      else
        hipLaunchKernelGGL((sparse_attn_bwd_rows_kernel<D, false, F16>), dim3(grid), dim3(kBwdThreads), 0, st, a);
      if ((rc = check_launch("sparse_attn_bwd_rows_kernel"))) return rc;
      if (a.ntiles == 0) continue;
      hipLaunchKernelGGL((sparse_attn_bwd_dkv_rows_kernel<D, F16>), dim3(grid), dim3(kRowsThreads), 0, st, a);
      if ((rc = check_launch("sparse_attn_bwd_dkv_rows_kernel"))) return rc;
      DkvReduceArgs r{};
      r.pair = vout;
      r.seg_lo = seg_lo + c * nkeys;
      r.seg_hi = seg_hi + c * nkeys;
      r.prow = a.prow;
      r.acc = reinterpret_cast<float*>(ws + pl.acc);
      r.dkv = dkv;
      r.dsb = dkvsb;
      r.dsn = dkvsn;
      r.prow0 = c * pl.rows;
      r.K = a.K;
      r.KP = a.ntiles * kAttnTK;
      r.HG = a.HG;
      r.N = a.N;
      r.first = row0 == 0;
      r.last = row0 + nr >= total_rows;
      hipLaunchKernelGGL((sparse_attn_bwd_dkv_reduce_kernel<D, F16>), dim3(static_cast<unsigned>(nkeys)),
                         dim3(ReduceShape<D>::NT), 0, st, r);
      if ((rc = check_launch("sparse_attn_bwd_dkv_reduce_kernel"))) return rc;
    }
  }
  hipLaunchKernelGGL(sparse_attn_bwd_dsink_kernel, dim3(static_cast<unsigned>(a.H)), dim3(256), 0, st, a.dsink_rows,
                     total_rows, 64 * a.HG, dsink);
  return check_launch("sparse_attn_bwd_dsink_kernel");
}

// ---------------------------------------------------------------------------
// inverted top-k index (flash_sparse/triton/inverted_topk.py:75-128)
// ---------------------------------------------------------------------------
// For key id b N + t: inv_count = its number of (query, slot) pairs, and the
// first min(count, k_max) entries of its inv_topk row the queries of those
// pairs in ascending (query, slot) order (the stable sort's order); the
// remaining entries are -1.
__global__ void inverted_fill_kernel(const uint32_t* pair, const int32_t* lo, const int32_t* hi, int64_t nkeys,
                                     int S, int K, int k_max, int32_t* inv_topk, int32_t* inv_count) {
  const int64_t kid = blockIdx.x;
  if (kid >= nkeys) return;
  const int a = lo[kid], c = hi[kid] - lo[kid];
  if (threadIdx.x == 0) inv_count[kid] = c;
  int32_t* row = inv_topk + kid * k_max;
  for (int j = threadIdx.x; j < k_max; j += blockDim.x)
    row[j] = j < c ? static_cast<int32_t>((pair[a + j] / static_cast<uint32_t>(K)) % static_cast<uint32_t>(S)) : -1;
}

struct InvPlan {
  size_t seg_lo, seg_hi, kin, kout, vin, vout, tmp, tmp_bytes, total;
};

static int inv_plan(int64_t B, int64_t S, int64_t K, int64_t N, InvPlan* p) {
  const int64_t nkeys = B * N;
  const size_t npairs = static_cast<size_t>(B) * S * K;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = bwd_align(off + bytes);
    return at;
  };
  p->seg_lo = take(static_cast<size_t>(nkeys) * 4);
  p->seg_hi = take(static_cast<size_t>(nkeys) * 4);
  p->kin = take(npairs * 4);
  p->kout = take(npairs * 4);
  p->vin = take(npairs * 4);
  p->vout = take(npairs * 4);
  size_t tmp = 0;
  if (npairs > 0) {
    const hipError_t e = rocprim::radix_sort_pairs(nullptr, tmp, static_cast<uint32_t*>(nullptr),
                                                   static_cast<uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
                                                   static_cast<uint32_t*>(nullptr), npairs, 0u, bwd_end_bit(nkeys),
                                                   static_cast<hipStream_t>(0));
    if (e != hipSuccess) return set_error(SI_ERR_LAUNCH, std::string("radix sort size query: ") + hipGetErrorString(e));
  }
  p->tmp_bytes = tmp;
  p->tmp = take(tmp);
  p->total = off;
  return SI_OK;
}

static bool bwd_supported_d(int64_t D) {
  return D == 32 || D == 64 || D == 128 || D == 256 || D == 512 || D == 576;
}

}  // namespace si

using namespace si;

extern "C" int64_t si_sparse_attn_bwd_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t D, int64_t N_kv,
                                                      int64_t K, int64_t max_bytes) {
  if (B < 0 || S < 0 || H <= 0 || D <= 0 || N_kv < 0 || K < 0 || max_bytes < 0) {
    set_error(SI_ERR_INVALID, "bad dimension");
    return -1;
  }
  if (!bwd_supported_d(D)) {
    set_error(SI_ERR_UNSUPPORTED, "unsupported head dim D=" + std::to_string(D));
    return -1;
  }
  if (B * N_kv >= (int64_t{1} << 31) || B * S >= (int64_t{1} << 31) || K > 0x7fffffff) {
    set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
    return -1;
  }
  BwdPlan p{};
  int rc = bwd_rows_for(B, S, H, D, N_kv, K, static_cast<size_t>(max_bytes), &p);
  if (rc) return -1;
  if (p.rows == 0 && B * S > 0) {  // not even one row fits: report the one-row need
    rc = bwd_plan(B, S, H, D, N_kv, K, 1, 1, &p);
    if (rc) return -1;
  }
  return static_cast<int64_t>(p.total);
}

extern "C" int si_sparse_attn_bwd_ragged(const void* q, const int64_t* q_strides, const void* kv,
                                         const int64_t* kv_strides, const float* attn_sink, const void* topk_idxs,
                                         int idx_is_i64, const int64_t* idx_strides, const void* o,
                                         const int64_t* o_strides, const float* lse, const int64_t* lse_strides,
                                         const void* dout, const int64_t* do_strides, int64_t B, int64_t S, int64_t H,
                                         int64_t D, int64_t N_kv, int64_t K, float softmax_scale, int qkv_dtype,
                                         void* dq, const int64_t* dq_strides, void* dkv, const int64_t* dkv_strides,
                                         float* dsink, void* workspace, int64_t workspace_bytes,
                                         const int32_t* row_len, const int64_t* row_len_strides, void* stream) {
  if (row_len && !row_len_strides) return set_error(SI_ERR_INVALID, "null row_len strides");
  if (qkv_dtype != SI_DTYPE_BF16 && qkv_dtype != SI_DTYPE_F16)
    return set_error(SI_ERR_INVALID, "qkv_dtype must be SI_DTYPE_BF16 (0) or SI_DTYPE_F16 (1)");
  if (!q_strides || !kv_strides || !idx_strides || !o_strides || !lse_strides || !do_strides || !dq_strides ||
      !dkv_strides)
    return set_error(SI_ERR_INVALID, "null stride argument");
  if (B < 0 || S < 0 || H <= 0 || D <= 0 || N_kv < 0 || K < 0 || workspace_bytes < 0)
    return set_error(SI_ERR_INVALID, "bad dimension");
  const bool rows = B > 0 && S > 0;
  if (rows && (!q || !attn_sink || !o || !lse || !dout || !dq || (K > 0 && !topk_idxs) || (N_kv > 0 && !kv)))
    return set_error(SI_ERR_INVALID, "null pointer argument");
  if (!dsink || (B > 0 && N_kv > 0 && !dkv)) return set_error(SI_ERR_INVALID, "null pointer argument");
  if (B * N_kv >= (int64_t{1} << 31) || B * S >= (int64_t{1} << 31) || K > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (H > 0x7fffffff) return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (!bwd_supported_d(D))
    return set_error(SI_ERR_UNSUPPORTED,
                     "unsupported head dim D=" + std::to_string(D) + " (supported: 32, 64, 128, 256, 512, 576)");
  if (q_strides[3] != 1 || kv_strides[2] != 1 || o_strides[3] != 1 || do_strides[3] != 1 || dq_strides[3] != 1 ||
      dkv_strides[2] != 1)
    return set_error(SI_ERR_INVALID, "q, kv, o, do, dq and dkv need a contiguous last dimension");
  if ((q_strides[0] | q_strides[1] | q_strides[2] | kv_strides[0] | kv_strides[1] | o_strides[0] | o_strides[1] |
       o_strides[2] | do_strides[0] | do_strides[1] | do_strides[2] | dq_strides[0] | dq_strides[1] | dq_strides[2] |
       dkv_strides[0] | dkv_strides[1]) % 8)
    return set_error(SI_ERR_INVALID, "strides must be multiples of 8 elements");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kv) | reinterpret_cast<uintptr_t>(o) |
       reinterpret_cast<uintptr_t>(dout) | reinterpret_cast<uintptr_t>(dq) | reinterpret_cast<uintptr_t>(dkv) |
       reinterpret_cast<uintptr_t>(workspace)) & 15)
    return set_error(SI_ERR_INVALID, "tensors and the workspace must be 16-byte aligned");
  if (N_kv > 0 && ((N_kv - 1) * kv_strides[1] + D) / 8 >= (int64_t{1} << 32))
    return set_error(SI_ERR_UNSUPPORTED, "kv batch larger than 64 GiB");
  BwdPlan pl{};
  int rc = bwd_rows_for(B, S, H, D, N_kv, K, static_cast<size_t>(workspace_bytes), &pl);
  if (rc) return rc;
  if (pl.rows == 0 && B * S > 0)
    return set_error(SI_ERR_INVALID, "workspace too small (see si_sparse_attn_bwd_workspace_bytes)");
  if (pl.total > 0 && !workspace) return set_error(SI_ERR_INVALID, "null workspace");

  AttnBwdArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qsb = q_strides[0]; a.qss = q_strides[1]; a.qsh = q_strides[2];
  a.kv = static_cast<const uint16_t*>(kv);
  a.kvsb = kv_strides[0]; a.kvsn = kv_strides[1];
  a.sink = attn_sink;
  a.idx = topk_idxs;
  a.isb = idx_strides[0]; a.iss = idx_strides[1]; a.isk = idx_strides[2];
  a.o = static_cast<const uint16_t*>(o);
  a.osb = o_strides[0]; a.oss = o_strides[1]; a.osh = o_strides[2];
  a.dout = static_cast<const uint16_t*>(dout);
  a.gsb = do_strides[0]; a.gss = do_strides[1]; a.gsh = do_strides[2];
  a.lse = lse;
  a.lsb = lse_strides[0]; a.lss = lse_strides[1]; a.lsh = lse_strides[2];
  a.dq = static_cast<uint16_t*>(dq);
  a.dqsb = dq_strides[0]; a.dqss = dq_strides[1]; a.dqsh = dq_strides[2];
  a.B = static_cast<int>(B); a.S = static_cast<int>(S); a.H = static_cast<int>(H);
  a.N = static_cast<int>(N_kv); a.K = static_cast<int>(K);
  a.HG = static_cast<int>((H + 63) / 64);
  a.ntiles = N_kv > 0 ? static_cast<int>((K + kAttnTK - 1) / kAttnTK) : 0;
  a.row_len = row_len;
  if (row_len) {
    a.rlsb = row_len_strides[0];
    a.rlss = row_len_strides[1];
  }
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.idx64 = idx_is_i64 ? 1 : 0;
  a.f16 = qkv_dtype == SI_DTYPE_F16 ? 1 : 0;
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t* dkvp = static_cast<uint16_t*>(dkv);
  const int64_t total_rows = B * S;
  auto run = [&](auto DC) {
    constexpr int DD = decltype(DC)::value;
    return a.f16 ? launch_bwd<DD, true>(a, pl, ws, total_rows, dkvp, dkv_strides[0], dkv_strides[1], dsink, st)
                 : launch_bwd<DD, false>(a, pl, ws, total_rows, dkvp, dkv_strides[0], dkv_strides[1], dsink, st);
  };
  switch (D) {
    case 32: return run(std::integral_constant<int, 32>{});
    case 64: return run(std::integral_constant<int, 64>{});
    case 128: return run(std::integral_constant<int, 128>{});
    case 256: return run(std::integral_constant<int, 256>{});
    case 512: return run(std::integral_constant<int, 512>{});
    default: return run(std::integral_constant<int, 576>{});
  }
}

extern "C" int si_sparse_attn_bwd(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                                  const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                                  const int64_t* idx_strides, const void* o, const int64_t* o_strides, const float* lse,
                                  const int64_t* lse_strides, const void* dout, const int64_t* do_strides, int64_t B,
                                  int64_t S, int64_t H, int64_t D, int64_t N_kv, int64_t K, float softmax_scale,
                                  int qkv_dtype, void* dq, const int64_t* dq_strides, void* dkv,
                                  const int64_t* dkv_strides, float* dsink, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  return si_sparse_attn_bwd_ragged(q, q_strides, kv, kv_strides, attn_sink, topk_idxs, idx_is_i64, idx_strides, o,
                                   o_strides, lse, lse_strides, dout, do_strides, B, S, H, D, N_kv, K, softmax_scale,
                                   qkv_dtype, dq, dq_strides, dkv, dkv_strides, dsink, workspace, workspace_bytes,
                                   nullptr, nullptr, stream);
}

static int inv_check(int64_t B, int64_t S, int64_t K, int64_t N, int64_t k_max) {
  if (B < 0 || S < 0 || K < 0 || N < 0 || k_max < 0) return set_error(SI_ERR_INVALID, "bad dimension");
  // pair positions (segment bounds) are int32
  if (B * N >= (int64_t{1} << 31) || B * S * K >= (int64_t{1} << 31) || S > 0x7fffffff || K > 0x7fffffff ||
      N * k_max >= (int64_t{1} << 40))
    return set_error(SI_ERR_UNSUPPORTED, "inverted index too large");
  return SI_OK;
}

extern "C" int64_t si_build_inverted_topk_workspace_bytes(int64_t B, int64_t S, int64_t K, int64_t n_kv) {
  if (inv_check(B, S, K, n_kv, 0)) return -1;
  InvPlan p{};
  if (inv_plan(B, S, K, n_kv, &p)) return -1;
  return static_cast<int64_t>(p.total);
}

extern "C" int si_build_inverted_topk(const void* topk_idxs, int idx_is_i64, const int64_t* idx_strides, int64_t B,
                                      int64_t S, int64_t K, int64_t n_kv, int64_t k_max, int32_t* inv_topk,
                                      int32_t* inv_count, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = inv_check(B, S, K, n_kv, k_max);
  if (rc) return rc;
  if (!idx_strides) return set_error(SI_ERR_INVALID, "null stride argument");
  const int64_t nkeys = B * n_kv;
  const int64_t npairs = B * S * K;
  if ((npairs > 0 && !topk_idxs) || (nkeys > 0 && (!inv_count || (k_max > 0 && !inv_topk))))
    return set_error(SI_ERR_INVALID, "null pointer argument");
  InvPlan pl{};
  if ((rc = inv_plan(B, S, K, n_kv, &pl))) return rc;
  if (static_cast<int64_t>(pl.total) > workspace_bytes || (pl.total > 0 && !workspace))
    return set_error(SI_ERR_INVALID, "workspace too small (see si_build_inverted_topk_workspace_bytes)");
  if (nkeys == 0) return SI_OK;
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* kin = reinterpret_cast<uint32_t*>(ws + pl.kin);
  uint32_t* kout = reinterpret_cast<uint32_t*>(ws + pl.kout);
  uint32_t* vin = reinterpret_cast<uint32_t*>(ws + pl.vin);
  uint32_t* vout = reinterpret_cast<uint32_t*>(ws + pl.vout);
  int32_t* seg_lo = reinterpret_cast<int32_t*>(ws + pl.seg_lo);
  int32_t* seg_hi = reinterpret_cast<int32_t*>(ws + pl.seg_hi);
  const int64_t fblocks = (nkeys + 255) / 256 < 65536 ? (nkeys + 255) / 256 : 65536;
  hipLaunchKernelGGL(sparse_attn_bwd_fill_kernel, dim3(static_cast<unsigned>(fblocks)), dim3(256), 0, st, seg_lo,
                     nkeys, 0);
  hipLaunchKernelGGL(sparse_attn_bwd_fill_kernel, dim3(static_cast<unsigned>(fblocks)), dim3(256), 0, st, seg_hi,
                     nkeys, 0);
  if ((rc = check_launch("sparse_attn_bwd_fill_kernel"))) return rc;
  if (npairs > 0) {
    const unsigned pblocks = static_cast<unsigned>((npairs + 255) / 256);
    hipLaunchKernelGGL(sparse_attn_bwd_pairs_kernel, dim3(pblocks), dim3(256), 0, st, topk_idxs, idx_is_i64 ? 1 : 0,
                       idx_strides[0], idx_strides[1], idx_strides[2], static_cast<int>(S), static_cast<int>(n_kv),
                       static_cast<int>(K), int64_t{0}, npairs, static_cast<uint32_t>(nkeys), B * S, nullptr,
                       int64_t{0}, int64_t{0}, kin, vin);
    if ((rc = check_launch("sparse_attn_bwd_pairs_kernel"))) return rc;
    size_t tmp_bytes = pl.tmp_bytes;
    const hipError_t e = rocprim::radix_sort_pairs(ws + pl.tmp, tmp_bytes, kin, kout, vin, vout,
                                                   static_cast<size_t>(npairs), 0u, bwd_end_bit(nkeys), st);
    if (e != hipSuccess) return set_error(SI_ERR_LAUNCH, std::string("radix sort: ") + hipGetErrorString(e));
    hipLaunchKernelGGL(sparse_attn_bwd_segments_kernel, dim3(pblocks), dim3(256), 0, st, kout, npairs,
                       static_cast<uint32_t>(nkeys), seg_lo, seg_hi);
    if ((rc = check_launch("sparse_attn_bwd_segments_kernel"))) return rc;
  }
  hipLaunchKernelGGL(inverted_fill_kernel, dim3(static_cast<unsigned>(nkeys)), dim3(64), 0, st, vout, seg_lo, seg_hi,
                     nkeys, static_cast<int>(S > 0 ? S : 1), static_cast<int>(K > 0 ? K : 1),
                     static_cast<int>(k_max), inv_topk, inv_count);
  return check_launch("inverted_fill_kernel");
}
