// Sparse-attention forward (MQA, attention sink) for gfx950.
//
// Reference behaviour being replaced:
//   * flash_sparse/triton/sparse_attn_fwd.py:40-177  (_sparse_attn_fwd_kernel)
//   * flash_sparse/triton/sparse_attn_fwd.py:180-292 (sparse_attn_fwd wrapper)
//   * flash_sparse/reference.py:44-130               (ground-truth semantics)
//
//   o[s,h,:] = Σ_j p_j kv[idx_j,:] / (Σ_j p_j + e^{sink_h - m}),
//   p_j = e^{scale·q[s,h]·kv[idx_j] - m},  idx_j = -1 (or out of range) masked,
//   lse[s,h] = log(Σ_j p_j + e^{sink_h - m}) + m.
//
// Design (up to 64 heads of one query row at a time per workgroup of 8 waves:
// four S^T/softmax "producer" waves and four P.V "consumer" waves, one of
// each per SIMD, so the matrix cores of a SIMD alternate between the two
// roles; at D >= 512 a workgroup takes 8 consecutive rows one after the other
// and fetches each next row's first index words during the current row):
//   * The row's top-k KV rows are gathered 32 at a time straight from L2/HBM
//     into a 4-slot LDS ring with global_load_lds (no staging registers) by
//     the producers, three tiles ahead of use; each row is read once per query
//     for all heads.  The tile barrier carries no release fence, so the copies
//     of later tiles stay in flight across it.
//     Rows are stored key-major with a per-key XOR swizzle of the 16-byte
//     chunks so that both LDS read patterns below are bank-conflict-free.
//   * S^T = K·Q^T (v_mfma_f32_16x16x32_bf16, keys on M, heads on N), split
//     across the producers by head (16 heads per wave, Q^T in VGPRs).  Each lane
//     then holds one head, so the online-softmax max and sum are in-lane plus
//     two xor exchanges.  The reference maximum is raised only when the tile
//     maximum exceeds it by 2^64 (the result is unchanged up to rounding), so
//     after the first valid tile the output accumulator is in practice never
//     rescaled.
//   * P^T (bf16) and the per-head rescale factors of all 64 heads are
//     exchanged through a small double-buffered LDS area; one barrier per
//     tile.
//   * O^T = V^T·P^T, split across the consumers by output dimension (the
//     16-dim blocks are dealt round-robin), so every V element is read from
//     LDS once.  The first consumer wave runs the index pipeline; each role
//     needs at most ~210 VGPRs and two waves fit a SIMD.
//     The V^T A-fragments are read from the key-major tile with
//     ds_read_b64_tr_b16 (two transposing reads give a lane 8 keys of one
//     dimension); the P^T B-fragments use the key order of the score
//     accumulators, so no register shuffles are needed.
//   * The normalised output is staged through LDS and written with
//     coalesced 16-byte stores.
#include <string>
#include <type_traits>

#include "attn_common.h"
#include "si_common.h"
#include "si_status.h"

namespace si {

struct SparseAttnArgs {
  const uint16_t* q;  // [B,S,H,D] bf16 or fp16 (f16)
  int64_t qsb, qss, qsh;
  const uint16_t* kv;  // [B,N,D], q's type
  int64_t kvsb, kvsn;
  const float* sink;   // [H]
  const void* idx;     // [B,S,K] int32 / int64
  int idx64;
  int64_t isb, iss, isk;
  uint16_t* o;         // [B,S,H,D], q's type
  int64_t osb, oss, osh;
  float* lse;          // [B,S,H]
  int64_t lsb, lss, lsh;
  int B, S, H, N, K;
  const int32_t* row_len;  // optional [B,S]: columns at or past row_len[b,s] are masked (tiles past it skipped)
  int64_t rlsb, rlss;
  int HG;              // head groups of 64
  float scale_log2;    // softmax_scale * log2(e)
  int f16;             // element type: 0 bf16, 1 fp16
  // Optional second KV tensor [B,N-N1,D] (kernel instantiation KV2): indices
  // in [N1, N) select its row index - N1, so a [kv ; kv_compressed] layout
  // needs no concatenated copy.
  const uint16_t* kv2;
  int64_t kv2sb, kv2sn;
  int N1;
};

// The reference maximum of a head moves only when a tile's maximum exceeds it
// by 2^64 (log2 units): p = 2^(x - m_ref) then stays below 2^64, far inside
// the fp32/bf16 exponent range, and the output accumulator is rescaled only
// on such a jump.  (Up to rounding the result equals the eager rescale.)
constexpr float kLazyRescale = 64.0f;
// With fp16 operands P = 2^(x - m_ref) must stay inside the fp16 range
// (max 65504): the reference moves once a tile's maximum exceeds it by 2^8.
constexpr float kLazyRescaleF16 = 8.0f;

// Threads of a workgroup: kAttnWaves S^T / softmax waves ("producers", 16
// heads each) and kAttnWaves P.V waves ("consumers", 16-dim output blocks
// dealt round-robin), one of each per SIMD.
constexpr int kAttnThreads = 2 * kAttnWaves * 64;

// Query rows per workgroup (ROWS), handled one after the other: while a
// row's last tiles run, the index wave copies the next row's first index
// words, so each row after the first starts without waiting for them (half
// of a row's prologue at D = 576).  Used where one workgroup fills a CU
// (D >= 512); with several workgroups per CU the others hide the prologue
// and a shorter grid only costs (measured: -3 % at D = 576, +27 % at D = 64
// for 8 rows).
template <int D>
constexpr int attn_rows_per_workgroup() {
  return D >= 512 ? 8 : 1;
}

// Published KV row offsets: 16-byte units from the batch's first KV row
// (32 bits) with one KV tensor; with two (KV2) signed byte offsets from the
// first tensor's batch base (64 bits), so that a key of either tensor costs
// one 64-bit add per copy, with no per-copy choice between two bases.
template <bool KV2>
using AttnRowOff = std::conditional_t<KV2, int64_t, uint32_t>;

template <int D, bool IDX64, bool F16, bool KV2>
__global__ __launch_bounds__(kAttnThreads) void sparse_attn_fwd_kernel(SparseAttnArgs a) {
  constexpr int kAttnRows = attn_rows_per_workgroup<D>();
  using SH = AttnShape<D>;
  constexpr int KS = SH::KS;
  constexpr int MBW = SH::MBW;
  constexpr int ROW = SH::ROW;
  __shared__ __attribute__((aligned(16))) char kv_lds[SH::LDS_KV];
  __shared__ __attribute__((aligned(16))) char p_lds[2][kAttnWaves * 64 * 16];  // P^T B-fragments per head block
  __shared__ float alpha_lds[2][64];
  __shared__ int live_lds[2];  // tile has at least one valid key (published with alpha)
  __shared__ float scale_lds[64];
  __shared__ __attribute__((aligned(16))) float bias_lds[kAttnRing][kAttnTK];  // 0: key used, -inf: masked
  __shared__ int tlive_lds[kAttnRing];  // the tile has at least one valid key (published with the biases)
  __shared__ AttnRowOff<KV2> rowoff_lds[kAttnRing][kAttnTK];  // offset of the key's KV row
  __shared__ __attribute__((aligned(16))) uint32_t idxraw_lds[2 * kAttnRing][2 * kAttnTK];  // raw index words

  const int lane = threadIdx.x & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  __builtin_assume(wave_all >= 0 && wave_all < 2 * kAttnWaves);
  const bool producer = wave_all < kAttnWaves;
  const int wave = producer ? wave_all : wave_all - kAttnWaves;  // index within the role
  __builtin_assume(wave >= 0 && wave < kAttnWaves);  // lets per-copy bounds fold at compile time
  const int g = lane >> 4;     // lane group 0..3
  const int i16 = lane & 15;
  const int nsg = (a.S + kAttnRows - 1) / kAttnRows;  // row groups
  // (XCD-aware block order, xcd_block_order: HCA attention -2.5 %, CSA
  // attention -2 % at S = 64K, config[3]'s scattered picks unchanged)
  const int lb = xcd_block_order();
  const int sg = lb % nsg;
  const int rest = lb / nsg;
  const int b = rest % a.B;
  const int hg = rest / a.B;
  const int hbase = hg * 64;
  // Columns of row r: K, or fewer when a row length is given (the rest are
  // masked and their tiles never run).  With no KV rows every key is masked:
  // the tile loop is skipped.
  auto row_klen = [&](int r) {
    int kl = a.K;
    if (a.row_len) {
      const int rl = a.row_len[b * a.rlsb + static_cast<int64_t>(r) * a.rlss];
      kl = rl < 0 ? 0 : (rl < a.K ? rl : a.K);
    }
    return kl;
  };
  const char* idx_base = static_cast<const char*>(a.idx) + b * a.isb * (IDX64 ? 8 : 4);
  bool idx_ready = false;  // (index wave) this row's first index words were copied during the previous row
  for (int jr = 0; jr < kAttnRows; ++jr) {
    const int s = sg * kAttnRows + jr;
    if (s >= a.S) break;
    const int klen = row_klen(s);
    const int ntiles = a.N > 0 ? (klen + kAttnTK - 1) / kAttnTK : 0;
    const int s_nx = (jr + 1 < kAttnRows && s + 1 < a.S) ? s + 1 : -1;
    const int klen_nx = s_nx >= 0 ? row_klen(s_nx) : 0;
    const int ntiles_nx = (s_nx >= 0 && a.N > 0) ? (klen_nx + kAttnTK - 1) / kAttnTK : 0;

    // Tile protocol (one barrier per tile).  Iteration `it`: the consumers
    // compute P.V of tile it while the producers compute S^T + softmax of tile
    // it+1 and publish its P^T and rescale factors; tile t lives in ring slot
    // t % 4 and its P^T in p_lds[t % 2].  The producers issue the copies of
    // tile it+3 at the start of the iteration into the slot of tile it-1
    // (finished by every wave in iteration it-1); they must land by the end of
    // iteration it+1, two iterations of gather latency.  The first consumer
    // wave copies the raw indices of tile it+6 at the start and publishes those
    // of tile it+5 (copied one iteration earlier) before the barrier.

    if (producer) {
      // ======================= S^T + online softmax ==========================
      const int hq = hbase + wave * 16 + i16;  // this lane's head
      const bool hvalid = hq < a.H;
      bf16x8 qf[KS];
      {
        const uint16_t* qrow = a.q + b * a.qsb + static_cast<int64_t>(s) * a.qss + static_cast<int64_t>(hq) * a.qsh;
  #pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          qf[ks] = hvalid ? *reinterpret_cast<const bf16x8*>(qrow + ks * 32 + g * 8) : bf16x8{};
      }

      // S^T A-fragment addresses: key 16mb + i16, chunk 4ks + g.  With
      // f = kv_swz(i16), (4ks + g) ^ f = 4 (ks ^ (f >> 2)) + (g ^ (f & 3)), so the
      // offset is a per-lane base (one per ks parity) plus 64 ks + 16 ROW mb.
      const int qf_swz = kv_swz<D>(i16);
      const int qbase = i16 * ROW + 16 * (g ^ (qf_swz & 3));
      const int qadj = 64 * (qf_swz >> 2);
      float m_ref = -1.0e30f;  // reference maximum of this lane's head (log2 domain)
      float l_run = 0.f;       // this lane's share of the denominator

      // ---- KV gather (issued by the producers, which wait at the tile barrier
      // for the P.V waves otherwise) -------------------------------------------
      const char* kvb = reinterpret_cast<const char*>(a.kv + b * a.kvsb);
      // Gather of tile `t` into its ring slot: LDS slot e (16 bytes at byte 16e)
      // holds chunk (e % CPR) ^ f(key) of key e / CPR.  This thread's key and
      // chunk (in 16-byte units) per copy are fixed, computed once; a copy's
      // source is kv + 16 (rowoff16[key] + dcoff), or kv + rowoff[key] + 16 dcoff
      // with two KV tensors.
      int dkey[SH::LPT], dcoff[SH::LPT];
  #pragma unroll
      for (int i = 0; i < SH::LPT; ++i) {
        const int e = i * SH::NT + static_cast<int>(threadIdx.x);
        dkey[i] = e / SH::CPR;
        dcoff[i] = (e % SH::CPR) ^ kv_swz<D>(dkey[i]);
      }
      using RowOff = AttnRowOff<KV2>;
      RowOff roff[SH::LPT];  // copy sources of the tile being gathered
      auto read_roff = [&](int t, RowOff (&dst)[SH::LPT]) {
        const int slot = t % kAttnRing;
  #pragma unroll
        for (int i = 0; i < SH::LPT; ++i) {
          if (i * SH::NT + wave * 64 < SH::CH)
            dst[i] = rowoff_lds[slot][dkey[i]] + (KV2 ? 16 * dcoff[i] : dcoff[i]);
          else
            dst[i] = 0;
        }
      };
      // Copy i of tile t (one 64-lane group of 16-byte slots); every 64-slot
      // group lies wholly inside or wholly outside the tile (CH % 64 == 0).
      auto dma = [&](int t, const RowOff (&ro)[SH::LPT], auto IC) {
        constexpr int i = decltype(IC)::value;
        const int e0 = i * SH::NT + wave * 64;
        char* dst = kv_lds + (t % kAttnRing) * SH::TILE + e0 * 16;
        // (passed as uint16_t*: a char* argument to this builtin makes clang
        // drop the host launch stubs of later instantiations)
        const uint16_t* src;
        if constexpr (KV2) {
          src = reinterpret_cast<const uint16_t*>(kvb + ro[i]);
        } else {
          src = reinterpret_cast<const uint16_t*>(kvb + (static_cast<uint64_t>(ro[i]) << 4));
        }
        if constexpr (SH::CH % SH::NT == 0 || i + 1 < SH::LPT) {
          __builtin_amdgcn_global_load_lds(src, (lds_void_t*)dst, 16, 0, 0);
        } else if (e0 < SH::CH) {
          __builtin_amdgcn_global_load_lds(src, (lds_void_t*)dst, 16, 0, 0);
        }
      };
      // The copies of tile `src` (its row offsets) into the ring slot of tile `dst`.
      auto issue_tile_from = [&](int src, int dst) {
        read_roff(src, roff);
        attn_static_for<0, SH::LPT>([&](auto IC) { dma(dst, roff, IC); });
      };


      // S^T = K Q^T of tile t for this wave's 16 heads (keys 16mb + 4g + r).
      // A-fragments stream through a QPD-deep register queue: each MFMA's
      // operand was read from LDS QPD k-steps earlier.
      constexpr int QPD = KS < 4 ? KS : 4;
      auto qk = [&](int t, f32x4 (&st)[2]) {
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
        st[0] = f32x4{0.f, 0.f, 0.f, 0.f};
        st[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto qk_step = [&](auto KC) {
          constexpr int ks = decltype(KC)::value;
          constexpr int later = (KS - 1 - ks) < (QPD - 1) ? (KS - 1 - ks) : (QPD - 1);  // k-steps issued after ks
          lds_wait<2 * later>(kq[ks % QPD][0], kq[ks % QPD][1]);
          st[0] = mfma16x16x32<F16>(kq[ks % QPD][0], qf[ks], st[0]);
          st[1] = mfma16x16x32<F16>(kq[ks % QPD][1], qf[ks], st[1]);
          if constexpr (ks + QPD < KS) qk_issue(std::integral_constant<int, ks + QPD>{});
        };
        attn_static_for<0, KS>(qk_step);
        mfma_result_fence(st[0], st[1]);
      };

      // Online softmax of tile t for head hq, in registers; the result (P^T as
      // a bf16 B-fragment and the head's rescale factor) is published by
      // softmax_store.
      struct SoftmaxOut {
        u32x4 w;
        float alpha;
      };
      auto softmax = [&](const f32x4 (&st)[2], const f32x4 (&bias)[2]) {
        SoftmaxOut out;
        float x[2][4];
  #pragma unroll
        for (int mb = 0; mb < 2; ++mb)
  #pragma unroll
          for (int r = 0; r < 4; ++r) x[mb][r] = __builtin_fmaf(st[mb][r], a.scale_log2, bias[mb][r]);
        // this lane's share of the tile maximum (its 8 keys)
        const float lmax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(x[0][0], x[0][1]), __builtin_fmaxf(x[0][2], x[0][3])),
                                           __builtin_fmaxf(__builtin_fmaxf(x[1][0], x[1][1]), __builtin_fmaxf(x[1][2], x[1][3])));
        // First valid key of the head: the accumulator and denominator are
        // still zero, so the reference moves without a rescale (alpha = 1).
        const bool first = m_ref == -1.0e30f;
        const float lazy = F16 ? kLazyRescaleF16 : kLazyRescale;
        // A head's reference moves iff one of its four lanes' keys lifts it, so
        // when no lane of the wave does (every tile after a head's first valid
        // one, in practice) the reference stays and the tile maximum over the
        // lane groups is not needed: the exponentials below use m_ref as is.
        const bool lift = first ? lmax > m_ref : lmax > m_ref + lazy;
        out.alpha = 1.0f;
        if (__builtin_amdgcn_ballot_w64(lift) != 0) {
          // tile maximum over the lane groups g ^ 1 and g ^ 2
          const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(lmax), __float_as_uint(lmax), false, false);
          float tmax = __builtin_fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
          const SwapPair r32 = permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax));
          tmax = __builtin_fmaxf(__uint_as_float(r32.x), __uint_as_float(r32.y));
          const bool raise = first ? tmax > m_ref : tmax > m_ref + lazy;
          const float m_new = raise ? tmax : m_ref;
          out.alpha = (raise && !first) ? __builtin_amdgcn_exp2f(m_ref - m_new) : 1.0f;
          m_ref = m_new;
        }
        f32x2 p[4];
  #pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          p[2 * mb] = f32x2{__builtin_amdgcn_exp2f(x[mb][0] - m_ref), __builtin_amdgcn_exp2f(x[mb][1] - m_ref)};
          p[2 * mb + 1] = f32x2{__builtin_amdgcn_exp2f(x[mb][2] - m_ref), __builtin_amdgcn_exp2f(x[mb][3] - m_ref)};
        }
        const float psum = ((p[0][0] + p[0][1]) + (p[1][0] + p[1][1])) + ((p[2][0] + p[2][1]) + (p[3][0] + p[3][1]));
        l_run = l_run * out.alpha + psum;
        // P^T B-fragment: k-slots 8g+0..3 <-> keys 4g+0..3, 8g+4..7 <-> keys 16+4g+0..3
  #pragma unroll
        for (int c = 0; c < 4; ++c) out.w[c] = pack2<F16>(p[c][0], p[c][1]);
        return out;
      };
      // (inline asm: the compiler makes a tracked LDS access that follows
      // LDS-DMA copies wait for all of them; the tile barrier's lgkmcnt(0)
      // orders these stores)
      auto softmax_store = [&](int t, const SoftmaxOut& r, bool live) {
        const uint32_t pa = lds_addr(&p_lds[t & 1][(wave * 64 + lane) * 16]);
        asm volatile("ds_write_b128 %0, %1" ::"v"(pa), "v"(r.w) : "memory");
        if (g == 0) {
          const uint32_t aa = lds_addr(reinterpret_cast<const char*>(&alpha_lds[t & 1][wave * 16 + i16]));
          asm volatile("ds_write_b32 %0, %1" ::"v"(aa), "v"(r.alpha) : "memory");
        }
        if (wave == 0 && lane == 0) {
          const uint32_t la = lds_addr(reinterpret_cast<const char*>(&live_lds[t & 1]));
          asm volatile("ds_write_b32 %0, %1" ::"v"(la), "v"(live ? 1 : 0) : "memory");
        }
      };
      // Key biases of tile t in the score-accumulator order (keys 4g+r, 16+4g+r);
      // the slot read is always inside the array, so no guard is needed.
      auto read_bias = [&](int t, f32x4 (&bias)[2]) {
        bias[0] = *reinterpret_cast<const f32x4*>(&bias_lds[t % kAttnRing][4 * g]);
        bias[1] = *reinterpret_cast<const f32x4*>(&bias_lds[t % kAttnRing][16 + 4 * g]);
      };
      // Whether any key of tile t is valid, as the index wave published it
      // with the biases (read with them, made wave-uniform at its use).  An
      // all-masked tile needs no S^T (its scores are finite + bias = -inf
      // either way, so the scores of the last computed tile serve) and no
      // P.V (P = 0).
      auto read_live = [&](int t) { return tlive_lds[t % kAttnRing]; };
      auto is_live = [&](int v) { return __builtin_amdgcn_readfirstlane(v) != 0; };
      const f32x4 zero4 = f32x4{0.f, 0.f, 0.f, 0.f};
      f32x4 st[2] = {zero4, zero4};  // S^T accumulators (kept across tiles, see above; one KV tensor)

      if (ntiles > 0) {
        // (prologue barriers without a release fence, like the tile barrier: a
        // fence would make the compiler wait here for the Q loads and for every
        // tile copy in flight, not just the ones the comments name)
        attn_tile_barrier();  // indices of tiles 0..3 published
        // Copies of tiles 0, 1 and 2.  A row with fewer tiles copies its last
        // tile again into the slots it does not use, so every row waits the same
        // way and the compiler sees that the Q loads (issued first) have landed
        // once tile 0 has.
        issue_tile_from(0, 0);
        issue_tile_from(ntiles > 1 ? 1 : ntiles - 1, 1);
        issue_tile_from(ntiles > 2 ? 2 : ntiles - 1, 2);
        // tile 0 (and every Q load) landed; the copies of tiles 1 and 2 may still be in flight
        __builtin_amdgcn_s_waitcnt(vm_lgkm0(2 * SH::LPT));
        attn_tile_barrier();  // tile 0 landed
        // Per-tile state alternates between two register sets (the loop runs
        // two tiles per trip), so nothing is copied from one tile to the next.
        f32x4 bias_a[2], bias_b[2];
        int live_a, live_b;
        RowOff roff_b[SH::LPT];
        {
          f32x4 bias[2];
          read_bias(0, bias);
          const int live0 = read_live(0);
          read_bias(1, bias_a);
          live_a = read_live(1);
          read_roff(3, roff);
          const bool live = is_live(live0);
          f32x4 st0[2] = {zero4, zero4};
          if (live) qk(0, st0);
          softmax_store(0, softmax(st0, bias), live);
          if constexpr (!KV2) {
            st[0] = st0[0];
            st[1] = st0[1];
          }
        }
        // tile 1 landed; the copies of tile 2 may still be in flight
        __builtin_amdgcn_s_waitcnt(vm_lgkm0(SH::LPT));
        attn_tile_barrier();  // tile 1 landed; P^T of tile 0 published; tile 0's biases and offsets read
        attn_tile_barrier();  // indices of tile 4 published
        // Iteration it with the state of tile it+1 in (bias_c, live_c), the
        // copy sources of tile it+3 in ro_c; it reads those of tiles it+2 and
        // it+4 into the other set.
        auto iteration = [&](int it, f32x4 (&bias_c)[2], int& live_c, f32x4 (&bias_n)[2], int& live_n,
                             const RowOff (&ro_c)[SH::LPT], RowOff (&ro_n)[SH::LPT]) {
          const bool issue = it + 3 < ntiles;
          // tracked LDS reads first, then the copies of tile it+3 into the slot
          // of tile it-1 (finished by every wave in iteration it-1)
          read_bias(it + 2, bias_n);    // slots read are always inside the arrays
          live_n = read_live(it + 2);
          read_roff(it + 4, ro_n);
          if (issue) attn_static_for<0, SH::LPT>([&](auto IC) { dma(it + 3, ro_c, IC); });
          if (it + 1 < ntiles) {
            const bool live = is_live(live_c);
            if constexpr (KV2) {
              // (zeroed per tile: this variant has no registers to spare)
              f32x4 stl[2] = {zero4, zero4};
              if (live) qk(it + 1, stl);
              softmax_store(it + 1, softmax(stl, bias_c), live);
            } else {
              if (live) qk(it + 1, st);
              softmax_store(it + 1, softmax(st, bias_c), live);
            }
          }
          // the copies of tile it+2 (issued one iteration ago) landed; those of
          // tile it+3 stay in flight across the barrier
          if (issue) __builtin_amdgcn_s_waitcnt(vm_lgkm0(SH::LPT));
          else __builtin_amdgcn_s_waitcnt(vm_lgkm0(0));
          attn_tile_barrier();
        };
        if constexpr (KV2) {
          // (64-bit copy sources: two register sets of them would not fit
          // beside the rest, so this variant copies them forward per tile)
          for (int it = 0; it < ntiles; ++it) {
            iteration(it, bias_a, live_a, bias_b, live_b, roff, roff_b);
            bias_a[0] = bias_b[0];
            bias_a[1] = bias_b[1];
            live_a = live_b;
  #pragma unroll
            for (int i = 0; i < SH::LPT; ++i) roff[i] = roff_b[i];
          }
        } else {
          for (int it = 0; it < ntiles; it += 2) {
            iteration(it, bias_a, live_a, bias_b, live_b, roff, roff_b);
            if (it + 1 < ntiles) iteration(it + 1, bias_b, live_b, bias_a, live_a, roff_b, roff);
          }
        }
      }

      // ---- denominators, sink, normalisation factor, lse ----------------------
      float l_tot;
      {  // sum over the four lane groups
        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
        l_tot = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
        const SwapPair r32 = permlane32_swap(__float_as_uint(l_tot), __float_as_uint(l_tot));
        l_tot = __uint_as_float(r32.x) + __uint_as_float(r32.y);
      }
      constexpr float kLog2e = 1.4426950408889634f;
      // (the sink is read only now: a load at the top would make the first
      // copies wait for every Q load)
      const float sink_v = hvalid ? a.sink[hq] : 0.f;
      const float sink2 = hvalid ? sink_v * kLog2e : -__builtin_inff();
      const float m_fin = __builtin_fmaxf(m_ref, sink2);
      const float resc = __builtin_amdgcn_exp2f(m_ref - m_fin);
      const float l_fin = l_tot * resc + __builtin_amdgcn_exp2f(sink2 - m_fin);
      const float scale = l_fin > 0.f ? resc / l_fin : 0.f;
      if (g == 0) {
        scale_lds[wave * 16 + i16] = scale;
        if (hvalid) {
          constexpr float kLn2 = 0.6931471805599453f;
          const float lse = l_fin > 0.f ? (__builtin_amdgcn_logf(l_fin) + m_fin) * kLn2 : -1.0e30f;
          a.lse[b * a.lsb + static_cast<int64_t>(s) * a.lss + static_cast<int64_t>(hq) * a.lsh] = lse;
        }
      }
      __syncthreads();  // normalisation factors published
      __syncthreads();  // output staged
    } else {
      // ============== P.V, KV gather and the index pipeline =====================
      const bool idx_wave = wave == 0;
      const char* idx_row = idx_base + static_cast<int64_t>(s) * a.iss * (IDX64 ? 8 : 4);
      const char* idx_row_nx = idx_base + static_cast<int64_t>(s_nx < 0 ? 0 : s_nx) * a.iss * (IDX64 ? 8 : 4);

      // Key indices of tile `t`: the index wave copies the raw index words into
      // idxraw_lds[t % 8] with a global_load_lds (nothing lands in registers, so
      // no loop-carried load result forces an early wait), and after its next
      // full wait reads them back, validates them and publishes validity and
      // row offsets to ring slot t % 4 for every wave.
      auto load_idx_of = [&](const char* row, int kl, int t) {
        // 64-bit indices: lane l copies word l & 1 of key l >> 1; 32-bit: key l & 31.
        int j = t * kAttnTK + (IDX64 ? (lane >> 1) : (lane & 31));
        j = j < kl ? j : kl - 1;  // kl > 0 whenever a tile exists
        const int64_t byte = static_cast<int64_t>(j) * a.isk * (IDX64 ? 8 : 4) + (IDX64 ? (lane & 1) * 4 : 0);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(row + byte),
                                         (lds_void_t*)(&idxraw_lds[t % (2 * kAttnRing)][0]), 4, 0, 0);
      };
      auto load_idx = [&](int t) { load_idx_of(idx_row, klen, t); };
      // The next row's first index words go out once this row's index work is
      // done (its last copy was waited for and its last publish read the raw
      // slots one iteration earlier).
      const int it_nx = ntiles > 5 ? ntiles - 5 : 0;
      const int np_nx = ntiles_nx < 6 ? ntiles_nx : 6;
      auto store_idx = [&](int t) {
        const int slot = t % kAttnRing;
        const int rslot = t % (2 * kAttnRing);
        const int ln = lane < kAttnTK ? lane : 0;
        const int64_t raw = IDX64 ? static_cast<int64_t>((static_cast<uint64_t>(idxraw_lds[rslot][2 * ln + 1]) << 32) |
                                                         idxraw_lds[rslot][2 * ln])
                                  : static_cast<int64_t>(static_cast<int32_t>(idxraw_lds[rslot][ln]));
        const bool ok = lane < kAttnTK && t * kAttnTK + lane < klen && raw >= 0 && raw < a.N;
        // whether any key of the tile is valid, for the producers
        const bool live = __builtin_amdgcn_ballot_w64(ok) != 0;
        if (lane == 0) tlive_lds[slot] = live ? 1 : 0;
        if (lane < kAttnTK) {
          bias_lds[slot][lane] = ok ? 0.f : -__builtin_inff();
          if constexpr (KV2) {
            // byte offsets from the first tensor's batch base; a masked key
            // reads the first row of a tensor that has rows
            const int64_t kv2_delta = reinterpret_cast<const char*>(a.kv2 + b * a.kv2sb) -
                                      reinterpret_cast<const char*>(a.kv + b * a.kvsb);
            const bool second = raw >= a.N1;
            rowoff_lds[slot][lane] = !ok ? (a.N1 > 0 ? int64_t{0} : kv2_delta)
                                     : second ? kv2_delta + (raw - a.N1) * a.kv2sn * 2
                                              : raw * a.kvsn * 2;
          } else {
            rowoff_lds[slot][lane] = static_cast<uint32_t>((ok ? raw : 0) * (a.kvsn / 8));
          }
        }
      };
      // V^T transposing-read address: source lane (g, i16) points at key
      // 4g + (i16 >> 2) (+16 for k-slots 4..7), dims d0 + 4 (i16 & 3) with
      // d0 = 16 (4j + wave); the chunk 8j + x, x = 2 wave + ((i16 & 3) >> 1) < 8,
      // swizzles to 8j + (x ^ f), so block j is at a fixed base + 128 j.
      const int tkey = 4 * g + (i16 >> 2);
      const int tx = 2 * wave + ((i16 & 3) >> 1);
      const int tbase = tkey * ROW + 16 * ((tx ^ kv_swz<D>(tkey)) & (SH::CPR - 1)) + 8 * (i16 & 1);

      f32x4 oacc[MBW][4];
  #pragma unroll
      for (int j = 0; j < MBW; ++j)
  #pragma unroll
        for (int nb = 0; nb < 4; ++nb) oacc[j][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

      // O^T += V^T P^T of tile `it` for this wave's 16-dim blocks and all 64
      // heads.  The P^T fragments and the V^T blocks are read from inline asm
      // with exact waits: blocks j and j+1 are in flight while block j's MFMAs
      // run (LDS operations complete in order, so waiting for "at most 2
      // outstanding" covers everything issued before block j+1).
      auto pv = [&](int it) {
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
          for (int nb = 0; nb < 4; ++nb) oacc[j][nb] = mfma16x16x32<F16>(vf, pbr[nb], oacc[j][nb]);
          if constexpr (j + 2 < MBW) {
            lo[j & 1] = tr_read<128 * (j + 2)>(ta);
            hi[j & 1] = tr_read<16 * ROW + 128 * (j + 2)>(ta);
          }
        };
        attn_static_for<0, MBW>(block);
      };

      // One consumer iteration: P.V of tile it and the index pipeline.
      auto iteration = [&](int it) {
        float al[4];
  #pragma unroll
        for (int nb = 0; nb < 4; ++nb) al[nb] = alpha_lds[it & 1][nb * 16 + i16];
        // wave-uniform in a scalar register, so the skip is a scalar branch
        // (MFMAs do not honour EXEC)
        const bool live = __builtin_amdgcn_readfirstlane(live_lds[it & 1]) != 0;
        if (idx_wave && it + 6 < ntiles) load_idx(it + 6);
        if (idx_wave && it == it_nx) {
          for (int t = 0; t < np_nx; ++t) load_idx_of(idx_row_nx, klen_nx, t);
        }

        const bool any_rescale = __builtin_amdgcn_ballot_w64(al[0] != 1.0f || al[1] != 1.0f || al[2] != 1.0f ||
                                                             al[3] != 1.0f) != 0;
        if (__builtin_expect(any_rescale, 0)) {
  #pragma unroll
          for (int j = 0; j < MBW; ++j)
  #pragma unroll
            for (int nb = 0; nb < 4; ++nb) oacc[j][nb] = oacc[j][nb] * al[nb];
        }
        if (live) pv(it);  // P = 0 for a tile without a valid key
        // the indices of tile it+5 (copied one iteration ago) landed; in the
        // index wave those of tile it+6 may stay in flight
        if (idx_wave && it + 6 < ntiles) __builtin_amdgcn_s_waitcnt(vm_lgkm0(1));
        else if (idx_wave && it >= it_nx && np_nx > 0)
          __builtin_amdgcn_s_waitcnt(vm_lgkm0(63));  // (the next row's index words stay in flight)
        else __builtin_amdgcn_s_waitcnt(vm_lgkm0(0));
        if (idx_wave && it + 5 < ntiles) store_idx(it + 5);
      };

      if (ntiles > 0) {
        // indices of tiles 0..5; tile 4 shares its row-offset / bias slot with
        // tile 0, so it is published once tile 0's entries have been read, and
        // tile 5 at the end of iteration 0
        if (idx_wave) {
          const int np = ntiles < 6 ? ntiles : 6;
          if (!idx_ready)
            for (int t = 0; t < np; ++t) load_idx(t);
          __builtin_amdgcn_s_waitcnt(0x7 << 4);
          for (int t = 0; t < np && t < 4; ++t) store_idx(t);
        }
        __syncthreads();  // indices of tiles 0..3 published
        __syncthreads();  // tile 0 landed
        __syncthreads();  // tile 1 landed; every wave has read tile 0's row offsets and biases
        if (idx_wave && ntiles > 4) store_idx(4);
        __syncthreads();  // indices of tile 4 published
        for (int it = 0; it < ntiles; ++it) {
          iteration(it);
          attn_tile_barrier();  // (store_idx's LDS stores complete first)
        }
      }
      __builtin_amdgcn_s_waitcnt(0x7 << 4);  // no gather may still target the ring
      if (idx_wave) idx_ready = ntiles > 0 && np_nx > 0;
      __syncthreads();  // normalisation factors published
      // Normalised O (bf16) staged head-major in LDS: [64 heads][OROW bytes].
      float sc[4];
  #pragma unroll
      for (int nb = 0; nb < 4; ++nb) sc[nb] = scale_lds[nb * 16 + i16];
  #pragma unroll
      for (int j = 0; j < MBW; ++j) {
        const int mbi = j * kAttnWaves + wave;
        if (SH::MBT % kAttnWaves == 0 || mbi < SH::MBT) {
  #pragma unroll
          for (int nb = 0; nb < 4; ++nb) {
            uint2 w;
            w.x = pack2<F16>(oacc[j][nb][0] * sc[nb], oacc[j][nb][1] * sc[nb]);
            w.y = pack2<F16>(oacc[j][nb][2] * sc[nb], oacc[j][nb][3] * sc[nb]);
            *reinterpret_cast<uint2*>(kv_lds + (nb * 16 + i16) * SH::OROW + (mbi * 16 + 4 * g) * 2) = w;
          }
        }
      }
      __syncthreads();  // output staged
    }

    // ---- coalesced 16-byte stores of the staged output (all threads) ---------
    const int hcount = (a.H - hbase) < 64 ? (a.H - hbase) : 64;
    uint16_t* obase = a.o + b * a.osb + static_cast<int64_t>(s) * a.oss + static_cast<int64_t>(hbase) * a.osh;
    for (int e = threadIdx.x; e < hcount * SH::CPR; e += kAttnThreads) {
      const int h = e / SH::CPR, c = e % SH::CPR;
      *reinterpret_cast<u32x4*>(obase + static_cast<int64_t>(h) * a.osh + c * 8) =
          *reinterpret_cast<const u32x4*>(kv_lds + h * SH::OROW + c * 16);
    }
    // (the next row's first barrier orders these reads of the staged output
    // before its copies into the ring)
  }
}

template <int D>
static int launch_attn(const SparseAttnArgs& a, hipStream_t st) {
  constexpr int R = attn_rows_per_workgroup<D>();
  const int64_t nblk = static_cast<int64_t>(a.B) * ((a.S + R - 1) / R) * a.HG;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  const dim3 grid(static_cast<unsigned>(nblk)), block(kAttnThreads);
  if (a.kv2) {  // (int32 indices: the CSA / HCA rows)
    if (a.f16) hipLaunchKernelGGL((sparse_attn_fwd_kernel<D, false, true, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((sparse_attn_fwd_kernel<D, false, false, true>), grid, block, 0, st, a);
  } else if (a.f16) {
    if (a.idx64) hipLaunchKernelGGL((sparse_attn_fwd_kernel<D, true, true, false>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((sparse_attn_fwd_kernel<D, false, true, false>), grid, block, 0, st, a);
  } else {
    if (a.idx64) hipLaunchKernelGGL((sparse_attn_fwd_kernel<D, true, false, false>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((sparse_attn_fwd_kernel<D, false, false, false>), grid, block, 0, st, a);
  }
  return check_launch("sparse_attn_fwd_kernel");
}

}  // namespace si

using namespace si;

// Shared body of the forward entries.  kv2 (with N_kv2 rows) is the optional
// second KV tensor: indices in [N_kv, N_kv + N_kv2) select its rows.
static int sparse_attn_fwd_entry(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                                 int64_t N_kv, const void* kv2, const int64_t* kv2_strides, int64_t N_kv2,
                                 const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                                 const int64_t* idx_strides, int64_t B, int64_t S, int64_t H, int64_t D, int64_t K,
                                 float softmax_scale, int qkv_dtype, void* o, const int64_t* o_strides, float* lse,
                                 const int64_t* lse_strides, const int32_t* row_len, const int64_t* row_len_strides,
                                 void* stream) {
  if (row_len && !row_len_strides) return set_error(SI_ERR_INVALID, "null row_len strides");
  if (qkv_dtype != SI_DTYPE_BF16 && qkv_dtype != SI_DTYPE_F16)
    return set_error(SI_ERR_INVALID, "qkv_dtype must be SI_DTYPE_BF16 (0) or SI_DTYPE_F16 (1)");
  if (!q_strides || !kv_strides || !idx_strides || !o_strides || !lse_strides)
    return set_error(SI_ERR_INVALID, "null stride argument");
  if (B < 0 || S < 0 || H <= 0 || D <= 0 || N_kv < 0 || K < 0) return set_error(SI_ERR_INVALID, "bad dimension");
  // Empty tensors may carry a null data pointer; only non-empty ones are dereferenced.
  const bool rows = B > 0 && S > 0;
  if (rows && (!q || !attn_sink || !o || !lse || (K > 0 && !topk_idxs) || (N_kv > 0 && !kv)))
    return set_error(SI_ERR_INVALID, "null pointer argument");
  if (B > 0x7fffffff || S > 0x7fffffff || N_kv > 0x7fffffff || K > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (H > 0x7fffffff) return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (q_strides[3] != 1 || kv_strides[2] != 1 || o_strides[3] != 1)
    return set_error(SI_ERR_INVALID, "q, kv and o need a contiguous last dimension");
  if ((q_strides[0] | q_strides[1] | q_strides[2] | kv_strides[0] | kv_strides[1]) % 8)
    return set_error(SI_ERR_INVALID, "q/kv strides must be multiples of 8 elements");
  if ((o_strides[0] | o_strides[1] | o_strides[2]) % 8) return set_error(SI_ERR_INVALID, "o strides must be multiples of 8");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kv)) & 15)
    return set_error(SI_ERR_INVALID, "q/kv must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(o) & 15) return set_error(SI_ERR_INVALID, "o must be 16-byte aligned");
  // With one KV tensor its row offsets are kept in 32 bits, in 16-byte units,
  // inside one batch (two tensors use 64-bit byte offsets).
  if (!kv2 && N_kv > 0 && ((N_kv - 1) * kv_strides[1] + D) / 8 >= (int64_t{1} << 32))
    return set_error(SI_ERR_UNSUPPORTED, "kv batch larger than 64 GiB");
  if (kv2) {
    if (!kv2_strides) return set_error(SI_ERR_INVALID, "null stride argument");
    if (N_kv2 < 0) return set_error(SI_ERR_INVALID, "bad dimension");
    if (N_kv + N_kv2 > 0x7fffffff) return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
    if (idx_is_i64) return set_error(SI_ERR_UNSUPPORTED, "two KV tensors take int32 indices");
    if (kv2_strides[2] != 1 || (kv2_strides[0] | kv2_strides[1]) % 8 || (reinterpret_cast<uintptr_t>(kv2) & 15))
      return set_error(SI_ERR_INVALID, "kv2 needs a contiguous last dimension, 16-byte rows and alignment");
  }
  SparseAttnArgs a{};
  if (kv2 && N_kv2 > 0) {
    a.kv2 = static_cast<const uint16_t*>(kv2);
    a.kv2sb = kv2_strides[0];
    a.kv2sn = kv2_strides[1];
    a.N1 = static_cast<int>(N_kv);
    N_kv += N_kv2;
  }
  a.q = static_cast<const uint16_t*>(q);
  a.qsb = q_strides[0]; a.qss = q_strides[1]; a.qsh = q_strides[2];
  a.kv = static_cast<const uint16_t*>(kv);
  a.kvsb = kv_strides[0]; a.kvsn = kv_strides[1];
  a.sink = attn_sink;
  a.idx = topk_idxs;
  a.idx64 = idx_is_i64 ? 1 : 0;
  a.isb = idx_strides[0]; a.iss = idx_strides[1]; a.isk = idx_strides[2];
  a.o = static_cast<uint16_t*>(o);
  a.osb = o_strides[0]; a.oss = o_strides[1]; a.osh = o_strides[2];
  a.lse = lse;
  a.lsb = lse_strides[0]; a.lss = lse_strides[1]; a.lsh = lse_strides[2];
  a.B = static_cast<int>(B); a.S = static_cast<int>(S); a.H = static_cast<int>(H);
  a.N = static_cast<int>(N_kv); a.K = static_cast<int>(K);
  a.row_len = row_len;
  if (row_len) {
    a.rlsb = row_len_strides[0];
    a.rlss = row_len_strides[1];
  }
  a.HG = static_cast<int>((H + 63) / 64);
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.f16 = qkv_dtype == SI_DTYPE_F16 ? 1 : 0;
  if (a.B == 0 || a.S == 0) return SI_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (D) {
    case 32: return launch_attn<32>(a, st);
    case 64: return launch_attn<64>(a, st);
    case 128: return launch_attn<128>(a, st);
    case 256: return launch_attn<256>(a, st);
    case 512: return launch_attn<512>(a, st);
    case 576: return launch_attn<576>(a, st);
    default:
      return set_error(SI_ERR_UNSUPPORTED,
                       "unsupported head dim D=" + std::to_string(D) + " (supported: 32, 64, 128, 256, 512, 576)");
  }
}

extern "C" int si_sparse_attn_fwd_ragged(const void* q, const int64_t* q_strides, const void* kv,
                                         const int64_t* kv_strides, const float* attn_sink, const void* topk_idxs,
                                         int idx_is_i64, const int64_t* idx_strides, int64_t B, int64_t S, int64_t H,
                                         int64_t D, int64_t N_kv, int64_t K, float softmax_scale, int qkv_dtype,
                                         void* o, const int64_t* o_strides, float* lse, const int64_t* lse_strides,
                                         const int32_t* row_len, const int64_t* row_len_strides, void* stream) {
  return sparse_attn_fwd_entry(q, q_strides, kv, kv_strides, N_kv, nullptr, nullptr, 0, attn_sink, topk_idxs,
                               idx_is_i64, idx_strides, B, S, H, D, K, softmax_scale, qkv_dtype, o, o_strides, lse,
                               lse_strides, row_len, row_len_strides, stream);
}

extern "C" int si_sparse_attn_fwd_kv2(const void* q, const int64_t* q_strides, const void* kv,
                                      const int64_t* kv_strides, int64_t N_kv, const void* kv2,
                                      const int64_t* kv2_strides, int64_t N_kv2, const float* attn_sink,
                                      const int32_t* topk_idxs, const int64_t* idx_strides, int64_t B, int64_t S,
                                      int64_t H, int64_t D, int64_t K, float softmax_scale, int qkv_dtype, void* o,
                                      const int64_t* o_strides, float* lse, const int64_t* lse_strides,
                                      const int32_t* row_len, const int64_t* row_len_strides, void* stream) {
  if (B > 0 && S > 0 && N_kv2 > 0 && !kv2) return set_error(SI_ERR_INVALID, "null pointer argument");
  // (a null kv2 with no rows is the one-tensor case)
  return sparse_attn_fwd_entry(q, q_strides, kv, kv_strides, N_kv, N_kv2 > 0 ? kv2 : nullptr, kv2_strides, N_kv2,
                               attn_sink, topk_idxs, 0, idx_strides, B, S, H, D, K, softmax_scale, qkv_dtype, o,
                               o_strides, lse, lse_strides, row_len, row_len_strides, stream);
}

extern "C" int si_sparse_attn_fwd(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                                  const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                                  const int64_t* idx_strides, int64_t B, int64_t S, int64_t H, int64_t D,
                                  int64_t N_kv, int64_t K, float softmax_scale, int qkv_dtype, void* o,
                                  const int64_t* o_strides, float* lse, const int64_t* lse_strides, void* stream) {
  return si_sparse_attn_fwd_ragged(q, q_strides, kv, kv_strides, attn_sink, topk_idxs, idx_is_i64, idx_strides, B, S,
                                   H, D, N_kv, K, softmax_scale, qkv_dtype, o, o_strides, lse, lse_strides, nullptr,
                                   nullptr, stream);
}
