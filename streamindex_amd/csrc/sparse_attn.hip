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
// Design (one query row per workgroup, 16 heads per wavefront):
//   * The row's top-k KV rows are gathered TK = 32 at a time from HBM/L2 with
//     16-byte loads (each row read once per query, not once per head block)
//     and written to LDS twice: key-major (swizzled) for the score MFMAs and
//     dim-major (transposed in registers) for the P·V MFMAs.
//   * Scores are computed transposed, S^T = KV·Q^T with
//     v_mfma_f32_16x16x32_bf16 (keys on M, heads on N), so each lane holds one
//     head: the online-softmax max/sum stay in-lane plus two xor exchanges.
//   * O^T = V^T·P^T uses the score accumulators directly as the B operand
//     (keys permuted consistently in both operands), and its output layout
//     puts one head per lane again, so the rescale by e^{m_old-m_new} is
//     lane-local.  Q lives in VGPRs for the whole row.
#include <string>

#include "si_common.h"
#include "si_status.h"

namespace si {

struct SparseAttnArgs {
  const uint16_t* q;  // [B,S,H,D] bf16
  int64_t qsb, qss, qsh;
  const uint16_t* kv;  // [B,N,D] bf16
  int64_t kvsb, kvsn;
  const float* sink;   // [H]
  const void* idx;     // [B,S,K] int32 / int64
  int idx64;
  int64_t isb, iss, isk;
  uint16_t* o;         // [B,S,H,D] bf16
  int64_t osb, oss, osh;
  float* lse;          // [B,S,H]
  int64_t lsb, lss, lsh;
  int B, S, H, N, K;
  float scale_log2;    // softmax_scale * log2(e)
};

constexpr int kTK = 32;  // keys per tile

template <int D>
__device__ __forceinline__ int kmaj_off(int key, int c) {
  constexpr int CPR = D / 8;
  constexpr int SW = CPR < 8 ? CPR : 8;
  return key * (D * 2) + ((c ^ (key % SW)) << 4);
}

// V^T rows hold kTK keys (64 bytes) padded to 72 bytes to stagger banks.
constexpr int kVRow = kTK * 2 + 8;

__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
  // round-to-nearest-even to bf16 (finite values)
  uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
  ua = (ua + 0x7fffu + ((ua >> 16) & 1u)) >> 16;
  ub = (ub + 0x7fffu + ((ub >> 16) & 1u)) >> 16;
  return ua | (ub << 16);
}

template <int D>
__global__ __launch_bounds__(512) void sparse_attn_fwd_kernel(SparseAttnArgs a) {
  constexpr int KS = D / 32;  // k-steps of the score MFMA
  constexpr int MD = D / 16;  // 16-dim blocks of the output MFMA
  constexpr int CPR = D / 8;
  __shared__ __attribute__((aligned(16))) char kmaj[kTK * D * 2];
  __shared__ __attribute__((aligned(16))) char vt[D * kVRow];
  __shared__ int sidx[kTK];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;     // lane group 0..3
  const int hl = lane & 15;    // head within the wave's 16
  const int nthreads = blockDim.x;
  const int s = blockIdx.x % a.S;
  const int b = blockIdx.x / a.S;
  const int h = wave * 16 + hl;
  const bool hvalid = h < a.H;

  // Q^T B-fragments: head h, dims 32ks + 8g .. +8.
  bf16x8 qf[KS];
  {
    const uint16_t* qrow = a.q + b * a.qsb + static_cast<int64_t>(s) * a.qss + static_cast<int64_t>(h) * a.qsh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks] = hvalid ? *reinterpret_cast<const bf16x8*>(qrow + ks * 32 + g * 8) : bf16x8{};
    }
  }

  f32x4 acc[MD];
#pragma unroll
  for (int md = 0; md < MD; ++md) acc[md] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -1.0e30f;  // running max (log2 domain), one head per lane
  float l_run = 0.f;       // this lane's share of the running denominator

  const char* idx_row = static_cast<const char*>(a.idx) +
                        (b * a.isb + static_cast<int64_t>(s) * a.iss) * (a.idx64 ? 8 : 4);
  const uint16_t* kvb = a.kv + b * a.kvsb;
  const int ntiles = (a.K + kTK - 1) / kTK;

  for (int it = 0; it < ntiles; ++it) {
    const int k0 = it * kTK;
    if (threadIdx.x < kTK) {
      const int j = k0 + threadIdx.x;
      int t = -1;
      if (j < a.K) {
        const int64_t off = static_cast<int64_t>(j) * a.isk;
        const int64_t v = a.idx64 ? reinterpret_cast<const int64_t*>(idx_row)[off]
                                  : static_cast<int64_t>(reinterpret_cast<const int32_t*>(idx_row)[off]);
        t = (v >= 0 && v < a.N) ? static_cast<int>(v) : -1;
      }
      sidx[threadIdx.x] = t;
    }
    __syncthreads();

    // Gather: block = 4 keys x 8 dims; key-major copy + transposed copy.
    for (int blk = threadIdx.x; blk < (kTK / 4) * CPR; blk += nthreads) {
      const int kg = blk / CPR, c = blk % CPR;
      u32x4 r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = sidx[kg * 4 + j];
        r[j] = t >= 0 ? *reinterpret_cast<const u32x4*>(kvb + static_cast<int64_t>(t) * a.kvsn + c * 8)
                      : u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(kmaj + kmaj_off<D>(kg * 4 + j, c)) = r[j];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // dims c*8 + 2e (low halves) and c*8 + 2e + 1 (high halves)
        uint2 lo2, hi2;
        lo2.x = pack_lo(r[0][e], r[1][e]);
        lo2.y = pack_lo(r[2][e], r[3][e]);
        hi2.x = pack_hi(r[0][e], r[1][e]);
        hi2.y = pack_hi(r[2][e], r[3][e]);
        *reinterpret_cast<uint2*>(vt + (c * 8 + 2 * e) * kVRow + kg * 8) = lo2;
        *reinterpret_cast<uint2*>(vt + (c * 8 + 2 * e + 1) * kVRow + kg * 8) = hi2;
      }
    }
    __syncthreads();

    // S^T = KV_tile · Q^T : keys 16mb + 4g + i, head hl.
    f32x4 st[2];
    st[0] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kmaj + kmaj_off<D>(mb * 16 + hl, ks * 4 + g));
        st[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], st[mb], 0, 0, 0);
      }
    }

    float tmax = -1.0e30f;
    float sv[2][4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = sidx[mb * 16 + g * 4 + i] >= 0;
        const float x = valid ? st[mb][i] * a.scale_log2 : -__builtin_inff();
        sv[mb][i] = x;
        tmax = __builtin_fmaxf(tmax, x);
      }
    }
    tmax = __builtin_fmaxf(tmax, shfl_xor_f32(tmax, lane, 16));
    tmax = __builtin_fmaxf(tmax, shfl_xor_f32(tmax, lane, 32));
    const float m_new = __builtin_fmaxf(m_run, tmax);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;

    float psum = 0.f;
    float p[2][4];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[mb][i] = __builtin_amdgcn_exp2f(sv[mb][i] - m_new);
        psum += p[mb][i];
      }
    }
    l_run = l_run * alpha + psum;

    // P^T B-fragment: k-slots 8g+0..3 <-> keys 4g+0..3, 8g+4..7 <-> keys 16+4g+0..3.
    bf16x8 pf;
    {
      u32x4 w;
      w[0] = f32x2_to_bf16x2(p[0][0], p[0][1]);
      w[1] = f32x2_to_bf16x2(p[0][2], p[0][3]);
      w[2] = f32x2_to_bf16x2(p[1][0], p[1][1]);
      w[3] = f32x2_to_bf16x2(p[1][2], p[1][3]);
      pf = __builtin_bit_cast(bf16x8, w);
    }

    // O^T[dims, heads] = alpha * O^T + V^T · P^T
#pragma unroll
    for (int md = 0; md < MD; ++md) {
      const char* vrow = vt + (md * 16 + hl) * kVRow;
      const uint2 v0 = *reinterpret_cast<const uint2*>(vrow + g * 8);
      const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 32 + g * 8);
      u32x4 vw;
      vw[0] = v0.x; vw[1] = v0.y; vw[2] = v1.x; vw[3] = v1.y;
      const bf16x8 vf = __builtin_bit_cast(bf16x8, vw);
      acc[md] = acc[md] * alpha;
      acc[md] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, acc[md], 0, 0, 0);
    }
    __syncthreads();
  }

  // Finish: total denominator over the four lane groups, then the sink.
  float l_tot = l_run + shfl_xor_f32(l_run, lane, 16);
  l_tot = l_tot + shfl_xor_f32(l_tot, lane, 32);
  constexpr float kLog2e = 1.4426950408889634f;
  const float sink2 = hvalid ? a.sink[h] * kLog2e : -__builtin_inff();
  const float m_fin = __builtin_fmaxf(m_run, sink2);
  const float resc = __builtin_amdgcn_exp2f(m_run - m_fin);
  const float l_fin = l_tot * resc + __builtin_amdgcn_exp2f(sink2 - m_fin);
  const float inv = l_fin > 0.f ? resc / l_fin : 0.f;

  if (hvalid) {
    uint16_t* orow = a.o + b * a.osb + static_cast<int64_t>(s) * a.oss + static_cast<int64_t>(h) * a.osh;
#pragma unroll
    for (int md = 0; md < MD; ++md) {
      uint2 w;
      w.x = f32x2_to_bf16x2(acc[md][0] * inv, acc[md][1] * inv);
      w.y = f32x2_to_bf16x2(acc[md][2] * inv, acc[md][3] * inv);
      *reinterpret_cast<uint2*>(orow + md * 16 + g * 4) = w;
    }
    if (g == 0) {
      constexpr float kLn2 = 0.6931471805599453f;
      const float lse = l_fin > 0.f ? (__builtin_amdgcn_logf(l_fin) + m_fin) * kLn2 : -1.0e30f;
      a.lse[b * a.lsb + static_cast<int64_t>(s) * a.lss + static_cast<int64_t>(h) * a.lsh] = lse;
    }
  }
}

template <int D>
static int launch_attn(const SparseAttnArgs& a, hipStream_t st) {
  const int nw = (a.H + 15) / 16;
  const int64_t nblk = static_cast<int64_t>(a.B) * a.S;
  if (nblk > 0x7fffffffLL) return set_error(SI_ERR_UNSUPPORTED, "grid too large");
  hipLaunchKernelGGL((sparse_attn_fwd_kernel<D>), dim3(static_cast<unsigned>(nblk)), dim3(nw * 64), 0, st, a);
  return check_launch("sparse_attn_fwd_kernel");
}

}  // namespace si

using namespace si;

extern "C" int si_sparse_attn_fwd(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                                  const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                                  const int64_t* idx_strides, int64_t B, int64_t S, int64_t H, int64_t D,
                                  int64_t N_kv, int64_t K, float softmax_scale, void* o, const int64_t* o_strides,
                                  float* lse, const int64_t* lse_strides, void* stream) {
  if (!q_strides || !kv_strides || !idx_strides || !o_strides || !lse_strides)
    return set_error(SI_ERR_INVALID, "null stride argument");
  if (B < 0 || S < 0 || H <= 0 || D <= 0 || N_kv < 0 || K < 0) return set_error(SI_ERR_INVALID, "bad dimension");
  // Empty tensors may carry a null data pointer; only non-empty ones are dereferenced.
  const bool rows = B > 0 && S > 0;
  if (rows && (!q || !attn_sink || !o || !lse || (K > 0 && !topk_idxs) || (N_kv > 0 && !kv)))
    return set_error(SI_ERR_INVALID, "null pointer argument");
  if (B > 0x7fffffff || S > 0x7fffffff || N_kv > 0x7fffffff || K > 0x7fffffff)
    return set_error(SI_ERR_UNSUPPORTED, "dimension exceeds int32");
  if (H > 128) return set_error(SI_ERR_UNSUPPORTED, "H > 128 is not supported");
  if (q_strides[3] != 1 || kv_strides[2] != 1 || o_strides[3] != 1)
    return set_error(SI_ERR_INVALID, "q, kv and o need a contiguous last dimension");
  if ((q_strides[0] | q_strides[1] | q_strides[2] | kv_strides[0] | kv_strides[1]) % 8)
    return set_error(SI_ERR_INVALID, "q/kv strides must be multiples of 8 elements");
  if ((o_strides[0] | o_strides[1] | o_strides[2]) % 4) return set_error(SI_ERR_INVALID, "o strides must be multiples of 4");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kv)) & 15)
    return set_error(SI_ERR_INVALID, "q/kv must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(o) & 7) return set_error(SI_ERR_INVALID, "o must be 8-byte aligned");
  SparseAttnArgs a{};
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
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
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
