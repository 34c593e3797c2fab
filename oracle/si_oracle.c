/*
 * CPU oracle for the StreamIndex CSA hot path.  TEST INFRASTRUCTURE ONLY:
 * this file is the checker that tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py compare the HIP kernels against.  No product
 * code path links, loads or calls it.
 *
 * It restates, from scratch, the reference's materialise-then-topk path:
 *   score      flash_sparse/reference.py:138-168   (eq. 16, fp32 einsum -> relu -> w-sum)
 *   mask/topk  eval/test_v4_indexer_parity.py:111-137 (illegal t >= (s+1)//ratio -> -inf,
 *              topk(min(k,T)), post-mask -> -1)
 *   tie order  docs/streaming_topk.md:46-60,301-312 (score desc, index asc)
 *   attention  flash_sparse/reference.py:44-130 (gather, sink-augmented softmax)
 *              flash_sparse/triton/sparse_attn_fwd.py:148-177 (LSE, -1e30 when empty)
 *   backward   flash_sparse/triton/sparse_attn_bwd.py:1-26,93-97,224-283 (from saved o, lse)
 *
 * Arithmetic: bf16 inputs are widened exactly; every dot product and every
 * head/key sum is accumulated in double, which is at least as accurate as the
 * reference's fp32 einsum and gives the "true" value the kernels are judged
 * against.  A float-accumulation variant of the score mirrors the reference's
 * working precision for gap diagnostics.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = ((uint32_t)b) << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* IEEE binary16 bits to float (exact: every fp16 value is an fp32 value).
 * Subnormals are man * 2^-24; exponent 31 is inf / NaN. */
static inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t ex = (h >> 10) & 0x1Fu;
  const uint32_t man = h & 0x3FFu;
  uint32_t u;
  if (ex == 0) {
    const float mag = (float)man * 5.9604644775390625e-08f; /* 2^-24 */
    memcpy(&u, &mag, sizeof u);
    u |= sign;
  } else if (ex == 31) {
    u = sign | 0x7F800000u | (man << 13);
  } else {
    u = sign | ((ex + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* A sparse-attention operand element: bf16 (f16 = 0) or fp16 (f16 = 1) bits. */
static inline double elem(uint16_t b, int f16) { return f16 ? (double)f16_to_f32(b) : (double)bf16_to_f32(b); }

void oracle_f16_to_f32(const uint16_t* h, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(h[i]);
}

/*
 * Scores of `nrows` query rows against the keys of one batch.
 *   q   [S, H, D] bf16 bits       k [T, D] bf16 bits       w [S, H] fp32
 *   rows[i] selects the query row; out [nrows, T] (double).
 *   lim: NULL, or per row the number of leading keys to score (the causal
 *        limit); out[r, t] for t >= lim[r] is set to NaN (never a legal key).
 * Follows reference.py:165-168: relu per head, then the weighted head sum.
 * Every (row, key) value is accumulated in a fixed order (d ascending inside
 * a head, heads ascending); keys are processed KB at a time so the compiler
 * vectorises across keys without reordering any single key's sums.
 */
#define SI_KB 8
typedef double si_v4d __attribute__((vector_size(32)));
typedef long long si_v4l __attribute__((vector_size(32)));
void oracle_indexer_scores_lim(const uint16_t* q, const uint16_t* k, const float* w, int64_t S, int64_t T,
                               int64_t H, int64_t D, const int64_t* rows, int64_t nrows, const int64_t* lim,
                               double* out) {
  (void)S;
  const int64_t nb = (T + SI_KB - 1) / SI_KB;
  /* keys transposed in blocks of SI_KB: kb[(b*D + d)*SI_KB + j] = k[b*SI_KB + j, d] (0 past T) */
  double* kb = (double*)aligned_alloc(32, sizeof(double) * (size_t)(nb * D * SI_KB + 4));
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nb; ++b)
    for (int64_t d = 0; d < D; ++d)
      for (int64_t j = 0; j < SI_KB; ++j) {
        const int64_t t = b * SI_KB + j;
        kb[(b * D + d) * SI_KB + j] = t < T ? (double)bf16_to_f32(k[t * D + d]) : 0.0;
      }
#pragma omp parallel
  {
    double* qd = (double*)malloc(sizeof(double) * (size_t)(H * D));
#pragma omp for schedule(dynamic, 1)
    for (int64_t r = 0; r < nrows; ++r) {
      const int64_t s = rows[r];
      for (int64_t i = 0; i < H * D; ++i) qd[i] = (double)bf16_to_f32(q[s * H * D + i]);
      const float* ws = w + s * H;
      int64_t L = lim ? lim[r] : T;
      L = L < 0 ? 0 : (L > T ? T : L);
      const int64_t nbr = (L + SI_KB - 1) / SI_KB;
      for (int64_t b = 0; b < nbr; ++b) {
        const si_v4d* kblk = (const si_v4d*)(kb + b * D * SI_KB);
        si_v4d acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = acc0;
        const si_v4d zero = acc0;
        for (int64_t h = 0; h < H; ++h) {
          const double* qh = qd + h * D;
          si_v4d dot0 = zero, dot1 = zero;
          for (int64_t d = 0; d < D; ++d) {
            const double qv = qh[d];
            dot0 += qv * kblk[2 * d];
            dot1 += qv * kblk[2 * d + 1];
          }
          const double wh = (double)ws[h];
          /* relu: the weighted term where dot > 0, else +0.0 (bit mask) */
          acc0 += (si_v4d)((si_v4l)(wh * dot0) & (dot0 > zero));
          acc1 += (si_v4d)((si_v4l)(wh * dot1) & (dot1 > zero));
        }
        for (int j = 0; j < SI_KB; ++j) {
          const int64_t t = b * SI_KB + j;
          if (t < L) out[r * T + t] = j < 4 ? acc0[j] : acc1[j - 4];
        }
      }
      for (int64_t t = L; t < T; ++t) out[r * T + t] = NAN;
    }
    free(qd);
  }
  free(kb);
}

void oracle_indexer_scores(const uint16_t* q, const uint16_t* k, const float* w, int64_t S, int64_t T,
                           int64_t H, int64_t D, const int64_t* rows, int64_t nrows, double* out) {
  oracle_indexer_scores_lim(q, k, w, S, T, H, D, rows, nrows, NULL, out);
}

/* Same as above in float accumulation (the reference's working precision). */
void oracle_indexer_scores_f32(const uint16_t* q, const uint16_t* k, const float* w, int64_t S, int64_t T,
                               int64_t H, int64_t D, const int64_t* rows, int64_t nrows, float* out) {
  (void)S;
  float* kf = (float*)malloc(sizeof(float) * (size_t)(T * D));
  for (int64_t i = 0; i < T * D; ++i) kf[i] = bf16_to_f32(k[i]);
#pragma omp parallel
  {
    float* qf = (float*)malloc(sizeof(float) * (size_t)(H * D));
#pragma omp for schedule(dynamic, 1)
    for (int64_t r = 0; r < nrows; ++r) {
      const int64_t s = rows[r];
      for (int64_t i = 0; i < H * D; ++i) qf[i] = bf16_to_f32(q[s * H * D + i]);
      const float* ws = w + s * H;
      for (int64_t t = 0; t < T; ++t) {
        const float* kt = kf + t * D;
        float acc = 0.0f;
        for (int64_t h = 0; h < H; ++h) {
          const float* qh = qf + h * D;
          float dot = 0.0f;
          for (int64_t d = 0; d < D; ++d) dot += qh[d] * kt[d];
          acc += ws[h] * (dot > 0.0f ? dot : 0.0f);
        }
        out[r * T + t] = acc;
      }
    }
    free(qf);
  }
  free(kf);
}

typedef struct {
  double v;
  int64_t i;
} si_pair;

/* (score desc, index asc): docs/streaming_topk.md:46-60. */
static int cmp_pair(const void* a, const void* b) {
  const si_pair* x = (const si_pair*)a;
  const si_pair* y = (const si_pair*)b;
  if (x->v > y->v) return -1;
  if (x->v < y->v) return 1;
  return (x->i < y->i) ? -1 : (x->i > y->i);
}

/*
 * Per-row top-k over legal keys.
 *   scores [nrows, T]; legal key t of row r: t < lim[r] and (mask == NULL or mask[r*T+t]).
 *   Output width top_k; positions past the number of legal keys get index -1
 *   and score -inf (eval/test_v4_indexer_parity.py:124-136 and the chunked
 *   driver's isinf -> -1 rule, chunked_indexer.py:154-155).
 */
void oracle_topk(const double* scores, int64_t nrows, int64_t T, const int64_t* lim, const uint8_t* mask,
                 int64_t top_k, int64_t* out_idx, double* out_score) {
#pragma omp parallel
  {
    si_pair* buf = (si_pair*)malloc(sizeof(si_pair) * (size_t)(T > 0 ? T : 1));
#pragma omp for schedule(dynamic, 4)
    for (int64_t r = 0; r < nrows; ++r) {
      int64_t n = 0;
      const int64_t L = lim[r] < T ? lim[r] : T;
      for (int64_t t = 0; t < L; ++t) {
        if (mask && !mask[r * T + t]) continue;
        buf[n].v = scores[r * T + t];
        buf[n].i = t;
        ++n;
      }
      qsort(buf, (size_t)n, sizeof(si_pair), cmp_pair);
      for (int64_t j = 0; j < top_k; ++j) {
        if (j < n) {
          out_idx[r * top_k + j] = buf[j].i;
          out_score[r * top_k + j] = buf[j].v;
        } else {
          out_idx[r * top_k + j] = -1;
          out_score[r * top_k + j] = -INFINITY;
        }
      }
    }
    free(buf);
  }
}

/*
 * Sparse attention with attention sink, MQA layout (reference.py:93-130), for
 * `nrows` query rows of one batch.
 *   q [nrows, H, D], kv [N, D]: bf16 bits (f16 = 0) or fp16 bits (f16 = 1);
 *   sink [H] fp32; idx [nrows, K] int64 (-1 = masked).  Out: o [nrows, H, D],
 *   lse [nrows, H].
 * The sink enters the denominator only.  LSE = log(sum) + max as in
 * sparse_attn_fwd.py:174-177 (sink included in the sum).
 */
void oracle_sparse_attn_t(const uint16_t* q, const uint16_t* kv, const float* sink, const int64_t* idx,
                          int64_t nrows, int64_t H, int64_t D, int64_t N, int64_t K, double scale, int f16,
                          double* o, double* lse) {
#pragma omp parallel
  {
    double* sc = (double*)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
    double* qd = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int64_t r = 0; r < nrows; ++r) {
      const int64_t* ir = idx + r * K;
      for (int64_t h = 0; h < H; ++h) {
        const uint16_t* qh = q + (r * H + h) * D;
        for (int64_t d = 0; d < D; ++d) qd[d] = elem(qh[d], f16);
        double mx = (double)sink[h];
        for (int64_t j = 0; j < K; ++j) {
          const int64_t t = ir[j];
          if (t < 0 || t >= N) {
            sc[j] = -INFINITY;
            continue;
          }
          const uint16_t* kr = kv + t * D;
          double dot = 0.0;
          for (int64_t d = 0; d < D; ++d) dot += qd[d] * elem(kr[d], f16);
          sc[j] = dot * scale;
          if (sc[j] > mx) mx = sc[j];
        }
        double* oh = o + (r * H + h) * D;
        for (int64_t d = 0; d < D; ++d) oh[d] = 0.0;
        if (mx == -INFINITY) {
          /* No valid key and a -inf sink: zero output and the kernel's
           * "empty" LSE sentinel (sparse_attn_fwd.py:159-161,174-175). */
          lse[r * H + h] = -1.0e30;
          continue;
        }
        double den = exp((double)sink[h] - mx);
        for (int64_t j = 0; j < K; ++j) {
          if (sc[j] == -INFINITY) continue;
          const double p = exp(sc[j] - mx);
          den += p;
          const uint16_t* kr = kv + ir[j] * D;
          for (int64_t d = 0; d < D; ++d) oh[d] += p * elem(kr[d], f16);
        }
        for (int64_t d = 0; d < D; ++d) oh[d] /= den;
        lse[r * H + h] = log(den) + mx;
      }
    }
    free(sc);
    free(qd);
  }
}

void oracle_sparse_attn(const uint16_t* q, const uint16_t* kv, const float* sink, const int64_t* idx,
                        int64_t nrows, int64_t H, int64_t D, int64_t N, int64_t K, double scale,
                        double* o, double* lse) {
  oracle_sparse_attn_t(q, kv, sink, idx, nrows, H, D, N, K, scale, 0, o, lse);
}

/*
 * Sparse-attention backward for `nrows` query rows of one batch, from the
 * forward's saved outputs, as the reference backward consumes them:
 *   maths      flash_sparse/triton/sparse_attn_bwd.py:1-26
 *   delta      sparse_attn_bwd.py:93-97   (sum_d o*do in fp32 from bf16 o, do)
 *   gradients  sparse_attn_bwd.py:247-283 (p = exp(s - lse), dp = p (do.v - delta) scale,
 *              dq = dp.kv, dkv[idx] += dp^T q + p^T do)
 *   dsink      sparse_attn_bwd.py:224-228 (-exp(sink - lse) delta, summed over rows)
 *   q, o, dout [nrows,H,D], kv [N,D]: bf16 bits (f16 = 0) or fp16 bits (f16 = 1); sink [H] fp32;
 *   lse [nrows,H] fp32; idx [nrows,K] int64 (-1 or out of range = masked).
 * Outputs, each optional (NULL = not wanted):
 *   dq    [nrows,H,D]  written;
 *   dkv   [nslot,D]    ACCUMULATED for keys t with key_slot[t] >= 0 into row
 *                      key_slot[t] (key_slot NULL: slot t, nslot = N);
 *   dsink [H]          ACCUMULATED (-sum_rows e^{sink-lse} delta).
 * A key listed twice in a row contributes twice, as the reference's
 * per-slot atomic adds do.  All sums in double.
 */
void oracle_sparse_attn_bwd_t(const uint16_t* q, const uint16_t* kv, const uint16_t* o, const uint16_t* dout,
                              const float* sink, const float* lse, const int64_t* idx, int64_t nrows, int64_t H,
                              int64_t D, int64_t N, int64_t K, double scale, const int64_t* key_slot, int64_t nslot,
                              int f16, double* dq, double* dkv, double* dsink) {
  const int pairs = dq != NULL || (dkv != NULL && nslot > 0);
#pragma omp parallel
  {
    double* qd = (double*)malloc(sizeof(double) * (size_t)D);
    double* gd = (double*)malloc(sizeof(double) * (size_t)D);
    double* kd = (double*)malloc(sizeof(double) * (size_t)D);
    double* my_dkv = dkv ? (double*)calloc((size_t)(nslot > 0 ? nslot : 1) * (size_t)D, sizeof(double)) : NULL;
    double* my_ds = (double*)calloc((size_t)H, sizeof(double));
#pragma omp for schedule(dynamic, 1)
    for (int64_t r = 0; r < nrows; ++r) {
      const int64_t* ir = idx + r * K;
      for (int64_t h = 0; h < H; ++h) {
        const int64_t rh = r * H + h;
        const double l = (double)lse[rh];
        double delta = 0.0;
        for (int64_t d = 0; d < D; ++d)
          delta += elem(o[rh * D + d], f16) * elem(dout[rh * D + d], f16);
        my_ds[h] -= exp((double)sink[h] - l) * delta;
        if (!pairs) continue;
        for (int64_t d = 0; d < D; ++d) {
          qd[d] = elem(q[rh * D + d], f16);
          gd[d] = elem(dout[rh * D + d], f16);
        }
        double* dqh = dq ? dq + rh * D : NULL;
        if (dqh) for (int64_t d = 0; d < D; ++d) dqh[d] = 0.0;
        for (int64_t j = 0; j < K; ++j) {
          const int64_t t = ir[j];
          if (t < 0 || t >= N) continue;
          const int64_t slot = key_slot ? key_slot[t] : t;
          if (!dqh && slot < 0) continue;
          const uint16_t* kr = kv + t * D;
          double qk = 0.0, gk = 0.0;
          for (int64_t d = 0; d < D; ++d) {
            kd[d] = elem(kr[d], f16);
            qk += qd[d] * kd[d];
            gk += gd[d] * kd[d];
          }
          const double p = exp(scale * qk - l);
          const double ds = p * (gk - delta) * scale; /* d loss / d (q.k) */
          if (dqh) for (int64_t d = 0; d < D; ++d) dqh[d] += ds * kd[d];
          if (my_dkv && slot >= 0) {
            double* acc = my_dkv + slot * D;
            for (int64_t d = 0; d < D; ++d) acc[d] += ds * qd[d] + p * gd[d];
          }
        }
      }
    }
#pragma omp critical
    {
      if (dkv)
        for (int64_t e = 0; e < nslot * D; ++e) dkv[e] += my_dkv[e];
      if (dsink)
        for (int64_t h = 0; h < H; ++h) dsink[h] += my_ds[h];
    }
    free(qd);
    free(gd);
    free(kd);
    free(my_dkv);
    free(my_ds);
  }
}

void oracle_sparse_attn_bwd(const uint16_t* q, const uint16_t* kv, const uint16_t* o, const uint16_t* dout,
                            const float* sink, const float* lse, const int64_t* idx, int64_t nrows, int64_t H,
                            int64_t D, int64_t N, int64_t K, double scale, const int64_t* key_slot, int64_t nslot,
                            double* dq, double* dkv, double* dsink) {
  oracle_sparse_attn_bwd_t(q, kv, o, dout, sink, lse, idx, nrows, H, D, N, K, scale, key_slot, nslot, 0, dq, dkv,
                           dsink);
}

/*
 * Counter-based N(0,1) draws: the CPU restatement of the generator in
 * streamindex_amd/csrc/synth.hip (Philox4x32-10 as published by Salmon et al.,
 * SC 2011; Box-Muller with ln / sin / cos, reciprocal and square root built
 * from additions, multiplies and fused multiply-adds only), so a slice of any
 * synthetic tensor can be recomputed here bit for bit.  Element i of (seed, stream): counter (i/4, stream, 0),
 * word pair (2 (i%4 / 2), +1), cosine for even i%4, sine for odd.
 */
static void syn_philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

static float syn_u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}
static uint32_t syn_f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

static float syn_recip(float d) {
  float y = fmaf(-0.225f, d, 0.96f);
  for (int i = 0; i < 3; ++i) y = fmaf(y, fmaf(-d, y, 1.0f), y);
  return y;
}

static float syn_sqrt(float t) {
  if (!(t > 0.0f)) return 0.0f;
  float y = syn_u2f(0x5F3759DFu - (syn_f2u(t) >> 1));
  const float h = 0.5f * t;
  for (int i = 0; i < 3; ++i) y = y * fmaf(-(h * y), y, 1.5f);
  return t * y;
}

static float syn_log(float u) {
  const uint32_t b = syn_f2u(u);
  int e = (int)(b >> 23) - 127;
  float m = syn_u2f((b & 0x7FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) * syn_recip(m + 1.0f);
  const float s2 = s * s;
  float p = fmaf(s2, 0.18181818f, 0.22222222f);
  p = fmaf(s2, p, 0.28571429f);
  p = fmaf(s2, p, 0.4f);
  p = fmaf(s2, p, 0.66666667f);
  const float lnm = fmaf(s * s2, p, 2.0f * s);
  const float ef = (float)e;
  return fmaf(ef, 0.693145752f, fmaf(ef, 1.42860677e-06f, lnm));
}

static void syn_sincos(float phi, float* c, float* s) {
  const float x2 = phi * phi;
  float pc = fmaf(x2, 2.08767570e-09f, -2.75573192e-07f);
  pc = fmaf(x2, pc, 2.48015873e-05f);
  pc = fmaf(x2, pc, -1.38888889e-03f);
  pc = fmaf(x2, pc, 4.16666667e-02f);
  pc = fmaf(x2, pc, -0.5f);
  *c = fmaf(x2, pc, 1.0f);
  float ps = fmaf(x2, -2.50521084e-08f, 2.75573192e-06f);
  ps = fmaf(x2, ps, -1.98412698e-04f);
  ps = fmaf(x2, ps, 8.33333333e-03f);
  ps = fmaf(x2, ps, -0.166666667f);
  *s = fmaf(phi * x2, ps, phi);
}

static void syn_box_muller(uint32_t x, uint32_t y, float* n0, float* n1) {
  const float u1 = (float)((x >> 8) + 1u) * 5.9604644775390625e-08f;
  const float r = syn_sqrt(-2.0f * syn_log(u1));
  const uint32_t y24 = y >> 8;
  const uint32_t quad = y24 >> 22;
  const float phi = (float)(y24 & 0x3FFFFFu) * 2.384185791015625e-07f * 1.57079637f;
  float c, s, cs, sn;
  syn_sincos(phi, &c, &s);
  if (quad == 0) {
    cs = c; sn = s;
  } else if (quad == 1) {
    cs = -s; sn = c;
  } else if (quad == 2) {
    cs = -c; sn = -s;
  } else {
    cs = s; sn = -c;
  }
  *n0 = r * cs;
  *n1 = r * sn;
}

static void syn_quad(uint64_t q, uint32_t k0, uint32_t k1, uint32_t stream, float v[4]) {
  uint32_t c[4] = {(uint32_t)q, (uint32_t)(q >> 32), stream, 0u};
  syn_philox(c, k0, k1);
  syn_box_muller(c[0], c[1], &v[0], &v[1]);
  syn_box_muller(c[2], c[3], &v[2], &v[3]);
}

static uint16_t syn_bf16(float f) {
  const uint32_t u = syn_f2u(f);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* Elements [start, start + n) scaled: fp32 (out32) or bf16 bits (out16); the other may be NULL. */
void oracle_fill_normal(int64_t start, int64_t n, uint64_t seed, uint32_t stream, float scale, float* out32,
                        uint16_t* out16) {
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const int64_t g = start + i;
    float v[4];
    syn_quad((uint64_t)g >> 2, k0, k1, stream, v);
    const float x = v[g & 3] * scale;
    if (out32) out32[i] = x;
    if (out16) out16[i] = syn_bf16(x);
  }
}

/*
 * Digest of a whole synthetic tensor of n elements (dtype 0 fp32, 1 bf16),
 * over its little-endian 16-bit words w_j: d1 = sum w_j, d2 = sum w_j (j mod
 * 65521 + 1), both mod 2^64.
 */
void oracle_normal_digest(int dtype, int64_t n, uint64_t seed, uint32_t stream, float scale, uint64_t* d1,
                          uint64_t* d2) {
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const int64_t nq = (n + 3) / 4;
  uint64_t a = 0, b = 0;
#pragma omp parallel for schedule(static) reduction(+ : a, b)
  for (int64_t q = 0; q < nq; ++q) {
    float v[4];
    syn_quad((uint64_t)q, k0, k1, stream, v);
    for (int t = 0; t < 4; ++t) {
      const int64_t i = q * 4 + t;
      if (i >= n) break;
      const float x = v[t] * scale;
      if (dtype == 1) {
        const uint64_t w = syn_bf16(x);
        a += w;
        b += w * (uint64_t)(i % 65521 + 1);
      } else {
        const uint32_t u = syn_f2u(x);
        const uint64_t lo = u & 0xFFFFu, hi = u >> 16;
        const int64_t j = 2 * i;
        a += lo + hi;
        b += lo * (uint64_t)(j % 65521 + 1) + hi * (uint64_t)((j + 1) % 65521 + 1);
      }
    }
  }
  *d1 = a;
  *d2 = b;
}

/* One Philox4x32-10 block (the bijection the generator draws from). */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
  syn_philox(c, key[0], key[1]);
  memcpy(out, c, sizeof c);
}

/* Synthetic elements at arbitrary flat indices idx[0..n), scaled; fp32 or bf16 bits. */
void oracle_fill_normal_at(const int64_t* idx, int64_t n, uint64_t seed, uint32_t stream, float scale, float* out32,
                           uint16_t* out16) {
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const int64_t g = idx[i];
    float v[4];
    syn_quad((uint64_t)g >> 2, k0, k1, stream, v);
    const float x = v[g & 3] * scale;
    if (out32) out32[i] = x;
    if (out16) out16[i] = syn_bf16(x);
  }
}
