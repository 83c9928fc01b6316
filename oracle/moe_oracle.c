/*
 * moe_oracle.c -- CPU restatement of the reference's MoE block arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  See moe_oracle.h for the contract,
 * the layouts and the reference citations.  Compiled with -O3
 * -ffp-contract=off and without fast-math, so every rounding below is the one
 * written: the only fused operations are the explicit fmaf() calls and the
 * _mm256_fmadd_ps() lanes that compute exactly the same fmaf().
 *
 * Pinning (no reference golden vector exists for this path): every function
 * here is checked by tests/test_oracle_pinning.py against closed forms,
 * float64 references, brute-force enumeration and special cases.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

static int g_force_scalar = 0;
static int g_threads = 0;

void orc_force_scalar(int on) { g_force_scalar = on; }

void orc_set_threads(int n) { g_threads = n; }

int orc_get_threads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* GEMM with one sequential fmaf chain per output (k ascending, from 0.0f).  */
/* Blocking over k keeps each chain's order: the running sum is parked in a  */
/* float buffer between k-blocks and resumed, which is exactly what the      */
/* register would have held.                                                 */
/* ------------------------------------------------------------------------ */

enum { MR = 8, NR = 8, MB = 64, NB = 64, KB = 256 };

/* acc[j][i] += sum over k in [0,kc) of P[k][i] * Bj[k], one fmaf per step. */
static void micro_scalar(const float *P, const float *const *Bj, int64_t kc,
                         float acc[NR][MR]) {
  for (int j = 0; j < NR; ++j) {
    const float *b = Bj[j];
    for (int i = 0; i < MR; ++i) {
      float a = acc[j][i];
      for (int64_t k = 0; k < kc; ++k) a = fmaf(P[k * MR + i], b[k], a);
      acc[j][i] = a;
    }
  }
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static void
micro_avx2(const float *P, const float *const *Bj, int64_t kc,
           float acc[NR][MR]) {
  __m256 c0 = _mm256_loadu_ps(acc[0]), c1 = _mm256_loadu_ps(acc[1]);
  __m256 c2 = _mm256_loadu_ps(acc[2]), c3 = _mm256_loadu_ps(acc[3]);
  __m256 c4 = _mm256_loadu_ps(acc[4]), c5 = _mm256_loadu_ps(acc[5]);
  __m256 c6 = _mm256_loadu_ps(acc[6]), c7 = _mm256_loadu_ps(acc[7]);
  const float *b0 = Bj[0], *b1 = Bj[1], *b2 = Bj[2], *b3 = Bj[3];
  const float *b4 = Bj[4], *b5 = Bj[5], *b6 = Bj[6], *b7 = Bj[7];
  for (int64_t k = 0; k < kc; ++k) {
    __m256 a = _mm256_loadu_ps(P + k * MR);
    c0 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b0 + k), c0);
    c1 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b1 + k), c1);
    c2 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b2 + k), c2);
    c3 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b3 + k), c3);
    c4 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b4 + k), c4);
    c5 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b5 + k), c5);
    c6 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b6 + k), c6);
    c7 = _mm256_fmadd_ps(a, _mm256_broadcast_ss(b7 + k), c7);
  }
  _mm256_storeu_ps(acc[0], c0); _mm256_storeu_ps(acc[1], c1);
  _mm256_storeu_ps(acc[2], c2); _mm256_storeu_ps(acc[3], c3);
  _mm256_storeu_ps(acc[4], c4); _mm256_storeu_ps(acc[5], c5);
  _mm256_storeu_ps(acc[6], c6); _mm256_storeu_ps(acc[7], c7);
}
#endif

static int use_avx2(void) {
#if defined(__x86_64__)
  if (g_force_scalar) return 0;
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
  return 0;
#endif
}

void orc_gemm_nt_chain(const float *A, int64_t M, const float *B, int64_t N,
                       int64_t K, float *C) {
  if (M <= 0 || N <= 0) return;
  const int avx = use_avx2();
  const int64_t mt = (M + MB - 1) / MB, nt = (N + NB - 1) / NB;
  const int64_t tiles = mt * nt;
  float *zero_row = (float *)calloc((size_t)(K > 0 ? K : 1), sizeof(float));
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(orc_get_threads())
#endif
  for (int64_t tile = 0; tile < tiles; ++tile) {
    const int64_t m0 = (tile / nt) * MB, n0 = (tile % nt) * NB;
    const int64_t mc = (M - m0 < MB) ? M - m0 : MB;
    const int64_t nc = (N - n0 < NB) ? N - n0 : NB;
    const int np = (int)((mc + MR - 1) / MR), nj = (int)((nc + NR - 1) / NR);
    float *panel = (float *)malloc(sizeof(float) * (size_t)KB * MR);
    float acc[MB / MR][NB / NR][NR][MR];
    memset(acc, 0, sizeof(acc));
    for (int64_t k0 = 0; k0 < K; k0 += KB) {
      const int64_t kc = (K - k0 < KB) ? K - k0 : KB;
      for (int p = 0; p < np; ++p) {
        /* pack 8 rows of A, k-slice [k0,k0+kc), rows past M are zero */
        for (int i = 0; i < MR; ++i) {
          const int64_t m = m0 + p * MR + i;
          for (int64_t k = 0; k < kc; ++k)
            panel[k * MR + i] = (m < M) ? A[m * K + k0 + k] : 0.0f;
        }
        for (int jb = 0; jb < nj; ++jb) {
          const float *bj[NR];
          for (int j = 0; j < NR; ++j) {
            const int64_t n = n0 + jb * NR + j;
            bj[j] = (n < N) ? B + n * K + k0 : zero_row;
          }
#if defined(__x86_64__)
          if (avx)
            micro_avx2(panel, bj, kc, acc[p][jb]);
          else
#endif
            micro_scalar(panel, bj, kc, acc[p][jb]);
        }
      }
    }
    for (int p = 0; p < np; ++p)
      for (int jb = 0; jb < nj; ++jb)
        for (int j = 0; j < NR; ++j)
          for (int i = 0; i < MR; ++i) {
            const int64_t m = m0 + p * MR + i, n = n0 + jb * NR + j;
            if (m < M && n < N) C[m * N + n] = acc[p][jb][j][i];
          }
    free(panel);
  }
  free(zero_row);
  (void)avx;
}

/* ------------------------------------------------------------------------ */
/* a1 gate                                                                   */
/* ------------------------------------------------------------------------ */

/* layer.cu:1440-1450: attn_matmul_tiled_kernel(logits, x, gate, M=T, N=E,
 * K=H); each output is threadResults += regM*regN over k ascending
 * (layer.cu:109-127), contracted by nvcc to an fmaf chain from 0.0f.  The
 * zero-padded float4 loads (layer.cu:44-46) add exact zeros only when K%16 != 0,
 * which leaves the chain unchanged: fmaf(0, b, acc) == acc. */
void orc_gate_logits(const float *x, const float *gate, int64_t T, int H, int E,
                     float *logits) {
  orc_gemm_nt_chain(x, T, gate, E, H, logits);
}

void orc_gate_logits_muladd(const float *x, const float *gate, int64_t T, int H,
                            int E, float *logits) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
  for (int64_t t = 0; t < T; ++t)
    for (int e = 0; e < E; ++e) {
      float acc = 0.0f;
      for (int k = 0; k < H; ++k) {
        float prod = x[t * H + k] * gate[(int64_t)e * H + k];
        acc = acc + prod;
      }
      logits[t * E + e] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* a2 / activations                                                          */
/* ------------------------------------------------------------------------ */

/* layer.cu:434: 1.0f / (1.0f + (float)exp(-(double)x)) -- exp in double, the
 * add and the divide in float with IEEE rounding. */
float orc_sigmoid(float x) {
  float e = (float)exp(-(double)x);
  return 1.0f / (1.0f + e);
}

/* layer.cu:728: x / (1.0f + expf(-x)). */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* ------------------------------------------------------------------------ */
/* a3 router                                                                 */
/* ------------------------------------------------------------------------ */

/* layer.cu:439-499, one token at a time. */
static void route_one(const float *lg, const float *bias, int E, int *idx_out,
                      float *w_out) {
  float max_scores[ORC_TOPK], max_probs[ORC_TOPK];
  int max_ids[ORC_TOPK];
  for (int i = 0; i < ORC_TOPK; ++i) { /* layer.cu:452-456 */
    max_scores[i] = -1e30f;
    max_probs[i] = 0.0f;
    max_ids[i] = -1;
  }
  for (int e = 0; e < E; ++e) { /* layer.cu:458-477 */
    const float prob = orc_sigmoid(lg[e]);
    const float score = prob + (bias ? bias[e] : 0.0f);
    if (score > max_scores[ORC_TOPK - 1]) {
      int pos = ORC_TOPK - 1;
      while (pos > 0 && score > max_scores[pos - 1]) {
        max_scores[pos] = max_scores[pos - 1];
        max_probs[pos] = max_probs[pos - 1];
        max_ids[pos] = max_ids[pos - 1];
        pos--;
      }
      max_scores[pos] = score;
      max_probs[pos] = prob;
      max_ids[pos] = e;
    }
  }
  float sum_prob = 0.0f; /* layer.cu:480-482, rank order */
  for (int i = 0; i < ORC_TOPK; ++i) sum_prob += max_probs[i];
  const float scale = (sum_prob > 1e-6f) ? (1.0f / sum_prob) : 1.0f; /* :484 */
  const float routed_scale = 1.0f; /* literal at layer.cu:1458 */
  for (int i = 0; i < ORC_TOPK; ++i) { /* layer.cu:487-491 */
    idx_out[i] = max_ids[i];
    w_out[i] = max_probs[i] * scale * routed_scale;
  }
}

void orc_route(const float *logits, const float *bias, int64_t T, int E,
               int *idx, float *w, int *counts) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
  for (int64_t t = 0; t < T; ++t)
    route_one(logits + t * E, bias, E, idx + t * ORC_TOPK, w + t * ORC_TOPK);
  if (counts) { /* layer.cu:493-497, after the memset at layer.cu:1434 */
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (int64_t t = 0; t < T; ++t)
      for (int k = 0; k < ORC_TOPK; ++k) {
        const int e = idx[t * ORC_TOPK + k];
        if (e >= 0 && e < E) counts[e]++;
      }
  }
}

/* ------------------------------------------------------------------------ */
/* a4 + a5 dispatch                                                          */
/* ------------------------------------------------------------------------ */

void orc_dispatch(const int *idx, int64_t T, int E, int *offsets, int *pos,
                  int *slot_token) {
  int *cursor = (int *)calloc((size_t)E, sizeof(int));
  for (int e = 0; e <= E; ++e) offsets[e] = 0;
  for (int64_t t = 0; t < T; ++t) /* counts (layer.cu:493-497) */
    for (int k = 0; k < ORC_TOPK; ++k) {
      const int e = idx[t * ORC_TOPK + k];
      if (e >= 0 && e < E) offsets[e + 1]++;
    }
  for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e]; /* :737-754 */
  for (int e = 0; e < E; ++e) cursor[e] = offsets[e];      /* write_pos :758 */
  for (int64_t t = 0; t < T; ++t)                          /* :518-541 */
    for (int k = 0; k < ORC_TOPK; ++k) {
      const int e = idx[t * ORC_TOPK + k];
      if (e >= 0 && e < E) {
        const int s = cursor[e]++;
        pos[t * ORC_TOPK + k] = s;
        slot_token[s] = (int)t;
      } else {
        pos[t * ORC_TOPK + k] = -1;
      }
    }
  free(cursor);
}

/* ------------------------------------------------------------------------ */
/* a6 / a7 experts                                                           */
/* ------------------------------------------------------------------------ */

void orc_expert_w1w3(const float *xrows, int64_t M, const float *w1,
                     const float *w3, int H, int I, float *inter) {
  if (M <= 0) return;
  float *s3 = (float *)malloc(sizeof(float) * (size_t)M * (size_t)I);
  orc_gemm_nt_chain(xrows, M, w1, I, H, inter); /* sum1, layer.cu:930-938 */
  orc_gemm_nt_chain(xrows, M, w3, I, H, s3);    /* sum3, layer.cu:940-948 */
  for (int64_t i = 0; i < M * (int64_t)I; ++i)  /* layer.cu:962-965 */
    inter[i] = orc_silu(inter[i]) * s3[i];
  free(s3);
}

void orc_expert_w2(const float *inter, int64_t M, const float *w2, int H, int I,
                   float *out) {
  orc_gemm_nt_chain(inter, M, w2, H, I, out); /* layer.cu:1088-1106, 1110-1120 */
}

/* ------------------------------------------------------------------------ */
/* a8 + a9 combine                                                           */
/* ------------------------------------------------------------------------ */

/* layer.cu:708-720: sum = 0; sum += val*weight for k ascending (contracted to
 * fmaf); then layer.cu:1866-1871 out = a + b with a = residual. */
static void combine_row(const float *const rows[ORC_TOPK],
                        const float wk[ORC_TOPK], const float *res, int H,
                        float *y) {
  for (int h = 0; h < H; ++h) {
    float sum = 0.0f;
    for (int k = 0; k < ORC_TOPK; ++k)
      if (rows[k]) sum = fmaf(rows[k][h], wk[k], sum);
    y[h] = res ? res[h] + sum : sum;
  }
}

void orc_combine(const float *sorted_out, const int *pos, const float *w,
                 const float *residual, int64_t T, int H, float *y) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
  for (int64_t t = 0; t < T; ++t) {
    const float *rows[ORC_TOPK];
    for (int k = 0; k < ORC_TOPK; ++k) {
      const int s = pos[t * ORC_TOPK + k];
      rows[k] = (s >= 0) ? sorted_out + (int64_t)s * H : NULL;
    }
    combine_row(rows, w + t * ORC_TOPK, residual ? residual + t * H : NULL, H,
                y + t * H);
  }
}

/* ------------------------------------------------------------------------ */
/* dense FFN (MLP::forward_gpu, layer.cu:1231-1269)                          */
/* ------------------------------------------------------------------------ */

float orc_silu_dexp(float x) { return x / (1.0f + (float)exp(-(double)x)); }

int orc_dense_mlp(const float *x, const float *w1, const float *w3, const float *w2,
                  const float *residual, int64_t T, int H, int I, float *y) {
  if (T <= 0) return 0;
  float *gate = (float *)malloc(sizeof(float) * (size_t)(T * I));
  float *up = (float *)malloc(sizeof(float) * (size_t)(T * I));
  if (!gate || !up) {
    free(gate);
    free(up);
    return -1;
  }
  orc_gemm_nt_chain(x, T, w1, I, H, gate); /* layer.cu:1250-1251 */
  orc_gemm_nt_chain(x, T, w3, I, H, up);   /* layer.cu:1254-1255 */
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
  for (int64_t i = 0; i < T * I; ++i) gate[i] = orc_silu_dexp(gate[i]) * up[i]; /* layer.cu:679-682 */
  orc_gemm_nt_chain(gate, T, w2, H, I, y);  /* layer.cu:1266-1268 */
  if (residual)
    for (int64_t i = 0; i < T * H; ++i) y[i] = residual[i] + y[i];
  free(gate);
  free(up);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* post-attention RMSNorm (layer.cu:144-193)                                 */
/* ------------------------------------------------------------------------ */

#define ORC_NORM_THREADS 256 /* RMSNorm::forward_gpu, layer.cu:1146 */
#define ORC_WARP 32

/* __shfl_down_sync(mask, v, off) over one 32-lane warp, all lanes at once:
 * lane l reads lane l+off, or its own value when l+off is outside the warp. */
static void shfl_down_add(float *v, int off) {
  float nv[ORC_WARP];
  for (int l = 0; l < ORC_WARP; ++l) nv[l] = v[l] + (l + off < ORC_WARP ? v[l + off] : v[l]);
  memcpy(v, nv, sizeof(nv));
}

static void rmsnorm_row(const float *src, const float *weight, int H, float *dst) {
  float part[ORC_NORM_THREADS];
  for (int t = 0; t < ORC_NORM_THREADS; ++t) { /* layer.cu:157-160 */
    float s = 0.0f;
    for (int i = t; i < H; i += ORC_NORM_THREADS) s = fmaf(src[i], src[i], s);
    part[t] = s;
  }
  float warp_sum[ORC_NORM_THREADS / ORC_WARP];
  for (int wi = 0; wi < ORC_NORM_THREADS / ORC_WARP; ++wi) { /* layer.cu:163-170 */
    float v[ORC_WARP];
    memcpy(v, part + wi * ORC_WARP, sizeof(v));
    for (int off = ORC_WARP / 2; off > 0; off /= 2) shfl_down_add(v, off);
    warp_sum[wi] = v[0];
  }
  float v[ORC_WARP]; /* layer.cu:173-182: warp 0, lanes >= 8 hold 0 */
  for (int l = 0; l < ORC_WARP; ++l) v[l] = l < ORC_NORM_THREADS / ORC_WARP ? warp_sum[l] : 0.0f;
  for (int off = (ORC_NORM_THREADS / ORC_WARP) / 2; off > 0; off /= 2) shfl_down_add(v, off);
  const float rms = 1.0f / sqrtf(v[0] / (float)H + 1e-5f); /* layer.cu:189 */
  for (int i = 0; i < H; ++i) dst[i] = (src[i] * rms) * weight[i]; /* layer.cu:191-193 */
}

void orc_rmsnorm(const float *h, const float *weight, int64_t T, int H, float *out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
  for (int64_t t = 0; t < T; ++t) rmsnorm_row(h + t * H, weight, H, out + t * H);
}

/* ------------------------------------------------------------------------ */
/* whole block                                                               */
/* ------------------------------------------------------------------------ */

#define ORC_MAX_EXPERTS 256

/* Adopts guide[] (another implementation's top-4 of one token, rank order)
 * in place of the oracle's own when it is a top-4 of the oracle's scores up
 * to eps: four distinct experts, each scoring at least the best excluded
 * expert minus eps, in non-increasing score order up to eps.  The weights
 * are then the reference's renormalisation (layer.cu:480-491) of the
 * oracle's own probabilities in the guide's order.  Returns 0 when the guide
 * equals the own choice, 1 when adopted, -1 when it is not a near-tie. */
static int adopt_guide(const float *lg, const float *bias, int E, const int *guide,
                       float eps, int *idx, float *w) {
  int same = 1;
  for (int k = 0; k < ORC_TOPK; ++k) same &= guide[k] == idx[k];
  if (same) return 0;
  float sc[ORC_MAX_EXPERTS], pr[ORC_MAX_EXPERTS];
  if (E > ORC_MAX_EXPERTS) return -1;
  for (int e = 0; e < E; ++e) {
    pr[e] = orc_sigmoid(lg[e]);
    sc[e] = pr[e] + (bias ? bias[e] : 0.0f);
  }
  int in[ORC_MAX_EXPERTS] = {0};
  for (int k = 0; k < ORC_TOPK; ++k) {
    const int e = guide[k];
    if (e < 0 || e >= E || in[e]) return -1;
    in[e] = 1;
    if (sc[e] != sc[e]) return -1; /* never a NaN score */
    if (k > 0 && sc[e] > sc[guide[k - 1]] + eps) return -1;
  }
  float lo = sc[guide[0]], hi = -INFINITY;
  for (int k = 1; k < ORC_TOPK; ++k) lo = fminf(lo, sc[guide[k]]);
  for (int e = 0; e < E; ++e)
    if (!in[e] && sc[e] == sc[e]) hi = fmaxf(hi, sc[e]);
  if (lo < hi - eps) return -1;
  float sum = 0.0f;
  for (int k = 0; k < ORC_TOPK; ++k) sum += pr[guide[k]];
  const float scale = (sum > 1e-6f) ? (1.0f / sum) : 1.0f;
  for (int k = 0; k < ORC_TOPK; ++k) {
    idx[k] = guide[k];
    w[k] = pr[guide[k]] * scale * 1.0f;
  }
  return 1;
}

static int moe_forward_impl(const float *x, const float *gate, const float *bias,
                            const float *w1, const float *w3, const float *w2,
                            const float *residual, int64_t T, int H, int I, int E,
                            const uint8_t *token_mask, float *y, float *logits_out,
                            int *idx_out, float *w_out, int *counts_out,
                            const int *guide, float eps, int64_t *n_adopted,
                            int64_t *n_hard);

int orc_moe_forward(const float *x, const float *gate, const float *bias,
                    const float *w1, const float *w3, const float *w2,
                    const float *residual, int64_t T, int H, int I, int E,
                    const uint8_t *token_mask, float *y, float *logits_out,
                    int *idx_out, float *w_out, int *counts_out) {
  return moe_forward_impl(x, gate, bias, w1, w3, w2, residual, T, H, I, E, token_mask, y,
                          logits_out, idx_out, w_out, counts_out, NULL, 0.0f, NULL, NULL);
}

int orc_moe_forward_guided(const float *x, const float *gate, const float *bias,
                           const float *w1, const float *w3, const float *w2,
                           const float *residual, int64_t T, int H, int I, int E,
                           const int *guide, float eps, float *y, int *idx_out,
                           int64_t *n_adopted, int64_t *n_hard) {
  if (!guide || !n_adopted || !n_hard) return -1;
  return moe_forward_impl(x, gate, bias, w1, w3, w2, residual, T, H, I, E, NULL, y, NULL,
                          idx_out, NULL, NULL, guide, eps, n_adopted, n_hard);
}

static int moe_forward_impl(const float *x, const float *gate, const float *bias,
                            const float *w1, const float *w3, const float *w2,
                            const float *residual, int64_t T, int H, int I, int E,
                            const uint8_t *token_mask, float *y, float *logits_out,
                            int *idx_out, float *w_out, int *counts_out,
                            const int *guide, float eps, int64_t *n_adopted,
                            int64_t *n_hard) {
  if (T < 0 || H <= 0 || I <= 0 || E < ORC_TOPK) return -1;
  const int64_t S = T * ORC_TOPK;
  int rc = -1;
  float *logits = (float *)malloc(sizeof(float) * (size_t)(T * E + 1));
  int *idx = (int *)malloc(sizeof(int) * (size_t)(S + 1));
  float *w = (float *)malloc(sizeof(float) * (size_t)(S + 1));
  int *counts = (int *)malloc(sizeof(int) * (size_t)E);
  int *offsets = (int *)malloc(sizeof(int) * (size_t)(E + 1));
  int *pos = (int *)malloc(sizeof(int) * (size_t)(S + 1));
  int *slot_token = (int *)malloc(sizeof(int) * (size_t)(S + 1));
  int64_t *compact = (int64_t *)malloc(sizeof(int64_t) * (size_t)(S + 1));
  float *xr = NULL, *inter = NULL, *outc = NULL;
  if (!logits || !idx || !w || !counts || !offsets || !pos || !slot_token ||
      !compact)
    goto done;

  orc_gate_logits(x, gate, T, H, E, logits);
  orc_route(logits, bias, T, E, idx, w, counts);
  if (guide) {
    int64_t na = 0, nh = 0;
    for (int64_t t = 0; t < T; ++t) {
      const int r = adopt_guide(logits + t * E, bias, E, guide + t * ORC_TOPK, eps,
                                idx + t * ORC_TOPK, w + t * ORC_TOPK);
      na += r == 1;
      nh += r < 0;
    }
    *n_adopted = na;
    *n_hard = nh;
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (int64_t t = 0; t < T * ORC_TOPK; ++t)
      if (idx[t] >= 0 && idx[t] < E) counts[idx[t]]++;
  }
  orc_dispatch(idx, T, E, offsets, pos, slot_token);

  /* slots whose token is selected get a compact row in outc */
  int64_t nsel = 0, maxrows = 0;
  for (int64_t s = 0; s < offsets[E]; ++s) {
    const int t = slot_token[s];
    compact[s] = (!token_mask || token_mask[t]) ? nsel++ : -1;
  }
  for (int e = 0; e < E; ++e) {
    int64_t m = 0;
    for (int64_t s = offsets[e]; s < offsets[e + 1]; ++s) m += compact[s] >= 0;
    if (m > maxrows) maxrows = m;
  }
  if (y && nsel > 0) {
    xr = (float *)malloc(sizeof(float) * (size_t)(maxrows * H));
    inter = (float *)malloc(sizeof(float) * (size_t)(maxrows * I));
    outc = (float *)malloc(sizeof(float) * (size_t)(nsel * H));
    if (!xr || !inter || !outc) goto done;
    for (int e = 0; e < E; ++e) {
      int64_t m = 0, first = -1;
      for (int64_t s = offsets[e]; s < offsets[e + 1]; ++s) {
        if (compact[s] < 0) continue;
        if (first < 0) first = compact[s];
        memcpy(xr + m * H, x + (int64_t)slot_token[s] * H, sizeof(float) * H);
        ++m;
      }
      if (m == 0) continue;
      /* compact rows of one expert are consecutive (slots ascend within e) */
      orc_expert_w1w3(xr, m, w1 + (int64_t)e * I * H, w3 + (int64_t)e * I * H,
                      H, I, inter);
      orc_expert_w2(inter, m, w2 + (int64_t)e * H * I, H, I, outc + first * H);
    }
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
    for (int64_t t = 0; t < T; ++t) {
      if (token_mask && !token_mask[t]) continue;
      const float *rows[ORC_TOPK];
      for (int k = 0; k < ORC_TOPK; ++k) {
        const int s = pos[t * ORC_TOPK + k];
        rows[k] = (s >= 0) ? outc + compact[s] * H : NULL;
      }
      combine_row(rows, w + t * ORC_TOPK, residual ? residual + t * H : NULL, H,
                  y + t * H);
    }
  } else if (y) {
    for (int64_t t = 0; t < T; ++t) {
      if (token_mask && !token_mask[t]) continue;
      const float *rows[ORC_TOPK] = {NULL, NULL, NULL, NULL};
      combine_row(rows, w + t * ORC_TOPK, residual ? residual + t * H : NULL, H,
                  y + t * H);
    }
  }
  if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)(T * E));
  if (idx_out) memcpy(idx_out, idx, sizeof(int) * (size_t)S);
  if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)S);
  if (counts_out) memcpy(counts_out, counts, sizeof(int) * (size_t)E);
  rc = 0;
done:
  free(logits); free(idx); free(w); free(counts); free(offsets); free(pos);
  free(slot_token); free(compact); free(xr); free(inter); free(outc);
  return rc;
}
