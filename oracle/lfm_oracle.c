/*
 * lfm_oracle.c -- CPU restatement of the reference's decoder arithmetic
 * around the MoE block.  TEST INFRASTRUCTURE ONLY (see lfm_oracle.h).
 * Built with -ffp-contract=off: the only fused operations are the explicit
 * fmaf() calls restating nvcc's contractions.
 */
#include "lfm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "moe_oracle.h"

#ifdef _OPENMP
#include <omp.h>
#endif

#define HD 64   /* head_dim (config.h:28) */
#define WARP 32

void orc_embed(const int *ids, int64_t T, const float *table, int H, int V, float *h) {
  for (int64_t t = 0; t < T; ++t) {
    const int id = ids[t];
    if (id >= 0 && id < V)
      memcpy(h + t * H, table + (int64_t)id * H, sizeof(float) * (size_t)H);
    else
      memset(h + t * H, 0, sizeof(float) * (size_t)H);
  }
}

void orc_rope_tables(float *cos_t, float *sin_t, int max_pos, int head_dim, float theta) {
  const int half = head_dim / 2;
  for (int i = 0; i < max_pos; ++i) {
    for (int j = 0; j < half; ++j) {
      const float th = powf(theta, -2.0f * (float)j / (float)head_dim);
      const float angle = (float)i * th;
      cos_t[(int64_t)i * head_dim + j] = cosf(angle);
      cos_t[(int64_t)i * head_dim + j + half] = cosf(angle);
      sin_t[(int64_t)i * head_dim + j] = sinf(angle);
      sin_t[(int64_t)i * head_dim + j + half] = sinf(angle);
    }
  }
}

void orc_qk_norm_rope(float *qkv, int ld, int64_t T, int seq, int heads, int kv_heads, int k_col,
                      const float *q_weight, const float *k_weight, const float *cos_t,
                      const float *sin_t) {
  const int per_tok = heads + kv_heads;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
  for (int64_t r = 0; r < T * per_tok; ++r) {
    const int64_t t = r / per_tok;
    const int hd = (int)(r % per_tok);
    const int is_q = hd < heads;
    float *p = qkv + t * ld + (is_q ? hd * HD : k_col + (hd - heads) * HD);
    float y[HD];
    orc_rmsnorm(p, is_q ? q_weight : k_weight, 1, HD, y); /* layer.cu:1638-1642 */
    const int s = (int)(t % seq);
    const float *c = cos_t + (int64_t)s * HD, *sn = sin_t + (int64_t)s * HD;
    for (int d = 0; d < HD / 2; ++d) { /* layer.cu:212-228 */
      const float q1 = y[d], q2 = y[d + HD / 2];
      p[d] = fmaf(q1, c[d], -(q2 * sn[d]));
      p[d + HD / 2] = fmaf(q2, c[d + HD / 2], q1 * sn[d + HD / 2]);
    }
  }
}

/* warpReduceSum (layer.cu:248-252): lane l adds lane l+off, or keeps its own
 * value when l+off is past the warp; the total lands in lane 0. */
static float warp_sum(const float *v0) {
  float v[WARP], nv[WARP];
  memcpy(v, v0, sizeof(v));
  for (int off = WARP / 2; off > 0; off /= 2) {
    for (int l = 0; l < WARP; ++l) nv[l] = v[l] + (l + off < WARP ? v[l + off] : v[l]);
    memcpy(v, nv, sizeof(v));
  }
  return v[0];
}

void orc_attention(const float *qkv, int ld, int batch, int seq, int heads, int kv_heads,
                   int k_col, int v_col, float *out) {
  const int group = heads / kv_heads;
  const float scale = 1.0f / sqrtf((float)HD); /* layer.cu:1668 */
  const int64_t ldo = (int64_t)heads * HD;
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic, 16) num_threads(orc_get_threads())
#endif
  for (int64_t bh = 0; bh < (int64_t)batch * heads; ++bh) {
    for (int i = 0; i < seq; ++i) {
      const int b = (int)(bh / heads), h = (int)(bh % heads), g = h / group;
      const int64_t t0 = (int64_t)b * seq;
      const float *q = qkv + (t0 + i) * ld + (int64_t)h * HD;
      float *sc = (float *)malloc(sizeof(float) * (size_t)(i + 1));
      float mx = -1e30f;
      for (int j = 0; j <= i; ++j) {
        const float *k = qkv + (t0 + j) * ld + k_col + (int64_t)g * HD;
        float part[WARP];
        for (int tx = 0; tx < WARP; ++tx) part[tx] = fmaf(q[tx], k[tx], q[tx + WARP] * k[tx + WARP]);
        const float score = warp_sum(part) * scale;
        sc[j] = score;
        if (score > mx) mx = score;
      }
      double sum = 0.0;
      for (int j = 0; j <= i; ++j) {
        const float v = (float)exp((double)(sc[j] - mx));
        sc[j] = v;
        sum += (double)v;
      }
      const float inv = (float)(1.0 / sum);
      float acc[HD];
      for (int d = 0; d < HD; ++d) acc[d] = 0.0f;
      for (int j = 0; j <= i; ++j) {
        const float prob = sc[j] * inv;
        const float *v = qkv + (t0 + j) * ld + v_col + (int64_t)g * HD;
        for (int d = 0; d < HD; ++d) acc[d] = fmaf(prob, v[d], acc[d]);
      }
      memcpy(out + (t0 + i) * ldo + (int64_t)h * HD, acc, sizeof(acc));
      free(sc);
    }
  }
}

void orc_shortconv(const float *bcg, const float *w, int batch, int seq, int H, int L, float *y) {
  const int64_t T = (int64_t)batch * seq;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
#endif
  for (int64_t t = 0; t < T; ++t) {
    const int s = (int)(t % seq);
    for (int h = 0; h < H; ++h) {
      float sum = 0.0f;
      for (int k = 0; k < L; ++k) {
        const int pos = s - (L - 1) + k;
        if (pos < 0) continue;
        const float *row = bcg + (t - (L - 1) + k) * 3 * H;
        const float bx = row[h] * row[2 * H + h];
        sum = fmaf(bx, w[(int64_t)h * L + k], sum);
      }
      y[t * H + h] = bcg[t * 3 * H + H + h] * sum;
    }
  }
}

void orc_add(const float *a, const float *b, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
