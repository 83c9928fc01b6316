/*
 * lfm_oracle.h -- CPU restatement of the reference's decoder-model arithmetic
 * around the MoE block (embedding, rotary tables, q/k norm + rotation,
 * causal GQA attention, short conv).
 *
 * TEST INFRASTRUCTURE ONLY, like moe_oracle.h: tests/, the smoke check and
 * bench.py's cpu_baseline leg may load it; the product never does.  Every
 * function cites the reference line it restates (risepower20/final
 * src/layer.cu unless noted).  The projections and the LM head are
 * orc_gemm_nt_chain (moe_oracle.h) and the norms orc_rmsnorm.
 *
 * Layouts: fp32 row-major; qkv [T][ld] with q heads at columns h*64, k heads
 * at k_col + g*64, v heads at v_col + g*64 (head_dim 64); token t = b*seq + s.
 */
#ifndef LFM_ORACLE_H
#define LFM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* embedding_lookup_kernel, model.cu:18-32: h[t] = table[ids[t]]; ids outside
 * [0, V) give a zero row (the reference reads out of bounds there). */
void orc_embed(const int *ids, int64_t T, const float *table, int H, int V, float *h);

/* RotaryEmbedding::init_gpu, layer.cu:1167-1178: theta_j = powf(theta,
 * -2.0f*j/head_dim), angle = (float)i * theta_j, cosf/sinf of the float
 * angle in columns j and j + head_dim/2. */
void orc_rope_tables(float *cos_t, float *sin_t, int max_pos, int head_dim, float theta);

/* In place on qkv: the q heads' and k heads' 64 values of every token are
 * normalised by rms_norm_kernel (orc_rmsnorm on a 64-wide row, launched with
 * 256 threads as layer.cu:1146 does: layer.cu:1638-1642) and rotated by
 * rope_transpose_kernel (layer.cu:195-231) for position s = t % seq:
 * out[d] = q1*c1 - q2*s1 and out[d+32] = q2*c2 + q1*s2 (q1 = x[d],
 * q2 = x[d+32]), each contracted by nvcc as fmaf(first product, -/+ second
 * product) -- the one choice here no reference output pins. */
void orc_qk_norm_rope(float *qkv, int ld, int64_t T, int seq, int heads, int kv_heads, int k_col,
                      const float *q_weight, const float *k_weight, const float *cos_t,
                      const float *sin_t);

/* fused_attn_gqa_kernel, layer.cu:262-354, for any seq (the reference's
 * keeps 16 scores per query, layer.cu:312): for query i of head h (kv head
 * g = h / (heads/kv_heads)), lane tx of a 32-lane warp forms
 * fmaf(q[tx], k_j[tx], q[tx+32]*k_j[tx+32]) (nvcc's contraction of
 * layer.cu:314-315), the warp sums the 32 with shuffle-down at 16..1
 * (layer.cu:248-252), score = sum * (1/sqrtf(64)), keys j > i get -1e30f
 * (layer.cu:317-320); m = the first maximum (strict >, from -1e30f); e_j =
 * (float)exp((double)(score_j - m)), summed in double in j order; inv =
 * (float)(1.0 / sum); out[d] = fmaf chain over j ascending of
 * (e_j * inv) * v_j[d] from 0 (layer.cu:336-345).  Keys after i are left
 * out: each of them adds exactly 0 in the reference.  out [T][heads*64]. */
void orc_attention(const float *qkv, int ld, int batch, int seq, int heads, int kv_heads,
                   int k_col, int v_col, float *out);

/* ShortConv's mix, layer.cu:360-429: Bx = B * gate (conv_transpose_split_
 * kernel), conv = fmaf chain over taps k = 0..L-1 with position s-L+1+k >= 0
 * of Bx * w[h][k] from 0 (causal_conv1d_kernel, layer.cu:397-404),
 * y = C * conv (conv_gating_transpose_kernel).  bcg [T][3H] = B|C|gate,
 * w [H][L], y [T][H]. */
void orc_shortconv(const float *bcg, const float *w, int batch, int seq, int H, int L, float *y);

/* out[i] = a[i] + b[i] (add_kernel, layer.cu:1860-1880); out may alias a or b. */
void orc_add(const float *a, const float *b, int64_t n, float *out);

#ifdef __cplusplus
}
#endif
#endif
