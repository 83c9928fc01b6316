/*
 * moe_oracle.h -- CPU restatement of the reference's sparse-MoE block arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * The product (final_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (risepower20/final,
 * src/layer.cu unless noted).  The reference's own CPU path is an empty stub
 * (layer.cu:1499-1503) and its tests/moe exists only as closed objects, so no
 * reference golden vector pins this file; the pinning checks are the closed
 * forms, brute-force and special-case tests in tests/test_oracle_*.py.
 *
 * Layouts (all fp32 row-major, as the reference stores them):
 *   x       [T][H]            gate    [E][H]   (layer.cu:1277-1278)
 *   bias    [E]               (layer.cu:1295-1299)
 *   w1, w3  [E][I][H]         w2      [E][H][I] (layer.cu:1282-1292, per-expert
 *                                      Linear weights, out x in)
 *   idx     [T][K] int32 (rank order), w [T][K] fp32, counts [E] int32
 *
 * K (experts per token) is fixed at 4, as in the reference router, which keeps
 * four running maxima regardless of k_experts (layer.cu:448-456).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_TOPK 4

/* Force the portable scalar fmaf() kernels (1) or allow AVX2/FMA (0, default).
 * Both produce bit-identical results; the switch exists so a test can prove it. */
void orc_force_scalar(int on);
/* Number of OpenMP threads used by the heavy loops (<=0: library default). */
void orc_set_threads(int n);
int orc_get_threads(void);

/* C[m][n] = sum_k A[m][k]*B[n][k] as one fmaf chain per output, k ascending,
 * starting from 0.0f.  This is the accumulation of every GEMM on the path:
 * attn_matmul_tiled_kernel layer.cu:109-127 (nvcc contracts "+= a*b" to FMA),
 * moe_persistent_fused_w1w3_kernel layer.cu:913-952 and
 * moe_persistent_w2_kernel layer.cu:1084-1106. */
void orc_gemm_nt_chain(const float *A, int64_t M, const float *B, int64_t N,
                       int64_t K, float *C);

/* a1: router logits, layer.cu:1438-1450 launching layer.cu:9-141. */
void orc_gate_logits(const float *x, const float *gate, int64_t T, int H, int E,
                     float *logits);
/* Sensitivity variant: acc = acc + x*g with two roundings (no contraction), the
 * arithmetic a host compiler without FMA would produce. Not on the path. */
void orc_gate_logits_muladd(const float *x, const float *gate, int64_t T, int H,
                            int E, float *logits);

/* a2: d_sigmoid, layer.cu:434. */
float orc_sigmoid(float x);
/* d_silu_opt, layer.cu:728. */
float orc_silu(float x);

/* a3: moe_router_topk_kernel, layer.cu:439-499, with routed_scale = 1.0f and
 * use_bias = true as launched at layer.cu:1453-1458 (bias may be NULL = no bias).
 * counts[E] is zeroed first (layer.cu:1434-1435). */
void orc_route(const float *logits, const float *bias, int64_t T, int E,
               int *idx, float *w, int *counts);

/* a4+a5: moe_scan_kernel layer.cu:730-768 and moe_scatter_kernel
 * layer.cu:501-542.  offsets[E+1] exclusive scan of counts; pos[T][K] = slot
 * of (t,k); slot_token[sum counts] = t.  The reference takes slots with
 * atomicAdd, so its order inside an expert is unspecified; this restatement
 * fixes it stable by token (ascending t), which is the order the HIP path
 * produces.  Entries with idx < 0 get pos = -1. */
void orc_dispatch(const int *idx, int64_t T, int E, int *offsets, int *pos,
                  int *slot_token);

/* a6: one expert over M gathered rows, moe_persistent_fused_w1w3_kernel
 * layer.cu:773-972: inter[m][n] = silu(x.w1[n]) * (x.w3[n]).
 * a7: moe_persistent_w2_kernel layer.cu:974-1126: out[m][h] = inter[m].w2[h]. */
void orc_expert_w1w3(const float *xrows, int64_t M, const float *w1,
                     const float *w3, int H, int I, float *inter);
void orc_expert_w2(const float *inter, int64_t M, const float *w2, int H, int I,
                   float *out);

/* a8+a9: moe_gather_deterministic_kernel layer.cu:695-721 (fma chain over k
 * from 0.0f) then the residual add_kernel layer.cu:1860-1880 as used at
 * layer.cu:1917 (y = residual + y) when residual != NULL. */
void orc_combine(const float *sorted_out, const int *pos, const float *w,
                 const float *residual, int64_t T, int H, float *y);

/* d_silu, layer.cu:436: x / (1.0f + (float)exp(-(double)x)), the SwiGLU of
 * the dense FFN (moe_swiglu_kernel layer.cu:670-691; the experts use
 * d_silu_opt, orc_silu). */
float orc_silu_dexp(float x);

/* Dense SwiGLU FFN, MLP::forward_gpu layer.cu:1231-1269 (I = 7168 in the
 * reference): gate = x W1^T and up = x W3^T (attn_matmul_tiled_kernel: one
 * fmaf chain per output over k ascending, layer.cu:109-127), inter =
 * d_silu(gate) * up (moe_swiglu_kernel layer.cu:670-691), y = inter W2^T
 * (the same chains over I), then y = residual + y (add_kernel layer.cu:1860-1880
 * as at layer.cu:1917) when residual != NULL.  x [T][H], w1/w3 [I][H],
 * w2 [H][I], y [T][H].  Returns 0, or -1 on allocation failure. */
int orc_dense_mlp(const float *x, const float *w1, const float *w3, const float *w2,
                  const float *residual, int64_t T, int H, int I, float *y);

/* Post-attention RMSNorm, rms_norm_kernel layer.cu:144-193 as launched by
 * RMSNorm::forward_gpu layer.cu:1144-1148 (one block of 256 threads per row,
 * warpSize 32).  Restated in the kernel's exact order: thread t (0..255)
 * accumulates h[i]*h[i] for i = t, t+256, ... from 0.0f with fmaf (nvcc's
 * default --fmad=true contracts "sum_sq += src[i] * src[i]"); each 32-thread
 * warp folds its sums with __shfl_down_sync at offsets 16, 8, 4, 2, 1 (lane l
 * adds lane l+off, or itself when l+off >= 32); warp 0 then folds the 8 warp
 * sums (lanes 8..31 hold 0) at offsets 4, 2, 1; rms = 1.0f / sqrtf(sum / H +
 * 1e-5f) (IEEE division and square root: no fast-math in the reference
 * build); out[i] = (h[i] * rms) * weight[i].  h, out: [T][H]; out may alias
 * h.  The fmaf choice is the one point not pinned by the reference (its
 * rounding differs from mul+add only in the partial sums' last bits). */
void orc_rmsnorm(const float *h, const float *weight, int64_t T, int H, float *out);

/* The whole block, SparseMoeBlock::forward_gpu layer.cu:1428-1498 (+1917).
 * token_mask (may be NULL = all) selects the tokens whose y row is computed;
 * routing (idx, w, counts, logits) always covers all T tokens, and rows of y
 * for unselected tokens are left untouched.  Any of logits/idx/w/counts may be
 * NULL.  Returns 0 on success, -1 on allocation failure or bad arguments. */
int orc_moe_forward(const float *x, const float *gate, const float *bias,
                    const float *w1, const float *w3, const float *w2,
                    const float *residual, int64_t T, int H, int I, int E,
                    const uint8_t *token_mask, float *y, float *logits, int *idx,
                    float *w, int *counts);

/* orc_moe_forward for all T tokens with the routing of another
 * implementation as a guide: where guide [T][4] (rank order) differs from the
 * oracle's own top-4 of a token but is a top-4 of the oracle's scores up to
 * eps (four distinct experts, none scoring more than eps below an excluded
 * expert, in non-increasing order up to eps), the oracle adopts it, with the
 * weights renormalised from its own probabilities in that order
 * (layer.cu:480-491); otherwise it keeps its own.  n_adopted counts adopted
 * tokens, n_hard the tokens whose guide is not a near-tie.  Used where the
 * oracle runs on inputs that differ from the other implementation's by
 * rounding only (a decoder's later layers), so that a near-tie decided the
 * other way is followed instead of diverging.  idx_out (may be NULL) gets the
 * routing used.  Returns 0, or -1 on bad arguments. */
int orc_moe_forward_guided(const float *x, const float *gate, const float *bias,
                           const float *w1, const float *w3, const float *w2,
                           const float *residual, int64_t T, int H, int I, int E,
                           const int *guide, float eps, float *y, int *idx_out,
                           int64_t *n_adopted, int64_t *n_hard);

#ifdef __cplusplus
}
#endif
#endif
