/*
 * lfm_capi.h -- C-ABI of the decoder model around the MoE block (gfx950).
 *
 * The kernels of an LFM2-8B-A1B-style decoder layer other than the MoE FFN
 * (risepower20/final src/layer.cu:144-429, 1508-1922; src/model.cu:18-116,
 * 469-559), as plain-pointer entry points the C++ layer classes
 * (include/layer.h, include/model.h) call, plus a handle on the whole
 * one-GPU model for FFI callers.  Every call returns an int status of enum
 * moe_status (include/moe_capi.h; moe_strerror names it) and never exits the
 * process.  Device pointers, fp32 row-major, 16-byte aligned; every kernel
 * call is asynchronous on `stream` with no host synchronisation.
 *
 * What is kept from the reference and what is not: the arithmetic of its
 * kernels where it is defined for the shapes (RMSNorm reduction order, rotary
 * tables and rotation, the conv's FMA chain, the gather); the projections run
 * on MFMA tiles (fp32 accumulation in another order than the reference's FMA
 * chains: results agree within fp32 rounding, not bit for bit); attention is
 * an online-softmax form of the reference's (which holds at most 16
 * positions, layer.cu:312); the 24-stage 4-GPU pipeline, P2P copies, dual
 * streams and the fp16 cuBLAS LM head are not built (one GPU, one stream).
 */
#ifndef LFM_CAPI_H
#define LFM_CAPI_H

#include <stddef.h>
#include <stdint.h>

#include "moe_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernels ------------------------------------------------------------ */

/* C[M][N] = A[M][K] . B[N][K]^T, plus R[M][N] when R != NULL (R may alias C).
 * Replaces attn_matmul_tiled_kernel (layer.cu:9-141: the q/k/v/o, in_proj
 * and out_proj projections, "A @ B^T" with B in PyTorch Linear [out][in]
 * layout) and lm_head_gemm_kernel (model.cu:42-116); R fuses the decoder's
 * residual add_kernel (layer.cu:1860-1880 as launched at 1912-1913).
 * N % 128 == 0, K % 32 == 0, M*K and M*N below 2^30 elements. */
int lfm_gemm_nt(const float *A, const float *B, float *C, const float *R, int M, int N, int K,
                moe_stream_t stream);

/* h[t][:] = table[ids[t]][:] for t < num_tokens: embedding_lookup_kernel
 * (model.cu:18-32).  table [vocab][hidden], hidden % 4 == 0.  An id outside
 * [0, vocab) gives a zero row and sets *bad_flag (device int, may be NULL) to
 * 1; the reference reads out of bounds there. */
int lfm_embed(const int *ids, const float *table, float *h, int num_tokens, int hidden,
              int vocab, int *bad_flag, moe_stream_t stream);

/* y = RMSNorm(x) * weight for `rows` rows of `dim`: rms_norm_kernel
 * (layer.cu:144-193) as RMSNorm::forward_gpu launches it (layer.cu:1144-1148),
 * bit for bit; row r of x starts at x + r*x_stride, of y at y + r*y_stride
 * (floats; strides let the model normalise only the last token of each
 * sequence, model.cu:486-501).  y may alias x. */
int lfm_rmsnorm(const float *x, long long x_stride, const float *weight, float *y,
                long long y_stride, int rows, int dim, moe_stream_t stream);

/* In place on qkv [batch*seq][ld]: the q heads (columns [0, heads*64)) and
 * the k heads (columns [k_col, k_col + kv_heads*64)) of every token are
 * RMS-normalised over their 64 values with q_weight / k_weight [64] (the
 * q_layernorm / k_layernorm of Attention::forward_gpu, layer.cu:1638-1642)
 * and rotated for position s = t % seq with cos/sin [>= seq][64]
 * (rope_transpose_kernel, layer.cu:195-231, without its transpose).
 * head_dim 64, heads + kv_heads <= 64; qkv, the weights and tables 16-byte
 * aligned, ld and k_col multiples of 4. */
int lfm_qk_norm_rope(float *qkv, int ld, const float *q_weight, const float *k_weight,
                     const float *cos_table, const float *sin_table, int batch, int seq,
                     int heads, int kv_heads, int k_col, moe_stream_t stream);

/* out[t][h*64 + d] = sum_j softmax_j(q_h(t) . k_g(j) / 8) v_g(j)[d] over the
 * keys j <= t of t's own sequence, g = h / (heads / kv_heads): the causal GQA
 * attention of fused_attn_gqa_kernel (layer.cu:262-354), for any seq.  q, k,
 * v are read from qkv [batch*seq][ld] at columns h*64, k_col + g*64 and
 * v_col + g*64.  head_dim 64, heads == 4 * kv_heads.  out [batch*seq][heads*64]. */
int lfm_attention(const float *qkv, int ld, float *out, int batch, int seq, int heads,
                  int kv_heads, int k_col, int v_col, moe_stream_t stream);

/* ShortConv's mix (conv_transpose_split_kernel, causal_conv1d_kernel and
 * conv_gating_transpose_kernel, layer.cu:360-429, token-major, bit for bit):
 * with B, C, g the column blocks [0,H), [H,2H), [2H,3H) of bcg
 * [batch*seq][3*hidden], y[t][h] = C[t][h] * sum_{k: s-L+1+k >= 0}
 * (B*g)[t-L+1+k][h] * conv_weight[h][k], s = t % seq, L = kernel.
 * y [batch*seq][hidden], hidden % 4 == 0, kernel <= 4 (the reference's is 3,
 * config.h:29). */
int lfm_shortconv(const float *bcg, const float *conv_weight, float *y, int batch, int seq,
                  int hidden, int kernel, moe_stream_t stream);

/* Rotary tables [max_pos][head_dim] in host memory, computed as
 * RotaryEmbedding::init_gpu does (layer.cu:1167-1178): theta_j =
 * powf(theta, -2.0f*j/head_dim), angle = (float)i * theta_j, cos/sin of the
 * float angle (cosf/sinf) in columns j and j + head_dim/2. */
int lfm_rope_tables(float *cos_out, float *sin_out, int max_pos, int head_dim, float theta);

/* ---- synthetic weights (no counterpart in the reference) --------------- */

/* dst[i] = std * N(0,1) sample (first + i) of (seed, stream): the generator
 * of include/moe_synth.h evaluated on the device (dst is device memory). */
int lfm_synth_normal(float *dst, size_t n, uint64_t seed, uint64_t stream_id, float std_dev,
                     uint64_t first, moe_stream_t stream);
/* dst[i] = value for i < n (device memory). */
int lfm_fill(float *dst, size_t n, float value, moe_stream_t stream);
/* Stream id of a tensor name: FNV-1a 64 of its bytes. */
uint64_t lfm_synth_stream_of(const char *name);
/* 1 if a synthetic model fills this tensor with ones (RMSNorm weights: names
 * ending in "norm.weight"), else 0 (N(0, std)). */
int lfm_synth_is_norm(const char *name);
/* The synthetic tensor `name` of n elements as a synthetic model holds it
 * (ones, or N(0, std) from (seed, lfm_synth_stream_of(name))), copied to host
 * memory.  Drawn on the current device; synchronous. */
int lfm_synth_tensor(uint64_t seed, const char *name, float std_dev, float *host_out, size_t n);

/* ---- the model (wraps LFM2Model, include/model.h) ---------------------- */

typedef struct lfm_model lfm_model;

/* Synthetic model: every weight drawn on the device by name (matrices and
 * expert bias N(0, weight_std), RMSNorm weights 1), embedding tied to the LM
 * head.  layer_types[i]: 0 attention, 1 short conv (NULL = the reference's
 * LAYER_TYPES, config.h:31); layers below num_dense_layers get the dense
 * SwiGLU FFN, the rest the MoE block.  Scratch for max_batch*max_seq
 * tokens, shared by all layers. */
typedef struct lfm_model_config {
  int num_layers;
  const int *layer_types;
  int num_dense_layers;
  int max_batch;
  int max_seq;
  uint64_t seed;
  float weight_std;
} lfm_model_config;

int lfm_model_create_synthetic(const lfm_model_config *cfg, lfm_model **out);
/* The reference's LFM2Model(model_file) (model.cu:124-137): tensors by name
 * from a model.bin; scratch for max_batch*max_seq tokens. */
int lfm_model_create_from_file(const char *path, int max_batch, int max_seq, lfm_model **out);
int lfm_model_destroy(lfm_model *m);

/* Last-token logits [batch][vocab] of token ids [batch][seq] (device int32):
 * embedding, every decoder layer, final RMSNorm, LM head -- the work of
 * LFM2Model::worker_stage over all stages (model.cu:403-559) on one GPU and
 * one stream. */
int lfm_model_forward(lfm_model *m, const int *ids, int batch, int seq, float *logits,
                      moe_stream_t stream);
/* The same in pieces: embedding into h [batch*seq][hidden]; decoder layer
 * `layer` in place on h (DecoderLayer::forward_gpu, layer.cu:1882-1919);
 * final norm of each sequence's last token + LM head. */
int lfm_model_embed(lfm_model *m, const int *ids, int batch, int seq, float *h,
                    moe_stream_t stream);
int lfm_model_layer_forward(lfm_model *m, int layer, float *h, int batch, int seq,
                            moe_stream_t stream);
int lfm_model_head(lfm_model *m, const float *h, int batch, int seq, float *logits,
                   moe_stream_t stream);
/* The MoE context of a layer (NULL for a dense layer): moe_last_routing on it
 * reads that layer's routing until the next MoE layer runs (all layers share
 * one scratch). */
int lfm_model_moe(lfm_model *m, int layer, moe_ctx **out);
/* Shape queries. */
int lfm_model_info(const lfm_model *m, int *num_layers, int *hidden, int *vocab, int *max_tokens);
/* MOE_OK, MOE_ERR_INVALID_ARG if an out-of-range token id was embedded since
 * the last call, or a MoE layer's device status.  Synchronises `stream`. */
int lfm_model_status(lfm_model *m, moe_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
