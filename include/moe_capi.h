/*
 * moe_capi.h -- C-ABI of the MI355X (gfx950) sparse-MoE block.
 *
 * The drop-in boundary for the MoE FFN path of a decoder layer: the
 * reference's SparseMoeBlock (risepower20/final include/layer.h:72-123,
 * src/layer.cu:1274-1503) re-implemented on hand-written HIP kernels.  Plain
 * pointers and sizes only; every call returns an int status (0 = MOE_OK) and
 * never exits the process (the reference's CHECK_CUDA calls exit(),
 * include/tensor.h:9-17).
 *
 * Semantics of one forward (SparseMoeBlock::forward_gpu, layer.cu:1428-1498):
 *   logits = x . gate^T                      (fp32, one FMA chain per output)
 *   p      = 1 / (1 + exp(-logit))          (exp in double)
 *   top-4 of p + bias, renormalised over the four p  (layer.cu:439-499)
 *   y[t]   = sum_k w[t,k] * W2_e (silu(W1_e x[t]) * (W3_e x[t]))   e = idx[t,k]
 *   y[t]  += residual[t]   when residual != NULL (add_kernel, layer.cu:1917)
 *
 * Threading: a context runs one forward at a time.  Calls on one context must
 * be ordered on one stream (the reference serialises a layer's forwards with a
 * per-stage event, model.cu:435,447); two streams sharing a context race on
 * its scratch.
 */
#ifndef MOE_CAPI_H
#define MOE_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moe_ctx moe_ctx;

/* hipStream_t without pulling in the HIP headers; 0 = the null stream. */
typedef void *moe_stream_t;

enum moe_status {
  MOE_OK = 0,
  MOE_ERR_INVALID_ARG = 1,   /* null pointer, bad size, misaligned buffer */
  MOE_ERR_UNSUPPORTED = 2,   /* dims the kernels are not built for */
  MOE_ERR_HIP = 3,           /* a HIP runtime call failed */
  MOE_ERR_OUT_OF_MEMORY = 4, /* device allocation failed */
  MOE_ERR_NOT_READY = 5,     /* forward before weights were set */
  MOE_ERR_TOO_MANY_TOKENS = 6, /* num_tokens > max_tokens of the context */
  MOE_ERR_DEVICE_TIMEOUT = 7, /* a kernel's bounded dependency wait expired */
  MOE_ERR_INTERNAL = 8       /* a kernel found an inconsistent dispatch plan */
};

/* Shapes.  Reference values (include/config.h:5,14-17): hidden 2048,
 * inter 1792, num_experts 32, top_k 4.  Supported: num_experts == 32,
 * top_k == 4, hidden % 256 == 0, inter % 256 == 0.  max_tokens sizes the
 * scratch (the reference hard-codes 4096, layer.cu:1399). */
typedef struct moe_dims {
  int hidden;
  int inter;
  int num_experts;
  int top_k;
  int max_tokens;
} moe_dims;

/* Replaces SparseMoeBlock::init_gpu's scratch allocation (layer.cu:1399-1425).
 * Allocates on the current HIP device. */
int moe_create(const moe_dims *dims, moe_ctx **out);

/* Replaces ~SparseMoeBlock (layer.cu:1302-1355).  Null is accepted. */
int moe_destroy(moe_ctx *ctx);

/* Replaces the weight upload of SparseMoeBlock::init_gpu (layer.cu:1358-1396)
 * and MLP::init_gpu (layer.cu:1216-1228).  gate [E][H], bias [E] (may be
 * NULL: no expert bias), w1[e]/w3[e] [I][H], w2[e] [H][I], fp32 row-major, the
 * layouts the reference loads by name (layer.cu:1277-1298).  Pointers are host
 * memory when src_on_device == 0, device memory otherwise.  The weights are
 * repacked once into the kernels' layout; the caller's buffers may be freed
 * afterwards.  Synchronises `stream` before returning. */
int moe_set_weights(moe_ctx *ctx, const float *gate, const float *bias,
                    const float *const *w1, const float *const *w3,
                    const float *const *w2, int src_on_device,
                    moe_stream_t stream);

/* Replaces SparseMoeBlock::forward_gpu (layer.cu:1428-1498) and, when
 * residual != NULL, the residual add_kernel after it (layer.cu:1917-1918).
 * x, y, residual: device [num_tokens][hidden] fp32, 16-byte aligned; y may
 * alias residual (in-place residual add) but not x.  Asynchronous on `stream`;
 * no host synchronisation inside. num_tokens == 0 is a no-op.  Same results
 * as moe_route + moe_experts; for batches of up to 8 tokens under the
 * weight-streaming plan the routing completes inside the experts launch
 * (moe_last_routing reads it after either). */
int moe_forward(moe_ctx *ctx, const float *x, float *y, const float *residual,
                int num_tokens, moe_stream_t stream);

/* moe_forward without allocating: no counterpart in the reference.  For
 * callers that cannot allocate device memory during a forward (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * kernels, plan and results as moe_route + moe_experts (bit for bit, and so
 * moe_forward's, which may route a decode batch of up to 8 tokens inside the
 * experts launch with the same arithmetic), but the routing,
 * intermediate and expert-output scratch is one file-scope device array per
 * GPU (8 MiB, set up by moe_create on that GPU) instead of the context's.
 * num_tokens <= 128 (and the rows must fit the array: 128 tokens at hidden
 * 2048 / inter 1792); larger returns MOE_ERR_TOO_MANY_TOKENS.  Calls no
 * hipMalloc/hipFree.  Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, or two contexts) race; calls ordered on
 * one stream do not.  Its device status (the array's own status word) is
 * read and cleared by the first moe_device_status of any context on that GPU
 * after a no-alloc call there.  moe_last_routing does not see its routing. */
int moe_forward_noalloc(moe_ctx *ctx, const float *x, float *y, const float *residual,
                        int num_tokens, moe_stream_t stream);

/* The two halves of moe_forward, for callers that time or inspect them:
 * moe_route = gate GEMM + sigmoid/top-4 + per-expert histogram and scan
 * (layer.cu:1438-1464); moe_experts = dispatch + grouped SwiGLU experts +
 * weighted combine (layer.cu:1466-1497).  moe_experts must follow moe_route on
 * the same stream with the same x and num_tokens; each moe_route serves one
 * moe_experts (a second call without a new route returns
 * MOE_ERR_INVALID_ARG). */
int moe_route(moe_ctx *ctx, const float *x, int num_tokens, moe_stream_t stream);
int moe_experts(moe_ctx *ctx, const float *x, float *y, const float *residual,
                int num_tokens, moe_stream_t stream);

/* Timing hook: moe_forward's own routing launch, which for decode batches
 * leaves the gate logits (and, for the MFMA plans up to 256 tokens, the exact
 * routing) to the experts launch that follows.  It must be followed by
 * moe_experts on the same stream with the same x and num_tokens and a y that
 * is not x; together they run exactly moe_forward's two kernels. */
int moe_route_forward(moe_ctx *ctx, const float *x, int num_tokens, moe_stream_t stream);

/* Routing from caller-supplied logits [num_tokens][E] (device): the sigmoid,
 * bias, top-4 and histogram of moe_router_topk_kernel (layer.cu:439-499)
 * without the gate GEMM.  Used by SparseMoeBlock::route_tokens (layer.h:91-93)
 * and by parity tests that craft ties.  Follow with moe_experts or read the
 * result with moe_last_routing. */
int moe_route_logits(moe_ctx *ctx, const float *logits, int num_tokens,
                     moe_stream_t stream);

/* Dense SwiGLU FFN of the first NUM_DENSE_LAYERS layers (config.h:16;
 * MLP::forward_gpu, layer.cu:1231-1269, INTERMEDIATE_SIZE = 7168):
 * y = W2 (silu(W1 x) * (W3 x)) [+ residual].  Replaces MLP::init_gpu
 * (layer.cu:1216-1228) and its missing scratch (the reference never allocates
 * temp_buf_gpu_, layer.cu:1237).  The context runs the MoE kernels with the
 * intermediate dimension cut into 4 chunks, every token sent to all four with
 * weight 1: hidden % 256 == 0 and inter % 1024 == 0 (inter / 4 == 1792 at
 * hidden 2048 gets the weight-streaming kernel for small batches).  Release
 * with moe_destroy.  moe_forward / moe_route / moe_set_weights reject a dense
 * context and moe_dense_* reject a MoE context. */
int moe_dense_create(int hidden, int inter, int max_tokens, moe_ctx **out);

/* A context that owns only its weights and runs on the scratch of `donor`
 * (routing, plan, intermediate and expert-output rows, normalised rows):
 * the decoder layers of one model run one after another on one stream, so
 * they need one scratch between them, not one each (the reference gives
 * every layer its own, layer.cu:1399-1425).  Replaces moe_create /
 * moe_dense_create for such layers: hidden and the per-expert intermediate
 * (inter, or inter / 4 for the dense FFN) must equal the donor's, max_tokens
 * must not exceed it, same device.  The donor must outlive the context, and
 * every context sharing a scratch must be used on one stream, one call after
 * another; moe_last_routing / moe_last_normed on any of them read the last
 * forward of any of them.  Released with moe_destroy. */
int moe_create_shared(const moe_dims *dims, moe_ctx *donor, moe_ctx **out);
int moe_dense_create_shared(int hidden, int inter, int max_tokens, moe_ctx *donor,
                            moe_ctx **out);
/* w1, w3 [inter][hidden], w2 [hidden][inter] (MLP's w1/w3/w2 tensors,
 * layer.cu:1199-1204); host memory when src_on_device == 0.  Synchronises
 * `stream`. */
int moe_dense_set_weights(moe_ctx *ctx, const float *w1, const float *w3, const float *w2,
                          int src_on_device, moe_stream_t stream);
/* x, y, residual (may be NULL): device [num_tokens][hidden]; y may alias
 * residual but not x.  Asynchronous on `stream`. */
int moe_dense_forward(moe_ctx *ctx, const float *x, float *y, const float *residual,
                      int num_tokens, moe_stream_t stream);

/* The post-attention RMSNorm weight [hidden] of the decoder layer that owns
 * this block (RMSNorm post_attention_layernorm_, layer.cu:1790-1793, weight
 * layers.{i}.ffn_norm.weight; RMSNorm::init_gpu uploads it,
 * layer.cu:1128-1142).  Host memory when src_on_device == 0.  Allocates the
 * normalised-row scratch ([max_tokens][hidden]) on first use.  Synchronises
 * `stream`. */
int moe_set_norm_weight(moe_ctx *ctx, const float *weight, int src_on_device,
                        moe_stream_t stream);

/* Steps 4-6 of DecoderLayer::forward_gpu (layer.cu:1903-1918) in one call:
 * out = h + MoE(rmsnorm(h)), with rmsnorm exactly rms_norm_kernel
 * (layer.cu:144-193, eps 1e-5) and the MoE block of moe_forward.  h, out:
 * device [num_tokens][hidden] fp32, 16-byte aligned; out may alias h (the
 * reference writes the layer output in place, layer.cu:1917).  Needs
 * moe_set_weights and moe_set_norm_weight.  For up to 256 tokens the router
 * normalises the rows it already stages (no extra launch); larger batches
 * run one normalisation kernel first.  Asynchronous on `stream`. */
int moe_forward_norm(moe_ctx *ctx, const float *h, float *out, int num_tokens,
                     moe_stream_t stream);

/* Copies the normalised rows of the last moe_forward_norm ([T][hidden]) to
 * host memory (parity tests: the reference's normed_hidden_gpu_,
 * layer.cu:1904-1905).  num_tokens is the row count xn holds and must equal
 * that call's T (else MOE_ERR_INVALID_ARG, nothing copied).  Synchronises
 * `stream`. */
int moe_last_normed(moe_ctx *ctx, float *xn, int num_tokens, moe_stream_t stream);

/* Copies the routing of the last moe_route/moe_forward to host memory:
 * idx [T][4] (rank order, -1 = none), w [T][4], counts [E], logits [T][E]
 * (any may be NULL).  num_tokens is the T the buffers are sized for and must
 * equal the routed T (else MOE_ERR_INVALID_ARG, nothing copied).
 * Synchronises `stream`.  The topk_indices_gpu_, topk_weights_gpu_ and
 * expert_counts_gpu_ of the reference (layer.h:99-107). */
int moe_last_routing(moe_ctx *ctx, int *idx, float *w, int *counts,
                     float *logits, int num_tokens, moe_stream_t stream);

/* Reads and clears the device status word: MOE_ERR_DEVICE_TIMEOUT if a
 * kernel's bounded dependency wait expired since the last call,
 * MOE_ERR_INTERNAL if a kernel met an out-of-range slot (and skipped it), else
 * MOE_OK.  Synchronises `stream`. */
int moe_device_status(moe_ctx *ctx, moe_stream_t stream);

/* Diagnostics: the slots per expert of the last expert-kernel plan (counts,
 * [E] host ints).  They equal the routing's counts, except after a deferred
 * decode routing (moe_forward of up to 8 tokens under the weight-streaming
 * plan), which gives a token a slot for every expert its score bounds leave
 * possible: a 5th or 6th one when two scores nearly tie at the 4th place.
 * Synchronises `stream`. */
int moe_last_plan_counts(moe_ctx *ctx, int *counts, moe_stream_t stream);

/* Which expert kernel moe_forward picks for num_tokens: 0 = weight-streaming
 * (small T), 32/64/128 = MFMA grouped GEMM with that many rows per tile. */
int moe_plan_tile_rows(const moe_ctx *ctx, int num_tokens);

/* Overrides the plan (tests): rows = -1 automatic, 0 streaming, 32/64/128.
 * Streaming covers batches of up to 1024 tokens; larger ones use 32. */
int moe_force_tile_rows(moe_ctx *ctx, int rows);

/* Test hook: scales the kernels' bounded-wait limit (1 = default, >1 shorter).
 * A value > 1 makes waits give up early and raise MOE_ERR_DEVICE_TIMEOUT;
 * every kernel still exits normally. */
int moe_set_wait_divisor(moe_ctx *ctx, int divisor);

/* Test hook: with on != 0, moe_forward's routing of a decode batch (<= 8
 * tokens, weight-streaming plan) leaves the gate-logit chains to the expert
 * kernel's waits that need them instead of to its first blocks: the path its
 * combine and fallback take when blocks start late because other kernels hold
 * the GPU.  Results are unchanged; only the timing differs. */
int moe_set_lazy_chains(moe_ctx *ctx, int on);

const char *moe_strerror(int status);

/* Library version string ("final_amd-moe <semver> gfx950"). */
const char *moe_version(void);

#ifdef __cplusplus
}
#endif
#endif
