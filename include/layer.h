// MoE FFN layer interface.  Drop-in for the reference's MLP / SparseMoeBlock
// (include/layer.h:48-123): same class names, constructors by tensor name,
// init_gpu / forward_gpu signatures with hipStream_t for cudaStream_t.  The
// GPU path is the HIP kernels behind include/moe_capi.h; errors throw
// std::runtime_error (the reference exits inside CHECK_CUDA).
#pragma once

#include <hip/hip_runtime_api.h>

#include <memory>
#include <string>
#include <vector>

#include "config.h"
#include "moe_capi.h"
#include "tensor.h"

// Expert weights (one SwiGLU FFN).  In the MoE block it is a weight holder:
// the block repacks all experts into one device layout.  Reference
// include/layer.h:48-69.
class MLP {
public:
  MLP(const std::string &w1_file, const std::string &w2_file,
      const std::string &w3_file);
  MLP(Tensor w1, Tensor w2, Tensor w3);  // in-memory weights
  ~MLP();
  MLP(MLP &&other) noexcept;
  MLP &operator=(MLP &&other) noexcept;
  MLP(const MLP &) = delete;
  MLP &operator=(const MLP &) = delete;

  // Dense FFN of layers 0-1 (layer.cu:1231-1269): y = W2 (silu(W1 x) * (W3 x))
  // on the MoE kernels (moe_dense_*, include/moe_capi.h).  forward: host
  // tensors x [T][H] -> y [T][H] (synchronous); forward_gpu: device pointers,
  // asynchronous on stream.  Both need init_gpu.
  void forward(const Tensor &x, Tensor &y);
  void forward_gpu(float *x, float *y, int batch, int seq_len, int hidden_size,
                   hipStream_t stream = 0);

  // Uploads the weights for forward_gpu (layer.cu:1216-1228): a dense context
  // with its own scratch for max_tokens() tokens.  The MoE block does not call
  // it: it uploads its experts itself.  w1_gpu_/w2_gpu_/w3_gpu_ stay null (the
  // weights live repacked inside the context).
  void init_gpu();
  void set_max_tokens(int n);  // before init_gpu (default 4096, layer.cu:1399)
  int max_tokens() const { return max_tokens_; }

  const Tensor &w1() const { return w1_; }
  const Tensor &w2() const { return w2_; }
  const Tensor &w3() const { return w3_; }

  float *w1_gpu_ = nullptr;
  float *w3_gpu_ = nullptr;
  float *w2_gpu_ = nullptr;
  float *temp_buf_gpu_ = nullptr;

private:
  Tensor w1_;  // [I][H]
  Tensor w3_;  // [I][H]
  Tensor w2_;  // [H][I]
  moe_ctx *dense_ctx_ = nullptr;
  int max_tokens_ = 4096;
  void release_gpu();
};

struct SparseMoeBlockTestAccess;

// Sparse MoE block: sigmoid+bias top-4 router over 32 SwiGLU experts.
// Reference include/layer.h:72-123, src/layer.cu:1274-1503.
class SparseMoeBlock {
public:
  // Loads layers.{i}.feed_forward.{gate.weight, experts.{e}.w{1,2,3}.weight,
  // expert_bias} through g_model_loader (layer.cu:1274-1300).
  explicit SparseMoeBlock(int layer_idx);
  // In-memory weights: gate [E][H], experts, expert_bias [E] (empty = none).
  SparseMoeBlock(int layer_idx, Tensor gate, std::vector<MLP> experts,
                 Tensor expert_bias);
  ~SparseMoeBlock();
  SparseMoeBlock(const SparseMoeBlock &) = delete;
  SparseMoeBlock &operator=(const SparseMoeBlock &) = delete;

  // Host tensors in and out: x [T][H] -> y [T][H], router_logits [T][E].
  // Runs the HIP path (device staging, synchronous); needs init_gpu().
  void forward(const Tensor &x, Tensor &y, Tensor &router_logits);

  // Allocates scratch for max_tokens() tokens and uploads the weights to the
  // current HIP device (layer.cu:1357-1426).
  void init_gpu();

  // y = MoE(x) for batch*seq_len tokens; device pointers, asynchronous on
  // stream (layer.cu:1428-1498).
  void forward_gpu(float *x, float *y, int batch, int seq_len, int hidden_size,
                   hipStream_t stream = 0);
  // y = residual + MoE(x): the block plus the decoder layer's residual add
  // (layer.cu:1908-1918) in one pass; y may alias residual.
  void forward_gpu(float *x, float *y, const float *residual, int batch,
                   int seq_len, int hidden_size, hipStream_t stream);

  // The decoder layer's post-attention RMSNorm weight [H] (RMSNorm,
  // layer.h:10-24, loaded as layers.{i}.post_attention_layernorm.weight at
  // layer.cu:1793).  After init_gpu.
  void set_post_attention_norm(const Tensor &weight);
  // Steps 4-6 of DecoderLayer::forward_gpu (layer.cu:1903-1918) in one call:
  // out = h + MoE(rmsnorm(h)), rmsnorm as rms_norm_kernel (layer.cu:144-193).
  // out may alias h (the reference updates the layer output in place).
  void forward_gpu_norm(float *h, float *out, int batch, int seq_len, int hidden_size,
                        hipStream_t stream = 0);

  int layer_idx() const { return layer_idx_; }
  int max_tokens() const { return max_tokens_; }
  void set_max_tokens(int n);  // before init_gpu
  moe_ctx *context() const { return ctx_; }

private:
  friend struct SparseMoeBlockTestAccess;

  Tensor gate_;  // router [E][H]
  std::vector<MLP> experts_;
  Tensor expert_bias_;  // [E] or empty

  // top-k experts and weights of each row of router_logits [T][E], computed on
  // the GPU by the block's router (sigmoid, +bias, top-4, renormalise).
  void route_tokens(const Tensor &router_logits, std::vector<int> &top_k_indices,
                    std::vector<float> &top_k_weights);

  moe_ctx *ctx_ = nullptr;
  int layer_idx_;
  int max_tokens_ = MOE_DEFAULT_MAX_TOKENS;
  void check_shapes() const;
};
