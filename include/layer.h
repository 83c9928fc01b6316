// Decoder-layer interface of the LFM2-8B-A1B-style model: drop-in for the
// reference's RMSNorm, RotaryEmbedding, MLP, SparseMoeBlock, Attention,
// ShortConv and DecoderLayer (include/layer.h:9-233): same class names,
// constructors by tensor name through g_model_loader, init_gpu / forward_gpu
// signatures with hipStream_t for cudaStream_t.  The GPU path is the HIP
// kernels behind include/moe_capi.h and include/lfm_capi.h; errors throw
// std::runtime_error (the reference exits inside CHECK_CUDA).
//
// Added to the reference's interface (none of it changes the original
// methods' meaning): in-memory and synthetic-weight constructors (the
// synthetic model has no model.bin), forward_gpu overloads that fold the
// decoder's residual add into the producing kernel, and a LayerWorkspace so
// that the layers of one model share their scratch.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "config.h"
#include "lfm_capi.h"
#include "moe_capi.h"
#include "tensor.h"

// Synthetic weights: every tensor is drawn on the device by name from
// (seed, lfm_synth_stream_of(name)) -- matrices and expert bias N(0, std),
// RMSNorm weights 1 (include/lfm_capi.h).  No counterpart in the reference.
struct SyntheticWeights {
  uint64_t seed = 0;
  float std_dev = 0.02f;
};

// One weight tensor of a layer: read by name through the model loader into a
// host Tensor (the reference's path, uploaded by upload()), given in memory,
// or drawn on the device by upload() for a synthetic model (no host copy).
class DeviceWeight {
public:
  DeviceWeight() = default;
  explicit DeviceWeight(const std::string &name);  // Tensor::load_from_file(name)
  DeviceWeight(const std::string &name, Tensor host);
  DeviceWeight(const std::string &name, std::vector<size_t> shape, const SyntheticWeights &s);
  ~DeviceWeight();
  DeviceWeight(DeviceWeight &&o) noexcept;
  DeviceWeight &operator=(DeviceWeight &&o) noexcept;
  DeviceWeight(const DeviceWeight &) = delete;
  DeviceWeight &operator=(const DeviceWeight &) = delete;

  // Allocates the device copy on the current device and fills it (synchronous).
  void upload();
  void release();
  float *gpu() const { return gpu_; }
  const std::string &name() const { return name_; }
  const std::vector<size_t> &shape() const { return shape_; }
  size_t size() const;
  bool synthetic() const { return synth_; }
  const Tensor &host() const { return host_; }

private:
  std::string name_;
  std::vector<size_t> shape_;
  Tensor host_;
  bool synth_ = false;
  SyntheticWeights syn_{};
  float *gpu_ = nullptr;
};

// Device buffers of a decoder layer's forward for up to max_tokens tokens.
// One workspace serves every layer of a model (the layers run one after
// another on one stream); a layer without one allocates its own in init_gpu,
// as the reference's DecoderLayer does (layer.cu:1834-1849).
struct LayerWorkspace {
  int max_tokens = 0;
  int hidden = 0;
  float *normed = nullptr;  // [Tmax][H]: the operator's RMSNorm output
  float *proj = nullptr;    // [Tmax][3H]: q|k|v of attention, B|C|gate of the conv
  float *mix = nullptr;     // [Tmax][H]: attention output / conv mix
  // FFN contexts run on one scratch: the first one created owns it
  moe_ctx *ffn_donor = nullptr;

  LayerWorkspace() = default;
  LayerWorkspace(int max_tokens, int hidden);
  ~LayerWorkspace();
  LayerWorkspace(const LayerWorkspace &) = delete;
  LayerWorkspace &operator=(const LayerWorkspace &) = delete;
};

// RMSNorm.  Reference include/layer.h:9-24, src/layer.cu:144-193, 1127-1150.
class RMSNorm {
public:
  RMSNorm(const std::string &weight_file);
  RMSNorm(const std::string &weight_name, size_t dim, const SyntheticWeights &s);
  explicit RMSNorm(Tensor weight);
  ~RMSNorm();
  // Host rows x [T][dim] -> y [T][dim] through the GPU (synchronous); needs init_gpu.
  void forward(const Tensor &x, Tensor &y);

  void init_gpu();
  // y = RMSNorm(x) for rows x [rows][hidden_dim] (device, asynchronous); y may alias x.
  void forward_gpu(float *x, float *y, int rows, int hidden_dim, hipStream_t stream = 0);

  const float *weight_gpu() const { return weight_.gpu(); }
  size_t dim() const { return weight_.size(); }
  const DeviceWeight &weight() const { return weight_; }

private:
  DeviceWeight weight_;
};

// Rotary position tables.  Reference include/layer.h:26-43, layer.cu:1155-1196.
class RotaryEmbedding {
public:
  RotaryEmbedding();  // MAX_POSITION_EMBEDDINGS positions
  explicit RotaryEmbedding(size_t max_seq_len);
  ~RotaryEmbedding();
  // The first seq_len rows of the tables [seq_len][HEAD_DIM] (host).
  void forward(size_t seq_len, Tensor &cos, Tensor &sin);

  void init_gpu();
  // Copies the first seq_len rows of the tables into cos / sin (device).
  void forward_gpu(size_t seq_len, float *cos, float *sin, hipStream_t stream = 0);

  float *cos_gpu_ = nullptr;  // [max_seq_len][HEAD_DIM]
  float *sin_gpu_ = nullptr;
  size_t max_seq_len() const { return max_seq_len_; }

private:
  Tensor cos_cached_;
  Tensor sin_cached_;
  size_t max_seq_len_;
};

// Dense SwiGLU FFN (layers 0-1), and one expert's weights inside the MoE
// block.  Reference include/layer.h:48-69, src/layer.cu:1200-1269.
class MLP {
public:
  MLP(const std::string &w1_file, const std::string &w2_file,
      const std::string &w3_file);
  MLP(Tensor w1, Tensor w2, Tensor w3);  // in-memory weights
  // Synthetic dense FFN: layers.{i}.feed_forward.w{1,2,3}.weight, w1/w3
  // [inter][hidden], w2 [hidden][inter].
  MLP(int layer_idx, int hidden, int inter, const SyntheticWeights &s);
  ~MLP();
  MLP(MLP &&other) noexcept;
  MLP &operator=(MLP &&other) noexcept;
  MLP(const MLP &) = delete;
  MLP &operator=(const MLP &) = delete;

  // y = W2 (silu(W1 x) * (W3 x)) on the MoE kernels (moe_dense_*,
  // include/moe_capi.h).  forward: host tensors x [T][H] -> y [T][H]
  // (synchronous); forward_gpu: device pointers, asynchronous on stream.
  // Both need init_gpu.
  void forward(const Tensor &x, Tensor &y);
  void forward_gpu(float *x, float *y, int batch, int seq_len, int hidden_size,
                   hipStream_t stream = 0);
  // y = residual + FFN(x); y may alias residual.
  void forward_gpu(float *x, float *y, const float *residual, int batch, int seq_len,
                   int hidden_size, hipStream_t stream);

  // Uploads the weights for forward_gpu (layer.cu:1216-1228): a dense context
  // with scratch for max_tokens() tokens (or on the scratch of
  // share_scratch_with's context).  The MoE block does not call it: it
  // uploads its experts itself.  w1_gpu_/w2_gpu_/w3_gpu_ stay null (the
  // weights live repacked inside the context).
  void init_gpu();
  void set_max_tokens(int n);  // before init_gpu (default 4096, layer.cu:1399)
  int max_tokens() const { return max_tokens_; }
  void share_scratch_with(moe_ctx *donor);  // before init_gpu
  moe_ctx *context() const { return dense_ctx_; }

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
  moe_ctx *donor_ = nullptr;
  int max_tokens_ = 4096;
  // synthetic weights (no host copy)
  bool synth_ = false;
  SyntheticWeights syn_{};
  int layer_idx_ = -1, syn_hidden_ = 0, syn_inter_ = 0;
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
  // Synthetic weights under the same names, drawn on the device by init_gpu.
  SparseMoeBlock(int layer_idx, int hidden, int inter, const SyntheticWeights &s);
  ~SparseMoeBlock();
  SparseMoeBlock(const SparseMoeBlock &) = delete;
  SparseMoeBlock &operator=(const SparseMoeBlock &) = delete;

  // Host tensors in and out: x [T][H] -> y [T][H], router_logits [T][E].
  // Runs the HIP path (device staging, synchronous); needs init_gpu().
  void forward(const Tensor &x, Tensor &y, Tensor &router_logits);

  // Allocates scratch for max_tokens() tokens (or uses share_scratch_with's)
  // and uploads the weights to the current HIP device (layer.cu:1357-1426).
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
  // layer.h:10-24, loaded as layers.{i}.ffn_norm.weight at layer.cu:1790-1793).
  // After init_gpu.  The device-pointer form takes a device copy.
  void set_post_attention_norm(const Tensor &weight);
  void set_post_attention_norm_gpu(const float *weight);
  // Steps 4-6 of DecoderLayer::forward_gpu (layer.cu:1903-1918) in one call:
  // out = h + MoE(rmsnorm(h)), rmsnorm as rms_norm_kernel (layer.cu:144-193).
  // out may alias h (the reference updates the layer output in place).
  void forward_gpu_norm(float *h, float *out, int batch, int seq_len, int hidden_size,
                        hipStream_t stream = 0);

  int layer_idx() const { return layer_idx_; }
  int max_tokens() const { return max_tokens_; }
  void set_max_tokens(int n);  // before init_gpu
  void share_scratch_with(moe_ctx *donor);  // before init_gpu
  moe_ctx *context() const { return ctx_; }
  int hidden() const;
  int inter() const;

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
  moe_ctx *donor_ = nullptr;
  int layer_idx_;
  int max_tokens_ = MOE_DEFAULT_MAX_TOKENS;
  bool synth_ = false;
  SyntheticWeights syn_{};
  int syn_hidden_ = 0, syn_inter_ = 0;
  void check_shapes() const;
  void upload_synthetic();
};

// Grouped-query attention with q/k RMSNorm and rotary embedding.  Reference
// include/layer.h:125-162, src/layer.cu:1508-1675.
class Attention {
public:
  // layers.{i}.self_attn.{q_proj, k_proj, v_proj, out_proj, q_layernorm,
  // k_layernorm}.weight through g_model_loader (layer.cu:1508-1526).
  Attention(int layer_idx);
  Attention(int layer_idx, const SyntheticWeights &s);
  ~Attention();
  // Host x [batch][seq][H] (or [seq][H]) -> output of the same shape, causal,
  // positions 0..seq-1; cos/sin [>= seq][HEAD_DIM]; attention_mask must be
  // null (the mask is causal).  Synchronous; needs init_gpu.
  void forward(const Tensor &x, const Tensor &cos, const Tensor &sin,
               const Tensor *attention_mask, Tensor &output);

  void init_gpu();
  // output = attention(x) (Attention::forward_gpu, layer.cu:1609-1675); cos /
  // sin: device tables [>= seq_len][HEAD_DIM].
  void forward_gpu(float *x, float *cos, float *sin, float *output, int batch,
                   int seq_len, int hidden_size, hipStream_t stream = 0);
  // output = residual + attention(x); output may alias residual, not x.
  void forward_gpu(float *x, float *cos, float *sin, const float *residual, float *output,
                   int batch, int seq_len, int hidden_size, hipStream_t stream);

  void set_workspace(LayerWorkspace *ws);  // before init_gpu
  void set_max_tokens(int n);              // own workspace size (default 4096)

private:
  DeviceWeight q_proj_, k_proj_, v_proj_, o_proj_;
  std::unique_ptr<RMSNorm> q_layernorm_;
  std::unique_ptr<RMSNorm> k_layernorm_;
  int layer_idx_;
  float *wqkv_gpu_ = nullptr;  // [q rows | k rows | v rows][H]
  LayerWorkspace *ws_ = nullptr;
  std::unique_ptr<LayerWorkspace> own_ws_;
  int max_tokens_ = 4096;
};

// Gated short convolution.  Reference include/layer.h:164-192,
// src/layer.cu:1680-1779.
class ShortConv {
public:
  // layers.{i}.conv.{conv, in_proj, out_proj}.weight (layer.cu:1680-1693).
  ShortConv(int layer_idx);
  ShortConv(int layer_idx, const SyntheticWeights &s);
  ~ShortConv();
  // Host x [batch][seq][H] (or [seq][H]) -> y of the same shape.  Synchronous.
  void forward(const Tensor &x, Tensor &y);

  void init_gpu();
  // y = out_proj(C * conv(B * gate)) (ShortConv::forward_gpu, layer.cu:1743-1779).
  void forward_gpu(float *x, float *y, int batch, int seq_len, int hidden_size,
                   hipStream_t stream = 0);
  // y = residual + shortconv(x); y may alias residual, not x.
  void forward_gpu(float *x, const float *residual, float *y, int batch, int seq_len,
                   int hidden_size, hipStream_t stream);

  void set_workspace(LayerWorkspace *ws);
  void set_max_tokens(int n);

private:
  DeviceWeight conv_weight_;      // [H][1][L]
  DeviceWeight in_proj_weight_;   // [3H][H]
  DeviceWeight out_proj_weight_;  // [H][H]
  int layer_idx_;
  LayerWorkspace *ws_ = nullptr;
  std::unique_ptr<LayerWorkspace> own_ws_;
  int max_tokens_ = 4096;
};

// One decoder layer: operator norm -> attention or short conv -> residual ->
// FFN norm -> MoE (or dense FFN) -> residual.  Reference
// include/layer.h:194-233, src/layer.cu:1784-1922.
class DecoderLayer {
public:
  // layers.{i}.{operator_norm, ffn_norm}.weight, the operator, and the MoE
  // block (layer_idx >= NUM_DENSE_LAYERS) or dense MLP (layer.cu:1784-1812).
  DecoderLayer(int layer_idx, bool is_attention_layer);
  // Synthetic weights; moe selects the FFN kind.
  DecoderLayer(int layer_idx, bool is_attention_layer, bool moe, const SyntheticWeights &s);
  ~DecoderLayer();
  // Host x [batch][seq][H] (or [seq][H]) -> output; cos/sin host tables;
  // attention_mask must be null.  Synchronous.
  void forward(const Tensor &x, const Tensor &cos, const Tensor &sin,
               const Tensor *attention_mask, Tensor &output);

  void init_gpu(int device_id);
  // output = layer(x) (DecoderLayer::forward_gpu, layer.cu:1882-1919); output
  // may alias x (the reference runs the layers in place on hidden_states).
  void forward_gpu(float *x, float *cos, float *sin, float *output, int batch,
                   int seq_len, int hidden_size, hipStream_t stream = 0);

  bool is_attention_layer() const { return is_attention_layer_; }
  int layer_idx() const { return layer_idx_; }
  void set_workspace(LayerWorkspace *ws);  // before init_gpu
  void set_max_tokens(int n);              // before init_gpu (own workspace)
  SparseMoeBlock *moe_block() const { return moe_block_.get(); }
  MLP *dense_mlp() const { return dense_mlp_.get(); }

private:
  int layer_idx_;
  bool is_attention_layer_;

  std::unique_ptr<RMSNorm> input_layernorm_;
  std::unique_ptr<RMSNorm> post_attention_layernorm_;
  std::unique_ptr<Attention> self_attn_;
  std::unique_ptr<ShortConv> short_conv_;
  std::unique_ptr<SparseMoeBlock> moe_block_;
  std::unique_ptr<MLP> dense_mlp_;

  LayerWorkspace *ws_ = nullptr;
  std::unique_ptr<LayerWorkspace> own_ws_;
  int max_tokens_ = 4096;
};
