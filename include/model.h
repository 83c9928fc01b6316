// LFM2-8B-A1B-style decoder model on one MI355X.  Drop-in for the reference's
// LFM2Model (include/model.h:26-96, src/model.cu): same constructor from a
// model file, the same forward(sample_idx, batch_size, ids, seq_len,
// output_buffer) / sync() pair.  The reference splits the 24 layers over 4
// GPUs as a 24-stage pipeline of worker threads with P2P copies and two
// streams per stage (model.cu:235-339, 385-560); here every stage runs on one
// GPU, on one stream, in order, and forward() enqueues stream-ordered work
// instead of pushing a task to stage 0.  Errors throw std::runtime_error.
#pragma once

#include <hip/hip_runtime_api.h>

#include <memory>
#include <string>
#include <vector>

#include "config.h"
#include "layer.h"
#include "model_loader.h"
#include "tensor.h"

// Shape of a synthetic model (no counterpart in the reference, whose model
// comes from model.bin).  Defaults: the reference's 24 layers and layer
// types, 2 dense layers; scratch for max_batch * max_seq tokens.
struct LFM2Config {
  int num_layers = (int)NUM_HIDDEN_LAYERS;
  std::vector<int> layer_types = std::vector<int>(LAYER_TYPES, LAYER_TYPES + NUM_HIDDEN_LAYERS);
  int num_dense_layers = (int)NUM_DENSE_LAYERS;
  int max_batch = 64;
  int max_seq = 512;
};

class LFM2Model {
public:
  // Reference model.cu:124-137: tensors by name from model_file (sets
  // g_model_loader), scratch for 64 sequences of 512 tokens.
  LFM2Model(const std::string &model_file);
  LFM2Model(const std::string &model_file, int max_batch, int max_seq);
  // Synthetic weights drawn on the device (embedding tied to the LM head).
  LFM2Model(const LFM2Config &cfg, const SyntheticWeights &s);
  ~LFM2Model();
  LFM2Model(const LFM2Model &) = delete;
  LFM2Model &operator=(const LFM2Model &) = delete;

  // Last-token logits of one sequence: logits [1][VOCAB_SIZE].  Synchronous.
  // (A warning stub in the reference, model.cu:562-569.)
  void forward(const std::vector<int> &input_ids, Tensor &logits);
  // Host ids [batch_size][seq_len] -> host output_buffer [batch_size][VOCAB]
  // (model.cu:341-355, 403-559); enqueued on the model's stream, finished by
  // sync().  sample_idx is accepted for the interface (the reference uses it
  // to pick a pipeline slot).  One call in flight at a time: the next call
  // reuses the staging buffers and waits for the previous one.
  void forward(int sample_idx, int batch_size, const int *input_ids_ptr, size_t seq_len,
               float *output_buffer);
  void sync();

  // Device pointers, asynchronous on `stream`, no host synchronisation:
  // ids [batch][seq] int32 -> logits [batch][vocab].
  void forward_gpu(const int *ids, int batch, int seq_len, float *logits, hipStream_t stream);
  // The same in pieces (for layer-wise checks): embedding into h
  // [batch*seq][H]; one decoder layer in place on h; final norm of each
  // sequence's last token and the LM head.
  void embed_gpu(const int *ids, int batch, int seq_len, float *h, hipStream_t stream);
  void layer_forward_gpu(int layer, float *h, int batch, int seq_len, hipStream_t stream);
  void head_gpu(const float *h, int batch, int seq_len, float *logits, hipStream_t stream);

  int num_layers() const { return (int)layers_.size(); }
  int max_tokens() const { return max_batch_ * max_seq_; }
  int max_batch() const { return max_batch_; }
  int max_seq() const { return max_seq_; }
  int vocab() const { return (int)vocab_; }
  DecoderLayer &layer(int i);
  // MOE_OK, MOE_ERR_INVALID_ARG after an out-of-range token id, or a MoE
  // layer's device status (moe_device_status).  Synchronises `stream`.
  int status(hipStream_t stream);

private:
  void build_from_loader();
  void init_gpu();
  void check_shape(int batch, int seq_len) const;

  int max_batch_ = 64, max_seq_ = 512;
  size_t vocab_ = VOCAB_SIZE;
  DeviceWeight embed_tokens_;  // [vocab][H]
  DeviceWeight lm_head_;       // [vocab][H]; empty = tied to embed_tokens_
  std::vector<std::unique_ptr<DecoderLayer>> layers_;
  std::unique_ptr<RMSNorm> norm_;
  std::unique_ptr<RotaryEmbedding> rotary_;
  std::unique_ptr<LayerWorkspace> ws_;
  float *hidden_ = nullptr;      // [Tmax][H]
  float *last_ = nullptr;        // [max_batch][H]: normalised last tokens
  float *logits_gpu_ = nullptr;  // [max_batch][vocab]: logits of host forwards
  int *ids_gpu_ = nullptr;       // [Tmax]: ids of host forwards
  int *bad_ids_ = nullptr;       // device flag set by the embedding
  hipStream_t stream_ = nullptr;
  int device_ = 0;
};
