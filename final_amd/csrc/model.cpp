// LFM2Model (include/model.h) and the model handle of the C-ABI
// (lfm_model_*, include/lfm_capi.h).  Reference: src/model.cu:124-569.
#include "model.h"

#include <iostream>
#include <new>
#include <stdexcept>
#include <string>

namespace {

void check(int rc, const char *what) {
  if (rc != MOE_OK) throw std::runtime_error(std::string(what) + ": " + moe_strerror(rc));
}

void check_hip(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename T>
T *dev_alloc(size_t n) {
  void *p = nullptr;
  check_hip(hipMalloc(&p, (n ? n : 1) * sizeof(T)), "hipMalloc");
  return static_cast<T *>(p);
}

template <typename T>
void dev_free(T *&p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

}  // namespace

LFM2Model::LFM2Model(const std::string &model_file) : LFM2Model(model_file, 64, 512) {}

LFM2Model::LFM2Model(const std::string &model_file, int max_batch, int max_seq)
    : max_batch_(max_batch), max_seq_(max_seq) {
  if (max_batch <= 0 || max_seq <= 0) throw std::invalid_argument("LFM2Model: sizes must be > 0");
  g_model_loader = std::make_unique<ModelLoader>(model_file);
  build_from_loader();
  init_gpu();
}

// model.cu:158-189: embeddings, the layers (attention where LAYER_TYPES is
// 0), the final norm and the LM head (tied to the embeddings when
// lm_head.weight is absent).
void LFM2Model::build_from_loader() {
  embed_tokens_ = DeviceWeight("embed_tokens.weight");
  if (embed_tokens_.shape().size() != 2 || embed_tokens_.shape()[1] != HIDDEN_SIZE)
    throw std::invalid_argument("LFM2Model: embed_tokens must be [vocab][hidden]");
  vocab_ = embed_tokens_.shape()[0];
  layers_.reserve(NUM_HIDDEN_LAYERS);
  for (size_t i = 0; i < NUM_HIDDEN_LAYERS; ++i)
    layers_.push_back(std::make_unique<DecoderLayer>((int)i, LAYER_TYPES[i] == 0));
  norm_ = std::make_unique<RMSNorm>("embedding_norm.weight");
  if (g_model_loader->has_tensor("lm_head.weight")) lm_head_ = DeviceWeight("lm_head.weight");
}

LFM2Model::LFM2Model(const LFM2Config &cfg, const SyntheticWeights &s)
    : max_batch_(cfg.max_batch), max_seq_(cfg.max_seq) {
  if (cfg.max_batch <= 0 || cfg.max_seq <= 0 || cfg.num_layers < 0 ||
      (int)cfg.layer_types.size() < cfg.num_layers)
    throw std::invalid_argument("LFM2Model: bad config");
  embed_tokens_ = DeviceWeight("embed_tokens.weight", {VOCAB_SIZE, HIDDEN_SIZE}, s);
  layers_.reserve(cfg.num_layers);
  for (int i = 0; i < cfg.num_layers; ++i)
    layers_.push_back(std::make_unique<DecoderLayer>(i, cfg.layer_types[i] == 0,
                                                     i >= cfg.num_dense_layers, s));
  norm_ = std::make_unique<RMSNorm>("embedding_norm.weight", HIDDEN_SIZE, s);
  init_gpu();
}

// One GPU: every layer on the current device, one workspace and one FFN
// scratch for all of them (model.cu:191-233 spreads them over 4 GPUs).
void LFM2Model::init_gpu() {
  check_hip(hipGetDevice(&device_), "hipGetDevice");
  check_hip(hipStreamCreate(&stream_), "hipStreamCreate");
  const int tmax = max_tokens();
  ws_ = std::make_unique<LayerWorkspace>(tmax, (int)HIDDEN_SIZE);
  embed_tokens_.upload();
  if (lm_head_.size()) lm_head_.upload();
  norm_->init_gpu();
  rotary_ = std::make_unique<RotaryEmbedding>((size_t)max_seq_);
  rotary_->init_gpu();
  for (auto &l : layers_) {
    l->set_workspace(ws_.get());
    l->init_gpu(device_);
  }
  hidden_ = dev_alloc<float>((size_t)tmax * HIDDEN_SIZE);
  last_ = dev_alloc<float>((size_t)max_batch_ * HIDDEN_SIZE);
  logits_gpu_ = dev_alloc<float>((size_t)max_batch_ * vocab_);
  ids_gpu_ = dev_alloc<int>((size_t)tmax);
  bad_ids_ = dev_alloc<int>(1);
  check_hip(hipMemset(bad_ids_, 0, sizeof(int)), "hipMemset");
  check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

LFM2Model::~LFM2Model() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  // the first FFN context owns the scratch the later ones use: release in
  // reverse order
  while (!layers_.empty()) layers_.pop_back();
  dev_free(hidden_);
  dev_free(last_);
  dev_free(logits_gpu_);
  dev_free(ids_gpu_);
  dev_free(bad_ids_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

DecoderLayer &LFM2Model::layer(int i) {
  if (i < 0 || i >= num_layers()) throw std::out_of_range("LFM2Model::layer");
  return *layers_[i];
}

void LFM2Model::check_shape(int batch, int seq_len) const {
  if (batch < 0 || seq_len < 0) throw std::invalid_argument("LFM2Model: negative batch/seq_len");
  if (batch > max_batch_ || seq_len > max_seq_)
    throw std::invalid_argument("LFM2Model: batch/seq_len beyond the model's scratch");
}

void LFM2Model::embed_gpu(const int *ids, int batch, int seq_len, float *h, hipStream_t stream) {
  check_shape(batch, seq_len);
  check(lfm_embed(ids, embed_tokens_.gpu(), h, batch * seq_len, (int)HIDDEN_SIZE, (int)vocab_,
                  bad_ids_, stream),
        "lfm_embed");
}

void LFM2Model::layer_forward_gpu(int layer, float *h, int batch, int seq_len, hipStream_t stream) {
  check_shape(batch, seq_len);
  this->layer(layer).forward_gpu(h, rotary_->cos_gpu_, rotary_->sin_gpu_, h, batch, seq_len,
                                 (int)HIDDEN_SIZE, stream);
}

// model.cu:481-536: the final norm of each sequence's last token (the
// reference normalises every token, then copies the last rows), then the LM
// head on those rows.
void LFM2Model::head_gpu(const float *h, int batch, int seq_len, float *logits, hipStream_t stream) {
  check_shape(batch, seq_len);
  if (batch == 0 || seq_len == 0) return;
  const long long H = (long long)HIDDEN_SIZE;
  check(lfm_rmsnorm(h + (size_t)(seq_len - 1) * H, (long long)seq_len * H, norm_->weight_gpu(), last_,
                    H, batch, (int)H, stream),
        "lfm_rmsnorm");
  const float *head = lm_head_.size() ? lm_head_.gpu() : embed_tokens_.gpu();
  check(lfm_gemm_nt(last_, head, logits, nullptr, batch, (int)vocab_, (int)H, stream),
        "lfm_gemm_nt lm_head");
}

void LFM2Model::forward_gpu(const int *ids, int batch, int seq_len, float *logits,
                            hipStream_t stream) {
  check_shape(batch, seq_len);
  if (batch == 0 || seq_len == 0) return;
  embed_gpu(ids, batch, seq_len, hidden_, stream);
  for (int i = 0; i < num_layers(); ++i) layer_forward_gpu(i, hidden_, batch, seq_len, stream);
  head_gpu(hidden_, batch, seq_len, logits, stream);
}

void LFM2Model::forward(int sample_idx, int batch_size, const int *input_ids_ptr, size_t seq_len,
                        float *output_buffer) {
  (void)sample_idx;
  check_shape(batch_size, (int)seq_len);
  if (batch_size == 0 || seq_len == 0) return;
  if (!input_ids_ptr || !output_buffer) throw std::invalid_argument("LFM2Model::forward: null buffer");
  const size_t T = (size_t)batch_size * seq_len;
  check_hip(hipMemcpyAsync(ids_gpu_, input_ids_ptr, T * sizeof(int), hipMemcpyHostToDevice, stream_),
            "hipMemcpyAsync");
  forward_gpu(ids_gpu_, batch_size, (int)seq_len, logits_gpu_, stream_);
  check_hip(hipMemcpyAsync(output_buffer, logits_gpu_, (size_t)batch_size * vocab_ * sizeof(float),
                           hipMemcpyDeviceToHost, stream_),
            "hipMemcpyAsync");
}

void LFM2Model::sync() { check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }

void LFM2Model::forward(const std::vector<int> &input_ids, Tensor &logits) {
  logits = Tensor({1, vocab_});
  if (input_ids.empty()) return;
  forward(0, 1, input_ids.data(), input_ids.size(), logits.data());
  sync();
}

int LFM2Model::status(hipStream_t stream) {
  int bad = 0;
  if (hipMemcpyAsync(&bad, bad_ids_, sizeof(int), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return MOE_ERR_HIP;
  if (bad) {
    if (hipMemsetAsync(bad_ids_, 0, sizeof(int), stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
      return MOE_ERR_HIP;
    return MOE_ERR_INVALID_ARG;
  }
  for (auto &l : layers_) {
    moe_ctx *c = l->moe_block() ? l->moe_block()->context()
                                : (l->dense_mlp() ? l->dense_mlp()->context() : nullptr);
    if (!c) continue;
    const int rc = moe_device_status(c, stream);
    if (rc != MOE_OK) return rc;
  }
  return MOE_OK;
}

// ---------------------------------------------------------------------------
// C-ABI handle
// ---------------------------------------------------------------------------

struct lfm_model {
  std::unique_ptr<LFM2Model> m;
};

namespace {

// Runs f, mapping the C++ layer's exceptions to status codes.
template <typename F>
int guarded(F &&f) {
  try {
    f();
    return MOE_OK;
  } catch (const std::bad_alloc &) {
    return MOE_ERR_OUT_OF_MEMORY;
  } catch (const std::invalid_argument &) {
    return MOE_ERR_INVALID_ARG;
  } catch (const std::out_of_range &) {
    return MOE_ERR_INVALID_ARG;
  } catch (const std::logic_error &) {
    return MOE_ERR_NOT_READY;
  } catch (const std::runtime_error &e) {
    const std::string w = e.what();
    if (w.find("out of memory") != std::string::npos) return MOE_ERR_OUT_OF_MEMORY;
    std::cerr << "lfm: " << w << "\n";
    return MOE_ERR_HIP;
  } catch (...) {
    return MOE_ERR_INTERNAL;
  }
}

hipStream_t S(moe_stream_t s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

int lfm_model_create_synthetic(const lfm_model_config *cfg, lfm_model **out) {
  if (!cfg || !out) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  if (cfg->num_layers < 0 || cfg->max_batch <= 0 || cfg->max_seq <= 0 || cfg->num_dense_layers < 0)
    return MOE_ERR_INVALID_ARG;
  LFM2Config c;
  c.num_layers = cfg->num_layers;
  c.layer_types.assign(cfg->num_layers, 1);
  for (int i = 0; i < cfg->num_layers; ++i)
    c.layer_types[i] = cfg->layer_types ? cfg->layer_types[i]
                                        : LAYER_TYPES[i % (int)NUM_HIDDEN_LAYERS];
  c.num_dense_layers = cfg->num_dense_layers;
  c.max_batch = cfg->max_batch;
  c.max_seq = cfg->max_seq;
  SyntheticWeights s;
  s.seed = cfg->seed;
  s.std_dev = cfg->weight_std;
  lfm_model *h = new (std::nothrow) lfm_model();
  if (!h) return MOE_ERR_OUT_OF_MEMORY;
  const int rc = guarded([&] { h->m = std::make_unique<LFM2Model>(c, s); });
  if (rc != MOE_OK) {
    delete h;
    return rc;
  }
  *out = h;
  return MOE_OK;
}

int lfm_model_create_from_file(const char *path, int max_batch, int max_seq, lfm_model **out) {
  if (!path || !out || max_batch <= 0 || max_seq <= 0) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  lfm_model *h = new (std::nothrow) lfm_model();
  if (!h) return MOE_ERR_OUT_OF_MEMORY;
  const int rc = guarded([&] { h->m = std::make_unique<LFM2Model>(path, max_batch, max_seq); });
  if (rc != MOE_OK) {
    delete h;
    return rc;
  }
  *out = h;
  return MOE_OK;
}

int lfm_model_destroy(lfm_model *m) {
  delete m;
  return MOE_OK;
}

int lfm_model_forward(lfm_model *m, const int *ids, int batch, int seq, float *logits,
                      moe_stream_t stream) {
  if (!m || (batch * seq > 0 && (!ids || !logits))) return MOE_ERR_INVALID_ARG;
  return guarded([&] { m->m->forward_gpu(ids, batch, seq, logits, S(stream)); });
}

int lfm_model_embed(lfm_model *m, const int *ids, int batch, int seq, float *h,
                    moe_stream_t stream) {
  if (!m || (batch * seq > 0 && (!ids || !h))) return MOE_ERR_INVALID_ARG;
  return guarded([&] { m->m->embed_gpu(ids, batch, seq, h, S(stream)); });
}

int lfm_model_layer_forward(lfm_model *m, int layer, float *h, int batch, int seq,
                            moe_stream_t stream) {
  if (!m || (batch * seq > 0 && !h)) return MOE_ERR_INVALID_ARG;
  return guarded([&] { m->m->layer_forward_gpu(layer, h, batch, seq, S(stream)); });
}

int lfm_model_head(lfm_model *m, const float *h, int batch, int seq, float *logits,
                   moe_stream_t stream) {
  if (!m || (batch * seq > 0 && (!h || !logits))) return MOE_ERR_INVALID_ARG;
  return guarded([&] { m->m->head_gpu(h, batch, seq, logits, S(stream)); });
}

int lfm_model_moe(lfm_model *m, int layer, moe_ctx **out) {
  if (!m || !out) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  return guarded([&] {
    SparseMoeBlock *b = m->m->layer(layer).moe_block();
    *out = b ? b->context() : nullptr;
  });
}

int lfm_model_info(const lfm_model *m, int *num_layers, int *hidden, int *vocab, int *max_tokens) {
  if (!m) return MOE_ERR_INVALID_ARG;
  if (num_layers) *num_layers = m->m->num_layers();
  if (hidden) *hidden = (int)HIDDEN_SIZE;
  if (vocab) *vocab = m->m->vocab();
  if (max_tokens) *max_tokens = m->m->max_tokens();
  return MOE_OK;
}

int lfm_model_status(lfm_model *m, moe_stream_t stream) {
  if (!m) return MOE_ERR_INVALID_ARG;
  return m->m->status(S(stream));
}

}  // extern "C"
