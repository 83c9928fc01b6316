// RMSNorm, RotaryEmbedding, Attention, ShortConv and DecoderLayer
// (include/layer.h) on top of the C-ABI kernels (include/lfm_capi.h,
// include/moe_capi.h).  Reference: src/layer.cu:1127-1196 (RMSNorm,
// RotaryEmbedding), 1508-1675 (Attention), 1680-1779 (ShortConv),
// 1784-1922 (DecoderLayer).
#include <sstream>
#include <stdexcept>
#include <string>

#include "layer.h"
#include "model_loader.h"

namespace {

void check(int rc, const char *what) {
  if (rc != MOE_OK) throw std::runtime_error(std::string(what) + ": " + moe_strerror(rc));
}

void check_hip(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

float *dev_alloc(size_t n) {
  void *p = nullptr;
  if (n) check_hip(hipMalloc(&p, n * sizeof(float)), "hipMalloc");
  return static_cast<float *>(p);
}

void dev_free(float *&p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

std::string name_of(int layer, const char *rest) {
  std::ostringstream ss;
  ss << "layers." << layer << "." << rest;
  return ss.str();
}

// Device buffer freed on scope exit.
struct DevBuf {
  float *p = nullptr;
  explicit DevBuf(size_t n) : p(dev_alloc(n)) {}
  ~DevBuf() { dev_free(p); }
};

// Rows of a host activation tensor [..][H] (2-D [T][H] or 3-D [B][S][H]).
void rows_of(const Tensor &x, size_t H, int *batch, int *seq) {
  if (x.ndim() == 3 && x.shape()[2] == H) {
    *batch = (int)x.shape()[0];
    *seq = (int)x.shape()[1];
  } else if (x.ndim() == 2 && x.shape()[1] == H) {
    *batch = 1;
    *seq = (int)x.shape()[0];
  } else {
    throw std::invalid_argument("activation must be [seq][hidden] or [batch][seq][hidden]");
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// DeviceWeight, LayerWorkspace
// ---------------------------------------------------------------------------

DeviceWeight::DeviceWeight(const std::string &name)
    : name_(name), host_(Tensor::load_from_file(name)) {
  shape_ = host_.shape();
}

DeviceWeight::DeviceWeight(const std::string &name, Tensor host)
    : name_(name), shape_(host.shape()), host_(std::move(host)) {}

DeviceWeight::DeviceWeight(const std::string &name, std::vector<size_t> shape,
                           const SyntheticWeights &s)
    : name_(name), shape_(std::move(shape)), synth_(true), syn_(s) {}

DeviceWeight::~DeviceWeight() { release(); }

DeviceWeight::DeviceWeight(DeviceWeight &&o) noexcept
    : name_(std::move(o.name_)), shape_(std::move(o.shape_)), host_(std::move(o.host_)),
      synth_(o.synth_), syn_(o.syn_), gpu_(o.gpu_) {
  o.gpu_ = nullptr;
}

DeviceWeight &DeviceWeight::operator=(DeviceWeight &&o) noexcept {
  if (this != &o) {
    release();
    name_ = std::move(o.name_);
    shape_ = std::move(o.shape_);
    host_ = std::move(o.host_);
    synth_ = o.synth_;
    syn_ = o.syn_;
    gpu_ = o.gpu_;
    o.gpu_ = nullptr;
  }
  return *this;
}

size_t DeviceWeight::size() const {
  size_t n = shape_.empty() ? 0 : 1;
  for (size_t d : shape_) n *= d;
  return n;
}

void DeviceWeight::release() { dev_free(gpu_); }

void DeviceWeight::upload() {
  release();
  const size_t n = size();
  gpu_ = dev_alloc(n);
  if (!n) return;
  if (synth_) {
    const int rc = lfm_synth_is_norm(name_.c_str())
                       ? lfm_fill(gpu_, n, 1.0f, nullptr)
                       : lfm_synth_normal(gpu_, n, syn_.seed, lfm_synth_stream_of(name_.c_str()),
                                          syn_.std_dev, 0, nullptr);
    check(rc, "synthetic weight");
    check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
  } else {
    check_hip(hipMemcpy(gpu_, host_.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  }
}

LayerWorkspace::LayerWorkspace(int tmax, int h) : max_tokens(tmax), hidden(h) {
  if (tmax <= 0 || h <= 0) throw std::invalid_argument("LayerWorkspace: sizes must be > 0");
  const size_t n = (size_t)tmax * h;
  try {
    normed = dev_alloc(n);
    proj = dev_alloc(3 * n);
    mix = dev_alloc(n);
  } catch (...) {
    dev_free(normed);
    dev_free(proj);
    dev_free(mix);
    throw;
  }
}

LayerWorkspace::~LayerWorkspace() {
  dev_free(normed);
  dev_free(proj);
  dev_free(mix);
}

// ---------------------------------------------------------------------------
// RMSNorm (layer.cu:1127-1150)
// ---------------------------------------------------------------------------

RMSNorm::RMSNorm(const std::string &weight_file) : weight_(weight_file) {}

RMSNorm::RMSNorm(const std::string &weight_name, size_t dim, const SyntheticWeights &s)
    : weight_(weight_name, {dim}, s) {}

RMSNorm::RMSNorm(Tensor weight) : weight_("", std::move(weight)) {}

RMSNorm::~RMSNorm() = default;

void RMSNorm::init_gpu() { weight_.upload(); }

void RMSNorm::forward_gpu(float *x, float *y, int rows, int hidden_dim, hipStream_t stream) {
  if (!weight_.gpu()) throw std::logic_error("RMSNorm::forward_gpu before init_gpu");
  if ((size_t)hidden_dim != weight_.size())
    throw std::invalid_argument("RMSNorm::forward_gpu: hidden_dim mismatch");
  check(lfm_rmsnorm(x, hidden_dim, weight_.gpu(), y, hidden_dim, rows, hidden_dim, stream),
        "lfm_rmsnorm");
}

void RMSNorm::forward(const Tensor &x, Tensor &y) {
  if (!weight_.gpu()) throw std::logic_error("RMSNorm::forward before init_gpu");
  const size_t D = weight_.size();
  if (x.size() % D != 0) throw std::invalid_argument("RMSNorm::forward: x must be [rows][dim]");
  const size_t rows = x.size() / D;
  y = Tensor(x.shape());
  if (!rows) return;
  DevBuf d(rows * D);
  check_hip(hipMemcpy(d.p, x.data(), rows * D * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  forward_gpu(d.p, d.p, (int)rows, (int)D, nullptr);
  check_hip(hipMemcpy(y.data(), d.p, rows * D * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
}

// ---------------------------------------------------------------------------
// RotaryEmbedding (layer.cu:1155-1196)
// ---------------------------------------------------------------------------

RotaryEmbedding::RotaryEmbedding() : RotaryEmbedding(MAX_POSITION_EMBEDDINGS) {}

RotaryEmbedding::RotaryEmbedding(size_t max_seq_len) : max_seq_len_(max_seq_len) {
  cos_cached_ = Tensor({max_seq_len_, HEAD_DIM});
  sin_cached_ = Tensor({max_seq_len_, HEAD_DIM});
  check(lfm_rope_tables(cos_cached_.data(), sin_cached_.data(), (int)max_seq_len_, (int)HEAD_DIM,
                        ROPE_THETA),
        "lfm_rope_tables");
}

RotaryEmbedding::~RotaryEmbedding() {
  dev_free(cos_gpu_);
  dev_free(sin_gpu_);
}

void RotaryEmbedding::init_gpu() {
  dev_free(cos_gpu_);
  dev_free(sin_gpu_);
  const size_t n = max_seq_len_ * HEAD_DIM;
  cos_gpu_ = dev_alloc(n);
  sin_gpu_ = dev_alloc(n);
  check_hip(hipMemcpy(cos_gpu_, cos_cached_.data(), n * sizeof(float), hipMemcpyHostToDevice),
            "hipMemcpy");
  check_hip(hipMemcpy(sin_gpu_, sin_cached_.data(), n * sizeof(float), hipMemcpyHostToDevice),
            "hipMemcpy");
}

void RotaryEmbedding::forward(size_t seq_len, Tensor &cos, Tensor &sin) {
  if (seq_len > max_seq_len_) throw std::invalid_argument("RotaryEmbedding: seq_len too long");
  cos = cos_cached_.slice(0, 0, seq_len);
  sin = sin_cached_.slice(0, 0, seq_len);
}

void RotaryEmbedding::forward_gpu(size_t seq_len, float *cos, float *sin, hipStream_t stream) {
  if (!cos_gpu_) throw std::logic_error("RotaryEmbedding::forward_gpu before init_gpu");
  if (seq_len > max_seq_len_) throw std::invalid_argument("RotaryEmbedding: seq_len too long");
  const size_t bytes = seq_len * HEAD_DIM * sizeof(float);
  check_hip(hipMemcpyAsync(cos, cos_gpu_, bytes, hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync");
  check_hip(hipMemcpyAsync(sin, sin_gpu_, bytes, hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync");
}

// ---------------------------------------------------------------------------
// Attention (layer.cu:1508-1675)
// ---------------------------------------------------------------------------

namespace {
constexpr int kQCols = (int)(NUM_ATTENTION_HEADS * HEAD_DIM);   // 2048
constexpr int kKVCols = (int)(NUM_KEY_VALUE_HEADS * HEAD_DIM);  // 512
}  // namespace

Attention::Attention(int layer_idx) : layer_idx_(layer_idx) {
  q_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.q_proj.weight"));
  k_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.k_proj.weight"));
  v_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.v_proj.weight"));
  o_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.out_proj.weight"));
  q_layernorm_ = std::make_unique<RMSNorm>(name_of(layer_idx, "self_attn.q_layernorm.weight"));
  k_layernorm_ = std::make_unique<RMSNorm>(name_of(layer_idx, "self_attn.k_layernorm.weight"));
}

Attention::Attention(int layer_idx, const SyntheticWeights &s) : layer_idx_(layer_idx) {
  const size_t H = HIDDEN_SIZE;
  q_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.q_proj.weight"), {(size_t)kQCols, H}, s);
  k_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.k_proj.weight"), {(size_t)kKVCols, H}, s);
  v_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.v_proj.weight"), {(size_t)kKVCols, H}, s);
  o_proj_ = DeviceWeight(name_of(layer_idx, "self_attn.out_proj.weight"), {H, (size_t)kQCols}, s);
  q_layernorm_ =
      std::make_unique<RMSNorm>(name_of(layer_idx, "self_attn.q_layernorm.weight"), HEAD_DIM, s);
  k_layernorm_ =
      std::make_unique<RMSNorm>(name_of(layer_idx, "self_attn.k_layernorm.weight"), HEAD_DIM, s);
}

Attention::~Attention() { dev_free(wqkv_gpu_); }

void Attention::set_workspace(LayerWorkspace *ws) { ws_ = ws; }

void Attention::set_max_tokens(int n) {
  if (n <= 0) throw std::invalid_argument("Attention::set_max_tokens: n <= 0");
  max_tokens_ = n;
}

void Attention::init_gpu() {
  const size_t H = HIDDEN_SIZE;
  if (q_proj_.shape() != std::vector<size_t>{(size_t)kQCols, H} ||
      k_proj_.shape() != std::vector<size_t>{(size_t)kKVCols, H} ||
      v_proj_.shape() != std::vector<size_t>{(size_t)kKVCols, H} ||
      o_proj_.shape() != std::vector<size_t>{H, (size_t)kQCols} ||
      q_layernorm_->dim() != HEAD_DIM || k_layernorm_->dim() != HEAD_DIM)
    throw std::invalid_argument("Attention: unexpected weight shapes");
  q_layernorm_->init_gpu();
  k_layernorm_->init_gpu();
  // q, k and v projections as one [3072][H] matrix: one GEMM per forward
  dev_free(wqkv_gpu_);
  wqkv_gpu_ = dev_alloc((size_t)(kQCols + 2 * kKVCols) * H);
  DeviceWeight *parts[3] = {&q_proj_, &k_proj_, &v_proj_};
  size_t off = 0;
  for (DeviceWeight *w : parts) {
    w->upload();
    check_hip(hipMemcpy(wqkv_gpu_ + off, w->gpu(), w->size() * sizeof(float),
                        hipMemcpyDeviceToDevice),
              "hipMemcpy");
    off += w->size();
    w->release();
  }
  o_proj_.upload();
  if (!ws_) {
    own_ws_ = std::make_unique<LayerWorkspace>(max_tokens_, (int)H);
    ws_ = own_ws_.get();
  }
}

void Attention::forward_gpu(float *x, float *cos, float *sin, float *output, int batch,
                            int seq_len, int hidden_size, hipStream_t stream) {
  forward_gpu(x, cos, sin, nullptr, output, batch, seq_len, hidden_size, stream);
}

void Attention::forward_gpu(float *x, float *cos, float *sin, const float *residual,
                            float *output, int batch, int seq_len, int hidden_size,
                            hipStream_t stream) {
  if (!wqkv_gpu_ || !ws_) throw std::logic_error("Attention::forward_gpu before init_gpu");
  if ((size_t)hidden_size != HIDDEN_SIZE)
    throw std::invalid_argument("Attention::forward_gpu: hidden_size mismatch");
  if (batch < 0 || seq_len < 0) throw std::invalid_argument("negative batch/seq_len");
  const int T = batch * seq_len;
  if (T > ws_->max_tokens) throw std::invalid_argument("Attention: more tokens than the workspace");
  if (T == 0) return;
  const int ld = kQCols + 2 * kKVCols;
  float *qkv = ws_->proj, *att = ws_->mix;
  // 1. projections (layer.cu:1616-1634), q|k|v in one GEMM
  check(lfm_gemm_nt(x, wqkv_gpu_, qkv, nullptr, T, ld, hidden_size, stream), "lfm_gemm_nt qkv");
  // 2-4. q/k norm and rotary embedding in place (layer.cu:1637-1659)
  check(lfm_qk_norm_rope(qkv, ld, q_layernorm_->weight_gpu(), k_layernorm_->weight_gpu(), cos, sin,
                         batch, seq_len, (int)NUM_ATTENTION_HEADS, (int)NUM_KEY_VALUE_HEADS, kQCols,
                         stream),
        "lfm_qk_norm_rope");
  // 5. causal GQA attention (layer.cu:1661-1669)
  check(lfm_attention(qkv, ld, att, batch, seq_len, (int)NUM_ATTENTION_HEADS,
                      (int)NUM_KEY_VALUE_HEADS, kQCols, kQCols + kKVCols, stream),
        "lfm_attention");
  // 6. output projection (layer.cu:1671-1675), plus the residual when given
  check(lfm_gemm_nt(att, o_proj_.gpu(), output, residual, T, hidden_size, kQCols, stream),
        "lfm_gemm_nt out_proj");
}

void Attention::forward(const Tensor &x, const Tensor &cos, const Tensor &sin,
                        const Tensor *attention_mask, Tensor &output) {
  if (attention_mask) throw std::invalid_argument("Attention::forward: the mask is causal");
  int batch = 0, seq = 0;
  rows_of(x, HIDDEN_SIZE, &batch, &seq);
  if (cos.size() < (size_t)seq * HEAD_DIM || sin.size() < (size_t)seq * HEAD_DIM)
    throw std::invalid_argument("Attention::forward: cos/sin shorter than the sequence");
  output = Tensor(x.shape());
  const size_t n = x.size(), nt = (size_t)seq * HEAD_DIM;
  if (!n) return;
  DevBuf dx(n), dy(n), dc(nt), ds(nt);
  check_hip(hipMemcpy(dx.p, x.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  check_hip(hipMemcpy(dc.p, cos.data(), nt * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  check_hip(hipMemcpy(ds.p, sin.data(), nt * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  forward_gpu(dx.p, dc.p, ds.p, dy.p, batch, seq, (int)HIDDEN_SIZE, nullptr);
  check_hip(hipMemcpy(output.data(), dy.p, n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
}

// ---------------------------------------------------------------------------
// ShortConv (layer.cu:1680-1779)
// ---------------------------------------------------------------------------

ShortConv::ShortConv(int layer_idx) : layer_idx_(layer_idx) {
  conv_weight_ = DeviceWeight(name_of(layer_idx, "conv.conv.weight"));
  in_proj_weight_ = DeviceWeight(name_of(layer_idx, "conv.in_proj.weight"));
  out_proj_weight_ = DeviceWeight(name_of(layer_idx, "conv.out_proj.weight"));
}

ShortConv::ShortConv(int layer_idx, const SyntheticWeights &s) : layer_idx_(layer_idx) {
  const size_t H = HIDDEN_SIZE;
  conv_weight_ = DeviceWeight(name_of(layer_idx, "conv.conv.weight"), {H, 1, CONV_KERNEL}, s);
  in_proj_weight_ = DeviceWeight(name_of(layer_idx, "conv.in_proj.weight"), {3 * H, H}, s);
  out_proj_weight_ = DeviceWeight(name_of(layer_idx, "conv.out_proj.weight"), {H, H}, s);
}

ShortConv::~ShortConv() = default;

void ShortConv::set_workspace(LayerWorkspace *ws) { ws_ = ws; }

void ShortConv::set_max_tokens(int n) {
  if (n <= 0) throw std::invalid_argument("ShortConv::set_max_tokens: n <= 0");
  max_tokens_ = n;
}

void ShortConv::init_gpu() {
  const size_t H = HIDDEN_SIZE;
  if (conv_weight_.size() != H * CONV_KERNEL ||
      in_proj_weight_.shape() != std::vector<size_t>{3 * H, H} ||
      out_proj_weight_.shape() != std::vector<size_t>{H, H})
    throw std::invalid_argument("ShortConv: unexpected weight shapes");
  conv_weight_.upload();
  in_proj_weight_.upload();
  out_proj_weight_.upload();
  if (!ws_) {
    own_ws_ = std::make_unique<LayerWorkspace>(max_tokens_, (int)H);
    ws_ = own_ws_.get();
  }
}

void ShortConv::forward_gpu(float *x, float *y, int batch, int seq_len, int hidden_size,
                            hipStream_t stream) {
  forward_gpu(x, nullptr, y, batch, seq_len, hidden_size, stream);
}

void ShortConv::forward_gpu(float *x, const float *residual, float *y, int batch, int seq_len,
                            int hidden_size, hipStream_t stream) {
  if (!ws_ || !in_proj_weight_.gpu()) throw std::logic_error("ShortConv::forward_gpu before init_gpu");
  if ((size_t)hidden_size != HIDDEN_SIZE)
    throw std::invalid_argument("ShortConv::forward_gpu: hidden_size mismatch");
  if (batch < 0 || seq_len < 0) throw std::invalid_argument("negative batch/seq_len");
  const int T = batch * seq_len;
  if (T > ws_->max_tokens) throw std::invalid_argument("ShortConv: more tokens than the workspace");
  if (T == 0) return;
  // 1. in_proj (layer.cu:1745-1758)
  check(lfm_gemm_nt(x, in_proj_weight_.gpu(), ws_->proj, nullptr, T, 3 * hidden_size, hidden_size,
                    stream),
        "lfm_gemm_nt in_proj");
  // 2-4. B*gate, causal conv, C* (layer.cu:1760-1773), token-major
  check(lfm_shortconv(ws_->proj, conv_weight_.gpu(), ws_->mix, batch, seq_len, hidden_size,
                      (int)CONV_KERNEL, stream),
        "lfm_shortconv");
  // 5. out_proj (layer.cu:1775-1778), plus the residual when given
  check(lfm_gemm_nt(ws_->mix, out_proj_weight_.gpu(), y, residual, T, hidden_size, hidden_size,
                    stream),
        "lfm_gemm_nt out_proj");
}

void ShortConv::forward(const Tensor &x, Tensor &y) {
  int batch = 0, seq = 0;
  rows_of(x, HIDDEN_SIZE, &batch, &seq);
  y = Tensor(x.shape());
  const size_t n = x.size();
  if (!n) return;
  DevBuf dx(n), dy(n);
  check_hip(hipMemcpy(dx.p, x.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  forward_gpu(dx.p, dy.p, batch, seq, (int)HIDDEN_SIZE, nullptr);
  check_hip(hipMemcpy(y.data(), dy.p, n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
}

// ---------------------------------------------------------------------------
// DecoderLayer (layer.cu:1784-1922)
// ---------------------------------------------------------------------------

DecoderLayer::DecoderLayer(int layer_idx, bool is_attention_layer)
    : layer_idx_(layer_idx), is_attention_layer_(is_attention_layer) {
  input_layernorm_ = std::make_unique<RMSNorm>(name_of(layer_idx, "operator_norm.weight"));
  post_attention_layernorm_ = std::make_unique<RMSNorm>(name_of(layer_idx, "ffn_norm.weight"));
  if (is_attention_layer)
    self_attn_ = std::make_unique<Attention>(layer_idx);
  else
    short_conv_ = std::make_unique<ShortConv>(layer_idx);
  if (static_cast<size_t>(layer_idx) >= NUM_DENSE_LAYERS) {
    moe_block_ = std::make_unique<SparseMoeBlock>(layer_idx);
  } else {
    dense_mlp_ = std::make_unique<MLP>(name_of(layer_idx, "feed_forward.w1.weight"),
                                       name_of(layer_idx, "feed_forward.w2.weight"),
                                       name_of(layer_idx, "feed_forward.w3.weight"));
  }
}

DecoderLayer::DecoderLayer(int layer_idx, bool is_attention_layer, bool moe,
                           const SyntheticWeights &s)
    : layer_idx_(layer_idx), is_attention_layer_(is_attention_layer) {
  input_layernorm_ =
      std::make_unique<RMSNorm>(name_of(layer_idx, "operator_norm.weight"), HIDDEN_SIZE, s);
  post_attention_layernorm_ =
      std::make_unique<RMSNorm>(name_of(layer_idx, "ffn_norm.weight"), HIDDEN_SIZE, s);
  if (is_attention_layer)
    self_attn_ = std::make_unique<Attention>(layer_idx, s);
  else
    short_conv_ = std::make_unique<ShortConv>(layer_idx, s);
  if (moe)
    moe_block_ = std::make_unique<SparseMoeBlock>(layer_idx, (int)HIDDEN_SIZE,
                                                  (int)MOE_INTERMEDIATE_SIZE, s);
  else
    dense_mlp_ = std::make_unique<MLP>(layer_idx, (int)HIDDEN_SIZE, (int)INTERMEDIATE_SIZE, s);
}

DecoderLayer::~DecoderLayer() = default;

void DecoderLayer::set_workspace(LayerWorkspace *ws) { ws_ = ws; }

void DecoderLayer::set_max_tokens(int n) {
  if (n <= 0) throw std::invalid_argument("DecoderLayer::set_max_tokens: n <= 0");
  max_tokens_ = n;
}

void DecoderLayer::init_gpu(int device_id) {
  check_hip(hipSetDevice(device_id), "hipSetDevice");
  if (!ws_) {
    own_ws_ = std::make_unique<LayerWorkspace>(max_tokens_, (int)HIDDEN_SIZE);
    ws_ = own_ws_.get();
  }
  input_layernorm_->init_gpu();
  post_attention_layernorm_->init_gpu();
  if (self_attn_) {
    self_attn_->set_workspace(ws_);
    self_attn_->init_gpu();
  }
  if (short_conv_) {
    short_conv_->set_workspace(ws_);
    short_conv_->init_gpu();
  }
  if (moe_block_) {
    moe_block_->set_max_tokens(ws_->max_tokens);
    if (ws_->ffn_donor) moe_block_->share_scratch_with(ws_->ffn_donor);
    moe_block_->init_gpu();
    moe_block_->set_post_attention_norm_gpu(post_attention_layernorm_->weight_gpu());
    if (!ws_->ffn_donor) ws_->ffn_donor = moe_block_->context();
  }
  if (dense_mlp_) {
    dense_mlp_->set_max_tokens(ws_->max_tokens);
    if (ws_->ffn_donor) dense_mlp_->share_scratch_with(ws_->ffn_donor);
    dense_mlp_->init_gpu();
    if (!ws_->ffn_donor) ws_->ffn_donor = dense_mlp_->context();
  }
}

void DecoderLayer::forward_gpu(float *x, float *cos, float *sin, float *output, int batch,
                               int seq_len, int hidden_size, hipStream_t stream) {
  if (!ws_) throw std::logic_error("DecoderLayer::forward_gpu before init_gpu");
  if ((size_t)hidden_size != HIDDEN_SIZE)
    throw std::invalid_argument("DecoderLayer::forward_gpu: hidden_size mismatch");
  if (batch < 0 || seq_len < 0) throw std::invalid_argument("negative batch/seq_len");
  const int T = batch * seq_len;
  if (T > ws_->max_tokens) throw std::invalid_argument("DecoderLayer: more tokens than the workspace");
  if (T == 0) return;
  // 1. operator norm (layer.cu:1886-1887)
  input_layernorm_->forward_gpu(x, ws_->normed, T, hidden_size, stream);
  // 2-3. operator and the first residual (layer.cu:1890-1901): output = x + op
  if (is_attention_layer_)
    self_attn_->forward_gpu(ws_->normed, cos, sin, x, output, batch, seq_len, hidden_size, stream);
  else
    short_conv_->forward_gpu(ws_->normed, x, output, batch, seq_len, hidden_size, stream);
  // 4-6. FFN norm, FFN and the second residual (layer.cu:1903-1918)
  if (moe_block_) {
    moe_block_->forward_gpu_norm(output, output, batch, seq_len, hidden_size, stream);
  } else {
    post_attention_layernorm_->forward_gpu(output, ws_->normed, T, hidden_size, stream);
    dense_mlp_->forward_gpu(ws_->normed, output, output, batch, seq_len, hidden_size, stream);
  }
}

void DecoderLayer::forward(const Tensor &x, const Tensor &cos, const Tensor &sin,
                           const Tensor *attention_mask, Tensor &output) {
  if (attention_mask) throw std::invalid_argument("DecoderLayer::forward: the mask is causal");
  int batch = 0, seq = 0;
  rows_of(x, HIDDEN_SIZE, &batch, &seq);
  output = Tensor(x.shape());
  const size_t n = x.size(), nt = (size_t)seq * HEAD_DIM;
  if (!n) return;
  if (is_attention_layer_ && (cos.size() < nt || sin.size() < nt))
    throw std::invalid_argument("DecoderLayer::forward: cos/sin shorter than the sequence");
  DevBuf dh(n), dc(is_attention_layer_ ? nt : 0), ds(is_attention_layer_ ? nt : 0);
  check_hip(hipMemcpy(dh.p, x.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  if (is_attention_layer_) {
    check_hip(hipMemcpy(dc.p, cos.data(), nt * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
    check_hip(hipMemcpy(ds.p, sin.data(), nt * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  }
  forward_gpu(dh.p, dc.p, ds.p, dh.p, batch, seq, (int)HIDDEN_SIZE, nullptr);
  check_hip(hipMemcpy(output.data(), dh.p, n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
}
