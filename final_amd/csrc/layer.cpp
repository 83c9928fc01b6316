// MLP / SparseMoeBlock (include/layer.h) on top of the C-ABI.
// Reference: src/layer.cu:1200-1229 (MLP), 1274-1503 (SparseMoeBlock).
#include "layer.h"

#include <sstream>
#include <stdexcept>
#include <string>

#include "model_loader.h"

namespace {

void check(int rc, const char *what) {
  if (rc != MOE_OK)
    throw std::runtime_error(std::string(what) + ": " + moe_strerror(rc));
}

void check_hip(hipError_t e, const char *what) {
  if (e != hipSuccess)
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

std::string expert_name(int layer, size_t e, const char *w) {
  std::ostringstream ss;
  ss << "layers." << layer << ".feed_forward.experts." << e << "." << w << ".weight";
  return ss.str();
}

// Device buffer freed on scope exit.
struct DevBuf {
  void *p = nullptr;
  explicit DevBuf(size_t bytes) {
    if (bytes) check_hip(hipMalloc(&p, bytes), "hipMalloc");
  }
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  float *f() { return static_cast<float *>(p); }
};

}  // namespace

// ---------------------------------------------------------------------------
// MLP
// ---------------------------------------------------------------------------

MLP::MLP(const std::string &w1_file, const std::string &w2_file,
         const std::string &w3_file)
    : w1_(Tensor::load_from_file(w1_file)), w3_(Tensor::load_from_file(w3_file)),
      w2_(Tensor::load_from_file(w2_file)) {}

MLP::MLP(Tensor w1, Tensor w2, Tensor w3)
    : w1_(std::move(w1)), w3_(std::move(w3)), w2_(std::move(w2)) {}

MLP::MLP(int layer_idx, int hidden, int inter, const SyntheticWeights &s)
    : synth_(true), syn_(s), layer_idx_(layer_idx), syn_hidden_(hidden), syn_inter_(inter) {
  if (hidden <= 0 || inter <= 0) throw std::invalid_argument("MLP: hidden and inter must be > 0");
}

MLP::~MLP() { release_gpu(); }

MLP::MLP(MLP &&o) noexcept
    : w1_gpu_(o.w1_gpu_), w3_gpu_(o.w3_gpu_), w2_gpu_(o.w2_gpu_),
      temp_buf_gpu_(o.temp_buf_gpu_), w1_(std::move(o.w1_)), w3_(std::move(o.w3_)),
      w2_(std::move(o.w2_)), dense_ctx_(o.dense_ctx_), donor_(o.donor_),
      max_tokens_(o.max_tokens_), synth_(o.synth_), syn_(o.syn_), layer_idx_(o.layer_idx_),
      syn_hidden_(o.syn_hidden_), syn_inter_(o.syn_inter_) {
  o.w1_gpu_ = o.w3_gpu_ = o.w2_gpu_ = o.temp_buf_gpu_ = nullptr;
  o.dense_ctx_ = nullptr;
}

MLP &MLP::operator=(MLP &&o) noexcept {
  if (this != &o) {
    release_gpu();
    w1_ = std::move(o.w1_);
    w2_ = std::move(o.w2_);
    w3_ = std::move(o.w3_);
    w1_gpu_ = o.w1_gpu_;
    w2_gpu_ = o.w2_gpu_;
    w3_gpu_ = o.w3_gpu_;
    temp_buf_gpu_ = o.temp_buf_gpu_;
    dense_ctx_ = o.dense_ctx_;
    donor_ = o.donor_;
    max_tokens_ = o.max_tokens_;
    synth_ = o.synth_;
    syn_ = o.syn_;
    layer_idx_ = o.layer_idx_;
    syn_hidden_ = o.syn_hidden_;
    syn_inter_ = o.syn_inter_;
    o.w1_gpu_ = o.w3_gpu_ = o.w2_gpu_ = o.temp_buf_gpu_ = nullptr;
    o.dense_ctx_ = nullptr;
  }
  return *this;
}

void MLP::release_gpu() {
  if (w1_gpu_) (void)hipFree(w1_gpu_);
  if (w2_gpu_) (void)hipFree(w2_gpu_);
  if (w3_gpu_) (void)hipFree(w3_gpu_);
  w1_gpu_ = w2_gpu_ = w3_gpu_ = nullptr;
  if (dense_ctx_) moe_destroy(dense_ctx_);
  dense_ctx_ = nullptr;
}

void MLP::set_max_tokens(int n) {
  if (dense_ctx_) throw std::logic_error("MLP::set_max_tokens after init_gpu");
  if (n <= 0) throw std::invalid_argument("MLP::set_max_tokens: n <= 0");
  max_tokens_ = n;
}

void MLP::share_scratch_with(moe_ctx *donor) {
  if (dense_ctx_) throw std::logic_error("MLP::share_scratch_with after init_gpu");
  donor_ = donor;
}

void MLP::init_gpu() {
  release_gpu();
  int I, H;
  if (synth_) {
    I = syn_inter_;
    H = syn_hidden_;
  } else {
    if (w1_.ndim() != 2 || w3_.shape() != w1_.shape() || w2_.ndim() != 2 ||
        w2_.shape()[0] != w1_.shape()[1] || w2_.shape()[1] != w1_.shape()[0])
      throw std::invalid_argument("MLP::init_gpu: w1/w3 must be [I][H] and w2 [H][I]");
    I = (int)w1_.shape()[0];
    H = (int)w1_.shape()[1];
  }
  if (donor_)
    check(moe_dense_create_shared(H, I, max_tokens_, donor_, &dense_ctx_), "moe_dense_create_shared");
  else
    check(moe_dense_create(H, I, max_tokens_, &dense_ctx_), "moe_dense_create");
  if (!synth_) {
    check(moe_dense_set_weights(dense_ctx_, w1_.data(), w3_.data(), w2_.data(), 0, nullptr),
          "moe_dense_set_weights");
    return;
  }
  // synthetic: draw the three matrices on the device under their names
  const size_t n = (size_t)I * H;
  DevBuf stage(3 * n * sizeof(float));
  const char *names[3] = {"w1", "w3", "w2"};
  for (int k = 0; k < 3; ++k) {
    std::ostringstream ss;
    ss << "layers." << layer_idx_ << ".feed_forward." << names[k] << ".weight";
    check(lfm_synth_normal(stage.f() + k * n, n, syn_.seed, lfm_synth_stream_of(ss.str().c_str()),
                           syn_.std_dev, 0, nullptr),
          "lfm_synth_normal");
  }
  check(moe_dense_set_weights(dense_ctx_, stage.f(), stage.f() + n, stage.f() + 2 * n, 1, nullptr),
        "moe_dense_set_weights");
}

void MLP::forward_gpu(float *x, float *y, int batch, int seq_len, int hidden_size,
                      hipStream_t stream) {
  forward_gpu(x, y, nullptr, batch, seq_len, hidden_size, stream);
}

void MLP::forward_gpu(float *x, float *y, const float *residual, int batch, int seq_len,
                      int hidden_size, hipStream_t stream) {
  if (!dense_ctx_) throw std::logic_error("MLP::forward_gpu before init_gpu");
  if (hidden_size != (synth_ ? syn_hidden_ : (int)w1_.shape()[1]))
    throw std::invalid_argument("MLP::forward_gpu: hidden_size mismatch");
  if (batch < 0 || seq_len < 0) throw std::invalid_argument("negative batch/seq_len");
  check(moe_dense_forward(dense_ctx_, x, y, residual, batch * seq_len, stream),
        "moe_dense_forward");
}

void MLP::forward(const Tensor &x, Tensor &y) {
  if (!dense_ctx_) throw std::logic_error("MLP::forward before init_gpu");
  const size_t H = synth_ ? (size_t)syn_hidden_ : w1_.shape()[1];
  if (x.ndim() < 1 || x.size() % H != 0)
    throw std::invalid_argument("MLP::forward: x must be [T][H]");
  const size_t T = x.size() / H;
  DevBuf dx(T * H * sizeof(float)), dy(T * H * sizeof(float));
  check_hip(hipMemcpy(dx.f(), x.data(), T * H * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
  check(moe_dense_forward(dense_ctx_, dx.f(), dy.f(), nullptr, (int)T, nullptr), "moe_dense_forward");
  y = Tensor({T, H});
  check_hip(hipMemcpy(y.data(), dy.f(), T * H * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
  check(moe_device_status(dense_ctx_, nullptr), "device status");
}

// ---------------------------------------------------------------------------
// SparseMoeBlock
// ---------------------------------------------------------------------------

SparseMoeBlock::SparseMoeBlock(int layer_idx) : layer_idx_(layer_idx) {
  std::ostringstream ss;
  ss << "layers." << layer_idx << ".feed_forward.gate.weight";
  gate_ = Tensor::load_from_file(ss.str());
  experts_.reserve(NUM_EXPERTS);
  for (size_t e = 0; e < NUM_EXPERTS; ++e)
    experts_.emplace_back(expert_name(layer_idx, e, "w1"), expert_name(layer_idx, e, "w2"),
                          expert_name(layer_idx, e, "w3"));
  if (USE_EXPERT_BIAS) {
    std::ostringstream sb;
    sb << "layers." << layer_idx << ".feed_forward.expert_bias";
    expert_bias_ = Tensor::load_from_file(sb.str());
  }
  check_shapes();
}

SparseMoeBlock::SparseMoeBlock(int layer_idx, Tensor gate, std::vector<MLP> experts,
                               Tensor expert_bias)
    : gate_(std::move(gate)), experts_(std::move(experts)),
      expert_bias_(std::move(expert_bias)), layer_idx_(layer_idx) {
  check_shapes();
}

SparseMoeBlock::SparseMoeBlock(int layer_idx, int hidden, int inter, const SyntheticWeights &s)
    : layer_idx_(layer_idx), synth_(true), syn_(s), syn_hidden_(hidden), syn_inter_(inter) {
  if (hidden <= 0 || inter <= 0)
    throw std::invalid_argument("SparseMoeBlock: hidden and inter must be > 0");
}

SparseMoeBlock::~SparseMoeBlock() { moe_destroy(ctx_); }

int SparseMoeBlock::hidden() const { return synth_ ? syn_hidden_ : (int)gate_.shape()[1]; }

int SparseMoeBlock::inter() const {
  return synth_ ? syn_inter_ : (int)experts_[0].w1().shape()[0];
}

void SparseMoeBlock::share_scratch_with(moe_ctx *donor) {
  if (ctx_) throw std::logic_error("SparseMoeBlock::share_scratch_with after init_gpu");
  donor_ = donor;
}

// Draws the block's tensors on the device under the reference's names
// (layer.cu:1277-1298) and packs them into the context.
void SparseMoeBlock::upload_synthetic() {
  const size_t H = syn_hidden_, I = syn_inter_, E = NUM_EXPERTS;
  const size_t ng = E * H, nw = I * H;
  DevBuf stage((ng + E + 3 * E * nw) * sizeof(float));
  float *gate = stage.f(), *bias = gate + ng, *w = bias + E;
  auto draw = [&](float *dst, size_t n, const std::string &name) {
    check(lfm_synth_normal(dst, n, syn_.seed, lfm_synth_stream_of(name.c_str()), syn_.std_dev, 0,
                           nullptr),
          "lfm_synth_normal");
  };
  std::ostringstream sg, sb;
  sg << "layers." << layer_idx_ << ".feed_forward.gate.weight";
  sb << "layers." << layer_idx_ << ".feed_forward.expert_bias";
  draw(gate, ng, sg.str());
  draw(bias, E, sb.str());
  std::vector<const float *> w1(E), w2(E), w3(E);
  for (size_t e = 0; e < E; ++e) {
    float *b = w + 3 * e * nw;
    draw(b, nw, expert_name(layer_idx_, e, "w1"));
    draw(b + nw, nw, expert_name(layer_idx_, e, "w3"));
    draw(b + 2 * nw, nw, expert_name(layer_idx_, e, "w2"));
    w1[e] = b;
    w3[e] = b + nw;
    w2[e] = b + 2 * nw;
  }
  check(moe_set_weights(ctx_, gate, USE_EXPERT_BIAS ? bias : nullptr, w1.data(), w3.data(),
                        w2.data(), 1, nullptr),
        "moe_set_weights");
}

void SparseMoeBlock::check_shapes() const {
  if (synth_) return;
  if (gate_.ndim() != 2 || gate_.shape()[0] != NUM_EXPERTS)
    throw std::invalid_argument("SparseMoeBlock: gate must be [32][hidden]");
  const size_t H = gate_.shape()[1];
  if (experts_.size() != NUM_EXPERTS)
    throw std::invalid_argument("SparseMoeBlock: need 32 experts");
  const size_t I = experts_[0].w1().ndim() == 2 ? experts_[0].w1().shape()[0] : 0;
  for (const MLP &m : experts_) {
    if (m.w1().shape() != std::vector<size_t>{I, H} ||
        m.w3().shape() != std::vector<size_t>{I, H} ||
        m.w2().shape() != std::vector<size_t>{H, I})
      throw std::invalid_argument("SparseMoeBlock: expert shapes must be w1,w3 [I][H], w2 [H][I]");
  }
  if (expert_bias_.size() != 0 && expert_bias_.size() != NUM_EXPERTS)
    throw std::invalid_argument("SparseMoeBlock: expert_bias must have 32 entries");
}

void SparseMoeBlock::set_max_tokens(int n) {
  if (ctx_) throw std::logic_error("SparseMoeBlock::set_max_tokens after init_gpu");
  if (n <= 0) throw std::invalid_argument("SparseMoeBlock::set_max_tokens: n <= 0");
  max_tokens_ = n;
}

void SparseMoeBlock::init_gpu() {
  if (ctx_) {
    moe_destroy(ctx_);
    ctx_ = nullptr;
  }
  moe_dims d{};
  d.hidden = hidden();
  d.inter = inter();
  d.num_experts = (int)NUM_EXPERTS;
  d.top_k = (int)NUM_EXPERTS_PER_TOK;
  d.max_tokens = max_tokens_;
  if (donor_)
    check(moe_create_shared(&d, donor_, &ctx_), "moe_create_shared");
  else
    check(moe_create(&d, &ctx_), "moe_create");
  if (synth_) {
    upload_synthetic();
    return;
  }
  std::vector<const float *> w1(NUM_EXPERTS), w2(NUM_EXPERTS), w3(NUM_EXPERTS);
  for (size_t e = 0; e < NUM_EXPERTS; ++e) {
    w1[e] = experts_[e].w1().data();
    w2[e] = experts_[e].w2().data();
    w3[e] = experts_[e].w3().data();
  }
  check(moe_set_weights(ctx_, gate_.data(),
                        expert_bias_.size() ? expert_bias_.data() : nullptr, w1.data(),
                        w3.data(), w2.data(), 0, nullptr),
        "moe_set_weights");
}

void SparseMoeBlock::forward_gpu(float *x, float *y, int batch, int seq_len,
                                 int hidden_size, hipStream_t stream) {
  forward_gpu(x, y, nullptr, batch, seq_len, hidden_size, stream);
}

void SparseMoeBlock::forward_gpu(float *x, float *y, const float *residual, int batch,
                                 int seq_len, int hidden_size, hipStream_t stream) {
  if (!ctx_) throw std::logic_error("SparseMoeBlock::forward_gpu before init_gpu");
  if (hidden_size != hidden())
    throw std::invalid_argument("SparseMoeBlock::forward_gpu: hidden_size mismatch");
  if (batch < 0 || seq_len < 0) throw std::invalid_argument("negative batch/seq_len");
  check(moe_forward(ctx_, x, y, residual, batch * seq_len, stream), "moe_forward");
}

void SparseMoeBlock::set_post_attention_norm(const Tensor &weight) {
  if (!ctx_) throw std::logic_error("SparseMoeBlock::set_post_attention_norm before init_gpu");
  if (weight.size() != (size_t)hidden())
    throw std::invalid_argument("SparseMoeBlock::set_post_attention_norm: weight must have H entries");
  check(moe_set_norm_weight(ctx_, weight.data(), 0, nullptr), "moe_set_norm_weight");
}

void SparseMoeBlock::set_post_attention_norm_gpu(const float *weight) {
  if (!ctx_) throw std::logic_error("SparseMoeBlock::set_post_attention_norm_gpu before init_gpu");
  check(moe_set_norm_weight(ctx_, weight, 1, nullptr), "moe_set_norm_weight");
}

void SparseMoeBlock::forward_gpu_norm(float *h, float *out, int batch, int seq_len,
                                      int hidden_size, hipStream_t stream) {
  if (!ctx_) throw std::logic_error("SparseMoeBlock::forward_gpu_norm before init_gpu");
  if (hidden_size != hidden())
    throw std::invalid_argument("SparseMoeBlock::forward_gpu_norm: hidden_size mismatch");
  if (batch < 0 || seq_len < 0) throw std::invalid_argument("negative batch/seq_len");
  check(moe_forward_norm(ctx_, h, out, batch * seq_len, stream), "moe_forward_norm");
}

void SparseMoeBlock::forward(const Tensor &x, Tensor &y, Tensor &router_logits) {
  if (!ctx_) throw std::logic_error("SparseMoeBlock::forward before init_gpu");
  const size_t H = (size_t)hidden();
  if (x.ndim() < 1 || x.size() % H != 0)
    throw std::invalid_argument("SparseMoeBlock::forward: x must be [T][hidden]");
  const size_t T = x.size() / H;
  y = Tensor({T, H});
  router_logits = Tensor({T, NUM_EXPERTS});
  if (T == 0) return;
  DevBuf dx(T * H * sizeof(float)), dy(T * H * sizeof(float));
  check_hip(hipMemcpy(dx.p, x.data(), T * H * sizeof(float), hipMemcpyHostToDevice),
            "hipMemcpy");
  check(moe_forward(ctx_, dx.f(), dy.f(), nullptr, (int)T, nullptr), "moe_forward");
  check_hip(hipMemcpy(y.data(), dy.p, T * H * sizeof(float), hipMemcpyDeviceToHost),
            "hipMemcpy");
  check(moe_last_routing(ctx_, nullptr, nullptr, nullptr, router_logits.data(), (int)T, nullptr),
        "moe_last_routing");
  check(moe_device_status(ctx_, nullptr), "device status");
}

void SparseMoeBlock::route_tokens(const Tensor &router_logits,
                                  std::vector<int> &top_k_indices,
                                  std::vector<float> &top_k_weights) {
  if (!ctx_) throw std::logic_error("SparseMoeBlock::route_tokens before init_gpu");
  if (router_logits.ndim() != 2 || router_logits.shape()[1] != NUM_EXPERTS)
    throw std::invalid_argument("route_tokens: logits must be [T][32]");
  const size_t T = router_logits.shape()[0];
  top_k_indices.assign(T * NUM_EXPERTS_PER_TOK, -1);
  top_k_weights.assign(T * NUM_EXPERTS_PER_TOK, 0.0f);
  if (T == 0) return;
  DevBuf dl(T * NUM_EXPERTS * sizeof(float));
  check_hip(hipMemcpy(dl.p, router_logits.data(), T * NUM_EXPERTS * sizeof(float),
                      hipMemcpyHostToDevice),
            "hipMemcpy");
  check(moe_route_logits(ctx_, dl.f(), (int)T, nullptr), "moe_route_logits");
  check(moe_last_routing(ctx_, top_k_indices.data(), top_k_weights.data(), nullptr,
                         nullptr, (int)T, nullptr),
        "moe_last_routing");
}
