// C++ tests of the reference-shaped interface (include/layer.h, tensor.h,
// model_loader.h) of the MoE block, driven the way the reference's engine
// drives SparseMoeBlock (weights by tensor name through g_model_loader,
// init_gpu, forward_gpu on device buffers).  Checks against the CPU oracle
// (oracle/liboracle.so), which only tests link.
//
//   test_layer cpu   Tensor, model.bin loader, construction by name, errors
//   test_layer gpu   SparseMoeBlock on the GPU vs the oracle
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "layer.h"
#include "model.h"
#include "model_loader.h"
#include "moe_synth.h"
#include "tensor.h"

extern "C" {
#include "../../oracle/moe_oracle.h"
}

struct SparseMoeBlockTestAccess {
  static void route(SparseMoeBlock &b, const Tensor &logits, std::vector<int> &idx,
                    std::vector<float> &w) {
    b.route_tokens(logits, idx, w);
  }
};

namespace {

int g_failed = 0, g_checks = 0;

#define CHECK(cond)                                                        \
  do {                                                                     \
    ++g_checks;                                                            \
    if (!(cond)) {                                                         \
      ++g_failed;                                                          \
      std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
    }                                                                      \
  } while (0)

bool throws(const std::function<void()> &f) {
  try {
    f();
  } catch (const std::exception &) {
    return true;
  }
  return false;
}

struct Entry {
  std::string name;
  std::vector<uint32_t> shape;
  std::vector<float> data;
};

// model.bin in the reference's format (src/model_loader.cpp:22-68).
void write_model(const std::string &path, const std::vector<Entry> &es) {
  uint64_t header = 12;
  for (const auto &e : es) header += 4 + e.name.size() + 4 + 4 * e.shape.size() + 8;
  std::ofstream f(path, std::ios::binary);
  f.write("LFM2", 4);
  const uint32_t version = 1, n = (uint32_t)es.size();
  f.write((const char *)&version, 4);
  f.write((const char *)&n, 4);
  uint64_t off = header;
  for (const auto &e : es) {
    const uint32_t len = (uint32_t)e.name.size(), nd = (uint32_t)e.shape.size();
    f.write((const char *)&len, 4);
    f.write(e.name.data(), len);
    f.write((const char *)&nd, 4);
    f.write((const char *)e.shape.data(), 4 * nd);
    f.write((const char *)&off, 8);
    off += e.data.size() * 4;
  }
  for (const auto &e : es) f.write((const char *)e.data.data(), (std::streamsize)(e.data.size() * 4));
}

std::vector<float> normal(std::mt19937 &rng, size_t n, float sd) {
  std::normal_distribution<float> d(0.0f, sd);
  std::vector<float> v(n);
  for (auto &x : v) x = d(rng);
  return v;
}

constexpr int kH = 256, kI = 256, kE = 32, kLayer = 5;

struct Weights {
  std::vector<float> gate, bias, w1, w3, w2;  // w1/w3 [E][I][H], w2 [E][H][I]
};

Weights make_weights(unsigned seed) {
  std::mt19937 rng(seed);
  Weights w;
  w.gate = normal(rng, (size_t)kE * kH, 0.1f);
  w.bias = normal(rng, kE, 0.02f);
  w.w1 = normal(rng, (size_t)kE * kI * kH, 0.05f);
  w.w3 = normal(rng, (size_t)kE * kI * kH, 0.05f);
  w.w2 = normal(rng, (size_t)kE * kH * kI, 0.05f);
  return w;
}

std::string model_path() { return "test_layer_model.bin"; }

void write_layer_model(const Weights &w) {
  std::vector<Entry> es;
  const std::string p = "layers." + std::to_string(kLayer) + ".feed_forward.";
  es.push_back({p + "gate.weight", {kE, kH}, w.gate});
  es.push_back({p + "expert_bias", {kE}, w.bias});
  for (int e = 0; e < kE; ++e) {
    const std::string q = p + "experts." + std::to_string(e) + ".";
    es.push_back({q + "w1.weight", {kI, kH},
                  std::vector<float>(w.w1.begin() + (size_t)e * kI * kH,
                                     w.w1.begin() + (size_t)(e + 1) * kI * kH)});
    es.push_back({q + "w2.weight", {kH, kI},
                  std::vector<float>(w.w2.begin() + (size_t)e * kH * kI,
                                     w.w2.begin() + (size_t)(e + 1) * kH * kI)});
    es.push_back({q + "w3.weight", {kI, kH},
                  std::vector<float>(w.w3.begin() + (size_t)e * kI * kH,
                                     w.w3.begin() + (size_t)(e + 1) * kI * kH)});
  }
  write_model(model_path(), es);
}

void cpu_tests() {
  // Tensor
  Tensor t({2, 3});
  CHECK(t.ndim() == 2 && t.size() == 6 && t.size(1) == 3 && t.size(-1) == 3);
  for (size_t i = 0; i < 6; ++i) t[i] = (float)i;
  CHECK(t.at(1, 2) == 5.0f);
  Tensor c = t;  // deep copy
  c[0] = 42.0f;
  CHECK(t[0] == 0.0f);
  Tensor v = t.view({3, 2});  // shares data
  v[1] = 7.0f;
  CHECK(t[1] == 7.0f);
  CHECK(throws([&] { t.view({4, 2}); }));
  CHECK(throws([&] { t.reshape({5}); }));
  CHECK(throws([&] { t.size(2); }));
  Tensor tt = t.transpose(0, 1);
  CHECK(tt.shape()[0] == 3 && tt.at(2, 1) == t.at(1, 2));
  Tensor s = t.slice(1, 1, 3);
  CHECK(s.shape()[1] == 2 && s.at(1, 0) == t.at(1, 1));
  Tensor m = std::move(c);
  CHECK(m[0] == 42.0f && c.size() == 0);
  t.save_to_file("test_layer_tensor.bin");
  Tensor r = Tensor::load_from_file("test_layer_tensor.bin");
  CHECK(r.shape() == t.shape() && std::memcmp(r.data(), t.data(), 24) == 0);
  CHECK(throws([] { Tensor::load_from_file("no_such_file.bin"); }));

  // model.bin loader and construction by name
  Weights w = make_weights(1);
  write_layer_model(w);
  g_model_loader = std::make_unique<ModelLoader>(model_path());
  const std::string p = "layers." + std::to_string(kLayer) + ".feed_forward.";
  CHECK(g_model_loader->num_tensors() == 2 + 3 * kE);
  CHECK(g_model_loader->has_tensor(p + "gate.weight"));
  CHECK(g_model_loader->get_shape(p + "experts.3.w2.weight") == std::vector<size_t>({kH, kI}));
  Tensor g = Tensor::load_from_file(p + "gate.weight");
  CHECK(std::memcmp(g.data(), w.gate.data(), w.gate.size() * 4) == 0);
  CHECK(throws([&] { g_model_loader->load_tensor("layers.0.missing"); }));
  MLP mlp(p + "experts.7.w1.weight", p + "experts.7.w2.weight", p + "experts.7.w3.weight");
  CHECK(std::memcmp(mlp.w3().data(), w.w3.data() + (size_t)7 * kI * kH, (size_t)kI * kH * 4) == 0);
  CHECK(throws([&] { mlp.forward_gpu(nullptr, nullptr, 1, 1, kH, 0); }));
  SparseMoeBlock blk(kLayer);
  CHECK(blk.layer_idx() == kLayer && blk.context() == nullptr);
  CHECK(throws([&] { blk.forward_gpu(nullptr, nullptr, 1, 1, kH, 0); }));  // before init_gpu
  CHECK(throws([] { SparseMoeBlock bad(kLayer + 1); }));                  // tensors absent
  {
    std::ofstream f("test_layer_bad.bin", std::ios::binary);
    f.write("XXXX", 4);
  }
  CHECK(throws([] { ModelLoader l("test_layer_bad.bin"); }));
  CHECK(throws([] { ModelLoader l("no_such_model.bin"); }));
  g_model_loader.reset();
}

bool close(float a, float b) { return std::fabs(a - b) <= 1e-4f + 1e-3f * std::fabs(b); }

void gpu_tests() {
  Weights w = make_weights(2);
  write_layer_model(w);
  g_model_loader = std::make_unique<ModelLoader>(model_path());
  SparseMoeBlock blk(kLayer);  // by name, like DecoderLayer (layer.cu:1803-1804)
  blk.set_max_tokens(512);
  blk.init_gpu();
  g_model_loader.reset();

  for (int T : {1, 37, 300}) {
    std::mt19937 rng(100 + T);
    std::vector<float> x = normal(rng, (size_t)T * kH, 1.0f);
    std::vector<float> res = normal(rng, (size_t)T * kH, 1.0f);
    std::vector<float> yref((size_t)T * kH), yres((size_t)T * kH), lref((size_t)T * kE);
    std::vector<int> iref((size_t)T * 4), cref(kE);
    std::vector<float> wref((size_t)T * 4);
    CHECK(orc_moe_forward(x.data(), w.gate.data(), w.bias.data(), w.w1.data(), w.w3.data(),
                          w.w2.data(), nullptr, T, kH, kI, kE, nullptr, yref.data(), lref.data(),
                          iref.data(), wref.data(), cref.data()) == 0);
    CHECK(orc_moe_forward(x.data(), w.gate.data(), w.bias.data(), w.w1.data(), w.w3.data(),
                          w.w2.data(), res.data(), T, kH, kI, kE, nullptr, yres.data(), nullptr,
                          nullptr, nullptr, nullptr) == 0);
    // device path: forward_gpu(x, y, batch, seq_len, hidden, stream)
    float *dx = nullptr, *dy = nullptr, *dr = nullptr;
    const size_t bytes = (size_t)T * kH * 4;
    CHECK(hipMalloc(&dx, bytes) == hipSuccess && hipMalloc(&dy, bytes) == hipSuccess &&
          hipMalloc(&dr, bytes) == hipSuccess);
    hipStream_t st;
    CHECK(hipStreamCreate(&st) == hipSuccess);
    CHECK(hipMemcpy(dx, x.data(), bytes, hipMemcpyHostToDevice) == hipSuccess);
    CHECK(hipMemcpy(dr, res.data(), bytes, hipMemcpyHostToDevice) == hipSuccess);
    blk.forward_gpu(dx, dy, 1, T, kH, st);
    std::vector<float> y((size_t)T * kH), yr((size_t)T * kH);
    CHECK(hipStreamSynchronize(st) == hipSuccess);
    CHECK(hipMemcpy(y.data(), dy, bytes, hipMemcpyDeviceToHost) == hipSuccess);
    blk.forward_gpu(dx, dr, dr, 1, T, kH, st);  // residual fused, in place
    CHECK(hipStreamSynchronize(st) == hipSuccess);
    CHECK(hipMemcpy(yr.data(), dr, bytes, hipMemcpyDeviceToHost) == hipSuccess);
    int bad = 0;
    for (size_t i = 0; i < y.size(); ++i) bad += !close(y[i], yref[i]) + !close(yr[i], yres[i]);
    CHECK(bad == 0);
    // host path: forward(x, y, router_logits), logits bit-exact
    Tensor tx({(size_t)T, (size_t)kH}, x.data(), true), ty, tl;
    blk.forward(tx, ty, tl);
    CHECK(std::memcmp(tl.data(), lref.data(), lref.size() * 4) == 0);
    bad = 0;
    for (size_t i = 0; i < y.size(); ++i) bad += !close(ty.data()[i], yref[i]);
    CHECK(bad == 0);
    // route_tokens on the oracle's logits: indices and weights bit-exact
    std::vector<int> idx;
    std::vector<float> wt;
    SparseMoeBlockTestAccess::route(blk, tl, idx, wt);
    CHECK(idx == iref);
    CHECK(std::memcmp(wt.data(), wref.data(), wref.size() * 4) == 0);
    (void)hipFree(dx);
    (void)hipFree(dy);
    (void)hipFree(dr);
    (void)hipStreamDestroy(st);
    std::printf("gpu T=%d ok\n", T);
  }
  // post-attention RMSNorm fused in front of the block, output in place
  {
    std::mt19937 rng(7);
    std::vector<float> nw = normal(rng, kH, 0.1f);
    for (float &v : nw) v += 1.0f;
    Tensor tnw({(size_t)kH}, nw.data(), true);
    blk.set_post_attention_norm(tnw);
    for (int T : {1, 37, 300}) {
      std::vector<float> h = normal(rng, (size_t)T * kH, 2.0f), xn((size_t)T * kH),
                         yref((size_t)T * kH);
      orc_rmsnorm(h.data(), nw.data(), T, kH, xn.data());
      CHECK(orc_moe_forward(xn.data(), w.gate.data(), w.bias.data(), w.w1.data(), w.w3.data(),
                            w.w2.data(), h.data(), T, kH, kI, kE, nullptr, yref.data(), nullptr,
                            nullptr, nullptr, nullptr) == 0);
      float *dh = nullptr;
      const size_t bytes = (size_t)T * kH * 4;
      CHECK(hipMalloc(&dh, bytes) == hipSuccess);
      CHECK(hipMemcpy(dh, h.data(), bytes, hipMemcpyHostToDevice) == hipSuccess);
      blk.forward_gpu_norm(dh, dh, 1, T, kH, 0);
      std::vector<float> y((size_t)T * kH);
      CHECK(hipDeviceSynchronize() == hipSuccess);
      CHECK(hipMemcpy(y.data(), dh, bytes, hipMemcpyDeviceToHost) == hipSuccess);
      int bad = 0;
      for (size_t i = 0; i < y.size(); ++i) bad += !close(y[i], yref[i]);
      CHECK(bad == 0);
      (void)hipFree(dh);
      std::printf("gpu norm T=%d ok\n", T);
    }
  }
  // dense FFN (MLP::forward_gpu, layer.cu:1231-1269) on the MoE kernels
  {
    constexpr int kDI = 1024;  // the intermediate must split into 4 chunks of 256
    std::mt19937 rng(9);
    std::vector<float> w1 = normal(rng, (size_t)kDI * kH, 0.05f),
                       w3 = normal(rng, (size_t)kDI * kH, 0.05f),
                       w2 = normal(rng, (size_t)kH * kDI, 0.05f);
    MLP dense(Tensor({(size_t)kDI, (size_t)kH}, w1.data(), true),
              Tensor({(size_t)kH, (size_t)kDI}, w2.data(), true),
              Tensor({(size_t)kDI, (size_t)kH}, w3.data(), true));
    CHECK(throws([&] { dense.forward_gpu(nullptr, nullptr, 1, 1, kH, 0); }));  // before init_gpu
    dense.set_max_tokens(256);
    dense.init_gpu();
    for (int T : {1, 24, 200}) {
      std::vector<float> x = normal(rng, (size_t)T * kH, 1.0f), yref((size_t)T * kH);
      CHECK(orc_dense_mlp(x.data(), w1.data(), w3.data(), w2.data(), nullptr, T, kH, kDI,
                          yref.data()) == 0);
      Tensor tx({(size_t)T, (size_t)kH}, x.data(), true), ty;
      dense.forward(tx, ty);
      int bad = 0;
      for (size_t i = 0; i < yref.size(); ++i) bad += !close(ty.data()[i], yref[i]);
      CHECK(bad == 0);
      std::printf("gpu dense T=%d ok\n", T);
    }
  }
  // route_tokens on crafted logits (equal logits, large margins) vs the oracle
  Tensor lt({3, (size_t)kE});
  lt.zero();
  for (int e : {30, 3, 17, 8}) lt.at(1, e) = 5.0f;
  for (int e = 0; e < kE; ++e) lt.at(2, e) = (float)(e % 4) * 0.25f;
  std::vector<int> idx, iref(12), cnt(kE);
  std::vector<float> wt, wref(12);
  SparseMoeBlockTestAccess::route(blk, lt, idx, wt);
  orc_route(lt.data(), w.bias.data(), 3, kE, iref.data(), wref.data(), cnt.data());
  CHECK(idx == iref);
  CHECK(std::memcmp(wt.data(), wref.data(), wref.size() * 4) == 0);
}

// The block at the reference's shapes (hidden 2048, inter 1792), in-memory
// weights: small batches reach the weight-streaming kernel.
void gpu_full_shape_tests() {
  constexpr int H = 2048, I = 1792;
  std::vector<float> gate((size_t)kE * H), bias(kE), w1((size_t)kE * I * H), w3(w1.size()),
      w2((size_t)kE * H * I);
  moe_synth_normal(3, 0, 0.02f, 0, gate.data(), gate.size());
  moe_synth_normal(3, 1, 0.02f, 0, bias.data(), bias.size());
  moe_synth_normal(3, 2, 0.02f, 0, w1.data(), w1.size());
  moe_synth_normal(3, 3, 0.02f, 0, w3.data(), w3.size());
  moe_synth_normal(3, 4, 0.02f, 0, w2.data(), w2.size());
  std::vector<MLP> experts;
  for (int e = 0; e < kE; ++e)
    experts.emplace_back(Tensor({(size_t)I, (size_t)H}, w1.data() + (size_t)e * I * H, true),
                         Tensor({(size_t)H, (size_t)I}, w2.data() + (size_t)e * H * I, true),
                         Tensor({(size_t)I, (size_t)H}, w3.data() + (size_t)e * I * H, true));
  SparseMoeBlock blk(kLayer, Tensor({(size_t)kE, (size_t)H}, gate.data(), true), std::move(experts),
                     Tensor({(size_t)kE}, bias.data(), true));
  blk.set_max_tokens(256);
  blk.init_gpu();
  CHECK(moe_plan_tile_rows(blk.context(), 8) == 0 && moe_plan_tile_rows(blk.context(), 10) == 0 &&
        moe_plan_tile_rows(blk.context(), 11) == 64 && moe_plan_tile_rows(blk.context(), 64) == 64);
  for (int T : {8, 20, 48, 64, 200}) {
    std::vector<float> x((size_t)T * H), yref((size_t)T * H);
    moe_synth_normal(3, 99, 1.0f, 0, x.data(), x.size());
    std::vector<int> iref((size_t)T * 4), cref(kE);
    CHECK(orc_moe_forward(x.data(), gate.data(), bias.data(), w1.data(), w3.data(), w2.data(),
                          nullptr, T, H, I, kE, nullptr, yref.data(), nullptr, iref.data(),
                          nullptr, cref.data()) == 0);
    Tensor tx({(size_t)T, (size_t)H}, x.data(), true), ty, tl;
    blk.forward(tx, ty, tl);
    std::vector<int> idx((size_t)T * 4), cnt(kE);
    CHECK(moe_last_routing(blk.context(), idx.data(), nullptr, cnt.data(), nullptr, T, nullptr) == 0);
    CHECK(idx == iref && cnt == cref);
    int bad = 0;
    for (size_t i = 0; i < yref.size(); ++i) bad += !close(ty.data()[i], yref[i]);
    CHECK(bad == 0);
    std::printf("gpu full-shape T=%d plan=%d ok\n", T, moe_plan_tile_rows(blk.context(), T));
  }
}

// The model through the reference's own entry points: LFM2Model::forward
// (sample_idx, batch, host ids, seq_len, host logits) + sync() equals the
// device-pointer forward bit for bit; DecoderLayer::forward on host tensors
// equals forward_gpu.
void gpu_model_tests() {
  LFM2Config cfg;
  cfg.num_layers = 2;
  cfg.layer_types = {1, 0};
  cfg.num_dense_layers = 1;  // one dense FFN, one MoE block
  cfg.max_batch = 2;
  cfg.max_seq = 40;
  SyntheticWeights s;
  s.seed = 5;
  LFM2Model model(cfg, s);
  const int B = 2, S = 40, V = model.vocab();
  std::vector<int> ids((size_t)B * S);
  for (size_t i = 0; i < ids.size(); ++i) ids[i] = (int)((i * 2654435761u) % (unsigned)V);
  std::vector<float> logits((size_t)B * V);
  model.forward(0, B, ids.data(), S, logits.data());
  model.sync();
  int *dids = nullptr;
  float *dlog = nullptr;
  CHECK(hipMalloc(&dids, ids.size() * 4) == hipSuccess && hipMalloc(&dlog, logits.size() * 4) == hipSuccess);
  CHECK(hipMemcpy(dids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice) == hipSuccess);
  model.forward_gpu(dids, B, S, dlog, nullptr);
  std::vector<float> l2(logits.size());
  CHECK(hipDeviceSynchronize() == hipSuccess);
  CHECK(hipMemcpy(l2.data(), dlog, l2.size() * 4, hipMemcpyDeviceToHost) == hipSuccess);
  CHECK(std::memcmp(l2.data(), logits.data(), l2.size() * 4) == 0);
  bool finite = true;
  for (float v : logits) finite = finite && std::isfinite(v);
  CHECK(finite);
  CHECK(model.status(nullptr) == MOE_OK);
  CHECK(throws([&] { model.forward(0, 3, ids.data(), S, logits.data()); }));  // beyond max_batch
  // DecoderLayer on host tensors vs on device buffers (attention layer 1)
  DecoderLayer &layer = model.layer(1);
  const size_t n = (size_t)S * HIDDEN_SIZE;
  std::vector<float> h(n);
  moe_synth_normal(5, 7, 1.0f, 0, h.data(), n);
  RotaryEmbedding rope((size_t)S);
  Tensor c, sn;
  rope.forward(S, c, sn);
  Tensor th({(size_t)S, HIDDEN_SIZE}, h.data(), true), tout;
  layer.forward(th, c, sn, nullptr, tout);
  rope.init_gpu();
  float *dh = nullptr;
  CHECK(hipMalloc(&dh, n * 4) == hipSuccess);
  CHECK(hipMemcpy(dh, h.data(), n * 4, hipMemcpyHostToDevice) == hipSuccess);
  layer.forward_gpu(dh, rope.cos_gpu_, rope.sin_gpu_, dh, 1, S, (int)HIDDEN_SIZE, nullptr);
  std::vector<float> hd(n);
  CHECK(hipDeviceSynchronize() == hipSuccess);
  CHECK(hipMemcpy(hd.data(), dh, n * 4, hipMemcpyDeviceToHost) == hipSuccess);
  CHECK(std::memcmp(hd.data(), tout.data(), n * 4) == 0);
  (void)hipFree(dids);
  (void)hipFree(dlog);
  (void)hipFree(dh);
  std::printf("gpu model ok\n");
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  try {
    if (mode == "cpu") cpu_tests();
    else if (mode == "gpu") {
      gpu_tests();
      gpu_full_shape_tests();
      gpu_model_tests();
    }
    else {
      std::fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
      return 2;
    }
  } catch (const std::exception &e) {
    std::fprintf(stderr, "FAIL exception: %s\n", e.what());
    return 1;
  }
  std::printf("%s: %d checks, %d failed\n", mode.c_str(), g_checks, g_failed);
  return g_failed ? 1 : 0;
}
