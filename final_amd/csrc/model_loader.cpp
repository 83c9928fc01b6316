// model.bin reader (include/model_loader.h); format of reference
// src/model_loader.cpp:22-68, lookup of :70-90.
#include "model_loader.h"

#include <cstring>
#include <stdexcept>

std::unique_ptr<ModelLoader> g_model_loader;

namespace {

template <typename T> T read_pod(std::ifstream &f, const std::string &what) {
  T v{};
  f.read(reinterpret_cast<char *>(&v), sizeof(T));
  if (!f) throw std::runtime_error("model file truncated reading " + what);
  return v;
}

}  // namespace

ModelLoader::ModelLoader(const std::string &model_file) : model_file_(model_file) {
  file_.open(model_file, std::ios::binary);
  if (!file_.is_open()) throw std::runtime_error("Cannot open model file: " + model_file);
  file_.seekg(0, std::ios::end);
  file_bytes_ = (uint64_t)file_.tellg();
  file_.seekg(0, std::ios::beg);
  load_index();
}

ModelLoader::~ModelLoader() {
  if (file_.is_open()) file_.close();
}

void ModelLoader::load_index() {
  char magic[4];
  file_.read(magic, 4);
  if (!file_ || std::memcmp(magic, "LFM2", 4) != 0)
    throw std::runtime_error("Invalid model file format: " + model_file_);
  (void)read_pod<uint32_t>(file_, "version");
  const uint32_t n = read_pod<uint32_t>(file_, "tensor count");
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t len = read_pod<uint32_t>(file_, "name length");
    if (len > (1u << 16)) throw std::runtime_error("model file: name too long");
    TensorInfo info;
    info.name.resize(len);
    file_.read(&info.name[0], len);
    if (!file_) throw std::runtime_error("model file truncated reading a name");
    const uint32_t nd = read_pod<uint32_t>(file_, "ndim");
    if (nd > 8) throw std::runtime_error("model file: bad ndim for " + info.name);
    info.shape.resize(nd);
    info.size = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      info.shape[d] = read_pod<uint32_t>(file_, "dim");
      info.size *= info.shape[d];
    }
    info.offset = read_pod<uint64_t>(file_, "offset");
    if (info.offset + info.size * sizeof(float) > file_bytes_)
      throw std::runtime_error("model file: data of " + info.name + " past end of file");
    index_[info.name] = info;
  }
}

bool ModelLoader::has_tensor(const std::string &name) const {
  return index_.find(name) != index_.end();
}

std::vector<size_t> ModelLoader::get_shape(const std::string &name) const {
  auto it = index_.find(name);
  if (it == index_.end()) throw std::runtime_error("Tensor not found: " + name);
  return it->second.shape;
}

Tensor ModelLoader::load_tensor(const std::string &name) {
  auto it = index_.find(name);
  if (it == index_.end()) throw std::runtime_error("Tensor not found: " + name);
  const TensorInfo &info = it->second;
  Tensor t(info.shape);
  std::lock_guard<std::mutex> lock(mu_);
  file_.clear();
  file_.seekg((std::streamoff)info.offset);
  file_.read(reinterpret_cast<char *>(t.data()), (std::streamsize)(info.size * sizeof(float)));
  if (!file_) throw std::runtime_error("model file read failed for " + name);
  return t;
}
