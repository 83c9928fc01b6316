// Single-file weight store ("model.bin") the layers load their tensors from by
// name.  Format of reference src/model_loader.cpp:22-68: "LFM2", u32 version,
// u32 count, then per tensor u32 name_len, name, u32 ndim, u32 dims[ndim],
// u64 byte offset of the fp32 data.  (The reference's header and source
// disagree on member names and do not compile together; this class keeps the
// header's public interface, include/model_loader.h:10-21.)
#pragma once

#include <cstdint>
#include <fstream>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "tensor.h"

class ModelLoader {
public:
  explicit ModelLoader(const std::string &model_file);
  ~ModelLoader();

  Tensor load_tensor(const std::string &name);
  bool has_tensor(const std::string &name) const;
  std::vector<size_t> get_shape(const std::string &name) const;
  size_t num_tensors() const { return index_.size(); }

private:
  struct TensorInfo {
    std::string name;
    std::vector<size_t> shape;
    uint64_t offset = 0;
    uint64_t size = 0;  // elements
  };

  std::string model_file_;
  std::ifstream file_;
  uint64_t file_bytes_ = 0;
  std::unordered_map<std::string, TensorInfo> index_;
  std::mutex mu_;

  void load_index();
};

// Global loader the name-based constructors read through (reference
// include/model.h:21, defined in model.cu:16).
extern std::unique_ptr<ModelLoader> g_model_loader;
