// Host fp32 tensor: the container weights and activations cross the C++
// boundary in.  Public interface of reference include/tensor.h:22-89 (same
// constructors, accessors and file format); errors throw instead of exiting.
#pragma once

#include <cstddef>
#include <memory>
#include <string>
#include <vector>

class ModelLoader;

class Tensor {
public:
  Tensor();
  Tensor(const std::vector<size_t> &shape);
  Tensor(const std::vector<size_t> &shape, float *data, bool copy = true);
  ~Tensor();

  Tensor(const Tensor &other);
  Tensor &operator=(const Tensor &other);
  Tensor(Tensor &&other) noexcept;
  Tensor &operator=(Tensor &&other) noexcept;

  size_t ndim() const { return shape_.size(); }
  const std::vector<size_t> &shape() const { return shape_; }
  size_t size() const { return size_; }
  size_t size(int dim) const;

  float *data() { return data_; }
  const float *data() const { return data_; }
  float &operator[](size_t idx) { return data_[idx]; }
  const float &operator[](size_t idx) const { return data_[idx]; }

  float &at(size_t i);
  float &at(size_t i, size_t j);
  float &at(size_t i, size_t j, size_t k);
  float &at(size_t i, size_t j, size_t k, size_t l);
  const float &at(size_t i) const;
  const float &at(size_t i, size_t j) const;
  const float &at(size_t i, size_t j, size_t k) const;
  const float &at(size_t i, size_t j, size_t k, size_t l) const;

  void reshape(const std::vector<size_t> &new_shape);
  Tensor view(const std::vector<size_t> &new_shape) const;

  // By tensor name through `loader` or the global g_model_loader, else from a
  // standalone file: u32 ndim, u32 dims[ndim], fp32 data (tensor.cu:175-216).
  static Tensor load_from_file(const std::string &filename,
                               ModelLoader *loader = nullptr);
  void save_to_file(const std::string &filename) const;

  Tensor transpose(int dim0, int dim1) const;  // 2-D only
  Tensor slice(int dim, size_t start, size_t end) const;
  Tensor copy() const;

  void fill(float value);
  void zero();
  void ones();

private:
  std::vector<size_t> shape_;
  size_t size_ = 0;
  float *data_ = nullptr;
  bool owns_data_ = false;

  void allocate();
  void deallocate();
  size_t compute_size() const;
  size_t compute_stride(int dim) const;
};
