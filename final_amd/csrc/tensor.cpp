// Host tensor (include/tensor.h).  Behaviour of reference src/tensor.cu:17-255.
#include "tensor.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <functional>
#include <numeric>
#include <stdexcept>

#include "model_loader.h"

Tensor::Tensor() = default;

Tensor::Tensor(const std::vector<size_t> &shape) : shape_(shape), owns_data_(true) {
  size_ = compute_size();
  allocate();
}

Tensor::Tensor(const std::vector<size_t> &shape, float *data, bool copy)
    : shape_(shape), owns_data_(copy) {
  size_ = compute_size();
  if (copy) {
    allocate();
    if (size_) std::memcpy(data_, data, size_ * sizeof(float));
  } else {
    data_ = data;
  }
}

Tensor::~Tensor() { deallocate(); }

Tensor::Tensor(const Tensor &other)
    : shape_(other.shape_), size_(other.size_), owns_data_(true) {
  allocate();
  if (size_) std::memcpy(data_, other.data_, size_ * sizeof(float));
}

Tensor &Tensor::operator=(const Tensor &other) {
  if (this != &other) {
    deallocate();
    shape_ = other.shape_;
    size_ = other.size_;
    owns_data_ = true;
    allocate();
    if (size_) std::memcpy(data_, other.data_, size_ * sizeof(float));
  }
  return *this;
}

Tensor::Tensor(Tensor &&other) noexcept
    : shape_(std::move(other.shape_)), size_(other.size_), data_(other.data_),
      owns_data_(other.owns_data_) {
  other.data_ = nullptr;
  other.size_ = 0;
  other.owns_data_ = false;
}

Tensor &Tensor::operator=(Tensor &&other) noexcept {
  if (this != &other) {
    deallocate();
    shape_ = std::move(other.shape_);
    size_ = other.size_;
    data_ = other.data_;
    owns_data_ = other.owns_data_;
    other.data_ = nullptr;
    other.size_ = 0;
    other.owns_data_ = false;
  }
  return *this;
}

void Tensor::allocate() {
  data_ = size_ ? new float[size_] : nullptr;
}

void Tensor::deallocate() {
  if (owns_data_) delete[] data_;
  data_ = nullptr;
}

size_t Tensor::compute_size() const {
  if (shape_.empty()) return 0;
  return std::accumulate(shape_.begin(), shape_.end(), (size_t)1,
                         std::multiplies<size_t>());
}

size_t Tensor::compute_stride(int dim) const {
  size_t s = 1;
  for (size_t i = (size_t)dim + 1; i < shape_.size(); ++i) s *= shape_[i];
  return s;
}

size_t Tensor::size(int dim) const {
  if (dim < 0) dim += (int)shape_.size();
  if (dim < 0 || (size_t)dim >= shape_.size())
    throw std::out_of_range("Tensor::size: dimension out of range");
  return shape_[dim];
}

float &Tensor::at(size_t i) { return data_[i]; }
float &Tensor::at(size_t i, size_t j) { return data_[i * shape_[1] + j]; }
float &Tensor::at(size_t i, size_t j, size_t k) {
  return data_[(i * shape_[1] + j) * shape_[2] + k];
}
float &Tensor::at(size_t i, size_t j, size_t k, size_t l) {
  return data_[((i * shape_[1] + j) * shape_[2] + k) * shape_[3] + l];
}
const float &Tensor::at(size_t i) const { return data_[i]; }
const float &Tensor::at(size_t i, size_t j) const { return data_[i * shape_[1] + j]; }
const float &Tensor::at(size_t i, size_t j, size_t k) const {
  return data_[(i * shape_[1] + j) * shape_[2] + k];
}
const float &Tensor::at(size_t i, size_t j, size_t k, size_t l) const {
  return data_[((i * shape_[1] + j) * shape_[2] + k) * shape_[3] + l];
}

void Tensor::reshape(const std::vector<size_t> &new_shape) {
  const size_t n = std::accumulate(new_shape.begin(), new_shape.end(), (size_t)1,
                                   std::multiplies<size_t>());
  if (n != size_) throw std::invalid_argument("Tensor::reshape: size mismatch");
  shape_ = new_shape;
}

Tensor Tensor::view(const std::vector<size_t> &new_shape) const {
  const size_t n = std::accumulate(new_shape.begin(), new_shape.end(), (size_t)1,
                                   std::multiplies<size_t>());
  if (n != size_) throw std::invalid_argument("Tensor::view: size mismatch");
  return Tensor(new_shape, data_, false);
}

Tensor Tensor::load_from_file(const std::string &filename, ModelLoader *loader) {
  if (loader) return loader->load_tensor(filename);
  if (g_model_loader) return g_model_loader->load_tensor(filename);
  std::ifstream f(filename, std::ios::binary);
  if (!f) throw std::runtime_error("Cannot open file: " + filename);
  uint32_t nd = 0;
  f.read(reinterpret_cast<char *>(&nd), sizeof(nd));
  if (!f || nd > 8) throw std::runtime_error("Bad tensor header: " + filename);
  std::vector<size_t> shape(nd);
  for (uint32_t i = 0; i < nd; ++i) {
    uint32_t d = 0;
    f.read(reinterpret_cast<char *>(&d), sizeof(d));
    shape[i] = d;
  }
  Tensor t(shape);
  f.read(reinterpret_cast<char *>(t.data()), (std::streamsize)(t.size() * sizeof(float)));
  if (!f) throw std::runtime_error("Truncated tensor file: " + filename);
  return t;
}

void Tensor::save_to_file(const std::string &filename) const {
  std::ofstream f(filename, std::ios::binary);
  if (!f) throw std::runtime_error("Cannot open file: " + filename);
  const uint32_t nd = (uint32_t)shape_.size();
  f.write(reinterpret_cast<const char *>(&nd), sizeof(nd));
  for (size_t d : shape_) {
    const uint32_t d32 = (uint32_t)d;
    f.write(reinterpret_cast<const char *>(&d32), sizeof(d32));
  }
  f.write(reinterpret_cast<const char *>(data_), (std::streamsize)(size_ * sizeof(float)));
  if (!f) throw std::runtime_error("Write failed: " + filename);
}

Tensor Tensor::transpose(int dim0, int dim1) const {
  if (shape_.size() != 2 || !((dim0 == 0 && dim1 == 1) || (dim0 == 1 && dim1 == 0)))
    throw std::invalid_argument("Tensor::transpose: 2-D (0,1) only");
  const size_t r = shape_[0], c = shape_[1];
  Tensor t({c, r});
  for (size_t i = 0; i < r; ++i)
    for (size_t j = 0; j < c; ++j) t.data_[j * r + i] = data_[i * c + j];
  return t;
}

Tensor Tensor::slice(int dim, size_t start, size_t end) const {
  if (dim < 0) dim += (int)shape_.size();
  if (dim < 0 || (size_t)dim >= shape_.size() || start > end || end > shape_[dim])
    throw std::out_of_range("Tensor::slice: bad range");
  std::vector<size_t> ns = shape_;
  ns[dim] = end - start;
  Tensor t(ns);
  const size_t inner = compute_stride(dim);
  size_t outer = 1;
  for (int i = 0; i < dim; ++i) outer *= shape_[i];
  for (size_t o = 0; o < outer; ++o)
    std::memcpy(t.data_ + o * (end - start) * inner,
                data_ + (o * shape_[dim] + start) * inner,
                (end - start) * inner * sizeof(float));
  return t;
}

Tensor Tensor::copy() const { return Tensor(shape_, data_, true); }

void Tensor::fill(float value) { std::fill(data_, data_ + size_, value); }
void Tensor::zero() { fill(0.0f); }
void Tensor::ones() { fill(1.0f); }
