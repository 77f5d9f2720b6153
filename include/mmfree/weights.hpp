// mmfree/weights.hpp -- read-only view of a model.mmfree (MMFREE1) weight blob.
//
// Interface of the reference loader (cpp/include/mmfree/weights.hpp:21-59): the blob is
// mmap'd, TensorRef views point into the mapping, get() throws std::runtime_error for a
// missing tensor. Unlike the reference, the header and every tensor's offset and size are
// validated against the file before use.
#pragma once

#include "mmfree/config.hpp"

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace mmfree {

struct TensorRef {
  const void* data = nullptr;
  std::vector<std::size_t> shape;
  bool is_int8 = false;

  std::size_t numel() const {
    std::size_t n = 1;
    for (auto s : shape) n *= s;
    return shape.empty() ? 0 : n;
  }
  std::size_t rows() const { return shape.empty() ? 0 : shape.front(); }
  std::size_t cols() const { return shape.empty() ? 0 : shape.back(); }
  const float* f32() const { return static_cast<const float*>(data); }
  const int8_t* i8() const { return static_cast<const int8_t*>(data); }
};

class Weights {
 public:
  explicit Weights(const std::string& path);
  ~Weights();
  Weights(const Weights&) = delete;
  Weights& operator=(const Weights&) = delete;

  const Config& config() const { return cfg_; }
  bool has(const std::string& name) const { return tensors_.count(name) != 0; }
  const TensorRef& get(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("weights: missing tensor " + name);
    return it->second;
  }
  // Tensor names in blob order.
  const std::vector<std::string>& names() const { return order_; }

 private:
  Config cfg_;
  std::unordered_map<std::string, TensorRef> tensors_;
  std::vector<std::string> order_;
  void* base_ = nullptr;
  std::size_t size_ = 0;
  int fd_ = -1;
};

}  // namespace mmfree
