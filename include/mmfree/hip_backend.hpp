// mmfree/hip_backend.hpp -- TernaryBackend on the MI355X.
//
// HipTernaryBackend keeps each projection resident on the GPU (2-bit packed, repacked once
// from the int8 blob layout) and computes the integer accumulation with the gfx950 kernels
// behind mmf_ternary_matmul. Projections are registered up front (register_projection ->
// proj_id, the FPGA backend's resident-weight contract: a call with that proj_id uses the
// resident weights) or on first use with proj_id == -1 (the reference passes -1 for
// unregistered tags, hgrn_model.cpp:45-52). A -1 call uses the weights at wq now: the
// resident copy is keyed by the wq pointer, the shape and a hash of the contents, and is
// re-uploaded in place when the buffer holds other weights. Not reentrant: one backend, one
// thread (like the reference Model).
#pragma once

#include "mmfree/ternary_backend.hpp"

#include <cstddef>
#include <cstdint>
#include <map>
#include <tuple>
#include <vector>

struct mmf_ctx;

namespace mmfree {

class HipTernaryBackend final : public TernaryBackend {
 public:
  explicit HipTernaryBackend(int device = 0, std::size_t batch = 64);
  ~HipTernaryBackend() override;
  HipTernaryBackend(const HipTernaryBackend&) = delete;
  HipTernaryBackend& operator=(const HipTernaryBackend&) = delete;

  // Upload wq [M, N] (int8, row-major); returns the proj_id for matmul calls.
  int register_projection(const std::int8_t* wq, std::size_t N, std::size_t M);

  void matmul(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq, std::size_t N,
              std::size_t M) override;
  std::size_t batch_size() const override { return batch_; }
  void matmul_batch(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                    std::size_t N, std::size_t M, std::size_t b) override;

 private:
  int resolve(int proj_id, const std::int8_t* wq, std::size_t N, std::size_t M);
  void ensure(std::size_t xbytes, std::size_t accbytes);
  mmf_ctx* ctx_ = nullptr;
  std::size_t batch_;
  struct Resident {
    int id;
    std::uint64_t hash;  // of the weights last uploaded from this buffer
  };
  std::map<std::tuple<const std::int8_t*, std::size_t, std::size_t>, Resident> by_ptr_;
  void* dx_ = nullptr;
  void* dacc_ = nullptr;
  std::size_t cap_x_ = 0, cap_acc_ = 0;
};

}  // namespace mmfree
