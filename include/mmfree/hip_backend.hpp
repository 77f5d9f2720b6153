// mmfree/hip_backend.hpp -- TernaryBackend on the MI355X.
//
// HipTernaryBackend keeps each projection resident on the GPU (2-bit packed, repacked once
// from the int8 blob layout) and computes the integer accumulation with the gfx950 kernels
// behind mmf_ternary_matmul_host: one host round trip per call (codes in, accumulators out,
// one synchronisation), and one round trip for a whole matmul_seq cluster (i/f/g).
//
// Two ways to address the weights, as the seam defines them (ternary_backend.hpp:26-31,
// model.hpp:74-79):
//  * registered: register_projection -> proj_id, or register_model(weights), which registers
//    every ternary projection of a blob and returns the tag -> proj_id registry that
//    Model::set_backend takes. A call with proj_id >= 0 uses the resident weights and reads
//    nothing from wq (the FPGA backend's resident-weight contract). This is the fast path.
//  * proj_id == -1 (a tag absent from the registry, hgrn_model.cpp:45-52): the call uses the
//    weights at wq now. The resident copy is keyed by the wq pointer and shape; every such
//    call compares wq byte for byte with the host copy of what was uploaded (an exact check,
//    as much host memory traffic as reading the weights once) and re-uploads in place when the
//    buffer holds other weights.
// Not reentrant: one backend, one thread (like the reference Model).
#pragma once

#include "mmfree/ternary_backend.hpp"
#include "mmfree/weights.hpp"

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <tuple>
#include <unordered_map>
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
  // Register the ternary projections of a blob: model.layers.<l>.{i,f,g,o,gate,down}_proj and
  // lm_head (the tags Model::run_proj uses, hgrn_model.cpp:104-188,245). Returns the registry
  // for Model::set_backend(backend, registry).
  std::unordered_map<std::string, int> register_model(const Weights& w);

  void matmul(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq, std::size_t N,
              std::size_t M) override;
  std::size_t batch_size() const override { return batch_; }
  void matmul_batch(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                    std::size_t N, std::size_t M, std::size_t b) override;
  // All k produce() calls, one round trip for the k matmuls, then all k consume() calls: the
  // same accumulators as the serial default (integer sums), and each consume(j) follows its
  // own matmul (ternary_backend.hpp:67-90).
  void matmul_seq(const int* proj_ids, const std::int8_t* const* wqs, int k,
                  const std::function<void(int, std::int32_t*)>& produce,
                  const std::function<void(int, const std::int32_t*)>& consume, std::size_t N, std::size_t M,
                  std::size_t b) override;

 private:
  int resolve(int proj_id, const std::int8_t* wq, std::size_t N, std::size_t M);
  mmf_ctx* ctx_ = nullptr;
  std::size_t batch_;
  struct Resident {
    int id;
    std::vector<std::int8_t> host;  // the weights last uploaded from this buffer
  };
  std::map<std::tuple<const std::int8_t*, std::size_t, std::size_t>, Resident> by_ptr_;
  std::vector<std::int32_t> seq_x_, seq_acc_;  // matmul_seq staging
};

}  // namespace mmfree
