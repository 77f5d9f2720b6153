// mmfree/model.hpp -- HGRN-Bit / MMfreeLM inference on one MI355X.
//
// Same public API and callback semantics as the reference Model
// (cpp/include/mmfree/model.hpp:27-120): the constructor takes the mmap'd Weights and the
// activation mode, forward() returns all logits, generate() decodes greedily or samples
// (temperature / top-k with std::mt19937_64 seeded by Sampling::seed, the reference's
// sampling steps), generate_serve() decodes B streams in lockstep with staggered first-token
// callbacks. All model compute runs on the GPU through the mmfree_hip.h C ABI; results are
// bit-identical to the reference engine's (Float and FixedQ510). The constructor uploads the
// weights (2-bit repack on the device) and throws std::runtime_error if no gfx950 device is
// available -- there is no CPU path.
#pragma once

#include "mmfree/config.hpp"
#include "mmfree/kernels.hpp"
#include "mmfree/weights.hpp"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>
#include <unordered_map>
#include <vector>

struct mmf_ctx;

namespace mmfree {

struct TernaryBackend;

struct Sampling {
  float temperature = 0.0f;  // <= 0: greedy argmax
  int top_k = 0;             // <= 0: full vocabulary
  std::uint64_t seed = 0;
};

class Model {
 public:
  explicit Model(const Weights& w, ActQuant aq = ActQuant::Float, int frac_bits = 10);
  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  void forward(const std::int64_t* ids, std::size_t T, std::vector<float>& logits);

  std::vector<std::int64_t> generate(const std::vector<std::int64_t>& ids, std::size_t new_tokens,
                                     std::int64_t eos_id = -1, const Sampling& samp = {},
                                     const std::function<void(std::int64_t)>& on_token = {});

  std::vector<std::vector<std::int64_t>> generate_serve(
      const std::vector<std::vector<std::int64_t>>& prompts, std::size_t new_tokens, std::int64_t eos_id = -1,
      const Sampling& samp = {}, const std::function<void(std::size_t, std::int64_t)>& on_token = {});

  const Config& config() const { return cfg_; }

  // The reference's backend injection (model.hpp:74-79, hgrn_model.cpp:40-78). The backend is
  // borrowed and must outlive the Model, as must the Weights. nullptr (the default) and a
  // HipTernaryBackend keep the projections on this engine's GPU kernels. Any other backend
  // receives the integer matmul of every FixedQ510 projection (tags
  // model.layers.{l}.{i,f,g,o,gate,down}_proj and lm_head; proj_ids maps a tag to the
  // backend's proj_id, -1 when absent): the GPU computes the RMSNorm and Q5.10 codes, the
  // backend the accumulators (batch_size() rows per call; the i/f/g cluster through
  // matmul_seq), the GPU dequantises and goes on. Float mode never uses the backend.
  void set_backend(TernaryBackend* be, std::unordered_map<std::string, int> proj_ids);

  // Recurrent state [num_hidden_layers][streams][hidden_size] after the last call.
  std::vector<float> state() const;
  // The underlying C ABI context (for timing and device-pointer use).
  mmf_ctx* context() const { return ctx_; }

 private:
  // the external integer matmul (mmf_model_set_matmul) that forwards to backend_
  static int backend_matmul(void* self, int layer, int proj, int k, const std::int32_t* codes, std::int32_t* acc,
                            std::size_t K, std::size_t N, std::size_t rows);
  void run_backend(int layer, int proj, int k, const std::int32_t* codes, std::int32_t* acc, std::size_t K,
                   std::size_t N, std::size_t rows);
  void check_call(int rc, const char* what);

  mmf_ctx* ctx_ = nullptr;
  const Weights& w_;
  Config cfg_;
  ActQuant aq_;
  int frac_bits_;
  std::size_t streams_ = 1;
  TernaryBackend* backend_ = nullptr;
  std::unordered_map<std::string, int> proj_ids_;
  std::string backend_error_;
};

}  // namespace mmfree
