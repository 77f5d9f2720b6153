// backend.cpp -- HipTernaryBackend: the TernaryBackend seam on the MI355X.
#include "mmfree/hip_backend.hpp"

#include <cstring>
#include <stdexcept>
#include <string>

#include "mmfree_hip.h"

namespace mmfree {
namespace {
void check(mmf_ctx* c, int rc, const char* what) {
  if (rc != MMF_OK) throw std::runtime_error(std::string(what) + ": " + mmf_last_error(c));
}
constexpr int kMaxSeq = 64;  // projections per mmf_ternary_matmul_host call
}  // namespace

HipTernaryBackend::HipTernaryBackend(int device, std::size_t batch) : batch_(batch ? batch : 1) {
  if (mmf_create(&ctx_, device) != MMF_OK) throw std::runtime_error(std::string("mmfree: ") + mmf_last_error(nullptr));
}

HipTernaryBackend::~HipTernaryBackend() { mmf_destroy(ctx_); }

int HipTernaryBackend::register_projection(const std::int8_t* wq, std::size_t N, std::size_t M) {
  int id = -1;
  // the seam's wq is [M outputs, N inputs]; the C ABI names them (N, K)
  check(ctx_, mmf_proj_register(ctx_, wq, M, N, 1.0f, nullptr, &id), "mmf_proj_register");
  return id;
}

std::unordered_map<std::string, int> HipTernaryBackend::register_model(const Weights& w) {
  std::unordered_map<std::string, int> reg;
  auto add = [&](const std::string& tag) {
    const TensorRef& t = w.get(tag + ".wq");
    if (t.shape.size() != 2 || !t.is_int8) throw std::runtime_error("HipTernaryBackend: " + tag + ".wq is not int8 [out, in]");
    reg[tag] = register_projection(t.i8(), t.shape[1], t.shape[0]);
  };
  static const char* names[6] = {"i_proj", "f_proj", "g_proj", "o_proj", "gate_proj", "down_proj"};
  for (std::size_t l = 0; l < w.config().num_hidden_layers; ++l)
    for (const char* n : names) add("model.layers." + std::to_string(l) + "." + n);
  add("lm_head");
  return reg;
}

int HipTernaryBackend::resolve(int proj_id, const std::int8_t* wq, std::size_t N, std::size_t M) {
  if (proj_id >= 0) {
    std::size_t n = 0, k = 0;
    check(ctx_, mmf_proj_shape(ctx_, proj_id, &n, &k), "mmf_proj_shape");
    if (n != M || k != N) throw std::runtime_error("HipTernaryBackend: proj_id shape differs from the call");
    return proj_id;
  }
  const std::size_t bytes = N * M;
  auto it = by_ptr_.find({wq, N, M});
  if (it == by_ptr_.end()) {
    const int id = register_projection(wq, N, M);
    by_ptr_.emplace(std::make_tuple(wq, N, M), Resident{id, std::vector<std::int8_t>(wq, wq + bytes)});
    return id;
  }
  // the weights at wq now, compared exactly with what was uploaded: a buffer refilled with
  // other weights (or another blob mapped at the same address) replaces the resident copy
  Resident& r = it->second;
  if (std::memcmp(r.host.data(), wq, bytes) != 0) {
    check(ctx_, mmf_proj_update(ctx_, r.id, wq), "mmf_proj_update");
    std::memcpy(r.host.data(), wq, bytes);
  }
  return r.id;
}

void HipTernaryBackend::matmul(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                               std::size_t N, std::size_t M) {
  matmul_batch(proj_id, x, acc, wq, N, M, 1);
}

void HipTernaryBackend::matmul_batch(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                                     std::size_t N, std::size_t M, std::size_t b) {
  if (b == 0) return;
  const int id = resolve(proj_id, wq, N, M);
  check(ctx_, mmf_ternary_matmul_host(ctx_, 1, &id, &x, &acc, b), "mmf_ternary_matmul_host");
}

void HipTernaryBackend::matmul_seq(const int* proj_ids, const std::int8_t* const* wqs, int k,
                                   const std::function<void(int, std::int32_t*)>& produce,
                                   const std::function<void(int, const std::int32_t*)>& consume, std::size_t N,
                                   std::size_t M, std::size_t b) {
  if (k <= 0) return;
  if (k > kMaxSeq || b == 0) {
    TernaryBackend::matmul_seq(proj_ids, wqs, k, produce, consume, N, M, b);
    return;
  }
  seq_x_.resize(static_cast<std::size_t>(k) * b * N);
  seq_acc_.resize(static_cast<std::size_t>(k) * b * M);
  int ids[kMaxSeq];
  const std::int32_t* xs[kMaxSeq];
  std::int32_t* accs[kMaxSeq];
  for (int j = 0; j < k; ++j) {
    std::int32_t* xj = seq_x_.data() + static_cast<std::size_t>(j) * b * N;
    produce(j, xj);
    ids[j] = resolve(proj_ids ? proj_ids[j] : -1, wqs[j], N, M);
    xs[j] = xj;
    accs[j] = seq_acc_.data() + static_cast<std::size_t>(j) * b * M;
  }
  check(ctx_, mmf_ternary_matmul_host(ctx_, k, ids, xs, accs, b), "mmf_ternary_matmul_host");
  for (int j = 0; j < k; ++j) consume(j, accs[j]);
}

}  // namespace mmfree
