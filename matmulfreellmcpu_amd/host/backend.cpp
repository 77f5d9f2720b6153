// backend.cpp -- HipTernaryBackend: the TernaryBackend seam on the MI355X.
#include "mmfree/hip_backend.hpp"

#include <stdexcept>
#include <string>

#include "content_hash.hpp"
#include "mmfree_hip.h"

namespace mmfree {
namespace {
void check(mmf_ctx* c, int rc, const char* what) {
  if (rc != MMF_OK) throw std::runtime_error(std::string(what) + ": " + mmf_last_error(c));
}
}  // namespace

HipTernaryBackend::HipTernaryBackend(int device, std::size_t batch) : batch_(batch ? batch : 1) {
  if (mmf_create(&ctx_, device) != MMF_OK) throw std::runtime_error(std::string("mmfree: ") + mmf_last_error(nullptr));
}

HipTernaryBackend::~HipTernaryBackend() {
  if (dx_) mmf_free(ctx_, dx_);
  if (dacc_) mmf_free(ctx_, dacc_);
  mmf_destroy(ctx_);
}

int HipTernaryBackend::register_projection(const std::int8_t* wq, std::size_t N, std::size_t M) {
  int id = -1;
  // the seam's wq is [M outputs, N inputs]; the C ABI names them (N, K)
  check(ctx_, mmf_proj_register(ctx_, wq, M, N, 1.0f, nullptr, &id), "mmf_proj_register");
  by_ptr_[{wq, N, M}] = Resident{id, detail::content_hash(wq, N * M)};
  return id;
}

int HipTernaryBackend::resolve(int proj_id, const std::int8_t* wq, std::size_t N, std::size_t M) {
  if (proj_id >= 0) {
    std::size_t n = 0, k = 0;
    check(ctx_, mmf_proj_shape(ctx_, proj_id, &n, &k), "mmf_proj_shape");
    if (n != M || k != N) throw std::runtime_error("HipTernaryBackend: proj_id shape differs from the call");
    return proj_id;
  }
  auto it = by_ptr_.find({wq, N, M});
  if (it == by_ptr_.end()) return register_projection(wq, N, M);
  // the weights at wq now: a buffer refilled with other weights (or another blob mapped at the
  // same address) replaces the resident copy in place
  const std::uint64_t h = detail::content_hash(wq, N * M);
  if (h != it->second.hash) {
    check(ctx_, mmf_proj_update(ctx_, it->second.id, wq), "mmf_proj_update");
    it->second.hash = h;
  }
  return it->second.id;
}

void HipTernaryBackend::ensure(std::size_t xbytes, std::size_t accbytes) {
  if (xbytes > cap_x_) {
    if (dx_) mmf_free(ctx_, dx_);
    dx_ = nullptr;
    check(ctx_, mmf_malloc(ctx_, &dx_, xbytes), "mmf_malloc");
    cap_x_ = xbytes;
  }
  if (accbytes > cap_acc_) {
    if (dacc_) mmf_free(ctx_, dacc_);
    dacc_ = nullptr;
    check(ctx_, mmf_malloc(ctx_, &dacc_, accbytes), "mmf_malloc");
    cap_acc_ = accbytes;
  }
}

void HipTernaryBackend::matmul(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                               std::size_t N, std::size_t M) {
  matmul_batch(proj_id, x, acc, wq, N, M, 1);
}

void HipTernaryBackend::matmul_batch(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                                     std::size_t N, std::size_t M, std::size_t b) {
  if (b == 0) return;
  const int id = resolve(proj_id, wq, N, M);
  ensure(b * N * sizeof(std::int32_t), b * M * sizeof(std::int32_t));
  check(ctx_, mmf_upload(ctx_, dx_, x, b * N * sizeof(std::int32_t)), "mmf_upload");
  check(ctx_, mmf_ternary_matmul(ctx_, id, static_cast<const std::int32_t*>(dx_), static_cast<std::int32_t*>(dacc_), b),
        "mmf_ternary_matmul");
  check(ctx_, mmf_download(ctx_, acc, dacc_, b * M * sizeof(std::int32_t)), "mmf_download");
}

}  // namespace mmfree
