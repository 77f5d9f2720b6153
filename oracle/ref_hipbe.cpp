// ref_hipbe.cpp -- attaches the MI355X TernaryBackend (mmfree::HipTernaryBackend, compiled
// here against the reference's own ternary_backend.hpp) to a reference Model through the
// reference's plugin seam, Model::set_backend (model.hpp:74-79). Test infrastructure: the
// parity test runs the reference engine's FixedQ510 generation with its integer projections
// on the GPU and requires the same ids and state as the reference's CPU run; bench.py times it.
#include <exception>
#include <memory>
#include <string>
#include <unordered_map>

#include "mmfree/hip_backend.hpp"
#include "mmfree/model.hpp"
#include "mmfree/weights.hpp"

extern "C" {

// Empty registry: every projection reaches the backend with proj_id -1 (the weights at wq).
void* ref_hipbe_attach(void* model, int device) {
  try {
    auto* be = new mmfree::HipTernaryBackend(device);
    static_cast<mmfree::Model*>(model)->set_backend(be, {});
    return be;
  } catch (const std::exception&) {
    return nullptr;
  }
}

// Every projection registered up front; the registry maps each tag to its resident proj_id
// (the deployment the seam's registry is for: model.hpp:74-79).
void* ref_hipbe_attach_registered(void* model, void* weights, int device) {
  std::unique_ptr<mmfree::HipTernaryBackend> be;
  try {
    be = std::make_unique<mmfree::HipTernaryBackend>(device);
    auto reg = be->register_model(*static_cast<const mmfree::Weights*>(weights));
    static_cast<mmfree::Model*>(model)->set_backend(be.get(), std::move(reg));
    return be.release();
  } catch (const std::exception&) {
    return nullptr;
  }
}

void ref_hipbe_detach(void* model, void* be) {
  static_cast<mmfree::Model*>(model)->set_backend(nullptr, {});
  delete static_cast<mmfree::HipTernaryBackend*>(be);
}

}  // extern "C"
