// ref_hipbe.cpp -- attaches the MI355X TernaryBackend (mmfree::HipTernaryBackend, compiled
// here against the reference's own ternary_backend.hpp) to a reference Model through the
// reference's plugin seam, Model::set_backend (model.hpp:74-79). Test infrastructure: the
// parity test runs the reference engine's FixedQ510 generation with its integer projections
// on the GPU and requires the same ids and state as the reference's CPU run.
#include <memory>
#include <string>
#include <unordered_map>

#include "mmfree/hip_backend.hpp"
#include "mmfree/model.hpp"

extern "C" {

void* ref_hipbe_attach(void* model, int device) {
  auto* be = new mmfree::HipTernaryBackend(device);
  static_cast<mmfree::Model*>(model)->set_backend(be, {});
  return be;
}

void ref_hipbe_detach(void* model, void* be) {
  static_cast<mmfree::Model*>(model)->set_backend(nullptr, {});
  delete static_cast<mmfree::HipTernaryBackend*>(be);
}

}  // extern "C"
