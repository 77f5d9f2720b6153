// kernels.cpp -- the reference's operator functions (kernels.hpp) on the MI355X.
//
// Host-pointer API: each call uploads its operands to the process's default context
// (device MMFREE_DEVICE or 0), runs the gfx950 kernels and downloads the result. Projection
// weights stay resident, one projection per (pointer, shape): each call compares the weights,
// scale and norm weight at that pointer exactly with the copy last uploaded; other weights are
// re-uploaded in place, another scale or norm weight replaces the projection (the old one is
// released), so device memory does not grow with refills.
// A FixedQ510 bitlinear with an external TernaryBackend follows the reference's split
// (bitlinear.cpp:39-94): the GPU computes the RMSNorm and the Q5.10 codes, the backend the
// integer accumulation (batch_size() rows per call, column ranges reported through on_cols),
// and each reported range is dequantised as (float)acc * (1 / (2^f * scale_w)).
#include "mmfree/kernels.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "mmfree/hip_backend.hpp"
#include "mmfree_hip.h"

namespace mmfree {
namespace {

void check(mmf_ctx* c, int rc, const char* what) {
  if (rc != MMF_OK) throw std::runtime_error(std::string(what) + ": " + mmf_last_error(c));
}

struct DevMem {
  mmf_ctx* c;
  void* p = nullptr;
  DevMem(mmf_ctx* ctx, std::size_t bytes, const void* host = nullptr) : c(ctx) {
    check(c, mmf_malloc(c, &p, bytes ? bytes : 1), "mmf_malloc");
    if (host && bytes) check(c, mmf_upload(c, p, host, bytes), "mmf_upload");
  }
  ~DevMem() { mmf_free(c, p); }
  template <class T> T* as() const { return static_cast<T*>(p); }
  void get(void* host, std::size_t bytes) const { check(c, mmf_download(c, host, p, bytes), "mmf_download"); }
};

struct Default {
  mmf_ctx* c = nullptr;
  std::mutex mu;
  struct Cached {
    int id;
    std::vector<std::int8_t> wq;  // what was uploaded
    float scale_w;
    std::vector<float> normw;
  };
  std::map<std::tuple<const void*, std::size_t, std::size_t>, Cached> projs;
  Default() {
    const char* e = std::getenv("MMFREE_DEVICE");
    if (mmf_create(&c, e ? std::atoi(e) : 0) != MMF_OK)
      throw std::runtime_error(std::string("mmfree: ") + mmf_last_error(nullptr));
  }
  ~Default() { mmf_destroy(c); }
  int proj(const int8_t* wq, std::size_t N, std::size_t K, float scale_w, const float* normw) {
    const auto key = std::make_tuple(static_cast<const void*>(wq), N, K);
    auto it = projs.find(key);
    if (it != projs.end()) {
      Cached& e = it->second;
      const bool same_norm = std::memcmp(&e.scale_w, &scale_w, sizeof scale_w) == 0 &&
                             std::memcmp(e.normw.data(), normw, K * sizeof(float)) == 0;
      if (same_norm) {
        if (std::memcmp(e.wq.data(), wq, N * K) != 0) {
          check(c, mmf_proj_update(c, e.id, wq), "mmf_proj_update");
          std::memcpy(e.wq.data(), wq, N * K);
        }
        return e.id;
      }
      check(c, mmf_proj_release(c, e.id), "mmf_proj_release");
      projs.erase(it);
    }
    int id = -1;
    check(c, mmf_proj_register(c, wq, N, K, scale_w, normw, &id), "mmf_proj_register");
    projs.emplace(key, Cached{id, std::vector<std::int8_t>(wq, wq + N * K), scale_w,
                              std::vector<float>(normw, normw + K)});
    return id;
  }
};

Default& dflt() {
  static Default d;
  return d;
}

int mode_of(ActQuant aq) {
  return aq == ActQuant::FixedQ510 ? MMF_FIXED_Q510 : aq == ActQuant::Int8Absmax ? MMF_INT8_ABSMAX : MMF_FLOAT;
}

bool foreign(TernaryBackend* be) { return be && !dynamic_cast<HipTernaryBackend*>(be); }

void norm_out_rows(Default& d, const DevMem& x, const float* w, float* norm_out, std::size_t rows, std::size_t K,
                   float eps) {
  DevMem dw(d.c, K * sizeof(float), w), dy(d.c, rows * K * sizeof(float));
  check(d.c, mmf_rmsnorm(d.c, dy.as<float>(), x.as<float>(), dw.as<float>(), rows, K, eps), "mmf_rmsnorm");
  dy.get(norm_out, rows * K * sizeof(float));
}

}  // namespace

void rmsnorm(float* y, const float* x, const float* weight, std::size_t rows, std::size_t cols, float eps) {
  if (!rows || !cols) return;
  Default& d = dflt();
  std::lock_guard<std::mutex> lk(d.mu);
  DevMem dx(d.c, rows * cols * 4, x), dw(d.c, cols * 4, weight), dy(d.c, rows * cols * 4);
  check(d.c, mmf_rmsnorm(d.c, dy.as<float>(), dx.as<float>(), dw.as<float>(), rows, cols, eps), "mmf_rmsnorm");
  dy.get(y, rows * cols * 4);
}

void bitlinear(float* out, const float* x, const float* norm_weight, const int8_t* wq, float scale_w, std::size_t rows,
               std::size_t in_dim, std::size_t out_dim, float eps, float* norm_out, ActQuant aq, int frac_bits,
               TernaryBackend* be, int proj_id) {
  if (!rows) return;
  Default& d = dflt();
  std::lock_guard<std::mutex> lk(d.mu);
  const std::size_t K = in_dim, N = out_dim;
  DevMem dx(d.c, rows * K * 4, x);
  if (norm_out) norm_out_rows(d, dx, norm_weight, norm_out, rows, K, eps);
  if (aq == ActQuant::FixedQ510 && foreign(be)) {
    DevMem dw(d.c, K * 4, norm_weight), dq(d.c, rows * K * 4);
    check(d.c, mmf_bitlinear_codes(d.c, dx.as<float>(), dw.as<float>(), dq.as<int32_t>(), rows, K, eps, frac_bits),
          "mmf_bitlinear_codes");
    std::vector<int32_t> q(rows * K);
    dq.get(q.data(), q.size() * 4);
    const float inv_fixed = 1.0f / (static_cast<float>(1u << frac_bits) * scale_w);
    const std::size_t B = std::max<std::size_t>(1, be->batch_size());
    std::vector<int32_t> acc(B * N);
    for (std::size_t r0 = 0; r0 < rows; r0 += B) {
      const std::size_t bn = std::min(B, rows - r0);
      be->matmul_batch_chunked(proj_id, q.data() + r0 * K, acc.data(), wq, K, N, bn,
                               [&](std::size_t col0, std::size_t ncols) {
                                 for (std::size_t j = 0; j < bn; ++j)
                                   for (std::size_t o = col0; o < col0 + ncols; ++o)
                                     out[(r0 + j) * N + o] = static_cast<float>(acc[j * N + o]) * inv_fixed;
                               });
    }
    return;
  }
  const int id = d.proj(wq, N, K, scale_w, norm_weight);
  DevMem dout(d.c, rows * N * 4);
  check(d.c, mmf_bitlinear(d.c, id, mode_of(aq), frac_bits, eps, dx.as<float>(), dout.as<float>(), rows, nullptr),
        "mmf_bitlinear");
  dout.get(out, rows * N * 4);
}

void bitlinear_cluster(float* const* outs, const float* x, const float* const* norm_weights, const int8_t* const* wqs,
                       const float* scale_w, int k, std::size_t rows, std::size_t in_dim, std::size_t out_dim, float eps,
                       int frac_bits, TernaryBackend* be, const int* proj_ids) {
  if (k <= 0 || !rows) return;
  const std::size_t K = in_dim, N = out_dim;
  if (foreign(be)) {
    // the reference's cluster over the seam (bitlinear.cpp:119-160): every projection's codes
    // from the GPU, then per chunk of batch_size() rows one matmul_seq whose produce hands
    // over projection j's codes and whose consume dequantises its accumulators
    std::vector<std::int32_t> q(static_cast<std::size_t>(k) * rows * K);
    {
      Default& d = dflt();
      std::lock_guard<std::mutex> lk(d.mu);
      DevMem dx(d.c, rows * K * 4, x), dq(d.c, rows * K * 4);
      for (int j = 0; j < k; ++j) {
        DevMem dw(d.c, K * 4, norm_weights[j]);
        check(d.c,
              mmf_bitlinear_codes(d.c, dx.as<float>(), dw.as<float>(), dq.as<int32_t>(), rows, K, eps, frac_bits),
              "mmf_bitlinear_codes");
        dq.get(q.data() + static_cast<std::size_t>(j) * rows * K, rows * K * 4);
      }
    }
    std::vector<int> ids(k, -1);
    if (proj_ids) ids.assign(proj_ids, proj_ids + k);
    const float qs = static_cast<float>(1u << frac_bits);
    const std::size_t B = std::max<std::size_t>(1, be->batch_size());
    for (std::size_t r0 = 0; r0 < rows; r0 += B) {
      const std::size_t bn = std::min(B, rows - r0);
      be->matmul_seq(
          ids.data(), wqs, k,
          [&](int j, std::int32_t* xq) { std::copy_n(q.data() + (j * rows + r0) * K, bn * K, xq); },
          [&](int j, const std::int32_t* acc) {
            const float inv_fixed = 1.0f / (qs * scale_w[j]);
            for (std::size_t e = 0; e < bn * N; ++e) outs[j][r0 * N + e] = static_cast<float>(acc[e]) * inv_fixed;
          },
          K, N, bn);
    }
    return;
  }
  if (k > 3) {  // the reference's equivalence: k bitlinear calls (kernels.hpp:46-50)
    for (int j = 0; j < k; ++j)
      bitlinear(outs[j], x, norm_weights[j], wqs[j], scale_w[j], rows, in_dim, out_dim, eps, nullptr,
                ActQuant::FixedQ510, frac_bits, be, proj_ids ? proj_ids[j] : -1);
    return;
  }
  Default& d = dflt();
  std::lock_guard<std::mutex> lk(d.mu);
  std::vector<int> ids(k);
  for (int j = 0; j < k; ++j) ids[j] = d.proj(wqs[j], N, K, scale_w[j], norm_weights[j]);
  DevMem dx(d.c, rows * K * 4, x);
  std::vector<DevMem*> douts;
  std::vector<float*> ptrs;
  for (int j = 0; j < k; ++j) {
    douts.push_back(new DevMem(d.c, rows * N * 4));
    ptrs.push_back(douts.back()->as<float>());
  }
  const int rc = mmf_bitlinear_cluster(d.c, ids.data(), k, MMF_FIXED_Q510, frac_bits, eps, dx.as<float>(), ptrs.data(),
                                       rows);
  if (rc == MMF_OK)
    for (int j = 0; j < k; ++j) douts[j]->get(outs[j], rows * N * 4);
  for (auto* p : douts) delete p;
  check(d.c, rc, "mmf_bitlinear_cluster");
}

void swiglu(float* out, const float* a, const float* b, std::size_t n) {
  if (!n) return;
  Default& d = dflt();
  std::lock_guard<std::mutex> lk(d.mu);
  DevMem da(d.c, n * 4, a), db(d.c, n * 4, b), dout(d.c, n * 4);
  check(d.c, mmf_swiglu(d.c, dout.as<float>(), da.as<float>(), db.as<float>(), n), "mmf_swiglu");
  dout.get(out, n * 4);
}

void hgrn_scan(float* out, const float* i, const float* f, std::size_t T, std::size_t D, float* state_io) {
  if (!T || !D) return;
  Default& d = dflt();
  std::lock_guard<std::mutex> lk(d.mu);
  DevMem di(d.c, T * D * 4, i), df(d.c, T * D * 4, f), dout(d.c, T * D * 4);
  DevMem dst(d.c, D * 4, state_io);
  check(d.c, mmf_hgrn_scan(d.c, dout.as<float>(), di.as<float>(), df.as<float>(), T, D, state_io ? dst.as<float>() : nullptr),
        "mmf_hgrn_scan");
  dout.get(out, T * D * 4);
  if (state_io) dst.get(state_io, D * 4);
}

void rmsnorm_swishgate(float* out, const float* g, const float* o, const float* weight, std::size_t rows,
                       std::size_t cols, float eps) {
  if (!rows || !cols) return;
  Default& d = dflt();
  std::lock_guard<std::mutex> lk(d.mu);
  DevMem dg(d.c, rows * cols * 4, g), dob(d.c, rows * cols * 4, o), dw(d.c, cols * 4, weight),
      dout(d.c, rows * cols * 4);
  check(d.c,
        mmf_rmsnorm_swishgate(d.c, dout.as<float>(), dg.as<float>(), dob.as<float>(), dw.as<float>(), rows, cols, eps),
        "mmf_rmsnorm_swishgate");
  dout.get(out, rows * cols * 4);
}

}  // namespace mmfree
