// ref_harness.cpp -- C entry points into the reference engine compiled from its own
// sources (see Makefile, target `ref`). Test infrastructure only: the parity tests call
// these through ctypes to pin the C restatement and to write golden fixtures.
//
// Each wrapper forwards to the reference function it names, with the reference's own
// argument meaning:
//   rmsnorm / bitlinear / bitlinear_cluster / swiglu / hgrn_scan / rmsnorm_swishgate
//     cpp/include/mmfree/kernels.hpp:29-68
//   simd::{sumsq, sigmoid, silu, swiglu, hgrn_step, quant_q510, expf_poly}
//     cpp/include/mmfree/simd.hpp:69-357
//   CpuBackend::matmul  cpp/include/mmfree/ternary_backend.hpp:96-103
//   Model::{forward, generate, generate_serve}  cpp/include/mmfree/model.hpp:37-70
//   Tokenizer::{encode, decode}  cpp/include/mmfree/tokenizer.hpp:15-37
// Per-layer capture reads the Model's private scratch and recurrent state, so model.hpp
// is included with `private` opened up (standard headers are included first so only the
// reference's own headers see the define).
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "mmfree/kernels.hpp"
#include "mmfree/simd.hpp"
#include "mmfree/ternary_backend.hpp"
#include "mmfree/tokenizer.hpp"
#include "mmfree/weights.hpp"
#define private public
#include "mmfree/model.hpp"
#undef private

using namespace mmfree;

namespace {
ActQuant aq_of(int mode) { return mode == 1 ? ActQuant::FixedQ510 : ActQuant::Float; }

struct RefModel {
  std::unique_ptr<Weights> w;
  std::unique_ptr<Model> m;
  std::string err;
};
thread_local std::string g_err;
}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

float ref_sumsq(const float* x, std::size_t n) { return simd::sumsq(x, n); }
float ref_expf_poly(float x) { return simd::expf_poly(x); }

void ref_sigmoid(float* out, const float* x, std::size_t n) { simd::sigmoid(out, x, n); }
void ref_silu(float* out, const float* x, std::size_t n) { simd::silu(out, x, n); }
void ref_swiglu_simd(float* out, const float* a, const float* b, std::size_t n) {
  simd::swiglu(out, a, b, n);
}
void ref_quant_q510(std::int32_t* yq, const float* y, float qs, std::size_t n) {
  simd::quant_q510(yq, y, qs, n);
}
float ref_ternary_dot_f32(const float* y, const std::int8_t* w, std::size_t n) {
  return simd::ternary_dot_f32(y, w, n);
}

void ref_rmsnorm(float* y, const float* x, const float* w, std::size_t rows, std::size_t cols,
                 float eps) {
  rmsnorm(y, x, w, rows, cols, eps);
}

void ref_bitlinear(float* out, const float* x, const float* normw, const std::int8_t* wq,
                   float scale_w, std::size_t rows, std::size_t in_dim, std::size_t out_dim,
                   float eps, float* norm_out, int mode, int frac_bits) {
  bitlinear(out, x, normw, wq, scale_w, rows, in_dim, out_dim, eps, norm_out, aq_of(mode),
            frac_bits, nullptr, -1);
}

void ref_bitlinear_cluster(float* const* outs, const float* x, const float* const* normws,
                           const std::int8_t* const* wqs, const float* scale_w, int k,
                           std::size_t rows, std::size_t in_dim, std::size_t out_dim, float eps,
                           int frac_bits) {
  std::vector<int> ids(k, -1);
  bitlinear_cluster(outs, x, normws, wqs, scale_w, k, rows, in_dim, out_dim, eps, frac_bits,
                    nullptr, ids.data());
}

void ref_ternary_matmul(const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                        std::size_t N, std::size_t M, std::size_t b) {
  CpuBackend be;
  be.matmul_batch(-1, x, acc, wq, N, M, b);
}

void ref_swiglu(float* out, const float* a, const float* b, std::size_t n) {
  swiglu(out, a, b, n);
}
void ref_hgrn_scan(float* out, const float* i, const float* f, std::size_t T, std::size_t D,
                   float* state_io) {
  hgrn_scan(out, i, f, T, D, state_io);
}
void ref_rmsnorm_swishgate(float* out, const float* g, const float* o, const float* w,
                           std::size_t rows, std::size_t cols, float eps) {
  rmsnorm_swishgate(out, g, o, w, rows, cols, eps);
}

// ---- model ---------------------------------------------------------------------------
void* ref_model_open(const char* blob, int mode, int frac_bits) {
  try {
    auto* r = new RefModel;
    r->w = std::make_unique<Weights>(blob);
    r->m = std::make_unique<Model>(*r->w, aq_of(mode), frac_bits);
    return r;
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void ref_model_close(void* h) { delete static_cast<RefModel*>(h); }

// The reference Model object itself (for attaching a TernaryBackend, ref_hipbe.cpp).
void* ref_model_ptr(void* h) { return static_cast<RefModel*>(h)->m.get(); }
// Its Weights (for registering the projections with a resident-weight backend).
void* ref_model_weights(void* h) { return static_cast<RefModel*>(h)->w.get(); }

// Model::generate; writes the full id stream into out_ids (capacity cap) and returns its
// length. Sampling per model.hpp:27-31.
long ref_model_generate(void* h, const std::int64_t* ids, std::size_t n, std::size_t new_tokens,
                        std::int64_t eos_id, float temperature, int top_k, std::uint64_t seed,
                        std::int64_t* out_ids, std::size_t cap) {
  auto* r = static_cast<RefModel*>(h);
  Sampling s;
  s.temperature = temperature;
  s.top_k = top_k;
  s.seed = seed;
  std::vector<std::int64_t> in(ids, ids + n);
  auto st = r->m->generate(in, new_tokens, eos_id, s, {});
  std::size_t len = st.size() < cap ? st.size() : cap;
  std::memcpy(out_ids, st.data(), len * sizeof(std::int64_t));
  return static_cast<long>(st.size());
}

// Per-layer recurrent state after the last generate(): [L, H].
void ref_model_state(void* h, float* out) {
  auto* r = static_cast<RefModel*>(h);
  std::memcpy(out, r->m->rstate_.data(), r->m->rstate_.size() * sizeof(float));
}

// Model::forward over T ids: logits [T, V].
void ref_model_forward(void* h, const std::int64_t* ids, std::size_t T, float* logits) {
  auto* r = static_cast<RefModel*>(h);
  std::vector<float> lg;
  r->m->forward(ids, T, lg);
  std::memcpy(logits, lg.data(), lg.size() * sizeof(float));
}

// Model::generate_serve over B prompts (flattened ids with per-prompt lengths). Output:
// out[b * cap_per + j] = stream b's j-th id; out_len[b] = its length.
void ref_model_generate_serve(void* h, const std::int64_t* flat, const std::size_t* lens,
                              std::size_t B, std::size_t new_tokens, std::int64_t eos_id,
                              float temperature, int top_k, std::uint64_t seed,
                              std::int64_t* out, std::size_t cap_per, std::size_t* out_len) {
  auto* r = static_cast<RefModel*>(h);
  std::vector<std::vector<std::int64_t>> prompts(B);
  std::size_t off = 0;
  for (std::size_t b = 0; b < B; ++b) {
    prompts[b].assign(flat + off, flat + off + lens[b]);
    off += lens[b];
  }
  Sampling s;
  s.temperature = temperature;
  s.top_k = top_k;
  s.seed = seed;
  auto st = r->m->generate_serve(prompts, new_tokens, eos_id, s, {});
  for (std::size_t b = 0; b < B; ++b) {
    std::size_t len = st[b].size() < cap_per ? st[b].size() : cap_per;
    std::memcpy(out + b * cap_per, st[b].data(), len * sizeof(std::int64_t));
    out_len[b] = st[b].size();
  }
}

// Layer-by-layer trace of a stateful prefill over T ids (Model::generate's prefill,
// hgrn_model.cpp:318-327): embeds the ids, then runs block(l) with the carried state
// rstate_[l], recording after each layer l:
//   h_out[l]   [T, H]  the hidden stream
//   st_out[l]  [H]     the recurrent state
//   i/f/g/scan/recur [l] [T, H] the block's scratch: i_proj output, f after the
//                               sigmoid and lower bound, g_proj output, the scan input
//                               silu(i)*(1-f), and the recurrence output
void ref_model_trace(void* h, const std::int64_t* ids, std::size_t T, float* h_out,
                     float* st_out, float* i_out, float* f_out, float* g_out, float* scan_out,
                     float* recur_out) {
  auto* r = static_cast<RefModel*>(h);
  Model& m = *r->m;
  const std::size_t H = m.cfg_.hidden_size, L = m.cfg_.num_hidden_layers;
  m.rstate_.assign(L * H, 0.0f);
  m.ensure_scratch(T);
  float* hb = m.hbuf_.data();
  const float* emb = r->w->get("model.embeddings").f32();
  for (std::size_t t = 0; t < T; ++t)
    std::memcpy(hb + t * H, emb + static_cast<std::size_t>(ids[t]) * H, H * sizeof(float));
  const std::size_t TH = T * H;
  for (std::size_t l = 0; l < L; ++l) {
    m.block(hb, T, l, &m.rstate_[l * H]);
    std::memcpy(h_out + l * TH, hb, TH * sizeof(float));
    std::memcpy(st_out + l * H, &m.rstate_[l * H], H * sizeof(float));
    if (i_out) std::memcpy(i_out + l * TH, m.i_.data(), TH * sizeof(float));
    if (f_out) std::memcpy(f_out + l * TH, m.f_.data(), TH * sizeof(float));
    if (g_out) std::memcpy(g_out + l * TH, m.g_.data(), TH * sizeof(float));
    if (scan_out) std::memcpy(scan_out + l * TH, m.scan_.data(), TH * sizeof(float));
    if (recur_out) std::memcpy(recur_out + l * TH, m.recur_.data(), TH * sizeof(float));
  }
}

// ---- tokenizer ----
void* ref_tok_open(const char* path) {
  try {
    return new Tokenizer(path);
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}
void ref_tok_close(void* h) { delete static_cast<Tokenizer*>(h); }
// ids of `text` (n bytes) into out (capacity cap); returns the count (may exceed cap)
long ref_tok_encode(void* h, const char* text, std::size_t n, int add_bos, std::int64_t* out, std::size_t cap) {
  const auto ids = static_cast<Tokenizer*>(h)->encode(std::string(text, n), add_bos != 0);
  for (std::size_t i = 0; i < ids.size() && i < cap; ++i) out[i] = ids[i];
  return static_cast<long>(ids.size());
}
// bytes of decode(ids) into out (capacity cap); returns the length (may exceed cap)
long ref_tok_decode(void* h, const std::int64_t* ids, std::size_t n, int skip_special, char* out, std::size_t cap) {
  const std::string s = static_cast<Tokenizer*>(h)->decode(std::vector<std::int64_t>(ids, ids + n), skip_special != 0);
  std::memcpy(out, s.data(), s.size() < cap ? s.size() : cap);
  return static_cast<long>(s.size());
}

}  // extern "C"
