// model.cpp -- mmfree::Model on the MI355X through the mmfree_hip.h C ABI.
//
// The model compute (prefill time scan, single-row decode kernels, batched serving steps,
// lm_head) runs on the GPU. Greedy generation stays on the device between tokens
// (mmf_model_generate); sampled generation brings each step's logits back and samples on the
// host with the reference's procedure (hgrn_model.cpp:263-303, 368-406): std::mt19937_64,
// uniform_real_distribution<double>, nth_element top-k, max-shifted exp of float differences
// divided by the temperature, cumulative search -- so equal logits give equal samples.
#include "mmfree/model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <random>
#include <stdexcept>
#include <string>

#include "mmfree/hip_backend.hpp"
#include "mmfree/profile.hpp"
#include "mmfree_hip.h"

namespace mmfree {
namespace {

void check(mmf_ctx* c, int rc, const char* what) {
  if (rc != MMF_OK) throw std::runtime_error(std::string(what) + ": " + mmf_last_error(c));
}

int device_index() {
  const char* e = std::getenv("MMFREE_DEVICE");
  return e ? std::atoi(e) : 0;
}

int mode_of(ActQuant aq) {
  switch (aq) {
    case ActQuant::FixedQ510: return MMF_FIXED_Q510;
    case ActQuant::Int8Absmax: return MMF_INT8_ABSMAX;
    default: return MMF_FLOAT;
  }
}

// One sampling decision over logits [V] (greedy: first index of the maximum).
std::int64_t pick(const float* lg, std::size_t V, const Sampling& s, std::mt19937_64& rng,
                  std::vector<std::size_t>& cand) {
  if (s.temperature <= 0.0f) {
    std::size_t best = 0;
    for (std::size_t v = 1; v < V; ++v)
      if (lg[v] > lg[best]) best = v;
    return static_cast<std::int64_t>(best);
  }
  cand.resize(V);
  for (std::size_t v = 0; v < V; ++v) cand[v] = v;
  const std::size_t k = (s.top_k > 0 && static_cast<std::size_t>(s.top_k) < V) ? static_cast<std::size_t>(s.top_k) : V;
  if (k < V) {
    std::nth_element(cand.begin(), cand.begin() + k, cand.end(),
                     [&](std::size_t a, std::size_t b) { return lg[a] > lg[b]; });
    cand.resize(k);
  }
  float top = lg[cand[0]];
  for (std::size_t j = 1; j < cand.size(); ++j) top = std::max(top, lg[cand[j]]);
  std::vector<double> w(cand.size());
  double total = 0.0;
  for (std::size_t j = 0; j < cand.size(); ++j) {
    w[j] = std::exp((lg[cand[j]] - top) / s.temperature);  // float expression, as the reference
    total += w[j];
  }
  std::uniform_real_distribution<double> uni(0.0, 1.0);
  const double r = uni(rng) * total;
  double acc = 0.0;
  for (std::size_t j = 0; j < cand.size(); ++j) {
    acc += w[j];
    if (r <= acc) return static_cast<std::int64_t>(cand[j]);
  }
  return static_cast<std::int64_t>(cand.back());
}

void trampoline(void* user, std::int64_t id) { (*static_cast<const std::function<void(std::int64_t)>*>(user))(id); }

// While the Profiler is on, one model call's device time per op goes into it: the engine
// brackets each launch with events (mmf_model_profile) and the totals are added under
// these labels when the call ends, one Profiler call per launch.
class DeviceOps {
 public:
  explicit DeviceOps(mmf_ctx* c) : c_(Profiler::instance().enabled() ? c : nullptr) {
    if (c_ && mmf_model_profile(c_, 1) != MMF_OK) c_ = nullptr;
  }
  ~DeviceOps() {
    if (!c_) return;
    static const char* const kLabel[MMF_PROF_KINDS] = {"norm+quant", "matmul", "gate+scan", "lm_head", "embed"};
    double us[MMF_PROF_KINDS];
    std::uint64_t n[MMF_PROF_KINDS];
    if (mmf_model_profile_read(c_, us, n) == MMF_OK)
      for (int k = 0; k < MMF_PROF_KINDS; ++k)
        for (std::uint64_t i = 0; i < n[k]; ++i)
          Profiler::instance().add(kLabel[k], static_cast<std::uint64_t>(1000.0 * us[k] / n[k]));
    mmf_model_profile(c_, 0);
  }
  DeviceOps(const DeviceOps&) = delete;
  DeviceOps& operator=(const DeviceOps&) = delete;

 private:
  mmf_ctx* c_;
};

}  // namespace

Model::Model(const Weights& w, ActQuant aq, int frac_bits)
    : w_(w), cfg_(w.config()), aq_(aq), frac_bits_(frac_bits) {
  const int rc = mmf_create(&ctx_, device_index());
  if (rc != MMF_OK) throw std::runtime_error(std::string("mmfree: ") + mmf_last_error(nullptr));
  try {
    mmf_config c{cfg_.vocab_size, cfg_.hidden_size, cfg_.num_hidden_layers, cfg_.intermediate_size,
                 cfg_.use_lower_bound ? 1 : 0, cfg_.rms_norm_eps};
    check_call(mmf_model_begin(ctx_, &c), "mmf_model_begin");
    for (const std::string& name : w.names()) {
      const TensorRef& t = w.get(name);
      check_call(mmf_model_tensor(ctx_, name.c_str(), t.is_int8 ? 1 : 0, t.shape.data(), static_cast<int>(t.shape.size()),
                                   t.data),
            "mmf_model_tensor");
    }
    check_call(mmf_model_finalize(ctx_, mode_of(aq), frac_bits), "mmf_model_finalize");
  } catch (...) {
    mmf_destroy(ctx_);
    ctx_ = nullptr;
    throw;
  }
}

Model::~Model() { mmf_destroy(ctx_); }

void Model::set_backend(TernaryBackend* be, std::unordered_map<std::string, int> proj_ids) {
  // a HipTernaryBackend runs the same kernels this Model already uses: nothing to route
  const bool external = be && !dynamic_cast<HipTernaryBackend*>(be);
  check_call(mmf_model_set_matmul(ctx_, external ? &Model::backend_matmul : nullptr, external ? this : nullptr),
        "mmf_model_set_matmul");
  backend_ = external ? be : nullptr;
  proj_ids_ = std::move(proj_ids);
}

// Called by the engine for each FixedQ510 projection group while an external backend is set.
// Exceptions must not cross the C ABI: the message is kept and rethrown by check_call.
int Model::backend_matmul(void* self, int layer, int proj, int k, const std::int32_t* codes, std::int32_t* acc,
                          std::size_t K, std::size_t N, std::size_t rows) {
  Model* m = static_cast<Model*>(self);
  try {
    m->run_backend(layer, proj, k, codes, acc, K, N, rows);
    return 0;
  } catch (const std::exception& e) {
    m->backend_error_ = e.what();
  } catch (...) {
    m->backend_error_ = "TernaryBackend threw a non-standard exception";
  }
  return 1;
}

// The reference's calls into the seam (bitlinear.cpp:39-94, :119-160): rows in chunks of
// batch_size(); one matmul_batch_chunked per chunk for a single projection, one matmul_seq
// per chunk for the i/f/g cluster. codes [k][rows][K] and acc [k][rows][N] are contiguous,
// so a chunk's rows are handed over in place.
void Model::run_backend(int layer, int proj, int k, const std::int32_t* codes, std::int32_t* acc, std::size_t K,
                        std::size_t N, std::size_t rows) {
  static const char* const kProj[6] = {"i_proj", "f_proj", "g_proj", "o_proj", "gate_proj", "down_proj"};
  if (k < 1 || k > 3 || proj < 0 || proj + k > (proj == 6 ? 7 : 6))
    throw std::runtime_error("mmfree: invalid projection group from the engine");
  int ids[3];
  const std::int8_t* wqs[3];
  for (int j = 0; j < k; ++j) {
    const std::string tag =
        proj == 6 ? std::string("lm_head") : "model.layers." + std::to_string(layer) + "." + kProj[proj + j];
    const TensorRef& wq = w_.get(tag + ".wq");
    if (wq.shape.size() != 2 || wq.shape[0] != N || wq.shape[1] != K)
      throw std::runtime_error("mmfree: " + tag + ".wq does not have the projection's shape");
    wqs[j] = wq.i8();
    auto it = proj_ids_.find(tag);
    ids[j] = it == proj_ids_.end() ? -1 : it->second;
  }
  const std::size_t B = std::max<std::size_t>(1, backend_->batch_size());
  std::vector<char> seen;
  for (std::size_t r0 = 0; r0 < rows; r0 += B) {
    const std::size_t bn = std::min(B, rows - r0);
    if (k == 1) {
      // every column must be reported exactly once (ternary_backend.hpp contract)
      seen.assign(N, 0);
      bool bad = false;
      backend_->matmul_batch_chunked(ids[0], codes + r0 * K, acc + r0 * N, wqs[0], K, N, bn,
                                     [&](std::size_t col0, std::size_t ncols) {
                                       if (col0 > N || ncols > N - col0) {
                                         bad = true;
                                         return;
                                       }
                                       for (std::size_t o = col0; o < col0 + ncols; ++o) bad |= seen[o]++ != 0;
                                     });
      if (bad || std::count(seen.begin(), seen.end(), 1) != static_cast<std::ptrdiff_t>(N))
        throw std::runtime_error("mmfree: the TernaryBackend did not report every column exactly once");
    } else {
      backend_->matmul_seq(
          ids, wqs, k,
          [&](int j, std::int32_t* xq) {
            std::copy_n(codes + (static_cast<std::size_t>(j) * rows + r0) * K, bn * K, xq);
          },
          [&](int j, const std::int32_t* a) {
            std::copy_n(a, bn * N, acc + (static_cast<std::size_t>(j) * rows + r0) * N);
          },
          K, N, bn);
    }
  }
}

void Model::check_call(int rc, const char* what) {
  if (rc == MMF_OK) return;
  if (!backend_error_.empty()) {
    std::string e;
    e.swap(backend_error_);
    throw std::runtime_error(e);
  }
  check(ctx_, rc, what);
}

void Model::forward(const std::int64_t* ids, std::size_t T, std::vector<float>& logits) {
  DeviceOps ops(ctx_);
  logits.assign(T * cfg_.vocab_size, 0.0f);
  check_call(mmf_model_forward(ctx_, ids, T, logits.data()), "mmf_model_forward");
}

std::vector<std::int64_t> Model::generate(const std::vector<std::int64_t>& ids, std::size_t new_tokens,
                                          std::int64_t eos_id, const Sampling& samp,
                                          const std::function<void(std::int64_t)>& on_token) {
  if (ids.empty()) throw std::runtime_error("mmfree: generate needs at least one prompt token");
  streams_ = 1;
  if (samp.temperature <= 0.0f) {  // greedy: the decode loop stays on the device
    DeviceOps ops(ctx_);
    std::vector<std::int64_t> out(ids.size() + new_tokens);
    std::size_t len = 0;
    check_call(mmf_model_generate(ctx_, ids.data(), ids.size(), new_tokens, eos_id, out.data(), out.size(), &len,
                                  on_token ? &trampoline : nullptr,
                                  on_token ? const_cast<void*>(static_cast<const void*>(&on_token)) : nullptr),
               "mmf_model_generate");
    out.resize(len);
    return out;
  }
  DeviceOps ops(ctx_);
  const std::size_t V = cfg_.vocab_size;
  std::vector<std::int64_t> stream = ids;
  std::vector<float> lg(V);
  std::vector<std::size_t> cand;
  std::mt19937_64 rng(samp.seed);
  check_call(mmf_model_reset(ctx_, 1), "mmf_model_reset");
  check_call(mmf_model_prefill(ctx_, 0, ids.data(), ids.size(), lg.data(), nullptr), "mmf_model_prefill");
  if (new_tokens == 0) return stream;
  for (std::size_t step = 0; step < new_tokens; ++step) {
    if (step > 0) {
      const std::int64_t t = stream.back();
      check_call(mmf_model_step(ctx_, &t, lg.data(), nullptr), "mmf_model_step");
    }
    std::int64_t t;
    {
      MMFREE_PROFILE("sample");
      t = pick(lg.data(), V, samp, rng, cand);
    }
    stream.push_back(t);
    if (on_token) on_token(t);
    if (t == eos_id) break;
  }
  return stream;
}

std::vector<std::vector<std::int64_t>> Model::generate_serve(
    const std::vector<std::vector<std::int64_t>>& prompts, std::size_t new_tokens, std::int64_t eos_id,
    const Sampling& samp, const std::function<void(std::size_t, std::int64_t)>& on_token) {
  const std::size_t B = prompts.size(), V = cfg_.vocab_size;
  std::vector<std::vector<std::int64_t>> streams = prompts;
  if (B == 0) return streams;
  for (const auto& p : prompts)
    if (p.empty()) throw std::runtime_error("mmfree: generate_serve needs a token in every prompt");
  const bool greedy = samp.temperature <= 0.0f;
  std::vector<std::mt19937_64> rng;
  rng.reserve(B);
  for (std::size_t b = 0; b < B; ++b) rng.emplace_back(samp.seed + b);
  std::vector<std::size_t> cand;
  std::vector<char> done(B, 0);
  std::vector<float> lg(greedy ? 0 : B * V);
  std::vector<std::int64_t> am(B);
  DeviceOps ops(ctx_);
  check_call(mmf_model_reset(ctx_, B), "mmf_model_reset");
  streams_ = B;
  // all prompts prefilled together (the same states and first tokens as the reference's
  // stream-by-stream prefill), then the first-token callbacks in stream order, each stream
  // sampling from its own generator (model.hpp:60-66, hgrn_model.cpp:412-428)
  {
    std::vector<std::int64_t> cat;
    std::vector<std::size_t> lens(B);
    for (std::size_t b = 0; b < B; ++b) {
      cat.insert(cat.end(), prompts[b].begin(), prompts[b].end());
      lens[b] = prompts[b].size();
    }
    check_call(mmf_model_prefill_streams(ctx_, B, cat.data(), lens.data(), greedy ? nullptr : lg.data(), am.data()),
          "mmf_model_prefill_streams");
  }
  for (std::size_t b = 0; b < B; ++b) {
    const std::int64_t t0 = greedy ? am[b] : pick(lg.data() + b * V, V, samp, rng[b], cand);
    streams[b].push_back(t0);
    if (on_token) on_token(b, t0);
    if (t0 == eos_id) done[b] = 1;
  }
  if (new_tokens <= 1) return streams;
  std::vector<std::int64_t> tok(B);
  for (std::size_t step = 1; step < new_tokens; ++step) {
    for (std::size_t b = 0; b < B; ++b) tok[b] = streams[b].back();
    check_call(mmf_model_step(ctx_, tok.data(), greedy ? nullptr : lg.data(), am.data()), "mmf_model_step");
    bool all_done = true;
    for (std::size_t b = 0; b < B; ++b) {
      if (done[b]) continue;
      const std::int64_t t = greedy ? am[b] : pick(lg.data() + b * V, V, samp, rng[b], cand);
      streams[b].push_back(t);
      if (on_token) on_token(b, t);
      if (t == eos_id) done[b] = 1;
      else all_done = false;
    }
    if (all_done) break;
  }
  return streams;
}

std::vector<float> Model::state() const {
  std::vector<float> st(cfg_.num_hidden_layers * streams_ * cfg_.hidden_size);
  check(ctx_, mmf_model_state(ctx_, st.data()), "mmf_model_state");
  return st;
}

}  // namespace mmfree
