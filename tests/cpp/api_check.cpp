// api_check.cpp -- drives the mmfree C++ API (libmmfree.so) for tests/test_gpu_api.py.
//   api_check BLOB DIR
// Reads raw inputs written by the test into DIR, writes raw outputs back:
//   bitlinear (Float / FixedQ510 / Int8Absmax, norm_out, FixedQ510 through an external
//   TernaryBackend and through HipTernaryBackend), rmsnorm, swiglu, hgrn_scan,
//   rmsnorm_swishgate; Model::generate (sampled) and Model::generate_serve (greedy, sampled);
//   Model::set_backend with a CpuBackend, a batching backend with a tag map and a throwing
//   backend; HipTernaryBackend with one host weight buffer refilled between calls.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <functional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "mmfree/hip_backend.hpp"
#include "mmfree/kernels.hpp"
#include "mmfree/model.hpp"
#include "mmfree/ternary_backend.hpp"
#include "mmfree/weights.hpp"

using namespace mmfree;

template <class T> std::vector<T> rd(const std::string& p) {
  std::ifstream f(p, std::ios::binary | std::ios::ate);
  if (!f) { std::fprintf(stderr, "missing %s\n", p.c_str()); std::exit(1); }
  std::vector<T> v(static_cast<std::size_t>(f.tellg()) / sizeof(T));
  f.seekg(0);
  f.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
  return v;
}
template <class T> void wr(const std::string& p, const std::vector<T>& v) {
  std::ofstream f(p, std::ios::binary);
  f.write(reinterpret_cast<const char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
}
void wr_streams(const std::string& p, const std::vector<std::vector<std::int64_t>>& s) {
  std::ofstream f(p);
  for (const auto& v : s) {
    for (std::size_t i = 0; i < v.size(); ++i) f << v[i] << (i + 1 < v.size() ? " " : "\n");
  }
}

// A plain CPU integer backend: the test's stand-in for an external (FPGA) backend.
struct TestCpuBackend final : TernaryBackend {
  std::size_t calls = 0;
  void matmul(int, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq, std::size_t N,
              std::size_t M) override {
    ++calls;
    for (std::size_t o = 0; o < M; ++o) {
      long long s = 0;
      for (std::size_t n = 0; n < N; ++n) s += static_cast<long long>(x[n]) * wq[o * N + n];
      acc[o] = static_cast<std::int32_t>(s);
    }
  }
  std::size_t batch_size() const override { return 3; }
};

// Batches 3 rows and reports each projection's columns in two ranges, the upper one first;
// counts the calls and checks that the tag map's proj_ids arrive (lm_head -> 77,
// layer 0 o_proj -> 5, every other tag -1).
struct ChunkedBackend final : TernaryBackend {
  std::size_t calls = 0, seq_calls = 0, lm_calls = 0, bad_ids = 0;
  void matmul(int, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq, std::size_t N,
              std::size_t M) override {
    for (std::size_t o = 0; o < M; ++o) {
      std::int64_t s = 0;
      for (std::size_t n = 0; n < N; ++n) s += static_cast<std::int64_t>(x[n]) * wq[o * N + n];
      acc[o] = static_cast<std::int32_t>(s);
    }
  }
  std::size_t batch_size() const override { return 3; }
  void matmul_batch_chunked(int proj_id, const std::int32_t* x, std::int32_t* acc, const std::int8_t* wq,
                            std::size_t N, std::size_t M, std::size_t b,
                            const std::function<void(std::size_t, std::size_t)>& on_cols) override {
    ++calls;
    if (proj_id == 77) ++lm_calls;
    else if (proj_id != -1 && proj_id != 5) ++bad_ids;
    matmul_batch(proj_id, x, acc, wq, N, M, b);
    const std::size_t half = M / 2;
    on_cols(half, M - half);
    if (half) on_cols(0, half);
  }
  void matmul_seq(const int* proj_ids, const std::int8_t* const* wqs, int k,
                  const std::function<void(int, std::int32_t*)>& produce,
                  const std::function<void(int, const std::int32_t*)>& consume, std::size_t N, std::size_t M,
                  std::size_t b) override {
    ++seq_calls;
    for (int j = 0; j < k; ++j)
      if (proj_ids[j] != -1) ++bad_ids;
    TernaryBackend::matmul_seq(proj_ids, wqs, k, produce, consume, N, M, b);
  }
};

struct ThrowingBackend final : TernaryBackend {
  void matmul(int, const std::int32_t*, std::int32_t*, const std::int8_t*, std::size_t, std::size_t) override {
    throw std::runtime_error("backend failure");
  }
};

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  const std::string blob = argv[1], d = std::string(argv[2]) + "/";
  // ---- operators ----
  std::istringstream dims(std::string(std::istreambuf_iterator<char>(std::ifstream(d + "dims.txt").rdbuf()), {}));
  std::size_t rows, K, N;
  float scale;
  dims >> rows >> K >> N >> scale;
  auto x = rd<float>(d + "x.f32"), nw = rd<float>(d + "nw.f32"), o2 = rd<float>(d + "o.f32");
  auto wq = rd<std::int8_t>(d + "wq.i8");
  std::vector<float> out(rows * N), norm(rows * K);
  bitlinear(out.data(), x.data(), nw.data(), wq.data(), scale, rows, K, N, 1e-6f, norm.data(), ActQuant::Float);
  wr(d + "bl_float.f32", out);
  wr(d + "bl_norm.f32", norm);
  bitlinear(out.data(), x.data(), nw.data(), wq.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::FixedQ510);
  wr(d + "bl_fixed.f32", out);
  bitlinear(out.data(), x.data(), nw.data(), wq.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::Int8Absmax);
  wr(d + "bl_int8.f32", out);
  TestCpuBackend cpu;
  bitlinear(out.data(), x.data(), nw.data(), wq.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::FixedQ510, 10,
            &cpu, -1);
  wr(d + "bl_fixed_cpube.f32", out);
  {  // the i/f/g cluster over the seam: three scales, one weight matrix
    const float* nws[3] = {nw.data(), nw.data(), nw.data()};
    const std::int8_t* wqs[3] = {wq.data(), wq.data(), wq.data()};
    const float scales[3] = {scale, 2.0f * scale, 0.5f * scale};
    std::vector<float> cl(3 * rows * N);
    float* outs[3] = {cl.data(), cl.data() + rows * N, cl.data() + 2 * rows * N};
    bitlinear_cluster(outs, x.data(), nws, wqs, scales, 3, rows, K, N, 1e-6f, 10, &cpu, nullptr);
    wr(d + "cluster_cpube.f32", cl);
  }
  HipTernaryBackend hip(0);
  bitlinear(out.data(), x.data(), nw.data(), wq.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::FixedQ510, 10,
            &hip, -1);
  wr(d + "bl_fixed_hipbe.f32", out);
  std::vector<std::int32_t> codes(rows * K), acc(rows * N);
  for (std::size_t i = 0; i < codes.size(); ++i) codes[i] = static_cast<std::int32_t>((i * 2654435761u) % 65536) - 32768;
  hip.matmul_batch(-1, codes.data(), acc.data(), wq.data(), K, N, rows);
  wr(d + "hipbe_codes.i32", codes);
  wr(d + "hipbe_acc.i32", acc);
  // one host buffer refilled with other weights between two proj_id -1 calls
  std::vector<std::int8_t> wbuf = wq;
  hip.matmul_batch(-1, codes.data(), acc.data(), wbuf.data(), K, N, rows);
  wr(d + "hipbe_reuse_acc1.i32", acc);
  for (std::size_t i = 0; i < wbuf.size(); ++i) wbuf[i] = static_cast<std::int8_t>((i * 7 + 3) % 3) - 1;
  hip.matmul_batch(-1, codes.data(), acc.data(), wbuf.data(), K, N, rows);
  wr(d + "hipbe_reuse_w2.i8", wbuf);
  wr(d + "hipbe_reuse_acc2.i32", acc);
  {  // the host operator functions' projection cache: one pointer refilled with other weights,
     // then another norm weight, then another scale (each result must follow the buffer)
    std::vector<std::int8_t> wb = wq;
    std::vector<float> nb = nw;
    bitlinear(out.data(), x.data(), nb.data(), wb.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::FixedQ510);
    wr(d + "bl_refill0.f32", out);
    wb = wbuf;
    bitlinear(out.data(), x.data(), nb.data(), wb.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::FixedQ510);
    wr(d + "bl_refill1.f32", out);
    for (std::size_t k = 0; k < K; ++k) nb[k] *= (k % 3 == 0) ? 1.5f : 0.75f;
    bitlinear(out.data(), x.data(), nb.data(), wb.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::FixedQ510);
    wr(d + "bl_refill2.f32", out);
    wr(d + "bl_refill_nw2.f32", nb);
    bitlinear(out.data(), x.data(), nb.data(), wb.data(), 2.0f * scale, rows, K, N, 1e-6f, nullptr,
              ActQuant::FixedQ510);
    wr(d + "bl_refill3.f32", out);
  }
  std::vector<float> y(rows * K);
  rmsnorm(y.data(), x.data(), nw.data(), rows, K, 1e-6f);
  wr(d + "rmsnorm.f32", y);
  rmsnorm_swishgate(y.data(), x.data(), o2.data(), nw.data(), rows, K, 1e-6f);
  wr(d + "swishgate.f32", y);
  swiglu(y.data(), x.data(), o2.data(), rows * K);
  wr(d + "swiglu.f32", y);
  std::vector<float> st(K, 0.5f);
  auto f = rd<float>(d + "f.f32");
  hgrn_scan(y.data(), x.data(), f.data(), rows, K, st.data());
  wr(d + "scan.f32", y);
  wr(d + "scan_state.f32", st);
  // ---- model ----
  Weights w(blob);
  std::vector<std::vector<std::int64_t>> prompts;
  {
    std::ifstream pf(d + "prompts.txt");
    std::string line;
    while (std::getline(pf, line)) {
      std::istringstream ls(line);
      std::vector<std::int64_t> p;
      std::int64_t t;
      while (ls >> t) p.push_back(t);
      if (!p.empty()) prompts.push_back(p);
    }
  }
  for (int mode = 0; mode < 2; ++mode) {
    Model m(w, mode ? ActQuant::FixedQ510 : ActQuant::Float);
    const std::string tag = mode ? "fixed" : "float";
    std::vector<std::vector<std::int64_t>> cb(prompts.size());
    auto s = m.generate_serve(prompts, 8, -1, Sampling{}, [&](std::size_t b, std::int64_t t) { cb[b].push_back(t); });
    wr_streams(d + "serve_" + tag + ".txt", s);
    wr_streams(d + "serve_" + tag + "_cb.txt", cb);
    Sampling smp;
    smp.temperature = 0.8f;
    smp.top_k = 40;
    smp.seed = 7;
    wr_streams(d + "serve_" + tag + "_sampled.txt", m.generate_serve(prompts, 8, -1, smp));
    wr_streams(d + "gen_" + tag + "_sampled.txt", {m.generate(prompts[0], 24, -1, smp)});
    Sampling full;
    full.temperature = 1.3f;
    full.seed = 11;
    wr_streams(d + "gen_" + tag + "_sampled_full.txt", {m.generate(prompts[0], 12, -1, full)});
    std::vector<std::int64_t> gcb;
    auto g = m.generate(prompts[0], 10, -1, Sampling{}, [&](std::int64_t t) { gcb.push_back(t); });
    wr_streams(d + "gen_" + tag + ".txt", {g, gcb});
  }
  // ---- Model::set_backend with backends that are not this engine's (FixedQ510) ----
  {
    Model m(w, ActQuant::FixedQ510);
    CpuBackend cpub;
    m.set_backend(&cpub, {});
    wr_streams(d + "be_cpu_gen.txt", {m.generate(prompts[0], 10)});
    wr_streams(d + "be_cpu_serve.txt", m.generate_serve(prompts, 6));
    Sampling smp;
    smp.temperature = 0.8f;
    smp.top_k = 40;
    smp.seed = 7;
    wr_streams(d + "be_cpu_gen_sampled.txt", {m.generate(prompts[0], 12, -1, smp)});
    std::vector<float> lg;
    m.forward(prompts[0].data(), prompts[0].size(), lg);
    wr(d + "be_cpu_forward.f32", lg);
    // a backend that batches 3 rows, reports columns in two ranges out of order, and sees
    // proj_ids from the tag map
    ChunkedBackend chk;
    std::unordered_map<std::string, int> ids{{"lm_head", 77}, {"model.layers.0.o_proj", 5}};
    m.set_backend(&chk, ids);
    wr_streams(d + "be_chunk_gen.txt", {m.generate(prompts[0], 10)});
    std::printf("chunked backend: calls=%zu seq=%zu lm_head_ids=%zu bad_ids=%zu\n", chk.calls, chk.seq_calls,
                chk.lm_calls, chk.bad_ids);
    // back to the engine's own kernels
    m.set_backend(nullptr, {});
    wr_streams(d + "be_none_gen.txt", {m.generate(prompts[0], 10)});
    // a backend whose matmul throws: the error reaches the caller
    ThrowingBackend thr;
    m.set_backend(&thr, {});
    bool threw = false;
    try {
      m.generate(prompts[0], 4);
    } catch (const std::runtime_error& e) {
      threw = std::string(e.what()).find("backend failure") != std::string::npos;
    }
    std::printf("throwing backend: %s\n", threw ? "error propagated" : "NO ERROR");
  }
  std::printf("ok calls=%zu\n", cpu.calls);
  return 0;
}
