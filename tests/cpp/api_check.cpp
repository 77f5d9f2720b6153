// api_check.cpp -- drives the mmfree C++ API (libmmfree.so) for tests/test_gpu_api.py.
//   api_check BLOB DIR
// Reads raw inputs written by the test into DIR, writes raw outputs back:
//   bitlinear (Float / FixedQ510 / Int8Absmax, norm_out, FixedQ510 through an external
//   TernaryBackend and through HipTernaryBackend), rmsnorm, swiglu, hgrn_scan,
//   rmsnorm_swishgate; Model::generate (sampled) and Model::generate_serve (greedy, sampled).
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <functional>
#include <sstream>
#include <string>
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
  HipTernaryBackend hip(0);
  bitlinear(out.data(), x.data(), nw.data(), wq.data(), scale, rows, K, N, 1e-6f, nullptr, ActQuant::FixedQ510, 10,
            &hip, -1);
  wr(d + "bl_fixed_hipbe.f32", out);
  std::vector<std::int32_t> codes(rows * K), acc(rows * N);
  for (std::size_t i = 0; i < codes.size(); ++i) codes[i] = static_cast<std::int32_t>((i * 2654435761u) % 65536) - 32768;
  hip.matmul_batch(-1, codes.data(), acc.data(), wq.data(), K, N, rows);
  wr(d + "hipbe_codes.i32", codes);
  wr(d + "hipbe_acc.i32", acc);
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
  std::printf("ok calls=%zu\n", cpu.calls);
  return 0;
}
