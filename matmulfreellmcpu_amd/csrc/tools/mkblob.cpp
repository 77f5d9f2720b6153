// mkblob.cpp -- write a seeded synthetic HGRN-Bit weight blob in the MMFREE1 layout.
//
// Layout (byte-compatible with the reference loader, cpp/src/io/weights.cpp:3-8,191-254,
// and its writer tools/provision.py:126-163):
//   "MMFREE1\n" | u64 LE header_len | JSON header | zero pad to 64 | data section
//   header = {"config": {...}, "tensors": {name: {dtype, shape, offset, nbytes}}}
//   offsets are relative to the data section and 64-byte aligned.
// Tensor names and order follow provision.py:101-124: model.embeddings, model.norm.w,
// lm_head.{wq,scale_w,normw}, lower_bounds, then per layer attn_norm.w, mlp_norm.w,
// g_norm.w and the six projections {i,f,g,o,gate,down}_proj.{wq,scale_w,normw}.
//
// Synthetic weights (the checkpoint itself needs the network):
//   latent W ~ N(0, 0.02)  ->  scale_w = 1/max(mean|W|, 1e-5),
//   wq = clamp(rne(W * scale_w), -1, 1)  (the ternarisation of tools/reference.py:138-142)
//   embeddings ~ N(0, 0.02); norm weights 1 (or 1 + N(0, 0.1) with --random-norms)
//   lower_bounds = cumsum(softmax(raw, 0)) - softmax(raw)[0] over layers (provision.py:108-111)
//   with raw = 0 (so lb[l] = l/L) or raw ~ N(0, 1) with --random-lb.
// Random numbers: splitmix64 streams, one per (tensor, 64Ki-element chunk), turned into
// normals by Box-Muller in double precision, so any thread count gives the same blob.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

struct Dims {
  std::size_t V = 32000, H = 1024, L = 24, I = 2816;
};

std::uint64_t splitmix64(std::uint64_t& s) {
  std::uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// uniform in (0, 1]
double unit(std::uint64_t& s) { return (static_cast<double>(splitmix64(s) >> 11) + 1.0) * 0x1.0p-53; }

constexpr std::size_t kChunk = 1u << 16;

// Fill out[0..n) with N(0, sigma) for tensor `tid` of the blob seeded with `seed`.
void normals(float* out, std::size_t n, std::uint64_t seed, std::uint64_t tid, double sigma) {
  const std::size_t chunks = (n + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(dynamic, 4)
  for (std::size_t c = 0; c < chunks; ++c) {
    std::uint64_t s = seed * 0x2545F4914F6CDD1Dull ^ (tid << 40) ^ (c * 0x9E3779B97F4A7C15ull);
    splitmix64(s);
    const std::size_t lo = c * kChunk, hi = (lo + kChunk < n) ? lo + kChunk : n;
    for (std::size_t i = lo; i < hi; i += 2) {
      double u1 = unit(s), u2 = unit(s);
      double r = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586476925 * u2;
      out[i] = static_cast<float>(sigma * r * std::cos(th));
      if (i + 1 < hi) out[i + 1] = static_cast<float>(sigma * r * std::sin(th));
    }
  }
}

struct Tensor {
  std::string name;
  bool i8;
  std::vector<std::size_t> shape;
  std::vector<unsigned char> bytes;
};

Tensor f32_tensor(const std::string& name, std::vector<std::size_t> shape, const std::vector<float>& v) {
  Tensor t{name, false, std::move(shape), {}};
  t.bytes.resize(v.size() * 4);
  std::memcpy(t.bytes.data(), v.data(), t.bytes.size());
  return t;
}

// Ternarise a latent [N, K] N(0, 0.02) matrix; appends wq and scale_w tensors.
void ternary(std::vector<Tensor>& out, const std::string& tag, std::size_t N, std::size_t K,
             std::uint64_t seed, std::uint64_t tid) {
  std::vector<float> w(N * K);
  normals(w.data(), w.size(), seed, tid, 0.02);
  const std::size_t chunks = (w.size() + kChunk - 1) / kChunk;
  std::vector<double> part(chunks, 0.0);
#pragma omp parallel for schedule(static)
  for (std::size_t c = 0; c < chunks; ++c) {
    double s = 0.0;
    const std::size_t lo = c * kChunk, hi = (lo + kChunk < w.size()) ? lo + kChunk : w.size();
    for (std::size_t i = lo; i < hi; ++i) s += std::fabs(static_cast<double>(w[i]));
    part[c] = s;
  }
  double sum = 0.0;
  for (double p : part) sum += p;
  double mean = sum / static_cast<double>(w.size());
  const float scale = static_cast<float>(1.0 / (mean > 1e-5 ? mean : 1e-5));
  Tensor wq{tag + ".wq", true, {N, K}, std::vector<unsigned char>(N * K)};
#pragma omp parallel for schedule(static)
  for (std::size_t i = 0; i < w.size(); ++i) {
    float q = std::nearbyintf(w[i] * scale);
    q = q > 1.0f ? 1.0f : (q < -1.0f ? -1.0f : q);
    wq.bytes[i] = static_cast<unsigned char>(static_cast<std::int8_t>(q));
  }
  out.push_back(std::move(wq));
  out.push_back(f32_tensor(tag + ".scale_w", {1}, {scale}));
}

std::vector<float> norm_weight(std::size_t n, bool random, std::uint64_t seed, std::uint64_t tid) {
  std::vector<float> v(n, 1.0f);
  if (random) {
    normals(v.data(), n, seed, tid, 0.1);
    for (auto& x : v) x += 1.0f;
  }
  return v;
}

std::string shape_json(const std::vector<std::size_t>& s) {
  std::string r = "[";
  for (std::size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

void usage() {
  std::fprintf(stderr,
               "usage: mmfree-mkblob --out PATH [--preset tiny|s0|s2|s3] [--vocab V] [--hidden H]\n"
               "                     [--layers L] [--inter I] [--seed N] [--random-norms]\n"
               "                     [--random-lb] [--no-lower-bound] [--eps E]\n"
               "presets: s0 = 370M (H1024 I2816 L24), s2 = 1.3B (H2048 I5632 L24),\n"
               "         s3 = 2.7B (H2560 I6912 L32), tiny = (V512 H64 I176 L3); vocab 32000\n");
}

}  // namespace

int main(int argc, char** argv) {
  Dims d;
  std::string out;
  std::uint64_t seed = 1234;
  bool random_norms = false, random_lb = false, lower_bound = true;
  double eps = 1e-6;
  for (int a = 1; a < argc; ++a) {
    std::string k = argv[a];
    auto next = [&]() -> const char* {
      if (a + 1 >= argc) { usage(); std::exit(2); }
      return argv[++a];
    };
    if (k == "--out") out = next();
    else if (k == "--preset") {
      std::string p = next();
      if (p == "tiny") d = {512, 64, 3, 176};
      else if (p == "s0") d = {32000, 1024, 24, 2816};
      else if (p == "s2") d = {32000, 2048, 24, 5632};
      else if (p == "s3") d = {32000, 2560, 32, 6912};
      else { usage(); return 2; }
    } else if (k == "--vocab") d.V = std::strtoull(next(), nullptr, 10);
    else if (k == "--hidden") d.H = std::strtoull(next(), nullptr, 10);
    else if (k == "--layers") d.L = std::strtoull(next(), nullptr, 10);
    else if (k == "--inter") d.I = std::strtoull(next(), nullptr, 10);
    else if (k == "--seed") seed = std::strtoull(next(), nullptr, 10);
    else if (k == "--random-norms") random_norms = true;
    else if (k == "--random-lb") random_lb = true;
    else if (k == "--no-lower-bound") lower_bound = false;
    else if (k == "--eps") eps = std::strtod(next(), nullptr);
    else { usage(); return 2; }
  }
  if (out.empty() || !d.V || !d.H || !d.L || !d.I) { usage(); return 2; }

  std::vector<Tensor> ts;
  std::uint64_t tid = 0;
  {
    std::vector<float> emb(d.V * d.H);
    normals(emb.data(), emb.size(), seed, tid++, 0.02);
    ts.push_back(f32_tensor("model.embeddings", {d.V, d.H}, emb));
  }
  ts.push_back(f32_tensor("model.norm.w", {d.H}, norm_weight(d.H, random_norms, seed, tid++)));
  ternary(ts, "lm_head", d.V, d.H, seed, tid++);
  ts.push_back(f32_tensor("lm_head.normw", {d.H}, norm_weight(d.H, random_norms, seed, tid++)));
  if (lower_bound) {
    // softmax over the layer axis, then cumsum - first (fp32, sequential like torch.cumsum)
    std::vector<float> raw(d.L * d.H, 0.0f), lb(d.L * d.H);
    if (random_lb) normals(raw.data(), raw.size(), seed, tid, 1.0);
    ++tid;
    for (std::size_t c = 0; c < d.H; ++c) {
      double mx = raw[c];
      for (std::size_t l = 1; l < d.L; ++l) mx = std::max<double>(mx, raw[l * d.H + c]);
      double z = 0.0;
      for (std::size_t l = 0; l < d.L; ++l) z += std::exp(raw[l * d.H + c] - mx);
      float acc = 0.0f, first = 0.0f;
      for (std::size_t l = 0; l < d.L; ++l) {
        float p = static_cast<float>(std::exp(raw[l * d.H + c] - mx) / z);
        if (l == 0) first = p;
        acc += p;
        lb[l * d.H + c] = acc - first;
      }
    }
    ts.push_back(f32_tensor("lower_bounds", {d.L, d.H}, lb));
  }
  const char* projs[6] = {"i_proj", "f_proj", "g_proj", "o_proj", "gate_proj", "down_proj"};
  for (std::size_t l = 0; l < d.L; ++l) {
    const std::string p = "model.layers." + std::to_string(l);
    ts.push_back(f32_tensor(p + ".attn_norm.w", {d.H}, norm_weight(d.H, random_norms, seed, tid++)));
    ts.push_back(f32_tensor(p + ".mlp_norm.w", {d.H}, norm_weight(d.H, random_norms, seed, tid++)));
    ts.push_back(f32_tensor(p + ".g_norm.w", {d.H}, norm_weight(d.H, random_norms, seed, tid++)));
    for (int j = 0; j < 6; ++j) {
      const std::size_t N = j == 4 ? 2 * d.I : d.H, K = j == 5 ? d.I : d.H;
      ternary(ts, p + "." + projs[j], N, K, seed, tid++);
      ts.push_back(f32_tensor(p + "." + projs[j] + ".normw", {K},
                              norm_weight(K, random_norms, seed, tid++)));
    }
  }

  auto align = [](std::size_t n) { return (n + 63) / 64 * 64; };
  std::string hdr = "{\"config\": {\"vocab_size\": " + std::to_string(d.V) +
                    ", \"hidden_size\": " + std::to_string(d.H) +
                    ", \"num_hidden_layers\": " + std::to_string(d.L) +
                    ", \"num_heads\": 1, \"expand_ratio\": 1, \"intermediate_size\": " +
                    std::to_string(d.I) + ", \"use_lower_bound\": " +
                    (lower_bound ? "true" : "false") + ", \"use_short_conv\": false";
  char ebuf[64];
  std::snprintf(ebuf, sizeof ebuf, "%.17g", eps);
  hdr += std::string(", \"rms_norm_eps\": ") + ebuf + "}, \"tensors\": {";
  std::size_t off = 0;
  std::vector<std::size_t> offs;
  for (std::size_t i = 0; i < ts.size(); ++i) {
    offs.push_back(off);
    hdr += (i ? ", \"" : "\"") + ts[i].name + "\": {\"dtype\": \"" + (ts[i].i8 ? "i8" : "f32") +
           "\", \"shape\": " + shape_json(ts[i].shape) + ", \"offset\": " + std::to_string(off) +
           ", \"nbytes\": " + std::to_string(ts[i].bytes.size()) + "}";
    off = align(off + ts[i].bytes.size());
  }
  hdr += "}}";
  const std::size_t data_len = off, data_start = align(16 + hdr.size());

  FILE* f = std::fopen(out.c_str(), "wb");
  if (!f) { std::perror(out.c_str()); return 1; }
  std::uint64_t hl = hdr.size();
  std::vector<unsigned char> pad(64, 0);
  bool ok = std::fwrite("MMFREE1\n", 1, 8, f) == 8 && std::fwrite(&hl, 8, 1, f) == 1 &&
            std::fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size() &&
            std::fwrite(pad.data(), 1, data_start - 16 - hdr.size(), f) == data_start - 16 - hdr.size();
  for (std::size_t i = 0; ok && i < ts.size(); ++i) {
    std::size_t end = (i + 1 < ts.size()) ? offs[i + 1] : data_len;
    std::size_t n = ts[i].bytes.size();
    ok = std::fwrite(ts[i].bytes.data(), 1, n, f) == n &&
         std::fwrite(pad.data(), 1, end - offs[i] - n, f) == end - offs[i] - n;
  }
  if (std::fclose(f) != 0) ok = false;
  if (!ok) { std::fprintf(stderr, "mkblob: write failed for %s\n", out.c_str()); return 1; }
  std::printf("wrote %s: V=%zu H=%zu L=%zu I=%zu seed=%llu, %zu tensors, %.1f MB\n", out.c_str(),
              d.V, d.H, d.L, d.I, static_cast<unsigned long long>(seed), ts.size(),
              (data_start + data_len) / 1e6);
  return 0;
}
