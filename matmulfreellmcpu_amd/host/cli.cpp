// cli.cpp -- mmfree-cli on the MI355X: the reference CLI's flags, inputs and outputs
// (cpp/app/main.cpp:14-40, 95-230), model compute on the GPU.
//
//   mmfree-cli "The capital of France is"       text in, streamed text out
//   echo "Once upon a time," | mmfree-cli        prompt from stdin
//   mmfree-cli --ids 1,415,310 --gen 8           ids in, full id stream out (no EOS stop)
//
//   --blob PATH --tokenizer PATH --mode float|fixed|int8 --frac N --gen N --temp T --top-k K
//   --seed N --ids a,b,c --decode-ids a,b,c --no-bos --no-eos --print-ids --show-ids
//   --logits-out PATH --bench --warmup N --reps N --profile
// Additions: --mode int8 (per-row int8 absmax activations), --device N (also MMFREE_DEVICE).
// Unknown flags exit 2, as in the reference. The tokenizer (default <blob dir>/tokenizer.mmtok)
// is loaded only when text is encoded or decoded.
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <fstream>
#include <functional>
#include <iostream>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "mmfree/bench.hpp"
#include "mmfree/model.hpp"
#include "mmfree/profile.hpp"
#include "mmfree/tokenizer.hpp"
#include "mmfree/weights.hpp"

using namespace mmfree;

static std::vector<std::int64_t> parse_ids(const std::string& s) {
  std::vector<std::int64_t> ids;
  std::size_t i = 0;
  while (i < s.size()) {
    while (i < s.size() && !(std::isdigit(static_cast<unsigned char>(s[i])) || s[i] == '-')) ++i;
    if (i >= s.size()) break;
    std::size_t j = i + (s[i] == '-' ? 1 : 0);
    while (j < s.size() && std::isdigit(static_cast<unsigned char>(s[j]))) ++j;
    if (j > i + (s[i] == '-' ? 1 : 0)) ids.push_back(std::stoll(s.substr(i, j - i)));
    i = j;
  }
  return ids;
}

static std::string tokenizer_beside(const std::string& blob) {
  const std::size_t slash = blob.find_last_of('/');
  return (slash == std::string::npos ? std::string() : blob.substr(0, slash + 1)) + "tokenizer.mmtok";
}

static int run(int argc, char** argv) {
  std::string blob = "model.mmfree", tokenizer_path, mode = "fixed", ids_arg, logits_out, decode_arg, prompt;
  bool have_prompt = false, no_bos = false, no_eos = false, print_ids = false, show_ids = false, bench = false,
       profile = false;
  int frac = 10, warmup = 1, reps = 3;
  std::size_t gen = 32;
  Sampling samp;
  bool have_seed = false;
  for (int a = 1; a < argc; ++a) {
    const std::string k = argv[a];
    auto next = [&]() -> const char* { return (a + 1 < argc) ? argv[++a] : ""; };
    if (k == "--blob") blob = next();
    else if (k == "--tokenizer") tokenizer_path = next();
    else if (k == "--mode") mode = next();
    else if (k == "--frac") frac = std::atoi(next());
    else if (k == "--gen") gen = static_cast<std::size_t>(std::atoll(next()));
    else if (k == "--temp" || k == "--temperature") samp.temperature = static_cast<float>(std::atof(next()));
    else if (k == "--top-k") samp.top_k = std::atoi(next());
    else if (k == "--seed") { samp.seed = std::strtoull(next(), nullptr, 10); have_seed = true; }
    else if (k == "--ids") ids_arg = next();
    else if (k == "--decode-ids") decode_arg = next();
    else if (k == "--no-bos") no_bos = true;
    else if (k == "--no-eos") no_eos = true;
    else if (k == "--print-ids") print_ids = true;
    else if (k == "--show-ids") show_ids = true;
    else if (k == "--logits-out") logits_out = next();
    else if (k == "--bench") bench = true;
    else if (k == "--warmup") warmup = std::atoi(next());
    else if (k == "--reps") reps = std::atoi(next());
    else if (k == "--profile") profile = true;
    else if (k == "--device") setenv("MMFREE_DEVICE", next(), 1);
    else if (!k.empty() && k[0] == '-') {
      std::fprintf(stderr, "unknown arg: %s\n", k.c_str());
      return 2;
    } else {
      prompt = k;  // the first positional argument is the prompt
      have_prompt = true;
    }
  }
  if (tokenizer_path.empty()) tokenizer_path = tokenizer_beside(blob);

  if (!decode_arg.empty()) {  // decode only: no weights, no device
    const Tokenizer tok(tokenizer_path);
    std::printf("%s\n", tok.decode(parse_ids(decode_arg)).c_str());
    return 0;
  }

  const bool ids_mode = !ids_arg.empty();
  const bool ids_out = print_ids || ids_mode;
  std::unique_ptr<Tokenizer> tok;
  if (!ids_mode || !ids_out) tok = std::make_unique<Tokenizer>(tokenizer_path);

  std::vector<std::int64_t> ids;
  if (ids_mode) {
    ids = parse_ids(ids_arg);
  } else {
    if (!have_prompt) {
      if (bench) {
        prompt = "The quick brown fox jumps over the lazy dog.";
      } else {
        std::string all, line;
        while (std::getline(std::cin, line)) all += line + "\n";
        while (!all.empty() && (all.back() == '\n' || all.back() == ' ')) all.pop_back();
        prompt = all;
      }
    }
    ids = tok->encode(prompt, !no_bos);
  }
  if (ids.empty()) {
    std::fprintf(stderr, "no input (pass a prompt, --ids, or pipe via stdin)\n");
    return 2;
  }

  ActQuant aq = ActQuant::Float;
  if (mode == "fixed") aq = ActQuant::FixedQ510;
  else if (mode == "int8") aq = ActQuant::Int8Absmax;
  else if (mode != "float") {
    std::fprintf(stderr, "unknown mode: %s (float|fixed|int8)\n", mode.c_str());
    return 2;
  }
  std::unique_ptr<Weights> w;
  std::unique_ptr<Model> model;
  if (gen > 0 || !logits_out.empty() || bench) {
    w = std::make_unique<Weights>(blob);
    model = std::make_unique<Model>(*w, aq, frac);
  }
  if (bench) {
    if (gen == 0) {
      std::fprintf(stderr, "--bench needs --gen > 0\n");
      return 2;
    }
    BenchOpts o;
    o.gen = gen;
    o.warmup = warmup;
    o.reps = reps;
    o.profile = profile;
    run_bench(*model, ids, o, blob.c_str(), mode.c_str(), frac);
    return 0;
  }
  if (samp.temperature > 0.0f && !have_seed) samp.seed = std::random_device{}();

  // text out: re-decode everything generated so far and print the new bytes (decoding a
  // single token is not safe: leading-space strip, byte-fallback sequences)
  const bool stream_text = !ids_out;
  std::vector<std::int64_t> shown_ids;
  std::string shown;
  std::function<void(std::int64_t)> on_token;
  if (stream_text) {
    on_token = [&](std::int64_t id) {
      shown_ids.push_back(id);
      std::string full = tok->decode(shown_ids);
      if (full.size() > shown.size()) {
        std::fwrite(full.data() + shown.size(), 1, full.size() - shown.size(), stdout);
        std::fflush(stdout);
      }
      shown = std::move(full);
    };
  }
  if (profile) {
    Profiler::instance().reset();
    Profiler::instance().enable(true);
  }
  // EOS stops text generation only; the ids path always produces exactly --gen tokens
  const std::int64_t eos = (!ids_mode && !no_eos && tok) ? tok->eos_id() : -1;
  const std::vector<std::int64_t> stream = gen > 0 ? model->generate(ids, gen, eos, samp, on_token) : ids;
  if (profile) Profiler::instance().enable(false);
  if (stream_text && gen > 0) std::fputc('\n', stdout);
  if (!logits_out.empty()) {
    std::vector<float> logits;
    model->forward(stream.data(), stream.size(), logits);
    const std::size_t V = model->config().vocab_size;
    std::ofstream f(logits_out, std::ios::binary);
    f.write(reinterpret_cast<const char*>(logits.data() + (stream.size() - 1) * V),
            static_cast<std::streamsize>(V * sizeof(float)));
  }
  const std::vector<std::int64_t> gen_ids(stream.begin() + static_cast<std::ptrdiff_t>(ids.size()), stream.end());
  if (show_ids) {
    std::fprintf(stderr, "prompt ids (%zu):", ids.size());
    for (auto t : ids) std::fprintf(stderr, " %lld", static_cast<long long>(t));
    std::fprintf(stderr, "\ngen ids (%zu):", gen_ids.size());
    for (auto t : gen_ids) std::fprintf(stderr, " %lld", static_cast<long long>(t));
    std::fprintf(stderr, "\n");
  }
  if (ids_out) {
    for (std::size_t i = 0; i < stream.size(); ++i)
      std::printf("%lld%s", static_cast<long long>(stream[i]), i + 1 < stream.size() ? " " : "\n");
  } else if (gen == 0) {
    std::printf("%s\n", tok->decode(gen_ids).c_str());
  }
  if (profile && gen > 0) print_profile(1);
  return 0;
}

int main(int argc, char** argv) {
  try {
    return run(argc, argv);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "mmfree-cli: %s\n", e.what());
    return 1;
  }
}
