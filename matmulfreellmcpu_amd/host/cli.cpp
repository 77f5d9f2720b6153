// cli.cpp -- mmfree-cli on the MI355X: the reference CLI's flags and outputs
// (cpp/app/main.cpp:14-40, 95-124), model compute on the GPU.
//
//   --blob PATH --tokenizer PATH --mode float|fixed|int8 --frac N --gen N --temp T --top-k K
//   --seed N --ids a,b,c --decode-ids a,b,c --no-bos --no-eos --print-ids --show-ids
//   --logits-out PATH --bench --warmup N --reps N --profile
// Additions: --mode int8 (per-row int8 absmax activations), --device N (also MMFREE_DEVICE).
// Unknown flags exit 2, as in the reference. Text prompts and --decode-ids need the
// tokenizer (tokenizer.mmtok), which this engine does not read: they exit 2 with a message;
// the validation path (--ids in, ids out) is complete.
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <fstream>
#include <functional>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "mmfree/bench.hpp"
#include "mmfree/model.hpp"
#include "mmfree/profile.hpp"
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

static int run(int argc, char** argv) {
  std::string blob = "model.mmfree", tokenizer_path, mode = "fixed", ids_arg, logits_out, decode_arg;
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
      have_prompt = true;
    }
  }
  (void)no_bos;
  (void)no_eos;
  (void)tokenizer_path;
  if (!decode_arg.empty() || ids_arg.empty()) {
    std::fprintf(stderr, "%s\n",
                 have_prompt || !decode_arg.empty()
                     ? "text prompts and --decode-ids need the tokenizer (tokenizer.mmtok), which this engine does "
                       "not read; pass token ids with --ids"
                     : "no input (pass --ids a,b,c)");
    return 2;
  }
  const std::vector<std::int64_t> ids = parse_ids(ids_arg);
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
  if (profile) {
    Profiler::instance().reset();
    Profiler::instance().enable(true);
  }
  // ids mode: no EOS stop, exactly --gen tokens (the reference's validation path)
  const std::vector<std::int64_t> stream = gen > 0 ? model->generate(ids, gen, -1, samp) : ids;
  if (profile) Profiler::instance().enable(false);
  if (!logits_out.empty()) {
    std::vector<float> logits;
    model->forward(stream.data(), stream.size(), logits);
    const std::size_t V = model->config().vocab_size;
    std::ofstream f(logits_out, std::ios::binary);
    f.write(reinterpret_cast<const char*>(logits.data() + (stream.size() - 1) * V),
            static_cast<std::streamsize>(V * sizeof(float)));
  }
  if (show_ids) {
    std::fprintf(stderr, "prompt ids (%zu):", ids.size());
    for (auto t : ids) std::fprintf(stderr, " %lld", static_cast<long long>(t));
    std::fprintf(stderr, "\ngen ids (%zu):", stream.size() - ids.size());
    for (std::size_t i = ids.size(); i < stream.size(); ++i) std::fprintf(stderr, " %lld", static_cast<long long>(stream[i]));
    std::fprintf(stderr, "\n");
  }
  (void)print_ids;  // ids mode always prints the id stream
  for (std::size_t i = 0; i < stream.size(); ++i)
    std::printf("%lld%s", static_cast<long long>(stream[i]), i + 1 < stream.size() ? " " : "\n");
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
