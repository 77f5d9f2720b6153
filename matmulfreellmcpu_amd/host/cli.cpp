// cli.cpp -- mmfree-cli on the MI355X. The command-line contract is the reference CLI's
// (cpp/app/main.cpp:14-40 flags and defaults, :95-248 behaviour); the model runs on the GPU.
//
// Contract, in the order a run applies it:
//   1. Arguments: every "--flag" of the table below; a flag that takes a value consumes the
//      next argument (or "" when there is none); numbers parse like atoi/atof/strtoull (junk
//      reads as 0). Any other argument starting with '-' prints "unknown arg: X" on stderr
//      and exits 2. A bare argument is the prompt (the last one wins).
//   2. --decode-ids: print the tokenizer's decoding of the ids plus '\n', exit 0; nothing
//      else is read.
//   3. Prompt ids: --ids (ids in, ids out, no tokenizer, no EOS stop), else the prompt text,
//      else stdin (lines joined by '\n', trailing newlines and spaces cut), else under
//      --bench the fixed sentence below; text is encoded with BOS unless --no-bos. No ids:
//      "no input (...)" on stderr, exit 2.
//   4. The weights and the model are loaded only when something runs them (--gen > 0,
//      --logits-out or --bench). --mode fixed (default) is Q5.10, int8 is per-row int8
//      absmax (an addition), any other value is float.
//   5. --bench: the timing harness (--gen must be > 0, else exit 2), then exit 0.
//   6. Generation: greedy unless --temp > 0 (seeded by --seed, else randomly); text mode
//      streams the decoded text as tokens arrive and stops at the tokenizer's EOS unless
//      --no-eos; ids mode always makes exactly --gen tokens.
//   7. Outputs: --logits-out writes the last position's logits of the full stream (raw
//      float32); --show-ids prints the prompt and generated ids on stderr; ids mode or
//      --print-ids prints the full id stream; --profile prints the op profile.
// Additions: --mode int8, --device N (or MMFREE_DEVICE). Errors thrown by the engine print
// "mmfree-cli: <message>" and exit 1.
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <fstream>
#include <functional>
#include <iostream>
#include <iterator>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "mmfree/bench.hpp"
#include "mmfree/model.hpp"
#include "mmfree/profile.hpp"
#include "mmfree/tokenizer.hpp"
#include "mmfree/weights.hpp"

namespace {

using mmfree::ActQuant;

constexpr const char* kBenchPrompt = "The quick brown fox jumps over the lazy dog.";

struct Options {
  std::string blob = "model.mmfree";
  std::string tokenizer;  // empty: tokenizer.mmtok in the blob's directory
  std::string mode = "fixed";
  std::string ids;        // --ids
  std::string decode;     // --decode-ids
  std::string logits_out;
  std::string prompt;
  bool has_prompt = false;
  int frac = 10;
  std::size_t gen = 32;
  float temp = 0.0f;
  int top_k = 0;
  unsigned long long seed = 0;
  bool has_seed = false;
  bool no_bos = false, no_eos = false, print_ids = false, show_ids = false;
  bool bench = false, profile = false;
  int warmup = 1, reps = 3;
};

// One row per flag: how its value is stored. Switches take no value.
struct FlagSpec {
  const char* name;
  std::function<void(Options&, const std::string&)> set;
  bool takes_value;
};

const std::vector<FlagSpec>& flag_table() {
  static const std::vector<FlagSpec> table = {
      {"--blob", [](Options& o, const std::string& v) { o.blob = v; }, true},
      {"--tokenizer", [](Options& o, const std::string& v) { o.tokenizer = v; }, true},
      {"--mode", [](Options& o, const std::string& v) { o.mode = v; }, true},
      {"--frac", [](Options& o, const std::string& v) { o.frac = std::atoi(v.c_str()); }, true},
      {"--gen", [](Options& o, const std::string& v) { o.gen = static_cast<std::size_t>(std::atoll(v.c_str())); },
       true},
      {"--temp", [](Options& o, const std::string& v) { o.temp = static_cast<float>(std::atof(v.c_str())); }, true},
      {"--temperature", [](Options& o, const std::string& v) { o.temp = static_cast<float>(std::atof(v.c_str())); },
       true},
      {"--top-k", [](Options& o, const std::string& v) { o.top_k = std::atoi(v.c_str()); }, true},
      {"--seed",
       [](Options& o, const std::string& v) {
         o.seed = std::strtoull(v.c_str(), nullptr, 10);
         o.has_seed = true;
       },
       true},
      {"--ids", [](Options& o, const std::string& v) { o.ids = v; }, true},
      {"--decode-ids", [](Options& o, const std::string& v) { o.decode = v; }, true},
      {"--logits-out", [](Options& o, const std::string& v) { o.logits_out = v; }, true},
      {"--warmup", [](Options& o, const std::string& v) { o.warmup = std::atoi(v.c_str()); }, true},
      {"--reps", [](Options& o, const std::string& v) { o.reps = std::atoi(v.c_str()); }, true},
      {"--device", [](Options&, const std::string& v) { setenv("MMFREE_DEVICE", v.c_str(), 1); }, true},
      {"--no-bos", [](Options& o, const std::string&) { o.no_bos = true; }, false},
      {"--no-eos", [](Options& o, const std::string&) { o.no_eos = true; }, false},
      {"--print-ids", [](Options& o, const std::string&) { o.print_ids = true; }, false},
      {"--show-ids", [](Options& o, const std::string&) { o.show_ids = true; }, false},
      {"--bench", [](Options& o, const std::string&) { o.bench = true; }, false},
      {"--profile", [](Options& o, const std::string&) { o.profile = true; }, false},
  };
  return table;
}

// Returns false (after the message) on an unknown flag.
bool parse_args(int argc, char** argv, Options& o) {
  const auto& table = flag_table();
  for (int a = 1; a < argc; ++a) {
    const std::string arg = argv[a];
    const FlagSpec* spec = nullptr;
    for (const auto& f : table)
      if (arg == f.name) spec = &f;
    if (spec) {
      std::string value;
      if (spec->takes_value && a + 1 < argc) value = argv[++a];
      spec->set(o, value);
    } else if (!arg.empty() && arg[0] == '-') {
      std::fprintf(stderr, "unknown arg: %s\n", arg.c_str());
      return false;
    } else {
      o.prompt = arg;
      o.has_prompt = true;
    }
  }
  if (o.tokenizer.empty()) {
    const std::size_t cut = o.blob.rfind('/');
    o.tokenizer = (cut == std::string::npos ? std::string() : o.blob.substr(0, cut + 1)) + "tokenizer.mmtok";
  }
  return true;
}

// Integers of a list such as "1,415,310" (any non-digit separates; a '-' directly before
// digits makes them negative).
std::vector<std::int64_t> id_list(const std::string& s) {
  std::vector<std::int64_t> out;
  std::size_t i = 0;
  while (i < s.size()) {
    const bool neg = s[i] == '-' && i + 1 < s.size() && std::isdigit(static_cast<unsigned char>(s[i + 1]));
    if (!neg && !std::isdigit(static_cast<unsigned char>(s[i]))) {
      ++i;
      continue;
    }
    std::size_t end = i + (neg ? 1 : 0);
    while (end < s.size() && std::isdigit(static_cast<unsigned char>(s[end]))) ++end;
    out.push_back(std::stoll(s.substr(i, end - i)));
    i = end;
  }
  return out;
}

std::string read_stdin_prompt() {
  std::string text((std::istreambuf_iterator<char>(std::cin)), std::istreambuf_iterator<char>());
  if (!text.empty() && text.back() != '\n') text.push_back('\n');  // every line ends in '\n'
  std::size_t keep = text.size();
  while (keep > 0 && (text[keep - 1] == '\n' || text[keep - 1] == ' ')) --keep;
  return text.substr(0, keep);
}

ActQuant quant_of(const std::string& mode) {
  if (mode == "fixed") return ActQuant::FixedQ510;
  if (mode == "int8") return ActQuant::Int8Absmax;
  return ActQuant::Float;
}

// Streams generated text: each token re-decodes everything generated so far and prints the
// bytes beyond what is already out (single-token decoding is not prefix-safe for BPE: the
// leading-space rule and byte-fallback sequences span tokens).
class TextStream {
 public:
  explicit TextStream(const mmfree::Tokenizer& tok) : tok_(tok) {}
  void push(std::int64_t id) {
    ids_.push_back(id);
    std::string now = tok_.decode(ids_);
    if (now.size() > printed_) {
      std::fwrite(now.data() + printed_, 1, now.size() - printed_, stdout);
      std::fflush(stdout);
    }
    printed_ = now.size();
  }

 private:
  const mmfree::Tokenizer& tok_;
  std::vector<std::int64_t> ids_;
  std::size_t printed_ = 0;
};

void print_id_line(std::FILE* f, const char* what, const std::vector<std::int64_t>& v) {
  std::fprintf(f, "%s (%zu):", what, v.size());
  for (std::int64_t t : v) std::fprintf(f, " %lld", static_cast<long long>(t));
  std::fprintf(f, "\n");
}

void write_last_logits(mmfree::Model& model, const std::vector<std::int64_t>& stream, const std::string& path) {
  std::vector<float> logits;
  model.forward(stream.data(), stream.size(), logits);
  const std::size_t V = model.config().vocab_size;
  std::ofstream f(path, std::ios::binary);
  f.write(reinterpret_cast<const char*>(logits.data() + (stream.size() - 1) * V),
          static_cast<std::streamsize>(V * sizeof(float)));
}

int run(int argc, char** argv) {
  Options o;
  if (!parse_args(argc, argv, o)) return 2;

  if (!o.decode.empty()) {
    const mmfree::Tokenizer tok(o.tokenizer);
    std::printf("%s\n", tok.decode(id_list(o.decode)).c_str());
    return 0;
  }

  // ids in means ids out; text in needs the tokenizer both ways
  const bool ids_in = !o.ids.empty();
  const bool ids_out = ids_in || o.print_ids;
  std::unique_ptr<mmfree::Tokenizer> tok;
  if (!ids_in) tok = std::make_unique<mmfree::Tokenizer>(o.tokenizer);

  std::vector<std::int64_t> prompt_ids;
  if (ids_in) {
    prompt_ids = id_list(o.ids);
  } else {
    const std::string text = o.has_prompt ? o.prompt : (o.bench ? std::string(kBenchPrompt) : read_stdin_prompt());
    prompt_ids = tok->encode(text, !o.no_bos);
  }
  if (prompt_ids.empty()) {
    std::fprintf(stderr, "no input (pass a prompt, --ids, or pipe via stdin)\n");
    return 2;
  }

  std::unique_ptr<mmfree::Weights> weights;
  std::unique_ptr<mmfree::Model> model;
  if (o.gen > 0 || !o.logits_out.empty() || o.bench) {
    weights = std::make_unique<mmfree::Weights>(o.blob);
    model = std::make_unique<mmfree::Model>(*weights, quant_of(o.mode), o.frac);
  }

  if (o.bench) {
    if (o.gen == 0) {
      std::fprintf(stderr, "--bench needs --gen > 0\n");
      return 2;
    }
    mmfree::BenchOpts bo;
    bo.gen = o.gen;
    bo.warmup = o.warmup;
    bo.reps = o.reps;
    bo.profile = o.profile;
    mmfree::run_bench(*model, prompt_ids, bo, o.blob.c_str(), o.mode.c_str(), o.frac);
    return 0;
  }

  mmfree::Sampling samp;
  samp.temperature = o.temp;
  samp.top_k = o.top_k;
  samp.seed = (o.temp > 0.0f && !o.has_seed) ? std::random_device{}() : o.seed;

  std::unique_ptr<TextStream> text;
  std::function<void(std::int64_t)> on_token;
  if (!ids_out) {
    text = std::make_unique<TextStream>(*tok);
    on_token = [&](std::int64_t id) { text->push(id); };
  }
  const std::int64_t eos = (tok && !ids_in && !o.no_eos) ? tok->eos_id() : -1;

  mmfree::Profiler& prof = mmfree::Profiler::instance();
  if (o.profile) {
    prof.reset();
    prof.enable(true);
  }
  std::vector<std::int64_t> stream = prompt_ids;
  if (o.gen > 0) stream = model->generate(prompt_ids, o.gen, eos, samp, on_token);
  if (o.profile) prof.enable(false);
  if (text && o.gen > 0) std::fputc('\n', stdout);

  if (!o.logits_out.empty()) write_last_logits(*model, stream, o.logits_out);
  const std::vector<std::int64_t> generated(stream.begin() + static_cast<std::ptrdiff_t>(prompt_ids.size()),
                                            stream.end());
  if (o.show_ids) {
    print_id_line(stderr, "prompt ids", prompt_ids);
    print_id_line(stderr, "gen ids", generated);
  }
  if (ids_out) {
    std::string line;
    for (std::size_t i = 0; i < stream.size(); ++i) line += (i ? " " : "") + std::to_string(stream[i]);
    std::printf("%s\n", line.c_str());
  } else if (o.gen == 0) {
    std::printf("%s\n", tok->decode(generated).c_str());
  }
  if (o.profile && o.gen > 0) mmfree::print_profile(1);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    return run(argc, argv);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "mmfree-cli: %s\n", e.what());
    return 1;
  }
}
