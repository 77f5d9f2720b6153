// profile.cpp -- the op profiler's table and the generation timing harness.
//
// Output formats follow the reference's (cpp/src/util/bench.cpp:16-120): scripts that parse
// `mmfree-cli --bench` and `--profile` read the same lines. The op labels are this engine's
// (Model feeds the device time of its kernels per op: norm+quant, matmul, gate+scan,
// lm_head, embed; host sampling as sample).
#include "mmfree/profile.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <numeric>

#include "mmfree/bench.hpp"
#include "mmfree_hip.h"

namespace mmfree {

Profiler& Profiler::instance() {
  static Profiler p;
  return p;
}

void Profiler::reset() {
  entries_.clear();
  slot_.clear();
  total_ = 0;
}

void Profiler::add(const char* label, std::uint64_t ns) {
  const auto ins = slot_.emplace(label, entries_.size());
  if (ins.second) entries_.push_back(Entry{label, 0, 0});
  Entry& e = entries_[ins.first->second];
  e.ns += ns;
  e.count += 1;
  total_ += ns;
}

std::vector<Profiler::Entry> Profiler::sorted() const {
  std::vector<std::size_t> order(entries_.size());
  std::iota(order.begin(), order.end(), std::size_t{0});
  std::stable_sort(order.begin(), order.end(),
                   [this](std::size_t a, std::size_t b) { return entries_[a].ns > entries_[b].ns; });
  std::vector<Entry> out;
  out.reserve(order.size());
  for (std::size_t i : order) out.push_back(entries_[i]);
  return out;
}

void print_profile(int runs) {
  const Profiler& prof = Profiler::instance();
  const double total_ms = static_cast<double>(prof.total_ns()) / 1e6;
  if (total_ms <= 0.0 || runs <= 0) {
    std::printf("\nprofile: no samples\n");
    return;
  }
  std::printf("\nop profile (%d run%s, instrumented ops only):\n", runs, runs == 1 ? "" : "s");
  std::printf("  %-12s %10s %8s %10s %10s\n", "op", "ms/run", "%", "calls/run", "us/call");
  double matmul_ms = 0.0;
  for (const Profiler::Entry& e : prof.sorted()) {
    const double ms = static_cast<double>(e.ns) / 1e6;
    std::printf("  %-12s %10.2f %7.1f%% %10.1f %10.2f\n", e.label.c_str(), ms / runs, 100.0 * ms / total_ms,
                static_cast<double>(e.count) / runs, e.count ? static_cast<double>(e.ns) / 1e3 / e.count : 0.0);
    if (e.label == "matmul" || e.label == "lm_head") matmul_ms += ms;
  }
  std::printf("  %-12s %10.2f %7.1f%%\n", "TOTAL", total_ms / runs, 100.0);
  std::printf("\n  matmul (incl lm_head): %.1f%% of profiled time;  other ops: %.1f%%\n",
              100.0 * matmul_ms / total_ms, 100.0 * (total_ms - matmul_ms) / total_ms);
}

namespace {

// One timed greedy generation with EOS off: the token callback stamps the first token (the
// end of the prefill) and the last one.
struct GenTiming {
  double prefill_s = 0, decode_s = 0, total_s = 0;
  std::size_t tokens = 0;
  double decode_tps() const { return tokens > 1 && decode_s > 0 ? (tokens - 1) / decode_s : 0.0; }
  double overall_tps() const { return total_s > 0 ? tokens / total_s : 0.0; }
};

GenTiming time_generation(Model& model, const std::vector<std::int64_t>& ids, std::size_t gen) {
  using clock = std::chrono::steady_clock;
  const clock::time_point start = clock::now();
  clock::time_point first = start, last = start;
  GenTiming t;
  model.generate(ids, gen, -1, Sampling{}, [&](std::int64_t) {
    last = clock::now();
    if (t.tokens++ == 0) first = last;
  });
  auto secs = [](clock::duration d) { return std::chrono::duration<double>(d).count(); };
  t.prefill_s = secs(first - start);
  t.decode_s = t.tokens > 1 ? secs(last - first) : 0.0;
  t.total_s = secs(last - start);
  return t;
}

}  // namespace

// The reference harness's protocol (bench.cpp:42-112): `warmup` untimed runs, then `reps`
// timed ones; prefill = time to the first token, decode tok/s = (n - 1) / (t_last - t_first),
// averaged over the runs. The profile covers the timed runs only. The "threads:" line counts
// host threads driving the engine (one); the GPU is named on the "device:" line.
BenchResult run_bench(Model& model, const std::vector<std::int64_t>& ids, const BenchOpts& opts,
                      const char* blob_label, const char* mode_label, int frac) {
  char dev[256] = "?";
  int cus = 0;
  mmf_device_info(model.context(), dev, sizeof dev, &cus);
  std::printf("mmfree-cli benchmark\n");
  std::printf("  blob:          %s\n", blob_label);
  std::printf("  mode:          %s (frac=%d)\n", mode_label, frac);
  std::printf("  threads:       %d\n", 1);
  std::printf("  device:        %s, %d CUs\n", dev, cus);
  std::printf("  prompt tokens: %zu\n", ids.size());
  std::printf("  gen tokens:    %zu\n", opts.gen);
  std::printf("  warmup/reps:   %d/%d\n\n", opts.warmup, opts.reps);
  for (int i = 0; i < opts.warmup; ++i) time_generation(model, ids, opts.gen);
  Profiler& prof = Profiler::instance();
  if (opts.profile) {
    prof.reset();
    prof.enable(true);
  }
  std::vector<GenTiming> runs;
  for (int i = 0; i < opts.reps; ++i) {
    runs.push_back(time_generation(model, ids, opts.gen));
    const GenTiming& r = runs.back();
    std::printf("  run %d: prefill %7.1f ms   decode %8.2f tok/s   overall %8.2f tok/s\n", i + 1, r.prefill_s * 1e3,
                r.decode_tps(), r.overall_tps());
  }
  const double n = opts.reps > 0 ? opts.reps : 1;
  double prefill = 0, decode = 0, total = 0;
  for (const GenTiming& r : runs) {
    prefill += r.prefill_s / n;
    decode += r.decode_tps() / n;
    total += r.total_s / n;
  }
  const double overall = total > 0 ? opts.gen / total : 0.0;
  std::printf("\n  avg prefill: %7.1f ms  (%.2f tok/s over %zu prompt tokens)\n", prefill * 1e3,
              prefill > 0 ? ids.size() / prefill : 0.0, ids.size());
  std::printf("  avg decode:  %8.2f tok/s\n", decode);
  std::printf("  avg overall: %8.2f tok/s  (%zu gen tokens / %.3f s)\n", overall, opts.gen, total);
  if (opts.profile) {
    prof.enable(false);
    print_profile(opts.reps);
  }
  return {prefill, decode, overall, ids.size(), opts.gen};
}

}  // namespace mmfree
