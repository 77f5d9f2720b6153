// profile.cpp -- Profiler accumulation and the generation timing harness.
#include "mmfree/profile.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>

#include "mmfree/bench.hpp"
#include "mmfree_hip.h"

namespace mmfree {

Profiler& Profiler::instance() {
  static Profiler p;
  return p;
}

void Profiler::add(const char* label, std::uint64_t ns) {
  for (auto& e : entries_)
    if (e.label == label) {
      e.ns += ns;
      ++e.count;
      return;
    }
  entries_.push_back({label, ns, 1});
}

std::vector<Profiler::Entry> Profiler::sorted() const {
  std::vector<Entry> v = entries_;
  std::sort(v.begin(), v.end(), [](const Entry& a, const Entry& b) { return a.ns > b.ns; });
  return v;
}

std::uint64_t Profiler::total_ns() const {
  std::uint64_t t = 0;
  for (const auto& e : entries_) t += e.ns;
  return t;
}

void print_profile(int runs) {
  auto& prof = Profiler::instance();
  const double total_ms = prof.total_ns() / 1e6;
  if (total_ms <= 0.0 || runs <= 0) {
    std::printf("\nprofile: no samples\n");
    return;
  }
  std::printf("\nop profile (%d run%s, instrumented host calls):\n", runs, runs == 1 ? "" : "s");
  std::printf("  %-12s %10s %8s %10s %10s\n", "op", "ms/run", "%", "calls/run", "us/call");
  for (const auto& e : prof.sorted()) {
    const double ms = e.ns / 1e6;
    std::printf("  %-12s %10.2f %7.1f%% %10.1f %10.2f\n", e.label.c_str(), ms / runs, 100.0 * ms / total_ms,
                static_cast<double>(e.count) / runs, e.count ? (e.ns / 1e3) / e.count : 0.0);
  }
  std::printf("  %-12s %10.2f %7.1f%%\n", "TOTAL", total_ms / runs, 100.0);
}

// Same timing protocol as the reference harness (cpp/src/util/bench.cpp:42-112): greedy,
// EOS off, `warmup` untimed runs, then `reps` timed runs; the on_token callback stamps the
// first (end of prefill) and last token; decode tok/s = (n - 1) / (t_last - t_first).
BenchResult run_bench(Model& model, const std::vector<std::int64_t>& ids, const BenchOpts& opts,
                      const char* blob_label, const char* mode_label, int frac) {
  using clk = std::chrono::steady_clock;
  auto secs = [](clk::duration d) { return std::chrono::duration<double>(d).count(); };
  struct Run {
    double prefill_s, decode_s, total_s;
    std::size_t n;
  };
  auto run_once = [&]() -> Run {
    const clk::time_point t0 = clk::now();
    clk::time_point first = t0, last = t0;
    std::size_t n = 0;
    model.generate(ids, opts.gen, -1, Sampling{}, [&](std::int64_t) {
      const clk::time_point now = clk::now();
      if (n == 0) first = now;
      last = now;
      ++n;
    });
    return {secs(first - t0), n > 1 ? secs(last - first) : 0.0, secs(last - t0), n};
  };
  char dev[256] = "?";
  int cus = 0;
  mmf_device_info(model.context(), dev, sizeof dev, &cus);
  std::printf("mmfree-cli benchmark\n");
  std::printf("  blob:          %s\n", blob_label);
  std::printf("  mode:          %s (frac=%d)\n", mode_label, frac);
  std::printf("  device:        %s, %d CUs\n", dev, cus);
  std::printf("  prompt tokens: %zu\n", ids.size());
  std::printf("  gen tokens:    %zu\n", opts.gen);
  std::printf("  warmup/reps:   %d/%d\n\n", opts.warmup, opts.reps);
  for (int i = 0; i < opts.warmup; ++i) run_once();
  if (opts.profile) {
    Profiler::instance().reset();
    Profiler::instance().enable(true);
  }
  double sp = 0, st = 0, sd = 0;
  for (int i = 0; i < opts.reps; ++i) {
    const Run r = run_once();
    const double dec = (r.n > 1 && r.decode_s > 0) ? (r.n - 1) / r.decode_s : 0.0;
    const double all = r.total_s > 0 ? r.n / r.total_s : 0.0;
    std::printf("  run %d: prefill %7.1f ms   decode %8.2f tok/s   overall %8.2f tok/s\n", i + 1, r.prefill_s * 1e3,
                dec, all);
    sp += r.prefill_s;
    st += r.total_s;
    sd += dec;
  }
  const double n = opts.reps > 0 ? opts.reps : 1;
  const double avg_prefill = sp / n, avg_dec = sd / n, avg_total = st / n;
  const double overall = avg_total > 0 ? opts.gen / avg_total : 0.0;
  std::printf("\n  avg prefill: %7.1f ms  (%.2f tok/s over %zu prompt tokens)\n", avg_prefill * 1e3,
              avg_prefill > 0 ? ids.size() / avg_prefill : 0.0, ids.size());
  std::printf("  avg decode:  %8.2f tok/s\n", avg_dec);
  std::printf("  avg overall: %8.2f tok/s  (%zu gen tokens / %.3f s)\n", overall, opts.gen, avg_total);
  if (opts.profile) {
    Profiler::instance().enable(false);
    print_profile(opts.reps);
  }
  return {avg_prefill, avg_dec, overall, ids.size(), opts.gen};
}

}  // namespace mmfree
