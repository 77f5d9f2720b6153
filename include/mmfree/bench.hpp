// mmfree/bench.hpp -- generation timing harness (tok/s), as the reference's
// (cpp/include/mmfree/bench.hpp:17-40): greedy, EOS off, warmup + timed reps; prefill = time
// to the first token, decode tok/s = (n - 1) / (t_last - t_first).
#pragma once

#include "mmfree/model.hpp"

#include <cstddef>
#include <cstdint>
#include <vector>

namespace mmfree {

struct BenchOpts {
  std::size_t gen = 32;
  int warmup = 1;
  int reps = 3;
  bool profile = false;
};

struct BenchResult {
  double avg_prefill_s = 0;
  double avg_decode_tps = 0;
  double avg_overall_tps = 0;
  std::size_t prompt_tokens = 0;
  std::size_t gen_tokens = 0;
};

BenchResult run_bench(Model& model, const std::vector<std::int64_t>& ids, const BenchOpts& opts,
                      const char* blob_label, const char* mode_label, int frac);

void print_profile(int runs);

}  // namespace mmfree
