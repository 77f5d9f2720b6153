// mmfree/profile.hpp -- wall-clock op profiler (off by default).
// Same public interface as the reference's (cpp/include/mmfree/profile.hpp:20-73). Model
// wraps its GPU calls in ScopedTimers (labels "generate", "prefill", "decode", "forward",
// "sample"); the per-kernel breakdown comes from rocprofv3 or mmf_model_time_decode /
// mmf_model_time_prefill.
#pragma once

#include <chrono>
#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace mmfree {

class Profiler {
 public:
  struct Entry {
    std::string label;
    std::uint64_t ns = 0;
    std::uint64_t count = 0;
  };
  static Profiler& instance();
  void enable(bool on) { enabled_ = on; }
  bool enabled() const { return enabled_; }
  void reset();
  void add(const char* label, std::uint64_t ns);
  // entries by total time, largest first (first-seen order among equal totals)
  std::vector<Entry> sorted() const;
  std::uint64_t total_ns() const { return total_; }

 private:
  bool enabled_ = false;
  std::vector<Entry> entries_;                  // in first-seen order
  std::unordered_map<std::string, std::size_t> slot_;  // label -> index into entries_
  std::uint64_t total_ = 0;
};

class ScopedTimer {
 public:
  explicit ScopedTimer(const char* label) : label_(label), on_(Profiler::instance().enabled()) {
    if (on_) t0_ = std::chrono::steady_clock::now();
  }
  ~ScopedTimer() {
    if (on_)
      Profiler::instance().add(label_, static_cast<std::uint64_t>(
                                           std::chrono::duration_cast<std::chrono::nanoseconds>(
                                               std::chrono::steady_clock::now() - t0_)
                                               .count()));
  }
  ScopedTimer(const ScopedTimer&) = delete;
  ScopedTimer& operator=(const ScopedTimer&) = delete;

 private:
  const char* label_;
  bool on_;
  std::chrono::steady_clock::time_point t0_;
};

#define MMFREE_PROFILE_CONCAT_(a, b) a##b
#define MMFREE_PROFILE_CONCAT(a, b) MMFREE_PROFILE_CONCAT_(a, b)
#define MMFREE_PROFILE(name) ::mmfree::ScopedTimer MMFREE_PROFILE_CONCAT(mmfree_timer_, __LINE__)(name)

}  // namespace mmfree
