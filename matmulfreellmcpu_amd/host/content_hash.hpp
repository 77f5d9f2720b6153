// content_hash.hpp -- 64-bit hash of a byte range, for caching resident projections by
// their weights (a caller may refill the same host buffer with other weights).
//
// Eight bytes per step, each word mixed by a multiply and an xor-shift; the length is mixed
// in at the end. A cache key, not a cryptographic digest: the keys also carry the buffer's
// address and shape.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>

namespace mmfree {
namespace detail {

inline std::uint64_t content_hash(const void* p, std::size_t n, std::uint64_t h = 0x243F6A8885A308D3ull) {
  const unsigned char* b = static_cast<const unsigned char*>(p);
  constexpr std::uint64_t kMul = 0x9E3779B97F4A7C15ull;
  std::size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    std::uint64_t w;
    std::memcpy(&w, b + i, 8);
    h = (h ^ w) * kMul;
    h ^= h >> 31;
  }
  std::uint64_t last = 0;
  for (std::size_t j = 0; i + j < n; ++j) last |= static_cast<std::uint64_t>(b[i + j]) << (8 * j);
  h = (h ^ last ^ (static_cast<std::uint64_t>(n) << 3)) * kMul;
  return h ^ (h >> 29);
}

}  // namespace detail
}  // namespace mmfree
