// tok_check.cpp -- drives mmfree::Tokenizer (libmmfree.so) for tests/test_tokenizer.py.
//   tok_check TOKENIZER REQUESTS RESULTS
// REQUESTS: records of u8 kind, then kind 0 (encode): u32 n + n text bytes; kind 1
// (decode): u32 n + n int64 ids. RESULTS, per record: encode -> ids with BOS, ids without
// (each u32 n + n int64); decode -> text skipping specials, text keeping them (u32 n + bytes).
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "mmfree/tokenizer.hpp"

namespace {
std::uint32_t u32(const std::string& b, std::size_t& at) {
  std::uint32_t v = 0;
  for (int i = 0; i < 4; ++i) v |= static_cast<std::uint32_t>(static_cast<unsigned char>(b[at + i])) << (8 * i);
  at += 4;
  return v;
}
void put_u32(std::string& o, std::uint32_t v) {
  for (int i = 0; i < 4; ++i) o.push_back(static_cast<char>((v >> (8 * i)) & 0xFF));
}
void put_ids(std::string& o, const std::vector<std::int64_t>& ids) {
  put_u32(o, static_cast<std::uint32_t>(ids.size()));
  o.append(reinterpret_cast<const char*>(ids.data()), ids.size() * sizeof(std::int64_t));
}
}  // namespace

int main(int argc, char** argv) {
  if (argc != 4) return 2;
  const mmfree::Tokenizer tok(argv[1]);
  std::ifstream in(argv[2], std::ios::binary);
  const std::string req((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  std::string out;
  for (std::size_t at = 0; at < req.size();) {
    const int kind = static_cast<unsigned char>(req[at++]);
    const std::uint32_t n = u32(req, at);
    if (kind == 0) {
      const std::string text = req.substr(at, n);
      at += n;
      put_ids(out, tok.encode(text, true));
      put_ids(out, tok.encode(text, false));
    } else {
      std::vector<std::int64_t> ids(n);
      for (std::uint32_t i = 0; i < n; ++i) {
        std::uint64_t v = 0;
        for (int b = 0; b < 8; ++b) v |= static_cast<std::uint64_t>(static_cast<unsigned char>(req[at + 8 * i + b])) << (8 * b);
        ids[i] = static_cast<std::int64_t>(v);
      }
      at += 8 * static_cast<std::size_t>(n);
      for (const bool skip : {true, false}) {
        const std::string s = tok.decode(ids, skip);
        put_u32(out, static_cast<std::uint32_t>(s.size()));
        out += s;
      }
    }
  }
  std::ofstream(argv[3], std::ios::binary) << out;
  return 0;
}
