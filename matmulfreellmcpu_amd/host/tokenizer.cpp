// tokenizer.cpp -- BPE encode / decode over tokenizer.mmtok (see mmfree/tokenizer.hpp).
// Host code only: tokenization is a few microseconds per prompt.
#include "mmfree/tokenizer.hpp"

#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <set>
#include <stdexcept>
#include <utility>

namespace mmfree {
namespace {

const char kMagic[8] = {'M', 'M', 'T', 'O', 'K', '1', '\n', '\0'};
const std::string kSpace = "\xE2\x96\x81";  // U+2581, SentencePiece's visible space

// Cursor over the whole file in memory, with bounds checks.
struct Reader {
  const std::string& buf;
  std::size_t at = 0;
  const std::string& path;
  void need(std::size_t n) const {
    if (at + n > buf.size()) throw std::runtime_error("tokenizer: truncated " + path);
  }
  std::uint32_t u32() {
    need(4);
    const auto* p = reinterpret_cast<const unsigned char*>(buf.data() + at);
    at += 4;
    return static_cast<std::uint32_t>(p[0]) | static_cast<std::uint32_t>(p[1]) << 8 |
           static_cast<std::uint32_t>(p[2]) << 16 | static_cast<std::uint32_t>(p[3]) << 24;
  }
  std::string str() {
    const std::uint32_t n = u32();
    need(n);
    std::string s = buf.substr(at, n);
    at += n;
    return s;
  }
};

// Byte length of the UTF-8 unit starting at s[i] (the rule the reference applies: only the
// lead byte is inspected; a unit running past the end is a single byte).
std::size_t unit_len(const std::string& s, std::size_t i) {
  const unsigned char c = static_cast<unsigned char>(s[i]);
  const std::size_t n = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : c >= 0xC0 ? 2 : 1;
  return i + n > s.size() ? 1 : n;
}

}  // namespace

Tokenizer::Tokenizer(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("tokenizer: cannot open " + path);
  const std::string buf((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (buf.size() < 8 || std::memcmp(buf.data(), kMagic, 8) != 0)
    throw std::runtime_error("tokenizer: bad magic in " + path);
  Reader r{buf, 8, path};
  const std::uint32_t nv = r.u32(), nm = r.u32();
  bos_ = static_cast<std::int32_t>(r.u32());
  eos_ = static_cast<std::int32_t>(r.u32());
  unk_ = static_cast<std::int32_t>(r.u32());
  pieces_.reserve(nv);
  ids_.reserve(2 * static_cast<std::size_t>(nv));
  for (std::uint32_t i = 0; i < nv; ++i) {
    pieces_.push_back(r.str());
    ids_.emplace(pieces_.back(), static_cast<int>(i));  // first occurrence wins
  }
  rank_.reserve(2 * static_cast<std::size_t>(nm));
  for (std::uint32_t i = 0; i < nm; ++i) rank_.emplace(r.str(), static_cast<int>(i));
  for (int b = 0; b < 256; ++b) {
    char name[8];
    std::snprintf(name, sizeof(name), "<0x%02X>", b);
    const auto it = ids_.find(name);
    byte_id_[b] = it == ids_.end() ? -1 : it->second;
  }
}

std::vector<std::int64_t> Tokenizer::encode(const std::string& text, bool add_bos) const {
  std::vector<std::int64_t> out;
  if (add_bos) out.push_back(bos_);
  if (text.empty()) return out;
  std::string norm = kSpace;
  norm.reserve(text.size() * 3 + 3);
  for (const char ch : text) {
    if (ch == ' ') norm += kSpace;
    else norm.push_back(ch);
  }
  // symbols: one per UTF-8 unit, linked left to right; dead symbols have empty text
  std::vector<std::string> sym;
  for (std::size_t i = 0; i < norm.size();) {
    const std::size_t n = unit_len(norm, i);
    sym.push_back(norm.substr(i, n));
    i += n;
  }
  const int ns = static_cast<int>(sym.size());
  std::vector<int> nxt(ns), prv(ns), pair_rank(ns, -1);  // pair_rank[i]: rank of (i, nxt[i])
  for (int i = 0; i < ns; ++i) {
    prv[i] = i - 1;
    nxt[i] = i + 1 < ns ? i + 1 : -1;
  }
  // every mergeable adjacent pair, ordered by (rank, left position): the set always holds
  // exactly the current pairs, so its first element is the next merge
  std::set<std::pair<int, int>> cand;
  auto link = [&](int l) {
    if (l < 0 || nxt[l] < 0) return;
    const auto it = rank_.find(sym[l] + " " + sym[nxt[l]]);
    if (it == rank_.end()) return;
    pair_rank[l] = it->second;
    cand.emplace(it->second, l);
  };
  auto unlink = [&](int l) {
    if (l < 0 || pair_rank[l] < 0) return;
    cand.erase({pair_rank[l], l});
    pair_rank[l] = -1;
  };
  for (int i = 0; i + 1 < ns; ++i) link(i);
  while (!cand.empty()) {
    const int l = cand.begin()->second;
    const int r = nxt[l];
    unlink(prv[l]);
    unlink(l);
    unlink(r);
    sym[l] += sym[r];
    sym[r].clear();
    nxt[l] = nxt[r];
    if (nxt[l] >= 0) prv[nxt[l]] = l;
    link(prv[l]);
    link(l);
  }
  for (int i = 0; i >= 0; i = nxt[i]) {
    const auto it = ids_.find(sym[i]);
    if (it != ids_.end()) {
      out.push_back(it->second);
    } else {
      for (const unsigned char c : sym[i]) out.push_back(byte_id_[c]);
    }
  }
  return out;
}

std::string Tokenizer::decode(const std::vector<std::int64_t>& ids, bool skip_special) const {
  std::string s;
  for (const std::int64_t id : ids) {
    if (id < 0 || static_cast<std::size_t>(id) >= pieces_.size()) continue;
    if (skip_special && (id == bos_ || id == eos_ || id == unk_)) continue;
    const std::string& p = pieces_[static_cast<std::size_t>(id)];
    if (p.size() == 6 && p.compare(0, 3, "<0x") == 0 && p[5] == '>') {
      s.push_back(static_cast<char>(std::strtol(p.substr(3, 2).c_str(), nullptr, 16)));
      continue;
    }
    for (std::size_t i = 0; i < p.size();) {
      if (p.compare(i, kSpace.size(), kSpace) == 0) {
        s.push_back(' ');
        i += kSpace.size();
      } else {
        s.push_back(p[i++]);
      }
    }
  }
  if (!s.empty() && s[0] == ' ') s.erase(0, 1);
  return s;
}

}  // namespace mmfree
