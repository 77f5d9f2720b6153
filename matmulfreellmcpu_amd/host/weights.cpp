// weights.cpp -- mmap'd, validated reader of the MMFREE1 weight blob.
//
// Format (the reference's, cpp/src/io/weights.cpp:3-8 and tools/provision.py:126-163):
//   "MMFREE1\n" | u64 LE header_len | JSON {"config": {...}, "tensors": {name: {dtype,
//   shape, offset, nbytes}}} | zero pad to 64 | data section (offsets relative to it).
#include "mmfree/weights.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <utility>

namespace mmfree {
namespace {

// A small JSON value and recursive-descent reader (objects keep their key order).
struct JVal {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<JVal> items;
  std::vector<std::pair<std::string, JVal>> fields;

  const JVal* at(const std::string& k) const {
    for (const auto& f : fields)
      if (f.first == k) return &f.second;
    return nullptr;
  }
};

class JReader {
 public:
  JReader(const char* b, const char* e) : p_(b), e_(e) {}

  JVal document() {
    JVal v = value();
    skip();
    if (p_ != e_) err("trailing characters after the header object");
    return v;
  }

 private:
  [[noreturn]] void err(const std::string& m) { throw std::runtime_error("weights: header JSON: " + m); }
  void skip() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
  }
  bool eat(char c) {
    skip();
    if (p_ < e_ && *p_ == c) {
      ++p_;
      return true;
    }
    return false;
  }
  void need(char c) {
    if (!eat(c)) err(std::string("expected '") + c + "'");
  }
  JVal value() {
    skip();
    if (p_ >= e_) err("unexpected end");
    JVal v;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = JVal::Object;
      if (eat('}')) return v;
      do {
        skip();
        std::string k = text();
        need(':');
        v.fields.emplace_back(std::move(k), value());
      } while (eat(','));
      need('}');
    } else if (c == '[') {
      ++p_;
      v.kind = JVal::Array;
      if (eat(']')) return v;
      do v.items.push_back(value());
      while (eat(','));
      need(']');
    } else if (c == '"') {
      v.kind = JVal::String;
      v.str = text();
    } else if (word("true")) {
      v.kind = JVal::Bool;
      v.b = true;
    } else if (word("false")) {
      v.kind = JVal::Bool;
    } else if (word("null")) {
    } else {
      char* end = nullptr;
      std::string tok;
      while (p_ < e_ && std::strchr("+-0123456789.eE", *p_)) tok.push_back(*p_++);
      if (tok.empty()) err("unexpected character");
      v.kind = JVal::Number;
      v.num = std::strtod(tok.c_str(), &end);
      if (end != tok.c_str() + tok.size()) err("bad number " + tok);
    }
    return v;
  }
  bool word(const char* w) {
    const std::size_t n = std::strlen(w);
    if (static_cast<std::size_t>(e_ - p_) >= n && std::strncmp(p_, w, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  std::string text() {
    if (p_ >= e_ || *p_ != '"') err("expected a string");
    ++p_;
    std::string s;
    while (p_ < e_ && *p_ != '"') {
      char c = *p_++;
      if (c == '\\') {
        if (p_ >= e_) err("bad escape");
        c = *p_++;
        switch (c) {
          case 'n': c = '\n'; break;
          case 't': c = '\t'; break;
          case 'r': c = '\r'; break;
          case 'b': c = '\b'; break;
          case 'f': c = '\f'; break;
          case 'u': {  // \uXXXX, kept as UTF-8 for the BMP
            if (e_ - p_ < 4) err("bad \\u escape");
            const unsigned cp = static_cast<unsigned>(std::strtoul(std::string(p_, 4).c_str(), nullptr, 16));
            p_ += 4;
            if (cp < 0x80) s.push_back(static_cast<char>(cp));
            else if (cp < 0x800) {
              s.push_back(static_cast<char>(0xC0 | (cp >> 6)));
              s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
            } else {
              s.push_back(static_cast<char>(0xE0 | (cp >> 12)));
              s.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
              s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
            }
            continue;
          }
          default: break;  // \" \\ \/
        }
      }
      s.push_back(c);
    }
    if (p_ >= e_) err("unterminated string");
    ++p_;
    return s;
  }
  const char* p_;
  const char* e_;
};

std::size_t as_size(const JVal& v, const std::string& what) {
  if (v.kind != JVal::Number || v.num < 0 || v.num != std::floor(v.num) || v.num > 9.0e15)
    throw std::runtime_error("weights: " + what + " is not a non-negative integer");
  return static_cast<std::size_t>(v.num);
}

}  // namespace

Weights::Weights(const std::string& path) {
  fd_ = ::open(path.c_str(), O_RDONLY);
  if (fd_ < 0) throw std::runtime_error("weights: cannot open " + path);
  struct stat st {};
  if (::fstat(fd_, &st) != 0) {
    ::close(fd_);
    throw std::runtime_error("weights: fstat failed for " + path);
  }
  size_ = static_cast<std::size_t>(st.st_size);
  if (size_ < 16) {
    ::close(fd_);
    throw std::runtime_error("weights: bad magic in " + path);
  }
  base_ = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (base_ == MAP_FAILED) {
    base_ = nullptr;
    ::close(fd_);
    throw std::runtime_error("weights: mmap failed for " + path);
  }
  try {
    const char* bytes = static_cast<const char*>(base_);
    if (std::memcmp(bytes, "MMFREE1\n", 8) != 0) throw std::runtime_error("weights: bad magic in " + path);
    std::uint64_t hl = 0;
    std::memcpy(&hl, bytes + 8, 8);
    if (hl > size_ - 16) throw std::runtime_error("weights: header length exceeds the file");
    const JVal root = JReader(bytes + 16, bytes + 16 + hl).document();
    const JVal* c = root.at("config");
    if (!c || c->kind != JVal::Object) throw std::runtime_error("weights: no config in header");
    auto u = [&](const char* k, std::size_t& dst) {
      if (const JVal* v = c->at(k)) dst = as_size(*v, std::string("config.") + k);
    };
    auto bo = [&](const char* k, bool& dst) {
      if (const JVal* v = c->at(k)) dst = v->kind == JVal::Bool ? v->b : v->num != 0.0;
    };
    u("vocab_size", cfg_.vocab_size);
    u("hidden_size", cfg_.hidden_size);
    u("num_hidden_layers", cfg_.num_hidden_layers);
    u("num_heads", cfg_.num_heads);
    u("expand_ratio", cfg_.expand_ratio);
    u("intermediate_size", cfg_.intermediate_size);
    bo("use_lower_bound", cfg_.use_lower_bound);
    bo("use_short_conv", cfg_.use_short_conv);
    if (const JVal* e = c->at("rms_norm_eps")) cfg_.rms_norm_eps = static_cast<float>(e->num);
    const JVal* ts = root.at("tensors");
    if (!ts || ts->kind != JVal::Object) throw std::runtime_error("weights: no tensors in header");
    const std::size_t data_start = (16 + hl + 63) / 64 * 64;
    for (const auto& kv : ts->fields) {
      const JVal& m = kv.second;
      const JVal* dt = m.at("dtype");
      const JVal* sh = m.at("shape");
      const JVal* of = m.at("offset");
      if (!dt || dt->kind != JVal::String || !sh || sh->kind != JVal::Array || !of)
        throw std::runtime_error("weights: malformed entry for " + kv.first);
      TensorRef ref;
      std::size_t esize;
      if (dt->str == "f32") esize = 4;
      else if (dt->str == "i8") { esize = 1; ref.is_int8 = true; }
      else throw std::runtime_error("weights: tensor " + kv.first + " has dtype " + dt->str);
      // every product and sum below is checked: a crafted header must not wrap a size to a
      // small number that passes the bounds check
      const std::runtime_error too_big("weights: tensor " + kv.first + " does not fit the file");
      std::size_t numel = 1;
      for (const auto& d : sh->items) {
        ref.shape.push_back(as_size(d, kv.first + ".shape"));
        if (__builtin_mul_overflow(numel, ref.shape.back(), &numel)) throw too_big;
      }
      std::size_t nbytes = 0, start = 0, end = 0;
      if (__builtin_mul_overflow(ref.shape.empty() ? 0 : numel, esize, &nbytes)) throw too_big;
      const std::size_t off = as_size(*of, kv.first + ".offset");
      if (const JVal* nb = m.at("nbytes"))
        if (as_size(*nb, kv.first + ".nbytes") != nbytes)
          throw std::runtime_error("weights: " + kv.first + " nbytes disagrees with its shape");
      if (__builtin_add_overflow(data_start, off, &start) || __builtin_add_overflow(start, nbytes, &end) ||
          end > size_)
        throw too_big;
      ref.data = bytes + data_start + off;
      if (tensors_.count(kv.first)) throw std::runtime_error("weights: duplicate tensor " + kv.first);
      tensors_.emplace(kv.first, std::move(ref));
      order_.push_back(kv.first);
    }
  } catch (...) {
    ::munmap(base_, size_);
    ::close(fd_);
    base_ = nullptr;
    fd_ = -1;
    throw;
  }
}

Weights::~Weights() {
  if (base_) ::munmap(base_, size_);
  if (fd_ >= 0) ::close(fd_);
}

}  // namespace mmfree
