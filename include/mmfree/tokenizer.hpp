// mmfree/tokenizer.hpp -- the text side of the CLI: SentencePiece-style BPE over the
// tokenizer.mmtok file the reference packs (tools/provision.py:170-219), with the
// reference's interface (cpp/include/mmfree/tokenizer.hpp:15-37).
//
// File: "MMTOK1\n\0", u32 vocab_size, u32 n_merges, i32 bos, eos, unk (little endian),
// then vocab_size pieces and n_merges rank-ordered "left right" merges, each a u32 byte
// length followed by UTF-8 bytes.
//
// encode: prepend U+2581 and map ' ' to U+2581; start from one symbol per UTF-8 code point
// (a lead byte >= 0xF0 / 0xE0 / 0xC0 opens a 4 / 3 / 2 byte sequence, anything else or a
// sequence cut short by the end of the text is one byte); repeatedly merge the adjacent
// pair with the lowest merge rank, the leftmost one on ties; emit each symbol's id, or its
// bytes as <0xNN> byte-fallback ids when the symbol is not a vocabulary piece. BOS first
// when add_bos; an empty text gives only BOS.
// decode: skip ids outside the vocabulary (and BOS/EOS/UNK when skip_special), turn
// <0xNN> pieces into raw bytes and U+2581 into spaces, drop one leading space.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace mmfree {

class Tokenizer {
 public:
  explicit Tokenizer(const std::string& path);

  std::vector<std::int64_t> encode(const std::string& text, bool add_bos = true) const;
  std::string decode(const std::vector<std::int64_t>& ids, bool skip_special = true) const;

  std::int64_t bos_id() const { return bos_; }
  std::int64_t eos_id() const { return eos_; }
  std::int64_t unk_id() const { return unk_; }
  std::size_t vocab_size() const { return pieces_.size(); }

 private:
  std::vector<std::string> pieces_;                   // id -> piece
  std::unordered_map<std::string, int> ids_;          // piece -> id
  std::unordered_map<std::string, int> rank_;         // "left right" -> merge rank
  int byte_id_[256];                                  // <0xNN> -> id, -1 if absent
  std::int64_t bos_ = 1, eos_ = 2, unk_ = 0;
};

}  // namespace mmfree
