// Host tokeniser: the reference's WordPieceTokenizer (internal/embed/tokenizer.go) restated in
// C++, with the vocabulary in a byte trie so the greedy longest match is one walk per piece.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace lle {

class Tokenizer {
 public:
  static constexpr int32_t kCLS = 101, kSEP = 102, kUNK = 100;

  // tokens[i] of lens[i] bytes is id i; a later duplicate takes the id (tokenizer.go:31-37).
  void build(const char* const* tokens, const int64_t* lens, int32_t n);
  int32_t vocab_size() const { return n_tokens_; }
  // Encode (tokenizer.go:47-78) of prefix + text, appended to *ids. max_len >= 1.
  void encode(const char* prefix, int64_t prefix_len, const char* text, int64_t len, int32_t max_len,
              std::vector<int32_t>* ids) const;

 private:
  void encode_word(const uint8_t* w, int64_t n, std::vector<int32_t>* ids) const;
  uint32_t child(uint32_t node, uint8_t b) const;
  uint32_t add_child(uint32_t node, uint8_t b);
  void grow();

  // Trie edges in an open-addressing table: key (node << 8 | byte) + 1 -> child node.
  std::vector<uint64_t> keys_;
  std::vector<uint32_t> vals_;
  uint64_t mask_ = 0;
  size_t n_edges_ = 0;
  std::vector<int32_t> id_;    // per node: token id ending there, or -1
  uint32_t prefix_node_ = 0;   // node after "▁" (U+2581), 0 when no token starts with it
  int32_t n_tokens_ = 0;
};

// GGUF metadata string array (readGGUFStringArray, tokenizer.go:198-230). Returns 0 or an
// LLE_E* code (message through fail()).
int read_gguf_string_array(const char* path, const char* key, std::vector<std::string>* out);

// Encode(prefix + texts[i]) for i in [0, n) on up to 8 host threads (lens == nullptr: strlen).
void tokenize_many(const Tokenizer& tk, const char* const* texts, const int64_t* lens, int32_t n, const char* prefix,
                   int64_t prefix_len, int32_t max_len, std::vector<std::vector<int32_t>>* ids_of);
}  // namespace lle

struct lle_tokenizer {
  lle::Tokenizer tok;
};
