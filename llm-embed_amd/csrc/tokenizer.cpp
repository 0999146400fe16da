// Host tokeniser (no GPU use): Go's WordPieceTokenizer restated natively.
//
//   strings.ToLower            tokenizer.go:50,155   UTF-8 decoded as Go does (an invalid byte is
//                                                    one U+FFFD), unicode.ToLower per rune
//   preTokenize                tokenizer.go:154-179  unicode.IsSpace splits; isBertPunct runes
//                                                    (:183-195) are words of their own
//   encodeWord                 tokenizer.go:82-140   greedy longest match over the word's bytes,
//                                                    "▁" on the first piece, byte fallbacks, [UNK]
//   Encode                     tokenizer.go:47-78    [CLS] pieces [SEP], truncation keeps [SEP]
//   readGGUFStringArray        tokenizer.go:198-306  KV scan after the 24-byte header
//
// The greedy search of encodeWord tries end = min(len, start + maxToken) down to start + 1 and
// takes the first candidate in the vocabulary: that is the longest vocabulary token that is a
// prefix of the remaining bytes, which one walk down a byte trie finds (the trie is never deeper
// than maxToken). The whole-word lookup (:84-88) and the prefixed single-byte fallback (:119-126)
// are cases of that walk; only the unprefixed single byte at start 0 (:128-133) is a separate
// lookup.
#include "tokenizer.h"

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <new>
#include <thread>

#include "../../include/llmembed.h"

namespace lle {

int fail(int code, const std::string& msg);

namespace {

struct CaseRun {
  uint32_t lo, hi, stride;
  int32_t delta;
};
struct CodeRange {
  uint32_t lo, hi;
};
#include "unicode_tables.inc"

// unicode.ToLower: simple lowercase mapping.
inline uint32_t to_lower(uint32_t r) {
  if (r < 0x80) return (r - 'A' < 26u) ? r + 32 : r;
  const CaseRun* e = std::upper_bound(kLowerRuns, kLowerRuns + sizeof(kLowerRuns) / sizeof(kLowerRuns[0]), r,
                                      [](uint32_t v, const CaseRun& c) { return v < c.lo; });
  if (e == kLowerRuns) return r;
  --e;
  if (r > e->hi || (r - e->lo) % e->stride) return r;
  return (uint32_t)((int32_t)r + e->delta);
}

// unicode.IsSpace: the Latin-1 list, else the White_Space property.
inline bool is_space(uint32_t r) {
  if (r <= 0xFF) return r == ' ' || (r >= 0x09 && r <= 0x0D) || r == 0x85 || r == 0xA0;
  return r == 0x1680 || (r >= 0x2000 && r <= 0x200A) || r == 0x2028 || r == 0x2029 || r == 0x202F ||
         r == 0x205F || r == 0x3000;
}

// isBertPunct (tokenizer.go:183-195): ASCII non-alphanumeric printables, category P, and the
// CJK ideograph blocks of isChinesePunct.
inline bool is_bert_punct(uint32_t r) {
  if (r < 0x80) return (r >= 0x21 && r <= 0x2F) || (r >= 0x3A && r <= 0x40) || (r >= 0x5B && r <= 0x60) || (r >= 0x7B && r <= 0x7E);
  if ((r >= 0x4E00 && r <= 0x9FFF) || (r >= 0x3400 && r <= 0x4DBF) || (r >= 0x20000 && r <= 0x2A6DF)) return true;
  const CodeRange* e = std::upper_bound(kPunctRanges, kPunctRanges + sizeof(kPunctRanges) / sizeof(kPunctRanges[0]), r,
                                        [](uint32_t v, const CodeRange& c) { return v < c.lo; });
  return e != kPunctRanges && r <= (e - 1)->hi;
}

// utf8.DecodeRune: returns the rune and advances *i; an invalid or truncated sequence is U+FFFD
// and consumes one byte.
inline uint32_t decode_rune(const uint8_t* s, int64_t n, int64_t* i) {
  const uint8_t c = s[*i];
  if (c < 0x80) {
    ++*i;
    return c;
  }
  int need;
  uint8_t lo = 0x80, hi = 0xBF;
  if (c >= 0xC2 && c <= 0xDF) need = 1;
  else if (c == 0xE0) need = 2, lo = 0xA0;
  else if ((c >= 0xE1 && c <= 0xEC) || c == 0xEE || c == 0xEF) need = 2;
  else if (c == 0xED) need = 2, hi = 0x9F;
  else if (c == 0xF0) need = 3, lo = 0x90;
  else if (c >= 0xF1 && c <= 0xF3) need = 3;
  else if (c == 0xF4) need = 3, hi = 0x8F;
  else {
    ++*i;
    return 0xFFFD;
  }
  if (*i + need >= n) {  // continuation bytes s[*i+1 .. *i+need] must exist
    ++*i;
    return 0xFFFD;
  }
  const uint8_t c1 = s[*i + 1];
  if (c1 < lo || c1 > hi) {
    ++*i;
    return 0xFFFD;
  }
  uint32_t r;
  if (need == 1) {
    r = ((c & 0x1Fu) << 6) | (c1 & 0x3Fu);
  } else {
    const uint8_t c2 = s[*i + 2];
    if (c2 < 0x80 || c2 > 0xBF) {
      ++*i;
      return 0xFFFD;
    }
    if (need == 2) {
      r = ((c & 0x0Fu) << 12) | ((c1 & 0x3Fu) << 6) | (c2 & 0x3Fu);
    } else {
      const uint8_t c3 = s[*i + 3];
      if (c3 < 0x80 || c3 > 0xBF) {
        ++*i;
        return 0xFFFD;
      }
      r = ((c & 0x07u) << 18) | ((c1 & 0x3Fu) << 12) | ((c2 & 0x3Fu) << 6) | (c3 & 0x3Fu);
    }
  }
  *i += need + 1;
  return r;
}

inline void append_utf8(uint32_t r, std::string* out) {
  if (r < 0x80) {
    out->push_back((char)r);
  } else if (r < 0x800) {
    out->push_back((char)(0xC0 | (r >> 6)));
    out->push_back((char)(0x80 | (r & 0x3F)));
  } else if (r < 0x10000) {
    out->push_back((char)(0xE0 | (r >> 12)));
    out->push_back((char)(0x80 | ((r >> 6) & 0x3F)));
    out->push_back((char)(0x80 | (r & 0x3F)));
  } else {
    out->push_back((char)(0xF0 | (r >> 18)));
    out->push_back((char)(0x80 | ((r >> 12) & 0x3F)));
    out->push_back((char)(0x80 | ((r >> 6) & 0x3F)));
    out->push_back((char)(0x80 | (r & 0x3F)));
  }
}

inline uint64_t edge_hash(uint64_t key) {
  key *= 0x9E3779B97F4A7C15ull;
  return key ^ (key >> 29);
}

}  // namespace

uint32_t Tokenizer::child(uint32_t node, uint8_t b) const {
  const uint64_t key = (((uint64_t)node << 8) | b) + 1;
  for (uint64_t h = edge_hash(key) & mask_;; h = (h + 1) & mask_) {
    const uint64_t k = keys_[h];
    if (k == key) return vals_[h];
    if (k == 0) return 0;
  }
}

void Tokenizer::grow() {
  std::vector<uint64_t> ok;
  std::vector<uint32_t> ov;
  ok.swap(keys_);
  ov.swap(vals_);
  const size_t cap = ok.empty() ? 1024 : ok.size() * 2;
  keys_.assign(cap, 0);
  vals_.assign(cap, 0);
  mask_ = cap - 1;
  for (size_t i = 0; i < ok.size(); i++) {
    if (!ok[i]) continue;
    uint64_t h = edge_hash(ok[i]) & mask_;
    while (keys_[h]) h = (h + 1) & mask_;
    keys_[h] = ok[i];
    vals_[h] = ov[i];
  }
}

uint32_t Tokenizer::add_child(uint32_t node, uint8_t b) {
  const uint32_t c = child(node, b);
  if (c) return c;
  if ((n_edges_ + 1) * 2 > keys_.size()) grow();
  const uint64_t key = (((uint64_t)node << 8) | b) + 1;
  uint64_t h = edge_hash(key) & mask_;
  while (keys_[h]) h = (h + 1) & mask_;
  const uint32_t nn = (uint32_t)id_.size();
  id_.push_back(-1);
  keys_[h] = key;
  vals_[h] = nn;
  n_edges_++;
  return nn;
}

void Tokenizer::build(const char* const* tokens, const int64_t* lens, int32_t n) {
  keys_.clear();
  vals_.clear();
  n_edges_ = 0;
  id_.assign(1, -1);  // root
  grow();
  for (int32_t i = 0; i < n; i++) {
    uint32_t node = 0;
    const uint8_t* t = (const uint8_t*)tokens[i];
    for (int64_t k = 0; k < lens[i]; k++) node = add_child(node, t[k]);
    if (node) id_[node] = i;  // the empty token is never a candidate (end > start, :98)
  }
  static const uint8_t kPrefix[3] = {0xE2, 0x96, 0x81};  // "▁" U+2581
  uint32_t node = 0;
  for (int k = 0; k < 3 && (k == 0 || node); k++) node = child(node, kPrefix[k]);
  prefix_node_ = node;
  n_tokens_ = n;
}

void Tokenizer::encode_word(const uint8_t* w, int64_t n, std::vector<int32_t>* ids) const {
  int64_t start = 0;
  while (start < n) {
    uint32_t node = start == 0 ? prefix_node_ : 0;
    int64_t best_end = -1;
    int32_t best_id = -1;
    if (start > 0 || prefix_node_) {
      for (int64_t k = start; k < n; k++) {
        node = child(node, w[k]);
        if (!node) break;
        if (id_[node] >= 0) {
          best_end = k + 1;
          best_id = id_[node];
        }
      }
    }
    if (best_end > 0) {
      ids->push_back(best_id);
      start = best_end;
      continue;
    }
    if (start == 0) {  // single byte without the prefix (:128-133)
      const uint32_t c = child(0, w[0]);
      if (c && id_[c] >= 0) {
        ids->push_back(id_[c]);
        start = 1;
        continue;
      }
    }
    ids->push_back(kUNK);
    start++;
  }
}

void Tokenizer::encode(const char* prefix, int64_t prefix_len, const char* text, int64_t len, int32_t max_len,
                       std::vector<int32_t>* ids) const {
  const size_t base = ids->size();
  ids->push_back(kCLS);
  std::string word;
  auto flush = [&]() {
    if (!word.empty()) {
      encode_word((const uint8_t*)word.data(), (int64_t)word.size(), ids);
      word.clear();
    }
  };
  // Decoding prefix and text separately equals decoding their concatenation except when the
  // prefix ends inside a multi-byte sequence; then the concatenation is decoded.
  std::string joined;
  const uint8_t* parts[2] = {(const uint8_t*)prefix, (const uint8_t*)text};
  int64_t plen[2] = {prefix ? prefix_len : 0, text ? len : 0};
  if (plen[0] > 0) {
    int64_t i = 0;
    bool clean = true;
    while (i < plen[0]) {
      const int64_t j = i;
      const uint32_t r = decode_rune(parts[0], plen[0], &i);
      if (r == 0xFFFD && i - j == 1 && parts[0][j] >= 0x80) {
        clean = false;
        break;
      }
    }
    if (!clean) {
      joined.assign((const char*)parts[0], (size_t)plen[0]);
      joined.append((const char*)parts[1], (size_t)plen[1]);
      parts[0] = (const uint8_t*)joined.data();
      plen[0] = (int64_t)joined.size();
      plen[1] = 0;
    }
  }
  for (int p = 0; p < 2; p++) {
    const uint8_t* s = parts[p];
    const int64_t n = plen[p];
    for (int64_t i = 0; i < n;) {
      if (s[i] < 0x80) {  // ASCII: the same decisions, no decode
        uint32_t c = s[i++];
        if (c == ' ' || (c >= 0x09 && c <= 0x0D)) {
          flush();
        } else if (is_bert_punct(c)) {
          flush();
          word.push_back((char)c);
          flush();
        } else {
          word.push_back((char)(c - 'A' < 26u ? c + 32 : c));
        }
        continue;
      }
      // Encode and preTokenize both lowercase; the mapping is idempotent, so once suffices
      const uint32_t r = to_lower(decode_rune(s, n, &i));
      if (is_space(r)) {
        flush();
      } else if (is_bert_punct(r)) {
        flush();
        append_utf8(r, &word);
        flush();
      } else {
        append_utf8(r, &word);
      }
    }
  }
  flush();
  ids->push_back(kSEP);
  if (ids->size() - base > (size_t)max_len) {
    ids->resize(base + max_len);
    ids->back() = kSEP;
  }
}

int read_gguf_string_array(const char* path, const char* key, std::vector<std::string>* out) {
  int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(LLE_EIO, std::string("tokenizer: open ") + path + ": " + strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    return fail(LLE_EIO, std::string("tokenizer: ") + path + ": too short for a GGUF header");
  }
  const size_t size = (size_t)st.st_size;
  void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) return fail(LLE_EIO, std::string("tokenizer: mmap ") + path);
  const uint8_t* p = (const uint8_t*)map + 24;
  const uint8_t* end = (const uint8_t*)map + size;
  bool ok = true;
  auto need = [&](uint64_t n) {
    if (!ok || (uint64_t)(end - p) < n) ok = false;
    return ok;
  };
  auto u32 = [&]() -> uint32_t {
    uint32_t v = 0;
    if (need(4)) memcpy(&v, p, 4), p += 4;
    return v;
  };
  auto u64 = [&]() -> uint64_t {
    uint64_t v = 0;
    if (need(8)) memcpy(&v, p, 8), p += 8;
    return v;
  };
  auto str = [&](std::string* s) {
    const uint64_t n = u64();
    if (!need(n)) return;
    if (s) s->assign((const char*)p, (size_t)n);
    p += n;
  };
  // skipGGUFValue (:268-306); unknown types are an error
  bool bad_type = false;
  auto skip = [&](uint32_t t, auto& self) -> void {
    switch (t) {
      case 0: case 1: case 7: need(1) && (p += 1); break;
      case 2: case 3: need(2) && (p += 2); break;
      case 4: case 5: case 6: need(4) && (p += 4); break;
      case 10: case 11: case 12: need(8) && (p += 8); break;
      case 8: str(nullptr); break;
      case 9: {
        const uint32_t et = u32();
        const uint64_t n = u64();
        for (uint64_t i = 0; i < n && ok && !bad_type; i++) self(et, self);
        break;
      }
      default: bad_type = true;
    }
  };
  uint64_t nkv;
  memcpy(&nkv, (const uint8_t*)map + 16, 8);
  int rc = LLE_OK;
  std::string k;
  bool found = false;
  for (uint64_t i = 0; i < nkv && ok && !bad_type; i++) {
    str(&k);
    const uint32_t t = u32();
    if (!ok) break;
    if (k == key && t == 9) {
      const uint32_t et = u32();
      if (et != 8) {
        rc = fail(LLE_EIO, "tokenizer: expected string array, got element type " + std::to_string(et));
        found = true;
        break;
      }
      const uint64_t n = u64();
      if (ok && n > (uint64_t)(end - p) / 8) ok = false;  // each string needs at least its length
      out->clear();
      for (uint64_t j = 0; j < n && ok; j++) {
        out->emplace_back();
        str(&out->back());
      }
      found = true;
      break;
    }
    skip(t, skip);
  }
  munmap(map, size);
  if (rc) return rc;
  if (!ok) return fail(LLE_EIO, std::string("tokenizer: ") + path + ": truncated GGUF metadata");
  if (bad_type) return fail(LLE_EIO, std::string("tokenizer: ") + path + ": unknown GGUF value type");
  if (!found) return fail(LLE_ENOTFOUND, std::string("tokenizer: key \"") + key + "\" not found in GGUF metadata");
  return LLE_OK;
}

}  // namespace lle

namespace lle {

// Tokenise texts [0, n) on up to `threads` host threads; ids_of[i] = Encode(prefix + text i).
void tokenize_many(const Tokenizer& tk, const char* const* texts, const int64_t* lens, int32_t n, const char* prefix,
                   int64_t prefix_len, int32_t max_len, std::vector<std::vector<int32_t>>* ids_of) {
  ids_of->assign((size_t)n, {});
  auto work = [&](int32_t lo, int32_t hi) {
    for (int32_t i = lo; i < hi; i++) {
      const int64_t len = lens ? lens[i] : (texts[i] ? (int64_t)strlen(texts[i]) : 0);
      tk.encode(prefix, prefix_len, texts[i], len, max_len, &(*ids_of)[i]);
    }
  };
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const int32_t nt = (int32_t)std::min<int64_t>({(int64_t)std::min(hw, 8u), (int64_t)(n + 31) / 32});
  if (nt <= 1) {
    work(0, n);
    return;
  }
  std::vector<std::thread> th;
  const int32_t per = (n + nt - 1) / nt;
  for (int32_t t = 0; t < nt; t++) {
    const int32_t lo = t * per, hi = std::min(n, lo + per);
    if (lo < hi) th.emplace_back(work, lo, hi);
  }
  for (auto& x : th) x.join();
}

}  // namespace lle

using lle::fail;

extern "C" {

int32_t lle_tokenizer_create(const char* const* tokens, const int64_t* lens, int32_t n, lle_tokenizer** out) {
  if (!out || n < 0 || (n > 0 && (!tokens || !lens))) return fail(LLE_EINVAL, "bad argument");
  for (int32_t i = 0; i < n; i++)
    if (lens[i] < 0 || (lens[i] > 0 && !tokens[i])) return fail(LLE_EINVAL, "bad token " + std::to_string(i));
  auto* t = new (std::nothrow) lle_tokenizer;
  if (!t) return fail(LLE_EINVAL, "out of host memory");
  t->tok.build(tokens, lens, n);
  *out = t;
  return LLE_OK;
}

int32_t lle_tokenizer_load_gguf(const char* path, lle_tokenizer** out) {
  if (!path || !out) return fail(LLE_EINVAL, "null argument");
  std::vector<std::string> toks;
  int rc = lle::read_gguf_string_array(path, "tokenizer.ggml.tokens", &toks);
  if (rc) return rc;
  if (toks.size() > (size_t)INT32_MAX) return fail(LLE_EUNSUPPORTED, "tokenizer: vocabulary too large");
  std::vector<const char*> p(toks.size());
  std::vector<int64_t> l(toks.size());
  for (size_t i = 0; i < toks.size(); i++) {
    p[i] = toks[i].data();
    l[i] = (int64_t)toks[i].size();
  }
  return lle_tokenizer_create(p.data(), l.data(), (int32_t)toks.size(), out);
}

int32_t lle_tokenizer_destroy(lle_tokenizer* t) {
  delete t;
  return LLE_OK;
}

int32_t lle_tokenizer_vocab_size(const lle_tokenizer* t, int32_t* n) {
  if (!t || !n) return fail(LLE_EINVAL, "null argument");
  *n = t->tok.vocab_size();
  return LLE_OK;
}

int32_t lle_tokenize(const lle_tokenizer* t, const char* text, int64_t len, int32_t max_len, int32_t* ids, int32_t cap,
                     int32_t* n_out) {
  if (!t || !n_out || (len > 0 && !text) || cap < 0 || (cap > 0 && !ids)) return fail(LLE_EINVAL, "bad argument");
  if (max_len < 1) return fail(LLE_EINVAL, "max_len must be at least 1");
  if (len < 0) len = text ? (int64_t)strlen(text) : 0;
  std::vector<int32_t> v;
  t->tok.encode(nullptr, 0, text, len, max_len, &v);
  *n_out = (int32_t)v.size();
  memcpy(ids, v.data(), sizeof(int32_t) * std::min<size_t>(v.size(), (size_t)cap));
  return LLE_OK;
}

int32_t lle_tokenize_batch(const lle_tokenizer* t, const char* const* texts, const int64_t* lens, int32_t n,
                           const char* prefix, int64_t prefix_len, int32_t max_len, int32_t L, int32_t* ids,
                           int32_t* mask, int32_t* n_tok) {
  if (!t || n < 0 || (n > 0 && (!texts || !n_tok)) || (prefix_len > 0 && !prefix)) return fail(LLE_EINVAL, "bad argument");
  if (max_len < 1) return fail(LLE_EINVAL, "max_len must be at least 1");
  if (ids && (L < 1 || !mask)) return fail(LLE_EINVAL, "ids needs mask and L >= 1");
  if (prefix && prefix_len < 0) prefix_len = (int64_t)strlen(prefix);
  std::vector<std::vector<int32_t>> v;
  lle::tokenize_many(t->tok, texts, lens, n, prefix, prefix_len, max_len, &v);
  int32_t longest = 0;
  for (int32_t i = 0; i < n; i++) {
    n_tok[i] = (int32_t)v[i].size();
    longest = std::max(longest, n_tok[i]);
  }
  if (!ids) return LLE_OK;
  if (longest > L) return fail(LLE_EINVAL, "a text needs " + std::to_string(longest) + " tokens, more than L = " + std::to_string(L));
  for (int32_t i = 0; i < n; i++) {
    int32_t* row = ids + (size_t)i * L;
    int32_t* mrow = mask + (size_t)i * L;
    const int32_t k = n_tok[i];
    memcpy(row, v[i].data(), sizeof(int32_t) * k);
    std::fill(row + k, row + L, 0);
    std::fill(mrow, mrow + k, 1);
    std::fill(mrow + k, mrow + L, 0);
  }
  return LLE_OK;
}

}  // extern "C"
