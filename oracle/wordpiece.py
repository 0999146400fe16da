"""Pure-Python restatement of the reference tokenizer (internal/embed/tokenizer.go).

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's CPU leg as the checker for the
library's native tokeniser (lle_tokenize / lle_embed_texts). The product never imports this.

Go semantics restated here, byte for byte:
  - strings.ToLower (tokenizer.go:50,155): UTF-8 decoded as Go does (an invalid byte is one
    U+FFFD), each rune mapped by unicode.ToLower (simple case mapping) and re-encoded.
  - preTokenize (:154-179): unicode.IsSpace splits; isBertPunct runes (:183-189, ASCII ranges,
    category P, CJK ideograph blocks :191-195) are words of their own; other runes accumulate.
  - encodeWord (:82-140): greedy longest match over BYTES of the word; the first piece carries
    the "▁" prefix; a start with no match falls back to the single byte (with prefix at
    start 0, then without), else [UNK]=100 and one byte is consumed.
  - Encode (:47-78): [CLS]=101, pieces, [SEP]=102; longer than max_len -> first max_len ids
    with [SEP] last.
  - readGGUFStringArray (:198-230): scans the KV section after the 24-byte header.

Unicode data: this interpreter's unicodedata (13.0.0 on Python 3.10); Go 1.26 uses a later
Unicode version, so code points assigned after 13.0 are outside what this restatement pins.
"""
from __future__ import annotations

import struct
import unicodedata

CLS, SEP, UNK = 101, 102, 100
PREFIX = "▁".encode()


# Go's unicode.IsSpace (unicode/graphic.go): Latin-1 list, else the White_Space property.
_LATIN1_SPACE = {0x09, 0x0A, 0x0B, 0x0C, 0x0D, 0x20, 0x85, 0xA0}
_WHITE_SPACE = {0x1680, 0x2028, 0x2029, 0x202F, 0x205F, 0x3000} | set(range(0x2000, 0x200B))


def is_space(r: int) -> bool:
    if r <= 0xFF:
        return r in _LATIN1_SPACE
    return r in _WHITE_SPACE


def is_bert_punct(r: int) -> bool:
    """isBertPunct, tokenizer.go:183-189 (with isChinesePunct, :191-195)."""
    if 0x21 <= r <= 0x2F or 0x3A <= r <= 0x40 or 0x5B <= r <= 0x60 or 0x7B <= r <= 0x7E:
        return True
    if unicodedata.category(chr(r)).startswith("P"):
        return True
    return 0x4E00 <= r <= 0x9FFF or 0x3400 <= r <= 0x4DBF or 0x20000 <= r <= 0x2A6DF


def to_lower_rune(r: int) -> int:
    """unicode.ToLower: the simple lowercase mapping (U+0130 -> U+0069; elsewhere str.lower)."""
    if 0xD800 <= r <= 0xDFFF:
        return r
    s = chr(r).lower()
    if len(s) == 1:
        return ord(s)
    return 0x69 if r == 0x130 else r


def decode_runes(b: bytes):
    """utf8.DecodeRune over b: yields runes; an invalid or truncated sequence is U+FFFD, width 1."""
    i, n = 0, len(b)
    while i < n:
        c = b[i]
        if c < 0x80:
            yield c
            i += 1
            continue
        if 0xC2 <= c <= 0xDF:
            need, lo, hi = 1, 0x80, 0xBF
        elif c == 0xE0:
            need, lo, hi = 2, 0xA0, 0xBF
        elif 0xE1 <= c <= 0xEC or 0xEE <= c <= 0xEF:
            need, lo, hi = 2, 0x80, 0xBF
        elif c == 0xED:
            need, lo, hi = 2, 0x80, 0x9F
        elif c == 0xF0:
            need, lo, hi = 3, 0x90, 0xBF
        elif 0xF1 <= c <= 0xF3:
            need, lo, hi = 3, 0x80, 0xBF
        elif c == 0xF4:
            need, lo, hi = 3, 0x80, 0x8F
        else:
            yield 0xFFFD
            i += 1
            continue
        ok = i + need < n  # continuation bytes b[i+1 .. i+need] present
        if ok:
            ok = lo <= b[i + 1] <= hi and all(0x80 <= b[i + k] <= 0xBF for k in range(2, need + 1))
        if not ok:
            yield 0xFFFD
            i += 1
            continue
        if need == 1:
            r = ((c & 0x1F) << 6) | (b[i + 1] & 0x3F)
        elif need == 2:
            r = ((c & 0x0F) << 12) | ((b[i + 1] & 0x3F) << 6) | (b[i + 2] & 0x3F)
        else:
            r = ((c & 0x07) << 18) | ((b[i + 1] & 0x3F) << 12) | ((b[i + 2] & 0x3F) << 6) | (b[i + 3] & 0x3F)
        yield r
        i += need + 1


def to_lower(b: bytes) -> bytes:
    """strings.ToLower on a byte string."""
    return "".join(chr(to_lower_rune(r)) for r in decode_runes(b)).encode("utf-8")


def pre_tokenize(b: bytes) -> list:
    """preTokenize, tokenizer.go:154-179: list of words (UTF-8 bytes)."""
    words, cur = [], []
    for r in decode_runes(to_lower(b)):
        if is_space(r):
            if cur:
                words.append("".join(cur).encode())
                cur = []
        elif is_bert_punct(r):
            if cur:
                words.append("".join(cur).encode())
                cur = []
            words.append(chr(r).encode())
        else:
            cur.append(chr(r))
    if cur:
        words.append("".join(cur).encode())
    return words


class Tokenizer:
    """WordPieceTokenizer (tokenizer.go:15-45): vocab token -> id (a later duplicate wins)."""

    def __init__(self, tokens):
        toks = [t if isinstance(t, bytes) else t.encode("utf-8") for t in tokens]
        self.id_to_tok = toks
        self.vocab = {}
        for i, t in enumerate(toks):
            self.vocab[t] = i
        self.max_token = max((len(t) for t in toks), default=0)

    def vocab_size(self) -> int:
        return len(self.id_to_tok)

    def encode_word(self, word: bytes) -> list:
        """encodeWord, tokenizer.go:82-140."""
        full = PREFIX + word
        if full in self.vocab:
            return [self.vocab[full]]
        ids, start, n = [], 0, len(word)
        while start < n:
            end = min(n, start + self.max_token)
            found = False
            while end > start:
                cand = (PREFIX + word[start:end]) if start == 0 else word[start:end]
                if cand in self.vocab:
                    ids.append(self.vocab[cand])
                    start = end
                    found = True
                    break
                end -= 1
            if found:
                continue
            if start == 0 and PREFIX + word[0:1] in self.vocab:
                ids.append(self.vocab[PREFIX + word[0:1]])
                start += 1
                continue
            if word[start:start + 1] in self.vocab:
                ids.append(self.vocab[word[start:start + 1]])
                start += 1
                continue
            ids.append(UNK)
            start += 1
        return ids

    def encode(self, text, max_len: int) -> list:
        """Encode, tokenizer.go:47-78 (the mask is all ones: len(ids) of them)."""
        b = text if isinstance(text, bytes) else text.encode("utf-8")
        ids = [CLS]
        for w in pre_tokenize(b):
            ids.extend(self.encode_word(w))
        ids.append(SEP)
        if len(ids) > max_len:
            ids = ids[:max_len]
            ids[max_len - 1] = SEP
        return ids


def read_gguf_string_array(path: str, key: str) -> list:
    """readGGUFStringArray, tokenizer.go:198-230 (value skipping as skipGGUFValue :268-306)."""
    with open(path, "rb") as f:
        data = f.read()
    pos = 24
    (nkv,) = struct.unpack_from("<Q", data, 16)

    def u32():
        nonlocal pos
        (v,) = struct.unpack_from("<I", data, pos)
        pos += 4
        return v

    def u64():
        nonlocal pos
        (v,) = struct.unpack_from("<Q", data, pos)
        pos += 8
        return v

    def gstr():
        nonlocal pos
        n = u64()
        s = data[pos:pos + n]
        if len(s) != n:
            raise EOFError("truncated string")
        pos += n
        return s

    sizes = {0: 1, 1: 1, 7: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 10: 8, 11: 8, 12: 8}

    def skip(t):
        nonlocal pos
        if t in sizes:
            pos += sizes[t]
        elif t == 8:
            gstr()
        elif t == 9:
            et, n = u32(), u64()
            for _ in range(n):
                skip(et)
        else:
            raise ValueError(f"unknown GGUF value type: {t}")

    for _ in range(nkv):
        k = gstr()
        t = u32()
        if k == key.encode() and t == 9:
            et = u32()
            if et != 8:
                raise ValueError(f"expected string array, got element type {et}")
            return [gstr() for _ in range(u64())]
        skip(t)
    raise KeyError(f"key {key!r} not found in GGUF metadata")
