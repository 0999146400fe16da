"""Host mirror of the reference tokenizer over the library's native tokeniser.

Reference: internal/embed/tokenizer.go
  WordPieceTokenizer{vocab, idToTok, maxToken}   :15-19
  LoadTokenizer(path)                            :22-45
  (*WordPieceTokenizer).Encode(text, maxLen)     :47-78
  (*WordPieceTokenizer).VocabSize()              :145-148
Tokenisation runs in libllmembed_hip.so (C++, host threads, no GPU use).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import LLEError, check, ptr


def _as_bytes(text) -> bytes:
    return text if isinstance(text, (bytes, bytearray)) else str(text).encode("utf-8", "surrogatepass")


class _TextArray:
    """Keeps n byte strings alive and exposes (const char* const*, const int64_t*) for the C ABI."""

    def __init__(self, texts):
        self.bufs = [_as_bytes(t) for t in texts]
        n = len(self.bufs)
        self.ptrs = (C.c_char_p * max(n, 1))(*self.bufs)
        self.lens = np.array([len(b) for b in self.bufs] or [0], np.int64)
        self.n = n


class WordPieceTokenizer:
    """Native tokeniser handle (WordPieceTokenizer, tokenizer.go:15-19)."""

    def __init__(self, handle: C.c_void_p):
        self.h = handle

    @classmethod
    def load(cls, path: str) -> "WordPieceTokenizer":
        """LoadTokenizer (tokenizer.go:22-45): vocabulary from GGUF `tokenizer.ggml.tokens`."""
        h = C.c_void_p()
        rc = _lib.lib().lle_tokenizer_load_gguf(path.encode(), C.byref(h))
        if rc:
            raise LLEError(rc, f"embed: load tokenizer: {_lib.lib().lle_last_error().decode()}")
        return cls(h)

    @classmethod
    def from_tokens(cls, tokens) -> "WordPieceTokenizer":
        arr = _TextArray(tokens)
        h = C.c_void_p()
        check(_lib.lib().lle_tokenizer_create(C.cast(arr.ptrs, C.c_void_p), ptr(arr.lens), arr.n, C.byref(h)))
        return cls(h)

    def vocab_size(self) -> int:
        n = C.c_int32()
        check(_lib.lib().lle_tokenizer_vocab_size(self.h, C.byref(n)))
        return n.value

    def encode(self, text, max_len: int):
        """Encode (tokenizer.go:47-78): (ids, mask), mask all ones."""
        b = _as_bytes(text)
        cap = len(b) + 2
        ids = np.empty(max(1, min(cap, max_len)), np.int32)
        n = C.c_int32()
        check(_lib.lib().lle_tokenize(self.h, b, len(b), max_len, ptr(ids), ids.size, C.byref(n)))
        if n.value > ids.size:  # more pieces than bytes + 2 cannot happen; keep the API total
            ids = np.empty(n.value, np.int32)
            check(_lib.lib().lle_tokenize(self.h, b, len(b), max_len, ptr(ids), ids.size, C.byref(n)))
        ids = ids[:n.value].copy()
        return ids, np.ones_like(ids)

    def encode_batch(self, texts, max_len: int, prefix: str = ""):
        """Encode(prefix + text) for every text on host threads: (ids [n][L], mask [n][L], counts)."""
        arr = _TextArray(texts)
        pb = _as_bytes(prefix)
        counts = np.zeros(max(arr.n, 1), np.int32)
        L = _lib.lib()
        check(L.lle_tokenize_batch(self.h, C.cast(arr.ptrs, C.c_void_p), ptr(arr.lens), arr.n, pb, len(pb),
                                   max_len, 0, None, None, ptr(counts)))
        width = int(counts[:arr.n].max()) if arr.n else 0
        ids = np.zeros((arr.n, max(width, 1)), np.int32)
        mask = np.zeros_like(ids)
        if arr.n:
            check(L.lle_tokenize_batch(self.h, C.cast(arr.ptrs, C.c_void_p), ptr(arr.lens), arr.n, pb, len(pb),
                                       max_len, ids.shape[1], ptr(ids), ptr(mask), ptr(counts)))
        return ids, mask, counts[:arr.n].copy()

    def close(self):
        if getattr(self, "h", None):
            _lib.lib().lle_tokenizer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
