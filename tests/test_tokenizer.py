"""Host tokeniser: the oracle restatement (oracle/wordpiece.py) pinned against library routines
and hand-derived cases, then the library's native tokeniser (lle_tokenize*) against the oracle.

Reference: internal/embed/tokenizer.go (Encode :47-78, encodeWord :82-140, preTokenize
:154-179, isBertPunct :183-195, readGGUFStringArray :198-306) and its test TestTokenizer
(internal/embed/embedder_test.go:147-177). No GPU is used: tokenisation is host work.
"""
import os
import random
import struct
import unicodedata

import numpy as np
import pytest

import wordpiece as wp
from llmembed import LLEError, WordPieceTokenizer, gguf, synth

# --------------------------------------------------------------------------------------------
# Vocabulary for the hand-derived cases: BERT's special ids, then a few pieces.
KAT_PIECES = ["▁hello", "▁world", "▁un", "believ", "able", "▁a", "a", "b", "▁,", "▁!", "▁σ", "▁i", "▁中", "▁x",
              "x", "▁hel", "lo", "▁é", "world", "σ"]


def kat_vocab(extra=()):
    toks = [f"[unused{i}]" for i in range(104)]
    toks[0] = "[PAD]"
    toks[100], toks[101], toks[102], toks[103] = "[UNK]", "[CLS]", "[SEP]", "[MASK]"
    return toks + KAT_PIECES + list(extra)


def ids_of(vocab, names):
    """Expected ids from token names (the last occurrence of a duplicate), CLS/SEP around."""
    pos = {t: i for i, t in enumerate(vocab)}
    return [101] + [100 if n == "UNK" else pos[n] for n in names] + [102]


# (text bytes, max_len, expected token names) — each derived by hand from tokenizer.go.
KATS = [
    (b"Hello, World!", 512, ["▁hello", "▁,", "▁world", "▁!"]),
    (b"unbelievable", 512, ["▁un", "believ", "able"]),             # greedy longest match, maxToken 10
    ("héllo".encode(), 512, ["UNK", "UNK", "UNK", "UNK", "lo"]),   # h; é as two bytes; l; lo
    ("é".encode(), 512, ["▁é"]),                                   # whole word with the prefix
    (b"ab", 512, ["▁a", "b"]),
    (b"ba", 512, ["b", "a"]),                                      # start-0 fallback without the prefix
    ("ΣΑΣ".encode(), 512, ["▁σ", "UNK", "UNK", "σ"]),              # Σ -> σ even word-final (no ς)
    ("İx".encode(), 512, ["▁i", "x"]),                             # unicode.ToLower(U+0130) = 'i'
    ("中文x".encode(), 512, ["▁中", "UNK", "UNK", "UNK", "▁x"]),    # CJK ideographs are words
    ("a\u00a0b".encode(), 512, ["▁a", "b"]),                      # NBSP is a space
    ("a\u200bb".encode(), 512, ["▁a", "UNK", "UNK", "UNK", "b"]),  # ZWSP is neither space nor punct
    ("x\u0085y".encode(), 512, ["▁x", "UNK"]),                     # NEL (C2 85) is a space
    (b"x\x85y", 512, ["▁x", "UNK", "UNK", "UNK", "UNK"]),          # a lone 0x85 byte -> U+FFFD (3 bytes)
    (b"hello_world", 512, ["▁hello", "UNK", "▁world"]),            # '_' is ASCII punctuation
    (b"aaaaaaaaaaaaa", 512, ["▁a"] + ["a"] * 12),
    (b"", 512, []),
    (b"  \t\n\r\x0b\x0c ", 512, []),
]
TRUNC = [(b"hello world", 4, [101, "▁hello", "▁world", 102]), (b"hello world", 3, [101, "▁hello", 102]),
         (b"hello world", 2, [101, 102]), (b"hello world", 1, [102])]


def resolve(vocab, seq):
    pos = {t: i for i, t in enumerate(vocab)}
    return [x if isinstance(x, int) else pos[x] for x in seq]


# --------------------------------------------------------------------------------------------
# Oracle pins


@pytest.mark.parametrize("text,max_len,names", KATS)
def test_oracle_known_answers(text, max_len, names):
    v = kat_vocab()
    assert wp.Tokenizer(v).encode(text, max_len) == ids_of(v, names)


@pytest.mark.parametrize("text,max_len,seq", TRUNC)
def test_oracle_truncation_keeps_sep(text, max_len, seq):
    v = kat_vocab()
    assert wp.Tokenizer(v).encode(text, max_len) == resolve(v, seq)


def test_oracle_later_duplicate_wins():
    v = kat_vocab(extra=["▁x"])
    assert wp.Tokenizer(v).encode(b"x", 512) == [101, len(v) - 1, 102]


def _go_decode(b: bytes):
    """utf8.DecodeRune stated through Python's strict decoder: at each position, the one width
    whose bytes decode to exactly one code point, else U+FFFD consuming one byte."""
    i, out = 0, []
    while i < len(b):
        for w in (1, 2, 3, 4):
            try:
                s = b[i:i + w].decode("utf-8")
            except UnicodeDecodeError:
                continue
            if len(s) == 1:
                out.append(ord(s))
                i += w
                break
        else:
            out.append(0xFFFD)
            i += 1
    return out


def test_oracle_utf8_decode_exhaustive_short_and_random_long():
    for a in range(256):
        assert list(wp.decode_runes(bytes([a]))) == _go_decode(bytes([a]))
        for c in range(256):
            b = bytes([a, c])
            assert list(wp.decode_runes(b)) == _go_decode(b), b
    rng = random.Random(7)
    for _ in range(100000):
        n = rng.randint(3, 6)
        b = bytes([rng.choice([rng.randint(0xC0, 0xF7), rng.randint(0x80, 0xBF), rng.randint(0, 0x7F)])
                   for _ in range(n)])
        assert list(wp.decode_runes(b)) == _go_decode(b), b


def test_oracle_is_space_is_the_white_space_property():
    """Go's unicode.IsSpace is White_Space; Python's str.isspace adds U+001C..U+001F."""
    ours = {c for c in range(0x110000) if wp.is_space(c)}
    py = {c for c in range(0x110000) if chr(c).isspace()} - set(range(0x1C, 0x20))
    assert ours == py


def test_oracle_lowercase_is_the_simple_mapping():
    assert wp.to_lower_rune(0x130) == 0x69          # simple mapping, not "i̇"
    assert wp.to_lower_rune(ord("Σ")) == ord("σ")   # no final-sigma context
    assert wp.to_lower_rune(ord("ǅ")) == ord("ǆ")   # titlecase digraph
    assert wp.to_lower(b"\xff") == "�".encode()
    for c in range(0x110000):  # idempotent, as Encode + preTokenize lowercase twice
        if not 0xD800 <= c <= 0xDFFF:
            assert wp.to_lower_rune(wp.to_lower_rune(c)) == wp.to_lower_rune(c)


def _stable_non_cjk_pool():
    """Code points below U+3000 whose category is the same in Unicode 3.2 and in this Python's
    Unicode (13.0): the `tokenizers` library's punctuation table predates 13.0, so characters
    assigned or recategorised since are left out of this comparison."""
    old = unicodedata.ucd_3_2_0
    pool = [chr(c) for c in range(0x20, 0x3000)
            if unicodedata.category(chr(c)) not in ("Cn", "Cs", "Co", "Cc")
            and old.category(chr(c)) == unicodedata.category(chr(c))]
    return pool + [" ", "\t", "\n", "\u00a0", "\u3000", "\u2009", "\x1c"]


def test_oracle_pretokenize_matches_bert_pretokenizer():
    """Outside the CJK blocks, preTokenize is BERT's whitespace + punctuation split, which the
    `tokenizers` library implements independently (BertPreTokenizer)."""
    from tokenizers import pre_tokenizers

    pre = pre_tokenizers.BertPreTokenizer()
    rng = random.Random(3)
    pool = _stable_non_cjk_pool()
    for _ in range(3000):
        text = "".join(rng.choice(pool) for _ in range(rng.randint(0, 40)))
        low = wp.to_lower(text.encode()).decode()
        ref = [w.encode() for w, _ in pre.pre_tokenize_str(low)]
        assert wp.pre_tokenize(text.encode()) == ref, repr(text)


def test_oracle_word_pieces_match_wordpiece_model():
    """Where `tokenizers`' WordPiece (greedy longest-match-first, "##" continuation) finds no
    unknown piece, encodeWord must give the same pieces ("▁x" <-> "x", "y" <-> "##y")."""
    from tokenizers import models

    toks = synth._tokens(30522)
    hf_vocab = {}
    for i, t in enumerate(toks):
        key = t[1:] if t.startswith("▁") else ("##" + t if not t.startswith("[") else t)
        hf_vocab.setdefault(key, i)
    model = models.WordPiece(hf_vocab, unk_token="[UNK]", max_input_chars_per_word=10 ** 6)
    ours = wp.Tokenizer(toks)
    checked = 0
    for text in synth.texts(400, seed=11):
        for w in wp.pre_tokenize(text.encode()):
            ref = [t.id for t in model.tokenize(w.decode())]
            if 100 in ref:
                continue
            assert ours.encode_word(w) == ref, w
            checked += 1
    assert checked > 5000


def test_reference_tokenizer_test(tmp_path):
    """TestTokenizer (embedder_test.go:147-177) on the synthetic GGUF's vocabulary."""
    spec = synth.ModelSpec(n_layer=1, d_model=64, n_head=1, d_ff=128)
    kvs, tensors = synth.build_tensors(spec, "Q8_0", 5)
    path = str(tmp_path / "tok.gguf")
    gguf.write(path, kvs, tensors)
    toks = wp.read_gguf_string_array(path, "tokenizer.ggml.tokens")
    assert len(toks) == 30522
    assert toks == [t.encode() for t in synth._tokens(30522)]
    for tok in (wp.Tokenizer(toks), WordPieceTokenizer.load(path)):
        if isinstance(tok, wp.Tokenizer):
            ids, mask = tok.encode(b"hello world", 512), None
            assert tok.vocab_size() == 30522
        else:
            ids, mask = tok.encode("hello world", 512)
            ids = ids.tolist()
            assert tok.vocab_size() == 30522
            assert mask.tolist() == [1] * len(ids)
        assert len(ids) >= 3 and ids[0] == 101 and ids[-1] == 102
        assert ids == [101, toks.index("▁hello".encode()), toks.index("▁world".encode()), 102]


# --------------------------------------------------------------------------------------------
# Native tokeniser (library, C++) against the oracle


@pytest.fixture(scope="module")
def vocab30k():
    return synth._tokens(30522)


@pytest.fixture(scope="module")
def native30k(vocab30k):
    return WordPieceTokenizer.from_tokens(vocab30k)


@pytest.mark.parametrize("text,max_len,names", KATS)
def test_native_known_answers(text, max_len, names):
    v = kat_vocab()
    ids, mask = WordPieceTokenizer.from_tokens(v).encode(text, max_len)
    assert ids.tolist() == ids_of(v, names)
    assert mask.tolist() == [1] * len(ids)


@pytest.mark.parametrize("text,max_len,seq", TRUNC)
def test_native_truncation(text, max_len, seq):
    v = kat_vocab()
    assert WordPieceTokenizer.from_tokens(v).encode(text, max_len)[0].tolist() == resolve(v, seq)


def test_native_duplicates_and_bad_arguments():
    v = kat_vocab(extra=["▁x"])
    t = WordPieceTokenizer.from_tokens(v)
    assert t.encode(b"x", 512)[0].tolist() == [101, len(v) - 1, 102]
    with pytest.raises(LLEError):
        t.encode(b"x", 0)


def test_native_matches_oracle_on_synthetic_texts(vocab30k, native30k):
    o = wp.Tokenizer(vocab30k)
    texts = synth.texts(1500, seed=21, min_words=0, max_words=120)
    ids, mask, counts = native30k.encode_batch(texts, 2048, prefix="search_query: ")
    for i, t in enumerate(texts):
        ref = o.encode(("search_query: " + t).encode(), 2048)
        assert counts[i] == len(ref)
        assert ids[i, :counts[i]].tolist() == ref, t
        assert mask[i].tolist() == [1] * counts[i] + [0] * (ids.shape[1] - counts[i])
        assert not ids[i, counts[i]:].any()
    # single-text entry point and short max_len agree too
    for t in texts[:200]:
        for ml in (5, 64):
            assert native30k.encode(t, ml)[0].tolist() == o.encode(t.encode(), ml)


def test_native_matches_oracle_on_random_bytes(vocab30k, native30k):
    """Invalid and truncated UTF-8, control bytes, mixed scripts."""
    o = wp.Tokenizer(vocab30k)
    rng = random.Random(5)
    alphabet = list(range(256)) + [ord(c) for c in "hello world abc,.!"] * 4
    texts = [bytes(rng.choice(alphabet) for _ in range(rng.randint(0, 48))) for _ in range(3000)]
    ids, _, counts = native30k.encode_batch(texts, 512)
    for i, t in enumerate(texts):
        assert ids[i, :counts[i]].tolist() == o.encode(t, 512), t


def test_native_every_code_point():
    """Every assigned code point (plus private-use and unassigned samples) through the native
    lowercase / space / punctuation tables: each is a token of its own, so the ids expose the
    lowercased code point and the word boundaries."""
    cps = [c for c in range(0x110000) if not 0xD800 <= c <= 0xDFFF and
           (unicodedata.category(chr(c)) not in ("Cn", "Co") or c % 997 == 0)]
    toks = kat_vocab()
    seen = set(toks)
    for c in cps + [wp.to_lower_rune(c) for c in cps] + [ord("q"), 0xFFFD]:
        for t in (chr(c), "▁" + chr(c)):
            if t not in seen:
                seen.add(t)
                toks.append(t)
    o = wp.Tokenizer(toks)
    nat = WordPieceTokenizer.from_tokens(toks)
    texts = ["q".join(chr(c) for c in cps[i:i + 400]).encode("utf-8") for i in range(0, len(cps), 400)]
    ids, _, counts = nat.encode_batch(texts, 4096)
    for i, t in enumerate(texts):
        assert ids[i, :counts[i]].tolist() == o.encode(t, 4096), i


def test_native_prefix_split_inside_a_character(vocab30k, native30k):
    """TaskPrefix + text is one Go string: a prefix ending inside a UTF-8 sequence joins the text."""
    v = kat_vocab()
    t = WordPieceTokenizer.from_tokens(v)
    ids, _, counts = t.encode_batch([b"\xa9"], 512, prefix=b"hello \xc3")
    assert ids[0, :counts[0]].tolist() == ids_of(v, ["▁hello", "▁é"])
    o = wp.Tokenizer(vocab30k)
    rng = random.Random(9)
    for _ in range(300):
        pre = bytes(rng.randint(0, 255) for _ in range(rng.randint(0, 6)))
        txt = bytes(rng.randint(0, 255) for _ in range(rng.randint(0, 6)))
        ids, _, counts = native30k.encode_batch([txt], 512, prefix=pre)
        assert ids[0, :counts[0]].tolist() == o.encode(pre + txt, 512)


def test_gguf_string_array_errors(tmp_path):
    """readGGUFStringArray: missing key, non-string element type, truncation."""
    kv_ok = [("general.architecture", gguf.T_STR, "nomic-bert"), ("x.n", gguf.T_U32, 3)]
    p1 = str(tmp_path / "nokey.gguf")
    gguf.write(p1, kv_ok, [])
    with pytest.raises(KeyError):
        wp.read_gguf_string_array(p1, "tokenizer.ggml.tokens")
    with pytest.raises(LLEError, match="ENOTFOUND"):
        WordPieceTokenizer.load(p1)
    p2 = str(tmp_path / "u32arr.gguf")
    gguf.write(p2, kv_ok + [("tokenizer.ggml.tokens", gguf.T_ARR, (gguf.T_U32, [1, 2, 3]))], [])
    with pytest.raises(ValueError):
        wp.read_gguf_string_array(p2, "tokenizer.ggml.tokens")
    with pytest.raises(LLEError, match="EIO"):
        WordPieceTokenizer.load(p2)
    p3 = str(tmp_path / "trunc.gguf")
    gguf.write(p3, kv_ok + [("tokenizer.ggml.tokens", gguf.T_ARR, (gguf.T_STR, ["a", "bb", "ccc"]))], [])
    data = open(p3, "rb").read()
    cut = data.index(b"ccc") + 1
    open(p3, "wb").write(data[:cut])
    with pytest.raises((EOFError, struct.error)):
        wp.read_gguf_string_array(p3, "tokenizer.ggml.tokens")
    with pytest.raises(LLEError, match="EIO"):
        WordPieceTokenizer.load(p3)
    with pytest.raises(LLEError, match="EIO"):
        WordPieceTokenizer.load(str(tmp_path / "missing.gguf"))
