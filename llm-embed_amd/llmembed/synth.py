"""Synthetic nomic-bert GGUF models and the benchmark configurations' inputs.

There is no network for the real nomic-embed-text-v1.5 checkpoint, so models are
random-init with the architecture the reference loads (internal/embed/bert.go:91-212):
  token_embd.weight [768, 30522], token_types.weight [768, 2] F32,
  token_embd_norm.{weight,bias} [768],
  blk.N.attn_qkv.weight [768, 2304], blk.N.attn_output.weight [768, 768],
  blk.N.attn_output_norm.{weight,bias}, blk.N.ffn_up.weight / ffn_gate.weight [768, 3072],
  blk.N.ffn_down.weight [3072, 768], blk.N.layer_output_norm.{weight,bias}.
Metadata keys and types follow bert.go:98-104 (u32 dims, f32 eps and rope base) and
tokenizer.go:23-27 (a string array of tokens), so the reference's Load() accepts the file.

Weight matrices and token_types are N(0, 0.02); LayerNorm gamma = 1 + 0.05 N(0,1) and
beta = 0.05 N(0,1) (so the affine part of every LayerNorm is exercised), stored F32.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np

from . import gguf
from .quant import F32, Q4_K, Q5_K, Q6_K, Q8_0, quantize

ARCH = "nomic-bert"
DOWN_Q6_LAYERS = (0, 3, 6, 9, 11)  # llama.cpp-like *_M mixtures: ffn_down promoted on these


@dataclass(frozen=True)
class ModelSpec:
    n_layer: int = 12
    d_model: int = 768
    n_head: int = 12
    d_ff: int = 3072
    vocab: int = 30522
    ctx: int = 2048
    eps: float = 1e-12
    rope_base: float = 1000.0


def mixture_types(mix: str, layer: int) -> dict:
    """Per-tensor ggml types of one layer for a named quantisation mixture."""
    pure = {"Q8_0": Q8_0, "Q6_K": Q6_K, "Q5_K": Q5_K, "Q4_K": Q4_K, "F32": F32}
    if mix in pure:
        t = pure[mix]
        return dict(qkv=t, out=t, up=t, gate=t, down=t, embd=t)
    if mix == "Q4_K_M":
        return dict(qkv=Q5_K, out=Q4_K, up=Q4_K, gate=Q4_K,
                    down=Q6_K if layer in DOWN_Q6_LAYERS else Q4_K, embd=Q4_K)
    if mix == "Q5_K_M":
        return dict(qkv=Q6_K, out=Q5_K, up=Q5_K, gate=Q5_K,
                    down=Q6_K if layer in DOWN_Q6_LAYERS else Q5_K, embd=Q5_K)
    raise ValueError(f"unknown mixture {mix}")


# --------------------------------------------------------------------------------------
# Synthetic vocabulary and text. The real nomic vocabulary (BERT uncased WordPiece as llama.cpp
# converts it: word-initial pieces carry "▁", continuation pieces lose their "##") is not
# available, so the vocabulary is generated in that shape: specials at BERT's ids, single
# characters with and without "▁", then words of a pseudo-English syllable lexicon (with "▁")
# and continuation pieces (without).

VOCAB_SEED = 0x70C4B
_SYL_ONSETS = ["", "b", "c", "d", "f", "g", "h", "j", "k", "l", "m", "n", "p", "r", "s", "t", "v", "w", "z",
               "br", "ch", "cl", "cr", "dr", "fl", "gr", "pl", "pr", "sh", "st", "th", "tr"]
_SYL_VOWELS = ["a", "e", "i", "o", "u", "ai", "ea", "ee", "io", "ou", "y"]
_SYL_CODAS = ["", "", "", "n", "r", "s", "t", "l", "m", "nd", "ng", "st", "ck"]
_EXTRA_CHARS = ("àáâäçèéêëìíîïñòóôöùúûüýÿßøåæœ"  # Latin-1 / Latin Extended lowercase
                "αβγδεζηθικλμνξοπρστυφχψω"        # Greek
                "абвгдежзийклмнопрстуфхцчшщыьэюя"  # Cyrillic
                "的一是不了在人有我他这个们中来上大为和国地到以说时要就出会")  # CJK


def lexicon(n: int, seed: int = VOCAB_SEED) -> list:
    """n distinct pseudo-English words of 1-4 syllables (deterministic)."""
    rng = np.random.default_rng(seed)
    words, seen = [], set()
    while len(words) < n:
        k = int(rng.choice([1, 2, 2, 3, 3, 4]))
        w = "".join(_SYL_ONSETS[rng.integers(len(_SYL_ONSETS))] + _SYL_VOWELS[rng.integers(len(_SYL_VOWELS))] +
                    _SYL_CODAS[rng.integers(len(_SYL_CODAS))] for _ in range(k))
        if 2 <= len(w) <= 16 and w not in seen:
            seen.add(w)
            words.append(w)
    return words


def _tokens(vocab: int) -> list:
    """Vocabulary of `vocab` distinct tokens: [PAD]=0, [UNK]=100, [CLS]=101, [SEP]=102,
    [MASK]=103, [unusedN] fillers below 999, then characters, words and pieces."""
    toks = [f"[unused{i}]" for i in range(min(vocab, 999))]
    toks[0] = "[PAD]"
    for i, s in {100: "[UNK]", 101: "[CLS]", 102: "[SEP]", 103: "[MASK]"}.items():
        if i < vocab:
            toks[i] = s
    seen = set(toks)
    extra = []

    def add(t):
        if t not in seen:
            seen.add(t)
            extra.append(t)

    chars = [chr(c) for c in range(0x21, 0x7F) if not "A" <= chr(c) <= "Z"] + list(_EXTRA_CHARS)
    for c in chars:
        add("▁" + c)
        add(c)
    for w in ("hello", "world", "search", "query", "document", "what", "is", "machine", "learning"):
        add("▁" + w)
    for suf in ("s", "es", "ed", "ing", "er", "ers", "ly", "tion", "ment", "ness", "able", "al", "ic", "ize"):
        add(suf)
    room = max(0, vocab - len(toks) - len(extra))
    words = lexicon(room)
    n_words = (room * 3) // 4
    for w in words[:n_words]:
        add("▁" + w)
    # continuation pieces: syllables and word tails
    for on in _SYL_ONSETS:
        for v in _SYL_VOWELS:
            for cd in _SYL_CODAS:
                if len(toks) + len(extra) < vocab:
                    add(on + v + cd)
    for w in words[n_words:]:
        if len(toks) + len(extra) >= vocab:
            break
        add(w[len(w) // 2:])
    i = 0
    while len(toks) + len(extra) < vocab:  # top up with digit strings
        add(str(i))
        i += 1
    return (toks + extra)[:vocab]


def texts(n: int, seed: int, min_words: int = 4, max_words: int = 90) -> list:
    """n synthetic texts: sentences over the lexicon (mostly in-vocabulary words, some unseen
    words that split into pieces), numbers, punctuation, capitals, a little non-ASCII."""
    rng = np.random.default_rng(seed)
    lex = lexicon(6000)
    out = []
    for _ in range(n):
        k = int(rng.integers(min_words, max_words + 1))
        ws = []
        for j in range(k):
            r = rng.random()
            if r < 0.75:
                w = lex[min(int(rng.zipf(1.3)) - 1, len(lex) - 1)]
            elif r < 0.88:
                w = lex[int(rng.integers(len(lex)))] + lex[int(rng.integers(len(lex)))][:3]
            elif r < 0.93:
                w = str(int(rng.integers(0, 100000)))
            elif r < 0.97:
                w = "".join(_EXTRA_CHARS[int(rng.integers(len(_EXTRA_CHARS)))] for _ in range(int(rng.integers(1, 4))))
            else:
                w = "🙂" if rng.random() < 0.5 else "naïve"
            if j == 0 or rng.random() < 0.08:
                w = w[:1].upper() + w[1:]
            if rng.random() < 0.1:
                w += ",.;:!?"[int(rng.integers(6))]
            ws.append(w)
        out.append(" ".join(ws))
    return out


def build_tensors(spec: ModelSpec, mix: str, seed: int, qkv_std: float = 0.02):
    """Returns (kvs, tensors) ready for gguf.write. qkv_std > 0.02 makes attention logits
    large enough that the softmax's x < -10 cutoff is active (used by parity tests)."""
    rng = np.random.default_rng(seed)
    D, F = spec.d_model, spec.d_ff

    def normal(*shape, std=0.02):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    def ln_pair():
        w = (1.0 + 0.05 * rng.standard_normal(D, dtype=np.float32)).astype(np.float32)
        b = (0.05 * rng.standard_normal(D, dtype=np.float32)).astype(np.float32)
        return w, b

    tensors = []

    def add(name, t, x, dims):
        tensors.append((name, dims, t, quantize(t, x, rng).reshape(-1)))

    t0 = mixture_types(mix, 0)
    add("token_embd.weight", t0["embd"], normal(spec.vocab, D), [D, spec.vocab])
    add("token_types.weight", F32, normal(2, D), [D, 2])
    w, b = ln_pair()
    add("token_embd_norm.weight", F32, w, [D])
    add("token_embd_norm.bias", F32, b, [D])
    for l in range(spec.n_layer):
        ty = mixture_types(mix, l)
        p = f"blk.{l}."
        add(p + "attn_qkv.weight", ty["qkv"], normal(3 * D, D, std=qkv_std), [D, 3 * D])
        add(p + "attn_output.weight", ty["out"], normal(D, D), [D, D])
        w, b = ln_pair()
        add(p + "attn_output_norm.weight", F32, w, [D])
        add(p + "attn_output_norm.bias", F32, b, [D])
        add(p + "ffn_up.weight", ty["up"], normal(F, D), [D, F])
        add(p + "ffn_gate.weight", ty["gate"], normal(F, D), [D, F])
        add(p + "ffn_down.weight", ty["down"], normal(D, F), [F, D])
        w, b = ln_pair()
        add(p + "layer_output_norm.weight", F32, w, [D])
        add(p + "layer_output_norm.bias", F32, b, [D])

    kvs = [
        ("general.architecture", gguf.T_STR, ARCH),
        ("general.name", gguf.T_STR, f"synthetic-nomic-bert-{mix}"),
        (f"{ARCH}.block_count", gguf.T_U32, spec.n_layer),
        (f"{ARCH}.context_length", gguf.T_U32, spec.ctx),
        (f"{ARCH}.embedding_length", gguf.T_U32, D),
        (f"{ARCH}.feed_forward_length", gguf.T_U32, F),
        (f"{ARCH}.attention.head_count", gguf.T_U32, spec.n_head),
        (f"{ARCH}.attention.layer_norm_epsilon", gguf.T_F32, spec.eps),
        (f"{ARCH}.rope.freq_base", gguf.T_F32, spec.rope_base),
        ("llmembed.synthetic.seed", gguf.T_U64, seed),
        ("llmembed.synthetic.mixture", gguf.T_STR, mix),
        ("llmembed.synthetic.init", gguf.T_STR,
         "matrices N(0,0.02); LN gamma 1+0.05N(0,1), beta 0.05N(0,1)"),
        ("tokenizer.ggml.tokens", gguf.T_ARR, (gguf.T_STR, _tokens(spec.vocab))),
    ]
    return kvs, tensors


def cache_dir() -> str:
    d = os.environ.get("LLE_CACHE")
    if not d:
        d = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))), "_cache")
    os.makedirs(d, exist_ok=True)
    return d


def model_path(spec: ModelSpec, mix: str, seed: int, qkv_std: float = 0.02) -> str:
    """Write (once) and return the path of a synthetic GGUF for (spec, mix, seed)."""
    name = (f"nomicbert_L{spec.n_layer}_d{spec.d_model}_h{spec.n_head}_f{spec.d_ff}_v{spec.vocab}"
            f"_c{spec.ctx}_{mix}_s{seed}" + ("" if qkv_std == 0.02 else f"_q{qkv_std:g}") + "_tk2.gguf")
    path = os.path.join(cache_dir(), name)
    if not os.path.exists(path):
        kvs, tensors = build_tensors(spec, mix, seed, qkv_std)
        tmp = path + f".tmp{os.getpid()}"
        gguf.write(tmp, kvs, tensors)
        os.replace(tmp, path)
    return path


# --------------------------------------------------------------------------------------
# Benchmark configurations (inputs as token ids + attention mask)

CONFIG_SEED = 0x11E3B0


def config_inputs(cfg: int, vocab: int = 30522, seed: int | None = None):
    """Token ids and masks [B][L] (int32) for configs 1, 3, 4, 5."""
    rng = np.random.default_rng(CONFIG_SEED + 1000 + cfg if seed is None else seed)
    if cfg == 1:
        ids = np.concatenate([[101], rng.integers(1000, 30522, 6), [102]]).astype(np.int32)[None, :]
        return ids, np.ones_like(ids)
    if cfg == 3:
        B, L = 64, 128
        lens = rng.integers(16, 129, B)
        return _padded(rng, B, L, lens, vocab)
    if cfg == 4:
        B, L = 256, 128
        ids = rng.integers(0, vocab, (B, L)).astype(np.int32)
        ids[:, 0], ids[:, -1] = 101, 102
        return ids, np.ones_like(ids)
    if cfg == 5:
        B, L = 8, 2048
        lens = rng.integers(1024, 2049, B)
        return _padded(rng, B, L, lens, vocab)
    raise ValueError(f"config {cfg} has no token inputs")


def _padded(rng, B, L, lens, vocab):
    ids = np.zeros((B, L), np.int32)
    mask = np.zeros((B, L), np.int32)
    for i, n in enumerate(lens):
        ids[i, :n] = rng.integers(0, vocab, n)
        mask[i, :n] = 1
    return ids, mask


CONFIG_MIX = {1: "Q8_0", 3: "Q4_K_M", 4: "Q8_0", 5: "Q8_0"}
