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


def _tokens(vocab: int) -> list:
    toks = [f"[unused{i}]" for i in range(vocab)]
    toks[0] = "[PAD]"
    for i, s in {100: "[UNK]", 101: "[CLS]", 102: "[SEP]", 103: "[MASK]"}.items():
        if i < vocab:
            toks[i] = s
    for i in range(1000, vocab):
        toks[i] = f"▁t{i}"
    return toks


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
            f"_c{spec.ctx}_{mix}_s{seed}" + ("" if qkv_std == 0.02 else f"_q{qkv_std:g}") + ".gguf")
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
