"""llmembed: MI355X (gfx950) nomic-bert encoder forward pass behind the llm-embed API.

The compute path is libllmembed_hip.so (hand-written HIP kernels); this package is the host
mirror of the reference's embed API plus the GGUF tooling used by tests and benchmarks.
"""
from . import gguf, quant, synth  # noqa: F401
from ._lib import LLEError, Weight, dequant, f16_to_f32, info, init, lib  # noqa: F401
from .embedder import BertModel, Embedder  # noqa: F401
from .tokenizer import WordPieceTokenizer  # noqa: F401

__all__ = ["gguf", "quant", "synth", "LLEError", "Weight", "dequant", "f16_to_f32", "info", "init", "lib",
           "BertModel", "Embedder", "WordPieceTokenizer"]
