"""Host-side mirror of the reference's embed API over the HIP C ABI.

Reference: internal/embed/embedder.go
  Embedder{model, tokenizer, targetDim, TaskPrefix}    :11-16
  Load(modelPath)                                        :19-42
  (*Embedder).Embed(text)                                :46-71
  (*Embedder).EmbedBatch(texts)                          :75-133
  Dim / SetTargetDim / Model                             :136-153
Embed and EmbedBatch take text, as the reference's do: TaskPrefix + text is tokenised by the
library's native tokeniser (internal/embed/tokenizer.go restated in C++) and embedded on the GPU.
They also take token ids (what Encode returns: [CLS] ... [SEP], mask all ones). EmbedBatch is
truly batched: texts are ordered by length and run as padded [B][L] forwards, each row
bit-identical to Embed of that text.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import LLEError, check, ptr
from .tokenizer import WordPieceTokenizer, _as_bytes, _TextArray


class BertModel:
    """Device-resident nomic-bert model (BertModel + PreDequant, internal/embed/bert.go:14-87,542-576)."""

    def __init__(self, handle: C.c_void_p):
        self.h = handle
        dims = np.zeros(6, np.int32)
        check(_lib.lib().lle_model_dims(self.h, ptr(dims)))
        (self.num_layers, self.hidden_dim, self.num_heads, self.ffn_dim, self.max_seq_len,
         self.vocab_size) = (int(x) for x in dims)
        self.head_dim = self.hidden_dim // self.num_heads

    @classmethod
    def load(cls, path: str) -> "BertModel":
        """LoadBertModel (bert.go:91-212) + upload."""
        h = C.c_void_p()
        check(_lib.lib().lle_model_load_gguf(path.encode(), C.byref(h)))
        return cls(h)

    def forward(self, ids, mask=None) -> np.ndarray:
        """Forward (bert.go:216-285): hidden states [L][hidden_dim] of one sequence, or
        [B][L][hidden_dim] of a padded batch."""
        ids = np.ascontiguousarray(ids, np.int32)
        single = ids.ndim == 1
        ids2 = ids[None, :] if single else ids
        mask2 = np.ones_like(ids2) if mask is None else np.ascontiguousarray(mask, np.int32).reshape(ids2.shape)
        B, L = ids2.shape
        out = np.empty((B, L, self.hidden_dim), np.float32)
        check(_lib.lib().lle_forward_hidden(self.h, ptr(ids2), ptr(mask2), B, L, ptr(out)))
        return out[0] if single else out

    def set_precision(self, precision: str):
        """'f16' (default): MFMA GEMMs on f16 operands, within the reference's tolerance. 'f32':
        the reference CPU path's own f32 arithmetic in its order (exact f32 weight copies are
        made on the first switch), embeddings equal to the reference's bit for bit."""
        code = {"f16": 0, "f32": 1}[precision]
        check(_lib.lib().lle_model_set_precision(self.h, code))

    def set_timing(self, on: bool):
        check(_lib.lib().lle_model_set_timing(self.h, 1 if on else 0))

    def set_timing_kernel(self, kernel_class: str | None):
        """Time only the launches of one kernel class (no per-forward synchronisation)."""
        check(_lib.lib().lle_model_set_timing_kernel(self.h, kernel_class.encode() if kernel_class else None))

    def timing(self) -> dict:
        n = C.c_int32()
        arr = (_lib.KernelTime * 64)()
        check(_lib.lib().lle_model_get_timing(self.h, arr, 64, C.byref(n)))
        return {arr[i].name.decode(): dict(launches=arr[i].launches, total_ms=arr[i].total_ms,
                                           flops=arr[i].flops, bytes=arr[i].bytes)
                for i in range(min(n.value, 64))}

    def close(self):
        if getattr(self, "h", None):
            _lib.lib().lle_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Embedder:
    """Public embedding API (embedder.go:11-16)."""

    def __init__(self, model: BertModel, tokenizer: WordPieceTokenizer | None = None):
        self._model = model
        self.tokenizer = tokenizer
        self.target_dim = model.hidden_dim
        self.task_prefix = "search_query: "  # embedder.go:40, prepended to text (:48)

    @classmethod
    def load(cls, model_path: str) -> "Embedder":
        """Load (embedder.go:19-42): model (uploaded, weights resident) and tokenizer."""
        try:
            m = BertModel.load(model_path)
        except LLEError as e:
            raise LLEError(e.code, f"embed: load model: {e}") from None
        return cls(m, WordPieceTokenizer.load(model_path))

    def _tok(self) -> WordPieceTokenizer:
        if self.tokenizer is None:
            raise LLEError(-1, "embed: no tokenizer (construct with one, or use Embedder.load)")
        return self.tokenizer

    def embed(self, ids, mask=None) -> np.ndarray:
        """Embed (embedder.go:46-71): forward + MeanPool + L2Normalize (+ Matryoshka). `ids` is
        text (str / bytes: TaskPrefix + text is tokenised) or one sequence of token ids."""
        if isinstance(ids, (str, bytes, bytearray)):
            return self.embed_batch([ids])[0]
        ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
        mask = np.ones_like(ids) if mask is None else np.ascontiguousarray(mask, np.int32).reshape(-1)
        out = np.empty(min(self.target_dim, self._model.hidden_dim), np.float32)
        rc = _lib.lib().lle_embed(self._model.h, ptr(ids), ptr(mask), ids.size, self.target_dim, ptr(out))
        if rc:
            raise LLEError(rc, f"embed: forward: {_lib.lib().lle_last_error().decode()}")
        return out

    def embed_texts(self, texts, max_batch_tokens: int = 0) -> np.ndarray:
        """EmbedBatch over text through lle_embed_texts: [n][dim], row i = Embed(texts[i])."""
        arr = _TextArray(texts)
        pb = _as_bytes(self.task_prefix)
        out = np.empty((arr.n, min(self.target_dim, self._model.hidden_dim)), np.float32)
        if arr.n:
            rc = _lib.lib().lle_embed_texts(self._model.h, self._tok().h, C.cast(arr.ptrs, C.c_void_p), ptr(arr.lens),
                                            arr.n, pb, len(pb), self.target_dim, max_batch_tokens, ptr(out))
            if rc:
                raise LLEError(rc, f"embed: batch: {_lib.lib().lle_last_error().decode()}")
        return out

    def embed_batch(self, seqs) -> list | None:
        """EmbedBatch (embedder.go:75-133), truly batched. `seqs` is a list of texts (str /
        bytes) or of token-id sequences; returns a list of vectors in input order."""
        n = len(seqs)
        if n == 0:
            return None
        if all(isinstance(s, (str, bytes, bytearray)) for s in seqs):
            return list(self.embed_texts(seqs))
        if n == 1:
            return [self.embed(seqs[0])]
        lens = [len(s) for s in seqs]
        L = max(lens)
        ids = np.zeros((n, L), np.int32)
        mask = np.zeros((n, L), np.int32)
        for i, s in enumerate(seqs):
            ids[i, :lens[i]] = s
            mask[i, :lens[i]] = 1
        return list(self.embed_padded(ids, mask))

    def embed_padded(self, ids, mask) -> np.ndarray:
        """Batched embed of a right-padded [B][L] id matrix with its attention mask."""
        ids = np.ascontiguousarray(ids, np.int32)
        mask = np.ascontiguousarray(mask, np.int32)
        B, L = ids.shape
        out = np.empty((B, min(self.target_dim, self._model.hidden_dim)), np.float32)
        rc = _lib.lib().lle_embed_batch(self._model.h, ptr(ids), ptr(mask), B, L, self.target_dim, ptr(out))
        if rc:
            raise LLEError(rc, f"embed: batch: {_lib.lib().lle_last_error().decode()}")
        return out

    def dim(self) -> int:
        return self.target_dim

    def set_target_dim(self, dim: int):
        """SetTargetDim (embedder.go:142-150): clamp to [1, hidden_dim]."""
        self.target_dim = max(1, min(int(dim), self._model.hidden_dim))

    def model(self) -> BertModel:
        return self._model
