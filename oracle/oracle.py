"""ctypes binding of the C oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker / CPU baseline. The product never imports this.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.join(os.path.dirname(_HERE), "llm-embed_amd")
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

from llmembed import gguf  # noqa: E402

_LIB = None


class Tensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("ne0", C.c_int64), ("ne1", C.c_int64),
                ("data", C.c_void_p), ("nbytes", C.c_int64)]


class ModelDesc(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("d_model", C.c_int32), ("n_head", C.c_int32),
                ("d_ff", C.c_int32), ("max_seq", C.c_int32), ("ln_eps", C.c_float),
                ("rope_base", C.c_float), ("token_embd", Tensor), ("token_types", Tensor),
                ("embd_norm_w", Tensor), ("embd_norm_b", Tensor)] + [
        (n, C.POINTER(Tensor)) for n in ("qkv", "out", "attn_norm_w", "attn_norm_b", "up", "gate",
                                         "down", "out_norm_w", "out_norm_b")]


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        P = C.c_void_p
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32_array.argtypes = [P, C.c_int64, P]
        L.orc_dequant.argtypes = [C.c_int32, P, C.c_int64, P]
        L.orc_gemm.argtypes = [P, C.c_int32, C.c_int32, P, C.c_int32, P, C.c_int32]
        L.orc_layernorm.argtypes = [P, P, P, C.c_float, C.c_int32]
        L.orc_gelu.argtypes = [P, C.c_int32]
        L.orc_softmax.argtypes = [P, C.c_int32]
        L.orc_dotf32.restype = C.c_float
        L.orc_dotf32.argtypes = [P, P, C.c_int32]
        L.orc_rope_table.argtypes = [C.c_int32, C.c_int32, C.c_float, P, P]
        L.orc_rope_apply.argtypes = [P, P, P, C.c_int32]
        L.orc_mean_pool.argtypes = [P, P, C.c_int32, C.c_int32, P]
        L.orc_l2_normalize.argtypes = [P, C.c_int32, P]
        L.orc_get_scale_min_k4.argtypes = [C.c_int32, P, P, P]
        L.orc_model_create.argtypes = [C.POINTER(ModelDesc), C.POINTER(C.c_void_p)]
        L.orc_model_destroy.argtypes = [P]
        L.orc_set_threads.argtypes = [P, C.c_int32, C.c_int32]
        L.orc_forward.argtypes = [P, P, P, C.c_int32, P]
        L.orc_embed.argtypes = [P, P, P, C.c_int32, C.c_int32, P]
        L.orc_embed_batch.argtypes = [P, P, P, C.c_int32, C.c_int32, C.c_int32, P, C.c_int32]
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def f16_to_f32(h) -> np.ndarray:
    """f16 bit patterns -> f32 array (bit-exact, NaN payloads included)."""
    h = np.ascontiguousarray(np.atleast_1d(h), np.uint16)
    out = np.empty(h.size, np.float32)
    lib().orc_f16_to_f32_array(_p(h), h.size, _p(out))
    return out


def dequant(t: int, data: np.ndarray, n: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n, np.float32)
    if lib().orc_dequant(t, _p(data), n, _p(out)) != 0:
        raise ValueError(f"oracle: unsupported type {t}")
    return out


def gemm(A: np.ndarray, W: np.ndarray, threads: int = 0) -> np.ndarray:
    """C = A @ W.T in the reference GemmPrePacked32 order. A [M,K] f32, W [N,K] f32."""
    A = np.ascontiguousarray(A, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    M, K = A.shape
    N = W.shape[0]
    Cm = np.empty((M, N), np.float32)
    lib().orc_gemm(_p(A), M, K, _p(W), N, _p(Cm), threads)
    return Cm


def layernorm(x, w, b, eps):
    x = np.array(x, np.float32, copy=True)
    w = np.ascontiguousarray(w, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    lib().orc_layernorm(_p(x), _p(w), _p(b), C.c_float(eps), x.size)
    return x


def gelu(x):
    x = np.array(x, np.float32, copy=True)
    lib().orc_gelu(_p(x), x.size)
    return x


def softmax(x):
    x = np.array(x, np.float32, copy=True)
    lib().orc_softmax(_p(x), x.size)
    return x


def rope_table(max_pos, head_dim, base):
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_table(max_pos, head_dim, C.c_float(base), _p(c), _p(s))
    return c, s


def mean_pool(h, mask):
    h = np.ascontiguousarray(h, np.float32)
    mask = np.ascontiguousarray(mask, np.int32)
    out = np.empty(h.shape[1], np.float32)
    lib().orc_mean_pool(_p(h), _p(mask), h.shape[0], h.shape[1], _p(out))
    return out


def l2_normalize(v):
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty_like(v)
    lib().orc_l2_normalize(_p(v), v.size, _p(out))
    return out


class OracleModel:
    """The reference model after Load(): LoadBertModel + PreDequant + RoPE table."""

    def __init__(self, path: str):
        g = gguf.read(path)
        self.g = g
        a = "nomic-bert."
        self.n_layer = g.get_u32(a + "block_count")
        self.d_model = g.get_u32(a + "embedding_length")
        self.d_ff = g.get_u32(a + "feed_forward_length")
        self.n_head = g.get_u32(a + "attention.head_count")
        self.max_seq = g.get_u32(a + "context_length")
        self.eps = g.get_f32(a + "attention.layer_norm_epsilon")
        self.rope_base = g.get_f32(a + "rope.freq_base")
        self._keep = []

        def t(name):
            ti = g.tensors[name]
            data = np.ascontiguousarray(g.tensor_bytes(name))
            self._keep.append(data)
            ne1 = int(ti.dims[1]) if len(ti.dims) > 1 else 1
            return Tensor(ti.type, int(ti.dims[0]), ne1, data.ctypes.data, data.nbytes)

        def arr(suffix):
            a_ = (Tensor * self.n_layer)(*[t(f"blk.{l}.{suffix}") for l in range(self.n_layer)])
            self._keep.append(a_)
            return a_

        tok = t("token_embd.weight")
        self._tok = self._keep[-1]
        d = ModelDesc(self.n_layer, self.d_model, self.n_head, self.d_ff, self.max_seq, self.eps,
                      self.rope_base, tok, t("token_types.weight"),
                      t("token_embd_norm.weight"), t("token_embd_norm.bias"),
                      arr("attn_qkv.weight"), arr("attn_output.weight"),
                      arr("attn_output_norm.weight"), arr("attn_output_norm.bias"),
                      arr("ffn_up.weight"), arr("ffn_gate.weight"), arr("ffn_down.weight"),
                      arr("layer_output_norm.weight"), arr("layer_output_norm.bias"))
        h = C.c_void_p()
        if lib().orc_model_create(C.byref(d), C.byref(h)) != 0:
            raise RuntimeError("oracle: model create failed")
        self.h = h
        # The oracle dequantises every matrix and vector at create time but gathers
        # token_embd rows from the raw bytes per call, so only that buffer must stay alive.
        self._keep = None

    def set_threads(self, gemm: int = 0, attn: int = 0):
        lib().orc_set_threads(self.h, gemm, attn)

    def forward(self, ids, mask=None):
        ids = np.ascontiguousarray(ids, np.int32)
        mask = np.ones_like(ids) if mask is None else np.ascontiguousarray(mask, np.int32)
        L = ids.size
        out = np.empty((L, self.d_model), np.float32)
        rc = lib().orc_forward(self.h, _p(ids), _p(mask), L, _p(out))
        if rc:
            raise RuntimeError(f"oracle forward failed ({rc})")
        return out

    def embed(self, ids, mask=None, out_dim=None):
        ids = np.ascontiguousarray(ids, np.int32)
        mask = np.ones_like(ids) if mask is None else np.ascontiguousarray(mask, np.int32)
        od = self.d_model if out_dim is None else out_dim
        out = np.empty(min(od, self.d_model), np.float32)
        rc = lib().orc_embed(self.h, _p(ids), _p(mask), ids.size, od, _p(out))
        if rc:
            raise RuntimeError(f"oracle embed failed ({rc})")
        return out

    def embed_batch(self, ids, mask, out_dim=None, workers: int = 0):
        ids = np.ascontiguousarray(ids, np.int32)
        mask = np.ascontiguousarray(mask, np.int32)
        B, L = ids.shape
        od = self.d_model if out_dim is None else out_dim
        out = np.empty((B, min(od, self.d_model)), np.float32)
        rc = lib().orc_embed_batch(self.h, _p(ids), _p(mask), B, L, od, _p(out), workers)
        if rc:
            raise RuntimeError(f"oracle embed_batch failed ({rc})")
        return out

    def __del__(self):
        try:
            if getattr(self, "h", None):
                lib().orc_model_destroy(self.h)
                self.h = None
        except Exception:
            pass
