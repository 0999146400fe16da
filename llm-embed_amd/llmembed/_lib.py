"""ctypes binding of libllmembed_hip.so (the C ABI declared in include/llmembed.h).

The product path is the HIP library; there is no CPU fallback here. Loading fails loudly
when the library is missing or no gfx950 device is present.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libllmembed_hip.so")

EXPORTS = [
    "lle_abi_version", "lle_init", "lle_last_error", "lle_info", "lle_f16_to_f32", "lle_dequant",
    "lle_model_create", "lle_model_load_gguf", "lle_model_destroy", "lle_model_dims", "lle_embed",
    "lle_embed_batch", "lle_embed_batch_async", "lle_forward_hidden", "lle_model_status",
    "lle_model_set_timing", "lle_model_set_timing_kernel", "lle_model_get_timing", "lle_weight_create", "lle_weight_destroy",
    "lle_weight_dequant", "lle_weight_dequant_f16", "lle_gemm", "lle_gemm_async", "lle_gemm_f16_async",
    "lle_tokenizer_load_gguf", "lle_tokenizer_create", "lle_tokenizer_destroy", "lle_tokenizer_vocab_size",
    "lle_tokenize", "lle_tokenize_batch", "lle_embed_texts", "lle_embed_packed_async", "lle_embed_packed_noalloc", "lle_model_set_precision",
]

ERRORS = {-1: "EINVAL", -2: "EDEVICE", -3: "ENOMEM", -4: "EUNSUPPORTED", -5: "EIO", -6: "ENOTFOUND"}


class LLEError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


class Tensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("ne0", C.c_int64), ("ne1", C.c_int64),
                ("data", C.c_void_p), ("nbytes", C.c_int64)]


class ModelDesc(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("d_model", C.c_int32), ("n_head", C.c_int32),
                ("d_ff", C.c_int32), ("max_seq", C.c_int32), ("ln_eps_bits", C.c_uint32),
                ("rope_base_bits", C.c_uint32), ("token_embd", Tensor), ("token_types", Tensor),
                ("embd_norm_w", Tensor), ("embd_norm_b", Tensor)] + [
        (n, C.POINTER(Tensor)) for n in ("qkv", "out", "attn_norm_w", "attn_norm_b", "up", "gate",
                                         "down", "out_norm_w", "out_norm_b")]


class KernelTime(C.Structure):
    _fields_ = [("name", C.c_char * 32), ("launches", C.c_int64), ("total_ms", C.c_double),
                ("flops", C.c_double), ("bytes", C.c_double)]


_LIB = None


def lib(path: str | None = None):
    global _LIB
    if _LIB is not None:
        return _LIB
    p = path or os.environ.get("LLE_LIB", LIB_PATH)
    if not os.path.exists(p):
        raise RuntimeError(f"{p} is missing: build it with `make -C llm-embed_amd` (or __graft_entry__.build())")
    L = C.CDLL(p)
    P, I32, I64 = C.c_void_p, C.c_int32, C.c_int64
    sig = {
        "lle_abi_version": ([], I32),
        "lle_init": ([I32], I32),
        "lle_last_error": ([], C.c_char_p),
        "lle_info": ([C.c_char_p, I32], I32),
        "lle_f16_to_f32": ([P, I64, P], I32),
        "lle_dequant": ([I32, P, I64, P], I32),
        "lle_model_create": ([C.POINTER(ModelDesc), C.POINTER(P)], I32),
        "lle_model_load_gguf": ([C.c_char_p, C.POINTER(P)], I32),
        "lle_model_destroy": ([P], I32),
        "lle_model_dims": ([P, P], I32),
        "lle_embed": ([P, P, P, I32, I32, P], I32),
        "lle_embed_batch": ([P, P, P, I32, I32, I32, P], I32),
        "lle_embed_batch_async": ([P, P, P, I32, I32, I32, P, P], I32),
        "lle_forward_hidden": ([P, P, P, I32, I32, P], I32),
        "lle_model_status": ([P, P], I32),
        "lle_model_set_timing": ([P, I32], I32),
        "lle_model_set_timing_kernel": ([P, C.c_char_p], I32),
        "lle_model_get_timing": ([P, C.POINTER(KernelTime), I32, P], I32),
        "lle_weight_create": ([I32, P, I32, I32, C.POINTER(P)], I32),
        "lle_weight_destroy": ([P], I32),
        "lle_weight_dequant": ([P, P], I32),
        "lle_weight_dequant_f16": ([P, P], I32),
        "lle_gemm": ([P, P, I32, P], I32),
        "lle_gemm_async": ([P, P, P, I32, P, P], I32),
        "lle_gemm_f16_async": ([P, P, I32, P, P, P], I32),
        "lle_tokenizer_load_gguf": ([C.c_char_p, C.POINTER(P)], I32),
        "lle_tokenizer_create": ([P, P, I32, C.POINTER(P)], I32),
        "lle_tokenizer_destroy": ([P], I32),
        "lle_tokenizer_vocab_size": ([P, P], I32),
        "lle_tokenize": ([P, C.c_char_p, I64, I32, P, I32, P], I32),
        "lle_tokenize_batch": ([P, P, P, I32, C.c_char_p, I64, I32, I32, P, P, P], I32),
        "lle_embed_texts": ([P, P, P, P, I32, C.c_char_p, I64, I32, I32, P], I32),
        "lle_embed_packed_async": ([P, P, P, I32, I32, I32, I32, P, P], I32),
        "lle_embed_packed_noalloc": ([P, P, P, I32, I32, I32, I32, P, P], I32),
        "lle_model_set_precision": ([P, I32], I32),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _LIB = L
    return L


def check(rc: int):
    if rc != 0:
        msg = lib().lle_last_error()
        raise LLEError(rc, msg.decode() if msg else "")
    return rc


def ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def init(device: int = 0):
    check(lib().lle_init(device))


def info() -> str:
    buf = C.create_string_buffer(1024)
    lib().lle_info(buf, 1024)
    return buf.value.decode()


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, np.uint16)
    out = np.empty(bits.size, np.float32)
    check(lib().lle_f16_to_f32(ptr(bits), bits.size, ptr(out)))
    return out


def dequant(t: int, blocks: np.ndarray, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty(n, np.float32)
    check(lib().lle_dequant(t, ptr(blocks), n, ptr(out)))
    return out


class Weight:
    """An uploaded quantised projection W [N][K] (GGUF dims [K, N])."""

    def __init__(self, t: int, blocks: np.ndarray, K: int, N: int):
        self._blocks = np.ascontiguousarray(blocks, np.uint8)
        h = C.c_void_p()
        check(lib().lle_weight_create(t, ptr(self._blocks), K, N, C.byref(h)))
        self.h, self.K, self.N, self.type = h, K, N, t
        self._blocks = None

    def dequant(self) -> np.ndarray:
        out = np.empty((self.N, self.K), np.float32)
        check(lib().lle_weight_dequant(self.h, ptr(out)))
        return out

    def dequant_f16(self) -> np.ndarray:
        """The GEMM's f16 operand values of this weight, [N][K] float16."""
        out = np.empty((self.N, self.K), np.uint16)
        check(lib().lle_weight_dequant_f16(self.h, ptr(out)))
        return out.view(np.float16)

    def gemm(self, X: np.ndarray) -> np.ndarray:
        X = np.ascontiguousarray(X, np.float32)
        M = X.shape[0]
        Y = np.empty((M, self.N), np.float32)
        check(lib().lle_gemm(self.h, ptr(X), M, ptr(Y)))
        return Y

    def part_floats(self, M: int) -> int:
        """Split-K workspace size of lle_gemm_f16_async below 1024 rows (0 from 1024)."""
        return ((self.K // 768) if self.K % 768 == 0 else (self.K // 256)) * M * self.N if M < 1024 else 0

    def gemm_f16_async(self, d_x16: int, M: int, d_y: int, d_part: int = 0, stream: int = 0):
        check(lib().lle_gemm_f16_async(self.h, d_x16, M, d_y, d_part or None, stream or None))

    def gemm_async(self, d_x: int, d_x16: int, M: int, d_y: int, stream: int = 0):
        check(lib().lle_gemm_async(self.h, C.c_void_p(d_x), C.c_void_p(d_x16), M, C.c_void_p(d_y),
                                   C.c_void_p(stream)))

    def close(self):
        if getattr(self, "h", None):
            lib().lle_weight_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
