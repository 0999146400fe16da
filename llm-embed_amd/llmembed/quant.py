"""GGML block quantisers for synthetic models (numpy, vectorised).

The reference only reads and dequantises GGUF weights; it has no quantiser. These
produce valid, fully-exercised bit fields for the block layouts the reference decodes:

* Q8_0  34 B / 32:  {f16 d, int8 q[32]}                        internal/ggml/tensor.go:119-159
* Q4_K 144 B / 256: {f16 d, f16 dmin, scales[12], qs[128]}     internal/ggml/quant_q4k.go:8-77
* Q5_K 176 B / 256: {f16 d, f16 dmin, scales[12], qh[32], qs[128]}  internal/ggml/quant_q5k.go:5-91
* Q6_K 210 B / 256: {ql[128], qh[64], int8 scales[16], f16 d}  internal/ggml/quant_q6k.go:5-75

The 6-bit scale/min packing is the inverse of getScaleMinK4 (quant_q4k.go:133-140).
Quantisation quality is not a parity concern: parity is defined on the dequantised values.
"""
from __future__ import annotations

import numpy as np

F32, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14
TYPE_NAMES = {F32: "F32", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
BLOCK = {F32: 1, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def row_bytes(t: int, n: int) -> int:
    """ByteSize of n elements (internal/gguf/reader.go:196-204)."""
    return (n // BLOCK[t]) * TYPE_SIZE[t]


def _f16(x: np.ndarray) -> np.ndarray:
    """Round to f16 (nearest-even) and return the f16 array."""
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def _safe_div(a, b):
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(b != 0, a / np.where(b != 0, b, 1), 0)
    return r


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """x: [..., K] f32 with K % 32 == 0 -> uint8 [..., K/32*34]."""
    x = np.asarray(x, dtype=np.float32)
    lead = x.shape[:-1]
    K = x.shape[-1]
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    d = amax / 127.0
    idv = _safe_div(np.float32(1.0), d.astype(np.float32)).astype(np.float32)
    q = np.clip(np.rint(b * idv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = _f16(d).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(*lead, (K // 32) * 34)


def _pack_scales_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of getScaleMinK4: sc, m [nb, 8] in 0..63 -> scales [nb, 12]."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    s = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    s[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    s[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    return s


def _kquant_affine(b: np.ndarray, nmax: int):
    """Sub-block affine quantisation x ~ d*sc*q - dmin*m with q in [0, nmax]."""
    nb = b.shape[0]
    sub = b.reshape(nb, 8, 32)
    mn = np.minimum(sub.min(axis=2), 0.0)
    mx = sub.max(axis=2)
    scale = (mx - mn) / nmax
    mins = -mn
    d16 = _f16(scale.max(axis=1) / 63.0)
    dm16 = _f16(mins.max(axis=1) / 63.0)
    d = d16.astype(np.float32)
    dm = dm16.astype(np.float32)
    sc = np.clip(np.rint(_safe_div(scale, d[:, None])), 0, 63).astype(np.uint8)
    mq = np.clip(np.rint(_safe_div(mins, dm[:, None])), 0, 63).astype(np.uint8)
    ds = (d[:, None] * sc.astype(np.float32))[:, :, None]
    dms = (dm[:, None] * mq.astype(np.float32))[:, :, None]
    q = np.clip(np.rint(_safe_div(sub + dms, ds)), 0, nmax).astype(np.uint8)
    return d16, dm16, sc, mq, q.reshape(nb, 256)


def quantize_q4_k(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    lead, K = x.shape[:-1], x.shape[-1]
    b = x.reshape(-1, 256)
    d16, dm16, sc, mq, q = _kquant_affine(b, 15)
    nb = b.shape[0]
    out = np.zeros((nb, 144), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dm16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = _pack_scales_k4(sc, mq)
    qg = q.reshape(nb, 4, 2, 32)  # group g: first 32 low nibble, next 32 high nibble
    out[:, 16:144] = ((qg[:, :, 0, :] & 0xF) | ((qg[:, :, 1, :] & 0xF) << 4)).reshape(nb, 128)
    return out.reshape(*lead, (K // 256) * 144)


def quantize_q5_k(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    lead, K = x.shape[:-1], x.shape[-1]
    b = x.reshape(-1, 256)
    d16, dm16, sc, mq, q = _kquant_affine(b, 31)
    nb = b.shape[0]
    out = np.zeros((nb, 176), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dm16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = _pack_scales_k4(sc, mq)
    qs = q.reshape(nb, 8, 32)  # sub-group s, position l
    hb = (qs >> 4) & 1
    qh = np.zeros((nb, 32), dtype=np.uint8)
    for s in range(8):
        qh |= (hb[:, s, :] << s).astype(np.uint8)
    out[:, 16:48] = qh
    qg = q.reshape(nb, 4, 2, 32)
    out[:, 48:176] = ((qg[:, :, 0, :] & 0xF) | ((qg[:, :, 1, :] & 0xF) << 4)).reshape(nb, 128)
    return out.reshape(*lead, (K // 256) * 176)


def quantize_q6_k(x: np.ndarray, rng: np.random.Generator | None = None) -> np.ndarray:
    """Symmetric 6-bit codes with int8 per-16 scales; when rng is given, half of the
    sub-block scales are stored negative (with negated codes) to exercise the sign bit."""
    x = np.asarray(x, dtype=np.float32)
    lead, K = x.shape[:-1], x.shape[-1]
    b = x.reshape(-1, 256)
    nb = b.shape[0]
    sub = b.reshape(nb, 16, 16)
    amax = np.abs(sub).max(axis=2)
    scale = amax / 31.0
    d16 = _f16(scale.max(axis=1) / 127.0)
    d = d16.astype(np.float32)
    sc = np.clip(np.rint(_safe_div(scale, d[:, None])), 0, 127).astype(np.int16)
    if rng is not None:
        neg = rng.random(sc.shape) < 0.5
        sc = np.where(neg, -sc, sc)
    ds = (d[:, None] * sc.astype(np.float32))[:, :, None]
    q = np.clip(np.rint(_safe_div(sub, ds)), -32, 31).astype(np.int16).reshape(nb, 256)
    u = (q + 32).astype(np.uint8)  # 0..63
    out = np.zeros((nb, 210), dtype=np.uint8)
    for c in range(2):
        uc = u[:, 128 * c:128 * (c + 1)].reshape(nb, 4, 32)  # quarter, l
        lo = uc & 0xF
        hi = uc >> 4
        out[:, 64 * c:64 * c + 32] = lo[:, 0] | (lo[:, 2] << 4)
        out[:, 64 * c + 32:64 * c + 64] = lo[:, 1] | (lo[:, 3] << 4)
        out[:, 128 + 32 * c:128 + 32 * c + 32] = hi[:, 0] | (hi[:, 1] << 2) | (hi[:, 2] << 4) | (hi[:, 3] << 6)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d16.view(np.uint8).reshape(-1, 2)
    return out.reshape(*lead, (K // 256) * 210)


def quantize(t: int, x: np.ndarray, rng: np.random.Generator | None = None) -> np.ndarray:
    if t == F32:
        x = np.ascontiguousarray(x, dtype=np.float32)
        return x.view(np.uint8).reshape(*x.shape[:-1], x.shape[-1] * 4)
    if t == Q8_0:
        return quantize_q8_0(x)
    if t == Q4_K:
        return quantize_q4_k(x)
    if t == Q5_K:
        return quantize_q5_k(x)
    if t == Q6_K:
        return quantize_q6_k(x, rng)
    raise ValueError(f"unsupported ggml type {t}")
