"""Second, independent restatement of the reference forward in numpy (float64 math).

TEST INFRASTRUCTURE ONLY. It shares no code with oracle.c: dequantisation is written
vectorised over whole blocks, reductions are numpy's (pairwise, float64), RoPE angles
are computed directly in float64. Used to pin the C oracle: a transcription slip in
either restatement (a dropped term, a swapped operand, a wrong bit offset) shows up
as a cosine gap far above the float32-vs-float64 rounding noise.

Reference semantics followed (all paths relative to the reference root):
  dequant   internal/ggml/tensor.go:130-191, quant_q4k.go:27-77,133-140,
            quant_q5k.go:29-91, quant_q6k.go:23-75
  forward   internal/embed/bert.go:216-445 (post-LN, gated GeLU FFN, interleaved RoPE)
  ops       internal/ggml/ops_simd.go (LN, rational-tanh GeLU, softmax with x<-10 -> 0)
  pooling   internal/embed/pool.go:8-54, internal/embed/embedder.go:46-71
"""
from __future__ import annotations

import numpy as np


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def _scale_min_k4(scales: np.ndarray):
    """scales [nb, 12] uint8 -> (sc, m) [nb, 8]; the 6-bit split of getScaleMinK4."""
    s = scales.astype(np.uint16)
    sc = np.empty((s.shape[0], 8), np.uint16)
    m = np.empty_like(sc)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def dequant(t: int, data: np.ndarray, n: int) -> np.ndarray:
    """Vectorised dequantisation, float32 arithmetic in the reference's operation order."""
    data = np.asarray(data, np.uint8)
    if t == 0:
        return data[: 4 * n].view(np.float32).copy()
    if t == 8:
        b = data[: (n // 32) * 34].reshape(-1, 34)
        d = f16_bits_to_f32(b[:, 0:2].copy().view(np.uint16)[:, 0])
        q = b[:, 2:].view(np.int8).astype(np.float32)
        return (q * d[:, None]).astype(np.float32).reshape(-1)
    if t in (12, 13, 15, 16):
        q5 = t != 12
        bs = 176 if q5 else 144
        b = data[: (n // 256) * bs].reshape(-1, bs)
        d = f16_bits_to_f32(b[:, 0:2].copy().view(np.uint16)[:, 0])
        dmin = f16_bits_to_f32(b[:, 2:4].copy().view(np.uint16)[:, 0])
        sc, m = _scale_min_k4(b[:, 4:16])
        qs = b[:, 48:176] if q5 else b[:, 16:144]
        qs = qs.reshape(-1, 4, 32)
        lo = (qs & 0xF).astype(np.uint8)
        hi = (qs >> 4).astype(np.uint8)
        q = np.stack([lo, hi], axis=2).reshape(-1, 8, 32)  # sub-block s = 2g + (0 low | 1 high)
        if q5:
            qh = b[:, 16:48]
            bits = np.stack([(qh >> s) & 1 for s in range(8)], axis=1)  # [nb, 8, 32]
            q = q | (bits << 4)
        ds = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
        dm = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)
        v = (ds[:, :, None] * q.astype(np.float32)).astype(np.float32) - dm[:, :, None]
        return v.astype(np.float32).reshape(-1)
    if t == 14:
        b = data[: (n // 256) * 210].reshape(-1, 210)
        d = f16_bits_to_f32(b[:, 208:210].copy().view(np.uint16)[:, 0])
        sc = b[:, 192:208].view(np.int8).astype(np.float32)  # [nb, 16]
        out = np.empty((b.shape[0], 256), np.float32)
        for c in range(2):
            ql = b[:, 64 * c:64 * c + 64]
            qh = b[:, 128 + 32 * c:128 + 32 * c + 32]
            quarters = [
                (ql[:, 0:32] & 0xF) | (((qh >> 0) & 3) << 4),
                (ql[:, 32:64] & 0xF) | (((qh >> 2) & 3) << 4),
                (ql[:, 0:32] >> 4) | (((qh >> 4) & 3) << 4),
                (ql[:, 32:64] >> 4) | (((qh >> 6) & 3) << 4),
            ]
            for qi, qv in enumerate(quarters):
                qq = qv.astype(np.int16) - 32
                e0 = 128 * c + 32 * qi
                s_idx = (e0 + np.arange(32)) // 16  # scale index = element / 16
                scale = (d[:, None] * sc[:, s_idx]).astype(np.float32)
                out[:, e0:e0 + 32] = (scale * qq.astype(np.float32)).astype(np.float32)
        return out.reshape(-1)
    raise ValueError(f"unsupported type {t}")


def _ln(x, w, b, eps):
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _gelu_r(v):
    t = 0.7978845608 * v * (1.0 + 0.044715 * v * v)
    th = t * (27.0 + t * t) / (27.0 + 9.0 * t * t)
    th = np.where(t > 4.97, 1.0, np.where(t < -4.97, -1.0, th))
    return 0.5 * v * (1.0 + th)


class NumpyModel:
    """Model weights dequantised to float64 matrices [N][K]."""

    def __init__(self, g):
        a = "nomic-bert."
        self.n_layer = g.get_u32(a + "block_count")
        self.D = g.get_u32(a + "embedding_length")
        self.F = g.get_u32(a + "feed_forward_length")
        self.H = g.get_u32(a + "attention.head_count")
        self.eps = float(g.get_f32(a + "attention.layer_norm_epsilon"))
        self.base = float(g.get_f32(a + "rope.freq_base"))
        self.g = g

        def mat(name):
            ti = g.tensors[name]
            K, N = int(ti.dims[0]), int(ti.dims[1]) if len(ti.dims) > 1 else 1
            return dequant(ti.type, g.tensor_bytes(name), K * N).reshape(N, K).astype(np.float64)

        def vec(name):
            ti = g.tensors[name]
            return dequant(ti.type, g.tensor_bytes(name), ti.n_elements).astype(np.float64)

        self.tok_info = g.tensors["token_embd.weight"]
        self.type0 = mat("token_types.weight")[0]
        self.enw, self.enb = vec("token_embd_norm.weight"), vec("token_embd_norm.bias")
        self.layers = []
        for l in range(self.n_layer):
            p = f"blk.{l}."
            self.layers.append(dict(
                qkv=mat(p + "attn_qkv.weight"), out=mat(p + "attn_output.weight"),
                anw=vec(p + "attn_output_norm.weight"), anb=vec(p + "attn_output_norm.bias"),
                up=mat(p + "ffn_up.weight"), gate=mat(p + "ffn_gate.weight"),
                down=mat(p + "ffn_down.weight"),
                onw=vec(p + "layer_output_norm.weight"), onb=vec(p + "layer_output_norm.bias")))

    def _tok_rows(self, ids):
        ti = self.tok_info
        from llmembed.quant import row_bytes
        rb = row_bytes(ti.type, self.D)
        raw = self.g.tensor_bytes("token_embd.weight")
        return np.stack([dequant(ti.type, raw[i * rb:(i + 1) * rb], self.D) for i in ids]).astype(np.float64)

    def forward(self, ids, mask):
        ids = np.asarray(ids)
        mask = np.asarray(mask)
        L, D, H = ids.size, self.D, self.H
        hd = D // H
        h = _ln(self._tok_rows(ids) + self.type0, self.enw, self.enb, self.eps)
        i = np.arange(hd // 2)
        inv_freq = self.base ** (-(2.0 * i) / hd)
        ang = np.arange(L)[:, None] * inv_freq[None, :]
        cos, sin = np.cos(ang), np.sin(ang)

        def rope(x):  # x [L, H, hd]
            x0, x1 = x[..., 0::2], x[..., 1::2]
            c, s = cos[:, None, :], sin[:, None, :]
            out = np.empty_like(x)
            out[..., 0::2] = x0 * c - x1 * s
            out[..., 1::2] = x0 * s + x1 * c
            return out

        for ly in self.layers:
            qkv = h @ ly["qkv"].T
            q = rope(qkv[:, :D].reshape(L, H, hd))
            k = rope(qkv[:, D:2 * D].reshape(L, H, hd))
            v = qkv[:, 2 * D:].reshape(L, H, hd)
            s = np.einsum("qhd,khd->hqk", q, k) / np.sqrt(hd)
            s = np.where((mask == 0)[None, None, :], -1e9, s)
            z = s - s.max(axis=-1, keepdims=True)
            e = np.where(z < -10.0, 0.0, np.exp(z))
            p = e / e.sum(axis=-1, keepdims=True)
            att = np.einsum("hqk,khd->qhd", p, v).reshape(L, D)
            h = _ln(h + att @ ly["out"].T, ly["anw"], ly["anb"], self.eps)
            g = _gelu_r(h @ ly["gate"].T) * (h @ ly["up"].T)
            h = _ln(h + g @ ly["down"].T, ly["onw"], ly["onb"], self.eps)
        return h

    def embed(self, ids, mask=None, out_dim=None):
        ids = np.asarray(ids)
        mask = np.ones_like(ids) if mask is None else np.asarray(mask)
        h = self.forward(ids, mask)
        sel = mask == 1
        pooled = h[sel].mean(axis=0) if sel.any() else np.zeros(self.D)
        v = pooled / np.linalg.norm(pooled)
        if out_dim is not None and out_dim < self.D:
            v = v[:out_dim] / np.linalg.norm(v[:out_dim])
        return v
