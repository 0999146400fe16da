"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the GPU parity checker.

Each check is chosen so that a plausible transcription slip fails it: reference KATs
(dot_test.go, dot_q5k_test.go, dot_q6k_test.go), exhaustive f16 decode against numpy,
structural invariants (Q4_K == Q5_K with qh = 0), a brute-force float64 GEMM, closed forms of
the elementwise ops, and an independent numpy restatement of the whole forward.
"""
import math

import numpy as np
import pytest

import kat
import numpy_ref
import oracle
from llmembed import gguf, quant, synth


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------------------- f16 decode
def test_f16_exhaustive_vs_numpy_and_closed_form():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_to_f32(h)
    exp = (h >> 10) & 0x1F
    mant = (h & 0x3FF).astype(np.uint32)
    sign = (h >> 15).astype(np.uint32)
    finite = exp != 0x1F
    ref = h.view(np.float16).astype(np.float32)
    assert np.array_equal(bits(ours)[finite], bits(ref)[finite])
    # Inf / NaN keep their payload: sign | 0xff << 23 | mant << 13 (tensor.go:186-189)
    nan_bits = (sign << 31) | (0xFF << 23) | (mant << 13)
    assert np.array_equal(bits(ours)[~finite], nan_bits[~finite])
    # subnormals are exactly mant * 2^-24
    sub = (exp == 0) & (mant != 0)
    assert np.array_equal(np.abs(ours[sub]).astype(np.float64), mant[sub] * 2.0 ** -24)


# ---------------------------------------------------------------------------- dequant KATs
@pytest.mark.parametrize("name,blk,x,expected", kat.q8_0_cases())
def test_q8_0_kat(name, blk, x, expected):
    v = oracle.dequant(quant.Q8_0, blk, 32)
    assert float(np.dot(v.astype(np.float64), x)) == expected


@pytest.mark.parametrize("case", kat.q5k_cases(), ids=lambda c: c[0])
def test_q5_k_kat(case):
    _, blk, expected = case
    v = oracle.dequant(quant.Q5_K, blk, 256)
    assert np.array_equal(v, expected)


def test_q5_k_highbit_only_512():
    v = oracle.dequant(quant.Q5_K, kat.q5k_highbit_only_block(), 256)
    assert float(v[96:128].sum()) == 512.0
    assert float(np.abs(v[:96]).sum() + np.abs(v[128:]).sum()) == 0.0


def test_q6_k_known_scales():
    v = oracle.dequant(quant.Q6_K, kat.q6k_known_scales(), 256)
    assert float(v.astype(np.float64).sum()) == kat.Q6K_KNOWN_SUM
    assert np.all(v == -31.0 * (10 + 5 * (np.arange(256) // 16)))


def test_scale_min_k4_roundtrip_through_q5k_packer():
    """makeQ5_KBlock packs 6-bit (scale, min) pairs; getScaleMinK4 must return them for all 8
    sub-blocks, which pins the split of sub-blocks 4-7 (high bits in bytes 0-7)."""
    import ctypes as C

    rng = np.random.default_rng(7)
    for _ in range(50):
        sc = rng.integers(0, 64, 8).tolist()
        mn = rng.integers(0, 64, 8).tolist()
        blk = kat.make_q5_k_block(1.0, 1.0, sc, mn, [0] * 256)
        scales = np.ascontiguousarray(blk[4:16])
        for j in range(8):
            a, b = C.c_uint8(), C.c_uint8()
            oracle.lib().orc_get_scale_min_k4(j, scales.ctypes.data, C.byref(a), C.byref(b))
            assert (a.value, b.value) == (sc[j], mn[j])


def test_q4_k_equals_q5_k_with_zero_qh():
    """Structural invariant: a Q4_K block and the Q5_K block with the same d/dmin/scales/qs and
    all-zero qh decode to identical bits (quant_q4k.go:51-73 vs quant_q5k.go:54-87)."""
    rng = np.random.default_rng(3)
    b4 = quant.quantize_q4_k(rng.standard_normal((8, 256)).astype(np.float32) * 0.05)
    for i in range(8):
        blk4 = b4[i]
        blk5 = np.zeros(176, np.uint8)
        blk5[0:16] = blk4[0:16]
        blk5[48:176] = blk4[16:144]
        assert np.array_equal(bits(oracle.dequant(quant.Q4_K, blk4, 256)), bits(oracle.dequant(quant.Q5_K, blk5, 256)))


@pytest.mark.parametrize("t", [quant.Q8_0, quant.Q4_K, quant.Q5_K, quant.Q6_K])
def test_dequant_matches_numpy_restatement_bitwise(t):
    rng = np.random.default_rng(11 + t)
    w = rng.standard_normal((16, 768)).astype(np.float32) * 0.02
    blocks = quant.quantize(t, w, rng)
    a = oracle.dequant(t, blocks.reshape(-1), w.size)
    b = numpy_ref.dequant(t, blocks.reshape(-1), w.size)
    assert np.array_equal(bits(a), bits(b))
    # and close to the quantised source (a wrong bit offset would be far off)
    tol = {quant.Q8_0: 0.01, quant.Q6_K: 0.03, quant.Q5_K: 0.05, quant.Q4_K: 0.1}[t]
    assert np.abs(a - w.reshape(-1)).max() <= tol * np.abs(w).max() + 1e-6


def test_dequant_random_bytes_q6k_q5k_q4k():
    """Random (not quantiser-made) blocks: every bit pattern of codes and scales is decoded the
    same by both restatements."""
    rng = np.random.default_rng(5)
    for t, bs in ((quant.Q4_K, 144), (quant.Q5_K, 176), (quant.Q6_K, 210), (quant.Q8_0, 34)):
        n = 256 if t != quant.Q8_0 else 32
        raw = rng.integers(0, 256, (64, bs), dtype=np.uint8)
        # keep the f16 scales finite
        if t == quant.Q6_K:
            raw[:, 208:210] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
        elif t == quant.Q8_0:
            raw[:, 0:2] = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
        else:
            raw[:, 0:2] = np.frombuffer(np.float16(0.03).tobytes(), np.uint8)
            raw[:, 2:4] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
        a = oracle.dequant(t, raw.reshape(-1), 64 * n)
        b = numpy_ref.dequant(t, raw.reshape(-1), 64 * n)
        assert np.array_equal(bits(a), bits(b)), t


# ---------------------------------------------------------------------------- GEMM
def test_gemm_vs_float64_bruteforce():
    rng = np.random.default_rng(1)
    for M, K, N in ((8, 768, 64), (13, 3072, 96), (1, 256, 32), (32, 768, 128)):
        A = rng.standard_normal((M, K)).astype(np.float32)
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        C = oracle.gemm(A, W)
        ref = A.astype(np.float64) @ W.astype(np.float64).T
        err = np.abs(C - ref).max() / np.abs(ref).max()
        assert err < 1e-5, (M, K, N, err)


def test_gemm_fma_tile_vs_scalar_edge_rows():
    """GemmPrePacked32 runs full 6-row tiles through the FMA micro-kernel and later rows through
    the unfused scalar loop (gemm_avx512.go:115-140). With K=2, A row = [1, 1+2^-12],
    W col = [-(1+2^-11), 1+2^-12]: FMA gives exactly 2^-24, the unfused loop gives 0."""
    a1 = np.float32(1 + 2 ** -12)
    A = np.tile(np.array([[1.0, a1]], np.float32), (7, 1))
    W = np.zeros((32, 2), np.float32)
    W[:, 0] = -(1 + 2 ** -11)
    W[:, 1] = a1
    C = oracle.gemm(A, W, threads=1)
    assert np.all(C[:6] == np.float32(2 ** -24))
    assert np.all(C[6] == 0.0)


# ---------------------------------------------------------------------------- elementwise
def test_gelu_closed_forms():
    v = np.array([0.0, 10.0, -10.0, 1.0, -1.0], np.float32)
    g = oracle.gelu(v)
    assert g[0] == 0.0 and g[1] == 10.0 and g[2] == 0.0
    # f64 restatement of the rational-tanh formula (ops_simd.go:27-42)
    for x, y in zip(v[3:], g[3:]):
        t = 0.7978845608 * x * (1 + 0.044715 * x * x)
        th = t * (27 + t * t) / (27 + 9 * t * t)
        assert abs(0.5 * x * (1 + th) - y) < 1e-6
    # the rational tanh is exactly 1 at t = 3 and exceeds 1 for 3 < |t| <= 4.97
    t = 4.0
    assert t * (27 + t * t) / (27 + 9 * t * t) > 1.0


def test_softmax_cutoff_and_mask():
    s = oracle.softmax(np.array([0.0, -10.5, -9.9, -1e9], np.float32))
    assert s[1] == 0.0 and s[3] == 0.0 and s[2] > 0.0
    assert abs(float(s.sum()) - 1.0) < 1e-6
    assert abs(s[0] / s[2] - math.exp(9.9)) / math.exp(9.9) < 1e-5


def test_rope_table_and_apply():
    c, s = oracle.rope_table(2048, 64, 1000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    i = np.arange(32)
    ang = np.arange(2048)[:, None] * (1000.0 ** (-(2.0 * i) / 64))[None, :]
    assert np.abs(c - np.cos(ang)).max() < 2e-4  # f32 angle rounding at pos ~2047
    x = np.random.default_rng(0).standard_normal(64).astype(np.float32)
    y = x.copy()
    import ctypes as C

    oracle.lib().orc_rope_apply(y.ctypes.data, c[777].ctypes.data, s[777].ctypes.data, 32)
    n0 = x[0::2] ** 2 + x[1::2] ** 2
    n1 = y[0::2] ** 2 + y[1::2] ** 2
    assert np.abs(n0 - n1).max() < 1e-5


def test_layernorm_constant_affine():
    x = np.random.default_rng(2).standard_normal(768).astype(np.float32) * 3 + 1
    y = oracle.layernorm(x, np.full(768, 2.0), np.full(768, 0.5), 1e-12)
    assert abs(float(y.mean()) - 0.5) < 1e-5
    assert abs(float(y.std()) - 2.0) < 1e-4


def test_pool_and_l2():
    h = np.tile(np.arange(8, dtype=np.float32), (5, 1))
    p = oracle.mean_pool(h, np.array([1, 1, 0, 1, 2], np.int32))
    assert np.array_equal(p, np.arange(8, dtype=np.float32))
    z = oracle.mean_pool(h, np.zeros(5, np.int32))
    assert np.all(z == 0)
    v = oracle.l2_normalize(np.array([3.0, 4.0], np.float32))
    assert np.allclose(v, [0.6, 0.8])
    assert np.all(oracle.l2_normalize(np.zeros(4, np.float32)) == 0)


# ---------------------------------------------------------------------------- forward
@pytest.mark.parametrize("mix", ["Q8_0", "Q4_K", "Q5_K", "Q6_K", "Q4_K_M", "F32"])
def test_forward_matches_numpy_restatement(small_spec, mix):
    path = synth.model_path(small_spec, mix, 100)
    om = oracle.OracleModel(path)
    nm = numpy_ref.NumpyModel(gguf.read(path))
    rng = np.random.default_rng(9)
    for L in (8, 37):
        ids = rng.integers(0, small_spec.vocab, L).astype(np.int32)
        a = om.embed(ids)
        b = nm.embed(ids)
        cos = float(np.dot(a, b) / np.linalg.norm(a) / np.linalg.norm(b))
        assert cos > 0.99999, (mix, L, cos)
        assert np.abs(a - b).max() < 1e-4
        # hidden states too
        ha = om.forward(ids)
        hb = nm.forward(ids, np.ones(L))
        assert np.abs(ha - hb).max() < 2e-3


def test_forward_masked_keys_and_matryoshka(small_spec):
    path = synth.model_path(small_spec, "Q8_0", 100)
    om = oracle.OracleModel(path)
    nm = numpy_ref.NumpyModel(gguf.read(path))
    rng = np.random.default_rng(4)
    ids = rng.integers(0, small_spec.vocab, 20).astype(np.int32)
    mask = np.ones(20, np.int32)
    mask[[3, 7, 15]] = 0
    a = om.embed(ids, mask)
    b = nm.embed(ids, mask)
    assert float(np.dot(a, b)) > 0.99999
    a256 = om.embed(ids, mask, out_dim=256)
    b256 = nm.embed(ids, mask, out_dim=256)
    assert a256.shape == (256,) and abs(float(np.linalg.norm(a256)) - 1) < 1e-6
    assert float(np.dot(a256, b256)) > 0.99999


def test_embed_batch_equals_embed(small_spec):
    """EmbedBatch == Embed bit for bit (embedder_test.go:116-145,212-253)."""
    path = synth.model_path(small_spec, "Q8_0", 100)
    om = oracle.OracleModel(path)
    rng = np.random.default_rng(8)
    B, L = 5, 24
    ids = rng.integers(0, small_spec.vocab, (B, L)).astype(np.int32)
    lens = [24, 7, 13, 1, 20]
    mask = np.zeros((B, L), np.int32)
    for i, n in enumerate(lens):
        mask[i, :n] = 1
    batch = om.embed_batch(ids, mask)
    for i, n in enumerate(lens):
        single = om.embed(ids[i, :n])
        assert np.array_equal(bits(single), bits(batch[i]))


def test_forward_errors(small_spec):
    path = synth.model_path(small_spec, "Q8_0", 100)
    om = oracle.OracleModel(path)
    with pytest.raises(RuntimeError):
        om.forward(np.array([small_spec.vocab], np.int32))
    with pytest.raises(RuntimeError):
        om.forward(np.zeros(small_spec.ctx + 1, np.int32))
