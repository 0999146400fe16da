"""GPU parity of the building blocks, through the C ABI: f16 decode, dequantisation (raw GGUF
layout and the GEMM's own re-laid-out planes), and the quantised projection GEMM (config 2).

Bars: bit-exact for f16 decode and dequantisation; GEMM outputs within a tolerance set by the
f16 rounding of X and W (each relative 2^-11 at most, 2^-12 rms), stated per test.
"""
import numpy as np
import pytest

import kat
import oracle
from llmembed import quant

pytestmark = pytest.mark.gpu

FORMATS = [quant.Q8_0, quant.Q4_K, quant.Q5_K, quant.Q6_K, quant.F32]


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_f16_decode_exhaustive(gpu):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(bits(gpu.f16_to_f32(h)), bits(oracle.f16_to_f32(h)))


@pytest.mark.parametrize("t", FORMATS)
def test_dequant_raw_bitexact(gpu, t):
    rng = np.random.default_rng(100 + t)
    w = (rng.standard_normal((24, 768)) * 0.02).astype(np.float32)
    blocks = quant.quantize(t, w, rng).reshape(-1)
    got = gpu.dequant(t, blocks, w.size)
    assert np.array_equal(bits(got), bits(oracle.dequant(t, blocks, w.size)))


def test_dequant_raw_kats(gpu):
    for _, blk, x, expected in kat.q8_0_cases():
        v = gpu.dequant(quant.Q8_0, blk, 32)
        assert float(np.dot(v.astype(np.float64), x)) == expected
    for _, blk, expected in kat.q5k_cases():
        assert np.array_equal(gpu.dequant(quant.Q5_K, blk, 256), expected)
    v = gpu.dequant(quant.Q5_K, kat.q5k_highbit_only_block(), 256)
    assert float(v[96:128].sum()) == 512.0
    v = gpu.dequant(quant.Q6_K, kat.q6k_known_scales(), 256)
    assert float(v.astype(np.float64).sum()) == kat.Q6K_KNOWN_SUM


def test_dequant_raw_random_bytes(gpu):
    """Arbitrary code / scale bytes (finite f16 scales), including subnormal f16 scales."""
    rng = np.random.default_rng(5)
    for t, bs, n in ((quant.Q4_K, 144, 256), (quant.Q5_K, 176, 256), (quant.Q6_K, 210, 256), (quant.Q8_0, 34, 32)):
        raw = rng.integers(0, 256, (64, bs), dtype=np.uint8)
        sub = np.frombuffer(np.uint16(0x0123).tobytes(), np.uint8)  # an f16 subnormal
        if t == quant.Q6_K:
            raw[:, 208:210] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
            raw[::3, 208:210] = sub
        elif t == quant.Q8_0:
            raw[:, 0:2] = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
            raw[::3, 0:2] = sub
        else:
            raw[:, 0:2] = np.frombuffer(np.float16(0.03).tobytes(), np.uint8)
            raw[:, 2:4] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
            raw[::3, 2:4] = sub
        flat = raw.reshape(-1)
        assert np.array_equal(bits(gpu.dequant(t, flat, 64 * n)), bits(oracle.dequant(t, flat, 64 * n))), t


@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("K,N", [(768, 2304), (3072, 768)])
def test_weight_planes_dequant_bitexact(gpu, t, K, N):
    """The GEMM's decoder on the uploaded planes reproduces DequantWeightMatrix bit for bit."""
    rng = np.random.default_rng(K + N + t)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    blocks = quant.quantize(t, w, rng)
    W = gpu.Weight(t, blocks, K, N)
    got = W.dequant()
    ref = oracle.dequant(t, blocks.reshape(-1), N * K).reshape(N, K)
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("t", FORMATS)
def test_weight_planes_f16_operand_bitexact(gpu, t):
    """The f16 MFMA operand of every weight equals the reference's f32 dequantisation rounded
    once to f16 (RNE, numpy's float32 -> float16), including subnormal f16 scales."""
    K, N = 768, 256
    rng = np.random.default_rng(40 + t)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[:8] *= 1e-4  # tiny rows: small and subnormal f16 scales and products
    blocks = quant.quantize(t, w, rng)
    got = gpu.Weight(t, blocks, K, N).dequant_f16()
    ref = oracle.dequant(t, blocks.reshape(-1), N * K).reshape(N, K).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_weight_q8_0_f16_operand_all_codes(gpu):
    """Q8_0's packed-f16 decode over every int8 code and a spread of f16 scales (normal,
    subnormal, large): q * d rounded once in f16 == RNE(f32 q * d)."""
    scales = np.array([1.0, 0.5, 3.0517578125e-05, 6.1035156e-05, 5.9604645e-08, 2.0e-06, 0.0123, 100.0, -0.75,
                       7.0e-3, 1.5e-5, 250.0, -3.3e-6, 0.031, 1.0e-7, 60.0], np.float16)
    N = 128
    codes = np.tile(np.arange(-128, 128, dtype=np.int16).astype(np.int8), (N, 1))  # 256 codes = 8 blocks / row
    blk = np.zeros((N, 8, 34), np.uint8)
    for r in range(N):
        for b in range(8):
            blk[r, b, 0:2] = np.frombuffer(scales[(r + b) % len(scales)].tobytes(), np.uint8)
            blk[r, b, 2:] = codes[r, 32 * b:32 * b + 32].view(np.uint8)
    got = gpu.Weight(quant.Q8_0, blk.reshape(-1), 256, N).dequant_f16()
    ref = oracle.dequant(quant.Q8_0, blk.reshape(-1), N * 256).reshape(N, 256).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_weight_q5k_alias_types(gpu):
    """DequantWeightMatrix maps ggml types 13, 15 and 16 to Q5_K (gemm.go:241)."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((128, 256)) * 0.02).astype(np.float32)
    blocks = quant.quantize(quant.Q5_K, w)
    ref = gpu.Weight(quant.Q5_K, blocks, 256, 128).dequant()
    for alias in (15, 16):
        assert np.array_equal(bits(gpu.Weight(alias, blocks, 256, 128).dequant()), bits(ref))


def _gemm_case(t, K, N, M, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    blocks = quant.quantize(t, w, rng)
    X = rng.standard_normal((M, K)).astype(np.float32)
    Wd = oracle.dequant(t, blocks.reshape(-1), N * K).reshape(N, K)
    return blocks, X, Wd


SHAPES = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]


def check_gemm(Y, ref, what):
    """Config-2 tolerance for an f16-operand path against the reference's f32 GEMM:
    max|Y - Yref| <= 1e-3 * max|Yref| (the survey's bound) and rms(Y - Yref) <= 1e-3 * rms(Yref).
    f16 rounding of X and W gives ~2e-4 relative rms error per output."""
    ref = ref.astype(np.float64)
    err = Y.astype(np.float64) - ref
    mx, inf = float(np.abs(err).max()), float(np.abs(ref).max())
    rms, rms_ref = float(np.sqrt(np.mean(err ** 2))), float(np.sqrt(np.mean(ref ** 2)))
    print(f"{what}: max|err| / max|Y| = {mx / inf:.2e}, rms ratio {rms / rms_ref:.2e}", flush=True)
    assert mx <= 1e-3 * inf, (what, mx / inf)
    assert rms <= 1e-3 * rms_ref, (what, rms / rms_ref)


@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("K,N", SHAPES)
@pytest.mark.parametrize("M", [8, 512])
def test_gemm_vs_oracle(gpu, t, K, N, M):
    """Config 2: Y = X W^T against the reference GemmPrePacked32 order on the dequantised W."""
    blocks, X, Wd = _gemm_case(t, K, N, M, 7 * K + N + M + t)
    W = gpu.Weight(t, blocks, K, N)
    check_gemm(W.gemm(X), oracle.gemm(X, Wd), f"gemm t={t} {K}x{N} M={M}")


_X_LARGE = {}


@pytest.mark.parametrize("t", FORMATS)
@pytest.mark.parametrize("K,N", SHAPES)
def test_gemm_large_m_vs_oracle(gpu, t, K, N):
    """Config 2 at M = 32768 for every (format, shape): 64 sampled rows against the oracle, and
    the same rows computed alone (the small-M kernels) give the same bits."""
    M = 32768
    rng = np.random.default_rng(3 + 11 * t + K + N)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    blocks = quant.quantize(t, w, rng)
    if K not in _X_LARGE:  # X f32 N(0, 1), shared by the formats and shapes of one K
        _X_LARGE.clear()
        _X_LARGE[K] = np.random.default_rng(K).standard_normal((M, K), dtype=np.float32)
    X = _X_LARGE[K]
    W = gpu.Weight(t, blocks, K, N)
    Y = W.gemm(X)
    rows = np.sort(rng.choice(M, 64, replace=False))
    Wd = oracle.dequant(t, blocks.reshape(-1), N * K).reshape(N, K)
    check_gemm(Y[rows], oracle.gemm(X[rows], Wd), f"gemm t={t} {K}x{N} M={M}")
    assert np.array_equal(bits(W.gemm(X[rows])), bits(Y[rows]))


@pytest.mark.parametrize("t", [quant.Q8_0, quant.Q4_K, quant.Q6_K])
def test_gemm_row_invariance(gpu, t):
    """A row's output bits do not depend on M or on which kernel (small-M split-K or large-M
    or 128/256-token tiles) computed it: the canonical chunk order is shared by all of them."""
    K, N = 3072, 768
    blocks, X, _ = _gemm_case(t, K, N, 1500, 99 + t)
    W = gpu.Weight(t, blocks, K, N)
    big = W.gemm(X)  # M >= 1024: 256-token tiles
    for rows in ([0], [5, 17, 299], list(range(64)), list(range(40, 120)), list(range(300, 1400))):
        part = W.gemm(X[rows])
        assert np.array_equal(bits(part), bits(big[rows])), rows


def test_weight_errors(gpu):
    with pytest.raises(gpu.LLEError):
        gpu.Weight(2, np.zeros(1024, np.uint8), 256, 128)  # Q4_0: not on the path
    with pytest.raises(gpu.LLEError):
        gpu.Weight(quant.Q8_0, np.zeros(34 * 10, np.uint8), 320, 1)  # N not a multiple of 128


@pytest.mark.parametrize("t,K,N", [(quant.Q8_0, 768, 2304), (quant.Q5_K, 3072, 768), (quant.Q4_K, 768, 3072)])
def test_gemm_f16_entry_matches_host_entry(gpu, t, K, N):
    """lle_gemm_f16_async (f16 activations on the device, caller's split-K workspace) gives the
    bits of lle_gemm (f32 host activations, rounded to f16 inside) at every M regime."""
    from llmembed import _hip

    for M in (8, 64, 100, 512, 1100):
        blocks, X, _ = _gemm_case(t, K, N, M, 5 * K + N + M + t)
        W = gpu.Weight(t, blocks, K, N)
        ref = W.gemm(X)
        x16 = _hip.DeviceBuffer.from_array(X.astype(np.float16))
        dy = _hip.DeviceBuffer(M * N * 4)
        dp = _hip.DeviceBuffer(max(W.part_floats(M), 1) * 4)
        for part in ((dp.value,) if M <= 64 else (dp.value, 0)):  # row blocks, or 128-row tiles
            W.gemm_f16_async(x16.value, M, dy.value, part)
            _hip.synchronize()
            assert np.array_equal(bits(dy.download((M, N), np.float32)), bits(ref)), (M, part)
