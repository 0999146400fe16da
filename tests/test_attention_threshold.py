"""The attention kernel's keep rule, tested on the CPU.

The reference keeps a key when fl(s - m) >= -10 (internal/ggml/ops_simd.go:46-82, SoftmaxInPlace
with fastExp's x < -10 cutoff), s = u / 8 the scaled score and m the row maximum, both f32. The
8-wave attention kernel (llm-embed_amd/csrc/attention.hip, keep_threshold) tests it instead as
u >= 8 * ceil_f32(m - 10 - 2^-21), the sum formed in f64. This test checks that the two agree
for every f32 u within 64 ulps of the threshold, over maxima of every magnitude: tiny ones
(where the f64 sum is inexact), ones near 10 (where m - 10 is tiny), large ones, the masked
maximum -1e9 and zero.
"""
import numpy as np
import pytest

F32 = np.float32


def keep_direct(u, m):
    # fmaf(u, 0.125, -m): u / 8 is exact in f32, so one rounding, of the subtraction
    return (F32(u) * F32(0.125)) - F32(m) >= F32(-10.0)


def ceil_f32(y):
    f = np.float32(y)  # round to nearest even
    if np.float64(f) < y:
        f = np.nextafter(f, np.float32(np.inf))
    return f


def keep_threshold(m):
    y = np.float64(F32(m)) + (-10.0 - 2.0 ** -21)
    return F32(8.0) * ceil_f32(y)


def maxima():
    rng = np.random.default_rng(7)
    vals = [0.0, -0.0, 1e-30, -1e-30, 2.0 ** -27, -(2.0 ** -27), 2.0 ** -21, 3 * 2.0 ** -22, 10.0, -10.0,
            np.nextafter(F32(10.0), F32(0.0)), np.nextafter(F32(10.0), F32(20.0)), 9.999999, 10.000001,
            -1e9, 1e9, 2.0 ** 30, -(2.0 ** 30), 3.5, -3.5, 1e-7, 123.456]
    vals += list(rng.normal(0, 3, 200)) + list(rng.normal(10, 1e-4, 200)) + list(rng.uniform(-60, 60, 200))
    vals += list(10.0 + rng.integers(-50, 50, 100) * 2.0 ** -20)  # on the f32 grid around 10
    return [F32(v) for v in vals]


@pytest.mark.parametrize("chunk", range(4))
def test_threshold_equals_reference_rule(chunk):
    ms = maxima()
    ms = ms[chunk::4]
    for m in ms:
        thr = keep_threshold(m)
        assert np.isfinite(thr)
        u = thr
        for _ in range(64):
            u = np.nextafter(u, F32(-np.inf))
        for _ in range(129):
            assert (u >= thr) == keep_direct(u, m), (float(m), float(u), float(thr))
            u = np.nextafter(u, F32(np.inf))


def test_threshold_is_the_smallest_kept_score():
    # the threshold itself is kept and its predecessor dropped (both rules), for every maximum
    for m in maxima():
        thr = keep_threshold(m)
        assert keep_direct(thr, m)
        assert not keep_direct(np.nextafter(thr, F32(-np.inf)), m)


def test_half_ulp_term_matters():
    # with the tie term left out (or doubled), some maximum near the grid disagrees with the
    # reference rule: the -2^-21 is what makes the boundary exact
    def thr_with(m, eps):
        return F32(8.0) * ceil_f32(np.float64(F32(m)) + (-10.0 - eps))

    for eps in (0.0, 2.0 ** -20):
        bad = 0
        for m in maxima():
            thr = thr_with(m, eps)
            lo = np.nextafter(thr, F32(-np.inf))
            bad += (not keep_direct(thr, m)) or keep_direct(lo, m)
        assert bad > 0, eps
