"""Known-answer inputs lifted from the reference's own tests, rebuilt in numpy.

The block builders restate the reference's test helpers so the KAT inputs are the same bytes:
  f32ToF16 (truncating, flushes subnormals)   internal/ggml/dot_test.go:25-48
  makeQ8_0Block                               internal/ggml/dot_test.go:11-22
  makeQ5_KBlock                               internal/ggml/dot_q5k_test.go:13-82
Expected values are the ones the reference tests assert (or, for Q6_K, the closed form of the
reference test input: see q6k_known_scales).
"""
from __future__ import annotations

import numpy as np


def f32_to_f16_trunc(f: float) -> int:
    bits = int(np.array([f], np.float32).view(np.uint32)[0])
    sign, exp, mant = (bits >> 31) & 1, (bits >> 23) & 0xFF, bits & 0x7FFFFF
    if exp == 0:
        return sign << 15
    if exp == 0xFF:
        return (sign << 15) | 0x7C00 | (mant >> 13)
    ne = exp - 127 + 15
    if ne >= 31:
        return (sign << 15) | 0x7C00
    if ne <= 0:
        return sign << 15
    return (sign << 15) | (ne << 10) | (mant >> 13)


def make_q8_0_block(scale: float, quants) -> np.ndarray:
    b = np.zeros(34, np.uint8)
    h = f32_to_f16_trunc(scale)
    b[0], b[1] = h & 0xFF, h >> 8
    b[2:] = np.asarray(quants, np.int8).view(np.uint8)
    return b


def make_q5_k_block(d, dmin, sub_scales, sub_mins, quants) -> np.ndarray:
    blk = np.zeros(176, np.uint8)
    hd, hm = f32_to_f16_trunc(d), f32_to_f16_trunc(dmin)
    blk[0], blk[1], blk[2], blk[3] = hd & 0xFF, hd >> 8, hm & 0xFF, hm >> 8
    sc = blk[4:16]
    for i in range(4):
        sc[i] = sub_scales[i] & 63
        sc[i + 4] = sub_mins[i] & 63
    for i in range(4, 8):
        s, m = sub_scales[i], sub_mins[i]
        sc[i + 4] = (s & 0xF) | ((m & 0xF) << 4)
        sc[i - 4] |= (s >> 4) << 6
        sc[i] |= (m >> 4) << 6
    qh = blk[16:48]
    qs = blk[48:176]
    q_off, sub = 0, 0
    for j in range(0, 256, 64):
        for l in range(32):
            q = int(quants[j + l])
            qs[q_off + l] = (qs[q_off + l] & 0xF0) | (q & 0xF)
            if q & 0x10:
                qh[l] |= 1 << sub
        sub += 1
        for l in range(32):
            q = int(quants[j + 32 + l])
            qs[q_off + l] = (qs[q_off + l] & 0x0F) | ((q & 0xF) << 4)
            if q & 0x10:
                qh[l] |= 1 << sub
        sub += 1
        q_off += 32
    return blk


def q5k_cases():
    """(name, block, expected f32 per element or None, x, expected dot or None)."""
    ones = [1] * 8
    zeros = [0] * 8
    out = []
    out.append(("all15", make_q5_k_block(1.0, 0.0, ones, zeros, [15] * 256), np.full(256, 15.0, np.float32)))
    out.append(("all16_highbit", make_q5_k_block(1.0, 0.0, ones, zeros, [16] * 256), np.full(256, 16.0, np.float32)))
    alt = [0 if i % 2 == 0 else 31 for i in range(256)]
    exp = np.array([-0.25 if i % 2 == 0 else 30.75 for i in range(256)], np.float32)
    out.append(("alternating", make_q5_k_block(0.5, 0.25, [2] * 8, [1] * 8, alt), exp))
    q = [0] * 256
    for i in range(0, 256, 32):
        q[i] = 16
    exp = np.array([16.0 if i % 32 == 0 else 0.0 for i in range(256)], np.float32)
    out.append(("highbit_positions", make_q5_k_block(1.0, 0.0, ones, zeros, q), exp))
    return out


def q5k_highbit_only_block():
    """dot_q5k_test.go:373-411: all low nibbles 0, the high bit of sub-group 3 set for every
    position, scale 1, min 0, x = 1: the sub-group's dot is 16 * 32 = 512."""
    q = [0] * 256
    for l in range(32):
        q[96 + l] = 16  # sub-group 3 = second half of j=1 group
    return make_q5_k_block(1.0, 0.0, [1] * 8, [0] * 8, q)


def q6k_known_scales() -> np.ndarray:
    """dot_q6k_test.go:59-103: ql = 0x11, qh = 0, scales 10+5i, d = f16 1.0, x = 1.
    Every code is (1 | 0<<4) - 32 = -31 and element e uses scale 10 + 5*(e // 16), so
    sum_e deq(e) = -31 * 16 * sum_i (10 + 5i) = -376960."""
    b = np.zeros(210, np.uint8)
    b[0:128] = 0x11
    b[192:208] = np.array([10 + 5 * i for i in range(16)], np.int8).view(np.uint8)
    b[208], b[209] = 0x00, 0x3C
    return b


Q6K_KNOWN_SUM = -376960.0


def q8_0_cases():
    return [
        ("ones", make_q8_0_block(1.0, [1] * 32), np.ones(32, np.float32), 32.0),
        ("neg", make_q8_0_block(0.5, [-1] * 32), np.full(32, 2.0, np.float32), -32.0),
    ]
