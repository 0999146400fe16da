// Device decoders for the GGUF block formats, on the raw GGUF layout (token embedding rows,
// lle_dequant) and on the re-laid-out weight planes used by the GEMMs (WeightDev).
//
// Every value is produced with the reference's arithmetic so results are bit-identical:
//   f16ToF32            internal/ggml/tensor.go:162-191 (integer restatement; NaN payload kept)
//   Q8_0  q*d           internal/ggml/tensor.go:130-159, gemm.go:270-282 (exact product)
//   Q4_K  (d*sc)*q-dmin*m   quant_q4k.go:27-77,133-140 (exact products, one rounding: fmaf
//                           of the exact product gives the same single rounding)
//   Q5_K  as Q4_K + bit     quant_q5k.go:29-91
//   Q6_K  (d*sc)*(q-32)     quant_q6k.go:23-75 (exact)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lle {

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  if (ex == 0x1fu) return __uint_as_float((sign << 31) | (0xffu << 23) | (mant << 13));
  if (ex != 0u) return __uint_as_float((sign << 31) | ((ex + 112u) << 23) | (mant << 13));
  // zero / subnormal: mant * 2^-24 is exact in f32
  const float f = (float)mant * 5.9604644775390625e-08f;
  return sign ? -f : f;
}

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* s, float& sc, float& m) {
  if (j < 4) {
    sc = (float)(s[j] & 63);
    m = (float)(s[j + 4] & 63);
  } else {
    sc = (float)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    m = (float)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

// ---------------------------------------------------------------------------------------
// Raw GGUF layout: element j of a row starting at `row` (row bytes per ByteSize).
__device__ __forceinline__ float deq_raw_elem(int type, const uint8_t* row, int j) {
  switch (type) {
    case 0:
      return __uint_as_float(*(const uint32_t*)(row + 4 * j));
    case 8: {
      const uint8_t* b = row + (j >> 5) * 34;
      const float d = f16_bits_to_f32(b[0] | (b[1] << 8));
      return (float)(int8_t)b[2 + (j & 31)] * d;
    }
    case 12:
    case 13: {
      const bool q5 = type == 13;
      const uint8_t* b = row + (j >> 8) * (q5 ? 176 : 144);
      const int e = j & 255, g = e >> 6, hi = (e >> 5) & 1, l = e & 31;
      const float d = f16_bits_to_f32(b[0] | (b[1] << 8));
      const float dmin = f16_bits_to_f32(b[2] | (b[3] << 8));
      float sc, m;
      scale_min_k4(2 * g + hi, b + 4, sc, m);
      const uint8_t byte = b[(q5 ? 48 : 16) + 32 * g + l];
      int q = hi ? (byte >> 4) : (byte & 0xF);
      if (q5) q |= ((b[16 + l] >> (2 * g + hi)) & 1) << 4;
      return fmaf(d * sc, (float)q, -(dmin * m));
    }
    case 14: {
      const uint8_t* b = row + (j >> 8) * 210;
      const int e = j & 255, c = e >> 7, el = e & 127, qq = el >> 5, l = el & 31;
      const uint8_t qlb = b[64 * c + 32 * (qq & 1) + l];
      const int lo = (qq >> 1) ? (qlb >> 4) : (qlb & 0xF);
      const int hi = (b[128 + 32 * c + l] >> (2 * qq)) & 3;
      const int q = (lo | (hi << 4)) - 32;
      const float d = f16_bits_to_f32(b[208] | (b[209] << 8));
      return (d * (float)(int8_t)b[192 + (e >> 4)]) * (float)q;
    }
    default:
      return __uint_as_float(0x7fc00000u);
  }
}

// ---------------------------------------------------------------------------------------
// Re-laid-out weight planes (see WeightDev in lle_internal.h). A "segment" is 16
// consecutive K elements of one row; k0 is a multiple of 16.
struct RawSeg {
  uint4 q;      // 16 bytes of codes (Q8_0 int8, K-quant nibbles) / first 16 B of f32
  uint4 hdr;    // Q4_K/Q5_K superblock header {d, dmin, scales[12]}; F32: bytes 16..31
  uint4 f32b;   // F32 bytes 32..47
  uint4 f32c;   // F32 bytes 48..63
  uint32_t x;   // Q8_0 scale bits / Q5_K qh word / Q6_K qh word
  uint32_t y;   // Q6_K: int8 scale (low byte) | d bits << 16
};

struct WPlanes {
  const uint8_t* p0;
  const uint8_t* p1;
  const uint8_t* p2;
  const uint8_t* p3;
  int K, N;
};

template <int FMT>
__device__ __forceinline__ RawSeg load_seg(const WPlanes& w, int n, int k0) {
  RawSeg r;
  const size_t N = (size_t)w.N;
  if constexpr (FMT == 8) {
    const size_t kb = (size_t)(k0 >> 5);
    r.q = *(const uint4*)(w.p0 + (kb * N + n) * 32 + ((k0 >> 4) & 1) * 16);
    r.x = ((const uint16_t*)w.p1)[kb * N + n];
  } else if constexpr (FMT == 12 || FMT == 13) {
    const size_t g = (size_t)(k0 >> 6);
    const int s = (k0 >> 4) & 3;
    r.q = *(const uint4*)(w.p0 + (g * N + n) * 32 + 16 * (s & 1));
    r.hdr = *(const uint4*)(w.p1 + ((g >> 2) * N + n) * 16);
    if constexpr (FMT == 13) r.x = ((const uint32_t*)w.p2)[(g * N + n) * 2 + (s >> 1)];
  } else if constexpr (FMT == 14) {
    const size_t g = (size_t)(k0 >> 6);
    const int s = (k0 >> 4) & 3;
    r.q = *(const uint4*)(w.p0 + (g * N + n) * 32 + 16 * (s & 1));
    r.x = *(const uint32_t*)(w.p1 + (g * N + n) * 16 + 4 * s);
    r.y = (uint32_t)w.p2[(g * N + n) * 4 + s] | ((uint32_t)((const uint16_t*)w.p3)[(g >> 2) * N + n] << 16);
  } else {  // F32
    const uint4* src = (const uint4*)(w.p0 + ((size_t)n * w.K + k0) * 4);
    r.q = src[0];
    r.hdr = src[1];
    r.f32b = src[2];
    r.f32c = src[3];
  }
  return r;
}

__device__ __forceinline__ uint32_t u4_word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Decode a segment into 16 floats.
template <int FMT>
__device__ __forceinline__ void decode_seg(const RawSeg& r, int k0, float* v) {
  if constexpr (FMT == 8) {
    const float d = f16_bits_to_f32(r.x);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int8_t q = (int8_t)((u4_word(r.q, i >> 2) >> (8 * (i & 3))) & 0xff);
      v[i] = (float)q * d;
    }
  } else if constexpr (FMT == 12 || FMT == 13) {
    const int g = k0 >> 6, s = (k0 >> 4) & 3, hi = s >> 1;
    uint8_t hb[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t w = u4_word(r.hdr, i);
      hb[4 * i + 0] = w & 0xff;
      hb[4 * i + 1] = (w >> 8) & 0xff;
      hb[4 * i + 2] = (w >> 16) & 0xff;
      hb[4 * i + 3] = (w >> 24) & 0xff;
    }
    const float d = f16_bits_to_f32(hb[0] | (hb[1] << 8));
    const float dmin = f16_bits_to_f32(hb[2] | (hb[3] << 8));
    float sc, m;
    scale_min_k4(2 * (g & 3) + hi, hb + 4, sc, m);
    const float ds = d * sc, dm = dmin * m;
    const uint32_t qh16 = (FMT == 13) ? ((r.x >> (16 * (s & 1))) & 0xffffu) : 0u;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t byte = (u4_word(r.q, i >> 2) >> (8 * (i & 3))) & 0xff;
      uint32_t q = hi ? (byte >> 4) : (byte & 0xF);
      if constexpr (FMT == 13) q |= ((qh16 >> i) & 1u) << 4;
      v[i] = fmaf(ds, (float)q, -dm);
    }
  } else if constexpr (FMT == 14) {
    const int s = (k0 >> 4) & 3, hi = s >> 1;
    const float d = f16_bits_to_f32(r.y >> 16);
    const float ds = d * (float)(int8_t)(r.y & 0xff);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t byte = (u4_word(r.q, i >> 2) >> (8 * (i & 3))) & 0xff;
      const int lo = hi ? (byte >> 4) : (byte & 0xF);
      const int h2 = (r.x >> (2 * i)) & 3;
      v[i] = ds * (float)((lo | (h2 << 4)) - 32);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[i] = __uint_as_float(u4_word(r.q, i));
      v[4 + i] = __uint_as_float(u4_word(r.hdr, i));
      v[8 + i] = __uint_as_float(u4_word(r.f32b, i));
      v[12 + i] = __uint_as_float(u4_word(r.f32c, i));
    }
  }
}

}  // namespace lle
