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
template <int TY>
__device__ __forceinline__ float deq_raw_t(const uint8_t* row, int j) {
  if constexpr (TY == 0) {
    return __uint_as_float(*(const uint32_t*)(row + 4 * j));
  } else if constexpr (TY == 8) {
    const uint8_t* b = row + (j >> 5) * 34;
    const float d = f16_bits_to_f32(b[0] | (b[1] << 8));
    return (float)(int8_t)b[2 + (j & 31)] * d;
  } else if constexpr (TY == 12 || TY == 13) {
    constexpr bool q5 = TY == 13;
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
  } else {
    static_assert(TY == 14, "raw type");
    const uint8_t* b = row + (j >> 8) * 210;
    const int e = j & 255, c = e >> 7, el = e & 127, qq = el >> 5, l = el & 31;
    const uint8_t qlb = b[64 * c + 32 * (qq & 1) + l];
    const int lo = (qq >> 1) ? (qlb >> 4) : (qlb & 0xF);
    const int hi = (b[128 + 32 * c + l] >> (2 * qq)) & 3;
    const int q = (lo | (hi << 4)) - 32;
    const float d = f16_bits_to_f32(b[208] | (b[209] << 8));
    return (d * (float)(int8_t)b[192 + (e >> 4)]) * (float)q;
  }
}

__device__ __forceinline__ float deq_raw_elem(int type, const uint8_t* row, int j) {
  switch (type) {
    case 0: return deq_raw_t<0>(row, j);
    case 8: return deq_raw_t<8>(row, j);
    case 12: return deq_raw_t<12>(row, j);
    case 13: return deq_raw_t<13>(row, j);
    case 14: return deq_raw_t<14>(row, j);
    default: return __uint_as_float(0x7fc00000u);
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

// ---------------------------------------------------------------------------------------
// Decode a segment straight to f16 (the GEMM operand). Every value equals the f32 decode
// above rounded once to f16 (round-to-nearest-even).
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t h2_bits(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t bits_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

__device__ __forceinline__ uint32_t pack_rn(float a, float b) {
  half2_t h;
  h.x = (_Float16)a;
  h.y = (_Float16)b;
  return h2_bits(h);
}

template <int FMT>
__device__ __forceinline__ void decode_seg_h(const RawSeg& r, int k0, uint4& lo, uint4& hi) {
  if constexpr (FMT == 8) {
    // q (int8) is exact in f16: bytes biased to q+128 are placed in the mantissa of 1024.0
    // (0x6400), giving 1024 + q + 128; subtracting 1152 leaves q exactly. q * d then rounds the
    // exact product once in f16, which is the f32 product (exact) rounded to f16.
    const half2_t d2 = bits_h2((r.x & 0xffffu) * 0x10001u);
    const half2_t bias = bits_h2(0x64806480u);  // 1152.0 in both halves
    uint32_t o[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const uint32_t u = u4_word(r.q, w) ^ 0x80808080u;
      const half2_t a = bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x05010400u)) - bias;
      const half2_t b = bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x05030402u)) - bias;
      o[2 * w] = h2_bits(a * d2);
      o[2 * w + 1] = h2_bits(b * d2);
    }
    lo = uint4{o[0], o[1], o[2], o[3]};
    hi = uint4{o[4], o[5], o[6], o[7]};
  } else if constexpr (FMT == 12 || FMT == 13 || FMT == 14) {
    // K-quants: the codes as bytes of four words, converted by byte (v_cvt_f32_ubyte*), one fma
    // per value with the same single rounding as decode_seg (the products are exact), packed
    // with round-to-nearest-even. Scale bytes are picked out of the header words by shifts.
    const int s = (k0 >> 4) & 3, hn = s >> 1;  // hn: high nibbles of the code bytes
    uint32_t qb[4];  // byte i of word w = code of element 4w + i
    float ds, off;   // value = fma(ds, code, off); Q6_K: ds * (code + off)
    if constexpr (FMT == 14) {
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.y >> 16));
      ds = d * (float)(int8_t)(r.y & 0xff);
      off = -32.0f;  // value = ds * (code - 32): subtract first, so code 32 gives ds * +0 (-0 for ds < 0)
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const uint32_t nib = hn ? (u4_word(r.q, w) >> 4) & 0x0F0F0F0Fu : u4_word(r.q, w) & 0x0F0F0F0Fu;
        const uint32_t t = (r.x >> (8 * w)) & 0xffu;  // four 2-bit high parts
        const uint32_t h2 = ((t << 4) | (t << 10) | (t << 16) | (t << 22)) & 0x30303030u;
        qb[w] = nib | h2;
      }
    } else {
      const int g = k0 >> 6, j = 2 * (g & 3) + hn, sh = 8 * (j & 3);
      const uint32_t y = (r.hdr.y >> sh) & 0xffu, z = (r.hdr.z >> sh) & 0xffu, w3 = (r.hdr.w >> sh) & 0xffu;
      const uint32_t sc = j < 4 ? (y & 63u) : ((w3 & 0xFu) | ((y >> 6) << 4));
      const uint32_t m = j < 4 ? (z & 63u) : ((w3 >> 4) | ((z >> 6) << 4));
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.hdr.x & 0xffffu));
      const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.hdr.x >> 16));
      ds = d * (float)sc;
      off = -(dmin * (float)m);
      const uint32_t qh16 = FMT == 13 ? (r.x >> (16 * (s & 1))) & 0xffffu : 0u;
#pragma unroll
      for (int w = 0; w < 4; w++) {
        uint32_t nib = hn ? (u4_word(r.q, w) >> 4) & 0x0F0F0F0Fu : u4_word(r.q, w) & 0x0F0F0F0Fu;
        if constexpr (FMT == 13)  // bit i of the 4-bit group -> bit 4 of byte i (no carries)
          nib |= (((qh16 >> (4 * w)) & 0xFu) * 0x00204081u & 0x01010101u) << 4;
        qb[w] = nib;
      }
    }
    auto val = [&](uint32_t code) {
      if constexpr (FMT == 14)
        return ds * ((float)code + off);  // exact, as (d*sc)*(q-32) in the reference
      else
        return fmaf(ds, (float)code, off);
    };
    uint32_t o[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
      o[2 * w] = pack_rn(val(qb[w] & 0xffu), val((qb[w] >> 8) & 0xffu));
      o[2 * w + 1] = pack_rn(val((qb[w] >> 16) & 0xffu), val(qb[w] >> 24));
    }
    lo = uint4{o[0], o[1], o[2], o[3]};
    hi = uint4{o[4], o[5], o[6], o[7]};
  } else {
    float v[16];
    decode_seg<FMT>(r, k0, v);
    lo = uint4{pack_rn(v[0], v[1]), pack_rn(v[2], v[3]), pack_rn(v[4], v[5]), pack_rn(v[6], v[7])};
    hi = uint4{pack_rn(v[8], v[9]), pack_rn(v[10], v[11]), pack_rn(v[12], v[13]), pack_rn(v[14], v[15])};
  }
}

// ---------------------------------------------------------------------------------------
// Buffer-resource loads for the large-M GEMM: every per-lane byte offset is loop-invariant and
// the per-K-step advance is a wave-uniform scalar offset, so a tile load costs no VALU.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

struct WRsrc {
  __amdgpu_buffer_rsrc_t r0, r1, r2, r3;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return uint4{t.x, t.y, t.z, t.w};
}

// Lane-invariant offsets of segment s (0..3, elements 16s..16s+15 of a 64-wide K step) of row n.
struct SegOff {
  int o0, o1, o2, o3;
};

template <int FMT>
__device__ __forceinline__ SegOff seg_off(int N, int K, int n, int s) {
  SegOff o{0, 0, 0, 0};
  if constexpr (FMT == 8) {
    o.o0 = ((s >> 1) * N + n) * 32 + (s & 1) * 16;
    o.o1 = ((s >> 1) * N + n) * 2;
  } else if constexpr (FMT == 12 || FMT == 13) {
    o.o0 = n * 32 + 16 * (s & 1);
    o.o1 = n * 16;
    o.o2 = n * 8 + 4 * (s >> 1);
  } else if constexpr (FMT == 14) {
    o.o0 = n * 32 + 16 * (s & 1);
    o.o1 = n * 16 + 4 * s;
    o.o2 = n * 4 + s;
    o.o3 = n * 2;
  } else {
    o.o0 = (n * K + 16 * s) * 4;
  }
  return o;
}

// Load segment (n, s) of 64-wide K step kt.
template <int FMT>
__device__ __forceinline__ RawSeg load_seg_buf(const WRsrc& w, const SegOff& o, int N, int kt) {
  RawSeg r;
  if constexpr (FMT == 8) {
    r.q = buf_load16(w.r0, o.o0, kt * 2 * N * 32);
    r.x = __builtin_amdgcn_raw_buffer_load_b16(w.r1, o.o1, kt * 2 * N * 2, 0);
  } else if constexpr (FMT == 12 || FMT == 13) {
    r.q = buf_load16(w.r0, o.o0, kt * N * 32);
    r.hdr = buf_load16(w.r1, o.o1, (kt >> 2) * N * 16);
    if constexpr (FMT == 13) r.x = __builtin_amdgcn_raw_buffer_load_b32(w.r2, o.o2, kt * N * 8, 0);
  } else if constexpr (FMT == 14) {
    r.q = buf_load16(w.r0, o.o0, kt * N * 32);
    r.x = __builtin_amdgcn_raw_buffer_load_b32(w.r1, o.o1, kt * N * 16, 0);
    const uint32_t sc = __builtin_amdgcn_raw_buffer_load_b8(w.r2, o.o2, kt * N * 4, 0);
    const uint32_t d = __builtin_amdgcn_raw_buffer_load_b16(w.r3, o.o3, (kt >> 2) * N * 2, 0);
    r.y = sc | (d << 16);
  } else {
    r.q = buf_load16(w.r0, o.o0, kt * 256);
    r.hdr = buf_load16(w.r0, o.o0 + 16, kt * 256);
    r.f32b = buf_load16(w.r0, o.o0 + 32, kt * 256);
    r.f32c = buf_load16(w.r0, o.o0 + 48, kt * 256);
  }
  return r;
}

}  // namespace lle
