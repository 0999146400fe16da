// Bit-preserving re-layout of GGUF weight blocks into the device planes described in
// lle_internal.h (WeightDev). Every code, scale and header byte of the GGUF blocks is
// stored verbatim (Q5_K's qh and Q6_K's ql/qh bits are only re-grouped per 64-element
// group), so the bytes per weight and the decoded values are exactly the GGUF ones.
// GGUF block layouts: internal/ggml/tensor.go:119-159 (Q8_0), quant_q4k.go:8-25 (Q4_K),
// quant_q5k.go:5-22 (Q5_K), quant_q6k.go:5-17 (Q6_K).
#include <string.h>

#include <vector>

#include "lle_internal.h"

namespace lle {

size_t weight_dev_bytes(int type, int K, int N) {
  const size_t n = (size_t)N, k = (size_t)K;
  switch (type) {
    case LLE_TYPE_Q8_0: return n * k + n * (k / 32) * 2;
    case LLE_TYPE_Q4_K: return n * (k / 2) + n * (k / 256) * 16;
    case LLE_TYPE_Q5_K: return n * (k / 2) + n * (k / 256) * 16 + n * (k / 64) * 8;
    case LLE_TYPE_Q6_K: return n * (k / 2) + n * (k / 4) + n * (k / 16) + n * (k / 256) * 2;
    case LLE_TYPE_F32: return n * k * 4;
    default: return 0;
  }
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Plane offsets inside one allocation (each plane 256-byte aligned).
void plane_offsets(int type, int K, int N, size_t off[4], size_t* total) {
  const size_t n = (size_t)N, k = (size_t)K;
  size_t sz[4] = {0, 0, 0, 0};
  switch (type) {
    case LLE_TYPE_Q8_0: sz[0] = n * k; sz[1] = n * (k / 32) * 2; break;
    case LLE_TYPE_Q4_K: sz[0] = n * (k / 2); sz[1] = n * (k / 256) * 16; break;
    case LLE_TYPE_Q5_K: sz[0] = n * (k / 2); sz[1] = n * (k / 256) * 16; sz[2] = n * (k / 64) * 8; break;
    case LLE_TYPE_Q6_K: sz[0] = n * (k / 2); sz[1] = n * (k / 4); sz[2] = n * (k / 16); sz[3] = n * (k / 256) * 2; break;
    case LLE_TYPE_F32: sz[0] = n * k * 4; break;
  }
  size_t o = 0;
  for (int i = 0; i < 4; i++) {
    off[i] = o;
    o = align256(o + sz[i]);
  }
  *total = o;
}

// gguf: N rows of row_bytes(type, K) bytes. dst: plane buffer laid out by plane_offsets.
void repack_rows(int type, const uint8_t* gguf, int K, int N, uint8_t* dst, const size_t off[4]) {
  const size_t n_ = (size_t)N;
  if (type == LLE_TYPE_F32) {
    memcpy(dst + off[0], gguf, n_ * K * 4);
    return;
  }
  if (type == LLE_TYPE_Q8_0) {
    const int nb = K / 32;
    const size_t rb = (size_t)nb * 34;
    uint8_t* codes = dst + off[0];
    uint8_t* sc = dst + off[1];
    for (size_t n = 0; n < n_; n++) {
      const uint8_t* row = gguf + n * rb;
      for (int b = 0; b < nb; b++) {
        const uint8_t* blk = row + (size_t)b * 34;
        memcpy(sc + ((size_t)b * n_ + n) * 2, blk, 2);
        memcpy(codes + ((size_t)b * n_ + n) * 32, blk + 2, 32);
      }
    }
    return;
  }
  const int nsb = K / 256;
  if (type == LLE_TYPE_Q4_K || type == LLE_TYPE_Q5_K) {
    const bool q5 = type == LLE_TYPE_Q5_K;
    const size_t bs = q5 ? 176 : 144;
    const size_t rb = (size_t)nsb * bs;
    uint8_t* qs = dst + off[0];
    uint8_t* hdr = dst + off[1];
    uint32_t* qh = (uint32_t*)(dst + off[2]);
    for (size_t n = 0; n < n_; n++) {
      const uint8_t* row = gguf + n * rb;
      for (int sb = 0; sb < nsb; sb++) {
        const uint8_t* blk = row + (size_t)sb * bs;
        memcpy(hdr + ((size_t)sb * n_ + n) * 16, blk, 16);  // d, dmin, scales[12]
        const uint8_t* src_qs = blk + (q5 ? 48 : 16);
        for (int g = 0; g < 4; g++) {
          const size_t grp = (size_t)sb * 4 + g;
          memcpy(qs + (grp * n_ + n) * 32, src_qs + 32 * g, 32);
          if (q5) {
            // word w bit l = high bit of element 32w + l of group g = bit (2g+w) of qh[l]
            const uint8_t* src_qh = blk + 16;
            for (int w = 0; w < 2; w++) {
              uint32_t word = 0;
              for (int l = 0; l < 32; l++) word |= (uint32_t)((src_qh[l] >> (2 * g + w)) & 1) << l;
              qh[(grp * n_ + n) * 2 + w] = word;
            }
          }
        }
      }
    }
    return;
  }
  if (type == LLE_TYPE_Q6_K) {
    const size_t rb = (size_t)nsb * 210;
    uint8_t* ql = dst + off[0];
    uint8_t* qh = dst + off[1];
    int8_t* sc = (int8_t*)(dst + off[2]);
    uint8_t* d = dst + off[3];
    uint8_t u[256];
    for (size_t n = 0; n < n_; n++) {
      const uint8_t* row = gguf + n * rb;
      for (int sb = 0; sb < nsb; sb++) {
        const uint8_t* blk = row + (size_t)sb * 210;
        // 6-bit code of element e (quant_q6k.go:37-47 layout)
        for (int e = 0; e < 256; e++) {
          const int c = e >> 7, el = e & 127, qq = el >> 5, l = el & 31;
          const uint8_t qlb = blk[64 * c + 32 * (qq & 1) + l];
          const int lo = (qq >> 1) ? (qlb >> 4) : (qlb & 0xF);
          const int hi = (blk[128 + 32 * c + l] >> (2 * qq)) & 3;
          u[e] = (uint8_t)(lo | (hi << 4));
        }
        memcpy(d + ((size_t)sb * n_ + n) * 2, blk + 208, 2);
        for (int g = 0; g < 4; g++) {
          const size_t grp = (size_t)sb * 4 + g;
          const uint8_t* ug = u + 64 * g;
          uint8_t* dql = ql + (grp * n_ + n) * 32;
          for (int l = 0; l < 32; l++) dql[l] = (uint8_t)((ug[l] & 0xF) | ((ug[32 + l] & 0xF) << 4));
          uint8_t* dqh = qh + (grp * n_ + n) * 16;
          for (int b = 0; b < 16; b++) {
            uint8_t v = 0;
            for (int t = 0; t < 4; t++) v |= (uint8_t)(((ug[4 * b + t] >> 4) & 3) << (2 * t));
            dqh[b] = v;
          }
          for (int s = 0; s < 4; s++) sc[(grp * n_ + n) * 4 + s] = (int8_t)blk[192 + 4 * g + s];
        }
      }
    }
  }
}

}  // namespace lle
