// Attention block as a device function (bidirectional masked multi-head attention, the
// reference's softmax semantics), run by the attention kernel (attention.hip).
#pragma once

#include "lle_internal.h"
#include "mfma_common.h"

namespace lle {

constexpr int AK = 64;   // keys per tile
constexpr int HD = 64;   // head dim
constexpr int APAD = 8;


typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Raw buffer of nbytes at base (loads at offsets >= nbytes return zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nbytes, 0x00020000);
}
// A wave-uniform pointer moved to scalar registers (64-bit products are formed on the VALU, and
// a buffer descriptor built from VGPRs turns every load into a readfirstlane loop).
__device__ __forceinline__ const __half* uniform_ptr(const __half* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const __half*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
// Smallest f32 not below y (y is computed in f64; see keep_threshold).
__device__ __forceinline__ float ceil_f32(double y) {
  float f = (float)y;
  if ((double)f < y) {
    unsigned int u = __float_as_uint(f);
    u = f == 0.f ? 1u : (f > 0.f ? u + 1u : u - 1u);  // one step towards +inf
    f = __uint_as_float(u);
  }
  return f;
}
// Keep rule of the reference's softmax, fl(s - m) >= -10 with s = u / 8 (exact), as a threshold
// on the unscaled score u. fl(x) >= -10 exactly when x >= -10 - 2^-21 (the f32 spacing below 10
// is 2^-20 and a tie rounds to the even -10), so a key is kept exactly when
// u >= 8 * ceil_f32(m - 10 - 2^-21). m is f32, and m + (-10 - 2^-21) is exact in f64 for
// 2^-26 <= |m| < 2^31; for smaller |m| no f32 lies within the f64 rounding error of the sum.
__device__ __forceinline__ float keep_threshold(float m_u) {
  const double y = (double)(m_u * 0.125f) + (-10.0 - 0x1p-21);
  return 8.f * ceil_f32(y);
}

// Maximum / minimum over lanes l, l ^ 16, l ^ 32 and l ^ 48 of a wave (the four lanes that hold
// one query's scores). v_permlane16_swap / v_permlane32_swap exchange 16-lane rows between two
// registers without an LDS round trip; afterwards each lane holds its own value in one register
// and its partner's in the other. max and min are order-free, so the result is the xor
// butterfly's bit for bit.
__device__ __forceinline__ float max_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float min_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fminf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fminf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff) {
  const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
  return uint4{t.x, t.y, t.z, t.w};
}

// NW waves per block (16 queries each). K / V^T tiles are double-buffered: the global loads of
// key tile kt+1 are issued before tile kt's MFMAs and land in the other LDS buffer afterwards.
// The 8-wave kernel is held to 128 VGPRs (4 waves per SIMD, two blocks per CU).
// LDS of one attention block, carved from one buffer: K tiles [2][AK][HD + APAD] f16, V^T
// tiles [2][HD][AK + APAD] f16, the tiles' masks [2][AK], their all-valid flags, the pass flag
// and the key-range scan's per-wave bounds.
template <int NW>
struct AttnShape {
  static constexpr size_t K = 0, V = K + 2 * AK * (HD + APAD) * 2, MASK = V + 2 * HD * (AK + APAD) * 2;
  static constexpr size_t FULL = MASK + 2 * AK * 4, REDO = FULL + 2 * 4, LO = REDO + 4, HI = LO + NW * 4;
  static constexpr size_t LDS = (HI + NW * 4 + 15) / 16 * 16;
};

// Block (qt, h, b) of the attention: query tile qt of head h of sequence b, NW waves, its LDS at
// `lds` (AttnShape<NW>::LDS bytes, 16-byte aligned).
template <int NW, bool EARLY>
__device__ __forceinline__ void attention_dev(const AttnArgs& a, int qt, int h, int b, unsigned char* lds) {
  using AS = AttnShape<NW>;
  lds = static_cast<unsigned char*>(__builtin_assume_aligned(lds, 16));
  constexpr int NT = NW * 64, AQB = NW * 16;
  // Long rows (8-wave blocks) test the keep rule as a per-query threshold on the unscaled score,
  // recomputed once per key tile (one f64 chain) in place of a fused multiply-add per score.
  // Short rows (one key tile) compare directly, off that chain's latency. Both keep exactly the
  // same keys, so every output bit is the same either way.
  constexpr bool THR = NW == 8;
  constexpr int CPT = (AK * HD / 8) / NT;  // 16-byte chunks of each tile per thread
  _Float16(*sK)[AK][HD + APAD] = reinterpret_cast<_Float16(*)[AK][HD + APAD]>(lds + AS::K);  // [key][dim]
  _Float16(*sV)[HD][AK + APAD] = reinterpret_cast<_Float16(*)[HD][AK + APAD]>(lds + AS::V);  // [dim][key]
  int(*sMask)[AK] = reinterpret_cast<int(*)[AK]>(lds + AS::MASK);
  int* sFull = reinterpret_cast<int*>(lds + AS::FULL);
  int& sRedo = *reinterpret_cast<int*>(lds + AS::REDO);

  // the compiler builtin, not threadIdx.x: this file is built with the IEEE-mode bit off, so
  // the device library's index functions (built with it on) are not inlined but called, and
  // every call waits for all outstanding loads first
  const int tid = __builtin_amdgcn_workitem_id_x(), lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, lr = lane & 15;
  const int L = a.L, Lp = a.Lp, H = a.H;
  const size_t head = (size_t)b * H + h;
  const int q = qt * AQB + wave * 16 + lr;
  // positions of this sequence held in Q / K / V^T: all L, or (packed rows) up to its last
  // valid token; keys and queries past them are zero / not written
  const int Lk = __builtin_amdgcn_readfirstlane(a.seq_off ? a.seq_off[b + 1] - a.seq_off[b] : L);  // uniform
  const size_t orow = a.seq_off ? (size_t)a.seq_off[b] : (size_t)b * L;
  // only valid (mask 1) queries may ask for the fixed-max pass: padding queries' outputs are
  // never used, and the pass decision must not depend on how a sequence was padded
  // (loaded here for every lane, clamped, and tested only after the pass: a conditional load
  // here made the compiler wait for it at once)
  const int qmask = a.mask[(size_t)b * L + min(q, L - 1)];

  // Q^T fragments (B operand of S): query q, dims ks*32 + 8g .. +7
  half8 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    if (q < Lk)
      qf[ks] = *(const half8*)(a.q + (head * Lp + q) * HD + ks * 32 + g * 8);
    else
      qf[ks] = half8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  uint4 kreg[CPT], vreg[CPT];
  int mreg = 0;
  // K and V^T tiles through buffer loads: the per-lane byte offsets are fixed and a tile adds
  // one constant. K's buffer is this head's first Lk rows, so rows at and past Lk read as zero
  // (range check); every visited tile lies below Lp, so each load is inside the allocation.
  // V^T's columns at and past Lk are never written and are zeroed in the tile that holds Lk.
  const __half* const kbase = uniform_ptr(a.k + head * Lp * HD);
  const __half* const vbase = uniform_ptr(a.vt + head * HD * Lp);
  int koff[CPT], voff[CPT];
#pragma unroll
  for (int i = 0; i < CPT; i++) {
    const int c = tid + i * NT, row = c >> 3, ch = c & 7;
    koff[i] = (row * HD + ch * 8) * 2;
    voff[i] = (row * Lp + ch * 8) * 2;
  }
  auto gload = [&](int kt) {
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, Lk * HD * 2);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, HD * Lp * 2);
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      kreg[i] = buf_load16(rk, koff[i] + kt * (AK * HD * 2));
      uint4 vv = buf_load16(rv, voff[i] + kt * (AK * 2));
      if ((kt + 1) * AK > Lk) {  // wave-uniform: the tile that holds Lk (or lies past it)
        const int c = tid + i * NT, ch = c & 7;
        const int nv = Lk - (kt * AK + ch * 8);
        vv.x &= (nv > 0 ? 0xFFFFu : 0u) | (nv > 1 ? 0xFFFF0000u : 0u);
        vv.y &= (nv > 2 ? 0xFFFFu : 0u) | (nv > 3 ? 0xFFFF0000u : 0u);
        vv.z &= (nv > 4 ? 0xFFFFu : 0u) | (nv > 5 ? 0xFFFF0000u : 0u);
        vv.w &= (nv > 6 ? 0xFFFFu : 0u) | (nv > 7 ? 0xFFFF0000u : 0u);
      }
      vreg[i] = vv;
    }
    if (tid < AK) {
      const int key = kt * AK + tid;
      mreg = key < L ? a.mask[(size_t)b * L + key] : 0;
    }
  };
  // [klo, khi): from the first to one past the last valid key of the sequence (all L keys when
  // none is valid: the softmax is then uniform over every key). EARLY (launched when one load
  // per thread covers the mask row, L <= NT): key tile 0's loads are issued right after the
  // mask load, before the scan needs them (the first valid key is nearly always in tile 0;
  // otherwise the tile is loaded again below). With longer rows they would sit in front of the
  // scan's remaining mask loads (loads complete in issue order).
  int* sLo = reinterpret_cast<int*>(lds + AS::LO);
  int* sHi = reinterpret_cast<int*>(lds + AS::HI);
  int klo, khi;
  bool novalid;
  {
    const int32_t* mrow = a.mask + (size_t)b * L;
    int lo = L, hi = -1, i0 = tid;
    if constexpr (EARLY) {
      const int mv0 = mrow[min(tid, L - 1)];  // unconditional: a guarded load was waited for at once
      gload(0);
      __builtin_amdgcn_sched_barrier(0);  // the tile's loads are issued before the test waits
      if (tid < L && mv0 != 0) {
        lo = tid;
        hi = tid;
      }
      i0 = tid + NT;
    }
#pragma unroll 4
    for (int i = i0; i < L; i += NT) {
      if (mrow[i] != 0) {
        lo = min(lo, i);
        hi = max(hi, i);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      lo = min(lo, __shfl_xor(lo, o));
      hi = max(hi, __shfl_xor(hi, o));
    }
    if (lane == 0) {
      sLo[wave] = lo;
      sHi[wave] = hi;
    }
    __syncthreads();
    lo = sLo[0];
    hi = sHi[0];
#pragma unroll
    for (int w = 1; w < NW; w++) {
      lo = min(lo, sLo[w]);
      hi = max(hi, sHi[w]);
    }
    klo = hi < 0 ? 0 : lo;
    khi = hi < 0 ? L : hi + 1;
    novalid = hi < 0;
  }
  const int t0 = klo / AK, t1 = (khi + AK - 1) / AK;
  if (qt * AQB >= khi) {
    // every query of this block lies past the last valid key, so it is padding (mask 0):
    // its output is never used, but stays finite (zero) for the next layer's masked P.V
    if (q < Lk) {
      __half* dst = a.out + (orow + q) * a.D + h * HD + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 4; dt++) *(uint2*)(dst + dt * 16) = uint2{0u, 0u};
    }
    return;
  }
  const float scale = 0.125f;  // float32(1/sqrt(64)), bert.go:362
  // exp(s - m) = 2^((u - 8 m) * log2(e) / 8): one fmaf with c1 = fl(log2 e) / 8 (exact scaling)
  const float c1 = 1.44269504f * 0.125f;
  // A masked key's unscaled score: -8e9 (s = -1e9 exactly). A sequence without a valid key has
  // every key masked, its softmax is uniform (and its rows are never pooled); 0 then gives the
  // same uniform weights without the cancellation of -8e9 * c1 against the reference point.
  const float mval = novalid ? 0.f : -8e9f;
  // Rows of P are scaled by 2^(-m_ref * c1), m_ref a query's running maximum (unscaled) as of its
  // last rescale. The accumulators are rescaled only when the running maximum has moved more
  // than kTau past m_ref, so P stays below e^(kTau / 8) (f16 range) and most key tiles skip the
  // rescale. Each query decides alone (its lanes hold the same maxima), so its arithmetic does
  // not depend on the other queries of its wave.
  constexpr float kTau = 64.f;

  float m_u = -INFINITY, smin = INFINITY;  // running maximum and smallest kept score (unscaled)
  floatx4 o[4];
  // row sums of P on the matrix core: an all-ones V^T fragment against the same P^T fragment
  // gives, in every row of its 16 x 16 result, the sum over the tile's keys of each query's f16
  // probabilities (the weights the P.V MFMAs use), so the normalisation divides by exactly the
  // weights the numerator summed
  floatx4 osum;
  half8 ones;
#pragma unroll
  for (int i = 0; i < 8; i++) ones[i] = (_Float16)1.0f;

  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int c = tid + i * NT, row = c >> 3, ch = c & 7;
      *(uint4*)&sK[buf][row][ch * 8] = kreg[i];
      *(uint4*)&sV[buf][row][ch * 8] = vreg[i];
    }
    if (tid < AK) sMask[buf][tid] = mreg;
    if (tid < 64) {  // wave 0: one flag per tile, set when all 64 keys are valid
      const bool all = __all(mreg == 1);
      if (tid == 0) sFull[buf] = all;
    }
  };

  if (tid == 0) sRedo = 0;
  for (int pass = 0; pass < 2; pass++) {
    const bool fixed = pass == 1;
    if (fixed) {
      __syncthreads();
      if (!sRedo) break;
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    osum = floatx4{0.f, 0.f, 0.f, 0.f};
    smin = INFINITY;
    // the fixed pass uses the final maximum for the keep rule and as the reference point
    float m_ref = fixed ? m_u : -INFINITY;
    float nb = -(m_ref * c1);
    float thr = fixed && THR ? keep_threshold(m_u) : 0.f;

    __syncthreads();  // the buffers of a previous pass are no longer read
    if (!EARLY || fixed || t0 != 0) gload(t0);  // else tile 0 is already in registers
    sstore(0);
    __syncthreads();
    for (int kt = t0; kt < t1; kt++) {
      const int buf = (kt - t0) & 1;
      const bool more = kt + 1 < t1;
      if (more) gload(kt + 1);

      // S^T tiles: st[t][r] = score of key kidx(t, r) for query q
      floatx4 st[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int krow = 32 * (t >> 1) + 8 * (lr >> 2) + 4 * (t & 1) + (lr & 3);
        floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
          const half8 kf = *(const half8*)&sK[buf][krow][ks * 32 + g * 8];
          acc = mfma16(kf, qf[ks], acc);
        }
        st[t] = acc;
      }
      // u = unscaled score; the reference's s = u * scale is exact (a power of two), so s is
      // never formed: a masked key gets u = -8e9 (u * scale = -1e9 exactly), maxima and minima
      // are taken on u and scaled afterwards, and s - m is fmaf(u, scale, -m), whose single
      // rounding is that of the subtraction.
      float s[16];
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) s[4 * t + r] = st[t][r];
      if (!sFull[buf]) {  // masked (and out-of-range) keys; tiles of valid keys skip the lookups
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (sMask[buf][32 * (t >> 1) + 8 * g + 4 * (t & 1) + r] == 0) s[4 * t + r] = mval;
      }
      // the tile's smallest score: when it is kept, so is every key of the tile
      float tmin = INFINITY;
#pragma unroll
      for (int i = 0; i < 16; i += 2) tmin = fminf(tmin, fminf(s[i], s[i + 1]));
      if (!fixed) {
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) tmax = fmaxf(tmax, s[i]);
        const float m_new = fmaxf(m_u, max_rows(tmax));
        if constexpr (THR) {
          // the threshold follows the maximum, which settles after the first few tiles
          if (__any(m_new != m_u)) thr = keep_threshold(m_new);
        }
        m_u = m_new;
        const bool need = m_u > m_ref + kTau;  // always on the first tile (m_ref = -inf)
        if (__any(need)) {
          const float alpha = need ? __builtin_amdgcn_exp2f((m_ref - m_u) * c1) : 1.f;
          osum *= alpha;
#pragma unroll
          for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
          m_ref = need ? m_u : m_ref;
          nb = -(m_ref * c1);
        }
      }
      // The keep rule fl(s - m) >= -10, tested as u >= thr (THR) or directly: the same keys.
      const float m_s = m_u * scale;
      auto keeps = [&](float u) {
        if constexpr (THR)
          return u >= thr;
        else
          return fmaf(u, scale, -m_s) >= -10.f;
      };
      float e[16];
#pragma unroll
      for (int i = 0; i < 16; i++) e[i] = __builtin_amdgcn_exp2f(fmaf(s[i], c1, nb));
      if (__any(!keeps(tmin))) {
        // some query of the wave drops a key of this tile: exp of a dropped key is discarded,
        // and the smallest kept score is taken over the kept keys (for a query that dropped
        // nothing both are what the tile minimum already holds)
        tmin = INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const bool keep = keeps(s[i]);
          e[i] = keep ? e[i] : 0.f;
          tmin = fminf(tmin, keep ? s[i] : INFINITY);
        }
      }
      smin = fminf(smin, tmin);  // smallest kept score (exact, order-free)
      // P^T fragments: keys 32j + 8g + 0..7
#pragma unroll
      for (int j = 0; j < 2; j++) {
        half8 pf;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          pf[r] = (_Float16)e[4 * (2 * j) + r];
          pf[4 + r] = (_Float16)e[4 * (2 * j + 1) + r];
        }
        if constexpr (NW == 8) {  // the four V^T fragment reads issued together, then the MFMAs
          half8 vf[4];
#pragma unroll
          for (int dt = 0; dt < 4; dt++) vf[dt] = *(const half8*)&sV[buf][dt * 16 + lr][32 * j + 8 * g];
#pragma unroll
          for (int dt = 0; dt < 4; dt++) o[dt] = mfma16(vf[dt], pf, o[dt]);
        } else {  // one read per MFMA: keeps the 4-wave kernel at 3 waves per SIMD
#pragma unroll
          for (int dt = 0; dt < 4; dt++) {
            const half8 vf = *(const half8*)&sV[buf][dt * 16 + lr][32 * j + 8 * g];
            o[dt] = mfma16(vf, pf, o[dt]);
          }
        }
        osum = mfma16(ones, pf, osum);
      }
      if (more) sstore(buf ^ 1);  // buffer buf^1 was last read in iteration kt-1
      __syncthreads();
    }
    if (!fixed) {
      const float sm = min_rows(smin) * scale;
      const bool qvalid = q < L && qmask == 1;
      const bool flag = qvalid && (sm - m_u * scale < -10.f);
      if (__any(flag)) sRedo = 1;  // benign race: every writer stores 1
    }
  }

  const float tot = osum[0];  // every row of osum holds the query's sum over all keys
  if (q < Lk) {
    const float inv = 1.f / tot;
    __half* dst = a.out + (orow + q) * a.D + h * HD + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
      __half2 lo = __floats2half2_rn(o[dt][0] * inv, o[dt][1] * inv);
      __half2 hi = __floats2half2_rn(o[dt][2] * inv, o[dt][3] * inv);
      uint2 pk;
      pk.x = *(uint32_t*)&lo;
      pk.y = *(uint32_t*)&hi;
      *(uint2*)(dst + dt * 16) = pk;
    }
  }
}

}  // namespace lle
