// Row primitives shared by the row kernels and the GEMM's fused LayerNorm tail: a 64-lane sum
// with the same bits in every lane, and LayerNormInPlace over one row per wave.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace lle {

constexpr int MAXE = 16;  // elements per lane: d_model <= 1024

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes, the same bits in every lane: butterflies inside each row of 16 lanes
// on the DPP crossbar (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror; each step
// adds two equal-sized partial sums, so both partners hold the same value), then the four row
// sums combined as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// LayerNormInPlace (internal/ggml/ops_simd.go:7-24): one-pass sum / sum of squares in f32,
// var = sumSq/n - mean^2, invStd = float32(1/sqrt(float64(var + eps))),
// y = (x - mean) * invStd * w + b. One wave per row; element j = lane + 64 i.
// LayerNorm of one row held as x[i] = element lane + 64 i; x is replaced by the output y.
// ln_apply with the row's weights and biases already in registers (wv[i], bv[i] for element
// lane + 64 i): callers load them before the row itself, so their latency overlaps the row's.
__device__ __forceinline__ void ln_apply_wb(float* x, int ne, int D, const float* wv, const float* bv, float eps) {
  float s = 0.f, ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      s += x[i];
      ss += x[i] * x[i];
    }
  s = wave_sum(s);
  ss = wave_sum(ss);
  const float nf = (float)D;
  const float mean = s / nf;
  const float var = ss / nf - mean * mean;
  const float inv = (float)(1.0 / sqrt((double)(var + eps)));
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) x[i] = (x[i] - mean) * inv * wv[i] + bv[i];
}

// ln_apply_wb in two steps, for a LayerNorm whose elementwise step runs later in another kernel:
// the row's mean and invStd (the same operations in the same order, so the same bits), and the
// elementwise step (x - mean) * invStd * w + b (never fused: the library is built with
// -ffp-contract=off).
__device__ __forceinline__ void ln_mean_inv(const float* x, int ne, int D, float eps, float& mean, float& inv) {
  float s = 0.f, ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      s += x[i];
      ss += x[i] * x[i];
    }
  s = wave_sum(s);
  ss = wave_sum(ss);
  const float nf = (float)D;
  mean = s / nf;
  const float var = ss / nf - mean * mean;
  inv = (float)(1.0 / sqrt((double)(var + eps)));
}
__device__ __forceinline__ float ln_elem(float x, float mean, float inv, float w, float b) {
  return (x - mean) * inv * w + b;
}

__device__ __forceinline__ void ln_apply(float* x, int ne, int D, const float* w, const float* b, float eps,
                                         int lane) {
  float wv[MAXE], bv[MAXE];  // issued before the reductions so their latency overlaps them
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      wv[i] = w[lane + 64 * i];
      bv[i] = b[lane + 64 * i];
    }
  ln_apply_wb(x, ne, D, wv, bv, eps);
}

// LayerNormInPlace of one row into hrow (f32) and h16row (f16).
__device__ __forceinline__ void ln_row(float* x, int ne, int D, const float* w, const float* b, float eps,
                                       int lane, float* hrow, __half* h16row) {
  ln_apply(x, ne, D, w, b, eps, lane);
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      const int j = lane + 64 * i;
      hrow[j] = x[i];
      h16row[j] = __float2half_rn(x[i]);
    }
}

}  // namespace lle
