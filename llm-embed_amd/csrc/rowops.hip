// Row kernels: embedding gather + LayerNorm, LayerNorm, masked mean-pool + L2 (+ Matryoshka),
// f32 <-> f16 helpers and the raw-GGUF dequantisation test kernel.
#include "deq_device.h"
#include "lle_internal.h"

namespace lle {

constexpr int MAXE = 16;  // elements per lane: d_model <= 1024

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// LayerNormInPlace (internal/ggml/ops_simd.go:7-24): one-pass sum / sum of squares in f32,
// var = sumSq/n - mean^2, invStd = float32(1/sqrt(float64(var + eps))),
// y = (x - mean) * invStd * w + b. One wave per row; element j = lane + 64 i.
__device__ __forceinline__ void ln_row(float* x, int ne, int D, const float* w, const float* b, float eps,
                                       int lane, float* hrow, __half* h16row) {
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
    if (i < ne) {
      const int j = lane + 64 * i;
      const float y = (x[i] - mean) * inv * w[j] + b[j];
      hrow[j] = y;
      h16row[j] = __float2half_rn(y);
    }
}

// Embedding stage (internal/embed/bert.go:220-249, getEmbedding :290-316):
// h = deq(token_embd[id]) + deq(token_types[0]), then LayerNorm(token_embd_norm).
__global__ __launch_bounds__(256) void embed_ln_kernel(EmbedArgs a) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.T) return;
  int id = a.ids[t];
  if (id < 0 || id >= a.vocab) {
    if (lane == 0) atomicOr(a.status, 1);
    id = 0;
  }
  const uint8_t* row = a.tok + (size_t)id * a.tok_row_bytes;
  const int ne = a.D / 64;
  float x[MAXE];
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      const int j = lane + 64 * i;
      x[i] = deq_raw_elem(a.tok_type, row, j) + a.type0[j];
    }
  ln_row(x, ne, a.D, a.w, a.b, a.eps, lane, a.h + (size_t)t * a.D, a.h16 + (size_t)t * a.D);
}

hipError_t launch_embed_ln(const EmbedArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(embed_ln_kernel, dim3((a.T + 3) / 4), dim3(256), 0, st, a);
  return hipGetLastError();
}

// Residual has already been added by the GEMM epilogue; normalise in place and emit f16.
__global__ __launch_bounds__(256) void ln_kernel(float* h, __half* h16, const float* w, const float* b,
                                                 float eps, int T, int D) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int ne = D / 64;
  float* row = h + (size_t)t * D;
  float x[MAXE];
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) x[i] = row[lane + 64 * i];
  ln_row(x, ne, D, w, b, eps, lane, row, h16 + (size_t)t * D);
}

hipError_t launch_ln(float* h, __half* h16, const float* w, const float* b, float eps, int T, int D,
                     hipStream_t st) {
  hipLaunchKernelGGL(ln_kernel, dim3((T + 3) / 4), dim3(256), 0, st, h, h16, w, b, eps, T, D);
  return hipGetLastError();
}

// MeanPool + L2Normalize (+ Matryoshka truncation and renormalisation):
// internal/embed/pool.go:8-54, internal/embed/embedder.go:50-68. Rows with mask == 1 are
// summed in row order in f32 (the reference's order), scaled by float32(1/count); the norm
// is accumulated in f64. One block per sequence.
__global__ __launch_bounds__(256) void pool_kernel(const float* __restrict__ h, const int32_t* __restrict__ mask,
                                                   int L, int D, int out_dim, float* __restrict__ out) {
  const int b = blockIdx.x, tid = threadIdx.x;
  __shared__ double red[256];
  __shared__ float vals[1024];
  float cnt = 0.f;
  for (int j = tid; j < D; j += 256) {
    float s = 0.f;
    cnt = 0.f;
    for (int i = 0; i < L; i++) {
      if (mask[(size_t)b * L + i] == 1) {
        s += h[((size_t)b * L + i) * D + j];
        cnt += 1.f;
      }
    }
    if (cnt != 0.f) s *= 1.0f / cnt;
    vals[j] = s;
  }
  __syncthreads();
  // L2Normalize over the first n values, twice when truncating (embedder.go:65-68)
  int n = D;
  for (int pass = 0; pass < 2; pass++) {
    double acc = 0.0;
    for (int j = tid; j < n; j += 256) acc += (double)vals[j] * (double)vals[j];
    red[tid] = acc;
    __syncthreads();
    for (int s2 = 128; s2 > 0; s2 >>= 1) {
      if (tid < s2) red[tid] += red[tid + s2];
      __syncthreads();
    }
    const double norm = sqrt(red[0]);
    __syncthreads();
    if (norm != 0.0) {
      const float inv = (float)(1.0 / norm);
      for (int j = tid; j < n; j += 256) vals[j] = vals[j] * inv;
    }
    __syncthreads();
    if (out_dim >= D) break;
    n = out_dim;
  }
  const int od = out_dim < D ? out_dim : D;
  for (int j = tid; j < od; j += 256) out[(size_t)b * od + j] = vals[j];
}

hipError_t launch_pool(const float* h, const int32_t* mask, int B, int L, int D, int out_dim, float* out,
                       hipStream_t st) {
  hipLaunchKernelGGL(pool_kernel, dim3(B), dim3(256), 0, st, h, mask, L, D, out_dim, out);
  return hipGetLastError();
}

__global__ void f32_to_f16_kernel(const float* __restrict__ x, __half* __restrict__ y, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = __float2half_rn(x[i]);
}

hipError_t launch_f32_to_f16(const float* x, __half* y, int64_t n, hipStream_t st) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

__global__ void f16_bits_kernel(const uint16_t* __restrict__ h, float* __restrict__ out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = f16_bits_to_f32(h[i]);
}

hipError_t launch_f16_to_f32_bits(const uint16_t* h, float* out, int64_t n, hipStream_t st) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(f16_bits_kernel, dim3((unsigned)blocks), dim3(256), 0, st, h, out, n);
  return hipGetLastError();
}

// Raw GGUF blocks -> f32 (Tensor.Dequantize, internal/ggml/tensor.go:51-66); one element per
// thread, rows of 256 elements so every K-quant superblock is whole.
__global__ void dequant_raw_kernel(int type, const uint8_t* __restrict__ blocks, int64_t n, float* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t bs = type == 0 ? 1 : type == 8 ? 32 : 256;
  const int64_t bb = type == 0 ? 4 : type == 8 ? 34 : type == 12 ? 144 : type == 13 ? 176 : 210;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t blk = i / bs;
    out[i] = deq_raw_elem(type, blocks + blk * bb, (int)(i - blk * bs));
  }
}

hipError_t launch_dequant_raw(int type, const uint8_t* blocks, int64_t n, float* out, hipStream_t st) {
  int64_t nb = (n + 255) / 256;
  if (nb > 65536) nb = 65536;
  if (nb < 1) nb = 1;
  hipLaunchKernelGGL(dequant_raw_kernel, dim3((unsigned)nb), dim3(256), 0, st, type, blocks, n, out);
  return hipGetLastError();
}

}  // namespace lle
