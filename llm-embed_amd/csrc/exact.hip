// Reference-exact f32 forward (lle_model_set_precision(m, LLE_PRECISION_F32)): the fp32
// fallback of the MFMA path. Every operation follows the reference CPU path's f32 arithmetic
// in the reference's order, so an embedding equals the reference's bit for bit, up to the last
// float64 ulp of exp() inside the softmax (glibc / Go math.Exp / the GPU's exp can differ there,
// which reaches an f32 result only on a rounding boundary).
//
//   GEMM (GemmPrePacked32, internal/ggml/gemm_avx512.go:67-147 with the micro-kernel
//   internal/ggml/gemm_avx512_amd64.s:22-195): C = 0; for each 128-wide K chunk the output's
//   partial sum starts at 0 and runs over k in order, fused (FMA) for rows inside a sequence's
//   full 6-row tiles, unfused (product rounded, then sum rounded) for the last L % 6 rows of a
//   sequence of L tokens; C = partial + C after each chunk. W is the f32 dequantisation (the
//   reference's PreDequant copy, internal/embed/bert.go:542-576).
//   QKV split + RoPE (bert.go:332-354, ops_simd.go:127-137), GeLU (ops_simd.go:27-42, exact
//   division), residual adds (bert.go:261-264,275-278), LayerNormInPlace (ops_simd.go:7-24:
//   sequential sums), attention (bert.go:356-402: DotF32's unroll-4 order, -1e9 mask, softmax
//   with exp in f64 and the x < -10 cutoff, sequential sum, P.V in key order), MeanPool and
//   L2Normalize (internal/embed/pool.go:8-54, f64 norm), Matryoshka (embedder.go:65-68).
// Device code is compiled with -ffp-contract=off: nothing fuses but the explicit fmaf of the
// GEMM's full rows.
#include "deq_device.h"
#include "lle_internal.h"

namespace lle {

namespace {

// Sequence of forward row t: (sequence b, position p, first row of the sequence, its length).
struct SeqPos {
  int b, p, row0, ls;
};
__device__ __forceinline__ SeqPos seq_of(const ExactArgs& a, int t) {
  const int tk = a.tokrow ? a.tokrow[t] : t;
  SeqPos s;
  s.b = tk / a.L;
  s.p = tk - s.b * a.L;
  if (a.seq_off) {
    s.row0 = a.seq_off[s.b];
    s.ls = a.seq_off[s.b + 1] - s.row0;
  } else {
    s.row0 = s.b * a.L;
    s.ls = a.L;
  }
  return s;
}

// The reference's GeLU: t = c0 v (1 + c1 v v), tanh ~ t (27 + t^2) / (27 + 9 t^2), +-1 past
// |t| 4.97, 0.5 v (1 + tanh); left-to-right evaluation, IEEE division.
__device__ __forceinline__ float gelu_exact(float v) {
  const float c0 = 0.7978845608f, c1 = 0.044715f;
  const float t = c0 * v * (1.0f + c1 * v * v);
  const float t2 = t * t;
  float th = t * (27.0f + t2) / (27.0f + 9.0f * t2);
  if (t > 4.97f)
    th = 1.0f;
  else if (t < -4.97f)
    th = -1.0f;
  return 0.5f * v * (1.0f + th);
}

// LayerNormInPlace on one row held in global memory, by one thread.
__device__ __forceinline__ void ln_seq(float* x, int D, const float* w, const float* b, float eps) {
  float sum = 0.0f, sumsq = 0.0f;
  for (int i = 0; i < D; i++) {
    const float v = x[i];
    sum += v;
    sumsq += v * v;
  }
  const float nf = (float)D;
  const float mean = sum / nf;
  const float var = sumsq / nf - mean * mean;
  const float inv = (float)(1.0 / sqrt((double)(var + eps)));
  for (int i = 0; i < D; i++) x[i] = (x[i] - mean) * inv * w[i] + b[i];
}

constexpr int XG_T = 64, XG_N = 64, XG_KC = 128, XG_LD = XG_KC + 4;

}  // namespace

// Embedding: h = deq(token_embd[id]) + token_types[0], LayerNorm (bert.go:220-249); one
// thread per row.
__global__ __launch_bounds__(64) void exact_embed_kernel(ExactArgs a) {
  const int t = blockIdx.x * 64 + threadIdx.x;
  if (t >= a.T) return;
  int id = a.ids[t];
  if (id < 0 || id >= a.vocab) {
    atomicOr(a.status, 1);
    id = 0;
  }
  const uint8_t* row = a.tok + (size_t)id * a.tok_row_bytes;
  float* h = a.h + (size_t)t * a.D;
  for (int j = 0; j < a.D; j++) h[j] = deq_raw_elem(a.tok_type, row, j) + a.type0[j];
  ln_seq(h, a.D, a.lnw, a.lnb, a.eps);
}

// LayerNorm of every row of h in place (after a residual add); one thread per row.
__global__ __launch_bounds__(64) void exact_ln_kernel(ExactArgs a) {
  const int t = blockIdx.x * 64 + threadIdx.x;
  if (t >= a.T) return;
  ln_seq(a.h + (size_t)t * a.D, a.D, a.lnw, a.lnb, a.eps);
}

// C[t][n] = X[t][:] . W[n][:] in the reference order, 64 tokens x 64 features per block, each
// thread 4 x 4 outputs; one 128-wide K chunk of both tiles in LDS at a time.
template <int EPI>
__global__ __launch_bounds__(256) void exact_gemm_kernel(ExactArgs a, ExactGemm g) {
  __shared__ __attribute__((aligned(16))) float sX[XG_T][XG_LD];
  __shared__ __attribute__((aligned(16))) float sW[XG_N][XG_LD];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * XG_T, n0 = blockIdx.x * XG_N;
  const int T = a.T, K = g.K;
  // fused rows: inside the sequence's full 6-row tiles
  bool fr[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = m0 + ty * 4 + i;
    if (t < T) {
      const SeqPos s = seq_of(a, t);
      fr[i] = s.p < 6 * (s.ls / 6);
    } else {
      fr[i] = true;
    }
  }
  const bool allf = fr[0] && fr[1] && fr[2] && fr[3];
  float c[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) c[i][j] = 0.0f;

  for (int k0 = 0; k0 < K; k0 += XG_KC) {
    const int kc = min(XG_KC, K - k0);  // K % 4 == 0
    __syncthreads();  // the previous chunk's reads are done
    for (int q = tid; q < XG_T * (XG_KC / 4); q += 256) {
      const int r = q / (XG_KC / 4), k4 = (q % (XG_KC / 4)) * 4;
      float4 xv = make_float4(0.f, 0.f, 0.f, 0.f), wv = make_float4(0.f, 0.f, 0.f, 0.f);
      if (k4 < kc) {
        if (m0 + r < T) xv = *(const float4*)(g.x + (size_t)(m0 + r) * K + k0 + k4);
        wv = *(const float4*)(g.w + (size_t)(n0 + r) * K + k0 + k4);
      }
      *(float4*)&sX[r][k4] = xv;
      *(float4*)&sW[r][k4] = wv;
    }
    __syncthreads();
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    if (allf) {
      for (int k = 0; k < kc; k += 4) {
        float4 av[4], bv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) av[i] = *(const float4*)&sX[ty * 4 + i][k];
#pragma unroll
        for (int j = 0; j < 4; j++) bv[j] = *(const float4*)&sW[tx * 4 + j][k];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            acc[i][j] = fmaf(av[i].x, bv[j].x, acc[i][j]);
            acc[i][j] = fmaf(av[i].y, bv[j].y, acc[i][j]);
            acc[i][j] = fmaf(av[i].z, bv[j].z, acc[i][j]);
            acc[i][j] = fmaf(av[i].w, bv[j].w, acc[i][j]);
          }
      }
    } else {  // a thread holding one of a sequence's last L % 6 rows: those rows unfused
      for (int k = 0; k < kc; k += 4) {
        float4 av[4], bv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) av[i] = *(const float4*)&sX[ty * 4 + i][k];
#pragma unroll
        for (int j = 0; j < 4; j++) bv[j] = *(const float4*)&sW[tx * 4 + j][k];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            if (fr[i]) {
              acc[i][j] = fmaf(av[i].x, bv[j].x, acc[i][j]);
              acc[i][j] = fmaf(av[i].y, bv[j].y, acc[i][j]);
              acc[i][j] = fmaf(av[i].z, bv[j].z, acc[i][j]);
              acc[i][j] = fmaf(av[i].w, bv[j].w, acc[i][j]);
            } else {
              acc[i][j] = acc[i][j] + av[i].x * bv[j].x;
              acc[i][j] = acc[i][j] + av[i].y * bv[j].y;
              acc[i][j] = acc[i][j] + av[i].z * bv[j].z;
              acc[i][j] = acc[i][j] + av[i].w * bv[j].w;
            }
          }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) c[i][j] = acc[i][j] + c[i][j];
  }

  const int f = n0 + tx * 4;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = m0 + ty * 4 + i;
    if (t >= T) continue;
    float* v = c[i];
    if constexpr (EPI == EPI_F32) {
      *(float4*)(g.y + (size_t)t * g.N + f) = make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (EPI == EPI_RESID) {
      // hiddens[i][j] += out[i][j]
      float4* yp = (float4*)(g.y + (size_t)t * g.N + f);
      float4 h = *yp;
      h.x = h.x + v[0];
      h.y = h.y + v[1];
      h.z = h.z + v[2];
      h.w = h.w + v[3];
      *yp = h;
    } else if constexpr (EPI == EPI_QKV) {
      // row = [Q | K | V]; RoPE on the (2i, 2i+1) pairs of every Q and K head at the token's
      // position in its sequence
      const int D = a.D, sec = f / D, fs = f - sec * D;
      if (sec < 2) {
        const int p = seq_of(a, t).p;
        const int pr = (fs % 64) / 2;  // pair index of (f, f+1) in the head
        const float* cs = a.rope_cos + (size_t)p * 32;
        const float* sn = a.rope_sin + (size_t)p * 32;
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const float x0 = v[2 * u], x1 = v[2 * u + 1], cc = cs[pr + u], ss = sn[pr + u];
          v[2 * u] = x0 * cc - x1 * ss;
          v[2 * u + 1] = x0 * ss + x1 * cc;
        }
      }
      float* dst = (sec == 0 ? a.q : sec == 1 ? a.k : a.v) + (size_t)t * D + fs;
      *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
    } else {  // EPI_GEGLU: interleaved rows (up q, gate q): gates = GeLU(gate) * up
      const int qf = f / 2;
      float* dst = g.y + (size_t)t * (g.N / 2) + qf;
      dst[0] = gelu_exact(v[1]) * v[0];
      dst[1] = gelu_exact(v[3]) * v[2];
    }
  }
}

// One wave per (query row, head): scores in the reference's order, softmax, P.V.
// Dynamic LDS: the sequence's scores (L floats) + one 64-key K tile.
__global__ __launch_bounds__(64) void exact_attention_kernel(ExactArgs a) {
  extern __shared__ float smem[];
  float* sS = smem;                      // [L]
  float* sK = smem + ((a.L + 3) & ~3);   // [64][65]
  const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int D = a.D, HD = 64;
  const SeqPos s = seq_of(a, t);
  const int ls = s.ls;
  const float* qrow = a.q + (size_t)t * D + h * HD;
  float qv[64];
#pragma unroll
  for (int d = 0; d < 64; d++) qv[d] = qrow[d];
  const float scale = 0.125f;  // float32(1/sqrt(64)), bert.go:362
  const int32_t* mrow = a.mask + (size_t)s.b * a.L;
  for (int k0 = 0; k0 < ls; k0 += 64) {
    const int nk = min(64, ls - k0);
    for (int q = lane; q < 64 * 16; q += 64) {  // 64 keys x 16 float4
      const int r = q >> 4, c4 = (q & 15) * 4;
      if (r < nk) {
        const float4 kv = *(const float4*)(a.k + (size_t)(s.row0 + k0 + r) * D + h * HD + c4);
        sK[r * 65 + c4] = kv.x;
        sK[r * 65 + c4 + 1] = kv.y;
        sK[r * 65 + c4 + 2] = kv.z;
        sK[r * 65 + c4 + 3] = kv.w;
      }
    }
    __syncthreads();
    if (lane < nk) {
      // DotF32 (ops_simd.go:85-97): sum += a0 b0 + a1 b1 + a2 b2 + a3 b3, left to right
      const float* kr = sK + lane * 65;
      float sum = 0.0f;
#pragma unroll
      for (int d = 0; d < 64; d += 4)
        sum += qv[d] * kr[d] + qv[d + 1] * kr[d + 1] + qv[d + 2] * kr[d + 2] + qv[d + 3] * kr[d + 3];
      float sc = sum * scale;
      if (mrow[k0 + lane] == 0) sc = -1e9f;
      sS[k0 + lane] = sc;
    }
    __syncthreads();
  }
  // SoftmaxInPlace (ops_simd.go:46-66): max, e = x < -10 ? 0 : float32(exp(float64(x))), sum in
  // key order, times 1/sum
  float mx = -INFINITY;
  for (int i = lane; i < ls; i += 64) mx = fmaxf(mx, sS[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  for (int i = lane; i < ls; i += 64) {
    const float x = sS[i] - mx;
    sS[i] = x < -10.0f ? 0.0f : (float)exp((double)x);
  }
  __syncthreads();
  float sum = 0.0f;
  if (lane == 0)
    for (int i = 0; i < ls; i++) sum += sS[i];
  sum = __shfl(sum, 0);
  const float inv = 1.0f / sum;
  for (int i = lane; i < ls; i += 64) sS[i] = sS[i] * inv;
  __syncthreads();
  // out[dd] = sum_v p_v V[v][dd] in key order; lane = dd
  float o = 0.0f;
  const float* vcol = a.v + (size_t)s.row0 * D + h * HD + lane;
  for (int i = 0; i < ls; i++) o += sS[i] * vcol[(size_t)i * D];
  a.att[(size_t)t * D + h * HD + lane] = o;
}

// MeanPool + L2Normalize (+ Matryoshka renormalisation); one block per sequence.
__global__ __launch_bounds__(256) void exact_pool_kernel(ExactArgs a, int B, int out_dim, float* out) {
  __shared__ float sP[1024];
  __shared__ float sInv[2];
  const int b = blockIdx.x, tid = threadIdx.x, D = a.D;
  const int row0 = a.seq_off ? a.seq_off[b] : b * a.L;
  const int ls = a.seq_off ? a.seq_off[b + 1] - row0 : a.L;
  const int32_t* mrow = a.mask + (size_t)b * a.L;
  float count = 0.0f;
  for (int p = 0; p < ls; p++)
    if (mrow[p] == 1) count++;
  for (int j = tid; j < D; j += 256) {
    float acc = 0.0f;
    for (int p = 0; p < ls; p++)
      if (mrow[p] == 1) acc += a.h[(size_t)(row0 + p) * D + j];
    if (count != 0.0f) {
      const float inv = 1.0f / count;
      acc = acc * inv;
    }
    sP[j] = acc;
  }
  __syncthreads();
  const int od = out_dim < D ? out_dim : D;
  if (tid == 0) {
    double n1 = 0.0;
    for (int j = 0; j < D; j++) n1 += (double)sP[j] * (double)sP[j];
    n1 = sqrt(n1);
    sInv[0] = n1 == 0.0 ? 1.0f : (float)(1.0 / n1);
    sInv[1] = n1 == 0.0 ? 0.0f : 1.0f;  // 1: multiply, 0: copy (zero vector)
  }
  __syncthreads();
  for (int j = tid; j < D; j += 256)
    if (sInv[1] != 0.0f) sP[j] = sP[j] * sInv[0];
  __syncthreads();
  if (od < D) {
    if (tid == 0) {
      double n2 = 0.0;
      for (int j = 0; j < od; j++) n2 += (double)sP[j] * (double)sP[j];
      n2 = sqrt(n2);
      sInv[0] = n2 == 0.0 ? 1.0f : (float)(1.0 / n2);
      sInv[1] = n2 == 0.0 ? 0.0f : 1.0f;
    }
    __syncthreads();
    for (int j = tid; j < od; j += 256) out[(size_t)b * od + j] = sInv[1] != 0.0f ? sP[j] * sInv[0] : sP[j];
  } else {
    for (int j = tid; j < D; j += 256) out[(size_t)b * od + j] = sP[j];
  }
}

hipError_t launch_exact_embed(const ExactArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(exact_embed_kernel, dim3((a.T + 63) / 64), dim3(64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_exact_ln(const ExactArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(exact_ln_kernel, dim3((a.T + 63) / 64), dim3(64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_exact_gemm(const ExactArgs& a, const ExactGemm& g, int epi, hipStream_t st) {
  if (g.N % XG_N != 0 || g.K % 4 != 0 || a.D > 1024) return hipErrorInvalidValue;
  const dim3 grid(g.N / XG_N, (a.T + XG_T - 1) / XG_T), blk(256);
  switch (epi) {
    case EPI_F32: hipLaunchKernelGGL((exact_gemm_kernel<EPI_F32>), grid, blk, 0, st, a, g); break;
    case EPI_RESID: hipLaunchKernelGGL((exact_gemm_kernel<EPI_RESID>), grid, blk, 0, st, a, g); break;
    case EPI_QKV: hipLaunchKernelGGL((exact_gemm_kernel<EPI_QKV>), grid, blk, 0, st, a, g); break;
    case EPI_GEGLU: hipLaunchKernelGGL((exact_gemm_kernel<EPI_GEGLU>), grid, blk, 0, st, a, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_exact_attention(const ExactArgs& a, hipStream_t st) {
  const size_t lds = ((size_t)((a.L + 3) & ~3) + 64 * 65) * 4;
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(exact_attention_kernel, dim3(a.T, a.H), dim3(64), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_exact_pool(const ExactArgs& a, int B, int out_dim, float* out, hipStream_t st) {
  if (a.D > 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(exact_pool_kernel, dim3(B), dim3(256), 0, st, a, B, out_dim, out);
  return hipGetLastError();
}

}  // namespace lle
