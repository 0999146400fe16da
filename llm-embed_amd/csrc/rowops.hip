// Row kernels: embedding gather + LayerNorm, LayerNorm, masked mean-pool + L2 (+ Matryoshka),
// f32 <-> f16 helpers and the raw-GGUF dequantisation test kernel.
#include "deq_device.h"
#include "lle_internal.h"
#include "row_device.h"

namespace lle {

// Embedding stage (internal/embed/bert.go:220-249, getEmbedding :290-316):
// h = deq(token_embd[id]) + deq(token_types[0]), then LayerNorm(token_embd_norm).
// One wave per token. The wave first issues the loads that do not depend on the token id (the
// type row and the LayerNorm weights), then copies the token's GGUF row into LDS with whole
// 16-byte (or 2-byte, for rows of odd 8-byte length) loads, and dequantises from there: the
// per-element scale and code loads of a raw row would otherwise be a dependent global round
// trip each.
template <int TY>
__global__ __launch_bounds__(256) void embed_ln_kernel(EmbedArgs a) {
  constexpr int RB = 4 * 64 * MAXE;  // bytes of the widest row on the path (F32 at the largest d_model)
  __shared__ __attribute__((aligned(16))) uint8_t srow[4][RB];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wv;
  if (t >= a.T) return;  // wave-uniform; the LDS row below is this wave's alone
  const int ne = a.D / 64;
  float ty[MAXE], lw[MAXE], lb[MAXE];
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      const int j = lane + 64 * i;
      ty[i] = a.type0[j];
      lw[i] = a.w[j];
      lb[i] = a.b[j];
    }
  int id = a.ids[t];
  if (id < 0 || id >= a.vocab) {
    if (lane == 0) atomicOr(a.status, 1);
    id = 0;
  }
  const uint8_t* row = a.tok + (size_t)id * a.tok_row_bytes;
  const int nb = (int)a.tok_row_bytes;
  if ((nb & 15) == 0 && (((uintptr_t)row) & 15) == 0) {
    for (int o = lane * 16; o < nb; o += 64 * 16) *(uint4*)&srow[wv][o] = *(const uint4*)(row + o);
  } else {
    for (int o = lane * 2; o < nb; o += 64 * 2) *(uint16_t*)&srow[wv][o] = *(const uint16_t*)(row + o);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float x[MAXE];
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) x[i] = deq_raw_t<TY>(srow[wv], lane + 64 * i) + ty[i];
  ln_apply_wb(x, ne, a.D, lw, lb, a.eps);
  float* hrow = a.h + (size_t)t * a.D;
  __half* h16row = a.h16 + (size_t)t * a.D;
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      const int j = lane + 64 * i;
      hrow[j] = x[i];
      h16row[j] = __float2half_rn(x[i]);
    }
}

hipError_t launch_embed_ln(const EmbedArgs& a, hipStream_t st) {
  if (a.tok_row_bytes > 4 * 64 * MAXE || a.tok_row_bytes % 2 || a.D > 64 * MAXE) return hipErrorInvalidValue;
  const dim3 g((a.T + 3) / 4), blk(256);
  switch (a.tok_type) {  // one instantiation per format keeps every row load in one basic block
    case 0: hipLaunchKernelGGL(embed_ln_kernel<0>, g, blk, 0, st, a); break;
    case 8: hipLaunchKernelGGL(embed_ln_kernel<8>, g, blk, 0, st, a); break;
    case 12: hipLaunchKernelGGL(embed_ln_kernel<12>, g, blk, 0, st, a); break;
    case 13: hipLaunchKernelGGL(embed_ln_kernel<13>, g, blk, 0, st, a); break;
    case 14: hipLaunchKernelGGL(embed_ln_kernel<14>, g, blk, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
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

// Ordered split-K reduction + residual add + LayerNorm for one row per wave (M <= 64 path);
// chunk counts: 768-wide chunks of K = 3072 (4) and the other d_ff / d_model ratios listed below.
// t = 0 + part[0] + part[1] + ... (gemm_reduce's order), h = h + t (the residual epilogue's add),
// then the LayerNorm of ln_kernel with the same element-to-lane mapping and reduction tree.
template <int NCH>
__global__ __launch_bounds__(256) void reduce_resid_ln_kernel(const float* __restrict__ part, int M, int N,
                                                              const float* src, float* h, __half* h16, const float* w,
                                                              const float* b, float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= M) return;
  const int ne = N / 64;
  float* row = h + (size_t)t * N;
  const float* srow = src + (size_t)t * N;  // the residual (== row when updating in place)
  // every load is issued before the first add (one memory round trip); adds in chunk order
  float pv[MAXE][NCH], x[MAXE];
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      const int j = lane + 64 * i;
      x[i] = srow[j];
#pragma unroll
      for (int c = 0; c < NCH; c++) pv[i][c] = part[((size_t)c * M + t) * N + j];
    }
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; c++) acc += pv[i][c];
      x[i] = x[i] + acc;
    }
  ln_row(x, ne, N, w, b, eps, lane, row, h16 + (size_t)t * N);
}

hipError_t launch_reduce_resid_ln(const float* part, int nch, int M, int N, const float* src, float* h, __half* h16,
                                  const float* w, const float* b, float eps, hipStream_t st) {
  const dim3 g((M + 3) / 4), blk(256);
  switch (nch) {
    case 2: hipLaunchKernelGGL(reduce_resid_ln_kernel<2>, g, blk, 0, st, part, M, N, src, h, h16, w, b, eps); break;
    case 3: hipLaunchKernelGGL(reduce_resid_ln_kernel<3>, g, blk, 0, st, part, M, N, src, h, h16, w, b, eps); break;
    case 4: hipLaunchKernelGGL(reduce_resid_ln_kernel<4>, g, blk, 0, st, part, M, N, src, h, h16, w, b, eps); break;
    case 8: hipLaunchKernelGGL(reduce_resid_ln_kernel<8>, g, blk, 0, st, part, M, N, src, h, h16, w, b, eps); break;
    case 12: hipLaunchKernelGGL(reduce_resid_ln_kernel<12>, g, blk, 0, st, part, M, N, src, h, h16, w, b, eps); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// MeanPool + L2Normalize (+ Matryoshka truncation and renormalisation):
// internal/embed/pool.go:8-54, internal/embed/embedder.go:50-68. Rows with mask == 1 are
// summed in row order in f32 (the reference's order), scaled by float32(1/count); the norm
// is accumulated in f64. One block per sequence: the kept rows are first compacted (in order)
// into an LDS list, then each thread sums 4 adjacent columns with 16 row loads in flight.
constexpr int POOL_MAXL = 8192;

// Ordered compaction of sequence b's kept positions (mask == 1) into rows[]: per-wave ballot +
// prefix over the 4 waves of a 256-thread block. Returns their count.
__device__ int pool_compact(const int32_t* __restrict__ mask, int b, int L, int* rows, int* wcount) {
  const int tid = threadIdx.x;
  int base = 0;
  for (int i0 = 0; i0 < L; i0 += 256) {
    const int i = i0 + tid;
    const bool keep = i < L && mask[(size_t)b * L + i] == 1;
    const unsigned long long bal = __ballot(keep);
    const int lane = tid & 63, wv = tid >> 6;
    if (lane == 0) wcount[wv] = __popcll(bal);
    __syncthreads();
    int off = base;
    for (int w2 = 0; w2 < wv; w2++) off += wcount[w2];
    if (keep) rows[off + __popcll(bal & ((1ull << lane) - 1ull))] = i;
    base += wcount[0] + wcount[1] + wcount[2] + wcount[3];
    __syncthreads();
  }
  return base;
}

// L2Normalize of the pooled row vals[0..D) over the first n values, twice when truncating
// (embedder.go:65-68), then min(out_dim, D) values to out.
__device__ void pool_finish(float* vals, double* red, int D, int out_dim, float* __restrict__ out) {
  const int tid = threadIdx.x;
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
  for (int j = tid; j < od; j += 256) out[j] = vals[j];
}

__global__ __launch_bounds__(256) void pool_kernel(const float* __restrict__ h, const int32_t* __restrict__ mask,
                                                   const int32_t* __restrict__ seq_off, int L, int D, int out_dim,
                                                   float* __restrict__ out) {
  const int b = blockIdx.x, tid = threadIdx.x;
  __shared__ double red[256];
  __shared__ __align__(16) float vals[1024];
  __shared__ int rows[POOL_MAXL];
  __shared__ int wcount[5];
  const int count = pool_compact(mask, b, L, rows, wcount);
  // packed rows: sequence b starts at row seq_off[b] and its kept positions all lie before
  // seq_off[b + 1] - seq_off[b] (positions past its last valid token were dropped)
  const float* hb = h + (size_t)(seq_off ? seq_off[b] : b * L) * D;
  const int c0 = 4 * tid;
  if (c0 < D) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    int i = 0;
    for (; i + 16 <= count; i += 16) {
      float4 v[16];
#pragma unroll
      for (int u = 0; u < 16; u++) v[u] = *(const float4*)(hb + (size_t)rows[i + u] * D + c0);
#pragma unroll
      for (int u = 0; u < 16; u++) {
        s.x += v[u].x;
        s.y += v[u].y;
        s.z += v[u].z;
        s.w += v[u].w;
      }
    }
    for (; i < count; i++) {
      const float4 v = *(const float4*)(hb + (size_t)rows[i] * D + c0);
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
    if (count != 0) {
      const float inv = 1.0f / (float)count;
      s.x *= inv;
      s.y *= inv;
      s.z *= inv;
      s.w *= inv;
    }
    *(float4*)(vals + c0) = s;
  }
  __syncthreads();
  pool_finish(vals, red, D, out_dim, out + (size_t)b * (out_dim < D ? out_dim : D));
}

// The last LayerNorm of a small forward fused with MeanPool + L2Normalize, one block per
// sequence. Its kept rows are normalised 16 at a time into LDS with reduce_resid_ln_kernel's
// arithmetic (residual + (0 + chunk partials in order), ln_row's LayerNorm), and added in row
// order as pool_kernel adds them; the scaling, norm and Matryoshka tail are pool_kernel's. So
// the output equals reduce_resid_ln_kernel followed by pool_kernel bit for bit, without the
// LayerNorm rows going through global memory.
constexpr int RLP_ROWS = 16;
template <int NCH>
__global__ __launch_bounds__(256) void reduce_ln_pool_kernel(const float* __restrict__ part, int M, const float* src,
                                                             const float* w, const float* bb, float eps,
                                                             const int32_t* __restrict__ mask,
                                                             const int32_t* __restrict__ seq_off, int L, int D,
                                                             int out_dim, float* __restrict__ out) {
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  __shared__ double red[256];
  __shared__ __align__(16) float vals[1024];
  __shared__ int rows[POOL_MAXL];
  __shared__ int wcount[5];
  __shared__ __align__(16) float lnrow[RLP_ROWS][1024];
  const int count = pool_compact(mask, b, L, rows, wcount);
  const int row0 = seq_off ? seq_off[b] : b * L;
  const int ne = D / 64, c0 = 4 * tid;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int i0 = 0; i0 < count; i0 += RLP_ROWS) {
    for (int k = wv; k < RLP_ROWS; k += 4) {  // wave wv: rows i0 + wv, + 4, + 8, + 12
      if (i0 + k < count) {
        const int t = row0 + rows[i0 + k];
        const float* srow = src + (size_t)t * D;
        float pv[MAXE][NCH], x[MAXE];
#pragma unroll
        for (int i = 0; i < MAXE; i++)
          if (i < ne) {
            const int j = lane + 64 * i;
            x[i] = srow[j];
#pragma unroll
            for (int c = 0; c < NCH; c++) pv[i][c] = part[((size_t)c * M + t) * D + j];
          }
#pragma unroll
        for (int i = 0; i < MAXE; i++)
          if (i < ne) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < NCH; c++) acc += pv[i][c];
            x[i] = x[i] + acc;
          }
        ln_apply(x, ne, D, w, bb, eps, lane);
#pragma unroll
        for (int i = 0; i < MAXE; i++)
          if (i < ne) lnrow[k][lane + 64 * i] = x[i];
      }
    }
    __syncthreads();
    if (c0 < D) {
      const int nr = count - i0 < RLP_ROWS ? count - i0 : RLP_ROWS;
      for (int u = 0; u < nr; u++) {
        const float4 v = *(const float4*)&lnrow[u][c0];
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
      }
    }
    __syncthreads();
  }
  if (c0 < D) {
    if (count != 0) {
      const float inv = 1.0f / (float)count;
      s.x *= inv;
      s.y *= inv;
      s.z *= inv;
      s.w *= inv;
    }
    *(float4*)(vals + c0) = s;
  }
  __syncthreads();
  pool_finish(vals, red, D, out_dim, out + (size_t)b * (out_dim < D ? out_dim : D));
}

hipError_t launch_reduce_ln_pool(const float* part, int nch, int M, const float* src, const float* w, const float* b,
                                 float eps, const int32_t* mask, const int32_t* seq_off, int B, int L, int D,
                                 int out_dim, float* out, hipStream_t st) {
  if (L > POOL_MAXL || D > 1024 || D % 64 || nch != 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(reduce_ln_pool_kernel<4>, dim3(B), dim3(256), 0, st, part, M, src, w, b, eps, mask, seq_off, L,
                     D, out_dim, out);
  return hipGetLastError();
}

// Tables of a packed batch given as B sequences back to back (T tokens, offsets in[0..B]).
// The offsets are first made safe to index with (one thread: B is small): nondecreasing, within
// [0, T], no sequence longer than L; any change sets status bit 2 and the results of that call
// are not meaningful, but every later access stays inside the buffers.
__global__ void pack_offsets_kernel(const int32_t* __restrict__ in, int B, int T, int L, int32_t* __restrict__ off,
                                    int32_t* status) {
  if (threadIdx.x != 0) return;
  bool bad = in[0] != 0;
  int prev = 0;
  off[0] = 0;
  for (int b = 0; b < B; b++) {
    const int e = in[b + 1];
    const int c = min(max(e, prev), min(T, prev + L));
    bad |= c != e;
    off[b + 1] = c;
    prev = c;
  }
  if (bad || prev != T) atomicOr(status, 2);
}

// tokrow[t] = b * L + position of row t; mask[b][p] = p < length of sequence b. Block B gives
// rows that no sequence covers (only after a bad offset table) an in-range placeholder.
__global__ void pack_tables_kernel(const int32_t* __restrict__ off, int B, int T, int L, int32_t* __restrict__ tokrow,
                                   int32_t* __restrict__ mask) {
  const int b = blockIdx.x;
  if (b == B) {
    for (int t = off[B] + (int)threadIdx.x; t < T; t += blockDim.x) tokrow[t] = 0;
    return;
  }
  const int o = off[b], n = off[b + 1] - o;
  for (int p = threadIdx.x; p < L; p += blockDim.x) {
    mask[(size_t)b * L + p] = p < n ? 1 : 0;
    if (p < n) tokrow[o + p] = b * L + p;
  }
}

hipError_t launch_pack_tables(const int32_t* in_off, int B, int T, int L, int32_t* off, int32_t* tokrow,
                              int32_t* mask, int32_t* status, hipStream_t st) {
  hipLaunchKernelGGL(pack_offsets_kernel, dim3(1), dim3(64), 0, st, in_off, B, T, L, off, status);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(pack_tables_kernel, dim3(B + 1), dim3(256), 0, st, off, B, T, L, tokrow, mask);
  return hipGetLastError();
}

hipError_t launch_pool(const float* h, const int32_t* mask, const int32_t* seq_off, int B, int L, int D, int out_dim,
                       float* out, hipStream_t st) {
  if (L > POOL_MAXL || D > 1024 || D % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pool_kernel, dim3(B), dim3(256), 0, st, h, mask, seq_off, L, D, out_dim, out);
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
