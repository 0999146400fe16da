// Row kernels: embedding gather + LayerNorm, LayerNorm, masked mean-pool + L2 (+ Matryoshka),
// f32 <-> f16 helpers and the raw-GGUF dequantisation test kernel.
#include "rowops_device.h"

namespace lle {

template <int TY>
__global__ __launch_bounds__(256) void embed_ln_kernel(EmbedArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[EMBED_LDS];
  embed_ln_dev<TY>(a, blockIdx.x, lds);
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

// ln_kernel with the f32 rows left unnormalised: writes the f16 rows and each row's mean and
// invStd (stats[t] = {mean, inv}); the next residual consumer applies the elementwise step
// itself (ln_elem) and gets ln_kernel's f32 bits.
__global__ __launch_bounds__(256) void ln_stats_kernel(const float* h, __half* h16, float2* stats, const float* w,
                                                       const float* b, float eps, int T, int D) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int ne = D / 64;
  const float* row = h + (size_t)t * D;
  float wv[MAXE], bv[MAXE], x[MAXE];
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) {
      wv[i] = w[lane + 64 * i];
      bv[i] = b[lane + 64 * i];
    }
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) x[i] = row[lane + 64 * i];
  float mean, inv;
  ln_mean_inv(x, ne, D, eps, mean, inv);
  __half* h16row = h16 + (size_t)t * D;
#pragma unroll
  for (int i = 0; i < MAXE; i++)
    if (i < ne) h16row[lane + 64 * i] = __float2half_rn(ln_elem(x[i], mean, inv, wv[i], bv[i]));
  if (lane == 0) stats[t] = make_float2(mean, inv);
}

hipError_t launch_ln_stats(const float* h, __half* h16, float2* stats, const float* w, const float* b, float eps,
                           int T, int D, hipStream_t st) {
  hipLaunchKernelGGL(ln_stats_kernel, dim3((T + 3) / 4), dim3(256), 0, st, h, h16, stats, w, b, eps, T, D);
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

template <int NCH>
__global__ __launch_bounds__(256) void reduce_ln_pool_kernel(const float* __restrict__ part, int M, const float* src,
                                                             const float* w, const float* bb, float eps,
                                                             const int32_t* __restrict__ mask,
                                                             const int32_t* __restrict__ seq_off, int L, int D,
                                                             int out_dim, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[RLP_LDS];
  reduce_ln_pool_dev<NCH>(part, M, src, w, bb, eps, mask, seq_off, L, D, out_dim, out, blockIdx.x, lds);
}

hipError_t launch_reduce_ln_pool(const float* part, int nch, int M, const float* src, const float* w, const float* b,
                                 float eps, const int32_t* mask, const int32_t* seq_off, int B, int L, int D,
                                 int out_dim, float* out, hipStream_t st) {
  if (L > POOL_MAXL || D > 1024 || D % 64 || (nch != 4 && nch != 0)) return hipErrorInvalidValue;
  if (nch == 4)
    hipLaunchKernelGGL(reduce_ln_pool_kernel<4>, dim3(B), dim3(256), 0, st, part, M, src, w, b, eps, mask, seq_off, L,
                       D, out_dim, out);
  else  // no partials: the rows of src are LayerNormed as they are (ln_kernel's input)
    hipLaunchKernelGGL(reduce_ln_pool_kernel<0>, dim3(B), dim3(256), 0, st, part, M, src, w, b, eps, mask, seq_off, L,
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

// Mean-pool of few long sequences: one block per (sequence, 64-column slice), so a sequence's
// rows are read by D / 64 CUs instead of one. Each column is summed over the kept rows in row
// order in f32 and scaled by 1 / count, exactly as pool_kernel does it, so the bits are the same.
// The 4 waves bring 64-row chunks into a 6-buffer LDS ring by LDS-DMA five chunks ahead (one
// 1 KB instruction = 4 rows x 256 bytes, gathered through the kept-row list); wave 0 adds them
// (lane = column). The scaled slice goes to vals[b][D]; pool_norm_kernel finishes each row.
typedef __attribute__((address_space(3))) void* pool_lds_t;
typedef unsigned int pool_rsrc_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void pool_dma16(pool_rsrc_t r, void* lds, int voff) {
  const uint32_t base = (uint32_t)(uintptr_t)(pool_lds_t)lds;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(base), "v"(voff), "s"(r)
               : "memory", "m0");
}
constexpr int PSL_CH = 64, PSL_NB = 6;  // rows per chunk, LDS buffers
__global__ __launch_bounds__(256) void pool_slice_kernel(const float* __restrict__ h, const int32_t* __restrict__ mask,
                                                         const int32_t* __restrict__ seq_off, int L, int D,
                                                         float* __restrict__ vals) {
  __shared__ int rows[POOL_MAXL];
  __shared__ int wcount[5];
  __shared__ __attribute__((aligned(1024))) float buf[PSL_NB][PSL_CH][64];
  const int b = blockIdx.x, col = blockIdx.y * 64, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int count = pool_compact(mask, b, L, rows, wcount);
  const float* hb = h + (size_t)(seq_off ? seq_off[b] : b * L) * D + col;
  const uint64_t a = (uint64_t)(uintptr_t)hb;
  const pool_rsrc_t rs = pool_rsrc_t{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, 0xffffffffu, 0x00020000u};
  const int nch = (count + PSL_CH - 1) / PSL_CH;
  // chunk c, instruction k of wave w: chunk rows w * 16 + 4 k + lane / 16, 16 bytes (lane % 16);
  // rows past the last kept one re-read it (never added)
  auto issue = [&](int c) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = min(c * PSL_CH + wave * 16 + 4 * k + (lane >> 4), count - 1);
      pool_dma16(rs, &buf[c % PSL_NB][wave * 16 + 4 * k][0], (rows[i] * D + (lane & 15) * 4) * 4);
    }
  };
  for (int c = 0; c < PSL_NB - 1 && c < nch; c++) issue(c);
  float s = 0.f;
  for (int c = 0; c < nch; c++) {
    // this wave's loads of chunk c have landed once only those of the (up to PSL_NB - 2)
    // younger chunks issued so far are in flight (4 instructions each)
    switch (min(nch - 1 - c, PSL_NB - 2)) {
      case 4: __builtin_amdgcn_s_waitcnt(16 & 0xF | (16 >> 4) << 14 | 0x7 << 4); break;  // vmcnt(16) lgkmcnt(0)
      case 3: __builtin_amdgcn_s_waitcnt(12 | 0x7 << 4); break;
      case 2: __builtin_amdgcn_s_waitcnt(8 | 0x7 << 4); break;
      case 1: __builtin_amdgcn_s_waitcnt(4 | 0x7 << 4); break;
      default: __builtin_amdgcn_s_waitcnt(0x7 << 4); break;
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (c + PSL_NB - 1 < nch) issue(c + PSL_NB - 1);  // into chunk c - 1's buffer, read before the barrier
    if (wave == 0) {
      const int n = min(PSL_CH, count - c * PSL_CH);
      const float* bc = &buf[c % PSL_NB][0][lane];
      int r = 0;
      for (; r + 16 <= n; r += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = bc[(r + u) * 64];
#pragma unroll
        for (int u = 0; u < 16; u++) s += v[u];
      }
      for (; r < n; r++) s += bc[r * 64];
    }
  }
  if (wave == 0) {
    if (count != 0) s *= 1.0f / (float)count;
    vals[(size_t)b * D + col + lane] = s;
  }
}

__global__ __launch_bounds__(256) void pool_norm_kernel(const float* __restrict__ vals, int D, int out_dim,
                                                        float* __restrict__ out) {
  __shared__ double red[256];
  __shared__ __align__(16) float v[1024];
  const int b = blockIdx.x;
  for (int j = threadIdx.x; j < D; j += 256) v[j] = vals[(size_t)b * D + j];
  __syncthreads();
  pool_finish(v, red, D, out_dim, out + (size_t)b * (out_dim < D ? out_dim : D));
}

hipError_t launch_pool(const float* h, const int32_t* mask, const int32_t* seq_off, int B, int L, int D, int out_dim,
                       float* out, float* scratch, size_t scratch_bytes, hipStream_t st) {
  if (L > POOL_MAXL || D > 1024 || D % 4) return hipErrorInvalidValue;
  // The sliced form when one block per sequence would leave most CUs idle on long rows
  // (config 5: 8 sequences of 1024-2048 rows, 84 us in pool_kernel).
  if (B <= 64 && L >= 512 && D % 64 == 0 && scratch && scratch_bytes >= (size_t)B * D * 4) {
    hipLaunchKernelGGL(pool_slice_kernel, dim3(B, D / 64), dim3(256), 0, st, h, mask, seq_off, L, D, scratch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(pool_norm_kernel, dim3(B), dim3(256), 0, st, scratch, D, out_dim, out);
    return hipGetLastError();
  }
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
