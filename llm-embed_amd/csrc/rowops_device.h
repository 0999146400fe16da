// Row stages as device functions: the embedding gather + LayerNorm, the pool helpers and the
// fused last LayerNorm + mean pool of small forwards, run by the row kernels (rowops.hip).
#pragma once

#include "deq_device.h"
#include "lle_internal.h"
#include "mfma_common.h"
#include "row_device.h"

namespace lle {

// Embedding stage (internal/embed/bert.go:220-249, getEmbedding :290-316):
// h = deq(token_embd[id]) + deq(token_types[0]), then LayerNorm(token_embd_norm).
// One wave per token. The wave first issues the loads that do not depend on the token id (the
// type row and the LayerNorm weights), then copies the token's GGUF row into LDS with whole
// 16-byte (or 2-byte, for rows of odd 8-byte length) loads, and dequantises from there: the
// per-element scale and code loads of a raw row would otherwise be a dependent global round
// trip each.
constexpr int EMBED_RB = 4 * 64 * MAXE;  // bytes of the widest row on the path (F32 at the largest d_model)
constexpr size_t EMBED_LDS = 4 * EMBED_RB;
// Block bx of the embedding stage (tokens 4 bx .. 4 bx + 3, one per wave), its LDS at `lds`
// (EMBED_LDS bytes, 16-byte aligned).
template <int TY>
__device__ __forceinline__ void embed_ln_dev(const EmbedArgs& a, int bx, unsigned char* lds) {
  uint8_t(*srow)[EMBED_RB] = reinterpret_cast<uint8_t(*)[EMBED_RB]>(lds);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int t = bx * 4 + wv;
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

// MeanPool + L2Normalize (+ Matryoshka truncation and renormalisation):
// internal/embed/pool.go:8-54, internal/embed/embedder.go:50-68. Rows with mask == 1 are
// summed in row order in f32 (the reference's order), scaled by float32(1/count); the norm
// is accumulated in f64. One block per sequence: the kept rows are first compacted (in order)
// into an LDS list, then each thread sums 4 adjacent columns with 16 row loads in flight.
constexpr int POOL_MAXL = 8192;

// Ordered compaction of sequence b's kept positions (mask == 1) into rows[]: per-wave ballot +
// prefix over the 4 waves of a 256-thread block. Returns their count.
__device__ __forceinline__ int pool_compact(const int32_t* __restrict__ mask, int b, int L, int* rows, int* wcount) {
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
__device__ __forceinline__ void pool_finish(float* vals, double* red, int D, int out_dim, float* __restrict__ out) {
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

// The last LayerNorm of a small forward fused with MeanPool + L2Normalize, one block per
// sequence. Its kept rows are normalised 16 at a time into LDS with reduce_resid_ln_kernel's
// arithmetic (residual + (0 + chunk partials in order), ln_row's LayerNorm), and added in row
// order as pool_kernel adds them; the scaling, norm and Matryoshka tail are pool_kernel's. So
// the output equals reduce_resid_ln_kernel followed by pool_kernel bit for bit, without the
// LayerNorm rows going through global memory.
constexpr int RLP_ROWS = 16;
// LDS of one reduce_ln_pool block: red double[256], vals float[1024], rows int[POOL_MAXL],
// wcount int[5] (padded to 32 bytes), lnrow float[RLP_ROWS][1024].
constexpr size_t RLP_RED = 0, RLP_VALS = RLP_RED + 256 * 8, RLP_ROWSOFF = RLP_VALS + 1024 * 4,
                 RLP_WCOUNT = RLP_ROWSOFF + POOL_MAXL * 4, RLP_LNROW = RLP_WCOUNT + 32,
                 RLP_LDS = RLP_LNROW + RLP_ROWS * 1024 * 4;
// Block b (sequence b) of the fused last LayerNorm + pool, its LDS at `lds` (RLP_LDS bytes).
template <int NCH>
__device__ __forceinline__ void reduce_ln_pool_dev(const float* __restrict__ part, int M, const float* src,
                                                   const float* w, const float* bb, float eps,
                                                   const int32_t* __restrict__ mask,
                                                   const int32_t* __restrict__ seq_off, int L, int D, int out_dim,
                                                   float* __restrict__ out, int b, unsigned char* lds) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  double* red = reinterpret_cast<double*>(lds + RLP_RED);
  float* vals = reinterpret_cast<float*>(lds + RLP_VALS);
  int* rows = reinterpret_cast<int*>(lds + RLP_ROWSOFF);
  int* wcount = reinterpret_cast<int*>(lds + RLP_WCOUNT);
  float(*lnrow)[1024] = reinterpret_cast<float(*)[1024]>(lds + RLP_LNROW);
  const int count = pool_compact(mask, b, L, rows, wcount);
  const int row0 = seq_off ? seq_off[b] : b * L;
  const int ne = D / 64, c0 = 4 * tid;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (D == 768) {
    // Two rows per wave at a time with 16-byte loads (rows 4 elements per lane, the partials
    // summed element-wise in the same order), staged in lnrow and read back in ln_row's element
    // mapping for the LayerNorm: 30 loads per lane in flight at once instead of 60 per row, which
    // went past the 63 a wave can have. Same arithmetic, same bits.
    float wv_[MAXE], bv_[MAXE];
#pragma unroll
    for (int i = 0; i < MAXE; i++)
      if (i < ne) {
        wv_[i] = w[lane + 64 * i];
        bv_[i] = bb[lane + 64 * i];
      }
    constexpr int G = 3, NEC = 12;  // D = 768
    for (int i0 = 0; i0 < count; i0 += RLP_ROWS) {
      for (int k0 = wv; k0 < RLP_ROWS; k0 += 8) {  // wave wv: rows k0 and k0 + 4, then + 8
        floatx4 xs[2][G], pv[2][G][NCH > 0 ? NCH : 1];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int k = k0 + 4 * h;
          const int t = row0 + rows[i0 + min(k, count - i0 - 1)];  // past the last row: re-read it
#pragma unroll
          for (int g = 0; g < G; g++) {
              const int j = g * 256 + lane * 4;
              xs[h][g] = *(const floatx4*)(src + (size_t)t * D + j);
#pragma unroll
              for (int c = 0; c < NCH; c++) pv[h][g][c] = *(const floatx4*)(part + ((size_t)c * M + t) * D + j);
            }
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int k = k0 + 4 * h;
#pragma unroll
          for (int g = 0; g < G; g++) {
              floatx4 x = xs[h][g];
              if constexpr (NCH > 0) {
                floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < NCH; c++) acc += pv[h][g][c];
                x.x = x.x + acc.x; x.y = x.y + acc.y; x.z = x.z + acc.z; x.w = x.w + acc.w;
              }
              *(floatx4*)&lnrow[k][g * 256 + lane * 4] = x;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int k = k0 + 4 * h;
          if (i0 + k < count) {
            float x[MAXE];
#pragma unroll
            for (int i = 0; i < NEC; i++) x[i] = lnrow[k][lane + 64 * i];
            ln_apply_wb(x, NEC, D, wv_, bv_, eps);
#pragma unroll
            for (int i = 0; i < NEC; i++) lnrow[k][lane + 64 * i] = x[i];
          }
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
  } else {
  for (int i0 = 0; i0 < count; i0 += RLP_ROWS) {
    for (int k = wv; k < RLP_ROWS; k += 4) {  // wave wv: rows i0 + wv, + 4, + 8, + 12
      if (i0 + k < count) {
        const int t = row0 + rows[i0 + k];
        const float* srow = src + (size_t)t * D;
        float pv[MAXE][NCH > 0 ? NCH : 1], x[MAXE];
#pragma unroll
        for (int i = 0; i < MAXE; i++)
          if (i < ne) {
            const int j = lane + 64 * i;
            x[i] = srow[j];
#pragma unroll
            for (int c = 0; c < NCH; c++) pv[i][c] = part[((size_t)c * M + t) * D + j];
          }
        if constexpr (NCH > 0) {
#pragma unroll
          for (int i = 0; i < MAXE; i++)
            if (i < ne) {
              float acc = 0.f;
#pragma unroll
              for (int c = 0; c < NCH; c++) acc += pv[i][c];
              x[i] = x[i] + acc;
            }
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

}  // namespace lle
