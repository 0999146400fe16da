// Quantised projection GEMMs for gfx950: Y[M][N] = X[M][K] . W^T with W quantised in HBM.
//
// Replaces gemmOrBatch -> GemmPrePacked32 (internal/embed/bert.go:579-638,
// internal/ggml/gemm_avx512.go:67-147) and the fused dequant-dot kernels
// (internal/ggml/dot_amd64.s) with MFMA dequant-GEMMs:
//   * W stays quantised in HBM (re-laid-out GGUF planes); each 16-element segment is
//     decoded with the reference arithmetic (deq_device.h), rounded once to f16 and staged
//     in LDS; X arrives as f16. v_mfma_f32_16x16x32_f16 accumulates in f32.
//   * Canonical reduction order, identical in every kernel variant so that a row's result
//     never depends on M, the tile it lands in or the batch it belongs to (the reference's
//     EmbedBatch == Embed contract, internal/embed/embedder_test.go:139-144):
//       K is cut into chunks (768 wide when K % 768 == 0, else 256); inside a chunk one MFMA
//       chain starting from 0 walks 64-wide steps (two 32-wide MFMAs each) in increasing k;
//       the chunk results are added into a running f32 total that starts at 0, in order.
//   * MFMA operand roles: A = W rows (features), B = X rows (tokens), so D[feature][token];
//     lane l holds features 4*(l/16)+r (r = 0..3) of token l%16.
//   * Epilogues: plain f32 store, residual add, QKV split + RoPE + head-major f16 scatter,
//     and GeLU(gate) * up on the row-interleaved up||gate matrix.
#include "deq_device.h"
#include "lle_internal.h"

namespace lle {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int KSTEP = 64;   // K per LDS stage
constexpr int LDP = 8;      // LDS row padding (halfs): 144 B rows spread 16 rows over all banks

struct GemmP {
  WPlanes w;
  const __half* x;
  int M, N, K;
  float* y;
  __half* q;
  __half* k;
  __half* vt;
  const float* rope_cos;
  const float* rope_sin;
  int L, Lp, H, D;
  __half* g;
  float* part;  // split-K partials [K/kchunk][M][N]
};

// GeLU with the reference's rational tanh (internal/ggml/ops_simd.go:27-42).
__device__ __forceinline__ float gelu_r(float v) {
  const float t = 0.7978845608f * v * (1.0f + 0.044715f * v * v);
  const float t2 = t * t;
  float th = t * (27.0f + t2) / (27.0f + 9.0f * t2);
  if (t > 4.97f) th = 1.0f;
  else if (t < -4.97f) th = -1.0f;
  return 0.5f * v * (1.0f + th);
}

// Epilogue for 4 consecutive output features f..f+3 (f % 4 == 0) of token m.
template <int EPI>
__device__ __forceinline__ void epilogue(const GemmP& p, int m, int f, floatx4 v) {
  if constexpr (EPI == EPI_F32) {
    *(floatx4*)(p.y + (size_t)m * p.N + f) = v;
  } else if constexpr (EPI == EPI_RESID) {
    floatx4* dst = (floatx4*)(p.y + (size_t)m * p.N + f);
    floatx4 h = *dst;
    // hiddens[i][j] += out[i][j]  (internal/embed/bert.go:262-264, 276-278)
    h.x = h.x + v.x; h.y = h.y + v.y; h.z = h.z + v.z; h.w = h.w + v.w;
    *dst = h;
  } else if constexpr (EPI == EPI_QKV) {
    // QKV row = [Q | K | V], heads 64-contiguous (bert.go:332-347); RoPE on Q and K with
    // the position = token index (bert.go:349-353, ops_simd.go:127-137).
    const int D = p.D;
    const int sec = f / D, fi = f - sec * D, h = fi >> 6, e = fi & 63;
    const int b = m / p.L, pos = m - b * p.L;
    if (sec < 2) {
      const float* cr = p.rope_cos + (size_t)pos * 32 + (e >> 1);
      const float* sr = p.rope_sin + (size_t)pos * 32 + (e >> 1);
      const float c0 = cr[0], s0 = sr[0], c1 = cr[1], s1 = sr[1];
      const float a0 = v.x * c0 - v.y * s0, a1 = v.x * s0 + v.y * c0;
      const float a2 = v.z * c1 - v.w * s1, a3 = v.z * s1 + v.w * c1;
      __half* dst = (sec == 0 ? p.q : p.k) + (((size_t)b * p.H + h) * p.Lp + pos) * 64 + e;
      __half2 lo = __floats2half2_rn(a0, a1), hi = __floats2half2_rn(a2, a3);
      uint2 pk;
      pk.x = *(uint32_t*)&lo;
      pk.y = *(uint32_t*)&hi;
      *(uint2*)dst = pk;
    } else {
      __half* dst = p.vt + (((size_t)b * p.H + h) * 64 + e) * p.Lp + pos;
      dst[0] = __float2half_rn(v.x);
      dst[(size_t)p.Lp] = __float2half_rn(v.y);
      dst[(size_t)2 * p.Lp] = __float2half_rn(v.z);
      dst[(size_t)3 * p.Lp] = __float2half_rn(v.w);
    }
  } else {  // EPI_GEGLU: rows interleaved (up q, gate q, up q+1, gate q+1)
    // gates = GeLU(gate) * up  (internal/embed/bert.go:431-436)
    const int qo = f >> 1, F = p.N >> 1;
    const float o0 = gelu_r(v.y) * v.x, o1 = gelu_r(v.w) * v.z;
    *(__half2*)(p.g + (size_t)m * F + qo) = __floats2half2_rn(o0, o1);
  }
}

__device__ __forceinline__ uint4 pack8(const float* v) {
  __half2 a = __floats2half2_rn(v[0], v[1]), b = __floats2half2_rn(v[2], v[3]);
  __half2 c = __floats2half2_rn(v[4], v[5]), d = __floats2half2_rn(v[6], v[7]);
  uint4 r;
  r.x = *(uint32_t*)&a;
  r.y = *(uint32_t*)&b;
  r.z = *(uint32_t*)&c;
  r.w = *(uint32_t*)&d;
  return r;
}

__device__ __forceinline__ floatx4 mfma16(const half8& a, const half8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------
// Canonical chunk of the K reduction: 768 when K is a multiple of 768 (every nomic-bert
// projection), else 256. Both kernel families derive it from K alone.
__host__ __device__ constexpr int kchunk_of(int K) { return (K % 768 == 0) ? 768 : 256; }

// Large-M kernel: BM x BN block tile, 4 waves in WM x WN, LDS double buffer over 64-wide K
// steps, dequantisation at LDS-store time (each weight decoded once per block tile).
// MULTI = K spans more than one canonical chunk (then a second accumulator set holds the
// running total). Two blocks per CU (launch bounds) so one block's loads overlap the other's
// MFMAs.
template <int FMT, int BM, int BN, int WM, int WN, int EPI, bool MULTI>
__global__ __launch_bounds__(256, 2) void gemm_big(GemmP p) {
  constexpr int TM = BM / WM, TN = BN / WN, FB = TN / 16, TB = TM / 16;
  constexpr int LDW = KSTEP + LDP;
  constexpr int XCH = BM * (KSTEP / 8);   // 16-byte chunks of the X tile
  constexpr int XPT = (XCH + 255) / 256;
  constexpr int WU = BN * (KSTEP / 16);   // 16-element W segments
  constexpr int WPT = (WU + 255) / 256;
  __shared__ __attribute__((aligned(16))) _Float16 sW[2][BN][LDW];
  __shared__ __attribute__((aligned(16))) _Float16 sX[2][BM][LDW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int M = p.M, K = p.K;
  const int KT = K / KSTEP;
  const int steps_per_chunk = kchunk_of(K) / KSTEP;

  floatx4 acc[FB][TB];
  floatx4 tot[MULTI ? FB : 1][MULTI ? TB : 1];
#pragma unroll
  for (int i = 0; i < FB; i++)
#pragma unroll
    for (int j = 0; j < TB; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (MULTI) {
#pragma unroll
    for (int i = 0; i < FB; i++)
#pragma unroll
      for (int j = 0; j < TB; j++) tot[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  uint4 xr[XPT];
  RawSeg wr[WPT];

  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int c = tid + i * 256;
      if (c < XCH) {
        const int row = c >> 3, ch = c & 7, m = m0 + row;
        xr[i] = m < M ? *(const uint4*)(p.x + (size_t)m * K + kt * KSTEP + ch * 8) : uint4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * 256;
      if (u < WU) wr[i] = load_seg<FMT>(p.w, n0 + (u >> 2), kt * KSTEP + (u & 3) * 16);
    }
  };
  auto sstore = [&](int st, int kt) {
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int c = tid + i * 256;
      if (c < XCH) *(uint4*)&sX[st][c >> 3][(c & 7) * 8] = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * 256;
      if (u < WU) {
        float v[16];
        decode_seg<FMT>(wr[i], kt * KSTEP + (u & 3) * 16, v);
        uint4* dst = (uint4*)&sW[st][u >> 2][(u & 3) * 16];
        dst[0] = pack8(v);
        dst[1] = pack8(v + 8);
      }
    }
  };

  gload(0);
  sstore(0, 0);
  __syncthreads();
  const int lr = lane & 15, lk = (lane >> 4) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int st = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      half8 af[FB], bf[TB];
#pragma unroll
      for (int i = 0; i < FB; i++) af[i] = *(const half8*)&sW[st][wn * TN + i * 16 + lr][ks * 32 + lk];
#pragma unroll
      for (int j = 0; j < TB; j++) bf[j] = *(const half8*)&sX[st][wm * TM + j * 16 + lr][ks * 32 + lk];
#pragma unroll
      for (int i = 0; i < FB; i++)
#pragma unroll
        for (int j = 0; j < TB; j++) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
    }
    if constexpr (MULTI) {
      if ((kt + 1) % steps_per_chunk == 0) {
#pragma unroll
        for (int i = 0; i < FB; i++)
#pragma unroll
          for (int j = 0; j < TB; j++) {
            tot[i][j] += acc[i][j];
            acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
          }
      }
    }
    if (kt + 1 < KT) sstore(st ^ 1, kt + 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < TB; j++) {
    const int m = m0 + wm * TM + j * 16 + lr;
    if (m < M) {
#pragma unroll
      for (int i = 0; i < FB; i++) {
        floatx4 v;
        if constexpr (MULTI) {
          v = tot[i][j];
        } else {
          v = floatx4{0.f, 0.f, 0.f, 0.f};
          v += acc[i][j];  // total = 0 + chunk, as the split-K reduction computes it
        }
        epilogue<EPI>(p, m, n0 + wn * TN + i * 16 + (lane >> 4) * 4, v);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Small-M kernel (M <= 64): one block per (64-row feature tile, canonical K chunk). Every
// global load of the block is issued before the first MFMA (one memory round trip); the chunk
// goes through LDS in 256-wide pieces while a single MFMA chain continues across them. The
// chunk result goes to part[chunk][m][n]; gemm_reduce adds the chunks in order.
template <int FMT, int BM, int NPIECE>
__global__ __launch_bounds__(256) void gemm_small(GemmP p) {
  constexpr int BN = 64, TB = BM / 16, PK = 256;
  constexpr int LDW = PK + LDP;
  constexpr int WU = BN * (PK / 16);  // 1024 segments per piece
  constexpr int WPT = WU / 256;
  constexpr int XCH = BM * (PK / 8);
  constexpr int XPT = (XCH + 255) / 256;
  constexpr bool AHEAD = FMT != 0;  // f32 weights are too wide to hold every piece in registers
  constexpr int NP = AHEAD ? NPIECE : 1;
  __shared__ __attribute__((aligned(16))) _Float16 sW[BN][LDW];
  __shared__ __attribute__((aligned(16))) _Float16 sX[BM][LDW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * BN, c = blockIdx.y, kbase = c * NPIECE * PK;
  const int M = p.M, K = p.K;

  RawSeg wr[NP][WPT];
  uint4 xr[NP][XPT];
  auto load_piece = [&](int slot, int kb) {
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * 256;
      wr[slot][i] = load_seg<FMT>(p.w, n0 + (u >> 4), kb + (u & 15) * 16);
    }
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int cc = tid + i * 256;
      if (cc < XCH) {
        const int row = cc >> 5, ch = cc & 31;
        xr[slot][i] = row < M ? *(const uint4*)(p.x + (size_t)row * K + kb + ch * 8) : uint4{0, 0, 0, 0};
      }
    }
  };
  if constexpr (AHEAD) {
#pragma unroll
    for (int pc = 0; pc < NPIECE; pc++) load_piece(pc, kbase + pc * PK);
  }

  const int lr = lane & 15, lk = (lane >> 4) * 8;
  floatx4 acc[TB];
#pragma unroll
  for (int j = 0; j < TB; j++) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int pc = 0; pc < NPIECE; pc++) {
    const int slot = AHEAD ? pc : 0;
    const int kb = kbase + pc * PK;
    if constexpr (!AHEAD) load_piece(0, kb);
    if (pc > 0) __syncthreads();
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int cc = tid + i * 256;
      if (cc < XCH) *(uint4*)&sX[cc >> 5][(cc & 31) * 8] = xr[slot][i];
    }
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * 256;
      float v[16];
      decode_seg<FMT>(wr[slot][i], kb + (u & 15) * 16, v);
      uint4* dst = (uint4*)&sW[u >> 4][(u & 15) * 16];
      dst[0] = pack8(v);
      dst[1] = pack8(v + 8);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < PK / 32; ks++) {
      const half8 af = *(const half8*)&sW[wave * 16 + lr][ks * 32 + lk];
#pragma unroll
      for (int j = 0; j < TB; j++) {
        const half8 bf = *(const half8*)&sX[j * 16 + lr][ks * 32 + lk];
        acc[j] = mfma16(af, bf, acc[j]);
      }
    }
  }
  float* part = p.part + (size_t)c * M * p.N;
#pragma unroll
  for (int j = 0; j < TB; j++) {
    const int m = j * 16 + lr;
    if (m < M) *(floatx4*)(part + (size_t)m * p.N + n0 + wave * 16 + (lane >> 4) * 4) = acc[j];
  }
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_reduce(GemmP p) {
  const int nq = p.N >> 2;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.M * nq) return;
  const int m = idx / nq, f = (idx - m * nq) * 4;
  const int nch = p.K / kchunk_of(p.K);
  floatx4 t = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nch; c++) t += *(const floatx4*)(p.part + ((size_t)c * p.M + m) * p.N + f);
  epilogue<EPI>(p, m, f, t);
}

// ---------------------------------------------------------------------------------------
template <int FMT, int BM, int EPI>
static hipError_t launch_small(const GemmP& p, hipStream_t st) {
  const int kc = kchunk_of(p.K);
  dim3 grid(p.N / 64, p.K / kc);
  if (kc == 768)
    hipLaunchKernelGGL((gemm_small<FMT, BM, 3>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_small<FMT, BM, 1>), grid, dim3(256), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int n = p.M * (p.N / 4);
  hipLaunchKernelGGL((gemm_reduce<EPI>), dim3((n + 255) / 256), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <int FMT, int EPI>
static hipError_t launch_fmt(const GemmP& p, hipStream_t st) {
  if (p.M <= 64) {
    if (p.M <= 16) return launch_small<FMT, 16, EPI>(p, st);
    if (p.M <= 32) return launch_small<FMT, 32, EPI>(p, st);
    return launch_small<FMT, 64, EPI>(p, st);
  }
  dim3 grid(p.N / 128, (p.M + 127) / 128);
  if (p.K > kchunk_of(p.K))
    hipLaunchKernelGGL((gemm_big<FMT, 128, 128, 2, 2, EPI, true>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_big<FMT, 128, 128, 2, 2, EPI, false>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_epi(int type, const GemmP& p, hipStream_t st) {
  switch (type) {
    case LLE_TYPE_Q8_0: return launch_fmt<8, EPI>(p, st);
    case LLE_TYPE_Q4_K: return launch_fmt<12, EPI>(p, st);
    case LLE_TYPE_Q5_K: return launch_fmt<13, EPI>(p, st);
    case LLE_TYPE_Q6_K: return launch_fmt<14, EPI>(p, st);
    case LLE_TYPE_F32: return launch_fmt<0, EPI>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm(const GemmArgs& a, int epi, hipStream_t st) {
  GemmP p;
  p.w = WPlanes{a.w->p0, a.w->p1, a.w->p2, a.w->p3, a.w->K, a.w->N};
  p.x = a.x;
  p.M = a.M;
  p.N = a.w->N;
  p.K = a.w->K;
  p.y = a.y;
  p.q = a.q;
  p.k = a.k;
  p.vt = a.vt;
  p.rope_cos = a.rope_cos;
  p.rope_sin = a.rope_sin;
  p.L = a.L;
  p.Lp = a.Lp;
  p.H = a.n_head;
  p.D = a.d_model;
  p.g = a.g;
  p.part = a.part;
  switch (epi) {
    case EPI_F32: return launch_epi<EPI_F32>(a.w->type, p, st);
    case EPI_RESID: return launch_epi<EPI_RESID>(a.w->type, p, st);
    case EPI_QKV: return launch_epi<EPI_QKV>(a.w->type, p, st);
    case EPI_GEGLU: return launch_epi<EPI_GEGLU>(a.w->type, p, st);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------------------
// Dequantise an uploaded weight with the GEMM's own segment decoder: out f32 [N][K].
template <int FMT>
__global__ void dequant_weight_kernel(WPlanes w, float* out) {
  const int64_t nseg = (int64_t)w.N * (w.K / 16);
  for (int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; s < nseg; s += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(s / (w.K / 16)), k0 = (int)(s % (w.K / 16)) * 16;
    RawSeg r = load_seg<FMT>(w, n, k0);
    float v[16];
    decode_seg<FMT>(r, k0, v);
    float* o = out + (size_t)n * w.K + k0;
#pragma unroll
    for (int i = 0; i < 16; i++) o[i] = v[i];
  }
}

hipError_t launch_dequant_weight(const WeightDev& wd, float* out, hipStream_t st) {
  WPlanes w{wd.p0, wd.p1, wd.p2, wd.p3, wd.K, wd.N};
  dim3 g(1024), b(256);
  switch (wd.type) {
    case LLE_TYPE_Q8_0: hipLaunchKernelGGL((dequant_weight_kernel<8>), g, b, 0, st, w, out); break;
    case LLE_TYPE_Q4_K: hipLaunchKernelGGL((dequant_weight_kernel<12>), g, b, 0, st, w, out); break;
    case LLE_TYPE_Q5_K: hipLaunchKernelGGL((dequant_weight_kernel<13>), g, b, 0, st, w, out); break;
    case LLE_TYPE_Q6_K: hipLaunchKernelGGL((dequant_weight_kernel<14>), g, b, 0, st, w, out); break;
    case LLE_TYPE_F32: hipLaunchKernelGGL((dequant_weight_kernel<0>), g, b, 0, st, w, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lle
