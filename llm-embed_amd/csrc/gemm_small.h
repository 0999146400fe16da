// Shared pieces of the projection GEMMs: the parameter block, the epilogues and the small-M
// GEMM as a device function (run by the gemm_small kernel in gemm.hip).
#pragma once

#include "deq_device.h"
#include "lle_internal.h"
#include "mfma_common.h"
#include "row_device.h"

namespace lle {

constexpr int KSTEP = 64;   // K per LDS stage

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
  const __half* w16;  // resident f16 copy of the weights [N][K], or null
  LnPrologue ln;      // LayerNorm prologue of the small-M kernel
  const int32_t* tokrow;  // packed rows: row m is padded token tokrow[m] (null: m)
};

// GeLU with the reference's rational tanh (internal/ggml/ops_simd.go:27-42):
//   t = 0.7978845608 v (1 + 0.044715 v v),  tanh ~ t (27 + t^2) / (27 + 9 t^2),  +-1 past |t| 4.97,
//   0.5 v (1 + tanh).
// Written for the up/gate GEMM's epilogue, which runs it on 100 M values per launch with the
// matrix cores idle: the quotient uses the hardware reciprocal (v_rcp_f32, 1 ulp) instead of a
// correctly rounded division, three of the multiply-adds are fused, and the clamp is a select
// (a branch per value before). Each changes the result by an ulp or so of f32 before it is
// rounded to f16 (2^-11); every GEMM path calls this one function, so they stay bit-identical.
__device__ __forceinline__ float gelu_r(float v) {
  const float t = (0.7978845608f * v) * fmaf(0.044715f * v, v, 1.0f);
  const float t2 = t * t;
  float r = t * (27.0f + t2) * __builtin_amdgcn_rcpf(fmaf(9.0f, t2, 27.0f));
  asm("" : "+v"(r));  // computed for every value: otherwise the select becomes a branch around it
  const float th = fabsf(t) > 4.97f ? copysignf(1.0f, t) : r;
  const float hv = 0.5f * v;
  return fmaf(hv, th, hv);
}

// Operands an epilogue reads from memory for features f..f+3 of token m: the residual
// (EPI_RESID) or the RoPE cos/sin pairs (EPI_QKV, Q and K sections). The small-M kernel issues
// these loads before its main loop so that they do not add a round trip at the end.
template <int EPI>
__device__ __forceinline__ floatx4 epi_operands(const GemmP& p, int m, int f) {
  if constexpr (EPI == EPI_RESID) {
    return *(const floatx4*)(p.y + (size_t)m * p.N + f);
  } else if constexpr (EPI == EPI_QKV) {
    const int sec = f / p.D, e = (f - sec * p.D) & 63;
    const int r = p.tokrow ? p.tokrow[m] : m;
    const int pos = r - (r / p.L) * p.L;
    if (sec < 2) {
      const float* cr = p.rope_cos + (size_t)pos * 32 + (e >> 1);
      const float* sr = p.rope_sin + (size_t)pos * 32 + (e >> 1);
      return floatx4{cr[0], sr[0], cr[1], sr[1]};
    }
    return floatx4{0.f, 0.f, 0.f, 0.f};
  } else {
    return floatx4{0.f, 0.f, 0.f, 0.f};
  }
}

// Epilogue for 4 consecutive output features f..f+3 (f % 4 == 0) of token m; `o` holds what
// epi_operands returned for the same (m, f).
template <int EPI>
__device__ __forceinline__ void epilogue_with(const GemmP& p, int m, int f, floatx4 v, floatx4 o) {
  if constexpr (EPI == EPI_F32) {
    *(floatx4*)(p.y + (size_t)m * p.N + f) = v;
  } else if constexpr (EPI == EPI_RESID) {
    // hiddens[i][j] += out[i][j]  (internal/embed/bert.go:262-264, 276-278)
    floatx4 h = o;
    h.x = h.x + v.x; h.y = h.y + v.y; h.z = h.z + v.z; h.w = h.w + v.w;
    *(floatx4*)(p.y + (size_t)m * p.N + f) = h;
  } else if constexpr (EPI == EPI_QKV) {
    // QKV row = [Q | K | V], heads 64-contiguous (bert.go:332-347); RoPE on Q and K with
    // the position = token index (bert.go:349-353, ops_simd.go:127-137).
    const int D = p.D;
    const int sec = f / D, fi = f - sec * D, h = fi >> 6, e = fi & 63;
    const int r = p.tokrow ? p.tokrow[m] : m;
    const int b = r / p.L, pos = r - b * p.L;
    if (sec < 2) {
      const float c0 = o.x, s0 = o.y, c1 = o.z, s1 = o.w;
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

template <int EPI>
__device__ __forceinline__ void epilogue(const GemmP& p, int m, int f, floatx4 v) {
  epilogue_with<EPI>(p, m, f, v, epi_operands<EPI>(p, m, f));
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


// LDS tiles are rows of 16-byte chunks; chunk c of row r is stored at c ^ (r & 7). A wave's
// ds_read_b128 of 16 rows x one chunk then spreads over all banks (measured on gfx950: 1.8x the
// read bandwidth of 16-byte-padded rows).
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ (row & 7); }

// ---------------------------------------------------------------------------------------
// Canonical chunk of the K reduction: 768 when K is a multiple of 768 (every nomic-bert
// projection), else 256. Both kernel families derive it from K alone.
__host__ __device__ constexpr int kchunk_of(int K) { return (K % 768 == 0) ? 768 : 256; }

// ---------------------------------------------------------------------------------------
// Small-M kernel (M <= 64): one block per (BN-row feature tile, canonical K chunk). Every
// global load of the block is issued before the first MFMA (one memory round trip); the chunk
// goes through LDS in 256-wide pieces while a single MFMA chain continues across them. The
// chunk result goes to part[chunk][m][n]; gemm_reduce adds the chunks in order.
// LNP > 0 (M <= 16, K = NPIECE * 256 = 768, one chunk): X = LayerNorm(ln.src + ordered sum of
// LNP-1 partial chunks) computed in every block with ln_row's arithmetic and written as f16
// straight into LDS for the whole K; block 0 also stores the f32 LayerNorm rows to ln.out.
// Shapes of the small-M kernel: per-thread weight registers and the LDS it carves.
template <int FMT, int BM, int BN, int NPIECE, int LNP>
struct SmallShape {
  static constexpr int NT = BN * 4, PK = 256;  // one wave per 16 features
  static constexpr int LDW = PK;               // XOR-swizzled chunks (swz)
  static constexpr int WU = BN * (PK / 16);    // segments per piece
  static constexpr int WPT = WU / NT;
  static constexpr bool AHEAD = FMT != 0;  // f32 weights are too wide to hold every piece in registers
  static constexpr int NP = AHEAD ? NPIECE : 1;
  static constexpr int KF = NPIECE * PK;   // LNP: the whole K
  // 16-row blocks (the smallest batches, latency-bound) decode every piece into its own LDS
  // buffer behind one barrier, and the MFMA chain then runs over the whole chunk without stops
  static constexpr bool ALLW = AHEAD && BM == 16;
  static constexpr int NWB = ALLW ? NPIECE : 1;
  // weight staging; with a LayerNorm prologue it first holds the prologue's 16 rows + w, b (f32)
  static constexpr size_t SWW = (size_t)NWB * BN * LDW * 2, SLN = LNP ? (size_t)(16 + 2) * KF * 4 : 0;
  static constexpr size_t SW = SWW > SLN ? SWW : SLN;
  static constexpr size_t SX = (size_t)(LNP ? 1 : NWB) * (LNP ? 1 : BM) * LDW * 2;
  static constexpr size_t SXF = (size_t)(LNP ? BM : 1) * (LNP ? KF : 8) * 2;
  static constexpr size_t LDS = SW + SX + SXF;  // bytes, every part a multiple of 16
};

// Block (bx, by, bz) of the small-M GEMM, its LDS at `lds` (SmallShape::LDS bytes, 16-byte
// aligned); wr holds the block's weight segments as they arrive.
template <int FMT, int BM, int BN, int NPIECE, int EPI, bool DIRECT, int LNP>
__device__ __forceinline__ void gemm_small_dev(const GemmP& p, int bx, int by, int bz, unsigned char* lds,
                                               RawSeg (&wr)[SmallShape<FMT, BM, BN, NPIECE, LNP>::NP]
                                                           [SmallShape<FMT, BM, BN, NPIECE, LNP>::WPT]) {
  using SS = SmallShape<FMT, BM, BN, NPIECE, LNP>;
  lds = static_cast<unsigned char*>(__builtin_assume_aligned(lds, 16));
  constexpr int NT = SS::NT, TB = BM / 16, PK = SS::PK, LDW = SS::LDW, WPT = SS::WPT;
  constexpr int XCH = BM * (PK / 8);
  constexpr int XPT = (XCH + NT - 1) / NT;
  constexpr bool AHEAD = SS::AHEAD;
  constexpr int NP = SS::NP, KF = SS::KF;
  constexpr bool ALLW = SS::ALLW;
  _Float16(*sW)[BN][LDW] = reinterpret_cast<_Float16(*)[BN][LDW]>(lds);
  _Float16(*sX)[LNP ? 1 : BM][LDW] = reinterpret_cast<_Float16(*)[LNP ? 1 : BM][LDW]>(lds + SS::SW);
  _Float16(*sXf)[LNP ? KF : 8] = reinterpret_cast<_Float16(*)[LNP ? KF : 8]>(lds + SS::SW + SS::SX);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = bx * BN, c = by, kbase = c * NPIECE * PK;
  const int mb = bz * BM;  // row block (gridDim.z > 1 for 64 < M < 1024)
  const int M = p.M, K = p.K;

  uint4 xr[NP][XPT];
  auto load_piece = [&](int slot, int kb) {
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * NT;
      wr[slot][i] = load_seg<FMT>(p.w, n0 + (u >> 4), kb + (u & 15) * 16);
    }
    if constexpr (LNP == 0) {
#pragma unroll
      for (int i = 0; i < XPT; i++) {
        const int cc = tid + i * NT;
        if (cc < XCH) {
          const int row = mb + (cc >> 5), ch = cc & 31;
          xr[slot][i] = row < M ? *(const uint4*)(p.x + (size_t)row * K + kb + ch * 8) : uint4{0, 0, 0, 0};
        }
      }
    }
  };
  // LayerNorm prologue: wave w normalises rows w, w + 4 (and w + 8, w + 12). Its inputs (the
  // residual rows, the partial chunks to add to them, the LayerNorm weights) are read with
  // 16-byte loads, 4 consecutive elements per lane, and summed element by element in
  // reduce_resid_ln_kernel's order, x + (0 + p0 + p1 + ...): 32 loads per lane for rows 0..7 and
  // the weights, so that with the weight stream (24) every load is in flight at once (a wave can
  // have 63; 144 four-byte loads made it wait for the first ones before issuing the weights).
  // The sums go through LDS, the weight staging area, which is free until the pieces are decoded,
  // into ln_row's element-to-lane mapping (element lane + 64 i), so the LayerNorm's arithmetic and
  // every output bit are unchanged. The inputs of rows 0..7 are loaded before the weight stream:
  // vector loads complete in issue order, so issued after it they could not be used before the
  // whole stream had arrived.
  constexpr int NPART = LNP > 0 ? LNP - 1 : 0, NE = LNP > 0 ? KF / 64 : 1;
  constexpr int G = LNP > 0 ? KF / 256 : 1;  // 16-byte groups per lane and row
  static_assert(LNP == 0 || (KF % 256 == 0 && (16 + 2) * KF * 4 <= SS::SW), "prologue staging");
  float* stg = reinterpret_cast<float*>(lds);  // rows [16][KF], then w and b [2][KF]
  constexpr int NPQ = NPART > 0 ? NPART : 1;
  floatx4 xs[2][G], pv[2][G][NPQ], wb4[2];  // native vectors: HIP's float4 struct kept these in memory
  // loads only (rows past M re-read row M - 1 and are not used): the sums come after the weight
  // stream is issued, so that no wait sits between these loads and it
  auto ln_issue = [&](int r0) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int r = min(r0 + wave + 4 * h, M - 1);
#pragma unroll
      for (int g = 0; g < G; g++) {
        const int j = g * 256 + lane * 4;
        xs[h][g] = *(const floatx4*)(p.ln.src + (size_t)r * KF + j);
#pragma unroll
        for (int q = 0; q < NPART; q++) pv[h][g][q] = *(const floatx4*)(p.ln.part + ((size_t)q * M + r) * KF + j);
      }
    }
  };
  auto ln_sum = [&]() {
    if constexpr (NPART > 0) {
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int g = 0; g < G; g++) {
          floatx4 t = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < NPART; q++) {
            t.x += pv[h][g][q].x; t.y += pv[h][g][q].y; t.z += pv[h][g][q].z; t.w += pv[h][g][q].w;
          }
          xs[h][g].x = xs[h][g].x + t.x; xs[h][g].y = xs[h][g].y + t.y;
          xs[h][g].z = xs[h][g].z + t.z; xs[h][g].w = xs[h][g].w + t.w;
        }
    }
  };
  if constexpr (LNP > 0) {
    const int wt = min(tid, KF / 4 - 1);  // threads past KF / 4 re-read the last group (not stored)
    wb4[0] = *(const floatx4*)(p.ln.w + wt * 4);
    wb4[1] = *(const floatx4*)(p.ln.b + wt * 4);
    ln_issue(0);
    __builtin_amdgcn_sched_barrier(0);  // these loads stay in front of the weight stream
  }
  if constexpr (AHEAD) {
#pragma unroll
    for (int pc = 0; pc < NPIECE; pc++) load_piece(pc, kbase + pc * PK);
  }

  if constexpr (LNP > 0) {
    __builtin_amdgcn_sched_barrier(0);  // nothing that waits on the prologue's loads moves above the stream
    static_assert(BM == 16 && DIRECT && KF <= 64 * MAXE && NT == 256, "LayerNorm prologue shape");
    float lw[MAXE], lb[MAXE];
    {  // every thread stores (those past KF / 4 the last group again): a store under a branch
       // let the compiler sink the loads behind the weight stream
      const int wt = min(tid, KF / 4 - 1);
      *(floatx4*)(stg + 16 * KF + wt * 4) = wb4[0];
      *(floatx4*)(stg + 17 * KF + wt * 4) = wb4[1];
    }
    auto ln_rows = [&](int r0) {
      // this wave's two rows into LDS and back in ln_row's mapping (the wave reads only what it
      // wrote, so a wave-level fence orders it)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int r = r0 + wave + 4 * h;
        if (r < M) {
#pragma unroll
          for (int g = 0; g < G; g++) *(floatx4*)(stg + r * KF + g * 256 + lane * 4) = xs[h][g];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int r = r0 + wave + 4 * h;
        float x[MAXE];
        if (r < M) {
#pragma unroll
          for (int i = 0; i < NE; i++) x[i] = stg[r * KF + lane + 64 * i];
          ln_apply_wb(x, NE, KF, lw, lb, p.ln.eps);
          if (bx == 0 && by == 0) {
#pragma unroll
            for (int i = 0; i < NE; i++) p.ln.out[(size_t)r * KF + lane + 64 * i] = x[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < NE; i++) x[i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < NE; i++) {
          const int k = lane + 64 * i;  // chunk k/8 stored at (k/8) ^ (r & 7), as swz
          sXf[r][(((k >> 3) ^ (r & 7)) << 3) + (k & 7)] = (_Float16)__float2half_rn(x[i]);
        }
      }
    };
    // barriers on LDS only (lgkmcnt): the weight stream stays in flight behind the prologue
    auto lds_barrier = [&]() {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt(63) expcnt(7) lgkmcnt(0)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    lds_barrier();  // the LayerNorm weights are in LDS
#pragma unroll
    for (int i = 0; i < NE; i++) {
      lw[i] = stg[16 * KF + lane + 64 * i];
      lb[i] = stg[17 * KF + lane + 64 * i];
    }
    ln_sum();
    ln_rows(0);
    if (M > 8) {  // rows 8..15
      ln_issue(8);
      ln_sum();
      ln_rows(8);
    }
    lds_barrier();  // every wave is done with the staging before the pieces are decoded there
  }

  const int lr = lane & 15, lg = lane >> 4;
  floatx4 eop[DIRECT ? TB : 1];
  if constexpr (DIRECT) {
#pragma unroll
    for (int j = 0; j < TB; j++)
      if (mb + j * 16 + lr < M) eop[j] = epi_operands<EPI>(p, mb + j * 16 + lr, n0 + wave * 16 + lg * 4);
  }
  floatx4 acc[TB];
#pragma unroll
  for (int j = 0; j < TB; j++) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  auto mma_piece = [&](int pc, int ws) {
#pragma unroll
    for (int ks = 0; ks < PK / 32; ks++) {
      const half8 af = *(const half8*)&sW[ws][wave * 16 + lr][swz(lr, ks * 4 + lg) * 8];
#pragma unroll
      for (int j = 0; j < TB; j++) {
        half8 bf;
        if constexpr (LNP > 0)
          bf = *(const half8*)&sXf[j * 16 + lr][(pc * (PK / 8) + swz(lr, ks * 4 + lg)) * 8];
        else
          bf = *(const half8*)&sX[ws][j * 16 + lr][swz(lr, ks * 4 + lg) * 8];
        acc[j] = mfma16(af, bf, acc[j]);
      }
    }
  };
#pragma unroll
  for (int pc = 0; pc < NPIECE; pc++) {
    const int slot = AHEAD ? pc : 0, ws = ALLW ? pc : 0;
    const int kb = kbase + pc * PK;
    if constexpr (!AHEAD) load_piece(0, kb);
    if (!ALLW && pc > 0) __syncthreads();
    if constexpr (LNP == 0) {
#pragma unroll
      for (int i = 0; i < XPT; i++) {
        const int cc = tid + i * NT;
        if (cc < XCH) *(uint4*)&sX[ws][cc >> 5][swz(cc >> 5, cc & 31) * 8] = xr[slot][i];
      }
    }
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * NT, row = u >> 4, sg = u & 15;
      uint4 lo, hi;
      decode_seg_h<FMT>(wr[slot][i], kb + sg * 16, lo, hi);
      *(uint4*)&sW[ws][row][swz(row, 2 * sg) * 8] = lo;
      *(uint4*)&sW[ws][row][swz(row, 2 * sg + 1) * 8] = hi;
    }
    if constexpr (!ALLW) {
      __syncthreads();
      mma_piece(pc, 0);
    }
  }
  if constexpr (ALLW) {
    __syncthreads();
#pragma unroll
    for (int pc = 0; pc < NPIECE; pc++) mma_piece(pc, pc);
  }
  if constexpr (DIRECT) {
    // single-chunk K: the total is 0 + this chunk, finished here with the epilogue
#pragma unroll
    for (int j = 0; j < TB; j++) {
      const int m = mb + j * 16 + lr;
      if (m < M) {
        floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
        v += acc[j];
        epilogue_with<EPI>(p, m, n0 + wave * 16 + lg * 4, v, eop[j]);
      }
    }
  } else {
    float* part = p.part + (size_t)c * M * p.N;
#pragma unroll
    for (int j = 0; j < TB; j++) {
      const int m = mb + j * 16 + lr;
      if (m < M) *(floatx4*)(part + (size_t)m * p.N + n0 + wave * 16 + (lane >> 4) * 4) = acc[j];
    }
  }
}

}  // namespace lle
