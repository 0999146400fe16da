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
#include <climits>
#include <type_traits>

#include "gemm_small.h"

namespace lle {

// Large-M kernel: BM x BN block tile, 4 waves in WM x WN, LDS double buffer over 64-wide K
// steps, dequantisation at LDS-store time (each weight decoded once per block tile).
// MULTI = K spans more than one canonical chunk (then a second accumulator set holds the
// running total). Two blocks per CU (launch bounds) so one block's loads overlap the other's
// MFMAs.
// LA = load lookahead in K steps (register sets in flight): 2 for 128-wide feature tiles, 1 for
// 256-wide ones whose 128 accumulators leave room for a single set.
template <int FMT, int BM, int BN, int WM, int WN, int EPI, bool MULTI, int LA>
__global__ __launch_bounds__(WM * WN * 64, 512 / (WM * WN * 64)) void gemm_big(GemmP p) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN, FB = TN / 16, TB = TM / 16;
  constexpr int LDW = KSTEP;  // 128-byte rows, 16-byte chunks XOR-swizzled by row (swz)
  constexpr int XCH = BM * (KSTEP / 8);   // 16-byte chunks of the X tile
  constexpr int XPT = XCH / NT;
  constexpr int WU = BN * (KSTEP / 16);   // 16-element W segments
  constexpr int WPT = WU / NT;
  __shared__ __attribute__((aligned(16))) _Float16 sW[2][BN][LDW];
  __shared__ __attribute__((aligned(16))) _Float16 sX[2][BM][LDW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  {
    // XCD-aware tile order. The dispatcher deals workgroups to the 8 XCDs round-robin
    // (workgroup b runs on XCD b % 8); each XCD has its own L2. The XCDs form an MG x NG grid
    // over the tile grid and walk their share N-fastest, so the feature tiles that share a
    // token tile's X run on one XCD while each XCD's weight tiles stay resident in its L2:
    // 128-wide tiles (N <= 2304: every weight tile fits) use MG = 8, NG = 1; the 256-wide tiles
    // of N = 6144 use MG = 4, NG = 2 (12 weight tiles, 2.5 MB per XCD). Any bijection is
    // correct; this is only cache locality.
    constexpr int NG = BN >= 256 ? 2 : 1, MG = 8 / NG;
    const int nt = gridDim.x, mt = gridDim.y, G = nt * mt;
    const int b = blockIdx.x + blockIdx.y * nt, xcd = b & 7, slot = b >> 3;
    if (nt % NG == 0 && mt % MG == 0) {
      const int ntl = nt / NG, mtl = mt / MG;
      n0 = ((xcd % NG) * ntl + slot % ntl) * BN;
      m0 = ((xcd / NG) * mtl + slot / ntl) * BM;
    } else if (NG == 1) {
      // contiguous runs of the N-fastest tile order, the first G % 8 XCDs one tile longer
      const int q = G >> 3, r = G & 7;
      const int t = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
      n0 = (t % nt) * BN;
      m0 = (t / nt) * BM;
    }
  }
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

  static_assert(XCH % NT == 0 && WU % NT == 0, "tile loads must cover whole passes of the block");
  // Two register sets of prefetched data: set s holds K step j with j % 2 == s. Iteration kt
  // computes step kt from LDS, stores step kt+1 (loaded one iteration earlier) into the other
  // LDS stage and issues the loads of step kt+2, so each load has two steps of MFMA work to
  // arrive. Loads are buffer loads with loop-invariant lane offsets; rows past M re-read row
  // M-1 (those rows only feed output rows that are never stored).
  uint4 xr[LA][XPT];
  RawSeg wr[LA][WPT];
  const int lr = lane & 15, lg = lane >> 4;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x);
  const WRsrc rw{make_rsrc(p.w.p0), make_rsrc(p.w.p1), make_rsrc(p.w.p2), make_rsrc(p.w.p3)};
  int xoff[XPT];
#pragma unroll
  for (int i = 0; i < XPT; i++) {
    const int c = tid + i * NT;
    xoff[i] = (min(m0 + (c >> 3), M - 1) * K + (c & 7) * 8) * 2;
  }
  // W segment u: row u % BN, segment u / BN, so a wave's LDS stores hit consecutive rows
  SegOff woff[WPT];
#pragma unroll
  for (int i = 0; i < WPT; i++) {
    const int u = tid + i * NT;
    woff[i] = seg_off<FMT>(p.N, K, n0 + u % BN, u / BN);
  }

  auto gload = [&](auto S, int kt) {
    constexpr int s = decltype(S)::value;
#pragma unroll
    for (int i = 0; i < XPT; i++) xr[s][i] = buf_load16(rx, xoff[i], kt * KSTEP * 2);
#pragma unroll
    for (int i = 0; i < WPT; i++) wr[s][i] = load_seg_buf<FMT>(rw, woff[i], p.N, kt);
  };
  // store register set `set` (holding K step kt) into LDS stage `st`
  auto sstore = [&](auto SET, auto ST, int kt) {
    constexpr int set = decltype(SET)::value, st = decltype(ST)::value;
#pragma unroll
    for (int i = 0; i < XPT; i++) {
      const int c = tid + i * NT;
      *(uint4*)&sX[st][c >> 3][swz(c >> 3, c & 7) * 8] = xr[set][i];
    }
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * NT;
      const int row = u % BN, sg = u / BN;
      uint4 lo, hi;
      decode_seg_h<FMT>(wr[set][i], kt * KSTEP + sg * 16, lo, hi);
      *(uint4*)&sW[st][row][swz(row, 2 * sg) * 8] = lo;
      *(uint4*)&sW[st][row][swz(row, 2 * sg + 1) * 8] = hi;
    }
  };
  // One K step on LDS stage S: all 16 operand fragments are read first; the decode + LDS store
  // of the next stage (sstore) is interleaved between the first half's MFMAs so the VALU and
  // ds_write work overlaps the matrix pipe instead of running while it idles.
  // One K step on LDS stage S, storing register set SET (K step kt+1) into stage SN on the way.
  // LA = 2: every fragment is read first and the store is interleaved with the first half's
  // MFMAs (its loads were issued a step earlier). LA = 1: fragments are read per half and the
  // store waits until the second half, giving this step's loads half a step more to land.
  auto step = [&](auto S, auto SN, auto SET, int kt, bool store_next) {
    constexpr int s = decltype(S)::value;
    if constexpr (LA == 2) {
      half8 af[2][FB], bf[2][TB];
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
#pragma unroll
        for (int i = 0; i < FB; i++) af[ks][i] = *(const half8*)&sW[s][wn * TN + i * 16 + lr][swz(lr, ks * 4 + lg) * 8];
#pragma unroll
        for (int j = 0; j < TB; j++) bf[ks][j] = *(const half8*)&sX[s][wm * TM + j * 16 + lr][swz(lr, ks * 4 + lg) * 8];
      }
#pragma unroll
      for (int i = 0; i < FB; i++)
#pragma unroll
        for (int j = 0; j < TB; j++) acc[i][j] = mfma16(af[0][i], bf[0][j], acc[i][j]);
      if (store_next) sstore(SET, SN, kt + 1);
      // ds_read all fragments, then per MFMA of the first half: two VALU ops and some ds_writes
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FB + TB), 0);
#pragma unroll
      for (int i = 0; i < FB * TB; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
#pragma unroll
      for (int i = 0; i < FB; i++)
#pragma unroll
        for (int j = 0; j < TB; j++) acc[i][j] = mfma16(af[1][i], bf[1][j], acc[i][j]);
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        half8 af[FB], bf[TB];
#pragma unroll
        for (int i = 0; i < FB; i++) af[i] = *(const half8*)&sW[s][wn * TN + i * 16 + lr][swz(lr, ks * 4 + lg) * 8];
#pragma unroll
        for (int j = 0; j < TB; j++) bf[j] = *(const half8*)&sX[s][wm * TM + j * 16 + lr][swz(lr, ks * 4 + lg) * 8];
#pragma unroll
        for (int i = 0; i < FB; i++)
#pragma unroll
          for (int j = 0; j < TB; j++) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
        if (ks == 1 && store_next) {
          sstore(SET, SN, kt + 1);
          __builtin_amdgcn_sched_group_barrier(0x100, FB + TB, 0);
#pragma unroll
          for (int i = 0; i < FB * TB; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
          }
        }
      }
    }
  };
  auto chunk_end = [&](int kt) {
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
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  // KT is a multiple of 4 (K % 256 == 0), so the loop runs in pairs of steps (stage indices
  // stay compile-time constants). The last pair is peeled: inside the loop every path issues
  // the same loads, so the compiler's vmcnt waits count only the older set.
  if constexpr (LA == 2) {
    gload(S0{}, 0);
    gload(S1{}, 1);
    sstore(S0{}, S0{}, 0);
    __syncthreads();
    int kt = 0;
    for (; kt < KT - 2; kt += 2) {
      gload(S0{}, kt + 2);  // set 0 <- step kt+2
      __builtin_amdgcn_sched_barrier(0);
      step(S0{}, S1{}, S1{}, kt, true);  // compute stage 0, store set 1 (step kt+1) -> stage 1
      chunk_end(kt);
      __syncthreads();
      gload(S1{}, kt + 3);  // set 1 <- step kt+3
      __builtin_amdgcn_sched_barrier(0);
      step(S1{}, S0{}, S0{}, kt + 1, true);  // compute stage 1, store set 0 (step kt+2) -> stage 0
      chunk_end(kt + 1);
      __syncthreads();
    }
    step(S0{}, S1{}, S1{}, kt, true);
    chunk_end(kt);
    __syncthreads();
    step(S1{}, S0{}, S0{}, kt + 1, false);
    chunk_end(kt + 1);
  } else {
    gload(S0{}, 0);
    sstore(S0{}, S0{}, 0);
    __syncthreads();
    int kt = 0;
    for (; kt < KT - 2; kt += 2) {
      gload(S0{}, kt + 1);
      __builtin_amdgcn_sched_barrier(0);
      step(S0{}, S1{}, S0{}, kt, true);  // compute stage 0, store step kt+1 -> stage 1
      chunk_end(kt);
      __syncthreads();
      gload(S0{}, kt + 2);
      __builtin_amdgcn_sched_barrier(0);
      step(S1{}, S0{}, S0{}, kt + 1, true);  // compute stage 1, store step kt+2 -> stage 0
      chunk_end(kt + 1);
      __syncthreads();
    }
    gload(S0{}, kt + 1);
    __builtin_amdgcn_sched_barrier(0);
    step(S0{}, S1{}, S0{}, kt, true);
    chunk_end(kt);
    __syncthreads();
    step(S1{}, S0{}, S0{}, kt + 1, false);
    chunk_end(kt + 1);
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
// Large-M GEMM on the resident f16 copy of the weights (RNE of the dequantisation, made once at
// upload, as the reference's PreDequant does in f32): both operands are plain f16, so both tiles
// go global -> LDS by buffer_load ... lds (LDS-DMA: no VGPR staging, no ds_write, no VALU), and
// the loads of K step kt+1 fly while step kt's MFMAs run. LDS layout, fragment reads, MFMA
// sequence, chunk totals and epilogue are gemm_big's, so every output bit is the same.
// One LDS-DMA instruction moves 1 KB = 8 tile rows; lane L fills slot L % 8 of row L / 8, so it
// fetches the logical 16-byte chunk (L % 8) ^ (row & 7) (the XOR swizzle applied on the load).
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from the buffer into LDS at lds + 16 * lane (one 1-KB row group per wave).
// Written as inline assembly: the compiler's wait-count pass tracks at most a few LDS-DMA
// stores and otherwise waits for all of them before every LDS read, which would serialise a
// multi-stage pipeline. The kernel orders these loads itself (s_waitcnt vmcnt + s_barrier).
typedef unsigned int u32x4_sgpr __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void dma16(u32x4_sgpr r, void* lds, int voff, int soff) {
  const uint32_t base = (uint32_t)(uintptr_t)(lds_ptr_t)lds;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(base), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}
// Buffer descriptor as four SGPRs: base, stride 0, num_records = 2^32 - 1, default format.
__device__ __forceinline__ u32x4_sgpr rsrc_words(const void* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return u32x4_sgpr{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, 0xffffffffu, 0x00020000u};
}

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_b64(__amdgpu_buffer_rsrc_t r, int off, uint32_t lo, uint32_t hi) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{lo, hi}, r, off, 0, 0);
}
__device__ __forceinline__ void st_b16(__amdgpu_buffer_rsrc_t r, int off, __half v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, off, 0, 0);
}

// Sequence and position of the token rows mb + j*16 + (lane & 15) of a QKV wave tile, computed
// once per tile for both the RoPE operand loads and the stores (rows past M use row M-1; their
// results are never stored).
template <int TB>
__device__ __forceinline__ void qkv_rows(const GemmP& p, int mb, int lane, int (&bs)[TB], int (&ps)[TB]) {
#pragma unroll
  for (int j = 0; j < TB; j++) {
    const int m = min(mb + j * 16 + (lane & 15), p.M - 1);
    const int r = p.tokrow ? p.tokrow[m] : m;
    bs[j] = r / p.L;
    ps[j] = r - bs[j] * p.L;
  }
}

// The RoPE cos/sin pairs of epi_operands<EPI_QKV> for a wave tile: the section of each 16-feature
// fragment (wave-uniform: fb is) is decided once per fragment, the position once per token row.
template <int FB, int TB>
__device__ __forceinline__ void qkv_rope_operands(const GemmP& p, const int (&ps)[TB], int fb, int lane,
                                                  floatx4 (&eop)[FB][TB]) {
  const int D = p.D, lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < FB; i++) {
    const int f0 = fb + i * 16;
    const int sec = f0 >= 2 * D ? 2 : (f0 >= D ? 1 : 0);
    const int e = (f0 - sec * D + lg * 4) & 63;
#pragma unroll
    for (int j = 0; j < TB; j++) {
      if (sec < 2) {
        const float2 c = *(const float2*)(p.rope_cos + ps[j] * 32 + (e >> 1));
        const float2 sn = *(const float2*)(p.rope_sin + ps[j] * 32 + (e >> 1));
        eop[i][j] = floatx4{c.x, sn.x, c.y, sn.y};
      } else {
        eop[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
}

// The QKV epilogue of a large-GEMM wave tile (features fb.., tokens mb..): the arithmetic of
// epilogue_with<EPI_QKV>, with the section / head split done once per 16-feature fragment (the
// fragment lies inside one head: D % 64 == 0), the (sequence, position) of each token row from
// qkv_rows, and 32-bit buffer offsets instead of 64-bit pointers.
template <int FB, int TB>
__device__ __forceinline__ void qkv_tile(const GemmP& p, const floatx4 (&acc)[FB][TB], const floatx4 (&eop)[FB][TB],
                                         const int (&bs)[TB], const int (&ps)[TB], int mb, int fb, int lane) {
  const int lr = lane & 15, lg = lane >> 4;
  const int D = p.D, Lp = p.Lp, H = p.H, M = p.M;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q), rk = make_rsrc(p.k), rv = make_rsrc(p.vt);
#pragma unroll
  for (int i = 0; i < FB; i++) {
    const int f0 = fb + i * 16;  // wave-uniform
    const int sec = f0 >= 2 * D ? 2 : (f0 >= D ? 1 : 0);
    const int fi = f0 - sec * D + lg * 4, h = fi >> 6, e = fi & 63;
#pragma unroll
    for (int j = 0; j < TB; j++) {
      if (mb + j * 16 + lr >= M) continue;
      floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
      v += acc[i][j];  // total = 0 + chunk
      if (sec < 2) {
        const floatx4 o = eop[i][j];
        const float c0 = o.x, s0 = o.y, c1 = o.z, s1 = o.w;
        const float a0 = v.x * c0 - v.y * s0, a1 = v.x * s0 + v.y * c0;
        const float a2 = v.z * c1 - v.w * s1, a3 = v.z * s1 + v.w * c1;
        const __half2 lo = __floats2half2_rn(a0, a1), hi = __floats2half2_rn(a2, a3);
        const int off = (((bs[j] * H + h) * Lp + ps[j]) * 64 + e) * 2;
        st_b64(sec == 0 ? rq : rk, off, __builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
      } else {
        const int off = (((bs[j] * H + h) * 64 + e) * Lp + ps[j]) * 2;
        st_b16(rv, off, __float2half_rn(v.x));
        st_b16(rv, off + Lp * 2, __float2half_rn(v.y));
        st_b16(rv, off + Lp * 4, __float2half_rn(v.z));
        st_b16(rv, off + Lp * 6, __float2half_rn(v.w));
      }
    }
  }
}

// qkv_tile with the RoPE cos / sin rows of the block's 256 tokens staged in LDS (rope: cos rows
// [256][32] f32, then sin rows; logical 16-byte chunk c of row r at slot c ^ (r & 7)) instead of
// held in registers; rl0 is the wave tile's first row in the block. Same arithmetic and stores.
template <int FB, int TB>
__device__ __forceinline__ void qkv_tile_lds(const GemmP& p, const floatx4 (&acc)[FB][TB], const float* rope,
                                             const int (&bs)[TB], const int (&ps)[TB], int rl0, int mb, int fb,
                                             int lane) {
  const int lr = lane & 15, lg = lane >> 4;
  const int D = p.D, Lp = p.Lp, H = p.H, M = p.M;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(p.q), rk = make_rsrc(p.k), rv = make_rsrc(p.vt);
#pragma unroll
  for (int i = 0; i < FB; i++) {
    const int f0 = fb + i * 16;  // wave-uniform
    const int sec = f0 >= 2 * D ? 2 : (f0 >= D ? 1 : 0);
    const int fi = f0 - sec * D + lg * 4, h = fi >> 6, e = fi & 63;
#pragma unroll
    for (int j = 0; j < TB; j++) {
      if (mb + j * 16 + lr >= M) continue;
      floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
      v += acc[i][j];  // total = 0 + chunk
      if (sec < 2) {
        const int rl = rl0 + j * 16 + lr;
        const int o = rl * 32 + (((e >> 3) ^ (rl & 7)) << 2) + ((e >> 1) & 3);  // floats e/2, e/2 + 1
        const float2 c = *(const float2*)(rope + o);
        const float2 sn = *(const float2*)(rope + 256 * 32 + o);
        const float c0 = c.x, s0 = sn.x, c1 = c.y, s1 = sn.y;
        const float a0 = v.x * c0 - v.y * s0, a1 = v.x * s0 + v.y * c0;
        const float a2 = v.z * c1 - v.w * s1, a3 = v.z * s1 + v.w * c1;
        const __half2 lo = __floats2half2_rn(a0, a1), hi = __floats2half2_rn(a2, a3);
        const int off = (((bs[j] * H + h) * Lp + ps[j]) * 64 + e) * 2;
        st_b64(sec == 0 ? rq : rk, off, __builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
      } else {
        const int off = (((bs[j] * H + h) * 64 + e) * Lp + ps[j]) * 2;
        st_b16(rv, off, __float2half_rn(v.x));
        st_b16(rv, off + Lp * 2, __float2half_rn(v.y));
        st_b16(rv, off + Lp * 4, __float2half_rn(v.z));
        st_b16(rv, off + Lp * 6, __float2half_rn(v.w));
      }
    }
  }
}

// LDS rows are 64 bytes (4 chunks of 16 B); chunk c of row r sits at c ^ swr(r), which spreads
// a 16-row fragment read over all banks.
__device__ __forceinline__ int swr(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

// Epilogue of one LDS-DMA wave tile (tokens mb.., features fb..): the QKV scatter, or the
// per-fragment epilogue of the other EPIs on the chunk total (MULTI) or 0 + the single chunk.
template <int EPI, bool MULTI, int FB, int TB, int TF, int TT, int PF, int PT, int QT>
__device__ __forceinline__ void tile_epilogue(const GemmP& p, const floatx4 (&acc)[FB][TB],
                                              const floatx4 (&tot)[TF][TT], const floatx4 (&eop)[PF][PT],
                                              const int (&qb)[QT], const int (&qp)[QT], int mb, int fb, int lane) {
  if constexpr (EPI == EPI_QKV && !MULTI) {
    qkv_tile<FB, TB>(p, acc, eop, qb, qp, mb, fb, lane);
  } else {
    const int lr = lane & 15;
#pragma unroll
    for (int j = 0; j < TB; j++) {
      const int m = mb + j * 16 + lr;
      if (m < p.M) {
#pragma unroll
        for (int i = 0; i < FB; i++) {
          floatx4 v;
          if constexpr (MULTI) {
            v = tot[i][j];
          } else {
            v = floatx4{0.f, 0.f, 0.f, 0.f};
            v += acc[i][j];  // total = 0 + chunk, as the split-K reduction computes it
          }
          if constexpr (EPI == EPI_QKV)
            epilogue_with<EPI>(p, m, fb + i * 16 + (lane >> 4) * 4, v, eop[i][j]);
          else
            epilogue<EPI>(p, m, fb + i * 16 + (lane >> 4) * 4, v);
        }
      }
    }
  }
}

// XCD-aware tile order of the LDS-DMA kernels (as gemm_big's): workgroup b runs on XCD b % 8,
// so the tile grid is cut into MG x NG shares, one per XCD, each walked N-fastest; concurrently
// running tiles of one XCD then share their X and W rows in its L2. 256-wide tiles use 4 N
// groups: each XCD's weight share (6 of up||gate's 24 column tiles, 2.4 MB) then stays in its
// L2 between rounds; measured at the same speed as 2 groups with a third fewer bytes fetched
// past L2 (FETCH_SIZE per launch 307 -> 209 MiB-equivalent counts).
template <int BM, int BN>
__device__ __forceinline__ void xcd_tile(int& m0, int& n0) {
  constexpr int NG = BN >= 256 ? 4 : 1, MG = 8 / NG;
  const int nt = gridDim.x, mt = gridDim.y, G = nt * mt;
  const int b = blockIdx.x + blockIdx.y * nt, xcd = b & 7, slot = b >> 3;
  n0 = blockIdx.x * BN;
  m0 = blockIdx.y * BM;
  if (nt % NG == 0 && mt % MG == 0) {
    const int ntl = nt / NG, mtl = mt / MG;
    n0 = ((xcd % NG) * ntl + slot % ntl) * BN;
    m0 = ((xcd / NG) * mtl + slot / ntl) * BM;
  } else {  // each XCD takes a contiguous run of the row-major tile order
    const int q = G >> 3, r = G & 7;
    const int t = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
    n0 = (t % nt) * BN;
    m0 = (t / nt) * BM;
  }
}

template <int BM, int BN, int WM, int WN, int NS, int EPI, bool MULTI>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_h(GemmP p) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN, FB = TN / 16, TB = TM / 16;
  // 1-KB loads per wave per K step; with BN = 288 the 36 W row groups are 5 per wave for waves
  // 0-3 and 4 for waves 4-7
  constexpr int XI = BM / 8 / NW, WI = (BN / 8 + NW - 1) / NW;
  static_assert(BM % (8 * NW) == 0 && BN % 8 == 0, "tile rows per wave");
  static_assert(NS == 2 || NS == 3, "stages");
  // NS stages of [BM X rows | BN W rows] x 128 bytes in one LDS array (stage offsets are
  // compile-time constants); after the K loop the array stages the epilogue's tile
  constexpr int X_STAGE = BM * KSTEP * 2, STAGE = X_STAGE + BN * KSTEP * 2;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * STAGE];
  typedef _Float16 KRow[KSTEP];
  auto stX = [&](auto S) { return (KRow*)(smem + decltype(S)::value * STAGE); };
  auto stW = [&](auto S) { return (KRow*)(smem + decltype(S)::value * STAGE + X_STAGE); };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int m0, n0;
  xcd_tile<BM, BN>(m0, n0);
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

  // The RoPE epilogue's cos/sin pairs are loaded before the K loop (their latency then hides
  // behind it; issued after the first LDS-DMA loads would break the vmcnt accounting below,
  // which counts on every older memory operation being complete). Rows past M load row M-1.
  // 256 x 256 QKV tiles (one section each: D % 256 == 0) cannot hold these operands beside
  // their accumulators; their cos / sin rows are brought into the stage the last K step leaves
  // free (ROPE_LDS) and read from LDS in the epilogue.
  constexpr bool QKV = EPI == EPI_QKV && !MULTI;
  constexpr bool ROPE_LDS = QKV && BM == 256 && (BN == 256 || BN == 288) && NS == 2;
  static_assert((BN / 8) % NW == 0 || NS == 2, "uneven W loads: the vmcnt accounting assumes 2 stages");
  constexpr bool PRE = EPI == EPI_QKV && !ROPE_LDS;
  floatx4 eop[PRE ? FB : 1][PRE ? TB : 1];
  int qb[(PRE || QKV) ? TB : 1], qp[(PRE || QKV) ? TB : 1];
  if constexpr (PRE) {
    qkv_rows<TB>(p, m0 + wm * TM, lane, qb, qp);
    qkv_rope_operands<FB, TB>(p, qp, n0 + wn * TN, lane, eop);
  }
  const int rsec = n0 >= 2 * p.D ? 2 : (n0 >= p.D ? 1 : 0);  // ROPE_LDS: the tile's section

  // loop-invariant byte offsets; the K step advances in the scalar offset. Rows past M re-read
  // row M-1 (they only feed output rows that are never stored).
  const u32x4_sgpr rx = rsrc_words(p.x), rw = rsrc_words(p.w16);
  // An uneven W share (BN = 288) keeps one vector offset, the row group's distance in the
  // scalar offset: rows j * NW * 8 apart have the same swizzle (r & 7), and five vector offsets
  // beside 144 accumulators spilled.
  constexpr bool W1 = (BN / 8) % NW != 0;
  int xo[XI], wo[W1 ? 1 : WI];
#pragma unroll
  for (int j = 0; j < XI; j++) {
    const int r = (wave + j * NW) * 8 + (lane >> 3), c = (lane & 7) ^ (r & 7);
    xo[j] = (min(m0 + r, M - 1) * K + c * 8) * 2;
  }
#pragma unroll
  for (int j = 0; j < (W1 ? 1 : WI); j++) {
    const int r = (wave + j * NW) * 8 + (lane >> 3), c = (lane & 7) ^ (r & 7);
    wo[j] = ((n0 + r) * K + c * 8) * 2;
  }
  auto issue = [&](auto S, int kt) {
    KRow* sx = stX(S);
    KRow* sw = stW(S);
#pragma unroll
    for (int j = 0; j < XI; j++) dma16(rx, &sx[(wave + j * NW) * 8][0], xo[j], kt * KSTEP * 2);
#pragma unroll
    for (int j = 0; j < WI; j++) {
      if constexpr (W1) {
        if (wave + j * NW < BN / 8)  // wave-uniform
          dma16(rw, &sw[(wave + j * NW) * 8][0], wo[0], (j * NW * 8 * K + kt * KSTEP) * 2);
      } else {
        dma16(rw, &sw[(wave + j * NW) * 8][0], wo[j], kt * KSTEP * 2);
      }
    }
  };
  const int lr = lane & 15, lg = lane >> 4;
  auto compute = [&](auto S, int kt) {
    const KRow* sw = stW(S);
    const KRow* sx = stX(S);
    half8 af[2][FB], bf[2][TB];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int i = 0; i < FB; i++) af[ks][i] = *(const half8*)&sw[wn * TN + i * 16 + lr][swz(lr, ks * 4 + lg) * 8];
#pragma unroll
      for (int j = 0; j < TB; j++) bf[ks][j] = *(const half8*)&sx[wm * TM + j * 16 + lr][swz(lr, ks * 4 + lg) * 8];
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int i = 0; i < FB; i++)
#pragma unroll
        for (int j = 0; j < TB; j++) acc[i][j] = mfma16(af[ks][i], bf[ks][j], acc[i][j]);
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
  };
  // NS LDS stages, loads issued NS-1 K steps ahead (KT % NS == 0). At the top of step kt each
  // wave waits until only the loads of the NS-2 younger steps are in flight (its step-kt loads
  // have landed) and its LDS reads are done; the barrier then makes every wave's step-kt data
  // visible and frees the stage of step kt-1 for the loads of step kt+NS-1. s_barrier is used
  // bare (with compiler-only fences): __syncthreads() would also wait for every load in flight.
  constexpr int PER_STEP = XI + WI;  // LDS-DMA instructions per wave per K step
  constexpr int VM = (NS - 2) * PER_STEP;
  static_assert(VM < 64, "vmcnt range");
  constexpr int WAIT = (VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4);  // vmcnt(VM) lgkmcnt(0)
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  auto step = [&](auto S, auto SN, int kt) {  // SN: the stage of step kt + NS - 1
    if (kt + NS - 2 < KT)
      __builtin_amdgcn_s_waitcnt(WAIT);
    else
      __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + NS - 1 < KT) {
      issue(SN, kt + NS - 1);
    } else if constexpr (ROPE_LDS) {
      if (kt == KT - 1 && rsec < 2) {  // SN (stage 0) was last read by step kt - 1
        // instruction j of wave w fills tile rows (4 w + j) * 8 + lane / 8 with the cos / sin
        // row of that token's position (rows past M: row M - 1), the lane fetching the logical
        // 16-byte chunk (lane % 8) ^ (row & 7)
        const u32x4_sgpr rc = rsrc_words(p.rope_cos), rs = rsrc_words(p.rope_sin);
        float* rope = (float*)(smem + decltype(SN)::value * STAGE);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int r = (wave * 4 + j) * 8 + (lane >> 3);
          const int m = min(m0 + r, M - 1);
          const int t = p.tokrow ? p.tokrow[m] : m;
          const int ro = ((t - (t / p.L) * p.L) * 32 + (((lane & 7) ^ (r & 7)) << 2)) * 4;
          dma16(rc, rope + (wave * 4 + j) * 8 * 32, ro, 0);
          dma16(rs, rope + 256 * 32 + (wave * 4 + j) * 8 * 32, ro, 0);
        }
      }
    }
    compute(S, kt);
  };
  issue(S0{}, 0);
  if constexpr (NS == 3) issue(S1{}, 1);
  for (int kt = 0; kt < KT; kt += NS) {
    if constexpr (NS == 2) {
      step(S0{}, S1{}, kt);
      step(S1{}, S0{}, kt + 1);
    } else {
      step(S0{}, S2{}, kt);
      step(S1{}, S0{}, kt + 1);
      step(S2{}, S1{}, kt + 2);
    }
  }
  if constexpr (ROPE_LDS) {
    qkv_rows<TB>(p, m0 + wm * TM, lane, qb, qp);
    if (rsec < 2) {  // wave-uniform: every wave's RoPE rows have landed
      __builtin_amdgcn_s_waitcnt(0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    qkv_tile_lds<FB, TB>(p, acc, (const float*)smem, qb, qp, wm * TM, m0 + wm * TM, n0 + wn * TN, lane);
    return;
  }

  if constexpr (EPI == EPI_GEGLU && BM == 256 && BN == 256 && WM == 4 && WN == 2 && !MULTI) {
    // GeGLU outputs go through LDS so that every global store is a full 16-byte chunk of a row
    // (8 lanes per 128-byte line): stored straight from the MFMA layout, each instruction wrote
    // 16 rows x 16 bytes and the stores took a sixth of the kernel. The 256 x 128 f16 tile:
    // chunk c of row r at c ^ (r & 15) (the low bits of a 16-row fragment's row).
    typedef _Float16 ORow[128];
    static_assert(sizeof(smem) >= 256 * sizeof(ORow), "staging");
    __syncthreads();  // every wave is done reading the last stage
    ORow* so = (ORow*)smem + (wm >> 1) * 128;
#pragma unroll
    for (int j = 0; j < TB; j++) {
      const int r = (wm & 1) * 64 + j * 16 + lr;
#pragma unroll
      for (int i = 0; i < FB; i++) {
        floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
        v += acc[i][j];  // total = 0 + chunk, as epilogue<EPI_GEGLU> receives it
        const float o0 = gelu_r(v.y) * v.x, o1 = gelu_r(v.w) * v.z;
        *(__half2*)&so[r][((wn * 8 + i) ^ (r & 15)) * 8 + lg * 2] = __floats2half2_rn(o0, o1);
      }
    }
    __syncthreads();
    const int F = p.N >> 1;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int q = tid + k * 512, row = q >> 4, c = q & 15, rr = row & 127;
      const uint4 val = *(const uint4*)&((const ORow*)smem)[row][(c ^ (rr & 15)) * 8];
      if (m0 + row < M)  // streaming store: measured faster than a cached one for this 200 MB output
        __builtin_nontemporal_store(u32x4_sgpr{val.x, val.y, val.z, val.w},
                                    (u32x4_sgpr*)(p.g + (size_t)(m0 + row) * F + (n0 >> 1) + c * 8));
    }
    return;
  }
  if constexpr (EPI == EPI_RESID && (BM == 256 || BM == 128) && BN == 128 && WM == 4 && WN == 2) {
    // h += X W^T through LDS: the f32 tile totals are staged (row r's 16-byte chunk c at
    // c ^ (r & 31)), then each thread reads 16 bytes of residual, adds and stores whole row chunks
    // (32 lanes per 512-byte row) instead of 16 rows x 64 bytes per instruction.
    typedef float TRow[128];
    static_assert(sizeof(smem) >= BM * sizeof(TRow), "staging");
    // all BM / 16 residual chunks of this thread are loaded first (rows past M: the last row,
    // never stored), so their one round trip overlaps the staging; the barriers below wait for
    // LDS only and leave them in flight
    const int N = p.N;
    constexpr int RC = BM / 16;
    floatx4 res[RC];
#pragma unroll
    for (int k = 0; k < RC; k++) {
      const int q = tid + k * 512, row = q >> 5, c = q & 31;
      res[k] = *(const floatx4*)(p.y + (size_t)min(m0 + row, M - 1) * N + n0 + c * 4);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): every wave is done reading the last stage
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    TRow* so = (TRow*)smem;
#pragma unroll
    for (int j = 0; j < TB; j++) {
      const int r = wm * TM + j * 16 + lr;
#pragma unroll
      for (int i = 0; i < FB; i++) {
        floatx4 v;
        if constexpr (MULTI) {
          v = tot[i][j];
        } else {
          v = floatx4{0.f, 0.f, 0.f, 0.f};
          v += acc[i][j];  // total = 0 + chunk, as the split-K reduction computes it
        }
        *(floatx4*)&so[r][((wn * 16 + i * 4 + lg) ^ (r & 31)) * 4] = v;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < RC; k++) {
      const int q = tid + k * 512, row = q >> 5, c = q & 31;
      const floatx4 v = *(const floatx4*)&so[row][(c ^ (row & 31)) * 4];
      // hiddens[i][j] += out[i][j]  (internal/embed/bert.go:262-264, 276-278)
      floatx4 h = res[k];
      h.x = h.x + v.x; h.y = h.y + v.y; h.z = h.z + v.z; h.w = h.w + v.w;
      if (m0 + row < M) __builtin_nontemporal_store(h, (floatx4*)(p.y + (size_t)(m0 + row) * N + n0 + c * 4));
    }
    return;
  }
  if constexpr (!ROPE_LDS) tile_epilogue<EPI, MULTI, FB, TB>(p, acc, tot, eop, qb, qp, m0 + wm * TM, n0 + wn * TN, lane);
}

// ---------------------------------------------------------------------------------------
// Full-row GEMM + residual + LayerNorm (h = LN(h + X W^T)) for N = 768: one block owns BM
// complete rows, so the LayerNorm runs in the epilogue instead of a second pass over h.
// 8 waves, each 96 features x BM tokens (6 x BM/16 MFMA tiles). K steps of 32 (one MFMA deep):
// the whole 768-row weight step is 48 KB of LDS, double-buffered. The per-accumulator MFMA
// sequence, the chunk totals, the residual add and ln_row are those of gemm_big + ln_kernel,
// so every output bit equals that path's (and the small-M path's).

constexpr int LN_N = 768, LN_KS = 32, LN_RS = LN_N + 4;  // LN staging row stride (floats)

// Epilogue of the full-row kernels: x = h + total (the residual epilogue's add) staged per 32
// tokens in LDS (row stride 772 floats: conflict-free), then LayerNorm by ln_row with
// ln_kernel's element-to-lane mapping (wave w: 4 rows per half). Call after a barrier that
// ends every read of the K-loop stages, which smem overlays.
template <int BM, bool DEFER = false>
__device__ __forceinline__ void rowln_finish(const floatx4 (&acc)[6][BM / 16], unsigned char* smem, const GemmP& p,
                                             const float* __restrict__ lnw, const float* __restrict__ lnb,
                                             float eps, __half* h16, int m0, int wn, int lane, const LnDefer& dfr) {
  constexpr int FB = 6, TN = 96;
  const int lr = lane & 15, lg = lane >> 4, M = p.M;
  float* sR = (float*)smem;
#pragma unroll
  for (int half = 0; half < BM / 32; half++) {
#pragma unroll
    for (int j = 2 * half; j < 2 * half + 2; j++) {
      const int tl = (j - 2 * half) * 16 + lr, m = m0 + j * 16 + lr;
#pragma unroll
      for (int i = 0; i < FB; i++) {
        const int f = wn * TN + i * 16 + lg * 4;
        floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
        v += acc[i][j];  // total = 0 + chunk
        floatx4 x = floatx4{0.f, 0.f, 0.f, 0.f};
        if (m < M) {
          floatx4 h = *(const floatx4*)(p.y + (size_t)m * LN_N + f);
          if constexpr (DEFER) {  // finish the pending LayerNorm of the residual (ln_elem)
            const float2 rs = dfr.stats[m];
            const floatx4 pw = *(const floatx4*)(dfr.w + f), pb = *(const floatx4*)(dfr.b + f);
            h.x = ln_elem(h.x, rs.x, rs.y, pw.x, pb.x);
            h.y = ln_elem(h.y, rs.x, rs.y, pw.y, pb.y);
            h.z = ln_elem(h.z, rs.x, rs.y, pw.z, pb.z);
            h.w = ln_elem(h.w, rs.x, rs.y, pw.w, pb.w);
          }
          x.x = h.x + v.x; x.y = h.y + v.y; x.z = h.z + v.z; x.w = h.w + v.w;
        }
        *(floatx4*)&sR[tl * LN_RS + f] = x;
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int tl = wn * 4 + r, m = m0 + half * 32 + tl;
      if (m < M) {
        float x[MAXE];
#pragma unroll
        for (int i = 0; i < MAXE; i++)
          if (i < LN_N / 64) x[i] = sR[tl * LN_RS + lane + 64 * i];
        ln_row(x, LN_N / 64, LN_N, lnw, lnb, eps, lane, p.y + (size_t)m * LN_N, h16 + (size_t)m * LN_N);
      }
    }
    __syncthreads();
  }
}

template <int FMT, int BM, bool DEFER = false>
__global__ __launch_bounds__(512, 1) void gemm_rowln(GemmP p, const float* __restrict__ lnw,
                                                     const float* __restrict__ lnb, float eps, __half* h16,
                                                     LnDefer dfr) {
  constexpr int NT = 512, WN = 8, TN = LN_N / WN, FB = TN / 16, TB = BM / 16;
  constexpr int WU = LN_N * (LN_KS / 16);  // 1536 weight segments per step
  constexpr int WPT = WU / NT;             // 3
  constexpr int XCH = BM * (LN_KS / 8);    // 16-byte X chunks per step
  constexpr int W_BYTES = 2 * LN_N * LN_KS * 2, X_BYTES = 2 * BM * LN_KS * 2;
  constexpr int R_BYTES = 32 * LN_RS * 4;
  constexpr int SMEM = (W_BYTES + X_BYTES) > R_BYTES ? (W_BYTES + X_BYTES) : R_BYTES;
  static_assert(WU % NT == 0 && XCH <= NT, "tile loads");
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  typedef _Float16 WStage[LN_N][LN_KS];
  typedef _Float16 XStage[BM][LN_KS];
  WStage* sW = (WStage*)smem;
  XStage* sX = (XStage*)(smem + W_BYTES);

  const int tid = threadIdx.x, lane = tid & 63, wn = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.x * BM;
  const int M = p.M, K = p.K;
  const int KT = K / LN_KS;

  floatx4 acc[FB][TB];
#pragma unroll
  for (int i = 0; i < FB; i++)
#pragma unroll
    for (int j = 0; j < TB; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x);
  const WRsrc rw{make_rsrc(p.w.p0), make_rsrc(p.w.p1), make_rsrc(p.w.p2), make_rsrc(p.w.p3)};
  // X chunk c (threads c < XCH): row c / 4, 8 halves at k = (c % 4) * 8; rows past M re-read M-1
  const bool xload = tid < XCH;
  const int xrow = tid >> 2, xch = tid & 3;
  const int xoff = (min(m0 + xrow, M - 1) * K + xch * 8) * 2;
  // W segment u = tid + i * NT: row u % 768, segment u / 768 of the 32-wide step; within the
  // 64-wide plane step that is segment 2 * (step & 1) + u / 768
  SegOff woff[2][WPT];
#pragma unroll
  for (int i = 0; i < WPT; i++) {
    const int u = tid + i * NT;
    woff[0][i] = seg_off<FMT>(LN_N, K, u % LN_N, u / LN_N);
    woff[1][i] = seg_off<FMT>(LN_N, K, u % LN_N, 2 + u / LN_N);
  }

  uint4 xr[2];
  RawSeg wr[2][WPT];
  // set s holds 32-wide step kt, kt % 2 == s
  auto gload = [&](auto S, int kt) {
    constexpr int s = decltype(S)::value;
    if (xload) xr[s] = buf_load16(rx, xoff, kt * LN_KS * 2);
#pragma unroll
    for (int i = 0; i < WPT; i++) wr[s][i] = load_seg_buf<FMT>(rw, woff[s][i], LN_N, kt >> 1);
  };
  auto sstore = [&](auto S, int kt) {  // register set S (= step kt) -> LDS stage S
    constexpr int s = decltype(S)::value;
    if (xload) *(uint4*)&sX[s][xrow][(xch ^ swr(xrow)) * 8] = xr[s];
#pragma unroll
    for (int i = 0; i < WPT; i++) {
      const int u = tid + i * NT, row = u % LN_N, sg = u / LN_N;
      uint4 lo, hi;
      decode_seg_h<FMT>(wr[s][i], kt * LN_KS + sg * 16, lo, hi);
      *(uint4*)&sW[s][row][((2 * sg) ^ swr(row)) * 8] = lo;
      *(uint4*)&sW[s][row][((2 * sg + 1) ^ swr(row)) * 8] = hi;
    }
  };
  // compute stage S (step kt); store register set SN (step kt + 1) into stage SN on the way
  auto step = [&](auto S, auto SN, int kt, bool store_next) {
    constexpr int s = decltype(S)::value;
    half8 af[FB], bf[TB];
#pragma unroll
    for (int i = 0; i < FB; i++) {
      const int f = wn * TN + i * 16 + lr;
      af[i] = *(const half8*)&sW[s][f][(lg ^ swr(f)) * 8];
    }
#pragma unroll
    for (int j = 0; j < TB; j++) {
      const int t = j * 16 + lr;
      bf[j] = *(const half8*)&sX[s][t][(lg ^ swr(t)) * 8];
    }
#pragma unroll
    for (int i = 0; i < FB; i++)
#pragma unroll
      for (int j = 0; j < TB; j++) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
    if (store_next) sstore(SN, kt + 1);
    __builtin_amdgcn_sched_group_barrier(0x100, FB + TB, 0);
#pragma unroll
    for (int i = 0; i < FB * TB; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  // KT is even (K % 64 == 0); pairs of steps keep stage indices compile-time constants, and the
  // last pair is peeled so that every in-loop path issues the same loads.
  gload(S0{}, 0);
  gload(S1{}, 1);
  sstore(S0{}, 0);
  __syncthreads();
  int kt = 0;
  for (; kt < KT - 2; kt += 2) {
    gload(S0{}, kt + 2);
    __builtin_amdgcn_sched_barrier(0);
    step(S0{}, S1{}, kt, true);
    __syncthreads();
    gload(S1{}, kt + 3);
    __builtin_amdgcn_sched_barrier(0);
    step(S1{}, S0{}, kt + 1, true);
    __syncthreads();
  }
  step(S0{}, S1{}, kt, true);
  __syncthreads();
  step(S1{}, S0{}, kt + 1, false);
  __syncthreads();  // every stage read: LDS is free for the row staging

  rowln_finish<BM, DEFER>(acc, smem, p, lnw, lnb, eps, h16, m0, wn, lane, dfr);
}

// Epilogue of the LDS-DMA full-row kernel, in 16-token slabs. Slab s's residual rows
// (16 x 768 f32) are brought into LDS by LDS-DMA (two buffers, row stride LN_RS floats) while
// the previous slab is normalised, the accumulators are added in place (x = h + (0 + total), as
// rowln_finish), and each wave normalises two rows with ln_row's arithmetic, so every bit equals
// rowln_finish's. The waits count this wave's younger memory operations exactly: slab s + 1's six
// DMA instructions and the 24 stores of each of its two rows of slab s - 1 (a skipped row past M
// stores nothing, which only makes the wait stricter).
// DEFER: the residual rows hold a pending LayerNorm (LnDefer): its weights and the block's row
// statistics come into LDS with the slab-0 weights, and each residual element read from a slab
// is first finished with ln_elem, which gives the f32 bits ln_kernel would have stored.
template <int BM, bool DEFER = false>
__device__ __forceinline__ void rowln_finish_dma(const floatx4 (&acc)[6][BM / 16], unsigned char* smem, const GemmP& p,
                                                 const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                 float eps, __half* h16, int m0, int wn, int lane, const LnDefer& dfr) {
  // the statistics come as one 1 KB LDS-DMA from row m0: 128 rows (64-row blocks read the next
  // 64 rows' too, unused; the statistics buffer extends 128 rows past the last row)
  static_assert(!DEFER || BM == 128 || BM == 64, "one statistics DMA per block");
  constexpr int FB = 6, TN = 96, NE = LN_N / 64, NSL = BM / 16;
  constexpr int SLAB = 16 * LN_RS * 4;  // bytes of one slab buffer
  constexpr int DMA_PER = 6;             // 48 KB-instructions per slab over 8 waves
  constexpr int ST = 2 * 2 * NE;         // stores per lane per slab: two rows, f32 + f16 each
  static_assert(NE == 12 && DMA_PER + ST < 64, "vmcnt range");
  const int lr = lane & 15, lg = lane >> 4, M = p.M;
  const u32x4_sgpr ry = rsrc_words(p.y);
  auto slab = [&](int s) { return (float*)(smem + (s & 1) * SLAB); };
  // instruction t of wave w moves the 1 KB part (6w + t) % 3 of slab row (6w + t) / 3 (rows
  // past M read row M - 1: they are never stored)
  auto dma_slab = [&](int s) {
    float* buf = slab(s);
#pragma unroll
    for (int t = 0; t < DMA_PER; t++) {
      const int idx = wn * DMA_PER + t, row = idx / 3, part = idx - row * 3;
      const int m = min(m0 + s * 16 + row, M - 1);
      dma16(ry, buf + row * LN_RS + part * 256, lane * 16, (m * LN_N + part * 256) * 4);
    }
  };
  auto wait_bar = [&](auto VMC) {
    constexpr int V = decltype(VMC)::value;
    __builtin_amdgcn_s_waitcnt((V & 0xF) | ((V >> 4) << 14) | (0x7 << 4));  // vmcnt(V) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // the LayerNorm weights and biases come into LDS with slab 0 (waves 0-5, one 1 KB part
  // each), so the epilogue has no global loads the compiler's wait counting would have to order
  // against the DMA
  // (DEFER: then the pending LayerNorm's weights and biases, and the block's rows of
  // {mean, invStd})
  float* sWB = (float*)(smem + 2 * SLAB);
  const float* sST = sWB + 4 * LN_N;
  float wv[MAXE], bv[MAXE];
  dma_slab(0);
  if (wn < 6) {
    const int part = wn % 3;
    dma16(rsrc_words(wn < 3 ? lnw : lnb), sWB + (wn / 3) * LN_N + part * 256, lane * 16, part * 1024);
    if constexpr (DEFER)
      dma16(rsrc_words(wn < 3 ? dfr.w : dfr.b), sWB + (2 + wn / 3) * LN_N + part * 256, lane * 16, part * 1024);
  } else if (DEFER && wn == 6) {
    dma16(rsrc_words(dfr.stats), sWB + 4 * LN_N, lane * 16, m0 * 8);
  }
#pragma unroll
  for (int s = 0; s < NSL; s++) {
    if (s + 1 < NSL) dma_slab(s + 1);  // its buffer was last read before the previous barrier
    if (s == 0)
      wait_bar(std::integral_constant<int, DMA_PER>{});
    else if (s + 1 < NSL)
      wait_bar(std::integral_constant<int, DMA_PER + ST>{});
    else
      wait_bar(std::integral_constant<int, ST>{});
    float* buf = slab(s);
    float2 rs;
    if constexpr (DEFER) rs = *(const float2*)(sST + (s * 16 + lr) * 2);
#pragma unroll
    for (int i = 0; i < FB; i++) {
      float* px = buf + lr * LN_RS + wn * TN + i * 16 + lg * 4;
      floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
      v += acc[i][s];  // total = 0 + chunk
      floatx4 h = *(const floatx4*)px;
      if constexpr (DEFER) {
        const int col = wn * TN + i * 16 + lg * 4;
        const floatx4 pw = *(const floatx4*)(sWB + 2 * LN_N + col), pb = *(const floatx4*)(sWB + 3 * LN_N + col);
        h.x = ln_elem(h.x, rs.x, rs.y, pw.x, pb.x);
        h.y = ln_elem(h.y, rs.x, rs.y, pw.y, pb.y);
        h.z = ln_elem(h.z, rs.x, rs.y, pw.z, pb.z);
        h.w = ln_elem(h.w, rs.x, rs.y, pw.w, pb.w);
      }
      floatx4 x;
      x.x = h.x + v.x; x.y = h.y + v.y; x.z = h.z + v.z; x.w = h.w + v.w;
      *(floatx4*)px = x;
    }
    wait_bar(std::integral_constant<int, 63>{});  // LDS only
    if (s == 0) {
#pragma unroll
      for (int i = 0; i < NE; i++) {
        wv[i] = sWB[lane + 64 * i];
        bv[i] = sWB[LN_N + lane + 64 * i];
      }
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int tl = wn * 2 + r, m = m0 + s * 16 + tl;
      if (m < M) {
        float x[MAXE];
#pragma unroll
        for (int i = 0; i < MAXE; i++)
          if (i < NE) x[i] = buf[tl * LN_RS + lane + 64 * i];
        ln_apply_wb(x, NE, LN_N, wv, bv, eps);
        float* hrow = p.y + (size_t)m * LN_N;
        __half* h16row = h16 + (size_t)m * LN_N;
#pragma unroll
        for (int i = 0; i < NE; i++) {
          hrow[lane + 64 * i] = x[i];
          h16row[lane + 64 * i] = __float2half_rn(x[i]);
        }
      }
    }
    if (s + 1 < NSL) wait_bar(std::integral_constant<int, 63>{});  // buffer s & 1 read by all
  }
}

// The full-row kernel on the resident f16 weights: both tiles by LDS-DMA (one instruction =
// 16 rows of 64 bytes; lane L fills slot L % 4 of row L / 4 with logical chunk (L % 4) ^ swr(row))
// through NS LDS stages (3 x 52 KB for 64 rows, 2 x 56 KB for 128), loads NS - 1 K steps ahead;
// MFMA order and epilogue as above.
template <int BM, int NS, bool DEFER = false>
__global__ __launch_bounds__(512, 1) void gemm_rowln_h(GemmP p, const float* __restrict__ lnw,
                                                       const float* __restrict__ lnb, float eps, __half* h16,
                                                       LnDefer dfr) {
  constexpr int WN = 8, TN = LN_N / WN, FB = TN / 16, TB = BM / 16;
  static_assert(NS == 2 || NS == 3, "stages");
  constexpr int W_STAGE = LN_N * LN_KS * 2, X_STAGE = BM * LN_KS * 2, STAGE = W_STAGE + X_STAGE;
  constexpr int WG = LN_N / 16 / WN;  // weight row groups per wave per step (6)
  constexpr int XG = BM / 16;         // X row groups per step (4): wave w loads group w % XG
  constexpr int PER_STEP = WG + 1;    // LDS-DMA instructions per wave per step
  constexpr int R_BYTES = 32 * LN_RS * 4;
  constexpr int SMEM = NS * STAGE > R_BYTES ? NS * STAGE : R_BYTES;
  static_assert(SMEM <= 160 * 1024, "LDS");
  static_assert(SMEM >= 2 * 16 * LN_RS * 4 + (DEFER ? 4 * LN_N * 4 + 1024 : 2 * LN_N * 4),
                "LDS of the epilogue's slabs and weights");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[SMEM];
  typedef _Float16 Row[LN_KS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wn = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.x * BM;
  const int M = p.M, K = p.K;
  const int KT = K / LN_KS;

  floatx4 acc[FB][TB];
#pragma unroll
  for (int i = 0; i < FB; i++)
#pragma unroll
    for (int j = 0; j < TB; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const u32x4_sgpr rx = rsrc_words(p.x), rw = rsrc_words(p.w16);
  int wo[WG];
#pragma unroll
  for (int g = 0; g < WG; g++) {
    const int r = (wn + g * WN) * 16 + (lane >> 2), c = (lane & 3) ^ swr(r);
    wo[g] = (r * K + c * 8) * 2;
  }
  const int xg = wn % XG;
  int xo;
  {
    const int r = xg * 16 + (lane >> 2), c = (lane & 3) ^ swr(r);
    xo = (min(m0 + r, M - 1) * K + c * 8) * 2;
  }
  auto stageW = [&](int s) { return (Row*)(smem + s * STAGE); };
  auto stageX = [&](int s) { return (Row*)(smem + s * STAGE + W_STAGE); };
  auto issue = [&](int s, int kt) {
    Row* sw = stageW(s);
#pragma unroll
    for (int g = 0; g < WG; g++) dma16(rw, &sw[(wn + g * WN) * 16][0], wo[g], kt * LN_KS * 2);
    dma16(rx, &stageX(s)[xg * 16][0], xo, kt * LN_KS * 2);  // waves w and w + 4 load the same rows
  };
  auto compute = [&](int s) {
    const Row* sw = stageW(s);
    const Row* sx = stageX(s);
    half8 af[FB], bf[TB];
#pragma unroll
    for (int i = 0; i < FB; i++) {
      const int f = wn * TN + i * 16 + lr;
      af[i] = *(const half8*)&sw[f][(lg ^ swr(f)) * 8];
    }
#pragma unroll
    for (int j = 0; j < TB; j++) {
      const int t = j * 16 + lr;
      bf[j] = *(const half8*)&sx[t][(lg ^ swr(t)) * 8];
    }
#pragma unroll
    for (int i = 0; i < FB; i++)
#pragma unroll
      for (int j = 0; j < TB; j++) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
  };
  constexpr int VM = (NS - 2) * PER_STEP;
  constexpr int WAIT = (VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4);  // vmcnt(VM) lgkmcnt(0)
  issue(0, 0);
  if constexpr (NS == 3) issue(1, 1);
  int stage = 0;
  for (int kt = 0; kt < KT; kt++) {  // as in gemm_h: wait for step kt's loads, barrier, refill
    if (kt + NS - 2 < KT)
      __builtin_amdgcn_s_waitcnt(WAIT);
    else
      __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + NS - 1 < KT) issue(stage == 0 ? NS - 1 : stage - 1, kt + NS - 1);
    compute(stage);
    stage = stage == NS - 1 ? 0 : stage + 1;
  }
  __syncthreads();  // every stage read: LDS is free for the row staging
  rowln_finish_dma<BM, DEFER>(acc, smem, p, lnw, lnb, eps, h16, m0, wn, lane, dfr);
}

// ---------------------------------------------------------------------------------------
// Small-M kernel (M <= 64): one block per (BN-row feature tile, canonical K chunk). Every
// global load of the block is issued before the first MFMA (one memory round trip); the chunk
// goes through LDS in 256-wide pieces while a single MFMA chain continues across them. The
// chunk result goes to part[chunk][m][n]; gemm_reduce adds the chunks in order.
// LNP > 0 (M <= 16, K = NPIECE * 256 = 768, one chunk): X = LayerNorm(ln.src + ordered sum of
// LNP-1 partial chunks) computed in every block with ln_row's arithmetic and written as f16
// straight into LDS for the whole K; block 0 also stores the f32 LayerNorm rows to ln.out.
template <int FMT, int BM, int BN, int NPIECE, int EPI, bool DIRECT, int LNP = 0>
__global__ __launch_bounds__(BN * 4) void gemm_small(GemmP p) {
  using SS = SmallShape<FMT, BM, BN, NPIECE, LNP>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[SS::LDS];
  RawSeg wr[SS::NP][SS::WPT];
  gemm_small_dev<FMT, BM, BN, NPIECE, EPI, DIRECT, LNP>(p, blockIdx.x, blockIdx.y, blockIdx.z, lds, wr);
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
// M <= 64, or 64 < M < 1024 in BM-row blocks (too few tokens to fill the GPU with 128-row
// tiles: 24 of them for a 512 x 768 output). K spanning one canonical chunk: one kernel,
// epilogue applied in place. Several chunks: per-chunk partials (nch x M x N floats in p.part),
// then gemm_reduce (or, when `reduce` is false, the caller's own ordered reduction, e.g. the
// fused residual + LayerNorm row kernel).
template <int FMT, int BM, int EPI>
static hipError_t launch_small(const GemmP& p, hipStream_t st, bool reduce) {
  constexpr int BN = 64;  // 16-feature one-wave blocks measured no faster at M = 8
  const int kc = kchunk_of(p.K);
  const int nch = p.K / kc;
  const dim3 grid(p.N / BN, nch, (p.M + BM - 1) / BM), blk(BN * 4);
  if (nch == 1) {
    if (kc == 768)
      hipLaunchKernelGGL((gemm_small<FMT, BM, BN, 3, EPI, true>), grid, blk, 0, st, p);
    else
      hipLaunchKernelGGL((gemm_small<FMT, BM, BN, 1, EPI, true>), grid, blk, 0, st, p);
    return hipGetLastError();
  }
  if (kc == 768)
    hipLaunchKernelGGL((gemm_small<FMT, BM, BN, 3, EPI, false>), grid, blk, 0, st, p);
  else
    hipLaunchKernelGGL((gemm_small<FMT, BM, BN, 1, EPI, false>), grid, blk, 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !reduce) return e;
  const int n = p.M * (p.N / 4);
  hipLaunchKernelGGL((gemm_reduce<EPI>), dim3((n + 255) / 256), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <int FMT, int EPI, int LNP>
static hipError_t launch_lnx3(const GemmP& p, hipStream_t st) {
  const dim3 grid(p.N / 64, 1), blk(256);
  hipLaunchKernelGGL((gemm_small<FMT, 16, 64, 3, EPI, true, LNP>), grid, blk, 0, st, p);
  return hipGetLastError();
}

template <int FMT, int EPI>
static hipError_t launch_lnx2(const GemmP& p, hipStream_t st) {
  switch (p.ln.part ? p.ln.nch : 0) {
    case 0: return launch_lnx3<FMT, EPI, 1>(p, st);
    case 4: return launch_lnx3<FMT, EPI, 5>(p, st);
    default: return hipErrorInvalidValue;
  }
}

template <int EPI>
static hipError_t launch_lnx1(int type, const GemmP& p, hipStream_t st) {
  switch (type) {
    case LLE_TYPE_Q8_0: return launch_lnx2<8, EPI>(p, st);
    case LLE_TYPE_Q4_K: return launch_lnx2<12, EPI>(p, st);
    case LLE_TYPE_Q5_K: return launch_lnx2<13, EPI>(p, st);
    case LLE_TYPE_Q6_K: return launch_lnx2<14, EPI>(p, st);
    case LLE_TYPE_F32: return launch_lnx2<0, EPI>(p, st);
    default: return hipErrorInvalidValue;
  }
}

// Compute units of the current device (blocks of one CU each fill the GPU at this count).
static int num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0)
    return 256;
  return n;
}

template <int FMT, int EPI>
static hipError_t launch_fmt(const GemmP& p, hipStream_t st, bool reduce) {
  if ((int64_t)p.M * p.K * 2 > INT32_MAX) return hipErrorInvalidValue;  // 32-bit buffer offsets
  if (p.M <= 64) {
    if (p.M <= 16) return launch_small<FMT, 16, EPI>(p, st, reduce);
    if (p.M <= 32) return launch_small<FMT, 32, EPI>(p, st, reduce);
    return launch_small<FMT, 64, EPI>(p, st, reduce);
  }
  const bool multi = p.K > kchunk_of(p.K);
  if (p.M < 1024 && (!multi || p.part)) return launch_small<FMT, 64, EPI>(p, st, reduce);
  if (p.M >= 1024 && p.w16) {
    // 2 stages of 64 KB; f32 outputs from N = 2048 (fewer N tiles leave a round mostly empty)
    if (!multi && p.N % 256 == 0 && (p.N >= 4096 || (EPI == EPI_F32 && p.N >= 2048))) {
      dim3 grid(p.N / 256, (p.M + 255) / 256);
      hipLaunchKernelGGL((gemm_h<256, 256, 4, 2, 2, EPI, false>), grid, dim3(512), 0, st, p);
      return hipGetLastError();
    }
    if constexpr (EPI == EPI_QKV) {
      // 256 x 256 or 256 x 288 tiles, 2 stages (64 / 68 KB), RoPE operands staged in LDS after the
      // K loop (the section is decided per 16-feature fragment, so a 288-wide tile may span two).
      // The width with fewer rounds of tiles on the CUs, weighted by the tile's fill per K step
      // (256 + BN rows), wins: N = 2304 takes 288 at 8192 tokens (one round against two) and at
      // 32768 (four against five).
      if (!multi && (p.K / KSTEP) % 2 == 0 && p.D % 16 == 0) {
        const int64_t mt = (p.M + 255) / 256, cus = num_cus();
        auto cost = [&](int bn) { return ((p.N / bn) * mt + cus - 1) / cus * (256 + bn); };
        const bool w256 = p.N % 256 == 0 && p.D % 256 == 0;
        dim3 grid(1, (p.M + 255) / 256);
        if (p.N % 288 == 0 && (!w256 || cost(288) < cost(256))) {
          grid.x = p.N / 288;
          hipLaunchKernelGGL((gemm_h<256, 288, 4, 2, 2, EPI, false>), grid, dim3(512), 0, st, p);
          return hipGetLastError();
        }
        if (w256) {
          grid.x = p.N / 256;
          hipLaunchKernelGGL((gemm_h<256, 256, 4, 2, 2, EPI, false>), grid, dim3(512), 0, st, p);
          return hipGetLastError();
        }
      }
    }
    if constexpr (EPI == EPI_RESID) {
      // 128-row tiles (3 stages of 32 KB) when they take fewer rounds of the CUs, weighted by
      // the fill per K step (BM + 128 rows): mid-size batches (e.g. 5017 rows: 240 blocks
      // instead of 120) keep every CU busy
      if ((p.K / KSTEP) % 3 == 0 && p.N % 128 == 0) {
        const int64_t cus = num_cus(), nt = p.N / 128;
        auto cost = [&](int bm) { return ((p.M + bm - 1) / bm * nt + cus - 1) / cus * (bm + 128); };
        if (cost(128) < cost(256)) {
          dim3 grid(p.N / 128, (p.M + 127) / 128);
          if (multi)
            hipLaunchKernelGGL((gemm_h<128, 128, 4, 2, 3, EPI, true>), grid, dim3(512), 0, st, p);
          else
            hipLaunchKernelGGL((gemm_h<128, 128, 4, 2, 3, EPI, false>), grid, dim3(512), 0, st, p);
          return hipGetLastError();
        }
      }
    }
    if ((p.K / KSTEP) % 3 == 0) {
      dim3 grid(p.N / 128, (p.M + 255) / 256);  // 3 stages of 48 KB
      if (multi)
        hipLaunchKernelGGL((gemm_h<256, 128, 4, 2, 3, EPI, true>), grid, dim3(512), 0, st, p);
      else
        hipLaunchKernelGGL((gemm_h<256, 128, 4, 2, 3, EPI, false>), grid, dim3(512), 0, st, p);
      return hipGetLastError();
    }
  }
  if (p.M >= 1024) {
    if (!multi && p.N >= 4096 && p.N % 256 == 0) {
      // 256 x 256 tiles: each X tile is read by half as many blocks, each decoded weight feeds
      // 256 tokens, and the 64 x 128 wave tiles need fewer LDS bytes per MAC
      dim3 grid(p.N / 256, (p.M + 255) / 256);
      hipLaunchKernelGGL((gemm_big<FMT, 256, 256, 4, 2, EPI, false, 1>), grid, dim3(512), 0, st, p);
      return hipGetLastError();
    }
    dim3 grid(p.N / 128, (p.M + 255) / 256);
    if (multi)
      hipLaunchKernelGGL((gemm_big<FMT, 256, 128, 4, 2, EPI, true, 2>), grid, dim3(512), 0, st, p);
    else
      hipLaunchKernelGGL((gemm_big<FMT, 256, 128, 4, 2, EPI, false, 2>), grid, dim3(512), 0, st, p);
    return hipGetLastError();
  }
  dim3 grid(p.N / 128, (p.M + 127) / 128);
  if (multi)
    hipLaunchKernelGGL((gemm_big<FMT, 128, 128, 2, 2, EPI, true, 2>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_big<FMT, 128, 128, 2, 2, EPI, false, 2>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_epi(int type, const GemmP& p, hipStream_t st, bool reduce = true) {
  switch (type) {
    case LLE_TYPE_Q8_0: return launch_fmt<8, EPI>(p, st, reduce);
    case LLE_TYPE_Q4_K: return launch_fmt<12, EPI>(p, st, reduce);
    case LLE_TYPE_Q5_K: return launch_fmt<13, EPI>(p, st, reduce);
    case LLE_TYPE_Q6_K: return launch_fmt<14, EPI>(p, st, reduce);
    case LLE_TYPE_F32: return launch_fmt<0, EPI>(p, st, reduce);
    default: return hipErrorInvalidValue;
  }
}

static GemmP make_params(const GemmArgs& a) {
  GemmP p{};
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
  p.w16 = a.w->w16;
  p.tokrow = a.tokrow;
  return p;
}

hipError_t launch_gemm(const GemmArgs& a, int epi, hipStream_t st) {
  const GemmP p = make_params(a);
  switch (epi) {
    case EPI_F32: return launch_epi<EPI_F32>(a.w->type, p, st);
    case EPI_RESID: return launch_epi<EPI_RESID>(a.w->type, p, st);
    case EPI_QKV: return launch_epi<EPI_QKV>(a.w->type, p, st);
    case EPI_GEGLU: return launch_epi<EPI_GEGLU>(a.w->type, p, st);
    default: return hipErrorInvalidValue;
  }
}

// h += X . W^T, then LayerNorm of h (rows of N = d_model) into h and h16. At M <= 64 with several
// K chunks the chunk reduction, residual add and LayerNorm run as one row kernel; otherwise the
// GEMM's residual epilogue is followed by the LayerNorm kernel. Both orders of operations are
// identical (same reduction order, same add, same LayerNorm), so results do not depend on M.
hipError_t launch_gemm_partials(const GemmArgs& a, hipStream_t st) {
  const GemmP p = make_params(a);
  if (p.M > 64 || p.K / kchunk_of(p.K) < 2) return hipErrorInvalidValue;
  return launch_epi<EPI_RESID>(a.w->type, p, st, false);
}

bool gemm_lnx_supported(const GemmArgs& a, const LnPrologue& ln) {
  return a.M <= 16 && a.w->K == 768 && a.w->N % 64 == 0 && (ln.part ? ln.nch == 4 : true);
}

hipError_t launch_gemm_lnx(const GemmArgs& a, int epi, const LnPrologue& ln, hipStream_t st) {
  if (!gemm_lnx_supported(a, ln)) return hipErrorInvalidValue;
  GemmP p = make_params(a);
  p.ln = ln;
  switch (epi) {
    case EPI_QKV: return launch_lnx1<EPI_QKV>(a.w->type, p, st);
    case EPI_GEGLU: return launch_lnx1<EPI_GEGLU>(a.w->type, p, st);
    default: return hipErrorInvalidValue;
  }
}

// Which kernels launch_gemm_resid_ln runs for a call (see the comments there).
enum class ResidPath { FULL128, FULLH64, FULLDEC, PARTS, SPLIT };
static ResidPath resid_path(const GemmP& p, int type) {
  const int nch = p.K / kchunk_of(p.K);
  const bool split_mid = p.w16 && p.M >= 1024 && (p.K / KSTEP) % 3 == 0 && p.N % 128 == 0 &&
                         (int64_t)((p.M + 255) / 256) * (p.N / 128) <= num_cus();
  if (p.M >= 128 * num_cus() && p.N == LN_N && nch == 1 && p.K % 64 == 0 && p.w16) return ResidPath::FULL128;
  if (!split_mid && p.M >= 1024 && p.N == LN_N && nch == 1 && p.K % 64 == 0 && p.w16 && type != LLE_TYPE_Q8_0 &&
      (p.K / LN_KS) % 3 == 0)
    return ResidPath::FULLH64;
  if (!split_mid && p.M >= 1024 && p.N == LN_N && nch == 1 && p.K % 64 == 0) return ResidPath::FULLDEC;
  if (p.M < 1024 && p.part && (nch == 2 || nch == 3 || nch == 4 || nch == 8 || nch == 12)) return ResidPath::PARTS;
  return ResidPath::SPLIT;
}

// The full-row kernels can finish a pending LayerNorm of their residual.
bool gemm_resid_ln_takes_defer(const GemmArgs& a) {
  const GemmP p = make_params(a);
  const ResidPath r = resid_path(p, a.w->type);
  return (int64_t)p.M * p.K * 2 <= INT32_MAX &&
         (r == ResidPath::FULL128 || r == ResidPath::FULLH64 || r == ResidPath::FULLDEC);
}

// The split path (tile GEMM with the residual epilogue, then the LayerNorm kernel) can leave its
// LayerNorm pending.
bool gemm_resid_ln_gives_defer(const GemmArgs& a) {
  const GemmP p = make_params(a);
  return (int64_t)p.M * p.K * 2 <= INT32_MAX && resid_path(p, a.w->type) == ResidPath::SPLIT;
}

hipError_t launch_gemm_resid_ln(const GemmArgs& a, const float* w, const float* b, float eps, __half* h16,
                                hipStream_t st, const LnDefer* defer_in, float2* stats_out) {
  const GemmP p = make_params(a);
  const int nch = p.K / kchunk_of(p.K);
  if ((int64_t)p.M * p.K * 2 > INT32_MAX) return hipErrorInvalidValue;  // 32-bit buffer offsets
  if ((defer_in && !gemm_resid_ln_takes_defer(a)) || (stats_out && !gemm_resid_ln_gives_defer(a)))
    return hipErrorInvalidValue;
  const LnDefer dfr = defer_in ? *defer_in : LnDefer{};
  // Without the f16 copy the decoding kernel (weights decoded in the loop, 64-row tiles) runs
  // 128-row tiles on the f16 copy (every format) once they give every CU a block: each block
  // streams the 1.2 MB weight once for twice the rows of the 64-row kernels (measured 0.103
  // against 0.112 ms at 32768 tokens); two 56 KB stages, 256 VGPRs, no spills. With fewer rows
  // the 64-row kernels keep more CUs busy (at 8192 / 16384 tokens: 0.054 / 0.055 ms against
  // 0.072 / 0.077 for 128-row tiles).
  // The full-row kernels stream the whole weight through every block, so a block takes about as
  // long as two 256 x 128 tiles of the split path (tile GEMM with the residual epilogue, then the
  // LayerNorm kernel). Below the row count at which the split path's tiles fill one round of the
  // CUs, the full-row kernels leave CUs idle and the split path is faster (bit-identical rows;
  // config 3's 8192 rows: 0.038 against 0.055 ms); from there on the full-row kernels win
  // (16384 rows: 0.055 against 0.064 ms).
  // Q8_0 keeps the decoding kernel at 64 rows: its packed decode is cheap and the block streams
  // half the weight bytes (measured 0.114 vs 0.124 ms at 32768 tokens); the K-quants' decode is
  // not cheap.
  switch (resid_path(p, a.w->type)) {
    case ResidPath::FULL128:
      if (defer_in)
        hipLaunchKernelGGL((gemm_rowln_h<128, 2, true>), dim3((p.M + 127) / 128), dim3(512), 0, st, p, w, b, eps, h16, dfr);
      else
        hipLaunchKernelGGL((gemm_rowln_h<128, 2>), dim3((p.M + 127) / 128), dim3(512), 0, st, p, w, b, eps, h16, dfr);
      return hipGetLastError();
    case ResidPath::FULLH64:
      if (defer_in)
        hipLaunchKernelGGL((gemm_rowln_h<64, 3, true>), dim3((p.M + 63) / 64), dim3(512), 0, st, p, w, b, eps, h16, dfr);
      else
        hipLaunchKernelGGL((gemm_rowln_h<64, 3>), dim3((p.M + 63) / 64), dim3(512), 0, st, p, w, b, eps, h16, dfr);
      return hipGetLastError();
    case ResidPath::FULLDEC: {
      const dim3 grid((p.M + 63) / 64), blk(512);
#define LLE_ROWLN(F)                                                                                  \
  do {                                                                                                \
    if (defer_in)                                                                                     \
      hipLaunchKernelGGL((gemm_rowln<F, 64, true>), grid, blk, 0, st, p, w, b, eps, h16, dfr);        \
    else                                                                                              \
      hipLaunchKernelGGL((gemm_rowln<F, 64>), grid, blk, 0, st, p, w, b, eps, h16, dfr);              \
  } while (0)
      switch (a.w->type) {
        case LLE_TYPE_Q8_0: LLE_ROWLN(8); break;
        case LLE_TYPE_Q4_K: LLE_ROWLN(12); break;
        case LLE_TYPE_Q5_K: LLE_ROWLN(13); break;
        case LLE_TYPE_Q6_K: LLE_ROWLN(14); break;
        case LLE_TYPE_F32: LLE_ROWLN(0); break;
        default: return hipErrorInvalidValue;
      }
#undef LLE_ROWLN
      return hipGetLastError();
    }
    case ResidPath::PARTS: {
      hipError_t e = launch_epi<EPI_RESID>(a.w->type, p, st, false);
      if (e != hipSuccess) return e;
      return launch_reduce_resid_ln(p.part, nch, p.M, p.N, p.y, p.y, h16, w, b, eps, st);
    }
    case ResidPath::SPLIT:
      break;
  }
  hipError_t e = launch_epi<EPI_RESID>(a.w->type, p, st, true);
  if (e != hipSuccess) return e;
  if (stats_out) return launch_ln_stats(p.y, h16, stats_out, w, b, eps, p.M, p.N, st);
  return launch_ln(p.y, h16, w, b, eps, p.M, p.N, st);
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

// The GEMM operand decode (f16) of an uploaded weight: out f16 bits [N][K].
template <int FMT>
__global__ void dequant_weight_h_kernel(WPlanes w, uint4* out) {
  const int64_t nseg = (int64_t)w.N * (w.K / 16);
  for (int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; s < nseg; s += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(s / (w.K / 16)), k0 = (int)(s % (w.K / 16)) * 16;
    RawSeg r = load_seg<FMT>(w, n, k0);
    uint4 lo, hi;
    decode_seg_h<FMT>(r, k0, lo, hi);
    out[((size_t)n * w.K + k0) / 8] = lo;
    out[((size_t)n * w.K + k0) / 8 + 1] = hi;
  }
}

hipError_t launch_dequant_weight_h(const WeightDev& wd, uint16_t* out, hipStream_t st) {
  WPlanes w{wd.p0, wd.p1, wd.p2, wd.p3, wd.K, wd.N};
  dim3 g(1024), b(256);
  uint4* o = (uint4*)out;
  switch (wd.type) {
    case LLE_TYPE_Q8_0: hipLaunchKernelGGL((dequant_weight_h_kernel<8>), g, b, 0, st, w, o); break;
    case LLE_TYPE_Q4_K: hipLaunchKernelGGL((dequant_weight_h_kernel<12>), g, b, 0, st, w, o); break;
    case LLE_TYPE_Q5_K: hipLaunchKernelGGL((dequant_weight_h_kernel<13>), g, b, 0, st, w, o); break;
    case LLE_TYPE_Q6_K: hipLaunchKernelGGL((dequant_weight_h_kernel<14>), g, b, 0, st, w, o); break;
    case LLE_TYPE_F32: hipLaunchKernelGGL((dequant_weight_h_kernel<0>), g, b, 0, st, w, o); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
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
