// Internal declarations shared by the HIP kernels and the host runtime.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <string>

#include "../../include/llmembed.h"

namespace lle {

// ---------------------------------------------------------------------------------------
// Error plumbing (thread-local last error, negative codes).
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
#define LLE_HIP(call)                                                                  \
  do {                                                                                 \
    hipError_t e_ = (call);                                                            \
    if (e_ != hipSuccess)                                                              \
      return ::lle::fail(LLE_EDEVICE, std::string(#call) + ": " + hipGetErrorString(e_)); \
  } while (0)

// ---------------------------------------------------------------------------------------
// Device-resident weight formats. Every format is a bit-preserving re-layout of the GGUF
// blocks into "k-group major" planes so that one 64-wide K step of BN consecutive rows is a
// contiguous, 16-byte aligned run per plane. Bytes per weight are exactly the GGUF ones.
//
//   Q8_0 : codes [K/32][N][32] int8       scales [K/32][N] f16 bits
//   Q4_K : qs    [K/64][N][32] (low nibble = element l, high = element 32+l of the group)
//          hdr   [K/256][N][16] = GGUF {d, dmin, scales[12]} verbatim
//   Q5_K : qs, hdr as Q4_K;  qh [K/64][N][2] u32: word w bit l = high bit of element 32w+l
//   Q6_K : ql    [K/64][N][32] (low nibble = element l, high = element 32+l), 4-bit low parts
//          qh    [K/64][N][16] (element e: byte e/4, bits 2(e%4)..+1), 2-bit high parts
//          sc    [K/64][N][4]  int8 scale of elements 16s..16s+15 of the group
//          d     [K/256][N]    f16 bits
//   F32  : [N][K] f32
struct WeightDev {
  int type = -1;
  int K = 0, N = 0;
  void* base = nullptr;  // one allocation holding every plane
  size_t bytes = 0;      // algorithmic bytes (= GGUF bytes)
  const uint8_t* p0 = nullptr;  // codes / qs / ql / f32
  const uint8_t* p1 = nullptr;  // scales / hdr / qh
  const uint8_t* p2 = nullptr;  // qh (Q5_K) / sc (Q6_K)
  const uint8_t* p3 = nullptr;  // d (Q6_K)
  // resident f16 copy [N][K] (RNE of the dequantisation) for the large-M GEMMs, or null
  __half* w16 = nullptr;
};

// Host-side re-layout of GGUF blocks of a [N][K] matrix into the planes above.
size_t weight_dev_bytes(int type, int K, int N);  // algorithmic (GGUF) bytes
void plane_offsets(int type, int K, int N, size_t off[4], size_t* total);
void repack_rows(int type, const uint8_t* gguf, int K, int N, uint8_t* dst, const size_t off[4]);

// ---------------------------------------------------------------------------------------
// Kernel launchers (defined in the .hip files). All enqueue on `st` and return hipError_t.

enum Epilogue { EPI_F32 = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_GEGLU = 3 };

struct GemmArgs {
  const WeightDev* w;
  const __half* x;  // [M][K] f16
  int M;
  // EPI_F32: y f32 [M][N]; EPI_RESID: y f32 [M][N] (+=)
  float* y;
  // EPI_QKV: q/k [B][H][Lp][64] f16, vt [B][H][64][Lp] f16
  __half* q;
  __half* k;
  __half* vt;
  const float* rope_cos;  // [max_seq][32]
  const float* rope_sin;
  int L, Lp, n_head, d_model;
  // EPI_GEGLU: out f16 [M][N/2]
  __half* g;
  // split-K partials for M <= 64: [K/256][M][N] f32
  float* part;
  // packed rows (padding removed): row m is token tokrow[m] = b * L + position of the padded
  // [B][L] batch; null when row m is token m
  const int32_t* tokrow;
};

hipError_t launch_gemm(const GemmArgs& a, int epi, hipStream_t st);
// A LayerNorm left pending by launch_ln_stats: the f32 rows hold its input, stats[t] = {mean,
// invStd}, and w / b are its weights; the consumer applies ln_elem to each element it reads.
struct LnDefer {
  const float* w;
  const float* b;
  const float2* stats;  // padded to a multiple of 128 rows (read in whole 128-row blocks)
};
// a.y (= h) += X . W^T, then LayerNorm(h; w, b, eps) into h and h16.
// defer_in: the residual a.y holds a pending LayerNorm (only where gemm_resid_ln_takes_defer).
// stats_out: leave this LayerNorm pending instead (h16 and stats_out written, h left as the sum;
// only where gemm_resid_ln_gives_defer).
hipError_t launch_gemm_resid_ln(const GemmArgs& a, const float* w, const float* b, float eps, __half* h16,
                                hipStream_t st, const LnDefer* defer_in = nullptr, float2* stats_out = nullptr);
bool gemm_resid_ln_takes_defer(const GemmArgs& a);
bool gemm_resid_ln_gives_defer(const GemmArgs& a);
// M <= 16, K = 768: GEMM whose X operand is LN(src [+ ordered sum of nch partials]) computed in
// every block (ln_row's arithmetic); block 0 also writes that LayerNorm output (f32) to ln_out.
// Replaces a LayerNorm (or reduce + residual + LayerNorm) kernel in front of the GEMM.
struct LnPrologue {
  const float* src;
  const float* part;  // [nch][M][768] or null
  int nch;
  const float* w;
  const float* b;
  float eps;
  float* out;
};
bool gemm_lnx_supported(const GemmArgs& a, const LnPrologue& ln);
hipError_t launch_gemm_lnx(const GemmArgs& a, int epi, const LnPrologue& ln, hipStream_t st);
// M <= 64, K spanning several canonical chunks: per-chunk partials only (part[c][M][N])
hipError_t launch_gemm_partials(const GemmArgs& a, hipStream_t st);
// h = LN(src + (0 + part[0] + ... + part[nch-1])) and h16 = f16(h); src may equal h
hipError_t launch_reduce_resid_ln(const float* part, int nch, int M, int N, const float* src, float* h, __half* h16,
                                  const float* w, const float* b, float eps, hipStream_t st);

hipError_t launch_f32_to_f16(const float* x, __half* y, int64_t n, hipStream_t st);
hipError_t launch_f16_to_f32_bits(const uint16_t* h, float* out, int64_t n, hipStream_t st);
hipError_t launch_dequant_raw(int type, const uint8_t* blocks, int64_t n, float* out, hipStream_t st);
hipError_t launch_dequant_weight(const WeightDev& w, float* out, hipStream_t st);
hipError_t launch_dequant_weight_h(const WeightDev& w, uint16_t* out, hipStream_t st);

struct EmbedArgs {
  const int32_t* ids;
  int T;
  int vocab;
  int tok_type;
  const uint8_t* tok;  // raw GGUF token_embd
  int64_t tok_row_bytes;
  const float* type0;  // [D]
  const float* w;
  const float* b;
  float eps;
  int D;
  float* h;
  __half* h16;
  int32_t* status;
};
hipError_t launch_embed_ln(const EmbedArgs& a, hipStream_t st);
hipError_t launch_ln(float* h, __half* h16, const float* w, const float* b, float eps, int T, int D,
                     hipStream_t st);
// ln_kernel that leaves the f32 rows as they are and writes h16 and stats[t] = {mean, invStd}
hipError_t launch_ln_stats(const float* h, __half* h16, float2* stats, const float* w, const float* b, float eps,
                           int T, int D, hipStream_t st);

struct AttnArgs {
  const __half* q;
  const __half* k;
  const __half* vt;
  const int32_t* mask;   // [B][L]
  __half* out;           // [B*L][D], or [T][D] rows seq_off[b] + q when packed
  int B, L, Lp, H, D;
  const int32_t* seq_off;  // packed: [B+1] first row of each sequence (it has seq_off[b+1] -
                           // seq_off[b] positions); null: sequence b is rows b*L .. b*L+L-1
};
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);

// scratch (B x D floats, may be null): the per-sequence means of the sliced form for few long rows
hipError_t launch_pool(const float* h, const int32_t* mask, const int32_t* seq_off, int B, int L, int D, int out_dim,
                       float* out, float* scratch, size_t scratch_bytes, hipStream_t st);
// launch_reduce_resid_ln (rows of N = D, nch = 4) followed by launch_pool, in one kernel that
// keeps the LayerNorm rows in LDS; bit-identical to the two kernels. The LayerNorm rows are not
// stored.
hipError_t launch_reduce_ln_pool(const float* part, int nch, int M, const float* src, const float* w, const float* b,
                                 float eps, const int32_t* mask, const int32_t* seq_off, int B, int L, int D,
                                 int out_dim, float* out, hipStream_t st);
// packed batch tables from caller offsets in_off[B+1]: sanitised offsets, tokrow [T], mask [B][L]
hipError_t launch_pack_tables(const int32_t* in_off, int B, int T, int L, int32_t* off, int32_t* tokrow,
                              int32_t* mask, int32_t* status, hipStream_t st);

// ---------------------------------------------------------------------------------------
// Reference-exact f32 forward (exact.hip): activations f32, weights the f32 dequantisation.
struct ExactArgs {
  int T, L, D, H;
  const int32_t* tokrow;   // packed rows: row t is padded token tokrow[t] = b * L + p (null: t)
  const int32_t* seq_off;  // packed: [B+1] first row of each sequence (null: rows b*L .. b*L+L-1)
  const int32_t* mask;     // [B][L]
  const int32_t* ids;      // embedding: token id of each row
  int vocab, tok_type;
  const uint8_t* tok;      // raw GGUF token_embd
  int64_t tok_row_bytes;
  const float* type0;      // token_types row 0
  int32_t* status;
  const float* lnw;        // LayerNorm weights of the current step
  const float* lnb;
  float eps;
  float* h;                // [T][D] residual stream
  float *q, *k, *v, *att;  // [T][D]
  const float* rope_cos;   // [max_seq][32]
  const float* rope_sin;
};
struct ExactGemm {
  const float* x;  // [T][K]
  const float* w;  // [N][K]
  int N, K;
  float* y;        // EPI_F32: [T][N]; EPI_RESID: [T][N] (+=); EPI_GEGLU: [T][N/2]; EPI_QKV: unused
};
hipError_t launch_exact_embed(const ExactArgs& a, hipStream_t st);
hipError_t launch_exact_ln(const ExactArgs& a, hipStream_t st);
hipError_t launch_exact_gemm(const ExactArgs& a, const ExactGemm& g, int epi, hipStream_t st);
hipError_t launch_exact_attention(const ExactArgs& a, hipStream_t st);
hipError_t launch_exact_pool(const ExactArgs& a, int B, int out_dim, float* out, hipStream_t st);

// ---------------------------------------------------------------------------------------
// No-allocation packed forward (lle_embed_packed_noalloc, noalloc.hip).
// Resolves the device address of the fixed scratch array on `device` (which must be current);
// once per device, thread-safe. Called by lle_init.
int noalloc_setup(int device);
int model_device(const lle_model* m);
// lle_embed_packed_async's forward with every activation buffer carved from `scratch`
// (scratch_bytes long) instead of the model's workspace; enqueued eagerly on `stream` (NULL: the
// model's stream), no graph capture, no timing events, no allocation.
int embed_packed_scratch(lle_model* m, const int32_t* d_ids, const int32_t* d_seq_off, int B, int T, int L,
                         int out_dim, float* d_out, hipStream_t stream, void* scratch, size_t scratch_bytes);

}  // namespace lle
