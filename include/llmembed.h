/*
 * libllmembed_hip.so — MI355X (gfx950) encoder forward pass for nomic-bert GGUF models.
 *
 * C ABI only: integers, pointers and sizes; floats travel as u32 bit patterns inside
 * structs (the reference's Windows MKL bridge passes every argument as a pointer for
 * the same reason: internal/ggml/mkl_windows.go:45,64-118). No torch / HIP types appear
 * in any signature; `stream` arguments are opaque hipStream_t values (NULL = the model's
 * own stream).
 *
 * Contract (mirrors what the reference's callers rely on):
 *   - Every entry point is re-entrant and callable from any OS thread; the device is set
 *     per call. Calls on one model are serialised internally (one forward at a time).
 *   - Host pointers are read or written only during the call; the library keeps none.
 *   - Host-pointer entry points are synchronous on return.
 *   - Return value: 0 on success, a negative LLE_E* code on failure; lle_last_error()
 *     returns a thread-local message for the last failure on the calling thread.
 */
#ifndef LLMEMBED_H
#define LLMEMBED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLE_ABI_VERSION 1

#define LLE_OK 0
#define LLE_EINVAL (-1)       /* bad argument, shape or id */
#define LLE_EDEVICE (-2)      /* no usable gfx950 device, or a HIP runtime failure */
#define LLE_ENOMEM (-3)       /* device allocation failed */
#define LLE_EUNSUPPORTED (-4) /* ggml type / model shape the path does not handle */
#define LLE_EIO (-5)          /* file open / read / parse failure */
#define LLE_ENOTFOUND (-6)    /* a required GGUF tensor or key is missing */

/* GGML tensor type ids (internal/gguf/reader.go:49-66). */
#define LLE_TYPE_F32 0
#define LLE_TYPE_Q8_0 8
#define LLE_TYPE_Q4_K 12
#define LLE_TYPE_Q5_K 13
#define LLE_TYPE_Q6_K 14

typedef struct lle_model lle_model;
typedef struct lle_weight lle_weight;

/* One GGUF tensor as it sits in the file: dims[0] = ne0 = inner K, ne1 = rows.
 * Replaces *ggml.Tensor{Name, Shape, Type, Data} (internal/ggml/tensor.go:13-18). */
typedef struct {
  int32_t type;
  int64_t ne0;
  int64_t ne1;
  const void* data;
  int64_t nbytes;
} lle_tensor;

/* Model description. Replaces BertModel's fields (internal/embed/bert.go:14-43,54-87) as
 * filled by LoadBertModel (:91-212); ln_eps / rope_base are float32 bit patterns. */
typedef struct {
  int32_t n_layer, d_model, n_head, d_ff, max_seq;
  uint32_t ln_eps_bits, rope_base_bits;
  lle_tensor token_embd, token_types, embd_norm_w, embd_norm_b;
  /* arrays of n_layer tensors each */
  const lle_tensor* qkv;
  const lle_tensor* out;
  const lle_tensor* attn_norm_w;
  const lle_tensor* attn_norm_b;
  const lle_tensor* up;
  const lle_tensor* gate;
  const lle_tensor* down;
  const lle_tensor* out_norm_w;
  const lle_tensor* out_norm_b;
} lle_model_desc;

/* Per-kernel-class timing collected with HIP events on the forward's stream. */
typedef struct {
  char name[32];
  int64_t launches;
  double total_ms;
  double flops; /* algorithmic FLOPs summed over launches */
  double bytes; /* algorithmic HBM bytes summed over launches */
} lle_kernel_time;

int32_t lle_abi_version(void);

/* Select and probe a device (gfx950 required). Replaces the MKL dlopen probe
 * initMKL (internal/ggml/mkl_linux.go:45-61): a failure here is what makes a host
 * fall back to its CPU path, as useMKL=false does. */
int32_t lle_init(int32_t device_ordinal);

const char* lle_last_error(void);

/* Human-readable backend description; SgemmInfo analogue (internal/ggml/sgemm.go:263-269). */
int32_t lle_info(char* buf, int32_t cap);

/* Test hook: f16 bit patterns -> f32 on the device, bit-exact with f16ToF32
 * (internal/ggml/tensor.go:162-191), NaN payloads included. */
int32_t lle_f16_to_f32(const uint16_t* h, int64_t n, float* out);

/* Test hook: dequantise raw GGUF blocks on the device; the same values as
 * Tensor.Dequantize / DequantWeightMatrix (internal/ggml/tensor.go:51-66,
 * internal/ggml/gemm.go:221-267), bit for bit. */
int32_t lle_dequant(int32_t ggml_type, const void* blocks, int64_t n_elements, float* out);

/* Upload a model: LoadBertModel + PreDequant + NewRoPETable
 * (internal/embed/bert.go:91-212,542-576; internal/ggml/ops_simd.go:107-124).
 * Weights stay quantised in HBM (bit-preserving re-layout); no host pointer is kept. */
int32_t lle_model_create(const lle_model_desc* desc, lle_model** out);

/* Parse a GGUF file and upload it (internal/gguf/reader.go:219-280 + the above). */
int32_t lle_model_load_gguf(const char* path, lle_model** out);

int32_t lle_model_destroy(lle_model* m);

/* dims[0..6] = n_layer, d_model, n_head, d_ff, max_seq, vocab. */
int32_t lle_model_dims(const lle_model* m, int32_t* dims);

/* Embed one sequence (Embedder.Embed after tokenisation, internal/embed/embedder.go:46-71):
 * forward + masked mean-pool + L2 (+ Matryoshka truncate/renormalise when out_dim < d_model).
 * out: min(out_dim, d_model) floats. */
int32_t lle_embed(lle_model* m, const int32_t* ids, const int32_t* mask, int32_t L, int32_t out_dim,
                  float* out);

/* Batched embed: B right-padded rows of length L (mask 1 = token, 0 = padding). Each row's
 * result equals lle_embed on that row bit for bit (batch invariance, as the reference's
 * EmbedBatch == Embed tests require: internal/embed/embedder_test.go:139-144,246-251).
 * Positions after a row's last mask-1 token are not computed (packed rows): they cannot reach
 * the embedding. out: B x min(out_dim, d_model). */
int32_t lle_embed_batch(lle_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t L,
                        int32_t out_dim, float* out);

/* Same on device pointers, enqueued on `stream` (NULL = the model's stream); returns after
 * enqueueing. A model's forwards share its workspace, so each is ordered after the model's
 * previous forward: on another stream than that one, `stream` first waits for an event that
 * marks its end (same stream: no wait). Async work must finish before lle_model_destroy. Token
 * ids outside [0, vocab) are clamped and reported by lle_model_status. */
int32_t lle_embed_batch_async(lle_model* m, const int32_t* d_ids, const int32_t* d_mask, int32_t B,
                              int32_t L, int32_t out_dim, float* d_out, void* stream);

/* Parity hook: hidden states [B*L][d_model] before pooling (BertModel.Forward output,
 * internal/embed/bert.go:216-285). */
int32_t lle_forward_hidden(lle_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t L,
                           float* hidden);

/* Packed batch on device pointers: the B sequences back to back in d_ids (T tokens, every one
 * valid: no padding is stored or computed), d_seq_off [B+1] int32 with d_seq_off[0] = 0 and
 * d_seq_off[B] = T; L >= the longest sequence (<= context_length). Row b of d_out equals
 * lle_embed of sequence b bit for bit. Enqueued on `stream`; an inconsistent offset table is
 * made safe and reported by lle_model_status (bit 2). Stream ordering as lle_embed_batch_async. */
int32_t lle_embed_packed_async(lle_model* m, const int32_t* d_ids, const int32_t* d_seq_off, int32_t B, int32_t T,
                               int32_t L, int32_t out_dim, float* d_out, void* stream);

/* No counterpart in the reference. For callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): lle_embed_packed_async's forward
 * (same arguments, same rows bit for bit) with every activation buffer in one fixed device array
 * of LLE_NOALLOC_SCRATCH_BYTES per device (set up by lle_init, held until the process ends),
 * so the call makes no device allocation. It runs eagerly on `stream` itself (NULL = the
 * model's stream), with no graph capture of its own and no timing events, so a caller may
 * capture it into its own graph. A batch whose activations do not fit is rejected with
 * LLE_EINVAL and a message giving the bytes it needs (for nomic-bert-base every batch of up to 512
 * tokens with B x (L rounded up to 64) <= 2048 fits). Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU race: serialise them (one stream, or wait for one before the next). */
#define LLE_NOALLOC_SCRATCH_BYTES (32 * 1024 * 1024)
int32_t lle_embed_packed_noalloc(lle_model* m, const int32_t* d_ids, const int32_t* d_seq_off, int32_t B, int32_t T,
                                 int32_t L, int32_t out_dim, float* d_out, void* stream);

/* Device-side status word of async forwards since the last host-pointer call (bits OR-ed):
 * 1 = a token id was out of range (clamped), 2 = a packed batch's offsets were inconsistent. */
int32_t lle_model_status(lle_model* m, int32_t* status);

/* Arithmetic of a model's forwards. LLE_PRECISION_F16 (the default): MFMA GEMMs on f16 operands
 * (weights rounded once from the exact dequantisation, activations rounded to f16 between
 * kernels) with f32 accumulation; within the per-vector tolerance of the reference. And
 * LLE_PRECISION_F32: the reference CPU path's own f32 arithmetic in its order (GemmPrePacked32's
 * 128-wide K chunks with FMA chains and unfused edge rows, internal/ggml/gemm_avx512.go:67-147;
 * sequential LayerNorm sums; DotF32 order; exp in f64; internal/embed/bert.go:216-445,
 * internal/ggml/ops_simd.go, internal/embed/pool.go), on f32 copies of the dequantised weights
 * made when it is selected (as PreDequant does, bert.go:542-576; 4 bytes per weight), so
 * embeddings equal the reference's bit for bit up to the last float64 ulp of exp. In F32 mode
 * lle_embed_batch_async and lle_embed_packed_noalloc return LLE_EUNSUPPORTED (use the host
 * entries or lle_embed_packed_async, which know each sequence's length). */
#define LLE_PRECISION_F16 0
#define LLE_PRECISION_F32 1
int32_t lle_model_set_precision(lle_model* m, int32_t precision);

/* Kernel timing: enable (1) / disable (0) and read per-kernel-class HIP-event totals.
 * lle_model_set_timing brackets every launch and synchronises at the end of each forward.
 * lle_model_set_timing_kernel brackets only the launches of one kernel class (e.g. "gemm_upgate";
 * NULL or "" disables timing) and does not synchronise per forward: its events are read by
 * lle_model_get_timing, which waits for the device. Both run forwards eagerly (no graph replay).
 * No counterpart in the reference (SgemmInfo, internal/ggml/sgemm.go:263-269, is its only
 * introspection); used by the benchmark. */
int32_t lle_model_set_timing(lle_model* m, int32_t enable);
int32_t lle_model_set_timing_kernel(lle_model* m, const char* kernel_class);
int32_t lle_model_get_timing(lle_model* m, lle_kernel_time* out, int32_t cap, int32_t* n_out);

/* Isolated quantised projection (gemmOrBatch, internal/embed/bert.go:579-638):
 * Y[M][N] = X[M][K] . W^T, W one GGUF tensor [K, N] (N rows of K, blocks along K). */
int32_t lle_weight_create(int32_t ggml_type, const void* blocks, int32_t K, int32_t N, lle_weight** out);
int32_t lle_weight_destroy(lle_weight* w);
/* Test hook: the uploaded (re-laid-out) weight dequantised by the GEMM's own decoder,
 * as f32 [N][K] (must equal DequantWeightMatrix bit for bit). */
int32_t lle_weight_dequant(const lle_weight* w, float* out);
/* Test hook: the same weight as the GEMM's f16 MFMA operand, f16 bits [N][K]; every value is
 * the f32 dequantisation rounded once to f16 (round-to-nearest-even). */
int32_t lle_weight_dequant_f16(const lle_weight* w, uint16_t* out);
/* Host pointers, synchronous. */
int32_t lle_gemm(const lle_weight* w, const float* X, int32_t M, float* Y);
/* Device pointers: X f32 [M][K] is converted to f16 into d_x16 (M*K halfs, caller-owned),
 * then Y f32 [M][N]; enqueued on stream. */
int32_t lle_gemm_async(const lle_weight* w, const float* d_X, void* d_x16, int32_t M, float* d_Y, void* stream);
/* The same projection on activations already held as f16 on the device (what the encoder's own
 * kernels hand each other): Y f32 [M][N] = X16 [M][K] . W^T, enqueued on stream. d_part is a
 * split-K workspace of (K % 768 == 0 ? K / 768 : K / 256) * M * N floats (the 768-wide K chunks
 * are summed in order): required for M <= 64; for 64 < M < 1024 it lets several-chunk K run on
 * row blocks that fill the GPU (NULL: 128-row tiles); unused from 1024 rows. */
int32_t lle_gemm_f16_async(const lle_weight* w, const void* d_x16, int32_t M, float* d_Y, float* d_part,
                           void* stream);

/* ---- Host tokeniser (no GPU use) ----------------------------------------------------------
 * WordPieceTokenizer (internal/embed/tokenizer.go:15-19): nomic's "▁"-prefixed vocabulary,
 * greedy longest match over the bytes of each lowercased, whitespace/punctuation-split word. */
typedef struct lle_tokenizer lle_tokenizer;

/* LoadTokenizer (tokenizer.go:22-45): the vocabulary is the GGUF metadata string array
 * `tokenizer.ggml.tokens`, read as readGGUFStringArray does (:198-306). */
int32_t lle_tokenizer_load_gguf(const char* path, lle_tokenizer** out);
/* The same from a token list: tokens[i] of lens[i] bytes has id i (a later duplicate wins). */
int32_t lle_tokenizer_create(const char* const* tokens, const int64_t* lens, int32_t n, lle_tokenizer** out);
int32_t lle_tokenizer_destroy(lle_tokenizer* t);
/* VocabSize (tokenizer.go:145-148). */
int32_t lle_tokenizer_vocab_size(const lle_tokenizer* t, int32_t* n);
/* Encode (tokenizer.go:47-78) of text[0..len) (len < 0: NUL-terminated): [CLS]=101, pieces,
 * [SEP]=102, cut to max_len (>= 1) with [SEP] last; the mask is all ones. Writes the first
 * min(count, cap) ids; *n_out = count. */
int32_t lle_tokenize(const lle_tokenizer* t, const char* text, int64_t len, int32_t max_len, int32_t* ids,
                     int32_t cap, int32_t* n_out);
/* Encode(prefix + texts[i]) for n texts on host threads (lens NULL: NUL-terminated texts;
 * prefix_len < 0: NUL-terminated prefix). n_tok[i] = token count. With ids != NULL, also
 * writes the right-padded batch ids / mask [n][L] (pad id 0, mask 0); LLE_EINVAL when a text
 * needs more than L tokens (call with ids NULL first to size L). */
int32_t lle_tokenize_batch(const lle_tokenizer* t, const char* const* texts, const int64_t* lens, int32_t n,
                           const char* prefix, int64_t prefix_len, int32_t max_len, int32_t L, int32_t* ids,
                           int32_t* mask, int32_t* n_tok);

/* EmbedBatch over text (internal/embed/embedder.go:46-133): out row i = Embed(prefix + texts[i])
 * with max_len = the model's context_length, bit for bit the row lle_embed gives for that
 * text's ids. Texts are tokenised on host threads, ordered by token count (longest first) and
 * run in batches of at most max_batch_tokens tokens (<= 0: 32768); padding is not computed
 * (packed rows, as lle_embed_batch). out: n x min(out_dim, d_model), in input order.
 * Synchronous. */
int32_t lle_embed_texts(lle_model* m, const lle_tokenizer* t, const char* const* texts, const int64_t* lens,
                        int32_t n, const char* prefix, int64_t prefix_len, int32_t out_dim,
                        int32_t max_batch_tokens, float* out);

#ifdef __cplusplus
}
#endif
#endif
