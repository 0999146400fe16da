/*
 * CPU oracle for the nomic-bert encoder forward pass of dbrushchenko/llm-embed.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * pure-Go CPU path, used as the parity checker and as the timed CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. The product (libllmembed_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Build: `make -C oracle` (gcc -O3 -ffp-contract=off; explicit fmaf only where
 * the reference's AVX-512 micro-kernel fuses).
 */
#ifndef LLE_ORACLE_H
#define LLE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (internal/gguf/reader.go:49-66) */
enum { ORC_F32 = 0, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14 };

float orc_f16_to_f32(uint16_t h);
void orc_f16_to_f32_array(const uint16_t* h, int64_t n, float* out);
int64_t orc_row_bytes(int32_t type, int64_t n_elements);
int32_t orc_dequant(int32_t type, const uint8_t* data, int64_t n_elements, float* out);
void orc_get_scale_min_k4(int32_t j, const uint8_t* scales, uint8_t* sc, uint8_t* m);

/* C[M][N] = A[M][K] . B[N][K]^T in GemmPrePacked32 order (fresh C, no accumulate-in). */
void orc_gemm(const float* A, int32_t M, int32_t K, const float* B, int32_t N, float* C,
              int32_t n_threads);

void orc_layernorm(float* x, const float* w, const float* b, float eps, int32_t n);
void orc_gelu(float* x, int32_t n);
void orc_softmax(float* x, int32_t n);
float orc_dotf32(const float* a, const float* b, int32_t n);
void orc_rope_table(int32_t max_pos, int32_t head_dim, float base, float* cos_tab, float* sin_tab);
void orc_rope_apply(float* x, const float* cos_row, const float* sin_row, int32_t n_rot);
void orc_mean_pool(const float* hidden, const int32_t* mask, int32_t L, int32_t dim, float* out);
void orc_l2_normalize(const float* v, int32_t n, float* out);

/* One tensor of the model as stored in the GGUF (dims[0] = inner K). */
typedef struct {
  int32_t type;
  int64_t ne0; /* inner (K) */
  int64_t ne1; /* outer (N / rows) */
  const uint8_t* data;
  int64_t nbytes;
} orc_tensor;

typedef struct {
  int32_t n_layer, d_model, n_head, d_ff, max_seq;
  float ln_eps, rope_base;
  orc_tensor token_embd, token_types, embd_norm_w, embd_norm_b;
  /* per layer, arrays of n_layer entries */
  const orc_tensor* qkv;
  const orc_tensor* out;
  const orc_tensor* attn_norm_w;
  const orc_tensor* attn_norm_b;
  const orc_tensor* up;
  const orc_tensor* gate;
  const orc_tensor* down;
  const orc_tensor* out_norm_w;
  const orc_tensor* out_norm_b;
} orc_model_desc;

typedef struct orc_model orc_model;

int32_t orc_model_create(const orc_model_desc* d, orc_model** out);
void orc_model_destroy(orc_model* m);
/* Worker count cap used for GEMM N-panel split (NumWorkers analogue). 0 = min(nproc, 8). */
void orc_set_threads(orc_model* m, int32_t n_gemm_threads, int32_t n_attn_threads);

/* Forward of ONE sequence of length L: hidden[L][d_model]. */
int32_t orc_forward(orc_model* m, const int32_t* ids, const int32_t* mask, int32_t L, float* hidden);
/* Embed of one sequence: forward + mean-pool + L2 (+ Matryoshka truncation to out_dim). */
int32_t orc_embed(orc_model* m, const int32_t* ids, const int32_t* mask, int32_t L, int32_t out_dim,
                  float* out);
/* EmbedBatch: B rows of a right-padded [B][L] batch; each row runs orc_embed on its valid
 * prefix (what the reference's tokenizer would have produced), on min(nproc,B,8) workers. */
int32_t orc_embed_batch(orc_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t L,
                        int32_t out_dim, float* out, int32_t n_workers);

#ifdef __cplusplus
}
#endif
#endif
