/*
 * CPU oracle: plain-C restatement of dbrushchenko/llm-embed's pure-Go encoder path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + timed CPU baseline). Nothing in the
 * product links this file. Arithmetic follows the Go source operation by operation:
 * Go float32 expressions are evaluated left to right in float32 with no contraction
 * (amd64, GOAMD64=v1), so this file is compiled with -ffp-contract=off and uses an
 * explicit fmaf() only where the reference's AVX-512 micro-kernel issues VFMADD231PS.
 * Go's float64 math.Exp/Pow/Cos/Sin are restated with libm's exp/pow/cos/sin; the two
 * may differ in the last float64 ulp, which reaches the float32 result only when it
 * sits on a float32 rounding boundary (parity of that last-ulp case is unpinned).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------- */
/* f16 -> f32: internal/ggml/tensor.go:162-191 (f16ToF32); the same result as
 * f16ToF32Fast at internal/ggml/ops_fast.go:229-254. Subnormals are normalised,
 * Inf/NaN keep their payload. */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u;
  int32_t exp = (int32_t)((h >> 10) & 0x1f);
  uint32_t mant = (uint32_t)h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign << 31;
      float f;
      memcpy(&f, &bits, 4);
      return f;
    }
    while ((mant & 0x400u) == 0) {
      mant <<= 1;
      exp--;
    }
    exp++;
    mant &= 0x3ffu;
    exp += 127 - 15;
    bits = (sign << 31) | ((uint32_t)exp << 23) | (mant << 13);
  } else if (exp < 31) {
    exp += 127 - 15;
    bits = (sign << 31) | ((uint32_t)exp << 23) | (mant << 13);
  } else {
    bits = (sign << 31) | (0xffu << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Array form: results written to memory, so NaN payloads survive the caller's float handling. */
void orc_f16_to_f32_array(const uint16_t* h, int64_t n, float* out) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(h[i]);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Bytes of one row of n elements (internal/gguf/reader.go:196-204 ByteSize). */
int64_t orc_row_bytes(int32_t type, int64_t n) {
  switch (type) {
    case ORC_F32: return n * 4;
    case ORC_Q8_0: return (n / 32) * 34;
    case ORC_Q4_K: return (n / 256) * 144;
    case ORC_Q5_K: case 15: case 16: return (n / 256) * 176;
    case ORC_Q6_K: return (n / 256) * 210;
    default: return -1;
  }
}

/* getScaleMinK4: internal/ggml/quant_q4k.go:133-140 */
void orc_get_scale_min_k4(int32_t j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* dequantQ8_0: internal/ggml/tensor.go:130-159 (and dequantQ8_0Row, gemm.go:270-282) */
static void deq_q8_0(const uint8_t* data, int64_t n, float* out) {
  int64_t nb = n / 32;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* blk = data + b * 34;
    float scale = orc_f16_to_f32(rd16(blk));
    for (int i = 0; i < 32; i++) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * scale;
  }
}

/* DequantQ4_K: internal/ggml/quant_q4k.go:27-77 */
static void deq_q4_k(const uint8_t* data, int64_t n, float* out) {
  int64_t nb = n / 256;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* blk = data + b * 144;
    float d = orc_f16_to_f32(rd16(blk));
    float dmin = orc_f16_to_f32(rd16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* qs = blk + 16;
    float* o = out + b * 256;
    int is = 0, qoff = 0;
    for (int j = 0; j < 256; j += 64) {
      uint8_t sc1, m1, sc2, m2;
      orc_get_scale_min_k4(is, scales, &sc1, &m1);
      float d1 = d * (float)sc1, dm1 = dmin * (float)m1;
      orc_get_scale_min_k4(is + 1, scales, &sc2, &m2);
      float d2 = d * (float)sc2, dm2 = dmin * (float)m2;
      for (int l = 0; l < 32; l++) o[j + l] = d1 * (float)(qs[qoff + l] & 0xF) - dm1;
      for (int l = 0; l < 32; l++) o[j + 32 + l] = d2 * (float)(qs[qoff + l] >> 4) - dm2;
      qoff += 32;
      is += 2;
    }
  }
}

/* DequantQ5_K: internal/ggml/quant_q5k.go:29-91 */
static void deq_q5_k(const uint8_t* data, int64_t n, float* out) {
  int64_t nb = n / 256;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* blk = data + b * 176;
    float d = orc_f16_to_f32(rd16(blk));
    float dmin = orc_f16_to_f32(rd16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    float* o = out + b * 256;
    int is = 0, qoff = 0;
    unsigned qhbit = 0;
    for (int j = 0; j < 256; j += 64) {
      uint8_t sc1, m1, sc2, m2;
      orc_get_scale_min_k4(is, scales, &sc1, &m1);
      float d1 = d * (float)sc1, dm1 = dmin * (float)m1;
      orc_get_scale_min_k4(is + 1, scales, &sc2, &m2);
      float d2 = d * (float)sc2, dm2 = dmin * (float)m2;
      for (int l = 0; l < 32; l++) {
        uint8_t q = (uint8_t)((qs[qoff + l] & 0xF) | (((qh[l] >> qhbit) & 1) << 4));
        o[j + l] = d1 * (float)q - dm1;
      }
      qhbit++;
      for (int l = 0; l < 32; l++) {
        uint8_t q = (uint8_t)((qs[qoff + l] >> 4) | (((qh[l] >> qhbit) & 1) << 4));
        o[j + 32 + l] = d2 * (float)q - dm2;
      }
      qhbit++;
      qoff += 32;
      is += 2;
    }
  }
}

/* DequantQ6_K: internal/ggml/quant_q6k.go:23-75. Go evaluates d*float32(sc)*float32(q)
 * left to right: (d*sc)*q. */
static void deq_q6_k(const uint8_t* data, int64_t n, float* out) {
  int64_t nb = n / 256;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* blk = data + b * 210;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const uint8_t* scales = blk + 192;
    float d = orc_f16_to_f32(rd16(blk + 208));
    float* o = out + b * 256;
    for (int c = 0; c < 256; c += 128) {
      int qloff = c / 2, qhoff = c / 4, scoff = c / 16;
      for (int l = 0; l < 32; l++) {
        int is = l / 16;
        int8_t q1 = (int8_t)((ql[qloff + l] & 0xF) | (((qh[qhoff + l] >> 0) & 3) << 4)) - 32;
        int8_t q2 = (int8_t)((ql[qloff + l + 32] & 0xF) | (((qh[qhoff + l] >> 2) & 3) << 4)) - 32;
        int8_t q3 = (int8_t)((ql[qloff + l] >> 4) | (((qh[qhoff + l] >> 4) & 3) << 4)) - 32;
        int8_t q4 = (int8_t)((ql[qloff + l + 32] >> 4) | (((qh[qhoff + l] >> 6) & 3) << 4)) - 32;
        int8_t s0 = (int8_t)scales[scoff + is + 0], s2 = (int8_t)scales[scoff + is + 2];
        int8_t s4 = (int8_t)scales[scoff + is + 4], s6 = (int8_t)scales[scoff + is + 6];
        o[c + l] = d * (float)s0 * (float)q1;
        o[c + l + 32] = d * (float)s2 * (float)q2;
        o[c + l + 64] = d * (float)s4 * (float)q3;
        o[c + l + 96] = d * (float)s6 * (float)q4;
      }
    }
  }
}

/* Type switch of DequantWeightMatrix (internal/ggml/gemm.go:221-267): 8 / 12 / 13,15,16 / 14 / 0.
 * Returns 0 on success, -1 for a type the reference does not handle. */
int32_t orc_dequant(int32_t type, const uint8_t* data, int64_t n, float* out) {
  switch (type) {
    case ORC_F32: memcpy(out, data, (size_t)n * 4); return 0;
    case ORC_Q8_0: deq_q8_0(data, n, out); return 0;
    case ORC_Q4_K: deq_q4_k(data, n, out); return 0;
    case ORC_Q5_K: case 15: case 16: deq_q5_k(data, n, out); return 0;
    case ORC_Q6_K: deq_q6_k(data, n, out); return 0;
    default: return -1;
  }
}

/* ------------------------------------------------------------------------- */
/* Elementwise ops: internal/ggml/ops_simd.go */

/* LayerNormInPlace: ops_simd.go:7-24 */
void orc_layernorm(float* x, const float* w, const float* b, float eps, int32_t n) {
  float nf = (float)n;
  float sum = 0.0f, sumsq = 0.0f;
  for (int i = 0; i < n; i++) {
    sum += x[i];
    sumsq += x[i] * x[i];
  }
  float mean = sum / nf;
  float var = sumsq / nf - mean * mean;
  float inv = (float)(1.0 / sqrt((double)(var + eps)));
  for (int i = 0; i < n; i++) x[i] = (x[i] - mean) * inv * w[i] + b[i];
}

/* GeLUInPlace: ops_simd.go:27-42 (rational tanh, clamp at |t| > 4.97) */
void orc_gelu(float* x, int32_t n) {
  const float c0 = 0.7978845608f, c1 = 0.044715f;
  for (int i = 0; i < n; i++) {
    float v = x[i];
    float t = c0 * v * (1.0f + c1 * v * v);
    float t2 = t * t;
    float th = t * (27.0f + t2) / (27.0f + 9.0f * t2);
    if (t > 4.97f)
      th = 1.0f;
    else if (t < -4.97f)
      th = -1.0f;
    x[i] = 0.5f * v * (1.0f + th);
  }
}

/* fastExp: ops_simd.go:70-82 */
static inline float fast_exp(float x) {
  if (x < -10.0f) return 0.0f;
  return (float)exp((double)x);
}

/* SoftmaxInPlace: ops_simd.go:46-66 */
void orc_softmax(float* x, int32_t n) {
  float mx = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  float sum = 0.0f;
  for (int i = 0; i < n; i++) {
    x[i] = fast_exp(x[i] - mx);
    sum += x[i];
  }
  float inv = 1.0f / sum;
  for (int i = 0; i < n; i++) x[i] *= inv;
}

/* DotF32: ops_simd.go:85-97 (unroll 4: sum += ((a0b0 + a1b1) + a2b2) + a3b3) */
float orc_dotf32(const float* a, const float* b, int32_t n) {
  float sum = 0.0f;
  int i = 0;
  for (; i <= n - 4; i += 4) sum += a[i] * b[i] + a[i + 1] * b[i + 1] + a[i + 2] * b[i + 2] + a[i + 3] * b[i + 3];
  for (; i < n; i++) sum += a[i] * b[i];
  return sum;
}

/* NewRoPETable: ops_simd.go:107-124. Tables are [max_pos][head_dim/2]. */
void orc_rope_table(int32_t max_pos, int32_t head_dim, float base, float* cos_tab, float* sin_tab) {
  int n_rot = head_dim / 2;
  for (int pos = 0; pos < max_pos; pos++) {
    for (int i = 0; i < n_rot; i++) {
      float freq = 1.0f / (float)pow((double)base, (double)(2 * i) / (double)head_dim);
      float theta = freq * (float)pos;
      cos_tab[(int64_t)pos * n_rot + i] = (float)cos((double)theta);
      sin_tab[(int64_t)pos * n_rot + i] = (float)sin((double)theta);
    }
  }
}

/* RoPETable.ApplyInPlace: ops_simd.go:127-137 (interleaved pairs 2i, 2i+1) */
void orc_rope_apply(float* x, const float* c, const float* s, int32_t n_rot) {
  for (int i = 0; i < n_rot; i++) {
    float x0 = x[2 * i], x1 = x[2 * i + 1];
    x[2 * i] = x0 * c[i] - x1 * s[i];
    x[2 * i + 1] = x0 * s[i] + x1 * c[i];
  }
}

/* MeanPool: internal/embed/pool.go:8-34 (rows with mask == 1, f32 sums in row order) */
void orc_mean_pool(const float* h, const int32_t* mask, int32_t L, int32_t dim, float* out) {
  for (int j = 0; j < dim; j++) out[j] = 0.0f;
  float count = 0.0f;
  for (int i = 0; i < L; i++) {
    if (mask[i] == 1) {
      for (int j = 0; j < dim; j++) out[j] += h[(int64_t)i * dim + j];
      count++;
    }
  }
  if (count == 0.0f) return;
  float inv = 1.0f / count;
  for (int j = 0; j < dim; j++) out[j] *= inv;
}

/* L2Normalize: internal/embed/pool.go:37-54 (f64 sum of squares) */
void orc_l2_normalize(const float* v, int32_t n, float* out) {
  double norm = 0.0;
  for (int i = 0; i < n; i++) norm += (double)v[i] * (double)v[i];
  norm = sqrt(norm);
  if (norm == 0.0) {
    if (out != v) memcpy(out, v, (size_t)n * 4);
    return;
  }
  float inv = (float)(1.0 / norm);
  for (int i = 0; i < n; i++) out[i] = v[i] * inv;
}

/* ------------------------------------------------------------------------- */
/* GEMM in GemmPrePacked32 order: internal/ggml/gemm_avx512.go:67-147 with the
 * micro-kernel internal/ggml/gemm_avx512_amd64.s:22-195.
 * B panels are PrePackBPanel32 layout [N/32][K][32] (gemm_avx512.go:47-64).
 * For each 32-column panel, each KC=128 chunk of K and each full 6-row tile:
 *   acc = 0; for k in chunk: acc = fma(A[r][k], B[k][j], acc); C += acc.
 * Rows past the last full 6-row tile take the scalar edge loop (no FMA):
 *   sum = 0; for k in chunk: sum += A[r][k]*B[k][j]; C += sum. */
#define MR 6
#define NR 32
#define KC 128

__attribute__((target_clones("avx512f", "avx2", "default"))) static void micro_6x32(
    const float* apack, const float* bp, float* c, int kc, int ldc) {
  float acc[MR][NR];
  for (int r = 0; r < MR; r++)
    for (int j = 0; j < NR; j++) acc[r][j] = 0.0f;
  for (int k = 0; k < kc; k++) {
    const float* b = bp + (int64_t)k * NR;
    for (int r = 0; r < MR; r++) {
      float a = apack[k * MR + r];
      for (int j = 0; j < NR; j++) acc[r][j] = fmaf(a, b[j], acc[r][j]);
    }
  }
  for (int r = 0; r < MR; r++)
    for (int j = 0; j < NR; j++) c[(int64_t)r * ldc + j] = acc[r][j] + c[(int64_t)r * ldc + j];
}

typedef struct {
  const float* A;
  const float* Bp;
  float* C;
  int M, N, K, p0, p1;
} gemm_job;

static void gemm_panels(const gemm_job* g) {
  float apack[MR * KC];
  const int M = g->M, N = g->N, K = g->K;
  for (int p = g->p0; p < g->p1; p++) {
    int j = p * NR;
    int nr = (j + NR > N) ? N - j : NR;
    for (int kc = 0; kc < K; kc += KC) {
      int kcl = (kc + KC > K) ? K - kc : KC;
      const float* bo = g->Bp + (int64_t)p * K * NR + (int64_t)kc * NR;
      for (int i = 0; i < M; i += MR) {
        int mr = (i + MR > M) ? M - i : MR;
        if (mr == MR && nr == NR) {
          int idx = 0;
          for (int kk = kc; kk < kc + kcl; kk++)
            for (int m = 0; m < MR; m++) apack[idx++] = g->A[(int64_t)(i + m) * K + kk];
          micro_6x32(apack, bo, g->C + (int64_t)i * N + j, kcl, N);
        } else {
          const float* po = g->Bp + (int64_t)p * K * NR;
          for (int ii = i; ii < i + mr && ii < M; ii++) {
            for (int jj = 0; jj < nr && j + jj < N; jj++) {
              float sum = 0.0f;
              for (int k = kc; k < kc + kcl; k++) sum += g->A[(int64_t)ii * K + k] * po[(int64_t)k * NR + jj];
              g->C[(int64_t)ii * N + j + jj] += sum;
            }
          }
        }
      }
    }
  }
}

static void* gemm_thread(void* arg) {
  gemm_panels((const gemm_job*)arg);
  return NULL;
}

static int default_workers(void) {
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  if (n > 8) return 8; /* NumWorkers: internal/ggml/ops_fast.go:217-226 */
  if (n < 2) return 1;
  return (int)n;
}

/* Panel-split driver; Bp in [N/32][K][32] layout. */
static void gemm_packed(const float* A, int M, int K, const float* Bp, int N, float* C, int nw) {
  memset(C, 0, sizeof(float) * (size_t)M * N);
  int panels = (N + NR - 1) / NR;
  if (nw <= 0) nw = default_workers();
  int ppw = (panels + nw - 1) / nw;
  gemm_job jobs[64];
  pthread_t th[64];
  int nj = 0;
  for (int w = 0; w < nw && w < 64; w++) {
    int p0 = w * ppw, p1 = p0 + ppw;
    if (p1 > panels) p1 = panels;
    if (p0 >= panels) break;
    jobs[nj] = (gemm_job){A, Bp, C, M, N, K, p0, p1};
    nj++;
  }
  if (nj == 1) {
    gemm_panels(&jobs[0]);
    return;
  }
  for (int t = 0; t < nj; t++) pthread_create(&th[t], NULL, gemm_thread, &jobs[t]);
  for (int t = 0; t < nj; t++) pthread_join(th[t], NULL);
}

static float* pack_panels(const float* B, int K, int N) {
  int panels = (N + NR - 1) / NR;
  float* pp = (float*)calloc((size_t)panels * K * NR, sizeof(float));
  for (int p = 0; p < panels; p++)
    for (int k = 0; k < K; k++)
      for (int n = 0; n < NR; n++) {
        int col = p * NR + n;
        if (col < N) pp[(int64_t)p * K * NR + (int64_t)k * NR + n] = B[(int64_t)col * K + k];
      }
  return pp;
}

void orc_gemm(const float* A, int32_t M, int32_t K, const float* B, int32_t N, float* C, int32_t nt) {
  float* pp = pack_panels(B, K, N);
  gemm_packed(A, M, K, pp, N, C, nt);
  free(pp);
}

/* ------------------------------------------------------------------------- */
/* Model: LoadBertModel + PreDequant (internal/embed/bert.go:91-212, 542-576) */

typedef struct {
  float *qkv, *out, *up, *gate, *down; /* PrePackBPanel32 panels */
  float *anw, *anb, *onw, *onb;
} orc_layer;

struct orc_model {
  int n_layer, d, n_head, head_dim, d_ff, max_seq;
  float eps, rope_base;
  orc_tensor token_embd;
  float* type0; /* token_types row 0 */
  float *enw, *enb;
  orc_layer* layers;
  float *rope_cos, *rope_sin;
  int n_qkv;
  int gemm_threads, attn_threads;
};

/* Tensor.Dequantize for small vectors (internal/ggml/tensor.go:51-66): 0/8/12/13/14 only. */
static float* load_vec(const orc_tensor* t, int n) {
  if (!(t->type == 0 || t->type == 8 || t->type == 12 || t->type == 13 || t->type == 14)) return NULL;
  float* v = (float*)malloc(sizeof(float) * (size_t)n);
  orc_dequant(t->type, t->data, n, v);
  return v;
}

/* DequantWeightMatrix: unknown types leave the matrix zero, as the reference's switch does. */
static float* load_mat(const orc_tensor* t, int K, int N) {
  float* w = (float*)calloc((size_t)N * K, sizeof(float));
  int64_t rb = orc_row_bytes(t->type, K);
  if (rb > 0)
    for (int n = 0; n < N; n++) orc_dequant(t->type, t->data + (int64_t)n * rb, K, w + (int64_t)n * K);
  float* pp = pack_panels(w, K, N);
  free(w);
  return pp;
}

int32_t orc_model_create(const orc_model_desc* d, orc_model** out) {
  if (d->n_layer <= 0 || d->d_model <= 0) return -1;
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  m->n_layer = d->n_layer;
  m->d = d->d_model;
  m->n_head = d->n_head;
  m->head_dim = d->d_model / d->n_head;
  m->d_ff = d->d_ff;
  m->max_seq = d->max_seq;
  m->eps = d->ln_eps;
  m->rope_base = d->rope_base;
  m->token_embd = d->token_embd;
  const int D = m->d;
  m->type0 = (float*)malloc(sizeof(float) * D);
  if (d->token_types.type == 0)
    memcpy(m->type0, d->token_types.data, sizeof(float) * D);
  else
    orc_dequant(d->token_types.type, d->token_types.data, D, m->type0);
  m->enw = load_vec(&d->embd_norm_w, D);
  m->enb = load_vec(&d->embd_norm_b, D);
  m->n_qkv = (int)d->qkv[0].ne1;
  m->layers = (orc_layer*)calloc((size_t)m->n_layer, sizeof(orc_layer));
  for (int l = 0; l < m->n_layer; l++) {
    orc_layer* L = &m->layers[l];
    L->qkv = load_mat(&d->qkv[l], D, (int)d->qkv[l].ne1);
    L->out = load_mat(&d->out[l], D, (int)d->out[l].ne1);
    L->up = load_mat(&d->up[l], D, (int)d->up[l].ne1);
    L->gate = load_mat(&d->gate[l], D, (int)d->gate[l].ne1);
    L->down = load_mat(&d->down[l], m->d_ff, (int)d->down[l].ne1);
    L->anw = load_vec(&d->attn_norm_w[l], D);
    L->anb = load_vec(&d->attn_norm_b[l], D);
    L->onw = load_vec(&d->out_norm_w[l], D);
    L->onb = load_vec(&d->out_norm_b[l], D);
  }
  int nrot = m->head_dim / 2;
  m->rope_cos = (float*)malloc(sizeof(float) * (size_t)m->max_seq * nrot);
  m->rope_sin = (float*)malloc(sizeof(float) * (size_t)m->max_seq * nrot);
  orc_rope_table(m->max_seq, m->head_dim, m->rope_base, m->rope_cos, m->rope_sin);
  m->gemm_threads = 0;
  m->attn_threads = 0;
  *out = m;
  return 0;
}

void orc_model_destroy(orc_model* m) {
  if (!m) return;
  for (int l = 0; l < m->n_layer; l++) {
    orc_layer* L = &m->layers[l];
    free(L->qkv); free(L->out); free(L->up); free(L->gate); free(L->down);
    free(L->anw); free(L->anb); free(L->onw); free(L->onb);
  }
  free(m->layers);
  free(m->type0); free(m->enw); free(m->enb);
  free(m->rope_cos); free(m->rope_sin);
  free(m);
}

void orc_set_threads(orc_model* m, int32_t g, int32_t a) {
  m->gemm_threads = g;
  m->attn_threads = a;
}

/* getEmbedding: internal/embed/bert.go:290-316 */
static int get_embedding(const orc_tensor* t, int idx, int dim, float* out) {
  int64_t rb;
  switch (t->type) {
    case 0: case 8: case 12: case 13: case 14: rb = orc_row_bytes(t->type, dim); break;
    default: return -1;
  }
  if (idx < 0 || (int64_t)(idx + 1) * rb > t->nbytes) return -1;
  orc_dequant(t->type, t->data + (int64_t)idx * rb, dim, out);
  return 0;
}

typedef struct {
  const orc_model* m;
  const float *Q, *K, *V;
  const int32_t* mask;
  float* out;
  int L, h0, h1;
} attn_job;

/* Per-head attention body: internal/embed/bert.go:364-402 */
static void* attn_heads(void* arg) {
  const attn_job* a = (const attn_job*)arg;
  const int D = a->m->d, hd = a->m->head_dim, L = a->L;
  const float scale = (float)(1.0 / sqrt((double)hd));
  float* scores = (float*)malloc(sizeof(float) * (size_t)L);
  for (int h = a->h0; h < a->h1; h++) {
    int off = h * hd;
    for (int qi = 0; qi < L; qi++) {
      for (int ki = 0; ki < L; ki++)
        scores[ki] = orc_dotf32(a->Q + (int64_t)qi * D + off, a->K + (int64_t)ki * D + off, hd) * scale;
      for (int ki = 0; ki < L; ki++)
        if (a->mask[ki] == 0) scores[ki] = -1e9f;
      orc_softmax(scores, L);
      for (int dd = 0; dd < hd; dd++) {
        float sum = 0.0f;
        for (int vi = 0; vi < L; vi++) sum += scores[vi] * a->V[(int64_t)vi * D + off + dd];
        a->out[(int64_t)qi * D + off + dd] = sum;
      }
    }
  }
  free(scores);
  return NULL;
}

/* Forward: internal/embed/bert.go:216-285 */
int32_t orc_forward(orc_model* m, const int32_t* ids, const int32_t* mask, int32_t L, float* hid) {
  const int D = m->d, H = m->n_head, hd = m->head_dim, F = m->d_ff, NQ = m->n_qkv;
  if (L <= 0 || L > m->max_seq) return -1;
  for (int i = 0; i < L; i++) {
    if (get_embedding(&m->token_embd, ids[i], D, hid + (int64_t)i * D)) return -2;
    for (int j = 0; j < D; j++) hid[(int64_t)i * D + j] = hid[(int64_t)i * D + j] + m->type0[j];
    orc_layernorm(hid + (int64_t)i * D, m->enw, m->enb, m->eps, D);
  }
  float* qkv = (float*)malloc(sizeof(float) * (size_t)L * NQ);
  float *Q = (float*)malloc(sizeof(float) * (size_t)L * D), *K = (float*)malloc(sizeof(float) * (size_t)L * D),
        *V = (float*)malloc(sizeof(float) * (size_t)L * D);
  float* att = (float*)malloc(sizeof(float) * (size_t)L * D);
  float* tmp = (float*)malloc(sizeof(float) * (size_t)L * D);
  float* ups = (float*)malloc(sizeof(float) * (size_t)L * F);
  float* gates = (float*)malloc(sizeof(float) * (size_t)L * F);
  const int nrot = hd / 2;
  int nat = m->attn_threads > 0 ? m->attn_threads : H;
  if (nat > H) nat = H;
  for (int l = 0; l < m->n_layer; l++) {
    const orc_layer* Ly = &m->layers[l];
    /* multiHeadAttention: bert.go:319-411 */
    gemm_packed(hid, L, D, Ly->qkv, NQ, qkv, m->gemm_threads);
    for (int i = 0; i < L; i++) {
      memcpy(Q + (int64_t)i * D, qkv + (int64_t)i * NQ, sizeof(float) * D);
      memcpy(K + (int64_t)i * D, qkv + (int64_t)i * NQ + D, sizeof(float) * D);
      memcpy(V + (int64_t)i * D, qkv + (int64_t)i * NQ + 2 * D, sizeof(float) * D);
      for (int h = 0; h < H; h++) {
        orc_rope_apply(Q + (int64_t)i * D + h * hd, m->rope_cos + (int64_t)i * nrot, m->rope_sin + (int64_t)i * nrot, nrot);
        orc_rope_apply(K + (int64_t)i * D + h * hd, m->rope_cos + (int64_t)i * nrot, m->rope_sin + (int64_t)i * nrot, nrot);
      }
    }
    attn_job jobs[64];
    pthread_t th[64];
    int per = (H + nat - 1) / nat, nj = 0;
    for (int t = 0; t < nat && t < 64; t++) {
      int h0 = t * per, h1 = h0 + per;
      if (h1 > H) h1 = H;
      if (h0 >= H) break;
      jobs[nj++] = (attn_job){m, Q, K, V, mask, att, L, h0, h1};
    }
    if (nj == 1)
      attn_heads(&jobs[0]);
    else {
      for (int t = 0; t < nj; t++) pthread_create(&th[t], NULL, attn_heads, &jobs[t]);
      for (int t = 0; t < nj; t++) pthread_join(th[t], NULL);
    }
    gemm_packed(att, L, D, Ly->out, D, tmp, m->gemm_threads);
    /* Residual + LayerNorm: bert.go:261-267 */
    for (int i = 0; i < L; i++) {
      for (int j = 0; j < D; j++) hid[(int64_t)i * D + j] += tmp[(int64_t)i * D + j];
      orc_layernorm(hid + (int64_t)i * D, Ly->anw, Ly->anb, m->eps, D);
    }
    /* ffnForward: bert.go:415-445 */
    gemm_packed(hid, L, D, Ly->up, F, ups, m->gemm_threads);
    gemm_packed(hid, L, D, Ly->gate, F, gates, m->gemm_threads);
    for (int i = 0; i < L; i++) {
      orc_gelu(gates + (int64_t)i * F, F);
      for (int j = 0; j < F; j++) gates[(int64_t)i * F + j] *= ups[(int64_t)i * F + j];
    }
    gemm_packed(gates, L, F, Ly->down, D, tmp, m->gemm_threads);
    /* Residual + LayerNorm: bert.go:275-281 */
    for (int i = 0; i < L; i++) {
      for (int j = 0; j < D; j++) hid[(int64_t)i * D + j] += tmp[(int64_t)i * D + j];
      orc_layernorm(hid + (int64_t)i * D, Ly->onw, Ly->onb, m->eps, D);
    }
  }
  free(qkv); free(Q); free(K); free(V); free(att); free(tmp); free(ups); free(gates);
  return 0;
}

/* Embed: internal/embed/embedder.go:46-71 */
int32_t orc_embed(orc_model* m, const int32_t* ids, const int32_t* mask, int32_t L, int32_t out_dim, float* out) {
  const int D = m->d;
  if (L <= 0 || L > m->max_seq) return -1;
  float* hid = (float*)malloc(sizeof(float) * (size_t)L * D);
  int rc = orc_forward(m, ids, mask, L, hid);
  if (rc) {
    free(hid);
    return rc;
  }
  float pooled[4096], normed[4096];
  orc_mean_pool(hid, mask, L, D, pooled);
  orc_l2_normalize(pooled, D, normed);
  if (out_dim > D) out_dim = D; /* SetTargetDim clamp: embedder.go:142-150 */
  if (out_dim < 1) out_dim = 1;
  if (out_dim < D)
    orc_l2_normalize(normed, out_dim, out);
  else
    memcpy(out, normed, sizeof(float) * D);
  free(hid);
  return 0;
}

typedef struct {
  orc_model* m;
  const int32_t *ids, *mask;
  int B, L, out_dim;
  float* out;
  int* next;
  pthread_mutex_t* mu;
  int* rc;
} batch_job;

static void* batch_worker(void* arg) {
  batch_job* j = (batch_job*)arg;
  for (;;) {
    pthread_mutex_lock(j->mu);
    int i = (*j->next)++;
    pthread_mutex_unlock(j->mu);
    if (i >= j->B) break;
    const int32_t* mk = j->mask + (int64_t)i * j->L;
    /* The reference's EmbedBatch embeds each text at its own (unpadded) length;
     * trailing padding positions are dropped to reproduce that. */
    int len = j->L;
    while (len > 0 && mk[len - 1] == 0) len--;
    int od = j->out_dim < j->m->d ? j->out_dim : j->m->d;
    int r = len > 0 ? orc_embed(j->m, j->ids + (int64_t)i * j->L, mk, len, j->out_dim, j->out + (int64_t)i * od) : -1;
    if (r) j->rc[i] = r;
  }
  return NULL;
}

/* EmbedBatch: internal/embed/embedder.go:75-133 (min(nproc, n, 8) workers, first error wins) */
int32_t orc_embed_batch(orc_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t L,
                        int32_t out_dim, float* out, int32_t nw) {
  if (B <= 0) return 0;
  if (nw <= 0) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    nw = (int)n;
    if (nw > B) nw = B;
    if (nw > 8) nw = 8;
  }
  if (nw > 64) nw = 64;
  int next = 0;
  pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
  int* rc = (int*)calloc((size_t)B, sizeof(int));
  batch_job job = {m, ids, mask, B, L, out_dim, out, &next, &mu, rc};
  pthread_t th[64];
  for (int t = 0; t < nw; t++) pthread_create(&th[t], NULL, batch_worker, &job);
  for (int t = 0; t < nw; t++) pthread_join(th[t], NULL);
  int r = 0;
  for (int i = 0; i < B; i++)
    if (rc[i]) {
      r = rc[i];
      break;
    }
  free(rc);
  return r;
}
