// Host runtime of libllmembed_hip.so: device probe, model upload, forward orchestration and
// the C-ABI entry points declared in include/llmembed.h.
//
// Mirrors the reference's model lifecycle:
//   LoadBertModel + PreDequant + NewRoPETable (internal/embed/bert.go:91-212,542-576,
//   internal/embed/embedder.go:19-42)  ->  lle_model_create / lle_model_load_gguf
//   Embed / EmbedBatch (internal/embed/embedder.go:46-133)  ->  lle_embed / lle_embed_batch
//   BertModel.Forward (internal/embed/bert.go:216-285)      ->  forward() below
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <climits>
#include <mutex>
#include <string>
#include <vector>

#include "lle_internal.h"
#include "tokenizer.h"

namespace lle {

static thread_local std::string g_err;
void set_error(const std::string& m) { g_err = m; }
int fail(int code, const std::string& m) {
  g_err = m;
  return code;
}

static int g_device = -1;
static std::mutex g_init_mu;

static int64_t row_bytes(int type, int64_t n) {
  switch (type) {
    case 0: return n * 4;
    case 8: return (n / 32) * 34;
    case 12: return (n / 256) * 144;
    case 13: case 15: case 16: return (n / 256) * 176;
    case 14: return (n / 256) * 210;
    default: return -1;
  }
}

static int ensure_init() {
  if (g_device >= 0) return LLE_OK;
  return lle_init(0);
}

struct Timer {
  std::string name;
  hipEvent_t a, b;
  double flops, bytes;
};

struct Layer {
  WeightDev qkv, out, upgate, down;
  float *anw = nullptr, *anb = nullptr, *onw = nullptr, *onb = nullptr;
};

// Activation buffers of one forward (device pointers). The model owns a grow-only set; the
// no-allocation entry carves one out of a fixed device array instead.
struct Workspace {
  float* h = nullptr;   // residual stream f32 [rows][D]
  float* h2 = nullptr;  // second residual buffer of the small-batch schedule [16][D]
  __half* h16 = nullptr;  // f16 copy of h (GEMM input)
  __half *q = nullptr, *k = nullptr, *vt = nullptr;  // [B][H][Lp][64] / [B][H][64][Lp]
  __half *attn = nullptr, *ff = nullptr;             // [rows][D], [rows][F]
  float* part = nullptr;                             // split-K partials below 1024 rows
  int32_t *ids = nullptr, *mask = nullptr, *tokrow = nullptr, *seq_off = nullptr;
  float* out = nullptr;  // [B][D] embeddings of host-pointer calls
};

}  // namespace lle

struct lle_weight {
  lle::WeightDev w;
  int device = 0;
  hipStream_t stream = nullptr;
};

struct lle_model {
  int device = 0;
  int n_layer = 0, D = 0, H = 0, F = 0, max_seq = 0, vocab = 0;
  float eps = 0.f, rope_base = 0.f;
  uint8_t* tok = nullptr;
  int tok_type = 0;
  int64_t tok_row_bytes = 0;
  float *type0 = nullptr, *enw = nullptr, *enb = nullptr;
  std::vector<lle::Layer> layers;
  // LLE_PRECISION_F32: f32 copies of the dequantised projection weights ([N][K] per layer:
  // qkv, out, up||gate interleaved, down) and the f32 activations of the exact forward
  int precision = LLE_PRECISION_F16;
  std::vector<float*> w32;  // 4 per layer
  size_t ex_T = 0;
  float *ex_h = nullptr, *ex_q = nullptr, *ex_k = nullptr, *ex_v = nullptr, *ex_att = nullptr, *ex_g = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  std::vector<void*> allocs;
  hipStream_t stream = nullptr;
  std::mutex mu;
  // workspace (grow-only)
  size_t ws_T = 0, ws_heads = 0, ws_part = 0;
  int ws_B = 0;
  lle::Workspace ws;
  int32_t* status = nullptr;  // device status word of async forwards (bits, see lle_model_status)
  // HIP graphs of small forwards, keyed by shape, rows and pointers. A key is captured
  // the second time it runs (a one-off shape, e.g. one text's length, stays eager) and entries
  // are evicted least recently used first.
  struct GraphEntry {
    int B, L, T, out_dim;
    const void *ids, *mask;
    void* out;
    hipGraphExec_t exec;  // null: seen once, not captured yet
    uint64_t last_use;
  };
  std::vector<GraphEntry> graphs;
  uint64_t graph_tick = 0;
  bool use_graphs = true;
  // Forwards share the workspace, so each is ordered after the previous one: ev_last marks the
  // end of the last forward enqueued, on last_stream; a forward on another stream waits for it.
  hipEvent_t ev_last = nullptr;
  hipStream_t last_stream = nullptr;
  bool ev_last_valid = false;
  // timing
  bool timing = false;
  std::string timing_only;  // non-empty: only this kernel class is bracketed, read at get_timing
  std::vector<lle::Timer> pending;
  std::vector<lle_kernel_time> totals;
  std::vector<hipEvent_t> event_pool;
};

namespace lle {

static int dev_alloc(lle_model* m, void** p, size_t bytes) {
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return fail(LLE_ENOMEM, std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e));
  m->allocs.push_back(*p);
  return LLE_OK;
}

static void clear_graphs(lle_model* m) {
  for (auto& g : m->graphs)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  m->graphs.clear();
}

static void ws_free(lle_model* m) {
  clear_graphs(m);
  Workspace& w = m->ws;
  void* bufs[] = {w.h, w.h2, w.h16, w.q, w.k, w.vt, w.attn, w.ff, w.part, w.ids, w.mask, w.tokrow, w.seq_off, w.out};
  for (void* b : bufs)
    if (b) (void)hipFree(b);
  w = Workspace{};
  m->ws_T = m->ws_heads = m->ws_part = 0;
  m->ws_B = 0;
}

#define WS_ALLOC(ptr, bytes)                                                            \
  do {                                                                                  \
    void* p_ = nullptr;                                                                 \
    hipError_t e_ = hipMalloc(&p_, (bytes) ? (bytes) : 256);                            \
    if (e_ != hipSuccess) {                                                             \
      ws_free(m);                                                                       \
      return fail(LLE_ENOMEM, std::string("workspace hipMalloc: ") + hipGetErrorString(e_)); \
    }                                                                                   \
    ptr = (decltype(ptr))p_;                                                            \
  } while (0)

static int wait_forwards(lle_model* m);

// Grow-only workspace for a [B][L] batch whose forward runs on `rows` token rows (B*L, or fewer
// when padding is packed away).
static int ensure_ws(lle_model* m, int B, int L, int64_t rows = -1) {
  const size_t T = (size_t)B * L;
  const int Lp = (L + 63) / 64 * 64;
  const size_t heads = (size_t)B * m->H * Lp * 64;
  auto nch = [](int K) { return (size_t)(K % 768 == 0 ? K / 768 : K / 256); };
  const size_t kd = nch(m->D), kf = nch(m->F);
  const size_t R = rows < 0 ? T : (size_t)rows;
  // split-K partials of the GEMMs below 1024 rows: chunks x rows x N floats
  const size_t part = R < 1024 ? std::max<size_t>(R, 64) * std::max({kd * 3 * m->D, kd * 2 * m->F, kf * m->D}) : 0;
  if (T <= m->ws_T && heads <= m->ws_heads && part <= m->ws_part && B <= m->ws_B) return LLE_OK;
  const size_t nT = std::max(T, m->ws_T), nH = std::max(heads, m->ws_heads), nP = std::max(part, m->ws_part);
  const int nB = std::max(B, m->ws_B);
  if (int rc = wait_forwards(m)) return rc;
  ws_free(m);
  Workspace& w = m->ws;
  WS_ALLOC(w.h, nT * m->D * 4);
  WS_ALLOC(w.h2, (size_t)16 * m->D * 4);
  WS_ALLOC(w.h16, nT * m->D * 2);
  WS_ALLOC(w.q, nH * 2);
  WS_ALLOC(w.k, nH * 2);
  WS_ALLOC(w.vt, nH * 2);
  WS_ALLOC(w.attn, nT * m->D * 2);
  WS_ALLOC(w.ff, nT * m->F * 2);
  if (nP) WS_ALLOC(w.part, nP * 4);
  WS_ALLOC(w.ids, nT * 4);
  WS_ALLOC(w.mask, nT * 4);
  WS_ALLOC(w.tokrow, nT * 4);
  WS_ALLOC(w.seq_off, ((size_t)nB + 1) * 4);
  WS_ALLOC(w.out, (size_t)nB * m->D * 4);
  m->ws_T = nT;
  m->ws_heads = nH;
  m->ws_part = nP;
  m->ws_B = nB;
  return LLE_OK;
}

static hipEvent_t get_event(lle_model* m) {
  if (!m->event_pool.empty()) {
    hipEvent_t e = m->event_pool.back();
    m->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  (void)hipEventCreate(&e);
  return e;
}

static void collect_timing(lle_model* m);

struct Scope {
  lle_model* m;
  hipStream_t st;
  Timer t;
  bool on;
  Scope(lle_model* m_, hipStream_t st_, const char* name, double flops, double bytes, bool allowed = true)
      : m(m_), st(st_), on(allowed && m_->timing && (m_->timing_only.empty() || m_->timing_only == name)) {
    if (on) {
      t.name = name;
      t.flops = flops;
      t.bytes = bytes;
      t.a = get_event(m);
      t.b = get_event(m);
      (void)hipEventRecord(t.a, st);
    }
  }
  ~Scope() {
    if (on) {
      (void)hipEventRecord(t.b, st);
      m->pending.push_back(t);
      // single-class mode reads its events at lle_model_get_timing; a caller that never reads
      // them is bounded here (the totals keep accumulating)
      if (m->pending.size() >= 4096) {
        (void)hipStreamSynchronize(st);
        collect_timing(m);
      }
    }
  }
};

static void collect_timing(lle_model* m) {
  for (auto& t : m->pending) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, t.a, t.b) != hipSuccess) ms = 0.f;
    auto it = std::find_if(m->totals.begin(), m->totals.end(),
                           [&](const lle_kernel_time& k) { return t.name == k.name; });
    if (it == m->totals.end()) {
      lle_kernel_time k;
      memset(&k, 0, sizeof(k));
      snprintf(k.name, sizeof(k.name), "%s", t.name.c_str());
      m->totals.push_back(k);
      it = m->totals.end() - 1;
    }
    it->launches += 1;
    it->total_ms += ms;
    it->flops += t.flops;
    it->bytes += t.bytes;
    m->event_pool.push_back(t.a);
    m->event_pool.push_back(t.b);
  }
  m->pending.clear();
}

#define LAUNCH(expr)                                                                 \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess) return fail(LLE_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

static double wbytes(const WeightDev& w) { return (double)w.bytes; }

// BertModel.Forward (internal/embed/bert.go:216-285) for B right-padded rows of length L,
// followed (when out != nullptr) by MeanPool + L2Normalize (+ Matryoshka).
// Packed rows of a padded [B][L] batch: only positions up to each sequence's last valid token
// are computed (rows of masked positions after it never reach a valid row: attention gives them
// weight 0 and the pool skips them). Row t is padded token tokrow[t]; sequence b owns rows
// seq_off[b] .. seq_off[b+1]-1. A sequence with no valid token keeps all L positions (its softmax
// is uniform over every key).
struct Packing {
  int T;
  const int32_t* tokrow;
  const int32_t* seq_off;
};

// Forwards of one model share its workspace, so each must run after the previous one on the
// device, whichever streams the callers use. Every forward ends by recording ev_last on its
// stream; a forward on a different stream first waits for that event (on one stream the order
// is already given, so a single-stream caller pays nothing). A stream that a caller is
// capturing into a graph is left alone: its graph defines its own order.
static bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}
static int order_begin(lle_model* m, hipStream_t st) {
  if (m->ev_last_valid && st != m->last_stream && !capturing(st)) LLE_HIP(hipStreamWaitEvent(st, m->ev_last, 0));
  return LLE_OK;
}
static int order_end(lle_model* m, hipStream_t st) {
  if (capturing(st)) return LLE_OK;
  LLE_HIP(hipEventRecord(m->ev_last, st));
  m->last_stream = st;
  m->ev_last_valid = true;
  return LLE_OK;
}
// Waits for every forward enqueued so far (before the workspace is freed or replaced).
static int wait_forwards(lle_model* m) {
  if (m->ev_last_valid) LLE_HIP(hipEventSynchronize(m->ev_last));
  LLE_HIP(hipStreamSynchronize(m->stream));
  return LLE_OK;
}

static void ex_free(lle_model* m) {
  float* bufs[] = {m->ex_h, m->ex_q, m->ex_k, m->ex_v, m->ex_att, m->ex_g};
  for (float* b : bufs)
    if (b) (void)hipFree(b);
  m->ex_h = m->ex_q = m->ex_k = m->ex_v = m->ex_att = m->ex_g = nullptr;
  m->ex_T = 0;
}

// f32 activations of the exact forward for `rows` token rows (grow-only).
static int ensure_exact_ws(lle_model* m, size_t rows) {
  if (rows <= m->ex_T) return LLE_OK;
  if (int rc = wait_forwards(m)) return rc;
  ex_free(m);
  const size_t D = m->D, F = m->F;
  float** dst[] = {&m->ex_h, &m->ex_q, &m->ex_k, &m->ex_v, &m->ex_att, &m->ex_g};
  const size_t n[] = {rows * D, rows * D, rows * D, rows * D, rows * D, rows * F};
  for (int i = 0; i < 6; i++) {
    hipError_t e = hipMalloc((void**)dst[i], std::max<size_t>(n[i], 64) * 4);
    if (e != hipSuccess) {
      ex_free(m);
      return fail(LLE_ENOMEM, std::string("exact workspace hipMalloc: ") + hipGetErrorString(e));
    }
  }
  m->ex_T = rows;
  return LLE_OK;
}

// BertModel.Forward in the reference's own f32 arithmetic (exact.hip), for B sequences of
// length L, or packed rows (pk): sequence b is rows seq_off[b] .. seq_off[b+1]-1 at its own
// length, as the reference embeds each text at its own length. The residual stream ends in
// m->ex_h; with d_out, MeanPool + L2Normalize (+ Matryoshka) into d_out.
static int forward_exact(lle_model* m, const int32_t* d_ids, const int32_t* d_mask, int B, int L, int out_dim,
                         float* d_out, hipStream_t st, const Packing* pk) {
  const int D = m->D, F = m->F, T = pk ? pk->T : B * L;
  int rc = ensure_exact_ws(m, (size_t)T);
  if (rc) return rc;
  ExactArgs a{};
  a.T = T;
  a.L = L;
  a.D = D;
  a.H = m->H;
  a.tokrow = pk ? pk->tokrow : nullptr;
  a.seq_off = pk ? pk->seq_off : nullptr;
  a.mask = d_mask;
  a.ids = d_ids;
  a.vocab = m->vocab;
  a.tok_type = m->tok_type;
  a.tok = m->tok;
  a.tok_row_bytes = m->tok_row_bytes;
  a.type0 = m->type0;
  a.status = m->status;
  a.eps = m->eps;
  a.h = m->ex_h;
  a.q = m->ex_q;
  a.k = m->ex_k;
  a.v = m->ex_v;
  a.att = m->ex_att;
  a.rope_cos = m->rope_cos;
  a.rope_sin = m->rope_sin;
  a.lnw = m->enw;
  a.lnb = m->enb;
  {
    Scope s(m, st, "embed_ln", 0, (double)T * (m->tok_row_bytes + D * 8));
    LAUNCH(launch_exact_embed(a, st));
  }
  for (int l = 0; l < m->n_layer; l++) {
    const Layer& ly = m->layers[l];
    float* const* w = &m->w32[(size_t)l * 4];
    {
      Scope s(m, st, "gemm_qkv", 2.0 * T * 3 * D * D, 3.0 * D * D * 4 + (double)T * D * 16);
      LAUNCH(launch_exact_gemm(a, ExactGemm{a.h, w[0], 3 * D, D, nullptr}, EPI_QKV, st));
    }
    {
      Scope s(m, st, "attention", 0, (double)T * D * 16);
      LAUNCH(launch_exact_attention(a, st));
    }
    {
      Scope s(m, st, "gemm_out_ln", 2.0 * T * D * D, (double)D * D * 4 + (double)T * D * 16);
      LAUNCH(launch_exact_gemm(a, ExactGemm{a.att, w[1], D, D, a.h}, EPI_RESID, st));
      a.lnw = ly.anw;
      a.lnb = ly.anb;
      LAUNCH(launch_exact_ln(a, st));
    }
    {
      Scope s(m, st, "gemm_upgate", 2.0 * T * 2 * F * D, 2.0 * F * D * 4 + (double)T * (D + F) * 4);
      LAUNCH(launch_exact_gemm(a, ExactGemm{a.h, w[2], 2 * F, D, m->ex_g}, EPI_GEGLU, st));
    }
    {
      Scope s(m, st, "gemm_down_ln", 2.0 * T * D * F, (double)D * F * 4 + (double)T * (F + 3 * D) * 4);
      LAUNCH(launch_exact_gemm(a, ExactGemm{m->ex_g, w[3], D, F, a.h}, EPI_RESID, st));
      a.lnw = ly.onw;
      a.lnb = ly.onb;
      LAUNCH(launch_exact_ln(a, st));
    }
  }
  if (d_out) {
    Scope s(m, st, "pool", 0, (double)T * D * 4);
    LAUNCH(launch_exact_pool(a, B, out_dim, d_out, st));
  }
  return LLE_OK;
}

// ids / mask / out are device pointers already placed in a workspace or the caller's; with
// `pk`, ids are the packed rows' ids and the mask stays [B][L]. The activations live in `w`;
// `timed` = false keeps the launches free of timing events (no host-side event creation).
static int forward(lle_model* m, const Workspace& w, const int32_t* d_ids, const int32_t* d_mask, int B, int L,
                   int out_dim, float* d_out, hipStream_t st, const Packing* pk = nullptr, bool timed = true) {
  if (m->precision == LLE_PRECISION_F32) return forward_exact(m, d_ids, d_mask, B, L, out_dim, d_out, st, pk);
  const int D = m->D, H = m->H, F = m->F;
  const int T = pk ? pk->T : B * L, Lp = (L + 63) / 64 * 64;
  const int32_t* tokrow = pk ? pk->tokrow : nullptr;
  const int32_t* seq_off = pk ? pk->seq_off : nullptr;
  {
    EmbedArgs a{d_ids, T, m->vocab, m->tok_type, m->tok, m->tok_row_bytes, m->type0, m->enw, m->enb, m->eps, D,
                w.h, w.h16, m->status};
    Scope s(m, st, "embed_ln", 0, (double)T * (m->tok_row_bytes + D * 6), timed);
    LAUNCH(launch_embed_ln(a, st));
  }
  // Batches of <= 16 tokens: each LayerNorm runs inside the GEMM that consumes it (every block
  // normalises the few rows itself, block 0 keeps the f32 rows for the next residual), which
  // removes two dependent kernels per layer. Residual stream: h (after attention) and h2 (after
  // the FFN input LayerNorm); the down projection leaves its four chunk partials for the next
  // layer's QKV prologue, and the last layer's go through one reduce + residual + LayerNorm.
  if (T <= 16 && D == 768 && F == 4 * 768) {
    for (int l = 0; l < m->n_layer; l++) {
      Layer& ly = m->layers[l];
      GemmArgs g{};
      g.M = T;
      g.rope_cos = m->rope_cos;
      g.rope_sin = m->rope_sin;
      g.L = L;
      g.Lp = Lp;
      g.n_head = H;
      g.d_model = D;
      g.part = w.part;
      g.tokrow = tokrow;
      {
        g.w = &ly.qkv;
        g.x = w.h16;
        g.q = w.q;
        g.k = w.k;
        g.vt = w.vt;
        Scope s(m, st, "gemm_qkv", 2.0 * T * ly.qkv.N * ly.qkv.K, wbytes(ly.qkv) + (double)T * (D * 2 + 3 * D * 2), timed);
        if (l == 0) {
          LAUNCH(launch_gemm(g, EPI_QKV, st));
        } else {
          const Layer& pv = m->layers[l - 1];
          const LnPrologue ln{w.h2, w.part, 4, pv.onw, pv.onb, m->eps, w.h};
          LAUNCH(launch_gemm_lnx(g, EPI_QKV, ln, st));
        }
      }
      {
        AttnArgs a{w.q, w.k, w.vt, d_mask, w.attn, B, L, Lp, H, D, seq_off};
        Scope s(m, st, "attention", 4.0 * B * (double)L * L * D, (double)T * D * 2 * 4, timed);
        LAUNCH(launch_attention(a, st));
      }
      {
        g.w = &ly.out;
        g.x = w.attn;
        g.y = w.h;
        Scope s(m, st, "gemm_out_ln", 2.0 * T * ly.out.N * ly.out.K, wbytes(ly.out) + (double)T * D * (2 + 8), timed);
        LAUNCH(launch_gemm(g, EPI_RESID, st));
      }
      {
        g.w = &ly.upgate;
        g.g = w.ff;
        const LnPrologue ln{w.h, nullptr, 0, ly.anw, ly.anb, m->eps, w.h2};
        Scope s(m, st, "gemm_upgate", 2.0 * T * ly.upgate.N * ly.upgate.K, wbytes(ly.upgate) + (double)T * (D * 4 + F * 2), timed);
        LAUNCH(launch_gemm_lnx(g, EPI_GEGLU, ln, st));
      }
      {
        g.w = &ly.down;
        g.x = w.ff;
        g.y = w.h2;
        Scope s(m, st, "gemm_down_ln", 2.0 * T * ly.down.N * ly.down.K, wbytes(ly.down) + (double)T * (F * 2 + D * 16), timed);
        LAUNCH(launch_gemm_partials(g, st));
      }
    }
    const Layer& last = m->layers[m->n_layer - 1];
    if (d_out) {  // the last LayerNorm's rows only feed the pool: one kernel, rows kept in LDS
      Scope s(m, st, "pool", 0, (double)T * D * 24, timed);
      LAUNCH(launch_reduce_ln_pool(w.part, 4, T, w.h2, last.onw, last.onb, m->eps, d_mask, seq_off, B, L, D,
                                   out_dim, d_out, st));
    } else {
      Scope s(m, st, "ln", 0, (double)T * D * 26, timed);
      LAUNCH(launch_reduce_resid_ln(w.part, 4, T, D, w.h2, w.h, w.h16, last.onw, last.onb, m->eps, st));
    }
    return LLE_OK;
  }
  bool pending = false;  // the residual rows hold a LayerNorm left pending (pend)
  LnDefer pend{};
  bool pooled = false;    // the last LayerNorm runs inside the pool
  for (int l = 0; l < m->n_layer; l++) {
    Layer& ly = m->layers[l];
    GemmArgs g{};
    g.M = T;
    g.rope_cos = m->rope_cos;
    g.rope_sin = m->rope_sin;
    g.L = L;
    g.Lp = Lp;
    g.n_head = H;
    g.d_model = D;
    g.part = w.part;
    g.tokrow = tokrow;
    {
      g.w = &ly.qkv;
      g.x = w.h16;
      g.q = w.q;
      g.k = w.k;
      g.vt = w.vt;
      Scope s(m, st, "gemm_qkv", 2.0 * T * ly.qkv.N * ly.qkv.K, wbytes(ly.qkv) + (double)T * (D * 2 + 3 * D * 2), timed);
      LAUNCH(launch_gemm(g, EPI_QKV, st));
    }
    {
      AttnArgs a{w.q, w.k, w.vt, d_mask, w.attn, B, L, Lp, H, D, seq_off};
      Scope s(m, st, "attention", 4.0 * B * (double)L * L * D, (double)T * D * 2 * 4, timed);
      LAUNCH(launch_attention(a, st));
    }
    {
      g.w = &ly.out;
      g.x = w.attn;
      g.y = w.h;
      Scope s(m, st, "gemm_out_ln", 2.0 * T * ly.out.N * ly.out.K, wbytes(ly.out) + (double)T * D * (2 + 18), timed);
      LAUNCH(launch_gemm_resid_ln(g, ly.anw, ly.anb, m->eps, w.h16, st, pending ? &pend : nullptr));
      pending = false;
    }
    {
      g.w = &ly.upgate;
      g.x = w.h16;
      g.g = w.ff;
      Scope s(m, st, "gemm_upgate", 2.0 * T * ly.upgate.N * ly.upgate.K, wbytes(ly.upgate) + (double)T * (D * 2 + F * 2), timed);
      LAUNCH(launch_gemm(g, EPI_GEGLU, st));
    }
    {
      g.w = &ly.down;
      g.x = w.ff;
      g.y = w.h;
      // Large batches leave this LayerNorm pending when the next out projection can finish it
      // while it reads its residual (same bits): the LayerNorm kernel then writes only the f16
      // rows and each row's mean and invStd, not the 4-byte rows (a third of its traffic). The
      // statistics go to the FFN buffer, free from here until the next up / gate projection.
      GemmArgs nx = g;
      if (l + 1 < m->n_layer) nx.w = &m->layers[l + 1].out;
      // (the full-row kernels read the statistics in whole 128-row blocks: up to 127 rows past T)
      pending = l + 1 < m->n_layer && (size_t)(T + 128) * sizeof(float2) <= (size_t)T * F * 2 &&
                gemm_resid_ln_gives_defer(g) && gemm_resid_ln_takes_defer(nx);
      float2* stats = (float2*)w.ff;
      // Many short sequences: the last LayerNorm runs inside the pool (one block per sequence,
      // its kept rows normalised 16 at a time in LDS and summed in row order; the same bits as
      // the LayerNorm kernel + pool), so neither the f32 nor the f16 rows are written
      pooled = d_out && l + 1 == m->n_layer && B >= 128 && L <= 256 && gemm_resid_ln_gives_defer(g);
      Scope s(m, st, "gemm_down_ln", 2.0 * T * ly.down.N * ly.down.K, wbytes(ly.down) + (double)T * (F * 2 + D * 18), timed);
      if (pooled)
        LAUNCH(launch_gemm(g, EPI_RESID, st));
      else
        LAUNCH(launch_gemm_resid_ln(g, ly.onw, ly.onb, m->eps, w.h16, st, nullptr, pending ? stats : nullptr));
      pend = LnDefer{ly.onw, ly.onb, stats};
    }
  }
  if (pooled) {
    const Layer& last = m->layers[m->n_layer - 1];
    Scope s(m, st, "pool", 0, (double)T * D * 4, timed);
    LAUNCH(launch_reduce_ln_pool(nullptr, 0, T, w.h, last.onw, last.onb, m->eps, d_mask, seq_off, B, L, D, out_dim,
                                 d_out, st));
  } else if (d_out) {
    Scope s(m, st, "pool", 0, (double)T * D * 4, timed);
    // the FFN buffer is free by now: it holds the sliced pool's per-sequence means
    LAUNCH(launch_pool(w.h, d_mask, seq_off, B, L, D, out_dim, d_out, (float*)w.ff, (size_t)T * F * 2, st));
  }
  return LLE_OK;
}

// Forwards of up to this many tokens are captured into a HIP graph and replayed: they are
// launch-bound (~60 kernels), and a replay removes the per-kernel host launch cost.
constexpr int64_t GRAPH_MAX_TOKENS = 4096;
constexpr size_t GRAPH_EXECS = 32;  // captured graphs kept per model
constexpr size_t GRAPH_KEYS = 128;  // keys remembered (captured or seen once)

static int run_forward(lle_model* m, const int32_t* d_ids, const int32_t* d_mask, int B, int L, int out_dim,
                       float* d_out, hipStream_t st, const Packing* pk = nullptr) {
  const int T = pk ? pk->T : B * L;
  // a stream the caller is capturing already records this forward into the caller's graph
  if (m->timing || !m->use_graphs || !st || (int64_t)B * L > GRAPH_MAX_TOKENS || m->precision != LLE_PRECISION_F16 ||
      capturing(st))
    return forward(m, m->ws, d_ids, d_mask, B, L, out_dim, d_out, st, pk);
  const uint64_t now = ++m->graph_tick;
  lle_model::GraphEntry* e = nullptr;
  for (auto& g : m->graphs)
    if (g.B == B && g.L == L && g.T == T && g.out_dim == out_dim && g.ids == d_ids && g.mask == d_mask &&
        g.out == d_out) {
      e = &g;
      break;
    }
  if (e && e->exec) {
    e->last_use = now;
    LLE_HIP(hipGraphLaunch(e->exec, st));
    return LLE_OK;
  }
  if (!e) {  // first sighting: run eagerly, remember the key
    if (m->graphs.size() >= GRAPH_KEYS) {
      auto lru = std::min_element(m->graphs.begin(), m->graphs.end(),
                                  [](const lle_model::GraphEntry& a, const lle_model::GraphEntry& b) {
                                    return a.last_use < b.last_use;
                                  });
      if (lru->exec) (void)hipGraphExecDestroy(lru->exec);
      m->graphs.erase(lru);
    }
    m->graphs.push_back({B, L, T, out_dim, d_ids, d_mask, d_out, nullptr, now});
    return forward(m, m->ws, d_ids, d_mask, B, L, out_dim, d_out, st, pk);
  }
  // second sighting: capture, keeping at most GRAPH_EXECS instantiated graphs. The capture runs
  // on the model's own non-blocking stream (held under the model's mutex, so nothing else is
  // enqueued on it meanwhile, and no other thread's legacy default stream waits on it); the
  // graph is then launched on the caller's stream.
  e->last_use = now;
  const size_t idx = (size_t)(e - m->graphs.data());
  size_t n_exec = 0;
  for (auto& g : m->graphs) n_exec += g.exec != nullptr;
  if (n_exec >= GRAPH_EXECS) {
    lle_model::GraphEntry* lru = nullptr;
    for (auto& g : m->graphs)
      if (g.exec && (!lru || g.last_use < lru->last_use)) lru = &g;
    (void)hipGraphExecDestroy(lru->exec);
    lru->exec = nullptr;
  }
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  if (hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal) == hipSuccess) {
    const int rc = forward(m, m->ws, d_ids, d_mask, B, L, out_dim, d_out, m->stream, pk);
    const hipError_t ce = hipStreamEndCapture(m->stream, &graph);
    if (rc == LLE_OK && ce == hipSuccess && graph && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess) {
      (void)hipGraphDestroy(graph);
      m->graphs[idx].exec = exec;
      LLE_HIP(hipGraphLaunch(exec, st));
      return LLE_OK;
    }
  }
  // the capture did not succeed: this forward runs eagerly (a genuine error shows there)
  if (graph) (void)hipGraphDestroy(graph);
  (void)hipGetLastError();
  return forward(m, m->ws, d_ids, d_mask, B, L, out_dim, d_out, st, pk);
}

// Bytes of one head buffer (Q, K or V^T) of a [B][L] batch: [B][H][Lp][64] f16.
static int64_t heads_bytes(const lle_model* m, int64_t B, int64_t L) { return B * m->H * ((L + 63) / 64 * 64) * 64 * 2; }
// The attention grid's z dimension is the sequence index.
constexpr int kMaxBatch = 65535;

static int check_batch(lle_model* m, int B, int L) {
  if (!m) return fail(LLE_EINVAL, "null model");
  if (B <= 0 || L <= 0) return fail(LLE_EINVAL, "B and L must be positive");
  if (L > m->max_seq)
    return fail(LLE_EINVAL, "sequence length " + std::to_string(L) + " exceeds context_length " + std::to_string(m->max_seq));
  // the GEMMs address X ([B*L][d_ff] f16 at most) with 32-bit buffer offsets
  if ((int64_t)B * L * std::max(m->F, m->D) * 2 > INT32_MAX)
    return fail(LLE_EINVAL, "batch too large: B*L*d_ff*2 bytes must stay below 2^31");
  // so do the QKV epilogue and the attention on the head buffers [B][H][Lp][64] f16, whose
  // rows are padded to Lp = L rounded up to 64 (up to 64 / L times the token count)
  if (heads_bytes(m, B, L) > INT32_MAX)
    return fail(LLE_EINVAL, "batch too large: B*n_head*Lp*64*2 bytes (Lp = L rounded up to 64) must stay below 2^31");
  if (B > kMaxBatch) return fail(LLE_EINVAL, "batch too large: more than 65535 sequences (attention grid)");
  if (L > 8192) return fail(LLE_EUNSUPPORTED, "sequence length above 8192 (the pooling kernel's row list)");
  return LLE_OK;
}

static int check_ids(lle_model* m, const int32_t* ids, int64_t n) {
  for (int64_t i = 0; i < n; i++)
    if (ids[i] < 0 || ids[i] >= m->vocab)
      return fail(LLE_EINVAL, "token embedding " + std::to_string(ids[i]) + ": id out of range [0, " + std::to_string(m->vocab) + ")");
  return LLE_OK;
}

// Host-pointer batch: H2D, forward, D2H, sync. Embeddings (not hidden states) run on packed
// rows when the mask has positions after a sequence's last valid token: those rows are dropped
// before the first kernel, so the GEMMs see only the rows that can reach an embedding.
static int run_host(lle_model* m, const int32_t* ids, const int32_t* mask, int B, int L, int out_dim, float* out,
                    float* hidden) {
  int rc = check_batch(m, B, L);
  if (rc) return rc;
  if (!ids || (!out && !hidden)) return fail(LLE_EINVAL, "null pointer");
  if ((rc = check_ids(m, ids, (int64_t)B * L))) return rc;
  const size_t T = (size_t)B * L;
  std::vector<int32_t> ones;
  if (!mask) {
    ones.assign(T, 1);
    mask = ones.data();
  }
  // packed rows: sequence b keeps positions [0, last valid + 1), or all L when none is valid
  std::vector<int32_t> pids, prow, soff;
  if (!hidden) {
    soff.resize((size_t)B + 1);
    int64_t rows = 0;
    for (int b = 0; b < B; b++) {
      const int32_t* mr = mask + (size_t)b * L;
      int n = L;
      while (n > 0 && mr[n - 1] == 0) n--;
      soff[b] = (int32_t)rows;
      rows += n ? n : L;
    }
    soff[B] = (int32_t)rows;
    if ((size_t)rows < T) {
      pids.resize((size_t)rows);
      prow.resize((size_t)rows);
      for (int b = 0; b < B; b++)
        for (int32_t t = soff[b], p = 0; t < soff[b + 1]; t++, p++) {
          pids[t] = ids[(size_t)b * L + p];
          prow[t] = b * L + p;
        }
    }
  }
  const bool packed = !pids.empty();
  std::lock_guard<std::mutex> lk(m->mu);
  LLE_HIP(hipSetDevice(m->device));
  if ((rc = ensure_ws(m, B, L, packed ? (int64_t)pids.size() : -1))) return rc;
  hipStream_t st = m->stream;
  if ((rc = order_begin(m, st))) return rc;
  Packing pk{(int)pids.size(), m->ws.tokrow, m->ws.seq_off};
  if (packed) {
    LLE_HIP(hipMemcpyAsync(m->ws.ids, pids.data(), pids.size() * 4, hipMemcpyHostToDevice, st));
    LLE_HIP(hipMemcpyAsync(m->ws.tokrow, prow.data(), prow.size() * 4, hipMemcpyHostToDevice, st));
    LLE_HIP(hipMemcpyAsync(m->ws.seq_off, soff.data(), soff.size() * 4, hipMemcpyHostToDevice, st));
  } else {
    LLE_HIP(hipMemcpyAsync(m->ws.ids, ids, T * 4, hipMemcpyHostToDevice, st));
  }
  LLE_HIP(hipMemcpyAsync(m->ws.mask, mask, T * 4, hipMemcpyHostToDevice, st));
  LLE_HIP(hipMemsetAsync(m->status, 0, 4, st));
  if ((rc = run_forward(m, m->ws.ids, m->ws.mask, B, L, out_dim, out ? m->ws.out : nullptr, st, packed ? &pk : nullptr)))
    return rc;
  const int od = std::min(out_dim, m->D);
  if (out) LLE_HIP(hipMemcpyAsync(out, m->ws.out, (size_t)B * od * 4, hipMemcpyDeviceToHost, st));
  if (hidden)
    LLE_HIP(hipMemcpyAsync(hidden, m->precision == LLE_PRECISION_F32 ? m->ex_h : m->ws.h, T * m->D * 4,
                           hipMemcpyDeviceToHost, st));
  if ((rc = order_end(m, st))) return rc;
  // host buffers above (pids, prow, soff, ones) must outlive the copies
  LLE_HIP(hipStreamSynchronize(st));
  if (m->timing && m->timing_only.empty()) collect_timing(m);
  return LLE_OK;
}

// Upload one projection: GGUF bytes of an [N][K] matrix -> re-laid-out planes in HBM.
static int upload_weight(int device, int type, const uint8_t* gguf, int K, int N, WeightDev* wd, std::vector<void*>* allocs) {
  if (type == 15 || type == 16) type = LLE_TYPE_Q5_K;  // DequantWeightMatrix maps 13,15,16 to Q5_K (gemm.go:241)
  if (!(type == 0 || type == 8 || type == 12 || type == 13 || type == 14))
    return fail(LLE_EUNSUPPORTED, "unsupported projection weight type " + std::to_string(type));
  if (K % 256 != 0 || N % 128 != 0)
    return fail(LLE_EUNSUPPORTED, "projection shape K=" + std::to_string(K) + " N=" + std::to_string(N) +
                                      " (need K % 256 == 0, N % 128 == 0)");
  size_t off[4], total;
  plane_offsets(type, K, N, off, &total);
  std::vector<uint8_t> host(total, 0);
  repack_rows(type, gguf, K, N, host.data(), off);
  void* d = nullptr;
  hipError_t e = hipMalloc(&d, total);
  if (e != hipSuccess) return fail(LLE_ENOMEM, std::string("weight hipMalloc: ") + hipGetErrorString(e));
  if (allocs) allocs->push_back(d);
  LLE_HIP(hipMemcpy(d, host.data(), total, hipMemcpyHostToDevice));
  wd->type = type;
  wd->K = K;
  wd->N = N;
  wd->base = d;
  wd->bytes = weight_dev_bytes(type, K, N);
  uint8_t* b = (uint8_t*)d;
  wd->p0 = b + off[0];
  wd->p1 = b + off[1];
  wd->p2 = b + off[2];
  wd->p3 = b + off[3];
  // Resident f16 copy [N][K] for the large-M GEMMs: the MFMA operand (RNE of the dequantised
  // value), made once here as the reference's PreDequant makes its f32 copy at load
  // (internal/embed/bert.go:542-576). Without memory for it the GEMMs decode on the fly.
  // LLE_NO_F16_COPY=1 (read per upload) skips the copy: tests use it to run the decoding path.
  const char* nocopy = getenv("LLE_NO_F16_COPY");
  void* h = nullptr;
  if (!(nocopy && nocopy[0] == '1') && hipMalloc(&h, (size_t)N * K * 2) == hipSuccess) {
    hipError_t e2 = launch_dequant_weight_h(*wd, (uint16_t*)h, nullptr);
    if (e2 == hipSuccess) e2 = hipStreamSynchronize(nullptr);
    if (e2 != hipSuccess) {
      (void)hipFree(h);
      if (!allocs) (void)hipFree(d);  // a model frees its allocs list itself
      return fail(LLE_EDEVICE, std::string("weight f16 copy: ") + hipGetErrorString(e2));
    }
    if (allocs) allocs->push_back(h);
    wd->w16 = (__half*)h;
  } else {
    (void)hipGetLastError();
  }
  (void)device;
  return LLE_OK;
}

static int check_tensor(const lle_tensor& t, const char* name, int64_t ne0, int64_t ne1) {
  if (!t.data) return fail(LLE_ENOTFOUND, std::string("tensor \"") + name + "\" not found");
  if (t.ne0 != ne0 || (ne1 >= 0 && t.ne1 != ne1))
    return fail(LLE_EINVAL, std::string(name) + ": shape [" + std::to_string(t.ne0) + ", " + std::to_string(t.ne1) +
                                "], expected [" + std::to_string(ne0) + ", " + std::to_string(ne1) + "]");
  const int64_t rb = row_bytes(t.type, t.ne0);
  if (rb < 0) return fail(LLE_EUNSUPPORTED, std::string(name) + ": unsupported ggml type " + std::to_string(t.type));
  int64_t need = 0;
  if (t.ne1 < 0 || __builtin_mul_overflow(rb, std::max<int64_t>(t.ne1, 1), &need) || t.nbytes < need)
    return fail(LLE_EINVAL, std::string(name) + ": data shorter than its ByteSize");
  return LLE_OK;
}

// Tensor.Dequantize of a small vector on the device (tensor.go:51-66 accepts 0/8/12/13/14).
static int upload_vec(lle_model* m, const lle_tensor& t, int n, float** out) {
  if (!(t.type == 0 || t.type == 8 || t.type == 12 || t.type == 13 || t.type == 14))
    return fail(LLE_EUNSUPPORTED, "ggml: dequantize not implemented for type " + std::to_string(t.type));
  const int64_t rb = row_bytes(t.type, n);
  void* raw = nullptr;
  int rc = dev_alloc(m, &raw, (size_t)rb);
  if (rc) return rc;
  LLE_HIP(hipMemcpy(raw, t.data, (size_t)rb, hipMemcpyHostToDevice));
  void* f = nullptr;
  if ((rc = dev_alloc(m, &f, (size_t)n * 4))) return rc;
  LAUNCH(launch_dequant_raw(t.type, (const uint8_t*)raw, n, (float*)f, m->stream));
  LLE_HIP(hipStreamSynchronize(m->stream));
  *out = (float*)f;
  return LLE_OK;
}

static void destroy_model(lle_model* m) {
  if (!m) return;
  (void)hipSetDevice(m->device);
  if (m->stream) (void)wait_forwards(m);
  ws_free(m);  // also destroys cached graphs
  ex_free(m);
  for (float* p : m->w32)
    if (p) (void)hipFree(p);
  for (void* p : m->allocs) (void)hipFree(p);
  for (auto& t : m->pending) {
    (void)hipEventDestroy(t.a);
    (void)hipEventDestroy(t.b);
  }
  for (auto e : m->event_pool) (void)hipEventDestroy(e);
  if (m->status) (void)hipFree(m->status);
  if (m->ev_last) (void)hipEventDestroy(m->ev_last);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

static int create_model(const lle_model_desc* d, lle_model** out) {
  if (!d || !out) return fail(LLE_EINVAL, "null argument");
  // the description is validated before the device is touched: a malformed model fails the
  // same way with or without a GPU
  int rc = LLE_OK;
  if (d->n_layer <= 0 || d->d_model <= 0) return fail(LLE_EINVAL, "embed: missing model params in GGUF metadata");
  if (d->n_head <= 0 || d->d_model % d->n_head != 0 || d->d_model / d->n_head != 64)
    return fail(LLE_EUNSUPPORTED, "head_dim must be 64 (d_model=" + std::to_string(d->d_model) + ", heads=" +
                                      std::to_string(d->n_head) + ")");
  if (d->d_model % 256 != 0 || d->d_model > 1024)
    return fail(LLE_EUNSUPPORTED, "d_model must be a multiple of 256 and <= 1024");
  if (d->d_ff <= 0 || d->d_ff % 256 != 0) return fail(LLE_EUNSUPPORTED, "feed_forward_length must be a multiple of 256");
  if (d->max_seq <= 0) return fail(LLE_EINVAL, "context_length must be positive");
  const int D = d->d_model, F = d->d_ff;
  if ((rc = check_tensor(d->token_embd, "token_embd.weight", D, -1))) return rc;
  if (!(d->token_embd.type == 0 || d->token_embd.type == 8 || d->token_embd.type == 12 || d->token_embd.type == 13 ||
        d->token_embd.type == 14))
    return fail(LLE_EUNSUPPORTED, "unsupported embedding type: " + std::to_string(d->token_embd.type));
  if ((rc = check_tensor(d->token_types, "token_types.weight", D, -1))) return rc;
  if ((rc = check_tensor(d->embd_norm_w, "token_embd_norm.weight", D, -1))) return rc;
  if ((rc = check_tensor(d->embd_norm_b, "token_embd_norm.bias", D, -1))) return rc;
  if (!d->qkv || !d->out || !d->up || !d->gate || !d->down || !d->attn_norm_w || !d->attn_norm_b || !d->out_norm_w ||
      !d->out_norm_b)
    return fail(LLE_EINVAL, "null layer tensor array");
  for (int l = 0; l < d->n_layer; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    if ((rc = check_tensor(d->qkv[l], (p + "attn_qkv.weight").c_str(), D, 3 * D))) return rc;
    if ((rc = check_tensor(d->out[l], (p + "attn_output.weight").c_str(), D, D))) return rc;
    if ((rc = check_tensor(d->up[l], (p + "ffn_up.weight").c_str(), D, F))) return rc;
    if ((rc = check_tensor(d->gate[l], (p + "ffn_gate.weight").c_str(), D, F))) return rc;
    if ((rc = check_tensor(d->down[l], (p + "ffn_down.weight").c_str(), F, D))) return rc;
    if ((rc = check_tensor(d->attn_norm_w[l], (p + "attn_output_norm.weight").c_str(), D, -1))) return rc;
    if ((rc = check_tensor(d->attn_norm_b[l], (p + "attn_output_norm.bias").c_str(), D, -1))) return rc;
    if ((rc = check_tensor(d->out_norm_w[l], (p + "layer_output_norm.weight").c_str(), D, -1))) return rc;
    if ((rc = check_tensor(d->out_norm_b[l], (p + "layer_output_norm.bias").c_str(), D, -1))) return rc;
    const int tu = d->up[l].type == 15 || d->up[l].type == 16 ? 13 : d->up[l].type;
    const int tg = d->gate[l].type == 15 || d->gate[l].type == 16 ? 13 : d->gate[l].type;
    if (tu != tg)
      return fail(LLE_EUNSUPPORTED, p + "ffn_up and ffn_gate have different ggml types; the fused up||gate GEMM needs one");
  }
  if (d->token_embd.ne1 <= 0 || d->token_embd.ne1 > INT32_MAX)
    return fail(LLE_EINVAL, "token_embd.weight: vocabulary size must be in [1, 2^31)");
  if ((rc = ensure_init())) return rc;

  lle_model* m = new lle_model();
  m->device = g_device;
  m->n_layer = d->n_layer;
  m->D = D;
  m->H = d->n_head;
  m->F = F;
  m->max_seq = d->max_seq;
  m->vocab = (int)d->token_embd.ne1;
  memcpy(&m->eps, &d->ln_eps_bits, 4);
  memcpy(&m->rope_base, &d->rope_base_bits, 4);
  auto bail = [&](int code) {
    destroy_model(m);
    return code;
  };
  if (hipSetDevice(m->device) != hipSuccess) return bail(fail(LLE_EDEVICE, "hipSetDevice failed"));
  // non-blocking: no other thread's legacy default stream waits on it (graphs are captured here)
  if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess)
    return bail(fail(LLE_EDEVICE, "hipStreamCreate failed"));
  if (hipEventCreateWithFlags(&m->ev_last, hipEventDisableTiming) != hipSuccess)
    return bail(fail(LLE_EDEVICE, "hipEventCreate failed"));
  if (hipMalloc((void**)&m->status, 4) != hipSuccess) return bail(fail(LLE_ENOMEM, "hipMalloc status"));
  (void)hipMemset(m->status, 0, 4);

  // token_embd stays in its GGUF layout: rows are gathered, not streamed.
  m->tok_type = d->token_embd.type;
  // getEmbedding (internal/embed/bert.go:290-316) gathers F32, Q8_0, Q4_K, Q5_K and Q6_K rows
  // only; the reference fails each Embed on another type, this library fails the load.
  if (m->tok_type != 0 && m->tok_type != 8 && (m->tok_type < 12 || m->tok_type > 14))
    return bail(fail(LLE_EUNSUPPORTED, "unsupported embedding type: " + std::to_string(m->tok_type)));
  m->tok_row_bytes = row_bytes(m->tok_type, D);
  const size_t tok_bytes = (size_t)m->tok_row_bytes * m->vocab;
  void* p = nullptr;
  if ((rc = dev_alloc(m, &p, tok_bytes))) return bail(rc);
  if (hipMemcpy(p, d->token_embd.data, tok_bytes, hipMemcpyHostToDevice) != hipSuccess)
    return bail(fail(LLE_EDEVICE, "upload token_embd"));
  m->tok = (uint8_t*)p;
  // getEmbedding(TokenTypes, 0): row 0 of token_types
  {
    lle_tensor t0 = d->token_types;
    t0.ne1 = 1;
    if ((rc = upload_vec(m, t0, D, &m->type0))) return bail(rc);
  }
  if ((rc = upload_vec(m, d->embd_norm_w, D, &m->enw))) return bail(rc);
  if ((rc = upload_vec(m, d->embd_norm_b, D, &m->enb))) return bail(rc);

  m->layers.resize(m->n_layer);
  for (int l = 0; l < m->n_layer; l++) {
    Layer& ly = m->layers[l];
    if ((rc = upload_weight(m->device, d->qkv[l].type, (const uint8_t*)d->qkv[l].data, D, 3 * D, &ly.qkv, &m->allocs)))
      return bail(rc);
    if ((rc = upload_weight(m->device, d->out[l].type, (const uint8_t*)d->out[l].data, D, D, &ly.out, &m->allocs)))
      return bail(rc);
    // up || gate, rows interleaved: fused row 2q = up row q, 2q+1 = gate row q
    {
      const int64_t rb = row_bytes(d->up[l].type, D);
      std::vector<uint8_t> fused((size_t)rb * 2 * F);
      const uint8_t* up = (const uint8_t*)d->up[l].data;
      const uint8_t* gt = (const uint8_t*)d->gate[l].data;
      for (int qrow = 0; qrow < F; qrow++) {
        memcpy(fused.data() + (size_t)(2 * qrow) * rb, up + (size_t)qrow * rb, rb);
        memcpy(fused.data() + (size_t)(2 * qrow + 1) * rb, gt + (size_t)qrow * rb, rb);
      }
      if ((rc = upload_weight(m->device, d->up[l].type, fused.data(), D, 2 * F, &ly.upgate, &m->allocs))) return bail(rc);
    }
    if ((rc = upload_weight(m->device, d->down[l].type, (const uint8_t*)d->down[l].data, F, D, &ly.down, &m->allocs)))
      return bail(rc);
    if ((rc = upload_vec(m, d->attn_norm_w[l], D, &ly.anw))) return bail(rc);
    if ((rc = upload_vec(m, d->attn_norm_b[l], D, &ly.anb))) return bail(rc);
    if ((rc = upload_vec(m, d->out_norm_w[l], D, &ly.onw))) return bail(rc);
    if ((rc = upload_vec(m, d->out_norm_b[l], D, &ly.onb))) return bail(rc);
  }

  // NewRoPETable (internal/ggml/ops_simd.go:107-124): f32 frequency, f32 angle, f64 cos/sin.
  {
    const int nrot = 32;
    std::vector<float> c((size_t)m->max_seq * nrot), s((size_t)m->max_seq * nrot);
    for (int pos = 0; pos < m->max_seq; pos++)
      for (int i = 0; i < nrot; i++) {
        const float freq = 1.0f / (float)pow((double)m->rope_base, (double)(2 * i) / 64.0);
        const float theta = freq * (float)pos;
        c[(size_t)pos * nrot + i] = (float)cos((double)theta);
        s[(size_t)pos * nrot + i] = (float)sin((double)theta);
      }
    void *dc = nullptr, *ds = nullptr;
    if ((rc = dev_alloc(m, &dc, c.size() * 4))) return bail(rc);
    if ((rc = dev_alloc(m, &ds, s.size() * 4))) return bail(rc);
    if (hipMemcpy(dc, c.data(), c.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ds, s.data(), s.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bail(fail(LLE_EDEVICE, "upload rope table"));
    m->rope_cos = (float*)dc;
    m->rope_sin = (float*)ds;
  }
  *out = m;
  return LLE_OK;
}

// Activations of a packed forward (T rows, B sequences of at most L tokens) laid out from
// `base`, each buffer 256-byte aligned: the sizes the model's own workspace gives the same call
// (ensure_ws with T rows). Returns the bytes needed; fills *w when base is non-null.
static size_t carve_packed(const lle_model* m, int B, int L, int T, uint8_t* base, Workspace* w) {
  const size_t D = m->D, F = m->F, R = (size_t)T;
  const size_t heads = (size_t)heads_bytes(m, B, L);
  auto nch = [](size_t K) { return K % 768 == 0 ? K / 768 : K / 256; };
  const size_t kd = nch(D), kf = nch(F);
  const size_t part = R < 1024 ? std::max<size_t>(R, 64) * std::max({kd * 3 * D, kd * 2 * F, kf * D}) * 4 : 0;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off += (std::max<size_t>(bytes, 1) + 255) & ~(size_t)255;
    return p;
  };
  Workspace x;
  x.h = (float*)take(R * D * 4);
  x.h2 = (float*)take(16 * D * 4);
  x.h16 = (__half*)take(R * D * 2);
  x.q = (__half*)take(heads);
  x.k = (__half*)take(heads);
  x.vt = (__half*)take(heads);
  x.attn = (__half*)take(R * D * 2);
  x.ff = (__half*)take(R * F * 2);
  x.part = part ? (float*)take(part) : nullptr;
  x.mask = (int32_t*)take((size_t)B * L * 4);
  x.tokrow = (int32_t*)take(R * 4);
  x.seq_off = (int32_t*)take(((size_t)B + 1) * 4);
  if (base && w) *w = x;
  return off;
}

int model_device(const lle_model* m) { return m ? m->device : -1; }

int embed_packed_scratch(lle_model* m, const int32_t* d_ids, const int32_t* d_seq_off, int B, int T, int L,
                         int out_dim, float* d_out, hipStream_t stream, void* scratch, size_t scratch_bytes) {
  int rc = check_batch(m, B, L);
  if (rc) return rc;
  if (!d_ids || !d_seq_off || !d_out) return fail(LLE_EINVAL, "null device pointer");
  if (T < 1 || (int64_t)T > (int64_t)B * L) return fail(LLE_EINVAL, "T must be in [1, B * L]");
  if (!scratch) return fail(LLE_EDEVICE, "no-allocation scratch not set up on this device");
  if (m->precision != LLE_PRECISION_F16)
    return fail(LLE_EUNSUPPORTED, "lle_embed_packed_noalloc runs the f16 forward only (the model is in F32 precision)");
  if (out_dim < 1) out_dim = 1;
  const size_t need = carve_packed(m, B, L, T, nullptr, nullptr);
  if (need > scratch_bytes)
    return fail(LLE_EINVAL, "lle_embed_packed_noalloc: this batch needs " + std::to_string(need) +
                                " bytes of scratch, above the fixed " + std::to_string(scratch_bytes) +
                                " (fewer tokens or sequences per call)");
  Workspace w;
  carve_packed(m, B, L, T, (uint8_t*)scratch, &w);
  std::lock_guard<std::mutex> lk(m->mu);
  LLE_HIP(hipSetDevice(m->device));
  const hipStream_t st = stream ? stream : m->stream;
  LAUNCH(launch_pack_tables(d_seq_off, B, T, L, w.seq_off, w.tokrow, w.mask, m->status, st));
  Packing pk{T, w.tokrow, w.seq_off};
  return forward(m, w, d_ids, w.mask, B, L, out_dim, d_out, st, &pk, /*timed=*/false);
}

}  // namespace lle

using namespace lle;

extern "C" {

int32_t lle_abi_version(void) { return LLE_ABI_VERSION; }

const char* lle_last_error(void) { return g_err.c_str(); }

int32_t lle_init(int32_t device) {
  std::lock_guard<std::mutex> lk(g_init_mu);
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) return fail(LLE_EDEVICE, "no HIP device available");
  if (device < 0 || device >= n) return fail(LLE_EINVAL, "device ordinal out of range");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(LLE_EDEVICE, std::string("hipGetDeviceProperties: ") + hipGetErrorString(e));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(LLE_EDEVICE, std::string("device is ") + prop.gcnArchName + ", this library is built for gfx950");
  e = hipSetDevice(device);
  if (e != hipSuccess) return fail(LLE_EDEVICE, std::string("hipSetDevice: ") + hipGetErrorString(e));
  const int rc = noalloc_setup(device);  // the no-allocation entry's device array, with `device` current
  if (rc) return rc;
  g_device = device;
  return LLE_OK;
}

int32_t lle_info(char* buf, int32_t cap) {
  if (!buf || cap <= 0) return fail(LLE_EINVAL, "null buffer");
  std::string s = "llmembed-hip abi=" + std::to_string(LLE_ABI_VERSION) + " arch=gfx950";
  if (g_device >= 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, g_device) == hipSuccess)
      s += std::string(" device=") + std::to_string(g_device) + " name=" + prop.name + " cus=" +
           std::to_string(prop.multiProcessorCount) + " hbm_gib=" + std::to_string(prop.totalGlobalMem >> 30);
  } else {
    s += " device=uninitialised";
  }
  s += " gemm=mfma_f32_16x16x32_f16(dequant->f16 in LDS, f32 accumulate, canonical K chunks of 768 (256 when K % 768 != 0))";
  s += " attention=mfma flash (online max, exact x<-10 cutoff)";
  snprintf(buf, (size_t)cap, "%s", s.c_str());
  return (int32_t)std::min<size_t>(s.size(), (size_t)cap - 1);
}

int32_t lle_f16_to_f32(const uint16_t* h, int64_t n, float* out) {
  if (!h || !out || n < 0) return fail(LLE_EINVAL, "bad argument");
  int rc = ensure_init();
  if (rc) return rc;
  LLE_HIP(hipSetDevice(g_device));
  void *dh = nullptr, *df = nullptr;
  LLE_HIP(hipMalloc(&dh, (size_t)std::max<int64_t>(n, 1) * 2));
  hipError_t e = hipMalloc(&df, (size_t)std::max<int64_t>(n, 1) * 4);
  if (e != hipSuccess) {
    (void)hipFree(dh);
    return fail(LLE_ENOMEM, "hipMalloc");
  }
  e = hipMemcpy(dh, h, (size_t)n * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_f16_to_f32_bits((const uint16_t*)dh, (float*)df, n, nullptr);
  if (e == hipSuccess) e = hipMemcpy(out, df, (size_t)n * 4, hipMemcpyDeviceToHost);
  (void)hipFree(dh);
  (void)hipFree(df);
  if (e != hipSuccess) return fail(LLE_EDEVICE, std::string("f16 decode: ") + hipGetErrorString(e));
  return LLE_OK;
}

int32_t lle_dequant(int32_t type, const void* blocks, int64_t n, float* out) {
  if (!blocks || !out || n < 0) return fail(LLE_EINVAL, "bad argument");
  if (type == 15 || type == 16) type = LLE_TYPE_Q5_K;
  const int64_t bs = type == 0 ? 1 : type == 8 ? 32 : 256;
  const int64_t rb = row_bytes(type, n);
  if (rb < 0) return fail(LLE_EUNSUPPORTED, "ggml: dequantize not implemented for type " + std::to_string(type));
  if (n % bs) return fail(LLE_EINVAL, "element count must be a whole number of blocks");
  int rc = ensure_init();
  if (rc) return rc;
  LLE_HIP(hipSetDevice(g_device));
  void *db = nullptr, *df = nullptr;
  LLE_HIP(hipMalloc(&db, (size_t)std::max<int64_t>(rb, 1)));
  hipError_t e = hipMalloc(&df, (size_t)std::max<int64_t>(n, 1) * 4);
  if (e != hipSuccess) {
    (void)hipFree(db);
    return fail(LLE_ENOMEM, "hipMalloc");
  }
  e = hipMemcpy(db, blocks, (size_t)rb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_dequant_raw(type, (const uint8_t*)db, n, (float*)df, nullptr);
  if (e == hipSuccess) e = hipMemcpy(out, df, (size_t)n * 4, hipMemcpyDeviceToHost);
  (void)hipFree(db);
  (void)hipFree(df);
  if (e != hipSuccess) return fail(LLE_EDEVICE, std::string("dequant: ") + hipGetErrorString(e));
  return LLE_OK;
}

int32_t lle_model_create(const lle_model_desc* d, lle_model** out) { return create_model(d, out); }

int32_t lle_model_destroy(lle_model* m) {
  if (!m) return fail(LLE_EINVAL, "null model");
  destroy_model(m);
  return LLE_OK;
}

int32_t lle_model_dims(const lle_model* m, int32_t* dims) {
  if (!m || !dims) return fail(LLE_EINVAL, "null argument");
  dims[0] = m->n_layer;
  dims[1] = m->D;
  dims[2] = m->H;
  dims[3] = m->F;
  dims[4] = m->max_seq;
  dims[5] = m->vocab;
  return LLE_OK;
}

int32_t lle_embed(lle_model* m, const int32_t* ids, const int32_t* mask, int32_t L, int32_t out_dim, float* out) {
  if (out_dim < 1) out_dim = 1;  // SetTargetDim clamps (embedder.go:142-150)
  return run_host(m, ids, mask, 1, L, out_dim, out, nullptr);
}

int32_t lle_embed_batch(lle_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t L, int32_t out_dim,
                        float* out) {
  if (out_dim < 1) out_dim = 1;
  return run_host(m, ids, mask, B, L, out_dim, out, nullptr);
}

int32_t lle_embed_texts(lle_model* m, const lle_tokenizer* t, const char* const* texts, const int64_t* lens,
                        int32_t n, const char* prefix, int64_t prefix_len, int32_t out_dim, int32_t max_batch_tokens,
                        float* out) {
  if (!m || !t || n < 0 || (n > 0 && (!texts || !out)) || (prefix_len > 0 && !prefix))
    return fail(LLE_EINVAL, "bad argument");
  if (n == 0) return LLE_OK;
  if (out_dim < 1) out_dim = 1;
  if (prefix && prefix_len < 0) prefix_len = (int64_t)strlen(prefix);
  // the GEMMs address [tokens][d_ff] f16 with 32-bit offsets (check_batch)
  const int64_t tok_cap = INT32_MAX / (2 * (int64_t)std::max(m->F, m->D));
  const int64_t budget = std::min<int64_t>(max_batch_tokens > 0 ? max_batch_tokens : 32768, tok_cap / 4);
  std::vector<std::vector<int32_t>> v;
  lle::tokenize_many(t->tok, texts, lens, n, prefix, prefix_len, m->max_seq, &v);
  // longest first; equal lengths keep input order
  std::vector<int32_t> order((size_t)n);
  for (int32_t i = 0; i < n; i++) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return v[a].size() > v[b].size(); });
  const int od = std::min(out_dim, m->D);
  std::vector<int32_t> ids, mask;
  std::vector<float> res;
  for (int32_t i = 0; i < n;) {
    const int L = (int)v[order[i]].size();
    const int64_t cap = std::max<int64_t>(budget, L);
    // the forward packs padding away (run_host), so a batch is cut at `budget` valid tokens;
    // its padded [B][L] tables stay within 4 x budget (buffers, 32-bit offsets)
    int32_t j = i + 1;
    int64_t valid = L;
    while (j < n && valid + (int64_t)v[order[j]].size() <= cap && (int64_t)(j - i + 1) * L <= 4 * cap &&
           j - i + 1 <= kMaxBatch && heads_bytes(m, j - i + 1, L) <= INT32_MAX) {
      valid += (int64_t)v[order[j]].size();
      j++;
    }
    const int B = j - i;
    ids.assign((size_t)B * L, 0);
    mask.assign((size_t)B * L, 0);
    for (int k = 0; k < B; k++) {
      const std::vector<int32_t>& s = v[order[i + k]];
      std::copy(s.begin(), s.end(), ids.begin() + (size_t)k * L);
      std::fill(mask.begin() + (size_t)k * L, mask.begin() + (size_t)k * L + s.size(), 1);
    }
    res.resize((size_t)B * od);
    const int rc = run_host(m, ids.data(), mask.data(), B, L, out_dim, res.data(), nullptr);
    if (rc) return rc;
    for (int k = 0; k < B; k++)
      memcpy(out + (size_t)order[i + k] * od, res.data() + (size_t)k * od, sizeof(float) * od);
    i = j;
  }
  return LLE_OK;
}

int32_t lle_forward_hidden(lle_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t L, float* hidden) {
  return run_host(m, ids, mask, B, L, m ? m->D : 0, nullptr, hidden);
}

int32_t lle_embed_batch_async(lle_model* m, const int32_t* d_ids, const int32_t* d_mask, int32_t B, int32_t L,
                              int32_t out_dim, float* d_out, void* stream) {
  int rc = check_batch(m, B, L);
  if (rc) return rc;
  if (!d_ids || !d_mask || !d_out) return fail(LLE_EINVAL, "null device pointer");
  if (out_dim < 1) out_dim = 1;
  std::lock_guard<std::mutex> lk(m->mu);
  if (m->precision != LLE_PRECISION_F16)
    return fail(LLE_EUNSUPPORTED, "F32 precision needs each sequence's length: use lle_embed_packed_async or a host entry");
  LLE_HIP(hipSetDevice(m->device));
  if ((rc = ensure_ws(m, B, L))) return rc;
  const hipStream_t st = stream ? (hipStream_t)stream : m->stream;
  if ((rc = order_begin(m, st))) return rc;
  if ((rc = run_forward(m, d_ids, d_mask, B, L, out_dim, d_out, st))) return rc;
  if ((rc = order_end(m, st))) return rc;
  if (m->timing && m->timing_only.empty()) {
    LLE_HIP(hipStreamSynchronize(st));
    collect_timing(m);
  }
  return LLE_OK;
}

int32_t lle_embed_packed_async(lle_model* m, const int32_t* d_ids, const int32_t* d_seq_off, int32_t B, int32_t T,
                               int32_t L, int32_t out_dim, float* d_out, void* stream) {
  int rc = check_batch(m, B, L);
  if (rc) return rc;
  if (!d_ids || !d_seq_off || !d_out) return fail(LLE_EINVAL, "null device pointer");
  if (T < 1 || (int64_t)T > (int64_t)B * L) return fail(LLE_EINVAL, "T must be in [1, B * L]");
  if (out_dim < 1) out_dim = 1;
  std::lock_guard<std::mutex> lk(m->mu);
  LLE_HIP(hipSetDevice(m->device));
  if ((rc = ensure_ws(m, B, L, T))) return rc;
  const hipStream_t st = stream ? (hipStream_t)stream : m->stream;
  if ((rc = order_begin(m, st))) return rc;
  LAUNCH(launch_pack_tables(d_seq_off, B, T, L, m->ws.seq_off, m->ws.tokrow, m->ws.mask, m->status, st));
  Packing pk{T, m->ws.tokrow, m->ws.seq_off};
  if ((rc = run_forward(m, d_ids, m->ws.mask, B, L, out_dim, d_out, st, &pk))) return rc;
  if ((rc = order_end(m, st))) return rc;
  if (m->timing && m->timing_only.empty()) {
    LLE_HIP(hipStreamSynchronize(st));
    collect_timing(m);
  }
  return LLE_OK;
}

int32_t lle_model_status(lle_model* m, int32_t* status) {
  if (!m || !status) return fail(LLE_EINVAL, "null argument");
  std::lock_guard<std::mutex> lk(m->mu);
  LLE_HIP(hipSetDevice(m->device));
  LLE_HIP(hipDeviceSynchronize());
  LLE_HIP(hipMemcpy(status, m->status, 4, hipMemcpyDeviceToHost));
  return LLE_OK;
}

int32_t lle_model_set_precision(lle_model* m, int32_t precision) {
  if (!m) return fail(LLE_EINVAL, "null model");
  if (precision != LLE_PRECISION_F16 && precision != LLE_PRECISION_F32)
    return fail(LLE_EINVAL, "precision must be LLE_PRECISION_F16 or LLE_PRECISION_F32");
  std::lock_guard<std::mutex> lk(m->mu);
  LLE_HIP(hipSetDevice(m->device));
  if (int rc = wait_forwards(m)) return rc;
  if (precision == LLE_PRECISION_F32 && m->w32.empty()) {
    // PreDequant (internal/embed/bert.go:542-576): every projection dequantised once to f32
    // [N][K] by the GEMM's own decoder (bit-exact with DequantWeightMatrix)
    std::vector<float*> w32((size_t)m->n_layer * 4, nullptr);
    auto undo = [&](int code, const std::string& msg) {
      for (float* p : w32)
        if (p) (void)hipFree(p);
      return fail(code, msg);
    };
    for (int l = 0; l < m->n_layer; l++) {
      const WeightDev* ws[4] = {&m->layers[l].qkv, &m->layers[l].out, &m->layers[l].upgate, &m->layers[l].down};
      for (int i = 0; i < 4; i++) {
        float* p = nullptr;
        hipError_t e = hipMalloc((void**)&p, (size_t)ws[i]->N * ws[i]->K * 4);
        if (e != hipSuccess) return undo(LLE_ENOMEM, std::string("f32 weight copy hipMalloc: ") + hipGetErrorString(e));
        w32[(size_t)l * 4 + i] = p;
        e = launch_dequant_weight(*ws[i], p, m->stream);
        if (e != hipSuccess) return undo(LLE_EDEVICE, std::string("f32 weight copy: ") + hipGetErrorString(e));
      }
    }
    hipError_t e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return undo(LLE_EDEVICE, std::string("f32 weight copy: ") + hipGetErrorString(e));
    m->w32 = w32;
  }
  m->precision = precision;
  return LLE_OK;
}

int32_t lle_model_set_timing(lle_model* m, int32_t enable) {
  if (!m) return fail(LLE_EINVAL, "null model");
  std::lock_guard<std::mutex> lk(m->mu);
  LLE_HIP(hipSetDevice(m->device));
  LLE_HIP(hipDeviceSynchronize());
  collect_timing(m);  // events of an earlier single-class run
  m->timing = enable != 0;  // timed forwards run eagerly (events around every launch)
  m->timing_only.clear();
  m->totals.clear();
  return LLE_OK;
}

int32_t lle_model_set_timing_kernel(lle_model* m, const char* kernel_class) {
  if (!m) return fail(LLE_EINVAL, "null model");
  std::lock_guard<std::mutex> lk(m->mu);
  LLE_HIP(hipSetDevice(m->device));
  LLE_HIP(hipDeviceSynchronize());
  collect_timing(m);
  m->totals.clear();
  m->timing = kernel_class && kernel_class[0];
  m->timing_only = m->timing ? std::string(kernel_class) : std::string();
  return LLE_OK;
}

int32_t lle_model_get_timing(lle_model* m, lle_kernel_time* out, int32_t cap, int32_t* n_out) {
  if (!m || !n_out) return fail(LLE_EINVAL, "null argument");
  std::lock_guard<std::mutex> lk(m->mu);
  if (!m->pending.empty()) {  // single-class mode reads its events here, after the forwards end
    LLE_HIP(hipSetDevice(m->device));
    LLE_HIP(hipDeviceSynchronize());
    collect_timing(m);
  }
  const int n = (int)m->totals.size();
  for (int i = 0; i < n && i < cap && out; i++) out[i] = m->totals[i];
  *n_out = n;
  return LLE_OK;
}

int32_t lle_weight_create(int32_t type, const void* blocks, int32_t K, int32_t N, lle_weight** out) {
  if (!blocks || !out || K <= 0 || N <= 0) return fail(LLE_EINVAL, "bad argument");
  int rc = ensure_init();
  if (rc) return rc;
  LLE_HIP(hipSetDevice(g_device));
  lle_weight* w = new lle_weight();
  w->device = g_device;
  if ((rc = upload_weight(g_device, type, (const uint8_t*)blocks, K, N, &w->w, nullptr))) {
    delete w;
    return rc;
  }
  if (hipStreamCreate(&w->stream) != hipSuccess) {
    (void)hipFree(w->w.base);
    if (w->w.w16) (void)hipFree(w->w.w16);
    delete w;
    return fail(LLE_EDEVICE, "hipStreamCreate");
  }
  *out = w;
  return LLE_OK;
}

int32_t lle_weight_destroy(lle_weight* w) {
  if (!w) return fail(LLE_EINVAL, "null weight");
  (void)hipSetDevice(w->device);
  (void)hipStreamSynchronize(w->stream);
  (void)hipFree(w->w.base);
  if (w->w.w16) (void)hipFree(w->w.w16);
  (void)hipStreamDestroy(w->stream);
  delete w;
  return LLE_OK;
}

int32_t lle_weight_dequant(const lle_weight* w, float* out) {
  if (!w || !out) return fail(LLE_EINVAL, "null argument");
  LLE_HIP(hipSetDevice(w->device));
  void* d = nullptr;
  const size_t n = (size_t)w->w.K * w->w.N;
  LLE_HIP(hipMalloc(&d, n * 4));
  hipError_t e = launch_dequant_weight(w->w, (float*)d, w->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
  if (e == hipSuccess) e = hipMemcpy(out, d, n * 4, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(LLE_EDEVICE, std::string("weight dequant: ") + hipGetErrorString(e));
  return LLE_OK;
}

int32_t lle_weight_dequant_f16(const lle_weight* w, uint16_t* out) {
  if (!w || !out) return fail(LLE_EINVAL, "null argument");
  LLE_HIP(hipSetDevice(w->device));
  void* d = nullptr;
  const size_t n = (size_t)w->w.K * w->w.N;
  LLE_HIP(hipMalloc(&d, n * 2));
  hipError_t e = launch_dequant_weight_h(w->w, (uint16_t*)d, w->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
  if (e == hipSuccess) e = hipMemcpy(out, d, n * 2, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(LLE_EDEVICE, std::string("weight dequant f16: ") + hipGetErrorString(e));
  return LLE_OK;
}

static int gemm_enqueue(const lle_weight* w, const float* dX, void* dx16, int M, float* dY, float* part, hipStream_t st) {
  LAUNCH(launch_f32_to_f16(dX, (__half*)dx16, (int64_t)M * w->w.K, st));
  GemmArgs g{};
  g.w = &w->w;
  g.x = (const __half*)dx16;
  g.M = M;
  g.y = dY;
  g.part = part;
  LAUNCH(launch_gemm(g, EPI_F32, st));
  return LLE_OK;
}

int32_t lle_gemm_async(const lle_weight* w, const float* d_X, void* d_x16, int32_t M, float* d_Y, void* stream) {
  if (!w || !d_X || !d_x16 || !d_Y || M <= 0) return fail(LLE_EINVAL, "bad argument");
  if (M <= 64) return fail(LLE_EINVAL, "lle_gemm_async needs M > 64 (small M uses a split-K workspace: use lle_gemm)");
  LLE_HIP(hipSetDevice(w->device));
  return gemm_enqueue(w, d_X, d_x16, M, d_Y, nullptr, stream ? (hipStream_t)stream : w->stream);
}

int32_t lle_gemm_f16_async(const lle_weight* w, const void* d_x16, int32_t M, float* d_Y, float* d_part,
                           void* stream) {
  if (!w || !d_x16 || !d_Y || M <= 0) return fail(LLE_EINVAL, "bad argument");
  if (M <= 64 && !d_part) return fail(LLE_EINVAL, "M <= 64 needs the split-K workspace d_part");
  if (M >= 1024) d_part = nullptr;
  LLE_HIP(hipSetDevice(w->device));
  GemmArgs g{};
  g.w = &w->w;
  g.x = (const __half*)d_x16;
  g.M = M;
  g.y = d_Y;
  g.part = d_part;
  hipStream_t st = stream ? (hipStream_t)stream : w->stream;
  LAUNCH(launch_gemm(g, EPI_F32, st));
  return LLE_OK;
}

int32_t lle_gemm(const lle_weight* w, const float* X, int32_t M, float* Y) {
  if (!w || !X || !Y || M <= 0) return fail(LLE_EINVAL, "bad argument");
  LLE_HIP(hipSetDevice(w->device));
  const size_t K = (size_t)w->w.K, N = (size_t)w->w.N;
  void *dX = nullptr, *dx16 = nullptr, *dY = nullptr, *dP = nullptr;
  hipError_t e = hipMalloc(&dX, M * K * 4);
  if (e == hipSuccess) e = hipMalloc(&dx16, M * K * 2);
  if (e == hipSuccess) e = hipMalloc(&dY, M * N * 4);
  if (e == hipSuccess && M < 1024) e = hipMalloc(&dP, (K % 768 == 0 ? K / 768 : K / 256) * (size_t)M * N * 4);
  int rc = LLE_OK;
  if (e != hipSuccess) rc = fail(LLE_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
  if (!rc && hipMemcpy(dX, X, M * K * 4, hipMemcpyHostToDevice) != hipSuccess) rc = fail(LLE_EDEVICE, "copy X");
  if (!rc) rc = gemm_enqueue(w, (const float*)dX, dx16, M, (float*)dY, (float*)dP, w->stream);
  if (!rc && hipStreamSynchronize(w->stream) != hipSuccess) rc = fail(LLE_EDEVICE, "gemm sync");
  if (!rc && hipMemcpy(Y, dY, M * N * 4, hipMemcpyDeviceToHost) != hipSuccess) rc = fail(LLE_EDEVICE, "copy Y");
  (void)hipFree(dX);
  (void)hipFree(dx16);
  (void)hipFree(dY);
  if (dP) (void)hipFree(dP);
  return rc;
}

}  // extern "C"
