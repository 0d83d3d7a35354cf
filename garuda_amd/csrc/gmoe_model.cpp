// gmoe_model.cpp — one decode step of a Llama-family MoE model on the device.
//
// LlamaBackend::logits_batch (garuda/src/llama/mod.rs:1134-1206) for its decode case:
// every sequence takes one new token. The step embeds the tokens, runs each layer as
// layer_batch_over does (:851-893) — h = norm(x, attn_norm); q, k, v projections;
// attend_one per token; x += wo(context); h = norm(x, ffn_norm); x += the MoE layer — then
// norm(x, output_norm), the output head, and greedy sampling (runtime/mod.rs:98-105).
// Everything is queued on the context's stream with no host synchronisation until the
// chosen tokens come back; the pieces are the library's own entry points (dense
// projections, paged attention, the MoE layer) and the glue kernels of gmoe_glue.hip.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/garuda_moe.h"
#include "gmoe_internal.h"

namespace gmoe {
void set_last_error(const char* msg);
void set_invalid_token(uint32_t token);
int ctx_device(gmoe_ctx* c);
hipStream_t ctx_stream(gmoe_ctx* c);
bool dense_shape(gmoe_ctx* c, uint32_t id, uint32_t* rows, uint32_t* cols);
bool layer_width(gmoe_ctx* c, uint32_t id, uint32_t* d, uint32_t* ne);
void kv_dims(gmoe_kv* kv, uint32_t* n_layers, uint32_t* q_dim, uint32_t* kv_dim);
gmoe_status kv_check_step(gmoe_kv* kv, const uint32_t* seqs, uint32_t n);
uint32_t kv_step_chunks(gmoe_kv* kv, uint32_t maxspan);
gmoe_status kv_reserve(gmoe_kv* kv, uint32_t n, uint32_t nchunk);
const void* kv_scratch_id(gmoe_kv* kv);
gmoe_status kv_plan_step(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, AttnEntry* ents, size_t stride,
                         uint32_t* maxspan);
void kv_commit_step(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, AttnEntry* ents, size_t stride);
void kv_snapshot(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, std::vector<uint32_t>& snap);
void kv_restore(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, const std::vector<uint32_t>& snap);
gmoe_status ctx_pin_layers(gmoe_ctx* c, const uint32_t* layers, uint32_t n);
void ctx_unpin_layers(gmoe_ctx* c, const uint32_t* layers, uint32_t n);
bool dense_tiled(gmoe_ctx* c, uint32_t id, const uint8_t** tiled, uint32_t* qtype);
gmoe_status kv_check_prefill(gmoe_kv* kv, uint32_t seq, uint32_t n);
gmoe_status kv_attend_dev(gmoe_kv* kv, uint32_t n, const AttnEntry* d_ent, uint32_t nchunk, const float* q,
                          const float* k, const float* v, uint32_t q_stride, uint32_t kv_stride, float* out,
                          hipStream_t st, uint32_t nsl = 1, uint64_t sl_stride = 0);
gmoe_status dense_forward_slices(gmoe_ctx* c, uint32_t id, const float* d_xs, uint32_t n, hipStream_t st,
                                 const float** parts, uint32_t* nsl, float* y_out = nullptr);
gmoe_status ffn_forward_normed(gmoe_ctx* c, uint32_t lid, float* d_x, const float* d_y, uint32_t nsl,
                               uint64_t y_stride, const float* d_w, float eps, float* d_h, uint32_t n, float* d_out,
                               hipStream_t st);
const void* ctx_scratch_id(gmoe_ctx* c);
void ctx_note_graph(gmoe_ctx* c, const uint32_t* layers, uint32_t n, hipStream_t st);
gmoe_status kv_attend(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, const float* q, const float* k,
                      const float* v, uint32_t q_stride, uint32_t kv_stride, float* out, hipStream_t st);
gmoe_status dense_stack(gmoe_ctx* c, const uint32_t* ids, uint32_t count, uint32_t* out);
}  // namespace gmoe

using namespace gmoe;

struct gmoe_model {
  gmoe_ctx* ctx = nullptr;
  gmoe_kv* kv = nullptr;
  uint32_t n_layers = 0, d = 0, vocab = 0, qd = 0, kvd = 0;
  float eps = 0.0f;
  std::vector<uint32_t> moe, wq, wk, wv, wo;
  // per layer, wq, wk and wv stacked into one weight of q_dim + 2 kv_dim rows (owned),
  // when their rows are whole 64-row tiles and they share type and math: one product
  // launch for the three, its output rows q | k | v
  std::vector<uint32_t> wqkv;
  uint32_t out_id = 0;
  float* qkv = nullptr;
  float* table = nullptr;  // [vocab][d] token embeddings (f32 rows)
  // or the token table kept packed: a dense weight of the model's own, its rows dequantised
  // per token (and, when the checkpoint ties them, the output head itself)
  uint32_t embd_id = kNoDense;
  const uint8_t* embd_tiled = nullptr;
  uint32_t embd_qt = 0;
  static constexpr uint32_t kNoDense = 0xFFFFFFFFu;
  // prompt chunks (gmoe_model_prefill): activations of up to kPrefillChunk tokens, the
  // chunk's tokens (device, and their pinned staging), allocated on the first prefill
  static constexpr uint32_t kPrefillChunk = 256;  // DEFAULT_PREFILL_CHUNK, llama/mod.rs:32
  float *px = nullptr, *ph = nullptr, *pq = nullptr, *pk = nullptr, *pv = nullptr, *pqkv = nullptr, *pcx = nullptr,
        *pao = nullptr, *py = nullptr;
  uint32_t* ptok = nullptr;
  uint32_t* pin_tok = nullptr;
  float* norms = nullptr;  // [2 n_layers + 1][d]: attn_norm, ffn_norm per layer, then output_norm
  // per-step activations for up to kModelMaxBatch tokens
  float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *cx = nullptr, *ao = nullptr,
        *y = nullptr, *logits = nullptr;
  uint32_t* next = nullptr;
  uint32_t* pin_next = nullptr;
  // Decode steps replayed from HIP graphs: a step's launches are captured once per (batch
  // size, attention chunks) and read the step's parameters from device memory (par: the
  // tokens, then every layer's attention entries; pin_par its pinned host copy). The
  // chunks are the step's longest span rounded up to a power of two, so a graph serves
  // until a sequence outgrows its bucket. Up to kGraphCache graphs are kept (least
  // recently replayed out), each while the scratch allocations its launches point into
  // stay where they were, so continuous batching whose batch size drifts replays instead
  // of capturing again.
  struct Graph {
    hipGraphExec_t exec = nullptr;
    uint32_t n = 0, nchunk = 0;
    const void* g_ctx = nullptr;
    const void* g_kv = nullptr;
    uint64_t used = 0;
  };
  static constexpr size_t kGraphCache = 8;
  bool graphs = true, graph_failed = false;
  hipStream_t cap = nullptr;  // captures run on a stream of the model's own, which no other caller queues on
  std::vector<Graph> gcache;
  uint64_t gclock = 0;
  uint8_t* par = nullptr;
  uint8_t* pin_par = nullptr;
  std::mutex mu;

  void drop_graphs() {
    for (auto& g : gcache)
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
    gcache.clear();
  }

  ~gmoe_model() {
    drop_graphs();
    if (cap) hipStreamDestroy(cap);
    if (pin_par) hipHostFree(pin_par);
    for (uint32_t id : wqkv) gmoe_dense_release(ctx, id);
    if (embd_id != kNoDense) gmoe_dense_release(ctx, embd_id);
    for (void* p : {(void*)table, (void*)norms, (void*)x, (void*)h, (void*)q, (void*)k, (void*)v, (void*)cx,
                    (void*)ao, (void*)y, (void*)logits, (void*)next, (void*)qkv, (void*)par, (void*)px, (void*)ph,
                    (void*)pq, (void*)pk, (void*)pv, (void*)pqkv, (void*)pcx, (void*)pao, (void*)py, (void*)ptok})
      if (p) (void)hipFree(p);
    if (pin_next) (void)hipHostFree(pin_next);
    if (pin_tok) (void)hipHostFree(pin_tok);
  }
};

namespace {

// Step parameters in device memory: tokens [kModelMaxBatch], then the attention entries
// [n_layers][kModelMaxBatch].
constexpr size_t kParEnt = kModelMaxBatch * 4;
size_t par_bytes(uint32_t n_layers) { return kParEnt + (size_t)n_layers * kModelMaxBatch * sizeof(AttnEntry); }

gmoe_status mfail(gmoe_status s, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  set_last_error(buf);
  return s;
}

#define M_TRY(expr)                                                                              \
  do {                                                                                           \
    hipError_t e_ = (expr);                                                                      \
    if (e_ != hipSuccess) return mfail(GMOE_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

#define S_TRY(expr)                 \
  do {                              \
    gmoe_status s_ = (expr);        \
    if (s_ != GMOE_OK) return s_;   \
  } while (0)

gmoe_status check_dense(gmoe_ctx* c, uint32_t id, uint32_t rows, uint32_t cols, const char* what, uint32_t l) {
  uint32_t r, k;
  if (!dense_shape(c, id, &r, &k)) return mfail(GMOE_ERR_INFERENCE, "%s of layer %u: unknown dense weight %u", what, l, id);
  if (r != rows || k != cols)
    return mfail(GMOE_ERR_MODEL, "%s of layer %u is %u x %u, the model needs %u x %u", what, l, r, k, rows, cols);
  return GMOE_OK;
}

}  // namespace

extern "C" {

gmoe_status gmoe_model_create(gmoe_ctx* ctx, const gmoe_model_desc* desc, gmoe_model** out) {
  if (!ctx || !desc || !out) return mfail(GMOE_ERR_INFERENCE, "null context, descriptor or output");
  *out = nullptr;
  const gmoe_model_desc& D = *desc;
  if (!D.kv || !D.moe_layers || !D.wq || !D.wk || !D.wv || !D.wo || !D.attn_norm || !D.ffn_norm ||
      !D.output_norm || !D.token_embd)
    return mfail(GMOE_ERR_INFERENCE, "null weight array in the model descriptor");
  if (D.n_layers == 0 || D.d_model == 0 || D.vocab == 0 || D.d_model % 4)
    return mfail(GMOE_ERR_CONFIG, "model dimensions must be positive, d_model a multiple of 4");
  if (D.d_model > 4u * 256u * kNormVec)
    return mfail(GMOE_ERR_CONFIG, "d_model %u is above the %u a norm workgroup holds", D.d_model, 4u * 256u * kNormVec);
  const bool tied = D.output == GMOE_OUTPUT_TIED;
  if (tied && D.output_math > GMOE_MATH_F32) return mfail(GMOE_ERR_CONFIG, "unknown output_math %u", D.output_math);
  uint32_t kl, qd, kvd;
  kv_dims(D.kv, &kl, &qd, &kvd);
  if (kl != D.n_layers) return mfail(GMOE_ERR_INFERENCE, "the KV cache has %u layers, the model %u", kl, D.n_layers);
  for (uint32_t l = 0; l < D.n_layers; l++) {
    uint32_t w, ne;
    if (!layer_width(ctx, D.moe_layers[l], &w, &ne))
      return mfail(GMOE_ERR_INFERENCE, "layer %u: unknown MoE layer %u", l, D.moe_layers[l]);
    if (w != D.d_model) return mfail(GMOE_ERR_MODEL, "MoE layer of layer %u has d_model %u, not %u", l, w, D.d_model);
    S_TRY(check_dense(ctx, D.wq[l], qd, D.d_model, "wq", l));
    S_TRY(check_dense(ctx, D.wk[l], kvd, D.d_model, "wk", l));
    S_TRY(check_dense(ctx, D.wv[l], kvd, D.d_model, "wv", l));
    S_TRY(check_dense(ctx, D.wo[l], D.d_model, qd, "wo", l));
  }
  if (!tied) S_TRY(check_dense(ctx, D.output, D.vocab, D.d_model, "output", D.n_layers));
  auto* m = new (std::nothrow) gmoe_model;
  if (!m) return mfail(GMOE_ERR_CONFIG, "out of host memory");
  m->ctx = ctx;
  m->kv = D.kv;
  m->n_layers = D.n_layers;
  m->d = D.d_model;
  m->vocab = D.vocab;
  m->qd = qd;
  m->kvd = kvd;
  m->eps = D.rms_eps;
  m->moe.assign(D.moe_layers, D.moe_layers + D.n_layers);
  m->wq.assign(D.wq, D.wq + D.n_layers);
  m->wk.assign(D.wk, D.wk + D.n_layers);
  m->wv.assign(D.wv, D.wv + D.n_layers);
  m->wo.assign(D.wo, D.wo + D.n_layers);
  m->out_id = D.output;
  auto fail = [&](gmoe_status s) {
    delete m;
    return s;
  };
  const hipError_t se = hipSetDevice(ctx_device(ctx));
  if (se != hipSuccess) return fail(mfail(GMOE_ERR_DEVICE, "hipSetDevice: %s", hipGetErrorString(se)));
  const size_t B = kModelMaxBatch, d = D.d_model;
  // the token table: f32 rows as they are; any other type, or a head tied to it, as a
  // dense weight of the model's own (registered from the packed rows, which it copies)
  const bool f32_table = D.token_embd_qtype == GMOE_F32 && !tied;
  if (!f32_table) {
    gmoe_dense_desc dd{};
    dd.rows = D.vocab;
    dd.cols = D.d_model;
    dd.qtype = D.token_embd_qtype;
    dd.math = tied ? D.output_math : GMOE_MATH_PACKED;
    dd.data = D.token_embd;
    uint32_t id;
    if (gmoe_status s = gmoe_dense_register(ctx, &dd, &id)) return fail(s);
    m->embd_id = id;
    if (!dense_tiled(ctx, id, &m->embd_tiled, &m->embd_qt))
      return fail(mfail(GMOE_ERR_INFERENCE, "token table registration lost"));
    if (tied) m->out_id = id;
  }
  const size_t table_bytes = f32_table ? (size_t)D.vocab * d * 4 : 0, norm_bytes = (2 * (size_t)D.n_layers + 1) * d * 4;
  struct Alloc {
    void** p;
    size_t bytes;
  } allocs[] = {{(void**)&m->table, table_bytes},     {(void**)&m->norms, norm_bytes},
                {(void**)&m->x, B * d * 4},           {(void**)&m->h, B * d * 4},
                {(void**)&m->q, B * qd * 4},          {(void**)&m->k, B * kvd * 4},
                {(void**)&m->v, B * kvd * 4},         {(void**)&m->cx, B * qd * 4},
                {(void**)&m->ao, kMaxKsg * B * d * 4}, {(void**)&m->y, B * d * 4},
                {(void**)&m->logits, B * D.vocab * 4}, {(void**)&m->next, B * 4},
                {(void**)&m->qkv, B * (qd + 2 * (size_t)kvd) * 4},
                {(void**)&m->par, par_bytes(D.n_layers)}};
  for (auto& a : allocs) {
    if (!a.bytes) continue;
    const hipError_t e = hipMalloc(a.p, a.bytes);
    if (e != hipSuccess) return fail(mfail(GMOE_ERR_CACHE, "device memory for the model: %s", hipGetErrorString(e)));
  }
  hipError_t e = hipHostMalloc((void**)&m->pin_next, B * 4, hipHostMallocDefault);
  if (e == hipSuccess) e = hipHostMalloc((void**)&m->pin_par, par_bytes(D.n_layers), hipHostMallocDefault);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&m->cap, hipStreamNonBlocking);
  if (e == hipSuccess && table_bytes) e = hipMemcpy(m->table, D.token_embd, table_bytes, hipMemcpyHostToDevice);
  for (uint32_t l = 0; l < D.n_layers && e == hipSuccess; l++) {
    e = hipMemcpy(m->norms + (2 * (size_t)l) * d, D.attn_norm + (size_t)l * d, d * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess)
      e = hipMemcpy(m->norms + (2 * (size_t)l + 1) * d, D.ffn_norm + (size_t)l * d, d * 4, hipMemcpyHostToDevice);
  }
  if (e == hipSuccess)
    e = hipMemcpy(m->norms + 2 * (size_t)D.n_layers * d, D.output_norm, d * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return fail(mfail(GMOE_ERR_DEVICE, "model upload: %s", hipGetErrorString(e)));
  if (qd % kTileRows == 0 && kvd % kTileRows == 0) {
    for (uint32_t l = 0; l < D.n_layers; l++) {
      const uint32_t parts[3] = {D.wq[l], D.wk[l], D.wv[l]};
      uint32_t id;
      if (dense_stack(ctx, parts, 3, &id) != GMOE_OK) break;  // (types differ: separate projections)
      m->wqkv.push_back(id);
    }
    if (m->wqkv.size() != D.n_layers) {
      for (uint32_t id : m->wqkv) gmoe_dense_release(ctx, id);
      m->wqkv.clear();
    }
  }
  *out = m;
  return GMOE_OK;
}

void gmoe_model_destroy(gmoe_model* m) {
  if (!m) return;
  hipSetDevice(ctx_device(m->ctx));
  hipStreamSynchronize(ctx_stream(m->ctx));
  delete m;
}

size_t gmoe_model_trace_floats(const gmoe_model* m, uint32_t n) {
  if (!m) return 0;
  const size_t per_layer = 7 * (size_t)m->d + 2 * (size_t)m->qd + 2 * (size_t)m->kvd;
  return (size_t)n * (m->n_layers * per_layer + 2 * (size_t)m->d);
}

static gmoe_status model_decode(gmoe_model* m, uint32_t n, const uint32_t* seqs, const uint32_t* tokens,
                                uint32_t* next, float* logits, float* trace);

gmoe_status gmoe_model_decode(gmoe_model* m, uint32_t n, const uint32_t* seqs, const uint32_t* tokens, uint32_t* next,
                              float* logits) {
  return model_decode(m, n, seqs, tokens, next, logits, nullptr);
}

gmoe_status gmoe_model_set_graphs(gmoe_model* m, int enable) {
  if (!m) return mfail(GMOE_ERR_INFERENCE, "null model");
  std::lock_guard<std::mutex> g(m->mu);
  m->graphs = enable != 0;
  if (!m->graphs && !m->gcache.empty()) {
    (void)hipSetDevice(ctx_device(m->ctx));
    (void)hipStreamSynchronize(ctx_stream(m->ctx));
    m->drop_graphs();
  }
  m->graph_failed = false;
  return GMOE_OK;
}

int gmoe_model_graph_ready(gmoe_model* m, uint32_t n) {
  if (!m) return 0;
  std::lock_guard<std::mutex> g(m->mu);
  for (const auto& e : m->gcache)
    if (e.n == n && e.exec) return 1;
  return 0;
}

gmoe_status gmoe_model_decode_trace(gmoe_model* m, uint32_t n, const uint32_t* seqs, const uint32_t* tokens,
                                    uint32_t* next, float* logits, float* trace) {
  if (!trace) return mfail(GMOE_ERR_INFERENCE, "null trace buffer");
  return model_decode(m, n, seqs, tokens, next, logits, trace);
}

}  // extern "C"

// The launches of one decode step on st, up to the greedy tokens in m->next. With tk,
// the tokens ride in the embedding's arguments and each layer's attention plans and
// commits its entries as it is queued; without, the tokens and every layer's entries are
// read from the step parameters in device memory (m->par, already committed), so the
// same launches serve every step: the form a graph captures. trace (eager only): every
// layer's activations copied to the host.
static gmoe_status step_launches(gmoe_model* m, uint32_t n, const uint32_t* seqs, const GlueTokens* tk, float* trace,
                                 hipStream_t st, uint32_t nchunk) {
  const uint32_t d = m->d;
  const uint32_t* dtok = reinterpret_cast<const uint32_t*>(m->par);
  const AttnEntry* dent = reinterpret_cast<const AttnEntry*>(m->par + kParEnt);
  // trace: n rows of `width` floats from `src` (rows `pitch` floats apart) at the trace's
  // running offset
  size_t at = 0;
  auto rec = [&](const float* src, uint32_t width, uint32_t pitch) -> hipError_t {
    if (!trace) return hipSuccess;
    const hipError_t e = hipMemcpy2DAsync(trace + at, (size_t)width * 4, src, (size_t)pitch * 4, (size_t)width * 4,
                                          n, hipMemcpyDeviceToHost, st);
    at += (size_t)n * width;
    return e;
  };
  if (m->embd_tiled)
    M_TRY(launch_embed_tiled(m->embd_qt, m->embd_tiled, d, tk, tk ? nullptr : dtok, n, m->x, st));
  else
    M_TRY(tk ? launch_embed(*tk, n, m->table, d, m->x, st) : launch_embed_dev(dtok, n, m->table, d, m->x, st));
  for (uint32_t l = 0; l < m->n_layers; l++) {
    // h = norm(x + previous layer's MoE output, attn_norm)
    M_TRY(launch_add_norm(m->x, l ? m->y : nullptr, m->norms + (2 * (size_t)l) * d, n, d, m->eps, m->h, st));
    M_TRY(rec(m->x, d, d));
    M_TRY(rec(m->h, d, d));
    const AttnEntry* le = dent + (size_t)l * kModelMaxBatch;
    if (!m->wqkv.empty()) {
      const uint32_t row = m->qd + 2 * m->kvd;
      if (tk) {
        S_TRY(gmoe_dense_forward_async(m->ctx, m->wqkv[l], m->h, n, m->qkv, st));
        M_TRY(rec(m->qkv, m->qd, row));
        M_TRY(rec(m->qkv + m->qd, m->kvd, row));
        M_TRY(rec(m->qkv + m->qd + m->kvd, m->kvd, row));
        S_TRY(kv_attend(m->kv, l, seqs, n, m->qkv, m->qkv + m->qd, m->qkv + m->qd + m->kvd, row, row, m->cx, st));
      } else {
        // the projection's K slices go straight to the attention's first launch, which
        // adds them in slice order as it reads q, k and v (no k_reduce_parts launch)
        const float* qkv;
        uint32_t nsl;
        S_TRY(dense_forward_slices(m->ctx, m->wqkv[l], m->h, n, st, &qkv, &nsl));
        S_TRY(kv_attend_dev(m->kv, n, le, nchunk, qkv, qkv + m->qd, qkv + m->qd + m->kvd, row, row, m->cx, st, nsl,
                            (uint64_t)n * row));
      }
    } else {
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wq[l], m->h, n, m->q, st));
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wk[l], m->h, n, m->k, st));
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wv[l], m->h, n, m->v, st));
      M_TRY(rec(m->q, m->qd, m->qd));
      M_TRY(rec(m->k, m->kvd, m->kvd));
      M_TRY(rec(m->v, m->kvd, m->kvd));
      if (tk) S_TRY(gmoe_attention_async(m->kv, l, seqs, n, m->q, m->k, m->v, m->cx, st));
      else S_TRY(kv_attend_dev(m->kv, n, le, nchunk, m->q, m->k, m->v, 0, 0, m->cx, st));
    }
    M_TRY(rec(m->cx, m->qd, m->qd));
    const float* ffn_norm = m->norms + (2 * (size_t)l + 1) * d;
    if (tk) {
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wo[l], m->cx, n, m->ao, st));
      M_TRY(rec(m->ao, d, d));
      M_TRY(launch_add_norm(m->x, m->ao, ffn_norm, n, d, m->eps, m->h, st));
      M_TRY(rec(m->x, d, d));
      M_TRY(rec(m->h, d, d));
      S_TRY(gmoe_ffn_forward_async(m->ctx, m->moe[l], m->h, nullptr, n, m->y, nullptr, nullptr, st));
    } else {
      // the output projection leaves its K slices in m->ao and the MoE front end adds them
      // to the residual and norms it (no k_reduce_parts and no k_add_norm launch)
      const float* ao;
      uint32_t nsl;
      S_TRY(dense_forward_slices(m->ctx, m->wo[l], m->cx, n, st, &ao, &nsl, m->ao));
      S_TRY(ffn_forward_normed(m->ctx, m->moe[l], m->x, ao, nsl, (uint64_t)n * d, ffn_norm, m->eps, m->h, n, m->y,
                               st));
    }
    M_TRY(rec(m->y, d, d));
  }
  M_TRY(launch_add_norm(m->x, m->y, m->norms + 2 * (size_t)m->n_layers * d, n, d, m->eps, m->h, st));
  M_TRY(rec(m->x, d, d));
  M_TRY(rec(m->h, d, d));
  S_TRY(gmoe_dense_forward_async(m->ctx, m->out_id, m->h, n, m->logits, st));
  M_TRY(launch_argmax(m->logits, n, m->vocab, m->next, st));
  return GMOE_OK;
}

// Captures the parameter-reading form of the step for batch n and nchunk attention
// chunks into the graph cache (nothing runs), on the model's own stream, so that no other
// caller's work on the context's stream joins the graph; the graph is launched on the
// context's stream. A capture or instantiation that fails leaves the model on eager steps.
static void capture_step(gmoe_model* m, uint32_t n, uint32_t nchunk) {
  hipStream_t st = m->cap;
  hipGraph_t g = nullptr;
  hipGraphExec_t exec = nullptr;
  gmoe_status s = GMOE_ERR_DEVICE;
  hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
  if (e == hipSuccess) {
    s = step_launches(m, n, nullptr, nullptr, nullptr, st, nchunk);
    e = hipStreamEndCapture(st, &g);
  }
  if (e == hipSuccess && s == GMOE_OK) e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (e != hipSuccess || s != GMOE_OK) {
    (void)hipGetLastError();
    m->graph_failed = true;
    ctx_note_graph(m->ctx, m->moe.data(), m->n_layers, ctx_stream(m->ctx));
    return;
  }
  // one graph per (n, nchunk): a stale one of the same key, or the least recently
  // replayed when the cache is full, makes room (every step synchronises its stream before
  // it returns, so none of them is running)
  auto victim = m->gcache.end();
  for (auto it = m->gcache.begin(); it != m->gcache.end(); ++it)
    if (it->n == n && it->nchunk == nchunk) victim = it;
  if (victim == m->gcache.end() && m->gcache.size() >= gmoe_model::kGraphCache)
    victim = std::min_element(m->gcache.begin(), m->gcache.end(),
                              [](const auto& a, const auto& b) { return a.used < b.used; });
  if (victim != m->gcache.end()) {
    (void)hipGraphExecDestroy(victim->exec);
    m->gcache.erase(victim);
  }
  gmoe_model::Graph ent;
  ent.exec = exec;
  ent.n = n;
  ent.nchunk = nchunk;
  ent.g_ctx = ctx_scratch_id(m->ctx);
  ent.g_kv = kv_scratch_id(m->kv);
  ent.used = ++m->gclock;
  m->gcache.push_back(ent);
  ctx_note_graph(m->ctx, m->moe.data(), m->n_layers, ctx_stream(m->ctx));
}

// The step's device work and the chosen tokens' return, with the sequences' positions
// committed as it goes; a failure may leave some committed (the caller restores them).
// *capture: the step ran the graph form directly and a graph of it is to be captured
// for *cap_chunks attention chunks.
static gmoe_status decode_body(gmoe_model* m, uint32_t n, const uint32_t* seqs, const GlueTokens& tk, uint32_t* next,
                               float* logits, float* trace, bool* capture, uint32_t* cap_chunks) {
  M_TRY(hipSetDevice(ctx_device(m->ctx)));
  hipStream_t st = ctx_stream(m->ctx);
  if (trace || !m->graphs || m->graph_failed) {
    S_TRY(step_launches(m, n, seqs, &tk, trace, st, 0));
  } else {
    // the step's parameters: tokens, and every layer's attention entries, planned, then
    // the scratch they need reserved, then committed (kv_check_step has refused any step
    // that would not fit), so a failed reservation commits nothing
    std::memcpy(m->pin_par, tk.tok, n * 4);
    AttnEntry* pent = reinterpret_cast<AttnEntry*>(m->pin_par + kParEnt);
    uint32_t maxspan;
    S_TRY(kv_plan_step(m->kv, seqs, n, pent, kModelMaxBatch, &maxspan));
    const uint32_t nchunk = kv_step_chunks(m->kv, maxspan);
    gmoe_model::Graph* g = nullptr;
    for (auto& e : m->gcache)
      if (e.n == n && e.nchunk == nchunk && e.g_ctx == ctx_scratch_id(m->ctx) && e.g_kv == kv_scratch_id(m->kv))
        g = &e;
    if (!g) S_TRY(kv_reserve(m->kv, n, nchunk));
    kv_commit_step(m->kv, seqs, n, pent, kModelMaxBatch);
    M_TRY(hipMemcpyAsync(m->par, m->pin_par, par_bytes(m->n_layers), hipMemcpyHostToDevice, st));
    if (g) {
      M_TRY(hipGraphLaunch(g->exec, st));
      g->used = ++m->gclock;
      ctx_note_graph(m->ctx, m->moe.data(), m->n_layers, st);
    } else {
      // this step runs its launches directly (sizing every scratch it needs); the graph is
      // captured after it, for the steps that follow
      S_TRY(step_launches(m, n, seqs, nullptr, nullptr, st, nchunk));
      *capture = true;
      *cap_chunks = nchunk;
    }
  }
  M_TRY(hipMemcpyAsync(m->pin_next, m->next, n * 4, hipMemcpyDeviceToHost, st));
  if (logits) M_TRY(hipMemcpyAsync(logits, m->logits, (size_t)n * m->vocab * 4, hipMemcpyDeviceToHost, st));
  M_TRY(hipStreamSynchronize(st));
  std::memcpy(next, m->pin_next, n * 4);
  return GMOE_OK;
}

static gmoe_status model_decode(gmoe_model* m, uint32_t n, const uint32_t* seqs, const uint32_t* tokens,
                                uint32_t* next, float* logits, float* trace) {
  if (!m || !seqs || !tokens || !next) return mfail(GMOE_ERR_INFERENCE, "null model, sequences, tokens or output");
  if (n == 0 || n > kModelMaxBatch)
    return mfail(GMOE_ERR_INFERENCE, "a decode step takes 1 to %u sequences, not %u", kModelMaxBatch, n);
  std::lock_guard<std::mutex> g(m->mu);
  // refuse before any device work, so a step cannot leave a sequence half-advanced
  GlueTokens tk{};
  for (uint32_t i = 0; i < n; i++) {
    if (tokens[i] >= m->vocab) set_invalid_token(tokens[i]);
    if (tokens[i] >= m->vocab) return mfail(GMOE_ERR_INVALID_TOKEN, "token %u is outside the %u-entry vocabulary", tokens[i], m->vocab);
    tk.tok[i] = tokens[i];
  }
  S_TRY(kv_check_step(m->kv, seqs, n));
  // the MoE layers run from the slab: every expert resident, and kept so until the step's
  // device work has finished
  S_TRY(ctx_pin_layers(m->ctx, m->moe.data(), m->n_layers));
  std::vector<uint32_t> snap;
  kv_snapshot(m->kv, seqs, n, snap);
  bool capture = false;
  uint32_t cap_chunks = 0;
  const gmoe_status s = decode_body(m, n, seqs, tk, next, logits, trace, &capture, &cap_chunks);
  if (s != GMOE_OK) {
    // a refused step leaves every sequence where it was: its queued work has finished
    // before the positions and pages it committed are given back
    (void)hipStreamSynchronize(ctx_stream(m->ctx));
    kv_restore(m->kv, seqs, n, snap);
  }
  ctx_unpin_layers(m->ctx, m->moe.data(), m->n_layers);
  if (s == GMOE_OK && capture) capture_step(m, n, cap_chunks);
  return s;
}

// ---- prompt prefill: forward_tail (llama/mod.rs:1027-1116) ----

namespace {

gmoe_status ensure_prefill_buffers(gmoe_model* m) {
  if (m->px) return GMOE_OK;
  const size_t C = gmoe_model::kPrefillChunk, d = m->d;
  struct Alloc {
    void** p;
    size_t bytes;
  } allocs[] = {{(void**)&m->px, C * d * 4},        {(void**)&m->ph, C * d * 4},
                {(void**)&m->pq, C * m->qd * 4},    {(void**)&m->pk, C * m->kvd * 4},
                {(void**)&m->pv, C * m->kvd * 4},   {(void**)&m->pqkv, C * (m->qd + 2 * (size_t)m->kvd) * 4},
                {(void**)&m->pcx, C * m->qd * 4},   {(void**)&m->pao, C * d * 4},
                {(void**)&m->py, C * d * 4},        {(void**)&m->ptok, C * 4}};
  for (auto& a : allocs) M_TRY(hipMalloc(a.p, a.bytes));
  M_TRY(hipHostMalloc((void**)&m->pin_tok, C * 4, hipHostMallocDefault));
  return GMOE_OK;
}

// One chunk of cn positions of sequence `seq`, layer-major (every layer over the chunk,
// then the next): the launches of a decode step over the chunk's rows, attention taking
// the chunk's positions as consecutive entries of the one sequence (each attending over
// the positions before it and itself), then norm(x, output_norm) of every row into ph.
gmoe_status chunk_launches(gmoe_model* m, uint32_t seq, uint32_t cn, hipStream_t st) {
  const uint32_t d = m->d;
  std::vector<uint32_t> seqs(cn, seq);
  if (m->embd_tiled)
    M_TRY(launch_embed_tiled(m->embd_qt, m->embd_tiled, d, nullptr, m->ptok, cn, m->px, st));
  else
    M_TRY(launch_embed_dev(m->ptok, cn, m->table, d, m->px, st));
  for (uint32_t l = 0; l < m->n_layers; l++) {
    M_TRY(launch_add_norm(m->px, l ? m->py : nullptr, m->norms + (2 * (size_t)l) * d, cn, d, m->eps, m->ph, st));
    if (!m->wqkv.empty()) {
      const uint32_t row = m->qd + 2 * m->kvd;
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wqkv[l], m->ph, cn, m->pqkv, st));
      S_TRY(kv_attend(m->kv, l, seqs.data(), cn, m->pqkv, m->pqkv + m->qd, m->pqkv + m->qd + m->kvd, row, row,
                      m->pcx, st));
    } else {
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wq[l], m->ph, cn, m->pq, st));
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wk[l], m->ph, cn, m->pk, st));
      S_TRY(gmoe_dense_forward_async(m->ctx, m->wv[l], m->ph, cn, m->pv, st));
      S_TRY(kv_attend(m->kv, l, seqs.data(), cn, m->pq, m->pk, m->pv, m->qd, m->kvd, m->pcx, st));
    }
    S_TRY(gmoe_dense_forward_async(m->ctx, m->wo[l], m->pcx, cn, m->pao, st));
    M_TRY(launch_add_norm(m->px, m->pao, m->norms + (2 * (size_t)l + 1) * d, cn, d, m->eps, m->ph, st));
    S_TRY(gmoe_ffn_forward_async(m->ctx, m->moe[l], m->ph, nullptr, cn, m->py, nullptr, nullptr, st));
  }
  M_TRY(launch_add_norm(m->px, m->py, m->norms + 2 * (size_t)m->n_layers * d, cn, d, m->eps, m->ph, st));
  return GMOE_OK;
}

gmoe_status prefill_body(gmoe_model* m, uint32_t seq, uint32_t n, const uint32_t* tokens, uint32_t n_last,
                         uint32_t* next, float* logits) {
  M_TRY(hipSetDevice(ctx_device(m->ctx)));
  S_TRY(ensure_prefill_buffers(m));
  hipStream_t st = ctx_stream(m->ctx);
  // chunks of kPrefillChunk from the front; the last one holds at least n_last positions,
  // whose normed states feed the head (forward_tail's `tail`)
  const uint32_t C = gmoe_model::kPrefillChunk;
  uint32_t lastc = n % C ? n % C : std::min(n, C);
  if (lastc < n_last) lastc = n_last;
  uint32_t cn = 0;
  for (uint32_t c0 = 0; c0 < n; c0 += cn) {
    const uint32_t rest = n - c0;
    cn = rest == lastc ? lastc : std::min(C, rest - lastc);
    M_TRY(hipStreamSynchronize(st));  // the pinned tokens of the previous chunk have been copied
    std::memcpy(m->pin_tok, tokens + c0, (size_t)cn * 4);
    M_TRY(hipMemcpyAsync(m->ptok, m->pin_tok, (size_t)cn * 4, hipMemcpyHostToDevice, st));
    S_TRY(chunk_launches(m, seq, cn, st));
  }
  const float* tail = m->ph + (size_t)(cn - n_last) * m->d;
  S_TRY(gmoe_dense_forward_async(m->ctx, m->out_id, tail, n_last, m->logits, st));
  M_TRY(launch_argmax(m->logits, n_last, m->vocab, m->next, st));
  M_TRY(hipMemcpyAsync(m->pin_next, m->next, n_last * 4, hipMemcpyDeviceToHost, st));
  if (logits) M_TRY(hipMemcpyAsync(logits, m->logits, (size_t)n_last * m->vocab * 4, hipMemcpyDeviceToHost, st));
  M_TRY(hipStreamSynchronize(st));
  std::memcpy(next, m->pin_next, n_last * 4);
  return GMOE_OK;
}

}  // namespace

extern "C" gmoe_status gmoe_model_prefill(gmoe_model* m, uint32_t seq, uint32_t n, const uint32_t* tokens,
                                          uint32_t n_last, uint32_t* next, float* logits) {
  if (!m || !tokens || !next) return mfail(GMOE_ERR_INFERENCE, "null model, tokens or output");
  if (n == 0) return mfail(GMOE_ERR_INFERENCE, "no new tokens to process for this context");
  if (n_last == 0 || n_last > n || n_last > kModelMaxBatch)
    return mfail(GMOE_ERR_INFERENCE, "asked for the last %u positions of %u (1 to %u)", n_last, n, kModelMaxBatch);
  std::lock_guard<std::mutex> g(m->mu);
  // refused before any layer runs: tokens outside the vocabulary, then the window and pool
  for (uint32_t i = 0; i < n; i++)
    if (tokens[i] >= m->vocab) {
      set_invalid_token(tokens[i]);
      return mfail(GMOE_ERR_INVALID_TOKEN, "token %u is outside the %u-entry vocabulary", tokens[i], m->vocab);
    }
  S_TRY(kv_check_prefill(m->kv, seq, n));
  S_TRY(ctx_pin_layers(m->ctx, m->moe.data(), m->n_layers));
  std::vector<uint32_t> snap;
  kv_snapshot(m->kv, &seq, 1, snap);
  const gmoe_status s = prefill_body(m, seq, n, tokens, n_last, next, logits);
  if (s != GMOE_OK) {
    (void)hipStreamSynchronize(ctx_stream(m->ctx));
    kv_restore(m->kv, &seq, 1, snap);
  }
  ctx_unpin_layers(m->ctx, m->moe.data(), m->n_layers);
  return s;
}
