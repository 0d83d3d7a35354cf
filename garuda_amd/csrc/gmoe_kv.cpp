// gmoe_kv.cpp — paged KV cache on the device and the decode-attention calls.
//
// The reference's KVCacheState (garuda/src/cache/mod.rs:221-600) holds one sequence's
// keys and values for one layer in blocks of `block_size` positions, capped at
// max_positions, with an optional sliding window (attention_start, :333-338). Here the
// blocks are pages of one device pool shared by every sequence and layer; the host keeps
// each (sequence, layer)'s length and page list, and the device keeps its page table,
// which the append kernel extends when a token opens a page. attend_one
// (llama/mod.rs:766-821) runs as three launches (gmoe_attn.hip).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <memory>
#include <mutex>
#include <vector>

#include "../../include/garuda_moe.h"
#include "gmoe_internal.h"

namespace gmoe {
void set_last_error(const char* msg);
int ctx_device(gmoe_ctx* c);
hipStream_t ctx_stream(gmoe_ctx* c);
}  // namespace gmoe

using namespace gmoe;

namespace {

gmoe_status kfail(gmoe_status s, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  set_last_error(buf);
  return s;
}

#define KV_TRY(expr)                                                                       \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess) return kfail(GMOE_ERR_DEVICE, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

constexpr int kPinSlots = 8;

struct Seq {
  bool open = false;
  std::vector<uint32_t> len;                 // [layer]
  std::vector<std::vector<uint32_t>> pages;  // [layer] page ids in position order
};

}  // namespace

struct gmoe_kv {
  gmoe_ctx* ctx = nullptr;
  gmoe_kv_desc d{};
  uint32_t kvd = 0, ppseq = 0;
  uint64_t page_floats = 0;
  float* pool = nullptr;      // [max_pages][2][block_size][kvd]
  uint32_t* tables = nullptr; // [max_seqs][n_layers][ppseq]
  std::vector<uint32_t> free_pages;
  std::vector<Seq> seqs;
  uint8_t* scratch = nullptr; // per call: entries, rotated q, chunk partials
  size_t scratch_bytes = 0;
  AttnEntry* pin = nullptr;   // pinned staging of the entries of calls above kAttnInline tokens, a ring
  uint32_t pin_cap = 0;       // entries per slot
  hipEvent_t pin_ev[kPinSlots]{};
  int pin_slot = 0;
  uint32_t fail_reserves = 0;  // test hook: reservations still to refuse (gmoe_kv_fail_reserves)
  std::mutex mu;

  ~gmoe_kv() {
    if (pool) hipFree(pool);
    if (tables) hipFree(tables);
    if (scratch) hipFree(scratch);
    if (pin) hipHostFree(pin);
    for (auto& e : pin_ev)
      if (e) hipEventDestroy(e);
  }
};

namespace {

gmoe_status grow_scratch(gmoe_kv* kv, size_t bytes) {
  if (bytes <= kv->scratch_bytes) return GMOE_OK;
  KV_TRY(hipDeviceSynchronize());  // queued calls may still use the old buffer
  if (kv->scratch) KV_TRY(hipFree(kv->scratch));
  kv->scratch = nullptr;
  kv->scratch_bytes = 0;
  const size_t want = std::max(bytes, (size_t)8 << 20);
  KV_TRY(hipMalloc(&kv->scratch, want));
  kv->scratch_bytes = want;
  return GMOE_OK;
}

gmoe_status grow_pinned(gmoe_kv* kv, uint32_t n) {
  if (n <= kv->pin_cap) return GMOE_OK;
  for (auto& e : kv->pin_ev) KV_TRY(hipEventSynchronize(e));
  if (kv->pin) KV_TRY(hipHostFree(kv->pin));
  kv->pin = nullptr;
  const uint32_t cap = std::max(n, 256u);
  KV_TRY(hipHostMalloc((void**)&kv->pin, kPinSlots * (size_t)cap * sizeof(AttnEntry), hipHostMallocDefault));
  kv->pin_cap = cap;
  return GMOE_OK;
}

// The call's entries (positions, windows, pages), checked against the window and the
// free pages but not committed; maxspan receives the longest span attended.
gmoe_status plan(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, AttnEntry* ent, uint32_t* maxspan) {
  const gmoe_kv_desc& D = kv->d;
  if (layer >= D.n_layers) return kfail(GMOE_ERR_INFERENCE, "layer %u of %u", layer, D.n_layers);
  if (n == 0 || !seqs) return kfail(GMOE_ERR_INFERENCE, "empty attention call");
  std::vector<uint32_t> extra(kv->seqs.size(), 0);  // this call's entries so far, per sequence
  uint32_t need_pages = 0;
  *maxspan = 1;
  for (uint32_t i = 0; i < n; i++) {
    const uint32_t s = seqs[i];
    if (s >= kv->seqs.size() || !kv->seqs[s].open) return kfail(GMOE_ERR_INFERENCE, "sequence %u is not open", s);
    const uint32_t pos = kv->seqs[s].len[layer] + extra[s]++;
    if (pos >= D.max_positions)
      return kfail(GMOE_ERR_CACHE, "context window of %u positions is exhausted", D.max_positions);
    if (pos % D.block_size == 0) need_pages++;
    const uint32_t start = D.sliding_window && pos + 1 > D.sliding_window ? pos + 1 - D.sliding_window : 0;
    *maxspan = std::max(*maxspan, pos + 1 - start);
    ent[i].pos = pos;
    ent[i].start = start;
    ent[i].pages = kv->tables + ((size_t)s * D.n_layers + layer) * kv->ppseq;
  }
  if (need_pages > kv->free_pages.size())
    return kfail(GMOE_ERR_CACHE, "the KV pool has %zu free pages, the call needs %u", kv->free_pages.size(),
                 need_pages);
  return GMOE_OK;
}

// Commits a planned call: lengths advance and pages are taken.
void commit(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, AttnEntry* ent) {
  const gmoe_kv_desc& D = kv->d;
  for (uint32_t i = 0; i < n; i++) {
    Seq& S = kv->seqs[seqs[i]];
    if (ent[i].pos % D.block_size == 0) {
      const uint32_t p = kv->free_pages.back();
      kv->free_pages.pop_back();
      S.pages[layer].push_back(p);
      ent[i].fresh = 1;
    } else {
      ent[i].fresh = 0;
    }
    ent[i].page = S.pages[layer][ent[i].pos / D.block_size];
    S.len[layer] = ent[i].pos + 1;
  }
}

// Scratch of a call of n entries and nchunk chunks: entries, rotated q, partials.
struct AttnLayout {
  size_t o_ent, o_qr, o_part, total;
};
AttnLayout layout(const gmoe_kv* kv, uint32_t n, uint32_t nchunk) {
  const gmoe_kv_desc& D = kv->d;
  const size_t qn = (size_t)n * D.n_heads * D.head_dim;
  AttnLayout l;
  l.o_ent = 0;
  l.o_qr = (n * sizeof(AttnEntry) + 255) & ~(size_t)255;
  l.o_part = l.o_qr + ((qn * 4 + 255) & ~(size_t)255);
  l.total = l.o_part + (size_t)n * D.n_heads * nchunk * (D.head_dim + 2) * 4;
  return l;
}

AttnArgs args(const gmoe_kv* kv, uint32_t n, uint32_t nchunk, const AttnLayout& l, const float* q, const float* k,
              const float* v, float* out, uint32_t q_stride, uint32_t kv_stride) {
  const gmoe_kv_desc& D = kv->d;
  AttnArgs a{};
  a.n = n;
  a.n_heads = D.n_heads;
  a.n_kv = D.n_kv_heads;
  a.hd = D.head_dim;
  a.bs = D.block_size;
  a.theta = D.rope_theta;
  a.scale = 1.0f / std::sqrt((float)D.head_dim);
  a.pool = kv->pool;
  a.page_floats = kv->page_floats;
  a.q = q;
  a.k = k;
  a.v = v;
  a.qr = reinterpret_cast<float*>(kv->scratch + l.o_qr);
  a.part = reinterpret_cast<float*>(kv->scratch + l.o_part);
  a.nchunk = nchunk;
  a.ctx = out;
  a.q_stride = q_stride ? q_stride : D.n_heads * D.head_dim;
  a.kv_stride = kv_stride ? kv_stride : kv->kvd;
  return a;
}

// Plans the call's entries and commits them (lengths advance and pages are taken only when
// the whole call fits), then queues the three launches.
gmoe_status attend(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, const float* q, const float* k,
                   const float* v, float* out, hipStream_t st, uint32_t q_stride = 0, uint32_t kv_stride = 0) {
  std::vector<AttnEntry> ent(n ? n : 1);
  uint32_t maxspan;
  if (gmoe_status s = plan(kv, layer, seqs, n, ent.data(), &maxspan)) return s;
  const uint32_t nchunk = (maxspan + kAttnChunk - 1) / kAttnChunk;
  const AttnLayout l = layout(kv, n, nchunk);
  if (gmoe_status s = grow_scratch(kv, l.total)) return s;
  if (n > kAttnInline)
    if (gmoe_status s = grow_pinned(kv, n)) return s;
  commit(kv, layer, seqs, n, ent.data());
  AttnArgs a = args(kv, n, nchunk, l, q, k, v, out, q_stride, kv_stride);
  if (n <= kAttnInline) {  // a decode batch: the entries ride in the kernel arguments
    std::copy(ent.begin(), ent.begin() + n, a.inl);
    a.ent = nullptr;
  } else {
    const int h = kv->pin_slot;
    kv->pin_slot = (h + 1) % kPinSlots;
    KV_TRY(hipEventSynchronize(kv->pin_ev[h]));  // the slot's previous copy has been read
    AttnEntry* pin = kv->pin + (size_t)h * kv->pin_cap;
    std::copy(ent.begin(), ent.begin() + n, pin);
    KV_TRY(hipMemcpyAsync(kv->scratch + l.o_ent, pin, n * sizeof(AttnEntry), hipMemcpyHostToDevice, st));
    KV_TRY(hipEventRecord(kv->pin_ev[h], st));
    a.ent = reinterpret_cast<const AttnEntry*>(kv->scratch + l.o_ent);
  }
  KV_TRY(launch_attention(a, st));
  return GMOE_OK;
}

}  // namespace

namespace gmoe {

// For the decode-step driver (gmoe_model.cpp): the cache's widths, and whether each of
// the (distinct) sequences can take one more position in every layer, refused before
// any layer has run (as logits_batch refuses, llama/mod.rs:1163-1176).
void kv_dims(gmoe_kv* kv, uint32_t* n_layers, uint32_t* q_dim, uint32_t* kv_dim) {
  *n_layers = kv->d.n_layers;
  *q_dim = kv->d.n_heads * kv->d.head_dim;
  *kv_dim = kv->kvd;
}

// Attention over rows of q, k and v that sit q_stride and kv_stride floats apart (the
// model step's stacked q|k|v projection), queued on st.
gmoe_status kv_attend(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, const float* q, const float* k,
                      const float* v, uint32_t q_stride, uint32_t kv_stride, float* out, hipStream_t st) {
  std::lock_guard<std::mutex> g(kv->mu);
  KV_TRY(hipSetDevice(ctx_device(kv->ctx)));
  return attend(kv, layer, seqs, n, q, k, v, out, st, q_stride, kv_stride);
}

gmoe_status kv_check_step(gmoe_kv* kv, const uint32_t* seqs, uint32_t n) {
  std::lock_guard<std::mutex> g(kv->mu);
  const gmoe_kv_desc& D = kv->d;
  uint64_t pages = 0;
  for (uint32_t i = 0; i < n; i++) {
    const uint32_t s = seqs[i];
    if (s >= kv->seqs.size() || !kv->seqs[s].open) return kfail(GMOE_ERR_INFERENCE, "sequence %u is not open", s);
    for (uint32_t j = 0; j < i; j++)
      if (seqs[j] == s) return kfail(GMOE_ERR_INFERENCE, "sequence %u appears twice in one decode step", s);
    for (uint32_t l = 0; l < D.n_layers; l++) {
      const uint32_t pos = kv->seqs[s].len[l];
      if (pos + 1 > D.max_positions)
        return kfail(GMOE_ERR_CACHE, "context window of %u positions is exhausted", D.max_positions);
      if (pos % D.block_size == 0) pages++;
    }
  }
  if (pages > kv->free_pages.size())
    return kfail(GMOE_ERR_CACHE, "the KV pool has %zu free pages, the step needs %llu", kv->free_pages.size(),
                 (unsigned long long)pages);
  return GMOE_OK;
}

// A prefill of n positions of one sequence (forward_tail, llama/mod.rs:1058-1066): the
// window and the pool checked for every layer before any layer runs.
gmoe_status kv_check_prefill(gmoe_kv* kv, uint32_t seq, uint32_t n) {
  std::lock_guard<std::mutex> g(kv->mu);
  const gmoe_kv_desc& D = kv->d;
  if (seq >= kv->seqs.size() || !kv->seqs[seq].open) return kfail(GMOE_ERR_INFERENCE, "sequence %u is not open", seq);
  uint64_t pages = 0;
  for (uint32_t l = 0; l < D.n_layers; l++) {
    const uint32_t len = kv->seqs[seq].len[l];
    if ((uint64_t)len + n > D.max_positions)
      return kfail(GMOE_ERR_CACHE, "%u tokens do not fit the %u-position context window (%u used)", n,
                   D.max_positions, len);
    for (uint64_t p = len; p < (uint64_t)len + n; p++)
      if (p % D.block_size == 0) pages++;
  }
  if (pages > kv->free_pages.size())
    return kfail(GMOE_ERR_CACHE, "the KV pool has %zu free pages, the prefill needs %llu", kv->free_pages.size(),
                 (unsigned long long)pages);
  return GMOE_OK;
}

// For decode steps replayed from a HIP graph (gmoe_model.cpp): the host plans every
// layer's entries (kv_plan_step), reserves the attention scratch, then commits them
// (kv_commit_step) and copies them to device memory the graph's attention launches read
// (kv_attend_dev). Those launches span a fixed number of chunks, the step's longest span
// rounded up to a power of two (kv_step_chunks), so one graph serves every step until a
// sequence outgrows the bucket; chunks past an entry's span are empty and merge as
// nothing, so the result is the same as over the entry's own chunks. kv_graph_chunks is
// the most a sequence can reach.
uint32_t kv_graph_chunks(gmoe_kv* kv) {
  const gmoe_kv_desc& D = kv->d;
  const uint32_t span = D.sliding_window ? std::min(D.sliding_window, D.max_positions) : D.max_positions;
  return (span + kAttnChunk - 1) / kAttnChunk;
}

uint32_t kv_step_chunks(gmoe_kv* kv, uint32_t maxspan) {
  const uint32_t need = (maxspan + kAttnChunk - 1) / kAttnChunk;
  uint32_t b = 1;
  while (b < need) b *= 2;
  return std::min(b, kv_graph_chunks(kv));
}

// Every layer's entries of a step (ents[l * stride + i]), planned but not committed, and
// the longest span any of them attends.
gmoe_status kv_plan_step(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, AttnEntry* ents, size_t stride,
                         uint32_t* maxspan) {
  std::lock_guard<std::mutex> g(kv->mu);
  *maxspan = 1;
  for (uint32_t l = 0; l < kv->d.n_layers; l++) {
    uint32_t ms;
    if (gmoe_status s = plan(kv, l, seqs, n, ents + (size_t)l * stride, &ms)) return s;
    *maxspan = std::max(*maxspan, ms);
  }
  return GMOE_OK;
}

void kv_commit_step(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, AttnEntry* ents, size_t stride) {
  std::lock_guard<std::mutex> g(kv->mu);
  for (uint32_t l = 0; l < kv->d.n_layers; l++) commit(kv, l, seqs, n, ents + (size_t)l * stride);
}

// The step's sequences as they stand (every layer's length and page count), and their
// return to it: pages taken since go back to the free list, lengths go back. A step that
// fails after committing positions restores them, so a refused step leaves every sequence
// where it was.
void kv_snapshot(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, std::vector<uint32_t>& snap) {
  std::lock_guard<std::mutex> g(kv->mu);
  snap.clear();
  for (uint32_t i = 0; i < n; i++) {
    const Seq& S = kv->seqs[seqs[i]];
    for (uint32_t l = 0; l < kv->d.n_layers; l++) {
      snap.push_back(S.len[l]);
      snap.push_back((uint32_t)S.pages[l].size());
    }
  }
}

void kv_restore(gmoe_kv* kv, const uint32_t* seqs, uint32_t n, const std::vector<uint32_t>& snap) {
  std::lock_guard<std::mutex> g(kv->mu);
  size_t at = 0;
  for (uint32_t i = 0; i < n && at + 2 * kv->d.n_layers <= snap.size(); i++) {
    Seq& S = kv->seqs[seqs[i]];
    for (uint32_t l = 0; l < kv->d.n_layers; l++, at += 2) {
      S.len[l] = snap[at];
      while (S.pages[l].size() > snap[at + 1]) {
        kv->free_pages.push_back(S.pages[l].back());
        S.pages[l].pop_back();
      }
    }
  }
}


gmoe_status kv_reserve(gmoe_kv* kv, uint32_t n, uint32_t nchunk) {
  std::lock_guard<std::mutex> g(kv->mu);
  KV_TRY(hipSetDevice(ctx_device(kv->ctx)));
  if (kv->fail_reserves) {
    kv->fail_reserves--;
    return kfail(GMOE_ERR_DEVICE, "attention scratch of %zu bytes: allocation refused (test hook)",
                 layout(kv, n, nchunk).total);
  }
  return grow_scratch(kv, layout(kv, n, nchunk).total);
}

const void* kv_scratch_id(gmoe_kv* kv) { return kv->scratch; }

gmoe_status kv_plan_commit(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, AttnEntry* ent) {
  std::lock_guard<std::mutex> g(kv->mu);
  uint32_t maxspan;
  if (gmoe_status s = plan(kv, layer, seqs, n, ent, &maxspan)) return s;
  commit(kv, layer, seqs, n, ent);
  return GMOE_OK;
}

gmoe_status kv_attend_dev(gmoe_kv* kv, uint32_t n, const AttnEntry* d_ent, uint32_t nchunk, const float* q,
                          const float* k, const float* v, uint32_t q_stride, uint32_t kv_stride, float* out,
                          hipStream_t st, uint32_t nsl, uint64_t sl_stride) {
  std::lock_guard<std::mutex> g(kv->mu);
  const AttnLayout l = layout(kv, n, nchunk);
  if (l.total > kv->scratch_bytes) return kfail(GMOE_ERR_INFERENCE, "attention scratch not reserved");
  if (nsl > kMaxKsg) return kfail(GMOE_ERR_INFERENCE, "%u K slices exceed %u", nsl, kMaxKsg);
  AttnArgs a = args(kv, n, nchunk, l, q, k, v, out, q_stride, kv_stride);
  a.ent = d_ent;
  a.nsl = nsl;
  a.sl_stride = sl_stride;
  KV_TRY(launch_attention(a, st));
  return GMOE_OK;
}

}  // namespace gmoe

extern "C" {

gmoe_status gmoe_kv_create(gmoe_ctx* ctx, const gmoe_kv_desc* desc, gmoe_kv** out) {
  if (!ctx || !desc || !out) return kfail(GMOE_ERR_INFERENCE, "null context, descriptor or output");
  *out = nullptr;
  const gmoe_kv_desc& D = *desc;
  if (D.n_layers == 0 || D.n_heads == 0 || D.n_kv_heads == 0 || D.head_dim == 0 || D.block_size == 0 ||
      D.max_positions == 0 || D.max_seqs == 0 || D.max_pages == 0)
    return kfail(GMOE_ERR_CONFIG, "KV cache dimensions must be positive");
  if (D.n_heads % D.n_kv_heads || D.n_heads / D.n_kv_heads > kAttnMaxGroup)
    return kfail(GMOE_ERR_MODEL, "n_heads %u must be a multiple of n_kv_heads %u, at most %u per kv head", D.n_heads,
                 D.n_kv_heads, kAttnMaxGroup);
  if (D.head_dim % 4 || D.head_dim > kAttnMaxHd)
    return kfail(GMOE_ERR_MODEL, "head_dim %u must be a multiple of 4 and at most %u", D.head_dim, kAttnMaxHd);
  if (!(D.rope_theta > 0.0f)) return kfail(GMOE_ERR_CONFIG, "rope_theta must be positive");
  std::unique_ptr<gmoe_kv> kv(new gmoe_kv);
  kv->ctx = ctx;
  kv->d = D;
  kv->kvd = D.n_kv_heads * D.head_dim;
  kv->ppseq = (D.max_positions + D.block_size - 1) / D.block_size;
  kv->page_floats = 2ull * D.block_size * kv->kvd;
  KV_TRY(hipSetDevice(ctx_device(ctx)));
  KV_TRY(hipMalloc(&kv->pool, D.max_pages * kv->page_floats * 4));
  KV_TRY(hipMalloc(&kv->tables, (size_t)D.max_seqs * D.n_layers * kv->ppseq * 4));
  for (auto& e : kv->pin_ev) KV_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  kv->free_pages.resize(D.max_pages);
  for (uint64_t i = 0; i < D.max_pages; i++) kv->free_pages[i] = (uint32_t)(D.max_pages - 1 - i);  // pops 0 first
  kv->seqs.resize(D.max_seqs);
  *out = kv.release();
  return GMOE_OK;
}

void gmoe_kv_destroy(gmoe_kv* kv) {
  if (!kv) return;
  hipSetDevice(ctx_device(kv->ctx));
  hipDeviceSynchronize();  // queued calls may still use its buffers
  delete kv;
}

gmoe_status gmoe_kv_seq_open(gmoe_kv* kv, uint32_t* seq) {
  if (!kv || !seq) return kfail(GMOE_ERR_INFERENCE, "null cache or output");
  std::lock_guard<std::mutex> g(kv->mu);
  for (uint32_t s = 0; s < kv->seqs.size(); s++)
    if (!kv->seqs[s].open) {
      Seq& S = kv->seqs[s];
      S.open = true;
      S.len.assign(kv->d.n_layers, 0);
      S.pages.assign(kv->d.n_layers, {});
      *seq = s;
      return GMOE_OK;
    }
  return kfail(GMOE_ERR_CACHE, "all %u sequences are open", kv->d.max_seqs);
}

gmoe_status gmoe_kv_seq_close(gmoe_kv* kv, uint32_t seq) {
  if (!kv) return kfail(GMOE_ERR_INFERENCE, "null cache");
  std::lock_guard<std::mutex> g(kv->mu);
  if (seq >= kv->seqs.size() || !kv->seqs[seq].open) return kfail(GMOE_ERR_INFERENCE, "sequence %u is not open", seq);
  KV_TRY(hipSetDevice(ctx_device(kv->ctx)));
  KV_TRY(hipDeviceSynchronize());  // queued calls may still read its pages
  Seq& S = kv->seqs[seq];
  for (auto& pl : S.pages)
    for (uint32_t p : pl) kv->free_pages.push_back(p);
  S = Seq{};
  return GMOE_OK;
}

gmoe_status gmoe_kv_seq_len(const gmoe_kv* kv, uint32_t seq, uint32_t layer, uint32_t* len) {
  if (!kv || !len) return kfail(GMOE_ERR_INFERENCE, "null cache or output");
  if (seq >= kv->seqs.size() || !kv->seqs[seq].open) return kfail(GMOE_ERR_INFERENCE, "sequence %u is not open", seq);
  if (layer >= kv->d.n_layers) return kfail(GMOE_ERR_INFERENCE, "layer %u of %u", layer, kv->d.n_layers);
  *len = kv->seqs[seq].len[layer];
  return GMOE_OK;
}

gmoe_status gmoe_kv_free_pages(gmoe_kv* kv, uint64_t* pages) {
  if (!kv || !pages) return kfail(GMOE_ERR_INFERENCE, "null cache or output");
  std::lock_guard<std::mutex> g(kv->mu);
  *pages = kv->free_pages.size();
  return GMOE_OK;
}

gmoe_status gmoe_kv_fail_reserves(gmoe_kv* kv, uint32_t count) {
  if (!kv) return kfail(GMOE_ERR_INFERENCE, "null cache");
  std::lock_guard<std::mutex> g(kv->mu);
  kv->fail_reserves = count;
  return GMOE_OK;
}

gmoe_status gmoe_attention(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, const float* q,
                           const float* k, const float* v, float* context) {
  if (!kv || !q || !k || !v || !context) return kfail(GMOE_ERR_INFERENCE, "null cache or activation pointer");
  std::lock_guard<std::mutex> g(kv->mu);
  KV_TRY(hipSetDevice(ctx_device(kv->ctx)));
  const gmoe_kv_desc& D = kv->d;
  const size_t qb = (size_t)n * D.n_heads * D.head_dim * 4, kb = (size_t)n * kv->kvd * 4;
  float* buf = nullptr;
  KV_TRY(hipMalloc(&buf, 2 * qb + 2 * kb));
  float *dq = buf, *dk = buf + qb / 4, *dv = dk + kb / 4, *dout = dv + kb / 4;
  hipStream_t st = ctx_stream(kv->ctx);
  hipError_t e = hipMemcpyAsync(dq, q, qb, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(dk, k, kb, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(dv, v, kb, hipMemcpyHostToDevice, st);
  gmoe_status s = e == hipSuccess ? attend(kv, layer, seqs, n, dq, dk, dv, dout, st)
                                  : kfail(GMOE_ERR_DEVICE, "attention inputs: %s", hipGetErrorString(e));
  if (s == GMOE_OK) {
    e = hipMemcpyAsync(context, dout, qb, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) s = kfail(GMOE_ERR_DEVICE, "attention: %s", hipGetErrorString(e));
  }
  hipStreamSynchronize(st);
  hipFree(buf);
  return s;
}

gmoe_status gmoe_attention_async(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, const float* d_q,
                                 const float* d_k, const float* d_v, float* d_context, void* stream) {
  if (!kv || !d_q || !d_k || !d_v || !d_context) return kfail(GMOE_ERR_INFERENCE, "null cache or activation pointer");
  std::lock_guard<std::mutex> g(kv->mu);
  KV_TRY(hipSetDevice(ctx_device(kv->ctx)));
  return attend(kv, layer, seqs, n, d_q, d_k, d_v, d_context, stream ? (hipStream_t)stream : ctx_stream(kv->ctx));
}

}  // extern "C"
