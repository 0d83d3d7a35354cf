// gmoe_api.cpp — host runtime behind include/garuda_moe.h.
//
// Owns the device context, the HBM expert slab (the L1 tier: cache::ExpertCache's
// byte-budgeted LRU, garuda/src/cache/mod.rs:18-137, holding still-packed experts),
// the per-context scratch arena, and the launch sequence of one feed-forward call:
//   route -> dispatch -> (activation quantiser) -> gate/up -> down -> combine.
// Every entry validates before touching the device so a refused call changes nothing
// (garuda/src/llama/mod.rs:1160-1172), and reports errors as status codes with a
// thread-local message (never aborts; core/mod.rs:255-258).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstdarg>
#include <deque>
#include <cstdio>
#include <cstring>
#include <list>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/garuda_moe.h"
#include "gmoe_internal.h"

using namespace gmoe;

namespace {

thread_local std::string g_err;
thread_local uint32_t g_bad_token = UINT32_MAX;  // the token of the last GMOE_ERR_INVALID_TOKEN

gmoe_status fail(gmoe_status s, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return s;
}

#define HIP_TRY(expr)                                                                    \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess)                                                                \
      return fail(GMOE_ERR_DEVICE, "%s failed: %s", #expr, hipGetErrorString(e_));       \
  } while (0)

const char* type_name(uint32_t t) {
  switch (t) {
    case F32: return "F32";
    case F16: return "F16";
    case Q4_0: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case Q8_0: return "Q8_0";
    case Q2_K: return "Q2_K";
    case Q3_K: return "Q3_K";
    case Q4_K: return "Q4_K";
    case Q5_K: return "Q5_K";
    case Q6_K: return "Q6_K";
  }
  return "unknown";
}

// quant/mod.rs:89-98
gmoe_status byte_size(uint32_t t, uint64_t n, uint64_t* out) {
  uint32_t e, b;
  if (!block_layout(t, &e, &b))
    return fail(GMOE_ERR_MODEL, "tensor type %s (%u) is not supported", type_name(t), t);
  if (n % e != 0)
    return fail(GMOE_ERR_MODEL, "%s tensor has %llu elements, not a multiple of the block size %u",
                type_name(t), (unsigned long long)n, e);
  *out = n / e * b;
  return GMOE_OK;
}

// Kernels walk F32/F16 rows 32 values at a time and the activation quantiser works per
// 32, so every product's K must be a multiple of 32 (true of every k-quant row).
bool k_ok(uint32_t t, uint32_t K) {
  uint32_t e, b;
  block_layout(t, &e, &b);
  return K % 32 == 0 && K % e == 0;
}

struct Slab {
  uint8_t* base = nullptr;
  uint64_t cap = 0;
  std::map<uint64_t, uint64_t> free_;  // offset -> size
  uint64_t used = 0;

  bool alloc(uint64_t size, uint64_t* off) {
    size = (size + 255) & ~uint64_t(255);
    for (auto it = free_.begin(); it != free_.end(); ++it) {
      if (it->second >= size) {
        *off = it->first;
        uint64_t rest = it->second - size, noff = it->first + size;
        free_.erase(it);
        if (rest) free_[noff] = rest;
        used += size;
        return true;
      }
    }
    return false;
  }
  void release(uint64_t off, uint64_t size) {
    size = (size + 255) & ~uint64_t(255);
    used -= size;
    auto it = free_.emplace(off, size).first;
    auto nx = std::next(it);
    if (nx != free_.end() && it->first + it->second == nx->first) {
      it->second += nx->second;
      free_.erase(nx);
    }
    if (it != free_.begin()) {
      auto pv = std::prev(it);
      if (pv->first + pv->second == it->first) {
        pv->second += it->second;
        free_.erase(it);
      }
    }
  }
};

struct Proj {
  uint32_t qtype, rows, cols;
  uint64_t row_bytes, bytes_dev;  // bytes_dev = size of the tiled matrix in the slab
  std::vector<const uint8_t*> host;      // per expert
};

using LruList = std::list<std::pair<uint32_t, uint32_t>>;  // (layer, expert), least recent first
using Keep = std::vector<std::pair<uint32_t, uint32_t>>;      // (layer, expert) pairs not to evict

// An expert's place on the staging thread's way (Layer::pending); GMOE_EXPERT_* says the
// same to callers.
enum : uint8_t { kAbsent = 0, kQueued = 1, kStaging = 2 };

struct Layer {
  uint32_t d, f, ne, k, gating, combine, math;
  Proj p[3];                      // gate, up, down
  float* router = nullptr;        // device
  const uint8_t** eptr = nullptr; // device [3][ne]
  std::vector<const uint8_t*> eptr_host;
  std::vector<int64_t> slot;      // per expert: slab offset or -1
  std::vector<LruList::iterator> lru_pos;  // per resident expert: its place in the LRU
  std::vector<uint8_t> pending;   // per expert: kAbsent, or queued / staging by the staging thread
  uint64_t expert_bytes = 0;
  // the stream of the layer's last queued call (null: none): an evicted expert's region is
  // free once that stream has drained. An event recorded per call would say exactly when,
  // but each record puts a marker on the GPU timeline (about 4 us a call).
  hipStream_t last_stream = nullptr;
  // experts pulled from a lower tier when staged (gmoe_layer_register_fetch) instead of
  // from host pointers given at registration
  gmoe_expert_fetch fetch = nullptr;
  void* fetch_user = nullptr;
  // model steps in flight that read every expert of the layer (ctx_pin_layers): while
  // non-zero no expert of the layer is chosen for eviction, nor evicted on request
  uint32_t pins = 0;
  bool alive = true;
};

struct Timing {
  hipEvent_t a, b, c;
};

// A dense packed projection (Weight::Packed / Weight::Full, llama/mod.rs:43-85), tiled in
// its own device allocation outside the expert slab's LRU: dense weights are read by every
// token, so they stay resident.
struct Dense {
  uint32_t qtype, rows, cols, math;
  uint8_t* tiled = nullptr;
  uint64_t tiled_bytes = 0;
  ExpertWork* work_tab = nullptr;  // [kDenseTab]: entry i is the call of i + 1 tokens
  bool alive = true;
};
// Calls of up to kDenseTab tokens read a precomputed work entry and the context's
// identity table (slot -> token, and token tiles) instead of a setup launch.
constexpr uint32_t kDenseTab = 2048;
// Experts a layer may have: the dispatch keeps three words per expert in LDS.
constexpr uint32_t kMaxExperts = 4096;

}  // namespace

namespace gmoe {
void set_last_error(const char* msg) { g_err = msg; }
void set_invalid_token(uint32_t token) { g_bad_token = token; }
}  // namespace gmoe

struct gmoe_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipStream_t copy_stream = nullptr;
  // Locks, taken in this order: mu serialises the entry points (an entry holds it from
  // start to end); slab_mu guards the slab, the LRU, the layers' residency and pending
  // states, the staging queue and the statistics; stage_mu guards the pinned halves and
  // the copy stream. Background staging (prefetch/mod.rs:102-127): gmoe_prefetch_step
  // queues predicted experts and `stager` stages them, taking slab_mu to reserve a region
  // and to publish the staged expert and stage_mu for the copy, never mu; an entry that
  // waits for it waits on cv, releasing slab_mu but keeping mu.
  std::mutex mu, slab_mu, stage_mu;
  std::thread stager;
  std::condition_variable cv;  // with slab_mu: queue, hold, stop and the pending states
  std::deque<std::pair<uint32_t, uint32_t>> queue;
  Keep prefetch_keep;          // the last prefetch step's used and predicted experts
  bool stop = false, hold = false;
  uint32_t staging = 0;        // experts the thread is staging now
  Slab slab;
  std::vector<std::unique_ptr<Layer>> layers;
  std::vector<std::unique_ptr<Dense>> dense;
  uint32_t* ident = nullptr;  // [kDenseTab] = 0, 1, 2, ... (device)
  LruList lru;
  gmoe_slab_stats stats{};
  uint8_t* pinned = nullptr;
  size_t pinned_bytes = 0;
  uint8_t* bounce = nullptr;  // device landing area of the pinned halves (same size)
  uint32_t* done = nullptr;   // front-end completion counter (device, zero between calls)
  hipEvent_t pin_ev[2]{};
  // scratch arena (calls on one context are ordered on one stream, so growing it waits for
  // the stream of the last call that used it)
  uint8_t* scratch = nullptr;
  size_t scratch_bytes = 0;
  hipStream_t scratch_stream = nullptr;  // the stream of the last call that used the arena
  // the device address of the allocation-free forward's static scratch (gmoe_noalloc.hip),
  // shared by every context on this device
  uint8_t* noalloc = nullptr;
  // timing
  bool timing = false;
  std::vector<Timing> pending;
  std::vector<Timing> pool;
  double t_ms[3] = {0, 0, 0};
  uint64_t t_cnt = 0;
};

// An entry point's hold on a context: mu for the call, slab_mu (releasable by a wait).
struct CtxLock {
  std::lock_guard<std::mutex> call;
  std::unique_lock<std::mutex> slab;
  explicit CtxLock(gmoe_ctx* c) : call(c->mu), slab(c->slab_mu) {}
};

namespace gmoe {
// for the other host modules (gmoe_kv.cpp)
int ctx_device(gmoe_ctx* c) { return c->device; }
hipStream_t ctx_stream(gmoe_ctx* c) { return c->stream; }
// the scratch arena's current allocation (launches captured into a graph point into it)
const void* ctx_scratch_id(gmoe_ctx* c) {
  std::lock_guard<std::mutex> g(c->slab_mu);
  return c->scratch;
}
// A graph launched on st uses the scratch arena and the given layers' experts: growing the
// arena or evicting one of those experts waits for st, as after the calls themselves.
void ctx_note_graph(gmoe_ctx* c, const uint32_t* layers, uint32_t n, hipStream_t st) {
  CtxLock g(c);
  c->scratch_stream = st;
  for (uint32_t i = 0; i < n; i++)
    if (layers[i] < c->layers.size() && c->layers[layers[i]] && c->layers[layers[i]]->alive)
      c->layers[layers[i]]->last_stream = st;
}
// A model step reads every expert of its layers from the device pointer tables (a graph
// replay, or the speculative front end): check that all are resident and keep them so,
// in one hold of the slab lock, until ctx_unpin_layers. Neither the staging thread nor
// another call can evict them meanwhile (reserve() passes them over, evict refuses).
gmoe_status ctx_pin_layers(gmoe_ctx* c, const uint32_t* layers, uint32_t n) {
  CtxLock g(c);
  for (uint32_t i = 0; i < n; i++) {
    const uint32_t l = layers[i];
    if (l >= c->layers.size() || !c->layers[l] || !c->layers[l]->alive)
      return fail(GMOE_ERR_INFERENCE, "MoE layer %u was released", l);
    const Layer& L = *c->layers[l];
    for (uint32_t e = 0; e < L.ne; e++)
      if (L.slot[e] < 0 || L.pending[e] == kStaging)
        return fail(GMOE_ERR_CACHE, "expert %u of layer %u is not resident", e, l);
  }
  for (uint32_t i = 0; i < n; i++) c->layers[layers[i]]->pins++;
  return GMOE_OK;
}
void ctx_unpin_layers(gmoe_ctx* c, const uint32_t* layers, uint32_t n) {
  CtxLock g(c);
  for (uint32_t i = 0; i < n; i++)
    if (layers[i] < c->layers.size() && c->layers[layers[i]] && c->layers[layers[i]]->pins)
      c->layers[layers[i]]->pins--;
  c->cv.notify_all();
}
}  // namespace gmoe

namespace {

// memcpy by up to kCopyThreads threads in 64 KiB-aligned slices: one thread reading a
// memory-mapped file into pinned memory is bound by its own page walks and copies, well
// below the host link's rate.
constexpr unsigned kCopyThreads = 8;
void par_copy(uint8_t* dst, const uint8_t* src, size_t n) {
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const unsigned t = (unsigned)std::min<size_t>({(size_t)kCopyThreads, (size_t)hw, n / (1u << 20) + 1});
  if (t <= 1) {
    memcpy(dst, src, n);
    return;
  }
  const size_t slice = (n / t + 65535) & ~(size_t)65535;
  std::vector<std::thread> pool;
  pool.reserve(t - 1);
  for (unsigned i = 1; i < t; i++) {
    const size_t a = std::min(n, i * slice), b = std::min(n, a + slice);
    if (a < b) pool.emplace_back([=] { memcpy(dst + a, src + a, b - a); });
  }
  memcpy(dst, src, std::min(n, slice));
  for (auto& th : pool) th.join();
}

// ---- staging: host packed rows -> pinned half -> device bounce half -> tiled slab ----
// Whole 64-row tiles move per pass; the copy and the tiling kernel of a pass run on the
// copy stream, and the half's event tells when both have finished with it.
gmoe_status stage_proj(gmoe_ctx* c, const Proj& P, const uint8_t* src, uint8_t* dst) {
  const size_t chunk = c->pinned_bytes / 2;
  const size_t tile_raw = (size_t)kTileRows * P.row_bytes;
  if (tile_raw > chunk)
    return fail(GMOE_ERR_CONFIG, "rows of %llu bytes exceed the staging buffer", (unsigned long long)P.row_bytes);
  const uint32_t rows_per = (uint32_t)(chunk / tile_raw) * kTileRows;
  int buf = 0;
  for (uint32_t r0 = 0; r0 < P.rows; r0 += rows_per, buf ^= 1) {
    const uint32_t nr = std::min(rows_per, P.rows - r0);
    const size_t nbytes = (size_t)nr * P.row_bytes;
    HIP_TRY(hipEventSynchronize(c->pin_ev[buf]));
    uint8_t* pin = c->pinned + buf * chunk;
    uint8_t* land = c->bounce + buf * chunk;
    par_copy(pin, src + (size_t)r0 * P.row_bytes, nbytes);
    HIP_TRY(hipMemcpyAsync(land, pin, nbytes, hipMemcpyHostToDevice, c->copy_stream));
    HIP_TRY(launch_tile_rows(P.qtype, land, r0, nr, P.rows, P.cols, dst, c->copy_stream));
    HIP_TRY(hipEventRecord(c->pin_ev[buf], c->copy_stream));
  }
  return GMOE_OK;
}

// Stage expert e's three matrices into the slab region at `off` and wait for the copies.
// Runs under stage_mu; reads only what registration fixed.
gmoe_status stage_expert(gmoe_ctx* c, const Layer& L, uint32_t e, uint64_t off, uint8_t* ptrs[3]) {
  uint8_t* base = c->slab.base + off;
  const void* src[3] = {nullptr, nullptr, nullptr};
  if (L.fetch) {  // MemoryManager::load_uncached (memory/mod.rs:114-146) behind the callback
    if (gmoe_status s = L.fetch(L.fetch_user, e, src)) return s;
    for (int p = 0; p < 3; p++)
      if (!src[p]) return fail(GMOE_ERR_MODEL, "expert %u: the tier returned no weights for tensor %d", e, p);
  } else {
    for (int p = 0; p < 3; p++) src[p] = L.p[p].host[e];
  }
  uint64_t o = 0;
  for (int p = 0; p < 3; p++) {
    if (gmoe_status s = stage_proj(c, L.p[p], static_cast<const uint8_t*>(src[p]), base + o)) return s;
    ptrs[p] = base + o;
    o += (L.p[p].bytes_dev + 255) & ~uint64_t(255);
  }
  HIP_TRY(hipStreamSynchronize(c->copy_stream));
  return GMOE_OK;
}

// Mark resident expert e of layer l most recently used (ExpertCache::get, cache/mod.rs:70-84).
void touch(gmoe_ctx* c, uint32_t l, uint32_t e) {
  Layer& L = *c->layers[l];
  if (L.slot[e] < 0) return;
  c->lru.splice(c->lru.end(), c->lru, L.lru_pos[e]);
}

// Wait until queued work on `st` has finished: the context's own streams directly; a
// caller's stream (which the caller may have destroyed since) through the whole device.
gmoe_status drain(gmoe_ctx* c, hipStream_t st) {
  if (!st) return GMOE_OK;
  if (st == c->stream || st == c->copy_stream) HIP_TRY(hipStreamSynchronize(st));
  else HIP_TRY(hipDeviceSynchronize());
  return GMOE_OK;
}

gmoe_status evict(gmoe_ctx* c, uint32_t l, uint32_t e) {
  Layer& L = *c->layers[l];
  if (L.slot[e] < 0) return GMOE_OK;
  // the slab region may still be read by the layer's queued calls
  if (gmoe_status s = drain(c, L.last_stream)) return s;
  L.last_stream = nullptr;
  c->slab.release((uint64_t)L.slot[e], L.expert_bytes);
  L.slot[e] = -1;
  for (int p = 0; p < 3; p++) L.eptr_host[p * L.ne + e] = nullptr;
  HIP_TRY(hipMemcpy(L.eptr, L.eptr_host.data(), L.eptr_host.size() * sizeof(void*), hipMemcpyHostToDevice));
  c->lru.erase(L.lru_pos[e]);
  c->stats.entries--;
  c->stats.bytes -= L.expert_bytes;
  return GMOE_OK;
}

// A slab region for one expert of layer l, evicting the least recently used experts not in
// `keep` (evict_ok false: free space only). The caller holds slab_mu.
gmoe_status reserve(gmoe_ctx* c, uint32_t l, bool evict_ok, const Keep* keep, uint64_t* off) {
  Layer& L = *c->layers[l];
  while (!c->slab.alloc(L.expert_bytes, off)) {
    if (!evict_ok) return fail(GMOE_ERR_CACHE, "HBM slab is full");
    auto victim = c->lru.end();
    for (auto it = c->lru.begin(); it != c->lru.end(); ++it) {
      bool kept = c->layers[it->first]->pins > 0;  // read by a model step in flight
      if (keep)
        for (auto& kp : *keep) kept |= (kp == *it);
      if (!kept) {
        victim = it;
        break;
      }
    }
    if (victim == c->lru.end())
      return fail(GMOE_ERR_CACHE, "HBM slab of %llu bytes cannot hold the experts this call needs",
                  (unsigned long long)c->slab.cap);
    auto v = *victim;
    if (gmoe_status s = evict(c, v.first, v.second)) return s;
    c->stats.evictions++;
  }
  return GMOE_OK;
}

// Publish expert e, staged at `off`, as resident (most recently used). The caller holds slab_mu.
gmoe_status publish(gmoe_ctx* c, uint32_t l, uint32_t e, uint64_t off, uint8_t* const ptrs[3]) {
  Layer& L = *c->layers[l];
  for (int p = 0; p < 3; p++) L.eptr_host[p * L.ne + e] = ptrs[p];
  HIP_TRY(hipMemcpy(L.eptr, L.eptr_host.data(), L.eptr_host.size() * sizeof(void*), hipMemcpyHostToDevice));
  L.slot[e] = (int64_t)off;
  L.lru_pos[e] = c->lru.emplace(c->lru.end(), l, e);
  c->stats.entries++;
  c->stats.bytes += L.expert_bytes;
  for (int p = 0; p < 3; p++) c->stats.h2d_bytes += (uint64_t)L.p[p].rows * L.p[p].row_bytes;
  return GMOE_OK;
}

// Make expert e of layer l resident, with slab_mu held through `lk`. `keep` marks experts of the
// current call that must not be evicted to make room; evict_ok = false only fills free
// space. An expert the staging thread has queued is taken off its queue and staged here;
// one it is staging now is waited for (the wait releases slab_mu).
gmoe_status make_resident(gmoe_ctx* c, std::unique_lock<std::mutex>& lk, uint32_t l, uint32_t e, bool evict_ok,
                          const Keep* keep) {
  Layer& L = *c->layers[l];
  c->cv.wait(lk, [&] { return L.pending[e] != kStaging; });
  if (L.slot[e] >= 0) {
    touch(c, l, e);
    return GMOE_OK;
  }
  if (L.pending[e] == kQueued) {
    c->queue.erase(std::remove(c->queue.begin(), c->queue.end(), std::make_pair(l, e)), c->queue.end());
    L.pending[e] = kAbsent;
    c->cv.notify_all();
  }
  uint64_t off;
  if (gmoe_status s = reserve(c, l, evict_ok, keep, &off)) return s;
  uint8_t* ptrs[3];
  gmoe_status s;
  {
    std::lock_guard<std::mutex> sg(c->stage_mu);
    s = stage_expert(c, L, e, off, ptrs);
  }
  if (s) {
    c->slab.release(off, L.expert_bytes);
    return s;
  }
  return publish(c, l, e, off, ptrs);
}

// The staging thread: stages queued experts one after another, unless held or stopped.
void stager_main(gmoe_ctx* c) {
  hipSetDevice(c->device);
  std::unique_lock<std::mutex> lk(c->slab_mu);
  for (;;) {
    c->cv.wait(lk, [&] { return c->stop || (!c->hold && !c->queue.empty()); });
    if (c->stop) break;
    const auto [l, e] = c->queue.front();
    c->queue.pop_front();
    Layer& L = *c->layers[l];
    if (!L.alive || L.slot[e] >= 0 || L.pending[e] != kQueued) continue;
    uint64_t off;
    if (reserve(c, l, true, &c->prefetch_keep, &off) != GMOE_OK) {  // no room: dropped, as a failed warm is
      L.pending[e] = kAbsent;
      c->cv.notify_all();
      continue;
    }
    L.pending[e] = kStaging;
    c->staging++;
    lk.unlock();
    uint8_t* ptrs[3];
    gmoe_status s;
    {
      std::lock_guard<std::mutex> sg(c->stage_mu);
      s = stage_expert(c, L, e, off, ptrs);
    }
    lk.lock();
    if (s == GMOE_OK) s = publish(c, l, e, off, ptrs);
    if (s != GMOE_OK) c->slab.release(off, L.expert_bytes);  // the forward stages it itself when routed
    L.pending[e] = kAbsent;
    c->staging--;
    c->cv.notify_all();
  }
}

// ---- scratch arena ----
struct ScratchPlan {
  size_t total = 0;
  size_t add(size_t bytes) {
    size_t o = total;
    total += (bytes + 255) & ~size_t(255);
    return o;
  }
};

struct Carved {
  FwdBufs B;
  float* d_hs;
  float* d_out;
  float* d_logits_in;
};

// Slot rows a call of n tokens may need: n*k routed pairs, or n*ne when the speculative
// front end may dispatch candidate pairs.
uint32_t slot_capacity(const Layer& L, uint32_t n) {
  const uint64_t spec = (uint64_t)n * L.ne;
  return spec <= kSpecMaxSlots ? (uint32_t)std::max<uint64_t>(spec, (uint64_t)n * L.k) : n * L.k;
}

LayerDev layer_dev(const Layer& L);
bool uses_int8(uint32_t math, uint32_t qt);

// The scratch of one launch sequence of n tokens: plan (base null) or carve. Buffers a
// call of this size does not use take no room: h is int8 (packed math into an int8
// down product) or f32, and only MFMA-prefill calls have token tiles and fp16 planes.
size_t plan_scratch(const Layer& L, uint32_t n, Carved* cv, uint8_t* base) {
  ScratchPlan P;
  const uint64_t nk = (uint64_t)n * L.k, ns = slot_capacity(L, n);
  const LayerDev D = layer_dev(L);
  const bool h8 = uses_int8(L.math, L.p[2].qtype), pf = prefill_ok(D, n), pq = !pf && prefill_packed_ok(D, n);
  // prefill: hi and lo planes of the activations (f32 math) or one plane of their codes
  // and the transposed per-token scales and sums (packed math, nkp slots a row), hi and
  // lo planes of h (both)
  const uint64_t nk_pf = (pf || pq) ? 2 * nk : 0, ns8 = h8 ? ns : 0, ns32 = h8 ? 0 : ns;
  const uint64_t nkp = pq ? nk + 64 : 0;
  size_t o_hs = P.add((size_t)n * L.d * 4), o_out = P.add((size_t)n * L.d * 4);
  size_t o_lin = P.add((size_t)n * L.ne * 4);
  size_t o_ids = P.add(nk * 4), o_w = P.add(nk * 4), o_lg = P.add((size_t)n * L.ne * 4);
  size_t o_xq = P.add((size_t)n * L.d), o_xs = P.add((size_t)n * (L.d / 32) * 4);
  size_t o_x16 = P.add((size_t)n * (L.d / 16) * 4);  // sums: at most one word per 16 values
  size_t o_off = P.add((L.ne + 1) * 4), o_act = P.add((L.ne + 1) * 4);
  size_t o_st = P.add(ns * 4), o_sw = P.add(ns * 4), o_sr = P.add(ns * 4), o_so = P.add(nk * 4);
  size_t o_hq = P.add(ns8 * L.f), o_hsc = P.add(ns8 * (L.f / 32) * 4), o_h16 = P.add(ns8 * (L.f / 16) * 4);
  size_t o_hf = P.add(ns32 * L.f * 4), o_y = P.add(kMaxKsg * ns * L.d * 4);
  size_t o_cand = P.add((size_t)n * L.ne * 4);
  size_t o_work = P.add((size_t)L.ne * sizeof(ExpertWork));
  const uint32_t pcap = (pf || pq) ? prefill_tiles_cap(n, L.k, L.ne) : 0;
  size_t o_pt = P.add((size_t)pcap * 4), o_xh = P.add(nk_pf * L.d * 2), o_hh = P.add(nk_pf * L.f * 2);
  const uint64_t nk_sh = (pf || pq) ? 2 * nk : 0;
  size_t o_xsh = P.add(nk_sh * (L.d / 16) * 2), o_hsh = P.add(nk_sh * (L.f / 16) * 2);
  size_t o_qxs = P.add(nkp * (L.d / 32) * 4), o_qxm = P.add(nkp * (L.d / 16) * 4);
  if (cv && base) {
    FwdBufs& B = cv->B;
    memset(&B, 0, sizeof B);
    cv->d_hs = (float*)(base + o_hs);
    cv->d_out = (float*)(base + o_out);
    cv->d_logits_in = (float*)(base + o_lin);
    B.ids = (uint32_t*)(base + o_ids);
    B.w = (float*)(base + o_w);
    B.logits = (float*)(base + o_lg);
    B.xq = (int8_t*)(base + o_xq);
    B.xs = (float*)(base + o_xs);
    B.xsum = (uint32_t*)(base + o_x16);
    B.offsets = (uint32_t*)(base + o_off);
    B.active = (uint32_t*)(base + o_act);
    B.slot_tok = (uint32_t*)(base + o_st);
    B.slot_w = (float*)(base + o_sw);
    B.slot_rank = (uint32_t*)(base + o_sr);
    B.slot_of = (uint32_t*)(base + o_so);
    B.hq = (int8_t*)(base + o_hq);
    B.hsc = (float*)(base + o_hsc);
    B.hsum = (uint32_t*)(base + o_h16);
    B.hf = (float*)(base + o_hf);
    B.y = (float*)(base + o_y);
    B.work = (ExpertWork*)(base + o_work);
    B.nslot = (uint32_t)ns;
    B.cand = (uint32_t*)(base + o_cand);
    B.ptile = (uint32_t*)(base + o_pt);
    B.ptile_cap = pcap;
    B.xh = (_Float16*)(base + o_xh);
    B.hh = (_Float16*)(base + o_hh);
    B.xsh = (_Float16*)(base + o_xsh);
    B.hsh = (_Float16*)(base + o_hsh);
    B.qxs = (float*)(base + o_qxs);
    B.qxsum = (float*)(base + o_qxm);
    B.nkp = (uint32_t)nkp;
  }
  return P.total;
}

gmoe_status ensure_scratch(gmoe_ctx* c, size_t bytes) {
  if (bytes <= c->scratch_bytes) return GMOE_OK;
  if (gmoe_status s = drain(c, c->scratch_stream)) return s;  // the last call that used the old arena
  c->scratch_stream = nullptr;
  if (c->scratch) HIP_TRY(hipFree(c->scratch));
  c->scratch = nullptr;
  c->scratch_bytes = 0;
  size_t want = std::max(bytes, (size_t)64 << 20);
  HIP_TRY(hipMalloc(&c->scratch, want));
  c->scratch_bytes = want;
  return GMOE_OK;
}

LayerDev layer_dev(const Layer& L) {
  LayerDev D;
  D.d = L.d; D.f = L.f; D.ne = L.ne; D.k = L.k;
  D.gating = L.gating; D.combine = L.combine; D.math = L.math;
  D.qt_gate = L.p[0].qtype; D.qt_up = L.p[1].qtype; D.qt_down = L.p[2].qtype;
  D.router = L.router;
  D.eptr = L.eptr;
  return D;
}

bool uses_int8(uint32_t math, uint32_t qt) { return math == GMOE_MATH_PACKED && has_int8_kernel(qt); }

Timing take_timing(gmoe_ctx* c) {
  if (!c->pool.empty()) {
    Timing t = c->pool.back();
    c->pool.pop_back();
    return t;
  }
  Timing t;
  hipEventCreate(&t.a);
  hipEventCreate(&t.b);
  hipEventCreate(&t.c);
  return t;
}

// The launch sequence of one call. B's activation/output pointers are set by the caller.
// timed = false never records kernel-timing events (creating one may allocate).
gmoe_status run_layer(gmoe_ctx* c, Layer& L, FwdBufs B, uint32_t n, hipStream_t st, bool timed = true) {
  LayerDev D = layer_dev(L);
  B.done = c->done;
  // int8 h only when the down product reads it; f32 h otherwise
  if (!uses_int8(L.math, L.p[2].qtype)) {
    B.hq = nullptr;
    B.hsc = nullptr;
    B.hsum = nullptr;
  } else {
    B.hf = nullptr;
  }
  const bool quant = uses_int8(L.math, L.p[0].qtype);
  // prefill-sized calls run the expert products on MFMA over token tiles: f32 math
  // (k_pf) or packed math (k_pq)
  const bool pf = prefill_ok(D, n), pq = !pf && prefill_packed_ok(D, n);
  if (!pf && !pq) {
    B.ptile = nullptr;
    B.xh = B.xsh = B.hh = B.hsh = nullptr;
  }
  if (!pq) B.qxs = B.qxsum = nullptr;
  // decode calls that compute their router logits: the expert products start on the
  // candidate experts, and the exact routing rides along in the gate/up launch. Any
  // expert may be a candidate, so every one must be resident.
  bool resident = true;
  for (uint32_t e = 0; e < L.ne; e++) resident &= L.slot[e] >= 0;
  const bool spec = !pf && !pq && !B.logits_in && resident && spec_ok(D, n);
  B.spec = spec ? 1u : 0u;
  if (B.nx && !spec) {  // hs made by its own launch, as the speculative front end would
    HIP_TRY(launch_add_norm_slices(B.nx, B.ny, B.nsl_y, B.nw, n, L.d, B.neps, B.nh, st));
    B.nx = nullptr;
  }
  // top-k <= 2 at decode batches: the down product adds into the output (zeroed by the
  // front end), no combine launch
  // (the front end zeroes out while it reads hs: not when they overlap, as in place)
  const uintptr_t ob = (uintptr_t)B.out, oe = ob + (size_t)n * L.d * 4, hb = (uintptr_t)B.hs,
                  he = hb + (size_t)n * L.d * 4;
  const bool fuse = !pf && !pq && down_atomic_ok(D, n) && (spec || front_small_ok(D, n)) && (oe <= hb || he <= ob);
  B.fuse_out = fuse ? 1u : 0u;
  if (!spec) B.nslot = n * L.k;
  RouteArgs ra{};
  if (spec) {
    ra.router = D.router;
    ra.hs = B.hs;
    ra.logits = B.logits;
    ra.ids = B.ids;
    ra.w = B.w;
    ra.n = n;
    ra.ne = D.ne;
    ra.k = D.k;
    ra.d = D.d;
    ra.gating = D.gating;
    ra.sec = std::min(D.d, kRouteSection);
    ra.tok_done = c->done + 64;
    ra.offsets = B.offsets;
    ra.slot_tok = B.slot_tok;
    ra.comb_slot = B.slot_of;  // unused by the speculative dispatch: the combine's slots
    ra.comb_w = B.slot_w;      // (n*k <= the n*ne candidate slots)
    ra.combine = D.combine;
    // a single-token call whose gate/up can route for itself folds the front end into
    // that launch; otherwise the front end runs first and dispatches
    ra.self = n == 1 && !B.nx && B.hq && gateup_self_ok(D, n) ? 1u : 0u;
    if (!ra.self) HIP_TRY(launch_spec_front(D, B, n, quant ? 1 : 0, st));
  } else if (front_small_ok(D, n)) {
    const bool split = n >= kFrontSplitTokens;
    HIP_TRY(launch_front_small(D, B, n, quant ? 1 : 0, !split, st));
    if (split) HIP_TRY(launch_dispatch_par(D, B, n, st));
  } else if (front_wide_ok(D, n)) {
    HIP_TRY(launch_front_wide(D, B, n, quant ? 1 : 0, st));
  } else {
    HIP_TRY(launch_route(D, B, n, st));
    HIP_TRY(launch_dispatch(D, B, n, st));
    if (quant) HIP_TRY(launch_quant_act(B.hs, n, L.d, B.xq, B.xs, B.xsum, L.p[0].qtype, st));
  }
  if (pf) HIP_TRY(launch_gather_f16(D, B, n, st));
  if (pq) HIP_TRY(launch_gather_codes(D, B, n, st));
  const uint32_t ksg = (pf || pq) ? prefill_ksg(D, B) : down_ksg(D, n * L.k);
  Timing tm{};
  timed = timed && c->timing;
  if (timed) {  // no timing events inside a graph being captured
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) timed = false;
  }
  if (timed) {
    tm = take_timing(c);
    HIP_TRY(hipEventRecord(tm.a, st));
  }
  HIP_TRY(pf ? launch_prefill_gateup(D, B, n, st) : pq ? launch_pq_gateup(D, B, n, st) : launch_gateup(D, B, n, ra, st));
  if (timed) HIP_TRY(hipEventRecord(tm.b, st));
  // packed prefill: the down product's input is the dequantised h (scale * q), whose
  // products k_pf makes exact; the down output is not requantised, so its summation order
  // is free (outputs within rtol 1e-3 / atol 1e-4)
  HIP_TRY((pf || pq) ? launch_prefill_down(D, B, n, ksg, st)
                     : fuse ? launch_down_atomic(D, B, n, st) : launch_down(D, B, n, st));
  if (timed) {
    HIP_TRY(hipEventRecord(tm.c, st));
    c->pending.push_back(tm);
  }
  if (!fuse) HIP_TRY(launch_combine(D, B, n, ksg, st));
  L.last_stream = st;
  return GMOE_OK;
}

// Tokens per layer launch sequence: the kernels index (token, expert) pairs in a grid
// dimension of at most 65535, so a longer batch runs as consecutive sequences. Each
// token's output depends on its own row only, so the split changes no result's meaning.
uint32_t call_tokens(const Layer& L) { return std::min<uint32_t>(4096u, 65535u / L.k); }

// The most scratch any launch sequence of an n-token call needs: the sequences are
// call_tokens long but the last, and the need is not monotonic in the length (the
// speculative front end's candidate slots stop at kSpecMaxSlots; MFMA prefill adds planes).
size_t call_scratch(const Layer& L, uint32_t n) {
  const uint32_t per = call_tokens(L), last = n % per;
  size_t need = plan_scratch(L, std::min(n, per), nullptr, nullptr);
  if (n > per && last) need = std::max(need, plan_scratch(L, last, nullptr, nullptr));
  return need;
}

gmoe_status check_ctx(gmoe_ctx* c) {
  if (!c) return fail(GMOE_ERR_INFERENCE, "null context");
  return GMOE_OK;
}

// ---- dense projections: Weight::matmul_rows(0, xs, n, out) (llama/mod.rs:160-195) ----
// The weight is the one "expert" of a down product: decode-sized calls quantise the
// activations per 32 (packed math) or read them as f32 and run the K-split down kernel;
// prefill-sized f32-math calls run it on MFMA over token tiles; the K slices are then
// added in order into out [n][rows].
LayerDev dense_dev(const Dense& W) {
  LayerDev D{};
  D.d = W.rows;
  D.f = W.cols;
  D.ne = 1;
  D.k = 1;
  D.math = W.math;
  D.qt_gate = D.qt_up = D.qt_down = W.qtype;
  return D;
}

struct DenseCarve {
  FwdBufs B;
  uint32_t ksg;
  bool pf, int8;
};

constexpr uint32_t kDenseFuseKsg = 4;

// Scratch of one dense call: plan (base null) or carve.
size_t plan_dense(const gmoe_ctx* c, const Dense& W, uint32_t n, uint8_t* base, DenseCarve* out) {
  const LayerDev D = dense_dev(W);
  const bool pf = prefill_dense_ok(D, n);
  const bool int8 = !pf && uses_int8(W.math, W.qtype);
  FwdBufs B{};
  B.nslot = n;
  B.ptile_cap = pf ? (n + kPfTok - 1) / kPfTok : 0;
  const uint32_t ksg = pf ? 0u : dense_ksg(D);  // prefill: from the carved buffers below
  ScratchPlan P;
  const size_t nx = (size_t)n * W.cols;
  size_t o_work = P.add(sizeof(ExpertWork)), o_off = P.add(8), o_act = P.add(8), o_tok = P.add((size_t)n * 4),
         o_pt = P.add((size_t)B.ptile_cap * 4 + 4);
  // packed math: with at least kDenseFuseKsg K slices each down workgroup stages a short
  // K range, and quantises its activations itself; with fewer, a quantiser launch first
  // (staging the f32 rows cost the 32000-row output head 2.3 us, saved q/k/v/o 11 us)
  const bool fuse = int8 && ksg >= kDenseFuseKsg;
  size_t o_q = 0, o_s = 0, o_16 = 0, o_xh = 0, o_xsh = 0;
  if (int8 && !fuse) {
    o_q = P.add(nx);
    o_s = P.add(nx / 32 * 4);
    o_16 = P.add(nx / 16 * 4);
  }
  if (pf) {
    o_xh = P.add(2 * nx * 2);
    o_xsh = P.add(2 * (nx / 16) * 2);
  }
  const size_t o_y = P.add((size_t)kMaxKsg * n * W.rows * 4);
  if (base && out) {
    B.work = (ExpertWork*)(base + o_work);
    B.offsets = (uint32_t*)(base + o_off);
    B.active = (uint32_t*)(base + o_act);
    B.slot_tok = (uint32_t*)(base + o_tok);
    B.ptile = pf ? (uint32_t*)(base + o_pt) : nullptr;
    if (int8 && !fuse) {
      B.hq = (int8_t*)(base + o_q);
      B.hsc = (float*)(base + o_s);
      B.hsum = (uint32_t*)(base + o_16);
    }
    if (pf) {
      B.xh = B.hh = (_Float16*)(base + o_xh);
      B.xsh = B.hsh = (_Float16*)(base + o_xsh);
    }
    B.y = (float*)(base + o_y);
    if (n <= kDenseTab) {  // the precomputed tables: no setup launch
      B.work = W.work_tab + (n - 1);
      B.slot_tok = c->ident;
      if (pf) B.ptile = c->ident;
    }
    out->B = B;
    out->pf = pf;
    out->int8 = int8;
    out->ksg = pf ? prefill_ksg(D, B) : ksg;
  }
  return P.total;
}

// out null: the K slices are left in cv.B.y ([cv.ksg][n][rows]) for the caller to add.
gmoe_status run_dense(const Dense& W, const DenseCarve& cv, const float* x, uint32_t n, float* out, hipStream_t st) {
  const LayerDev D = dense_dev(W);
  FwdBufs B = cv.B;
  if (n > kDenseTab)
    HIP_TRY(launch_dense_setup(B.work, B.offsets, B.active, B.ptile, B.ptile_cap, B.slot_tok, W.tiled, n, st));
  if (cv.pf) {
    LayerDev Gd = D;  // the gather reads rows of the input's width
    Gd.d = W.cols;
    B.hs = x;
    HIP_TRY(launch_gather_f16(Gd, B, n, st));
    HIP_TRY(launch_prefill_down(D, B, n, cv.ksg, st));
  } else {
    if (cv.int8 && B.hq) {
      HIP_TRY(launch_quant_act(x, n, W.cols, B.hq, B.hsc, B.hsum, W.qtype, st));
    } else {  // f32 math, or packed math quantised in the down kernel's staging (hq null)
      B.hq = nullptr;
      B.hsc = nullptr;
      B.hsum = nullptr;
      B.hf = const_cast<float*>(x);
    }
    HIP_TRY(launch_down(D, B, n, st, cv.ksg));
  }
  if (out) HIP_TRY(launch_reduce_parts(B.y, cv.ksg, (size_t)n * W.rows, out, st));
  return GMOE_OK;
}

gmoe_status mark_scratch(gmoe_ctx* c, hipStream_t st) {
  c->scratch_stream = st;
  return GMOE_OK;
}

gmoe_status get_dense(gmoe_ctx* c, uint32_t id, Dense** out) {
  if (id >= c->dense.size() || !c->dense[id] || !c->dense[id]->alive)
    return fail(GMOE_ERR_INFERENCE, "unknown dense weight id %u", id);
  *out = c->dense[id].get();
  return GMOE_OK;
}

// A dense call without its slice sum: *parts holds [*nsl][n][rows] K slices in the
// context's scratch (or in y_out, kMaxKsg * n * rows floats), which the caller's next
// launch on st adds in slice order (the sum k_reduce_parts makes), before any other call
// on the context reuses the scratch.
gmoe_status dense_slices(gmoe_ctx* c, uint32_t id, const float* d_xs, uint32_t n, hipStream_t st, const float** parts,
                         uint32_t* nsl, float* y_out) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!d_xs || !parts || !nsl) return fail(GMOE_ERR_INFERENCE, "null activation or output pointer");
  if (n == 0) return fail(GMOE_ERR_INFERENCE, "empty batch");
  CtxLock g(c);
  Dense* W;
  if (gmoe_status s = get_dense(c, id, &W)) return s;
  HIP_TRY(hipSetDevice(c->device));
  if (gmoe_status s = ensure_scratch(c, plan_dense(c, *W, n, nullptr, nullptr))) return s;
  DenseCarve cv;
  plan_dense(c, *W, n, c->scratch, &cv);
  if (y_out) cv.B.y = y_out;  // [kMaxKsg][n][rows] floats of the caller's
  if (gmoe_status s = run_dense(*W, cv, d_xs, n, nullptr, st)) return s;
  *parts = cv.B.y;
  *nsl = cv.ksg;
  return mark_scratch(c, st);
}

gmoe_status get_layer(gmoe_ctx* c, uint32_t id, Layer** out) {
  if (id >= c->layers.size() || !c->layers[id] || !c->layers[id]->alive)
    return fail(GMOE_ERR_INFERENCE, "unknown layer id %u", id);
  *out = c->layers[id].get();
  return GMOE_OK;
}

// One launch sequence of at most call_tokens(L) tokens, host pointers (the context held
// through `lk`, its slab lock).
gmoe_status forward_chunk(gmoe_ctx* c, std::unique_lock<std::mutex>& lk, uint32_t lid, Layer* L, const float* hs,
                          const float* logits, uint32_t n, float* out, uint32_t* ids, float* w) {
  Carved cv;
  size_t need = plan_scratch(*L, n, nullptr, nullptr);
  if (gmoe_status s = ensure_scratch(c, need)) return s;
  plan_scratch(*L, n, &cv, c->scratch);
  hipStream_t st = c->stream;
  HIP_TRY(hipMemcpyAsync(cv.d_hs, hs, (size_t)n * L->d * 4, hipMemcpyHostToDevice, st));
  FwdBufs B = cv.B;
  B.hs = cv.d_hs;
  B.out = cv.d_out;
  B.logits_in = nullptr;
  if (logits) {
    HIP_TRY(hipMemcpyAsync(cv.d_logits_in, logits, (size_t)n * L->ne * 4, hipMemcpyHostToDevice, st));
    B.logits_in = cv.d_logits_in;
  }
  // residency: route first if anything is missing, then stage exactly what is routed
  bool all = true;
  for (uint32_t e = 0; e < L->ne; e++) all &= L->slot[e] >= 0;
  std::vector<uint32_t> hid((size_t)n * L->k);
  if (!all) {
    LayerDev D = layer_dev(*L);
    HIP_TRY(launch_route(D, B, n, st));
    HIP_TRY(hipMemcpyAsync(hid.data(), B.ids, hid.size() * 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    std::vector<std::pair<uint32_t, uint32_t>> keep;
    for (uint32_t v : hid) {
      auto kp = std::make_pair(lid, v);
      if (std::find(keep.begin(), keep.end(), kp) == keep.end()) keep.push_back(kp);
    }
    // first wait for any of them the staging thread is copying now, then make them all
    // resident without releasing the lock, so that none is evicted before the launch
    c->cv.wait(lk, [&] {
      for (auto& kp : keep)
        if (L->pending[kp.second] == kStaging) return false;
      return true;
    });
    for (auto& kp : keep) {
      if (L->slot[kp.second] >= 0) c->stats.hits++;
      else c->stats.misses++;
      if (gmoe_status s = make_resident(c, lk, lid, kp.second, true, &keep)) return s;
    }
    // Only the routed experts are resident now: the layer runs from these exact logits.
    // The speculative front end would also compute products for candidate experts near
    // the top-k cut, which need not be resident.
    if (!B.logits_in) {
      HIP_TRY(hipMemcpyAsync(cv.d_logits_in, B.logits, (size_t)n * L->ne * 4, hipMemcpyDeviceToDevice, st));
      B.logits_in = cv.d_logits_in;
    }
  }
  if (gmoe_status s = run_layer(c, *L, B, n, st)) return s;
  c->scratch_stream = st;
  HIP_TRY(hipMemcpyAsync(out, B.out, (size_t)n * L->d * 4, hipMemcpyDeviceToHost, st));
  if (all) HIP_TRY(hipMemcpyAsync(hid.data(), B.ids, hid.size() * 4, hipMemcpyDeviceToHost, st));
  if (ids) HIP_TRY(hipMemcpyAsync(ids, B.ids, (size_t)n * L->k * 4, hipMemcpyDeviceToHost, st));
  if (w) HIP_TRY(hipMemcpyAsync(w, B.w, (size_t)n * L->k * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (all) {  // every routed expert was resident: one hit per distinct expert, as above
    std::vector<uint32_t> u(hid);
    std::sort(u.begin(), u.end());
    c->stats.hits += (uint64_t)(std::unique(u.begin(), u.end()) - u.begin());
  }
  // the LRU sees each routed expert as fetched in token order, then rank order, as the
  // engine's loader fetches them (moe/mod.rs:98-112 -> ExpertCache::get); experts that
  // were not routed keep their place
  for (uint32_t e : hid) touch(c, lid, e);
  return GMOE_OK;
}

gmoe_status forward_host(gmoe_ctx* c, uint32_t lid, const float* hs, const float* logits, uint32_t n,
                         float* out, uint32_t* ids, float* w) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!hs || !out) return fail(GMOE_ERR_INFERENCE, "null activation pointer");
  if (n == 0) return fail(GMOE_ERR_INFERENCE, "empty batch");
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, lid, &L)) return s;
  HIP_TRY(hipSetDevice(c->device));
  const uint32_t per = call_tokens(*L);
  for (uint32_t t0 = 0; t0 < n; t0 += per) {
    const uint32_t m = std::min(per, n - t0);
    const size_t k = L->k;
    if (gmoe_status s = forward_chunk(c, g.slab, lid, L, hs + (size_t)t0 * L->d,
                                      logits ? logits + (size_t)t0 * L->ne : nullptr,
                                      m, out + (size_t)t0 * L->d, ids ? ids + t0 * k : nullptr, w ? w + t0 * k : nullptr))
      return s;
  }
  return GMOE_OK;
}

// The work records of every token count up to kDenseTab (and the context's identity
// table) for W->tiled; frees W->tiled on failure.
gmoe_status dense_tables(gmoe_ctx* c, Dense* W) {
  std::vector<ExpertWork> tab(kDenseTab);
  for (uint32_t i = 0; i < kDenseTab; i++) tab[i] = ExpertWork{{W->tiled, W->tiled, W->tiled}, 0, 0, i + 1, 0};
  hipError_t e = hipMalloc(&W->work_tab, tab.size() * sizeof(ExpertWork));
  if (e == hipSuccess) e = hipMemcpy(W->work_tab, tab.data(), tab.size() * sizeof(ExpertWork), hipMemcpyHostToDevice);
  if (e == hipSuccess && !c->ident) {
    std::vector<uint32_t> id(kDenseTab);
    for (uint32_t i = 0; i < kDenseTab; i++) id[i] = i;
    e = hipMalloc(&c->ident, kDenseTab * 4);
    if (e == hipSuccess) e = hipMemcpy(c->ident, id.data(), kDenseTab * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess && c->ident) {
      hipFree(c->ident);
      c->ident = nullptr;
    }
  }
  if (e != hipSuccess) {
    hipFree(W->tiled);
    W->tiled = nullptr;
    if (W->work_tab) hipFree(W->work_tab);
    W->work_tab = nullptr;
    return fail(GMOE_ERR_DEVICE, "dense weight tables: %s", hipGetErrorString(e));
  }
  return GMOE_OK;
}

}  // namespace

namespace gmoe {

// The dense call without its slice sum, for the model step (dense_slices).
gmoe_status dense_forward_slices(gmoe_ctx* c, uint32_t id, const float* d_xs, uint32_t n, hipStream_t st,
                                 const float** parts, uint32_t* nsl, float* y_out) {
  return dense_slices(c, id, d_xs, n, st, parts, nsl, y_out);
}

// The MoE feed-forward of a model step with its input made by its own front end: hs =
// RMSNorm(x + the sum of y's nsl K slices) * w, written to h (and x updated), as
// k_add_norm<true> makes it; calls that take another front end run that launch first.
gmoe_status ffn_forward_normed(gmoe_ctx* c, uint32_t lid, float* d_x, const float* d_y, uint32_t nsl,
                               uint64_t y_stride, const float* d_w, float eps, float* d_h, uint32_t n, float* d_out,
                               hipStream_t st) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!d_x || !d_y || !d_w || !d_h || !d_out) return fail(GMOE_ERR_INFERENCE, "null activation pointer");
  if (n == 0) return fail(GMOE_ERR_INFERENCE, "empty batch");
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, lid, &L)) return s;
  for (uint32_t e = 0; e < L->ne; e++)
    if (L->slot[e] < 0) return fail(GMOE_ERR_CACHE, "expert %u of layer %u is not resident", e, lid);
  HIP_TRY(hipSetDevice(c->device));
  const uint32_t per = call_tokens(*L);
  if (gmoe_status s = ensure_scratch(c, call_scratch(*L, n))) return s;
  for (uint32_t t0 = 0; t0 < n; t0 += per) {
    const uint32_t m = std::min(per, n - t0);
    Carved cv;
    plan_scratch(*L, m, &cv, c->scratch);
    FwdBufs B = cv.B;
    B.hs = d_h + (size_t)t0 * L->d;
    B.logits_in = nullptr;
    B.out = d_out + (size_t)t0 * L->d;
    B.nx = d_x + (size_t)t0 * L->d;
    B.ny = d_y + (size_t)t0 * L->d;
    B.nw = d_w;
    B.nh = d_h + (size_t)t0 * L->d;
    B.neps = eps;
    B.nsl_y = nsl;
    B.ny_stride = y_stride;
    if (gmoe_status s = run_layer(c, *L, B, m, st)) return s;
    c->scratch_stream = st;
  }
  return GMOE_OK;
}

// One dense weight made of registered ones laid end to end: its rows are theirs in order
// (out = [W0 x; W1 x; ...]). They share type, width and math, and every one but the last
// has a whole number of 64-row tiles, so the tiled bytes simply follow one another.
gmoe_status dense_stack(gmoe_ctx* c, const uint32_t* ids, uint32_t count, uint32_t* out) {
  CtxLock g(c);
  if (count == 0) return fail(GMOE_ERR_INFERENCE, "nothing to stack");
  std::vector<Dense*> parts(count);
  for (uint32_t i = 0; i < count; i++)
    if (gmoe_status s = get_dense(c, ids[i], &parts[i])) return s;
  auto W = std::make_unique<Dense>();
  W->qtype = parts[0]->qtype;
  W->cols = parts[0]->cols;
  W->math = parts[0]->math;
  for (uint32_t i = 0; i < count; i++) {
    const Dense& P = *parts[i];
    if (P.qtype != W->qtype || P.cols != W->cols || P.math != W->math)
      return fail(GMOE_ERR_MODEL, "stacked weights differ in type, width or math");
    if (i + 1 < count && P.rows % kTileRows)
      return fail(GMOE_ERR_MODEL, "a stacked weight's rows (%u) are not whole tiles of %u", P.rows, kTileRows);
    W->rows += P.rows;
    W->tiled_bytes += P.tiled_bytes;
  }
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipMalloc(&W->tiled, W->tiled_bytes));
  hipError_t e = hipSuccess;
  uint64_t off = 0;
  for (uint32_t i = 0; i < count && e == hipSuccess; i++) {
    e = hipMemcpy(W->tiled + off, parts[i]->tiled, parts[i]->tiled_bytes, hipMemcpyDeviceToDevice);
    off += parts[i]->tiled_bytes;
  }
  if (e != hipSuccess) {
    hipFree(W->tiled);
    return fail(GMOE_ERR_DEVICE, "stacking dense weights: %s", hipGetErrorString(e));
  }
  if (gmoe_status s = dense_tables(c, W.get())) return s;
  *out = (uint32_t)c->dense.size();
  c->dense.push_back(std::move(W));
  return GMOE_OK;
}

// Shapes of registered weights, for the decode-step driver (gmoe_model.cpp).
bool dense_shape(gmoe_ctx* c, uint32_t id, uint32_t* rows, uint32_t* cols) {
  CtxLock g(c);
  Dense* W;
  if (get_dense(c, id, &W) != GMOE_OK) return false;
  *rows = W->rows;
  *cols = W->cols;
  return true;
}

// The tiled bytes of a dense weight and its type (a model's packed token table reads its
// rows from them).
bool dense_tiled(gmoe_ctx* c, uint32_t id, const uint8_t** tiled, uint32_t* qtype) {
  CtxLock g(c);
  Dense* W;
  if (get_dense(c, id, &W) != GMOE_OK) return false;
  *tiled = W->tiled;
  *qtype = W->qtype;
  return true;
}

bool layer_width(gmoe_ctx* c, uint32_t id, uint32_t* d, uint32_t* ne) {
  CtxLock g(c);
  Layer* L;
  if (get_layer(c, id, &L) != GMOE_OK) return false;
  *d = L->d;
  *ne = L->ne;
  return true;
}

}  // namespace gmoe

extern "C" {

uint32_t gmoe_abi_version(void) { return GMOE_ABI_VERSION; }

const char* gmoe_last_error(void) { return g_err.c_str(); }

uint32_t gmoe_last_invalid_token(void) { return g_bad_token; }

gmoe_status gmoe_init(int device, uint64_t slab_bytes, gmoe_ctx** out) {
  if (!out) return fail(GMOE_ERR_INFERENCE, "null output pointer");
  *out = nullptr;
  int count = 0;
  HIP_TRY(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) return fail(GMOE_ERR_DEVICE, "device %d not present (%d visible)", device, count);
  HIP_TRY(hipSetDevice(device));
  std::unique_ptr<gmoe_ctx> c(new gmoe_ctx);
  c->device = device;
  {
    void* p = nullptr;
    const hipError_t e = noalloc_scratch(device, &p);
    if (e != hipSuccess)
      return fail(GMOE_ERR_DEVICE, "looking up the allocation-free scratch on device %d: %s", device,
                  hipGetErrorString(e));
    c->noalloc = static_cast<uint8_t*>(p);
  }
  HIP_TRY(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
  HIP_TRY(hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking));
  if (slab_bytes) {
    if (hipMalloc(&c->slab.base, slab_bytes) != hipSuccess)
      return fail(GMOE_ERR_CACHE, "cannot reserve an HBM slab of %llu bytes", (unsigned long long)slab_bytes);
    c->slab.cap = slab_bytes;
    c->slab.free_[0] = slab_bytes;
  }
  c->stats.capacity = slab_bytes;
  // two 16 MiB halves: a half's host copy and the other half's DMA overlap, and each
  // copy's working set stays within the host's last-level cache (measured: 32 MiB gives
  // 42 GB/s from a mapped file, 64 MiB 28 GB/s, against a 57 GB/s pinned link)
  c->pinned_bytes = (size_t)32 << 20;
  HIP_TRY(hipHostMalloc((void**)&c->pinned, c->pinned_bytes, hipHostMallocDefault));
  HIP_TRY(hipMalloc(&c->bounce, c->pinned_bytes));
  // [0]: front-end workgroups done; [64 .. 64 + kSpecMaxSlots): per-token routing counters
  HIP_TRY(hipMalloc(&c->done, (64 + kSpecMaxSlots) * 4));
  HIP_TRY(hipMemset(c->done, 0, (64 + kSpecMaxSlots) * 4));
  HIP_TRY(hipEventCreateWithFlags(&c->pin_ev[0], hipEventDisableTiming));
  HIP_TRY(hipEventCreateWithFlags(&c->pin_ev[1], hipEventDisableTiming));
  HIP_TRY(hipEventRecord(c->pin_ev[0], c->copy_stream));
  HIP_TRY(hipEventRecord(c->pin_ev[1], c->copy_stream));
  gmoe_ctx* raw = c.get();
  c->stager = std::thread([raw] { stager_main(raw); });
  *out = c.release();
  return GMOE_OK;
}

void gmoe_shutdown(gmoe_ctx* c) {
  if (!c) return;
  {  // the staging thread finishes the expert it is copying and stops
    std::lock_guard<std::mutex> lk(c->slab_mu);
    c->stop = true;
  }
  c->cv.notify_all();
  if (c->stager.joinable()) c->stager.join();
  hipSetDevice(c->device);
  hipStreamSynchronize(c->stream);
  hipStreamSynchronize(c->copy_stream);
  for (auto& L : c->layers)
    if (L) {
      hipFree(L->router);
      hipFree((void*)L->eptr);
    }
  for (auto& t : c->pending) c->pool.push_back(t);
  for (auto& t : c->pool) {
    hipEventDestroy(t.a);
    hipEventDestroy(t.b);
    hipEventDestroy(t.c);
  }
  for (auto& W : c->dense)
    if (W) {
      if (W->tiled) hipFree(W->tiled);
      if (W->work_tab) hipFree(W->work_tab);
    }
  if (c->ident) hipFree(c->ident);
  if (c->slab.base) hipFree(c->slab.base);
  if (c->scratch) hipFree(c->scratch);
  if (c->pinned) hipHostFree(c->pinned);
  if (c->bounce) hipFree(c->bounce);
  if (c->done) hipFree(c->done);
  hipEventDestroy(c->pin_ev[0]);
  hipEventDestroy(c->pin_ev[1]);
  hipStreamDestroy(c->stream);
  hipStreamDestroy(c->copy_stream);
  delete c;
}

}  // extern "C"

namespace {

// gmoe_layer_register and gmoe_layer_register_fetch: with `fetch` set the tensors' host
// pointers are not read (each expert comes from fetch when it is staged) and nothing is
// staged here, so every expert is loaded when first routed, as MoeEngine loads it.
gmoe_status register_layer(gmoe_ctx* c, const gmoe_layer_desc* desc, gmoe_expert_fetch fetch, void* user,
                           uint32_t* layer_id) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!desc || !layer_id) return fail(GMOE_ERR_INFERENCE, "null descriptor");
  const gmoe_layer_desc& D = *desc;
  if (D.d_model == 0 || D.d_ff == 0 || D.n_experts == 0)
    return fail(GMOE_ERR_CONFIG, "d_model, d_ff and n_experts must be non-zero");
  if (D.top_k == 0 || D.top_k > D.n_experts)
    return fail(GMOE_ERR_CONFIG, "top_k (%u) must be in 1..=%u", D.top_k, D.n_experts);
  if (D.top_k > 32) return fail(GMOE_ERR_CONFIG, "top_k above 32 is not supported");
  if (D.n_experts > kMaxExperts)
    return fail(GMOE_ERR_CONFIG, "n_experts (%u) above %u is not supported", D.n_experts, kMaxExperts);
  if (D.gating > 3 || D.combine > 1 || D.math > 1) return fail(GMOE_ERR_CONFIG, "unknown gating/combine/math");
  if (!D.router) return fail(GMOE_ERR_MODEL, "router weights missing");
  const gmoe_tensor* T[3] = {&D.gate, &D.up, &D.down};
  std::unique_ptr<Layer> L(new Layer);
  L->d = D.d_model; L->f = D.d_ff; L->ne = D.n_experts; L->k = D.top_k;
  L->gating = D.gating; L->combine = D.combine; L->math = D.math;
  for (int p = 0; p < 3; p++) {
    Proj& P = L->p[p];
    P.qtype = T[p]->qtype;
    P.rows = p < 2 ? D.d_ff : D.d_model;
    P.cols = p < 2 ? D.d_model : D.d_ff;
    uint64_t rb;
    if (gmoe_status s = byte_size(P.qtype, P.cols, &rb)) return s;
    if (!k_ok(P.qtype, P.cols))
      return fail(GMOE_ERR_MODEL, "%s rows of %u values: width must be a multiple of 32", type_name(P.qtype), P.cols);
    P.row_bytes = rb;
    Unit un;
    if (!unit_of(P.qtype, &un)) return fail(GMOE_ERR_MODEL, "unsupported tensor type %u", P.qtype);
    P.bytes_dev = tiled_bytes(un, P.rows, P.cols);
    if (fetch) continue;
    P.host.resize(L->ne);
    if (T[p]->layout == GMOE_LAYOUT_STACKED) {
      if (!T[p]->data) return fail(GMOE_ERR_MODEL, "stacked tensor %d has no data", p);
      for (uint32_t e = 0; e < L->ne; e++)
        P.host[e] = (const uint8_t*)T[p]->data + (uint64_t)e * P.rows * rb;
    } else if (T[p]->layout == GMOE_LAYOUT_SPLIT) {
      if (!T[p]->experts) return fail(GMOE_ERR_MODEL, "split tensor %d has no expert list", p);
      for (uint32_t e = 0; e < L->ne; e++) {
        if (!T[p]->experts[e]) return fail(GMOE_ERR_MODEL, "expert %u of tensor %d is missing", e, p);
        P.host[e] = (const uint8_t*)T[p]->experts[e];
      }
    } else {
      return fail(GMOE_ERR_CONFIG, "unknown tensor layout %u", T[p]->layout);
    }
  }
  if (L->p[0].qtype != L->p[1].qtype)
    return fail(GMOE_ERR_MODEL, "gate (%s) and up (%s) must share a type", type_name(L->p[0].qtype),
                type_name(L->p[1].qtype));
  if (uses_int8(L->math, L->p[2].qtype) && L->f % 32)
    return fail(GMOE_ERR_MODEL, "d_ff must be a multiple of 32");
  for (int p = 0; p < 3; p++) L->expert_bytes += (L->p[p].bytes_dev + 255) & ~uint64_t(255);

  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipMalloc(&L->router, (size_t)L->ne * L->d * 4));
  HIP_TRY(hipMemcpy(L->router, D.router, (size_t)L->ne * L->d * 4, hipMemcpyHostToDevice));
  L->eptr_host.assign(3 * L->ne, nullptr);
  HIP_TRY(hipMalloc((void**)&L->eptr, 3 * L->ne * sizeof(void*)));
  HIP_TRY(hipMemcpy(L->eptr, L->eptr_host.data(), 3 * L->ne * sizeof(void*), hipMemcpyHostToDevice));
  L->slot.assign(L->ne, -1);
  L->lru_pos.resize(L->ne);
  L->pending.assign(L->ne, kAbsent);
  L->fetch = fetch;
  L->fetch_user = user;
  uint32_t id = (uint32_t)c->layers.size();
  c->layers.push_back(std::move(L));
  Layer& LL = *c->layers.back();
  for (uint32_t e = 0; e < LL.ne && !fetch; e++) {
    gmoe_status s = make_resident(c, g.slab, id, e, false, nullptr);
    if (s == GMOE_ERR_CACHE) break;  // the rest stays on the host tier
    if (s) return s;
  }
  *layer_id = id;
  return GMOE_OK;
}

}  // namespace

extern "C" {

gmoe_status gmoe_layer_register(gmoe_ctx* c, const gmoe_layer_desc* desc, uint32_t* layer_id) {
  return register_layer(c, desc, nullptr, nullptr, layer_id);
}

gmoe_status gmoe_layer_register_fetch(gmoe_ctx* c, const gmoe_layer_desc* desc, gmoe_expert_fetch fetch, void* user,
                                      uint32_t* layer_id) {
  if (!fetch) return fail(GMOE_ERR_INFERENCE, "null fetch callback");
  return register_layer(c, desc, fetch, user, layer_id);
}

gmoe_status gmoe_layer_release(gmoe_ctx* c, uint32_t id) {
  if (gmoe_status s = check_ctx(c)) return s;
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, id, &L)) return s;
  if (L->pins) return fail(GMOE_ERR_CACHE, "layer %u is in use by a model step", id);
  HIP_TRY(hipSetDevice(c->device));
  // its queued experts leave the staging queue; the one being staged is waited for
  c->queue.erase(std::remove_if(c->queue.begin(), c->queue.end(), [&](const auto& q) { return q.first == id; }),
                 c->queue.end());
  for (uint32_t e = 0; e < L->ne; e++)
    if (L->pending[e] == kQueued) L->pending[e] = kAbsent;
  c->cv.wait(g.slab, [&] {
    for (uint32_t e = 0; e < L->ne; e++)
      if (L->pending[e] == kStaging) return false;
    return true;
  });
  for (uint32_t e = 0; e < L->ne; e++)
    if (gmoe_status s = evict(c, id, e)) return s;
  hipFree(L->router);
  hipFree((void*)L->eptr);
  L->router = nullptr;
  L->eptr = nullptr;
  L->alive = false;
  return GMOE_OK;
}

gmoe_status gmoe_ffn_forward(gmoe_ctx* c, uint32_t layer, const float* hs, uint32_t n, float* out,
                             uint32_t* ids, float* w) {
  return forward_host(c, layer, hs, nullptr, n, out, ids, w);
}

gmoe_status gmoe_ffn_forward_logits(gmoe_ctx* c, uint32_t layer, const float* hs, const float* logits,
                                    uint32_t n, float* out, uint32_t* ids, float* w) {
  if (!logits) return fail(GMOE_ERR_INFERENCE, "null logits");
  return forward_host(c, layer, hs, logits, n, out, ids, w);
}

gmoe_status gmoe_ffn_forward_async(gmoe_ctx* c, uint32_t lid, const float* d_hs, const float* d_logits,
                                   uint32_t n, float* d_out, uint32_t* d_ids, float* d_w, void* stream) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!d_hs || !d_out) return fail(GMOE_ERR_INFERENCE, "null activation pointer");
  if (n == 0) return fail(GMOE_ERR_INFERENCE, "empty batch");
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, lid, &L)) return s;
  for (uint32_t e = 0; e < L->ne; e++)
    if (L->slot[e] < 0) return fail(GMOE_ERR_CACHE, "expert %u of layer %u is not resident", e, lid);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = stream ? (hipStream_t)stream : c->stream;
  const uint32_t per = call_tokens(*L);
  if (gmoe_status s = ensure_scratch(c, call_scratch(*L, n))) return s;
  for (uint32_t t0 = 0; t0 < n; t0 += per) {
    const uint32_t m = std::min(per, n - t0);
    Carved cv;
    plan_scratch(*L, m, &cv, c->scratch);
    FwdBufs B = cv.B;
    B.hs = d_hs + (size_t)t0 * L->d;
    B.logits_in = d_logits ? d_logits + (size_t)t0 * L->ne : nullptr;
    B.out = d_out + (size_t)t0 * L->d;
    if (d_ids) B.ids = d_ids + (size_t)t0 * L->k;
    if (d_w) B.w = d_w + (size_t)t0 * L->k;
    if (gmoe_status s = run_layer(c, *L, B, m, st)) return s;
    c->scratch_stream = st;
  }
  return GMOE_OK;
}

gmoe_status gmoe_ffn_forward_noalloc(gmoe_ctx* c, uint32_t lid, const float* d_hs, const float* d_logits,
                                     uint32_t n, float* d_out, uint32_t* d_ids, float* d_w, void* stream) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!d_hs || !d_out) return fail(GMOE_ERR_INFERENCE, "null activation pointer");
  if (n == 0) return fail(GMOE_ERR_INFERENCE, "empty batch");
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, lid, &L)) return s;
  for (uint32_t e = 0; e < L->ne; e++)
    if (L->slot[e] < 0) return fail(GMOE_ERR_CACHE, "expert %u of layer %u is not resident", e, lid);
  if (!c->noalloc) return fail(GMOE_ERR_DEVICE, "the allocation-free scratch is not set up on device %d", c->device);
  const size_t need = call_scratch(*L, n);
  if (need > kNoAllocScratchBytes)
    return fail(GMOE_ERR_INFERENCE,
                "a call of %u tokens on this layer needs %zu bytes of scratch; the allocation-free forward has %zu "
                "(use gmoe_ffn_forward_async)",
                n, need, kNoAllocScratchBytes);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = stream ? (hipStream_t)stream : c->stream;
  // every call on this GPU shares the array: this one runs after the previous one's work
  hipError_t oe;
  auto order = noalloc_begin(c->device, st, &oe);
  HIP_TRY(oe);
  const uint32_t per = call_tokens(*L);
  for (uint32_t t0 = 0; t0 < n; t0 += per) {
    const uint32_t m = std::min(per, n - t0);
    Carved cv;
    plan_scratch(*L, m, &cv, c->noalloc);
    FwdBufs B = cv.B;
    B.hs = d_hs + (size_t)t0 * L->d;
    B.logits_in = d_logits ? d_logits + (size_t)t0 * L->ne : nullptr;
    B.out = d_out + (size_t)t0 * L->d;
    if (d_ids) B.ids = d_ids + (size_t)t0 * L->k;
    if (d_w) B.w = d_w + (size_t)t0 * L->k;
    if (gmoe_status s = run_layer(c, *L, B, m, st, false)) {
      (void)noalloc_end(c->device, st);
      return s;
    }
  }
  HIP_TRY(noalloc_end(c->device, st));
  return GMOE_OK;
}

gmoe_status gmoe_expert_prefetch(gmoe_ctx* c, uint32_t lid, uint32_t e) {
  if (gmoe_status s = check_ctx(c)) return s;
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, lid, &L)) return s;
  if (e >= L->ne) return fail(GMOE_ERR_INFERENCE, "expert %u out of range", e);
  HIP_TRY(hipSetDevice(c->device));
  std::vector<std::pair<uint32_t, uint32_t>> keep{{lid, e}};
  return make_resident(c, g.slab, lid, e, true, &keep);
}

int gmoe_expert_is_resident(gmoe_ctx* c, uint32_t lid, uint32_t e) {
  if (!c) return 0;
  CtxLock g(c);
  if (lid >= c->layers.size() || !c->layers[lid] || !c->layers[lid]->alive) return 0;
  Layer& L = *c->layers[lid];
  return e < L.ne && L.slot[e] >= 0;
}

gmoe_status gmoe_expert_evict(gmoe_ctx* c, uint32_t lid, uint32_t e) {
  if (gmoe_status s = check_ctx(c)) return s;
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, lid, &L)) return s;
  if (e >= L->ne) return fail(GMOE_ERR_INFERENCE, "expert %u out of range", e);
  if (L->pins) return fail(GMOE_ERR_CACHE, "layer %u is in use by a model step", lid);
  HIP_TRY(hipSetDevice(c->device));
  c->cv.wait(g.slab, [&] { return L->pending[e] != kStaging; });
  if (L->pending[e] == kQueued) {
    c->queue.erase(std::remove(c->queue.begin(), c->queue.end(), std::make_pair(lid, e)), c->queue.end());
    L->pending[e] = kAbsent;
  }
  return evict(c, lid, e);
}

int gmoe_expert_state(gmoe_ctx* c, uint32_t lid, uint32_t e) {
  if (!c) return GMOE_EXPERT_ABSENT;
  CtxLock g(c);
  if (lid >= c->layers.size() || !c->layers[lid] || !c->layers[lid]->alive) return GMOE_EXPERT_ABSENT;
  Layer& L = *c->layers[lid];
  if (e >= L.ne) return GMOE_EXPERT_ABSENT;
  if (L.slot[e] >= 0) return GMOE_EXPERT_RESIDENT;
  return L.pending[e] == kQueued ? GMOE_EXPERT_QUEUED : L.pending[e] == kStaging ? GMOE_EXPERT_STAGING
                                                                                    : GMOE_EXPERT_ABSENT;
}

gmoe_status gmoe_prefetch_hold(gmoe_ctx* c, int hold) {
  if (gmoe_status s = check_ctx(c)) return s;
  CtxLock g(c);
  c->hold = hold != 0;
  c->cv.notify_all();
  return GMOE_OK;
}

gmoe_status gmoe_prefetch_wait(gmoe_ctx* c) {
  if (gmoe_status s = check_ctx(c)) return s;
  CtxLock g(c);
  c->cv.wait(g.slab, [&] { return c->staging == 0 && (c->hold || c->queue.empty()); });
  return GMOE_OK;
}

gmoe_status gmoe_slab_get_stats(gmoe_ctx* c, gmoe_slab_stats* out) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!out) return fail(GMOE_ERR_INFERENCE, "null output");
  CtxLock g(c);
  *out = c->stats;
  return GMOE_OK;
}

// ---- single steps ----

gmoe_status gmoe_dense_register(gmoe_ctx* c, const gmoe_dense_desc* desc, uint32_t* id) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!desc || !id || !desc->data) return fail(GMOE_ERR_INFERENCE, "null descriptor, data or id");
  if (desc->math > 1) return fail(GMOE_ERR_CONFIG, "unknown math %u", desc->math);
  if (desc->rows == 0 || desc->cols == 0) return fail(GMOE_ERR_MODEL, "empty dense weight");
  uint64_t rb;
  if (gmoe_status s = byte_size(desc->qtype, desc->cols, &rb)) return s;
  if (!k_ok(desc->qtype, desc->cols)) return fail(GMOE_ERR_MODEL, "dense width %u is not a multiple of 32", desc->cols);
  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  auto W = std::make_unique<Dense>();
  W->qtype = desc->qtype;
  W->rows = desc->rows;
  W->cols = desc->cols;
  W->math = desc->math;
  Unit un;
  unit_of(W->qtype, &un);
  W->tiled_bytes = tiled_bytes(un, W->rows, W->cols);
  HIP_TRY(hipMalloc(&W->tiled, W->tiled_bytes));
  if (gmoe_status s = dense_tables(c, W.get())) return s;
  Proj P;
  P.qtype = W->qtype;
  P.rows = W->rows;
  P.cols = W->cols;
  P.row_bytes = rb;
  P.bytes_dev = W->tiled_bytes;
  gmoe_status s;
  {
    std::lock_guard<std::mutex> sg(c->stage_mu);  // the pinned halves and the copy stream
    s = stage_proj(c, P, static_cast<const uint8_t*>(desc->data), W->tiled);
    if (s == GMOE_OK && hipStreamSynchronize(c->copy_stream) != hipSuccess)
      s = fail(GMOE_ERR_DEVICE, "staging the dense weight failed");
  }
  if (s != GMOE_OK) {
    hipStreamSynchronize(c->copy_stream);
    hipFree(W->tiled);
    hipFree(W->work_tab);
    return s;
  }
  *id = (uint32_t)c->dense.size();
  c->dense.push_back(std::move(W));
  return GMOE_OK;
}

gmoe_status gmoe_dense_release(gmoe_ctx* c, uint32_t id) {
  if (gmoe_status s = check_ctx(c)) return s;
  CtxLock g(c);
  Dense* W;
  if (gmoe_status s = get_dense(c, id, &W)) return s;
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipDeviceSynchronize());  // queued work on any stream may still read it
  hipFree(W->tiled);
  hipFree(W->work_tab);
  W->tiled = nullptr;
  W->work_tab = nullptr;
  W->alive = false;
  return GMOE_OK;
}

gmoe_status gmoe_dense_forward(gmoe_ctx* c, uint32_t id, const float* xs, uint32_t n, float* out) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!xs || !out) return fail(GMOE_ERR_INFERENCE, "null activation pointer");
  if (n == 0) return fail(GMOE_ERR_INFERENCE, "empty batch");
  CtxLock g(c);
  Dense* W;
  if (gmoe_status s = get_dense(c, id, &W)) return s;
  HIP_TRY(hipSetDevice(c->device));
  ScratchPlan io;
  const size_t o_x = io.add((size_t)n * W->cols * 4), o_o = io.add((size_t)n * W->rows * 4);
  const size_t need = io.total + plan_dense(c, *W, n, nullptr, nullptr);
  if (gmoe_status s = ensure_scratch(c, need)) return s;
  DenseCarve cv;
  plan_dense(c, *W, n, c->scratch + io.total, &cv);
  hipStream_t st = c->stream;
  float* dx = (float*)(c->scratch + o_x);
  float* dout = (float*)(c->scratch + o_o);
  HIP_TRY(hipMemcpyAsync(dx, xs, (size_t)n * W->cols * 4, hipMemcpyHostToDevice, st));
  if (gmoe_status s = run_dense(*W, cv, dx, n, dout, st)) return s;
  if (gmoe_status s = mark_scratch(c, st)) return s;
  HIP_TRY(hipMemcpyAsync(out, dout, (size_t)n * W->rows * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return GMOE_OK;
}

gmoe_status gmoe_dense_forward_async(gmoe_ctx* c, uint32_t id, const float* d_xs, uint32_t n, float* d_out,
                                     void* stream) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!d_xs || !d_out) return fail(GMOE_ERR_INFERENCE, "null activation pointer");
  if (n == 0) return fail(GMOE_ERR_INFERENCE, "empty batch");
  CtxLock g(c);
  Dense* W;
  if (gmoe_status s = get_dense(c, id, &W)) return s;
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = stream ? (hipStream_t)stream : c->stream;
  if (gmoe_status s = ensure_scratch(c, plan_dense(c, *W, n, nullptr, nullptr))) return s;
  DenseCarve cv;
  plan_dense(c, *W, n, c->scratch, &cv);
  if (gmoe_status s = run_dense(*W, cv, d_xs, n, d_out, st)) return s;
  return mark_scratch(c, st);
}

static_assert(GMOE_DENSE_MAX_SLICES == kMaxKsg, "the dense call's K slices");

gmoe_status gmoe_dense_forward_slices_async(gmoe_ctx* c, uint32_t id, const float* d_xs, uint32_t n, float* d_parts,
                                            uint32_t* nsl, void* stream) {
  if (!d_parts) return fail(GMOE_ERR_INFERENCE, "null slice buffer");
  const float* parts = nullptr;
  return dense_slices(c, id, d_xs, n, stream ? (hipStream_t)stream : (c ? c->stream : nullptr), &parts, nsl, d_parts);
}

gmoe_status gmoe_prefetch_step(gmoe_ctx* c, gmoe_predictor* p, uint32_t lid, uint32_t base, const uint32_t* prev,
                               uint32_t nprev, const uint32_t* used, uint32_t nused, const uint32_t* pl,
                               uint32_t npl, uint32_t depth, uint32_t* pred, uint32_t* npred, uint32_t* launched,
                               uint32_t* skipped) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!p || !npred || (depth && !pred) || (nprev && !prev) || (nused && !used) || (npl && !pl))
    return fail(GMOE_ERR_INFERENCE, "null predictor, ids or output");
  // prefetch/mod.rs:84-100: score last step's guess, learn the transition, predict
  if (npl)
    if (gmoe_status s = gmoe_predictor_score(p, pl, npl, used, nused)) return s;
  if (nprev)
    if (gmoe_status s = gmoe_predictor_observe(p, prev, nprev, used, nused)) return s;
  if (gmoe_status s = gmoe_predictor_predict(p, used, nused, depth, pred, npred)) return s;
  uint32_t nl = 0, ns = 0;
  CtxLock g(c);
  Layer* L;
  if (gmoe_status s = get_layer(c, lid, &L)) return s;
  HIP_TRY(hipSetDevice(c->device));
  // the experts this step and the step before used, and the ones predicted, stay; only
  // experts idle for two steps may be evicted to make room for a prediction (a wrong
  // guess that evicted last step's expert cost a miss whenever routing came back to it)
  Keep keep;
  for (uint32_t i = 0; i < nused; i++)
    if (used[i] >= base && used[i] - base < L->ne) keep.emplace_back(lid, used[i] - base);
  for (uint32_t i = 0; i < nprev; i++)
    if (prev[i] >= base && prev[i] - base < L->ne) keep.emplace_back(lid, prev[i] - base);
  for (uint32_t i = 0; i < *npred; i++)
    if (pred[i] >= base && pred[i] - base < L->ne) keep.emplace_back(lid, pred[i] - base);
  c->prefetch_keep = keep;
  // PrefetchEngine::warm: an expert already resident, queued or being staged is skipped;
  // the others are queued for the staging thread, and the call returns at once
  for (uint32_t i = 0; i < *npred; i++) {
    if (pred[i] < base || pred[i] - base >= L->ne) continue;  // another layer's expert
    const uint32_t e = pred[i] - base;
    if (L->slot[e] >= 0 || L->pending[e] != kAbsent) {
      ns++;
      continue;
    }
    L->pending[e] = kQueued;
    c->queue.emplace_back(lid, e);
    nl++;
  }
  if (nl) c->cv.notify_all();
  if (launched) *launched = nl;
  if (skipped) *skipped = ns;
  return GMOE_OK;
}

gmoe_status gmoe_dequant(gmoe_ctx* c, uint32_t qt, const void* blocks, uint64_t nbytes, uint64_t n,
                         float* out) {
  if (gmoe_status s = check_ctx(c)) return s;
  uint64_t want;
  if (gmoe_status s = byte_size(qt, n, &want)) return s;
  if (nbytes != want)
    return fail(GMOE_ERR_MODEL, "%s tensor: expected %llu bytes for %llu elements, got %llu", type_name(qt),
                (unsigned long long)want, (unsigned long long)n, (unsigned long long)nbytes);
  if ((qt == F32 || qt == F16) && n % 32)
    return fail(GMOE_ERR_MODEL, "%s dequant on the device takes multiples of 32 values", type_name(qt));
  if (n == 0) return GMOE_OK;
  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  uint8_t* db = nullptr;
  float* dout = nullptr;
  HIP_TRY(hipMalloc(&db, nbytes + 16));
  hipError_t e1 = hipMalloc(&dout, n * 4);
  if (e1 != hipSuccess) {
    hipFree(db);
    return fail(GMOE_ERR_DEVICE, "hipMalloc: %s", hipGetErrorString(e1));
  }
  uint32_t el, by;
  block_layout(qt, &el, &by);
  uint64_t nb = (qt == F32 || qt == F16) ? n / 32 : n / el;
  hipError_t e = hipMemcpy(db, blocks, nbytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_dequant(qt, db, nb, dout, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess) e = hipMemcpy(out, dout, n * 4, hipMemcpyDeviceToHost);
  hipFree(db);
  hipFree(dout);
  if (e != hipSuccess) return fail(GMOE_ERR_DEVICE, "dequant: %s", hipGetErrorString(e));
  return GMOE_OK;
}

gmoe_status gmoe_expf(gmoe_ctx* c, const float* x, uint64_t n, float* y) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (n == 0) return GMOE_OK;
  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  float *dx = nullptr, *dy = nullptr;
  HIP_TRY(hipMalloc(&dx, n * 4));
  hipError_t e = hipMalloc(&dy, n * 4);
  if (e == hipSuccess) e = hipMemcpy(dx, x, n * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_expf(dx, dy, n, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess) e = hipMemcpy(y, dy, n * 4, hipMemcpyDeviceToHost);
  hipFree(dx);
  if (dy) hipFree(dy);
  if (e != hipSuccess) return fail(GMOE_ERR_DEVICE, "expf: %s", hipGetErrorString(e));
  return GMOE_OK;
}

// A one-off layer around a single matrix: expert 0's down projection, every vector
// routed to it, so the split-K down kernel computes out[b*rows + r].
gmoe_status gmoe_matmul(gmoe_ctx* c, uint32_t qt, uint32_t math, const void* w, uint64_t nbytes, uint32_t rows,
                        uint32_t cols, const float* xs, uint32_t n, float* out) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (math > 1) return fail(GMOE_ERR_CONFIG, "unknown math");
  uint64_t rb;
  if (gmoe_status s = byte_size(qt, cols, &rb)) return s;
  if (nbytes != rb * rows)
    return fail(GMOE_ERR_MODEL, "%s matmul: weight is %llu bytes, expected %llu (%u rows x %llu)", type_name(qt),
                (unsigned long long)nbytes, (unsigned long long)(rb * rows), rows, (unsigned long long)rb);
  if (!k_ok(qt, cols)) return fail(GMOE_ERR_MODEL, "matmul width must be a multiple of 32");
  if (n == 0 || rows == 0) return fail(GMOE_ERR_INFERENCE, "matmul dimension mismatch");
  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  Unit un;
  unit_of(qt, &un);
  size_t wbytes = tiled_bytes(un, rows, cols);
  size_t nb_x = (size_t)n * cols;
  // device layout: [w tiled][w raw][x f32][xq][xs][x sums][y][out][offsets(2)][active(2)][eptr(3)][work(1)]
  ScratchPlan P;
  size_t o_w = P.add(wbytes), o_raw = P.add(nbytes), o_x = P.add(nb_x * 4), o_q = P.add(nb_x), o_s = P.add(nb_x / 32 * 4),
         o_16 = P.add(nb_x / 16 * 4), o_y = P.add(kMaxKsg * (size_t)n * rows * 4), o_o = P.add((size_t)n * rows * 4), o_off = P.add(8), o_act = P.add(8),
         o_ep = P.add(3 * sizeof(void*)), o_wk = P.add(sizeof(ExpertWork));
  uint8_t* base = nullptr;
  HIP_TRY(hipMalloc(&base, P.total));
  uint32_t offs[2] = {0, n}, act[2] = {1, 0};
  const uint8_t* ep[3] = {base + o_w, base + o_w, base + o_w};
  hipError_t e = hipMemcpy(base + o_raw, w, nbytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_tile_rows(qt, base + o_raw, 0, rows, rows, cols, base + o_w, c->stream);
  if (e == hipSuccess) e = hipMemcpy(base + o_x, xs, nb_x * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(base + o_off, offs, 8, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(base + o_act, act, 8, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(base + o_ep, ep, sizeof ep, hipMemcpyHostToDevice);
  ExpertWork wk{{base + o_w, base + o_w, base + o_w}, 0, 0, n, 0};
  if (e == hipSuccess) e = hipMemcpy(base + o_wk, &wk, sizeof wk, hipMemcpyHostToDevice);
  LayerDev D{};
  D.d = rows; D.f = cols; D.ne = 1; D.k = 1; D.math = math;
  D.qt_gate = D.qt_up = D.qt_down = qt;
  D.eptr = (const uint8_t* const*)(base + o_ep);
  FwdBufs B{};
  B.offsets = (uint32_t*)(base + o_off);
  B.active = (uint32_t*)(base + o_act);
  B.y = (float*)(base + o_y);
  B.nslot = n;
  B.work = (ExpertWork*)(base + o_wk);
  if (uses_int8(math, qt)) {
    B.hq = (int8_t*)(base + o_q);
    B.hsc = (float*)(base + o_s);
    B.hsum = (uint32_t*)(base + o_16);
    if (e == hipSuccess) e = launch_quant_act((const float*)(base + o_x), n, cols, B.hq, B.hsc, B.hsum, qt, c->stream);
  } else {
    B.hf = (float*)(base + o_x);
  }
  if (e == hipSuccess) e = launch_down(D, B, n, c->stream);
  float* dout = (float*)(base + o_o);
  if (e == hipSuccess) e = launch_reduce_parts(B.y, down_ksg(D, n), (size_t)n * rows, dout, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess) e = hipMemcpy(out, dout, (size_t)n * rows * 4, hipMemcpyDeviceToHost);
  hipFree(base);
  if (e != hipSuccess) return fail(GMOE_ERR_DEVICE, "matmul: %s", hipGetErrorString(e));
  return GMOE_OK;
}

gmoe_status gmoe_route(gmoe_ctx* c, uint32_t gating, const float* router, const float* x, uint32_t d, uint32_t ne,
                       uint32_t k, uint32_t n, uint32_t* ids, float* w, float* logits_out) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (gating > 3) return fail(GMOE_ERR_CONFIG, "unknown gating");
  if (k == 0 || k > ne || k > 32) return fail(GMOE_ERR_CONFIG, "top_k (%u) must be in 1..=%u", k, ne);
  if (n == 0 || !x || !ids || !w) return fail(GMOE_ERR_INFERENCE, "bad route arguments");
  if (router && d % 4) return fail(GMOE_ERR_INFERENCE, "router width must be a multiple of 4");
  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  ScratchPlan P;
  size_t xlen = router ? (size_t)n * d : (size_t)n * ne;
  size_t o_r = P.add(router ? (size_t)ne * d * 4 : 4), o_x = P.add(xlen * 4), o_i = P.add((size_t)n * k * 4),
         o_w = P.add((size_t)n * k * 4), o_l = P.add((size_t)n * ne * 4);
  uint8_t* base = nullptr;
  HIP_TRY(hipMalloc(&base, P.total));
  hipError_t e = hipSuccess;
  if (router) e = hipMemcpy(base + o_r, router, (size_t)ne * d * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(base + o_x, x, xlen * 4, hipMemcpyHostToDevice);
  LayerDev D{};
  D.d = d; D.ne = ne; D.k = k; D.gating = gating;
  D.router = (const float*)(base + o_r);
  FwdBufs B{};
  if (router) B.hs = (const float*)(base + o_x);
  else B.logits_in = (const float*)(base + o_x);
  B.ids = (uint32_t*)(base + o_i);
  B.w = (float*)(base + o_w);
  B.logits = (float*)(base + o_l);
  if (e == hipSuccess) e = launch_route(D, B, n, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess) e = hipMemcpy(ids, B.ids, (size_t)n * k * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(w, B.w, (size_t)n * k * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && logits_out) e = hipMemcpy(logits_out, B.logits, (size_t)n * ne * 4, hipMemcpyDeviceToHost);
  hipFree(base);
  if (e != hipSuccess) return fail(GMOE_ERR_DEVICE, "route: %s", hipGetErrorString(e));
  return GMOE_OK;
}

gmoe_status gmoe_dispatch(gmoe_ctx* c, const uint32_t* ids, const float* w, uint32_t n, uint32_t k, uint32_t ne,
                          uint32_t* offsets, uint32_t* slot_token, float* slot_weight, uint32_t* slot_rank) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (!ids || !w || !offsets || n == 0 || k == 0 || k > ne) return fail(GMOE_ERR_INFERENCE, "bad dispatch arguments");
  if (ne > kMaxExperts) return fail(GMOE_ERR_CONFIG, "n_experts (%u) above %u is not supported", ne, kMaxExperts);
  for (uint64_t i = 0; i < (uint64_t)n * k; i++)
    if (ids[i] >= ne) return fail(GMOE_ERR_INFERENCE, "expert id %u out of range", ids[i]);
  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  size_t nk = (size_t)n * k;
  ScratchPlan P;
  size_t o_i = P.add(nk * 4), o_w = P.add(nk * 4), o_off = P.add((ne + 1) * 4), o_act = P.add((ne + 1) * 4),
         o_st = P.add(nk * 4), o_sw = P.add(nk * 4), o_sr = P.add(nk * 4), o_so = P.add(nk * 4);
  uint8_t* base = nullptr;
  HIP_TRY(hipMalloc(&base, P.total));
  hipError_t e = hipMemcpy(base + o_i, ids, nk * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(base + o_w, w, nk * 4, hipMemcpyHostToDevice);
  LayerDev D{};
  D.ne = ne; D.k = k;
  FwdBufs B{};
  B.ids = (uint32_t*)(base + o_i);
  B.w = (float*)(base + o_w);
  B.offsets = (uint32_t*)(base + o_off);
  B.active = (uint32_t*)(base + o_act);
  B.slot_tok = (uint32_t*)(base + o_st);
  B.slot_w = (float*)(base + o_sw);
  B.slot_rank = (uint32_t*)(base + o_sr);
  B.slot_of = (uint32_t*)(base + o_so);
  if (e == hipSuccess) e = launch_dispatch(D, B, n, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e == hipSuccess) e = hipMemcpy(offsets, B.offsets, (ne + 1) * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && slot_token) e = hipMemcpy(slot_token, B.slot_tok, nk * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && slot_weight) e = hipMemcpy(slot_weight, B.slot_w, nk * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && slot_rank) e = hipMemcpy(slot_rank, B.slot_rank, nk * 4, hipMemcpyDeviceToHost);
  hipFree(base);
  if (e != hipSuccess) return fail(GMOE_ERR_DEVICE, "dispatch: %s", hipGetErrorString(e));
  return GMOE_OK;
}

gmoe_status gmoe_set_kernel_timing(gmoe_ctx* c, int on) {
  if (gmoe_status s = check_ctx(c)) return s;
  CtxLock g(c);
  c->timing = on != 0;
  return GMOE_OK;
}

// which: 0 = gate/up kernel, 1 = down kernel, 2 = both (gate/up start to down end)
gmoe_status gmoe_kernel_time(gmoe_ctx* c, uint32_t which, double* total_ms, uint64_t* count) {
  if (gmoe_status s = check_ctx(c)) return s;
  if (which > 2 || !total_ms || !count) return fail(GMOE_ERR_INFERENCE, "bad kernel_time arguments");
  CtxLock g(c);
  HIP_TRY(hipSetDevice(c->device));
  for (auto& t : c->pending) {
    HIP_TRY(hipEventSynchronize(t.c));
    float a = 0, b = 0, ab = 0;
    HIP_TRY(hipEventElapsedTime(&a, t.a, t.b));
    HIP_TRY(hipEventElapsedTime(&b, t.b, t.c));
    HIP_TRY(hipEventElapsedTime(&ab, t.a, t.c));
    c->t_ms[0] += a;
    c->t_ms[1] += b;
    c->t_ms[2] += ab;
    c->t_cnt++;
    c->pool.push_back(t);
  }
  c->pending.clear();
  *total_ms = c->t_ms[which];
  *count = c->t_cnt;
  return GMOE_OK;
}

}  // extern "C"
