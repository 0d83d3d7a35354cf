// gmoe_l2.cpp — the synthetic engine's expert tiers below the HBM slab.
//
// garuda's MoeEngine pulls each routed expert through MemoryManager
// (garuda/src/memory/mod.rs:114-184): the L1 RAM cache, else the L2 directory's
// `expert_{id}.bin`, else the same file in the L3 directory (copied into L2 on the way
// up), else a deterministic synthesis that is then written to L2. Here the L1 tier is the
// HBM slab; this file is the L2/L3 side feeding it. A file is read as
// weights::expert_from_bytes reads it (weights/mod.rs:123-164): little-endian f32, gate
// [f x d] then up [f x d] then down [d x f], exactly 3*f*d*4 bytes, every value finite.
// An expert with no file is synthesised with weights::synthesize_expert
// (weights/mod.rs:98-109, the splitmix64 stream of :17-35) and written to L2, as
// MemoryManager::load_uncached does (:138-145); a failed write or promotion is not an
// error, since the weights are already held.
//
// A handle from gmoe_l2_open loads every expert at open and keeps L2 files mapped, so the
// slab stages an evicted expert again from the same bytes; one from gmoe_tiers_open loads
// an expert each time it is fetched (one load_uncached per fetch, counted by the tier it
// came from), which is how a layer registered with gmoe_l2_layer_register pulls it.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/garuda_moe.h"

namespace gmoe {
void set_last_error(const char* msg);
}

struct gmoe_l2 {
  std::string dir, l3dir;  // l3dir empty: no L3 tier
  bool lazy = false;
  uint32_t d = 0, f = 0, ne = 0, id_base = 0;
  struct Src {
    const float* w = nullptr;  // gate | up | down
    void* map = nullptr;       // the mapped L2 file, or null when read or synthesised
    size_t map_bytes = 0;
    std::vector<float> own;    // weights read from L3 or synthesised
    bool synth = false;        // own holds the synthesis
  };
  std::vector<Src> src;
  std::vector<const void*> ptr[3];  // per expert: gate, up, down (gmoe_l2_open)
  // weights handed out by an earlier fetch and since replaced: a caller may still be
  // reading them, so they are kept until the handle closes
  std::vector<Src> retired;
  gmoe_l2_counts counts{};
  mutable std::mutex mu;            // loads and counts
};

namespace {

gmoe_status l2_fail(gmoe_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
gmoe_status l2_fail(gmoe_status s, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  gmoe::set_last_error(buf);
  return s;
}

// weights/mod.rs:17-23
uint64_t splitmix64(uint64_t& s) {
  s += 0x9E3779B97F4A7C15ull;
  uint64_t z = s;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// weights/mod.rs:26-35: the top 24 bits as an exact f32 in [0, 1), then (u*2 - 1)*bound
// (each operation rounded on its own; this file is built without contraction)
void seeded(uint64_t seed, size_t n, float bound, float* out) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; i++) {
    const float u = (float)(splitmix64(s) >> 40) / (float)(1u << 24);
    out[i] = (u * 2.0f - 1.0f) * bound;
  }
}

// weights/mod.rs:38-40
float bound(size_t fan_in) { return 1.0f / std::sqrt((float)fan_in); }

// weights/mod.rs:98-109
void synthesize_expert(uint32_t id, uint32_t d, uint32_t f, float* w) {
  const uint64_t kExpert = 0x6761727564611000ull;  // seeds::EXPERT
  const uint64_t seed = kExpert ^ ((uint64_t)id * 0x9E3779B97F4A7C15ull);
  const size_t fd = (size_t)f * d;
  seeded(seed, fd, bound(d), w);
  seeded(seed ^ 0xAAAAAAAAull, fd, bound(d), w + fd);
  seeded(seed ^ 0x55555555ull, fd, bound(f), w + 2 * fd);
}

// Write the expert_to_bytes layout (weights/mod.rs:112-121) to `path` through a
// temporary name, so a reader never sees a partial file. Little-endian host.
bool write_expert(const std::string& path, const float* w, size_t n) {
  const std::string tmp = path + ".tmp";
  FILE* fp = fopen(tmp.c_str(), "wb");
  if (!fp) return false;
  const bool ok = fwrite(w, sizeof(float), n, fp) == n;
  if (fclose(fp) != 0 || !ok || rename(tmp.c_str(), path.c_str()) != 0) {
    unlink(tmp.c_str());
    return false;
  }
  return true;
}

void drop(gmoe_l2::Src& s) {
  if (s.map) munmap(s.map, s.map_bytes);
  s.map = nullptr;
  s.map_bytes = 0;
  s.w = nullptr;
  std::vector<float>().swap(s.own);
}

void release(gmoe_l2* t) {
  for (auto& s : t->src) drop(s);
  for (auto& s : t->retired) drop(s);
  delete t;
}

// Sets expert e's source aside (kept until close) so that a new load can take its place.
void retire(gmoe_l2* t, gmoe_l2::Src& s) {
  if (s.map || !s.own.empty()) t->retired.push_back(std::move(s));
  s = gmoe_l2::Src{};
}

std::string path_in(const std::string& dir, uint32_t id) { return dir + "/expert_" + std::to_string(id) + ".bin"; }

bool exists(const std::string& path) {
  struct stat st {};
  return stat(path.c_str(), &st) == 0;
}

// weights::expert_from_bytes's checks (weights/mod.rs:130-148) on n values of one expert
gmoe_status check_values(uint32_t id, const float* w, size_t n) {
  for (size_t i = 0; i < n; i++)
    if (!std::isfinite(w[i])) return l2_fail(GMOE_ERR_MODEL, "expert %u: non-finite weight at index %zu", id, i);
  return GMOE_OK;
}

// An expert file of `bytes` bytes: mapped (map_it) or read into s.own.
gmoe_status read_file(const gmoe_l2* t, uint32_t id, const std::string& path, bool map_it, gmoe_l2::Src& s) {
  const size_t n = 3 * (size_t)t->f * t->d, bytes = n * sizeof(float);
  const int fdsc = open(path.c_str(), O_RDONLY);
  if (fdsc < 0) return l2_fail(GMOE_ERR_MODEL, "expert %u: cannot open %s", id, path.c_str());
  struct stat st {};
  if (fstat(fdsc, &st) != 0) {
    close(fdsc);
    return l2_fail(GMOE_ERR_MODEL, "expert %u: cannot stat %s", id, path.c_str());
  }
  if ((size_t)st.st_size != bytes) {
    close(fdsc);
    return l2_fail(GMOE_ERR_MODEL, "expert %u: expected %zu bytes for dims %ux%u, found %lld", id, bytes, t->d, t->f,
                   (long long)st.st_size);
  }
  if (map_it) {
    void* m = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fdsc, 0);
    close(fdsc);
    if (m == MAP_FAILED) return l2_fail(GMOE_ERR_MODEL, "expert %u: cannot map %s", id, path.c_str());
    if (gmoe_status e = check_values(id, static_cast<const float*>(m), n)) {
      munmap(m, bytes);
      return e;
    }
    s.map = m;
    s.map_bytes = bytes;
    s.w = static_cast<const float*>(m);
    return GMOE_OK;
  }
  std::vector<float> v(n);
  size_t got = 0;
  while (got < bytes) {
    const ssize_t r = read(fdsc, reinterpret_cast<char*>(v.data()) + got, bytes - got);
    if (r <= 0) break;
    got += (size_t)r;
  }
  close(fdsc);
  if (got != bytes) return l2_fail(GMOE_ERR_MODEL, "expert %u: short read of %s", id, path.c_str());
  if (gmoe_status e = check_values(id, v.data(), n)) return e;
  s.own.swap(v);
  s.w = s.own.data();
  return GMOE_OK;
}

// MemoryManager::load_uncached (memory/mod.rs:114-146) for expert e of the handle, into
// t->src[e]. Weights handed out before are never freed while the handle lives: a load
// whose bytes are the ones already held (the same L2 file still mapped, or the same
// synthesis) reuses them, and any other replaces them after setting them aside. The
// caller holds t->mu.
gmoe_status load_uncached(gmoe_l2* t, uint32_t e) {
  const uint32_t id = t->id_base + e;
  const size_t n = 3 * (size_t)t->f * t->d;
  const std::string l2path = path_in(t->dir, id);
  auto& s = t->src[e];
  if (exists(l2path)) {
    if (!s.map) {
      gmoe_l2::Src fresh;
      if (gmoe_status r = read_file(t, id, l2path, true, fresh)) return r;
      retire(t, s);
      s = std::move(fresh);
    }
    t->counts.l2++;
    return GMOE_OK;
  }
  if (!t->l3dir.empty()) {
    const std::string l3path = path_in(t->l3dir, id);
    if (exists(l3path)) {
      gmoe_l2::Src fresh;
      if (gmoe_status r = read_file(t, id, l3path, false, fresh)) return r;
      retire(t, s);
      s = std::move(fresh);
      if (write_expert(l2path, s.w, n)) t->counts.promoted++;  // one tier shallower next time
      t->counts.l3++;
      return GMOE_OK;
    }
  }
  // nowhere on disk: synthesise (the same values every time) and materialise into L2
  if (s.map || s.own.size() != n || !s.synth) {
    gmoe_l2::Src fresh;
    fresh.own.resize(n);
    synthesize_expert(id, t->d, t->f, fresh.own.data());
    fresh.w = fresh.own.data();
    fresh.synth = true;
    retire(t, s);
    s = std::move(fresh);
  }
  if (write_expert(l2path, s.w, n)) t->counts.written++;
  t->counts.synthesised++;
  return GMOE_OK;
}

gmoe_status open_tiers(const char* dir, const char* l3dir, uint32_t d_model, uint32_t d_ff, uint32_t n_experts,
                       uint32_t id_base, bool lazy, gmoe_l2** out) {
  if (!dir || !out) return l2_fail(GMOE_ERR_INFERENCE, "null directory or output");
  *out = nullptr;
  if (!d_model || !d_ff || !n_experts) return l2_fail(GMOE_ERR_CONFIG, "d_model, d_ff and n_experts must be non-zero");
  gmoe_l2* t = new gmoe_l2;
  t->dir = dir;
  t->l3dir = l3dir ? l3dir : "";
  t->lazy = lazy;
  t->d = d_model;
  t->f = d_ff;
  t->ne = n_experts;
  t->id_base = id_base;
  t->src.resize(n_experts);
  if (!lazy) {
    const size_t fd = (size_t)d_ff * d_model;
    for (uint32_t e = 0; e < n_experts; e++) {
      if (gmoe_status s = load_uncached(t, e)) {
        release(t);
        return s;
      }
      const float* w = t->src[e].w;
      t->ptr[0].push_back(w);
      t->ptr[1].push_back(w + fd);
      t->ptr[2].push_back(w + 2 * fd);
    }
  }
  *out = t;
  return GMOE_OK;
}

// gmoe_expert_fetch over a handle (gmoe_l2_layer_register)
gmoe_status fetch_cb(void* user, uint32_t expert, const void* weights[3]) {
  return gmoe_l2_fetch(static_cast<gmoe_l2*>(user), expert, weights);
}

}  // namespace

extern "C" {

gmoe_status gmoe_fill_seeded(uint64_t seed, uint64_t n, float b, float* out) {
  if (n && !out) return l2_fail(GMOE_ERR_INFERENCE, "null output");
  seeded(seed, n, b, out);
  return GMOE_OK;
}

gmoe_status gmoe_l2_open(const char* dir, uint32_t d_model, uint32_t d_ff, uint32_t n_experts, uint32_t id_base,
                         gmoe_l2** out) {
  return open_tiers(dir, nullptr, d_model, d_ff, n_experts, id_base, false, out);
}

gmoe_status gmoe_tiers_open(const char* l2_dir, const char* l3_dir, uint32_t d_model, uint32_t d_ff,
                            uint32_t n_experts, uint32_t id_base, gmoe_l2** out) {
  return open_tiers(l2_dir, l3_dir, d_model, d_ff, n_experts, id_base, true, out);
}

gmoe_status gmoe_l2_fetch(gmoe_l2* t, uint32_t expert, const void* weights[3]) {
  if (!t || !weights) return l2_fail(GMOE_ERR_INFERENCE, "null tier or output");
  if (expert >= t->ne)
    return l2_fail(GMOE_ERR_MODEL, "expert %u does not exist (model has %u)", t->id_base + expert,
                   t->id_base + t->ne);
  std::lock_guard<std::mutex> g(t->mu);
  const float* w;
  if (t->lazy) {
    if (gmoe_status s = load_uncached(t, expert)) return s;
    w = t->src[expert].w;
  } else {
    w = t->src[expert].w;  // loaded at open and held
  }
  const size_t fd = (size_t)t->f * t->d;
  weights[0] = w;
  weights[1] = w + fd;
  weights[2] = w + 2 * fd;
  return GMOE_OK;
}

int gmoe_l2_locate(const gmoe_l2* t, uint32_t expert) {
  if (!t || expert >= t->ne) return -1;
  const uint32_t id = t->id_base + expert;
  if (exists(path_in(t->dir, id))) return GMOE_TIER_L2;
  if (!t->l3dir.empty() && exists(path_in(t->l3dir, id))) return GMOE_TIER_L3;
  return GMOE_TIER_SYNTHESISED;
}

void gmoe_l2_close(gmoe_l2* t) {
  if (t) release(t);
}

gmoe_status gmoe_l2_get_counts(const gmoe_l2* t, gmoe_l2_counts* out) {
  if (!t || !out) return l2_fail(GMOE_ERR_INFERENCE, "null tier or output");
  std::lock_guard<std::mutex> g(t->mu);
  *out = t->counts;
  return GMOE_OK;
}

gmoe_status gmoe_l2_layer_desc(const gmoe_l2* t, const float* router, uint32_t top_k, uint32_t gating,
                               uint32_t combine, gmoe_layer_desc* out) {
  if (!t || !router || !out) return l2_fail(GMOE_ERR_INFERENCE, "null tier, router or output");
  if (t->lazy)
    return l2_fail(GMOE_ERR_CONFIG, "a tier from gmoe_tiers_open loads experts on demand: use gmoe_l2_layer_register");
  gmoe_layer_desc& D = *out;
  memset(&D, 0, sizeof D);
  D.d_model = t->d;
  D.d_ff = t->f;
  D.n_experts = t->ne;
  D.top_k = top_k;
  D.gating = gating;
  D.combine = combine;
  D.math = GMOE_MATH_F32;  // simd::matvec over f32 experts (moe/mod.rs:82-90)
  D.router = router;
  gmoe_tensor* T[3] = {&D.gate, &D.up, &D.down};
  for (int p = 0; p < 3; p++) {
    T[p]->qtype = GMOE_F32;
    T[p]->layout = GMOE_LAYOUT_SPLIT;
    T[p]->experts = t->ptr[p].data();
  }
  return GMOE_OK;
}

gmoe_status gmoe_l2_layer_register(gmoe_ctx* ctx, gmoe_l2* t, const float* router, uint32_t top_k, uint32_t gating,
                                   uint32_t combine, uint32_t* layer_id) {
  if (!t || !router || !layer_id) return l2_fail(GMOE_ERR_INFERENCE, "null tier, router or output");
  gmoe_layer_desc D;
  memset(&D, 0, sizeof D);
  D.d_model = t->d;
  D.d_ff = t->f;
  D.n_experts = t->ne;
  D.top_k = top_k;
  D.gating = gating;
  D.combine = combine;
  D.math = GMOE_MATH_F32;  // simd::matvec over f32 experts (moe/mod.rs:82-90)
  D.router = router;
  gmoe_tensor* T[3] = {&D.gate, &D.up, &D.down};
  for (int p = 0; p < 3; p++) {
    T[p]->qtype = GMOE_F32;
    T[p]->layout = GMOE_LAYOUT_SPLIT;
  }
  return gmoe_layer_register_fetch(ctx, &D, fetch_cb, t, layer_id);
}

}  // extern "C"
