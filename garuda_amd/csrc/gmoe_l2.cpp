// gmoe_l2.cpp — the synthetic engine's expert tiers below the HBM slab.
//
// garuda's MoeEngine pulls each routed expert through MemoryManager
// (garuda/src/memory/mod.rs:114-184): the L1 RAM cache, else the L2 directory's
// `expert_{id}.bin`, else (L3 aside) a deterministic synthesis that is then written to
// L2. Here the L1 tier is the HBM slab; this file is the L2 side feeding it. A file is
// read as weights::expert_from_bytes reads it (weights/mod.rs:123-164): little-endian
// f32, gate [f x d] then up [f x d] then down [d x f], exactly 3*f*d*4 bytes, every value
// finite. An expert with no file is synthesised with weights::synthesize_expert
// (weights/mod.rs:98-109, the splitmix64 stream of :17-35) and written there, as
// MemoryManager::load_uncached does (:138-145); a failed write is not an error, since
// the weights are already held. The files stay mapped while the handle lives, so the
// slab stages an evicted expert again from the same bytes.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/garuda_moe.h"

namespace gmoe {
void set_last_error(const char* msg);
}

struct gmoe_l2 {
  std::string dir;
  uint32_t d = 0, f = 0, ne = 0, id_base = 0;
  struct Src {
    const float* w = nullptr;  // gate | up | down
    void* map = nullptr;       // the mapped file, or null when synthesised
    size_t map_bytes = 0;
    std::vector<float> own;    // synthesised weights
  };
  std::vector<Src> src;
  std::vector<const void*> ptr[3];  // per expert: gate, up, down
  gmoe_l2_counts counts{};
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

void release(gmoe_l2* t) {
  for (auto& s : t->src)
    if (s.map) munmap(s.map, s.map_bytes);
  delete t;
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
  if (!dir || !out) return l2_fail(GMOE_ERR_INFERENCE, "null directory or output");
  *out = nullptr;
  if (!d_model || !d_ff || !n_experts) return l2_fail(GMOE_ERR_CONFIG, "d_model, d_ff and n_experts must be non-zero");
  gmoe_l2* t = new gmoe_l2;
  t->dir = dir;
  t->d = d_model;
  t->f = d_ff;
  t->ne = n_experts;
  t->id_base = id_base;
  t->src.resize(n_experts);
  const size_t fd = (size_t)d_ff * d_model, n = 3 * fd, bytes = n * sizeof(float);
  for (uint32_t e = 0; e < n_experts; e++) {
    const uint32_t id = id_base + e;
    const std::string path = t->dir + "/expert_" + std::to_string(id) + ".bin";
    auto& s = t->src[e];
    const int fdsc = open(path.c_str(), O_RDONLY);
    if (fdsc >= 0) {  // weights::expert_from_bytes
      struct stat st {};
      if (fstat(fdsc, &st) != 0) {
        close(fdsc);
        release(t);
        return l2_fail(GMOE_ERR_MODEL, "expert %u: cannot stat %s", id, path.c_str());
      }
      if ((size_t)st.st_size != bytes) {
        close(fdsc);
        release(t);
        return l2_fail(GMOE_ERR_MODEL, "expert %u: expected %zu bytes for dims %ux%u, found %lld", id, bytes, d_model,
                       d_ff, (long long)st.st_size);
      }
      void* m = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fdsc, 0);
      close(fdsc);
      if (m == MAP_FAILED) {
        release(t);
        return l2_fail(GMOE_ERR_MODEL, "expert %u: cannot map %s", id, path.c_str());
      }
      s.map = m;
      s.map_bytes = bytes;
      s.w = static_cast<const float*>(m);
      for (size_t i = 0; i < n; i++)
        if (!std::isfinite(s.w[i])) {
          release(t);
          return l2_fail(GMOE_ERR_MODEL, "expert %u: non-finite weight at index %zu", id, i);
        }
      t->counts.l2++;
    } else {  // nowhere on disk: synthesise and materialise into L2
      s.own.resize(n);
      synthesize_expert(id, d_model, d_ff, s.own.data());
      s.w = s.own.data();
      if (write_expert(path, s.w, n)) t->counts.written++;
      t->counts.synthesised++;
    }
    t->ptr[0].push_back(s.w);
    t->ptr[1].push_back(s.w + fd);
    t->ptr[2].push_back(s.w + 2 * fd);
  }
  *out = t;
  return GMOE_OK;
}

void gmoe_l2_close(gmoe_l2* t) {
  if (t) release(t);
}

gmoe_status gmoe_l2_get_counts(const gmoe_l2* t, gmoe_l2_counts* out) {
  if (!t || !out) return l2_fail(GMOE_ERR_INFERENCE, "null tier or output");
  *out = t->counts;
  return GMOE_OK;
}

gmoe_status gmoe_l2_layer_desc(const gmoe_l2* t, const float* router, uint32_t top_k, uint32_t gating,
                               uint32_t combine, gmoe_layer_desc* out) {
  if (!t || !router || !out) return l2_fail(GMOE_ERR_INFERENCE, "null tier, router or output");
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

}  // extern "C"
