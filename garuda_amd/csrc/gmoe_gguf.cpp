// gmoe_gguf.cpp — GGUF checkpoints as the source of the HBM expert slab.
//
// Host code only. A gmoe_gguf handle holds the file (read-only mapping, or a borrowed
// buffer), its parsed header, metadata and tensor descriptors, and the small buffers a
// layer descriptor needs beside the file bytes (per-expert pointer tables of the split
// layout, F16 routers widened to f32). Layer descriptors point straight into the
// mapping: gmoe_layer_register stages experts from there through the pinned
// double-buffered copy path, and re-stages an evicted expert from the same bytes.
//
// The parser follows garuda/src/gguf/mod.rs:247-330 rule for rule: every read is
// bounds-checked, a string's length is checked against the bytes left before anything
// is allocated, an array's count against what the remaining bytes could encode at its
// element type's minimum size (:201-214, :231-244), the header's tensor and key counts
// against 24 and 13 bytes each (:267-277), nesting is capped at depth 8 (:182-185),
// dims at 4 (:295-297), and the data section starts at the next general.alignment
// boundary (:313-321). Error texts follow the reference's.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/garuda_moe.h"
#include "gmoe_internal.h"

namespace gmoe {
void set_last_error(const char* msg);  // gmoe_api.cpp: the thread's gmoe_last_error text
}

namespace {

using gmoe::block_layout;

gmoe_status gfail(gmoe_status s, const char* fmt, ...) {
  char buf[512];
  int n = snprintf(buf, sizeof buf, "gguf: ");
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf + n, sizeof buf - n, fmt, ap);
  va_end(ap);
  gmoe::set_last_error(buf);
  return s;
}

struct Value {
  uint32_t type = 0;
  uint32_t elem = 0;  // arrays
  uint64_t u = 0;     // integers, bool
  double f = 0.0;     // f32, f64
  std::string s;      // strings
  std::vector<Value> items;
};

struct Tensor {
  std::string name;
  uint32_t n_dims = 0, type = 0;
  uint64_t dims[4] = {0, 0, 0, 0};
  uint64_t offset = 0;
  uint64_t n_elements() const {
    uint64_t n = 1;
    for (uint32_t i = 0; i < n_dims; i++) n *= dims[i];
    return n;
  }
};

struct ParseError {
  std::string msg;
};

// gguf/mod.rs:113-245
struct Cursor {
  const uint8_t* buf;
  size_t len, pos = 0;

  const uint8_t* take(uint64_t n) {
    if (n > len - pos) {  // pos <= len always
      char m[128];
      snprintf(m, sizeof m, "truncated: wanted %llu bytes at offset %zu", (unsigned long long)n, pos);
      throw ParseError{m};
    }
    const uint8_t* p = buf + pos;
    pos += n;
    return p;
  }
  uint8_t u8() { return *take(1); }
  uint16_t u16() { uint16_t v; memcpy(&v, take(2), 2); return v; }
  uint32_t u32() { uint32_t v; memcpy(&v, take(4), 4); return v; }
  uint64_t u64() { uint64_t v; memcpy(&v, take(8), 8); return v; }

  std::string string() {
    const uint64_t n = u64();
    if (n > len - pos) {
      char m[160];
      snprintf(m, sizeof m, "string of %llu bytes overruns the %zu-byte file", (unsigned long long)n, len);
      throw ParseError{m};
    }
    const uint8_t* p = take(n);
    if (!valid_utf8(p, n)) throw ParseError{"string is not valid UTF-8"};
    return std::string(reinterpret_cast<const char*>(p), n);
  }

  // Rust's str::from_utf8: shortest forms only, no surrogates, at most U+10FFFF.
  static bool valid_utf8(const uint8_t* p, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
      const uint8_t c = p[i];
      if (c < 0x80) { i++; continue; }
      int k;
      uint32_t lo = 0x80, hi = 0xbf;
      if (c >= 0xc2 && c <= 0xdf) k = 1;
      else if (c == 0xe0) { k = 2; lo = 0xa0; }
      else if ((c >= 0xe1 && c <= 0xec) || c == 0xee || c == 0xef) k = 2;
      else if (c == 0xed) { k = 2; hi = 0x9f; }
      else if (c == 0xf0) { k = 3; lo = 0x90; }
      else if (c >= 0xf1 && c <= 0xf3) k = 3;
      else if (c == 0xf4) { k = 3; hi = 0x8f; }
      else return false;
      if (n - i - 1 < (uint64_t)k) return false;
      if (p[i + 1] < lo || p[i + 1] > hi) return false;
      for (int j = 2; j <= k; j++)
        if (p[i + j] < 0x80 || p[i + j] > 0xbf) return false;
      i += k + 1;
    }
    return true;
  }

  // gguf/mod.rs:227-244: the fewest file bytes one value of a type can take
  static uint64_t min_value_bytes(uint32_t t) {
    switch (t) {
      case 0: case 1: case 7: return 1;
      case 2: case 3: return 2;
      case 4: case 5: case 6: return 4;
      case 8: return 8;
      case 9: return 12;
      case 10: case 11: case 12: return 8;
    }
    return 1;
  }

  // gguf/mod.rs:180-222
  Value value(uint32_t type, int depth) {
    if (depth > 8) throw ParseError{"metadata nests too deeply"};
    Value v;
    v.type = type;
    switch (type) {
      case 0: v.u = u8(); break;
      case 1: v.u = (uint64_t)(int64_t)(int8_t)u8(); break;
      case 2: v.u = u16(); break;
      case 3: v.u = (uint64_t)(int64_t)(int16_t)u16(); break;
      case 4: v.u = u32(); break;
      case 5: v.u = (uint64_t)(int64_t)(int32_t)u32(); break;
      case 6: { uint32_t b = u32(); float x; memcpy(&x, &b, 4); v.f = x; break; }
      case 7: v.u = u8() != 0; break;
      case 8: v.s = string(); break;
      case 9: {
        v.elem = u32();
        const uint64_t n = u64();
        const uint64_t remaining = len - pos, mb = min_value_bytes(v.elem);
        if (n > remaining / mb) {
          char m[160];
          snprintf(m, sizeof m, "array of %llu elements overruns the %zu-byte file", (unsigned long long)n, len);
          throw ParseError{m};
        }
        v.items.reserve(n);  // bounded by the check above
        for (uint64_t i = 0; i < n; i++) v.items.push_back(value(v.elem, depth + 1));
        break;
      }
      case 10: v.u = u64(); break;
      case 11: v.u = u64(); break;
      case 12: { uint64_t b = u64(); memcpy(&v.f, &b, 8); break; }
      default: {
        char m[96];
        snprintf(m, sizeof m, "unknown metadata value type %u", type);
        throw ParseError{m};
      }
    }
    return v;
  }
};

// Value::as_u64 (gguf/mod.rs:36-49): unsigned integers, and signed ones that are >= 0
bool as_u64(const Value& v, uint64_t* out) {
  switch (v.type) {
    case 0: case 2: case 4: case 10: *out = v.u; return true;
    case 1: case 3: case 5: case 11:
      if ((int64_t)v.u < 0) return false;
      *out = v.u;
      return true;
  }
  return false;
}

// The split layout's per-expert pointer tables and the widened routers of the layer
// descriptors handed out, kept until the handle closes.
struct LayerBufs {
  std::vector<const void*> experts[3];
  std::vector<float> router;
};

}  // namespace

struct gmoe_gguf {
  const uint8_t* bytes = nullptr;
  size_t len = 0;
  void* map = nullptr;  // our mapping, or null for a borrowed buffer
  size_t map_len = 0;
  uint32_t version = 0;
  uint64_t n_kv_file = 0;
  std::map<std::string, Value> meta;
  std::vector<Tensor> tensors;
  std::multimap<std::string, size_t> by_name;
  size_t data_offset = 0;
  std::vector<std::unique_ptr<LayerBufs>> descs;  // one per descriptor handed out

  ~gmoe_gguf() {
    if (map) munmap(map, map_len);
  }
};

namespace {

// Gguf::parse, gguf/mod.rs:247-324
gmoe_status parse_into(gmoe_gguf* g) {
  try {
    Cursor c{g->bytes, g->len};
    const uint8_t* magic = c.take(4);
    if (memcmp(magic, "GGUF", 4) != 0) {
      char m[96];
      snprintf(m, sizeof m, "bad magic [%02x, %02x, %02x, %02x], expected [47, 47, 55, 46]", magic[0], magic[1],
               magic[2], magic[3]);
      throw ParseError{m};
    }
    g->version = c.u32();
    if (g->version < 2 || g->version > 3) {
      char m[64];
      snprintf(m, sizeof m, "unsupported version %u", g->version);
      throw ParseError{m};
    }
    const uint64_t n_tensors = c.u64(), n_kv = c.u64();
    const uint64_t remaining = g->len - c.pos;
    if (n_tensors > remaining / 24 || n_kv > remaining / 13) {
      char m[200];
      snprintf(m, sizeof m,
               "header claims %llu tensors and %llu metadata entries, more than the remaining %llu bytes can describe",
               (unsigned long long)n_tensors, (unsigned long long)n_kv, (unsigned long long)remaining);
      throw ParseError{m};
    }
    g->n_kv_file = n_kv;
    for (uint64_t i = 0; i < n_kv; i++) {
      std::string key = c.string();
      const uint32_t t = c.u32();
      g->meta[key] = c.value(t, 0);  // a repeated key keeps its last value, as BTreeMap::insert
    }
    g->tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
      Tensor t;
      t.name = c.string();
      t.n_dims = c.u32();
      if (t.n_dims > 4) {
        std::string m = "tensor '" + t.name + "' claims " + std::to_string(t.n_dims) + " dimensions";
        throw ParseError{m};
      }
      for (uint32_t j = 0; j < t.n_dims; j++) t.dims[j] = c.u64();
      t.type = c.u32();
      t.offset = c.u64();
      g->by_name.emplace(t.name, g->tensors.size());
      g->tensors.push_back(std::move(t));
    }
    uint64_t align = 32;
    auto it = g->meta.find("general.alignment");
    if (it != g->meta.end()) {
      uint64_t a;
      if (as_u64(it->second, &a)) align = a;
    }
    if (align == 0 || (align & (align - 1)) != 0) {
      char m[96];
      snprintf(m, sizeof m, "alignment %llu is not a power of two", (unsigned long long)align);
      throw ParseError{m};
    }
    g->data_offset = (c.pos + align - 1) / align * align;
  } catch (const ParseError& e) {
    return gfail(GMOE_ERR_MODEL, "%s", e.msg.c_str());
  } catch (const std::bad_alloc&) {
    return gfail(GMOE_ERR_MODEL, "out of host memory while parsing");
  }
  return GMOE_OK;
}

// The first tensor named `name` (Gguf::tensor, gguf/mod.rs:393-395: a linear find)
const Tensor* find(const gmoe_gguf* g, const std::string& name) {
  auto it = g->by_name.lower_bound(name);  // equal keys keep insertion order: the first
  return it == g->by_name.end() || it->first != name ? nullptr : &g->tensors[it->second];
}

void fill_value(const Value& v, gmoe_gguf_value* out) {
  out->type = v.type;
  out->elem_type = v.elem;
  out->u = v.u;
  out->f = v.f;
  out->str = v.type == 8 ? v.s.c_str() : nullptr;
  out->len = v.type == 8 ? v.s.size() : v.type == 9 ? v.items.size() : 0;
  out->node = &v;
}

// quant::byte_size for a whole tensor (0: no block layout, or not whole blocks)
uint64_t tensor_bytes(const Tensor& t) {
  uint32_t e, b;
  if (!block_layout(t.type, &e, &b)) return 0;
  const uint64_t n = t.n_elements();
  return n % e ? 0 : n / e * b;
}

// The file bytes of a tensor (start, length) when they lie inside the file.
bool tensor_range(const gmoe_gguf* g, const Tensor& t, uint64_t* start, uint64_t* nbytes) {
  *nbytes = tensor_bytes(t);
  if (*nbytes == 0 && t.n_elements() != 0) return false;
  const uint64_t s = (uint64_t)g->data_offset + t.offset;
  if (s < t.offset) return false;  // overflow
  if (s > g->len || *nbytes > g->len - s) return false;
  *start = s;
  return true;
}

void fill_tensor(const gmoe_gguf* g, const Tensor& t, gmoe_gguf_tensor_info* out) {
  out->name = t.name.c_str();
  out->n_dims = t.n_dims;
  out->qtype = t.type;
  for (int i = 0; i < 4; i++) out->dims[i] = t.dims[i];
  out->offset = t.offset;
  out->n_elements = t.n_elements();
  uint64_t s, nb;
  const bool in = tensor_range(g, t, &s, &nb);
  out->nbytes = tensor_bytes(t);
  out->data = in ? g->bytes + s : nullptr;
}

// {arch}.{suffix} as an integer (Gguf::arch_u64, gguf/mod.rs:368-373)
bool arch_u64(const gmoe_gguf* g, const char* suffix, uint64_t* out) {
  auto a = g->meta.find("general.architecture");
  if (a == g->meta.end() || a->second.type != 8) return false;
  auto it = g->meta.find(a->second.s + "." + suffix);
  return it != g->meta.end() && as_u64(it->second, out);
}

struct MoeDims {
  uint64_t d, f, ne, k, layers;
};

gmoe_status moe_dims(const gmoe_gguf* g, MoeDims* m) {
  auto a = g->meta.find("general.architecture");
  if (a == g->meta.end() || a->second.type != 8) return gfail(GMOE_ERR_MODEL, "no general.architecture");
  const char* arch = a->second.s.c_str();
  struct { const char* key; uint64_t* dst; } need[] = {
      {"embedding_length", &m->d}, {"feed_forward_length", &m->f}, {"block_count", &m->layers}};
  for (auto& n : need)
    if (!arch_u64(g, n.key, n.dst)) return gfail(GMOE_ERR_MODEL, "gguf is missing %s.%s", arch, n.key);
  // LlamaConfig::from_gguf (llama/mod.rs:462-463): absent expert counts are 0, a dense model
  if (!arch_u64(g, "expert_count", &m->ne)) m->ne = 0;
  if (!arch_u64(g, "expert_used_count", &m->k)) m->k = 0;
  if (m->d > UINT32_MAX || m->f > UINT32_MAX || m->ne > UINT32_MAX || m->k > UINT32_MAX)
    return gfail(GMOE_ERR_MODEL, "model dimensions do not fit in 32 bits");
  return GMOE_OK;
}

// load_weight / pinned_weight (llama/mod.rs:320-381): the named tensor, checked to
// hold rows x cols elements whose bytes lie inside the file.
gmoe_status weight(const gmoe_gguf* g, const std::string& name, uint64_t rows, uint64_t cols, const Tensor** out,
                   uint64_t* start) {
  const Tensor* t = find(g, name);
  if (!t) return gfail(GMOE_ERR_MODEL, "tensor '%s' not found", name.c_str());
  if (t->n_elements() != rows * cols)
    return gfail(GMOE_ERR_MODEL, "tensor '%s' has %llu elements, expected %llu", name.c_str(),
                 (unsigned long long)t->n_elements(), (unsigned long long)(rows * cols));
  uint32_t e, b;
  if (!block_layout(t->type, &e, &b))
    return gfail(GMOE_ERR_MODEL, "tensor '%s': type %u is not supported", name.c_str(), t->type);
  uint64_t nb;
  if (!tensor_range(g, *t, start, &nb))
    return gfail(GMOE_ERR_MODEL, "tensor '%s' runs past the end of its buffer", name.c_str());
  *out = t;
  return GMOE_OK;
}

std::string blk(uint32_t l, const char* name) { return "blk." + std::to_string(l) + "." + name + ".weight"; }
std::string blk_e(uint32_t l, const char* name, uint64_t e) {
  return "blk." + std::to_string(l) + "." + name + "." + std::to_string(e) + ".weight";
}

bool stacked_layer(const gmoe_gguf* g, uint32_t l) { return find(g, blk(l, "ffn_gate_exps")) != nullptr; }
bool split_layer(const gmoe_gguf* g, uint32_t l) { return find(g, blk_e(l, "ffn_gate", 0)) != nullptr; }

}  // namespace

extern "C" {

gmoe_status gmoe_gguf_parse(const void* bytes, uint64_t len, gmoe_gguf** out) {
  if (!out) return gfail(GMOE_ERR_INFERENCE, "null output pointer");
  *out = nullptr;
  if (!bytes && len) return gfail(GMOE_ERR_INFERENCE, "null buffer of %llu bytes", (unsigned long long)len);
  std::unique_ptr<gmoe_gguf> g(new (std::nothrow) gmoe_gguf);
  if (!g) return gfail(GMOE_ERR_MODEL, "out of host memory");
  g->bytes = static_cast<const uint8_t*>(bytes);
  g->len = len;
  gmoe_status s = parse_into(g.get());
  if (s != GMOE_OK) return s;
  *out = g.release();
  return GMOE_OK;
}

gmoe_status gmoe_gguf_open(const char* path, gmoe_gguf** out) {
  if (!out) return gfail(GMOE_ERR_INFERENCE, "null output pointer");
  *out = nullptr;
  if (!path) return gfail(GMOE_ERR_INFERENCE, "null path");
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return gfail(GMOE_ERR_MODEL, "cannot open %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    close(fd);
    return gfail(GMOE_ERR_MODEL, "cannot stat %s: %s", path, strerror(e));
  }
  std::unique_ptr<gmoe_gguf> g(new (std::nothrow) gmoe_gguf);
  if (!g) {
    close(fd);
    return gfail(GMOE_ERR_MODEL, "out of host memory");
  }
  if (st.st_size > 0) {
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      const int e = errno;
      close(fd);
      return gfail(GMOE_ERR_MODEL, "cannot map %s: %s", path, strerror(e));
    }
    g->map = m;
    g->map_len = (size_t)st.st_size;
    g->bytes = static_cast<const uint8_t*>(m);
    g->len = (size_t)st.st_size;
  }
  close(fd);  // the mapping keeps the file
  gmoe_status s = parse_into(g.get());
  if (s != GMOE_OK) return s;
  *out = g.release();
  return GMOE_OK;
}

void gmoe_gguf_close(gmoe_gguf* g) { delete g; }

gmoe_status gmoe_gguf_get_header(const gmoe_gguf* g, gmoe_gguf_header* out) {
  if (!g || !out) return gfail(GMOE_ERR_INFERENCE, "null handle or output");
  out->version = g->version;
  out->n_tensors = g->tensors.size();
  out->n_keys = g->meta.size();
  out->data_offset = g->data_offset;
  out->file_bytes = g->len;
  return GMOE_OK;
}

gmoe_status gmoe_gguf_key_at(const gmoe_gguf* g, uint64_t i, const char** key) {
  if (!g || !key) return gfail(GMOE_ERR_INFERENCE, "null handle or output");
  if (i >= g->meta.size()) return gfail(GMOE_ERR_NOT_FOUND, "key index %llu of %zu", (unsigned long long)i, g->meta.size());
  auto it = g->meta.begin();
  std::advance(it, (long)i);
  *key = it->first.c_str();
  return GMOE_OK;
}

gmoe_status gmoe_gguf_get_value(const gmoe_gguf* g, const char* key, gmoe_gguf_value* out) {
  if (!g || !key || !out) return gfail(GMOE_ERR_INFERENCE, "null handle, key or output");
  auto it = g->meta.find(key);
  if (it == g->meta.end()) return gfail(GMOE_ERR_NOT_FOUND, "no metadata key '%s'", key);
  fill_value(it->second, out);
  return GMOE_OK;
}

gmoe_status gmoe_gguf_array_item(const gmoe_gguf* g, const gmoe_gguf_value* array, uint64_t i, gmoe_gguf_value* out) {
  if (!g || !array || !out || !array->node) return gfail(GMOE_ERR_INFERENCE, "null handle, value or output");
  const Value& v = *static_cast<const Value*>(array->node);
  if (v.type != 9) return gfail(GMOE_ERR_INFERENCE, "value is not an array");
  if (i >= v.items.size())
    return gfail(GMOE_ERR_INFERENCE, "index %llu past the %zu elements of the array", (unsigned long long)i,
                 v.items.size());
  fill_value(v.items[i], out);
  return GMOE_OK;
}

gmoe_status gmoe_gguf_tensor_at(const gmoe_gguf* g, uint64_t i, gmoe_gguf_tensor_info* out) {
  if (!g || !out) return gfail(GMOE_ERR_INFERENCE, "null handle or output");
  if (i >= g->tensors.size())
    return gfail(GMOE_ERR_NOT_FOUND, "tensor index %llu of %zu", (unsigned long long)i, g->tensors.size());
  fill_tensor(g, g->tensors[i], out);
  return GMOE_OK;
}

gmoe_status gmoe_gguf_find_tensor(const gmoe_gguf* g, const char* name, gmoe_gguf_tensor_info* out) {
  if (!g || !name || !out) return gfail(GMOE_ERR_INFERENCE, "null handle, name or output");
  const Tensor* t = find(g, name);
  if (!t) return gfail(GMOE_ERR_NOT_FOUND, "tensor '%s' not found", name);
  fill_tensor(g, *t, out);
  return GMOE_OK;
}

}  // extern "C"

namespace {

// Ffn::Dense (llama/mod.rs:608-613, :913-920): "a dense FFN is one expert spanning the
// whole tensor". It is described as one expert, top-1, with a zero router: every gating
// gives that expert weight 1 exactly (a softmax over one logit is 1, a renormalisation
// divides by 1), so the combine adds y * 1 to zero and the layer's output is
// expert_batch's, the dense arm's.
gmoe_status dense_layer_desc(gmoe_gguf* g, const MoeDims& m, uint32_t layer, uint32_t math, gmoe_layer_desc* out) {
  if (!find(g, blk(layer, "ffn_gate")))
    return gfail(GMOE_ERR_MODEL,
                 "layer %u has no feed-forward tensors (blk.%u.ffn_gate_exps, blk.%u.ffn_gate.0 or blk.%u.ffn_gate)",
                 layer, layer, layer, layer);
  auto bufs = std::make_unique<LayerBufs>();
  bufs->router.assign(m.d, 0.0f);
  gmoe_layer_desc D{};
  D.d_model = (uint32_t)m.d;
  D.d_ff = (uint32_t)m.f;
  D.n_experts = 1;
  D.top_k = 1;
  D.gating = GMOE_GATING_LLAMA;
  D.combine = GMOE_COMBINE_EXPERT_ORDER;
  D.math = math;
  D.router = bufs->router.data();
  const char* base[3] = {"ffn_gate", "ffn_up", "ffn_down"};
  const uint64_t rows[3] = {m.f, m.f, m.d}, cols[3] = {m.d, m.d, m.f};
  gmoe_tensor* dst[3] = {&D.gate, &D.up, &D.down};
  for (int w = 0; w < 3; w++) {
    const Tensor* t;
    uint64_t st;
    if (gmoe_status s = weight(g, blk(layer, base[w]), rows[w], cols[w], &t, &st)) return s;
    dst[w]->qtype = t->type;
    dst[w]->layout = GMOE_LAYOUT_STACKED;
    dst[w]->data = g->bytes + st;
    dst[w]->experts = nullptr;
  }
  g->descs.push_back(std::move(bufs));
  *out = D;
  return GMOE_OK;
}

}  // namespace

extern "C" {

gmoe_status gmoe_gguf_layer_desc(gmoe_gguf* g, uint32_t layer, uint32_t gating, uint32_t combine, uint32_t math,
                                 gmoe_layer_desc* out) {
  if (!g || !out) return gfail(GMOE_ERR_INFERENCE, "null handle or output");
  MoeDims m;
  gmoe_status s = moe_dims(g, &m);
  if (s != GMOE_OK) return s;
  if (layer >= m.layers)
    return gfail(GMOE_ERR_INFERENCE, "layer %u of a %llu-layer model", layer, (unsigned long long)m.layers);
  // llama/mod.rs:590-613: MoE when the model declares experts and the block has the
  // stacked or the split expert tensors, else a dense FFN
  const bool stacked = m.ne > 0 && stacked_layer(g, layer);
  if (!stacked && !(m.ne > 0 && split_layer(g, layer))) return dense_layer_desc(g, m, layer, math, out);
  auto bufs = std::make_unique<LayerBufs>();
  gmoe_layer_desc D{};
  D.d_model = (uint32_t)m.d;
  D.d_ff = (uint32_t)m.f;
  D.n_experts = (uint32_t)m.ne;
  D.top_k = (uint32_t)m.k;
  D.gating = gating;
  D.combine = combine;
  D.math = math;

  // router: ffn_gate_inp, [ne x d]
  const Tensor* rt;
  uint64_t rs;
  if ((s = weight(g, blk(layer, "ffn_gate_inp"), m.ne, m.d, &rt, &rs)) != GMOE_OK) return s;
  if (rt->type == gmoe::F32 && rs % 4 == 0) {
    D.router = reinterpret_cast<const float*>(g->bytes + rs);
  } else if (rt->type == gmoe::F32 || rt->type == gmoe::F16) {
    const uint64_t n = m.ne * m.d;
    bufs->router.resize(n);
    if (rt->type == gmoe::F32) {
      memcpy(bufs->router.data(), g->bytes + rs, n * 4);
    } else {
      for (uint64_t i = 0; i < n; i++) {
        uint16_t h;
        memcpy(&h, g->bytes + rs + 2 * i, 2);
        bufs->router[i] = (float)__builtin_bit_cast(_Float16, h);  // exact
      }
    }
    D.router = bufs->router.data();
  } else {
    return gfail(GMOE_ERR_MODEL, "router blk.%u.ffn_gate_inp has type %u; F32 and F16 routers are supported", layer,
                 rt->type);
  }

  // experts: gate/up [f x d], down [d x f] per expert (llama/mod.rs:591-606)
  const char* base[3] = {"ffn_gate", "ffn_up", "ffn_down"};
  const uint64_t rows[3] = {m.f, m.f, m.d}, cols[3] = {m.d, m.d, m.f};
  gmoe_tensor* dst[3] = {&D.gate, &D.up, &D.down};
  for (int w = 0; w < 3; w++) {
    const Tensor* t;
    uint64_t st;
    if (stacked) {
      const std::string name = std::string(base[w]) + "_exps";
      if ((s = weight(g, blk(layer, name.c_str()), m.ne * rows[w], cols[w], &t, &st)) != GMOE_OK) return s;
      dst[w]->qtype = t->type;
      dst[w]->layout = GMOE_LAYOUT_STACKED;
      dst[w]->data = g->bytes + st;
      dst[w]->experts = nullptr;
    } else {
      bufs->experts[w].resize(m.ne);
      uint32_t qt = 0;
      for (uint64_t e = 0; e < m.ne; e++) {
        if ((s = weight(g, blk_e(layer, base[w], e), rows[w], cols[w], &t, &st)) != GMOE_OK) return s;
        if (e == 0) qt = t->type;
        if (t->type != qt)
          return gfail(GMOE_ERR_MODEL, "blk.%u.%s: expert %llu has type %u, expert 0 type %u (one type per matrix)",
                       layer, base[w], (unsigned long long)e, t->type, qt);
        bufs->experts[w][e] = g->bytes + st;
      }
      dst[w]->qtype = qt;
      dst[w]->layout = GMOE_LAYOUT_SPLIT;
      dst[w]->data = nullptr;
      dst[w]->experts = bufs->experts[w].data();
    }
  }
  g->descs.push_back(std::move(bufs));
  *out = D;
  return GMOE_OK;
}

gmoe_status gmoe_gguf_expert_ranges(gmoe_gguf* g, uint32_t layer, uint32_t expert, uint64_t offset[3],
                                    uint64_t length[3]) {
  if (!g || !offset || !length) return gfail(GMOE_ERR_INFERENCE, "null handle or output");
  MoeDims m;
  gmoe_status s = moe_dims(g, &m);
  if (s != GMOE_OK) return s;
  if (layer >= m.layers || expert >= m.ne)
    return gfail(GMOE_ERR_INFERENCE, "layer %u / expert %u outside %llu layers of %llu experts", layer, expert,
                 (unsigned long long)m.layers, (unsigned long long)m.ne);
  const bool stacked = stacked_layer(g, layer);
  if (!stacked && !split_layer(g, layer)) return gfail(GMOE_ERR_MODEL, "layer %u has no expert tensors", layer);
  const char* base[3] = {"ffn_gate", "ffn_up", "ffn_down"};
  const uint64_t rows[3] = {m.f, m.f, m.d}, cols[3] = {m.d, m.d, m.f};
  for (int w = 0; w < 3; w++) {
    const Tensor* t;
    uint64_t st;
    uint32_t e, b;
    if (stacked) {
      const std::string name = std::string(base[w]) + "_exps";
      if ((s = weight(g, blk(layer, name.c_str()), m.ne * rows[w], cols[w], &t, &st)) != GMOE_OK) return s;
      block_layout(t->type, &e, &b);
      if (cols[w] % e) return gfail(GMOE_ERR_MODEL, "rows of %s are not whole blocks", t->name.c_str());
      const uint64_t row_bytes = cols[w] / e * b;
      offset[w] = st + expert * rows[w] * row_bytes;
      length[w] = rows[w] * row_bytes;
    } else {
      if ((s = weight(g, blk_e(layer, base[w], expert), rows[w], cols[w], &t, &st)) != GMOE_OK) return s;
      offset[w] = st;
      length[w] = tensor_bytes(*t);
    }
  }
  return GMOE_OK;
}

}  // extern "C"
