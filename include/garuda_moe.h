/*
 * garuda_moe.h — C-ABI of the MI355X mixture-of-experts feed-forward path.
 *
 * Drop-in boundary for Garuda's MoE FFN (hanumanit/garuda 0.31.0). The library
 * replaces the body of `LlamaBackend::feed_forward_batch` for `Ffn::Moe`
 * (garuda/src/llama/mod.rs:922-997): routing, token->expert dispatch, the
 * SwiGLU expert products on still-packed GGUF blocks, and the gate-weighted
 * combine. Everything else in `logits_batch` (llama/mod.rs:1134-1202) stays on
 * the caller's side, so the plugin contract of `core::InferenceBackend`
 * (garuda/src/core/mod.rs:232-348) is unchanged.
 *
 * Plain C types only. The caller owns every host pointer it passes; the library
 * owns device memory (the HBM expert slab and per-context scratch). Every entry
 * point validates its arguments before touching the device, returns a status and
 * never aborts; a refused call changes nothing (llama/mod.rs:1160-1172).
 * gmoe_last_error() returns the calling thread's message for the last failure.
 */
#ifndef GARUDA_MOE_H
#define GARUDA_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GMOE_ABI_VERSION 6u

/* Status codes. Mirrors the GarudaError variants the reference returns on this
 * path (garuda/src/core/mod.rs:10-47). */
typedef enum gmoe_status {
  GMOE_OK = 0,
  GMOE_ERR_MODEL = 1,     /* GarudaError::Model: unsupported ggml type, byte-length mismatch */
  GMOE_ERR_INFERENCE = 2, /* GarudaError::Inference: n/d mismatch, unknown layer */
  GMOE_ERR_CACHE = 3,     /* GarudaError::Cache: the HBM slab cannot hold what is asked */
  GMOE_ERR_CONFIG = 4,    /* GarudaError::Config: top_k outside 1..=n_experts (core/mod.rs:103-108) */
  GMOE_ERR_DEVICE = 5,    /* HIP runtime failure; the context stays usable for teardown */
  GMOE_ERR_NOT_FOUND = 6, /* no such GGUF metadata key or tensor (the reference's `None`) */
  GMOE_ERR_INVALID_TOKEN = 7 /* GarudaError::InvalidToken: a token outside the vocabulary */
} gmoe_status;

/* ggml type ids (garuda/src/quant/mod.rs:22-30). */
enum {
  GMOE_F32 = 0, GMOE_F16 = 1, GMOE_Q4_0 = 2, GMOE_Q8_0 = 8, GMOE_Q2_K = 10,
  GMOE_Q3_K = 11, GMOE_Q4_K = 12, GMOE_Q5_K = 13, GMOE_Q6_K = 14
};

/* Gating rule. LLAMA is feed_forward_batch's own (llama/mod.rs:938-949: softmax over
 * all experts, stable sort, top-k, renormalise). The other three are
 * router::RouterType (garuda/src/router/mod.rs:17-37, :58-118). */
enum {
  GMOE_GATING_LLAMA = 0, GMOE_GATING_MIXTRAL = 1, GMOE_GATING_DEEPSEEK = 2, GMOE_GATING_QWEN = 3
};

/* Order of the weighted sum over a token's experts: ascending expert id
 * (llama/mod.rs:977-995) or routed rank (moe/mod.rs:104-109). */
enum { GMOE_COMBINE_EXPERT_ORDER = 0, GMOE_COMBINE_RANK_ORDER = 1 };

/* Arithmetic of the expert products. PACKED is Weight::Packed under `mmap = true`
 * (llama/mod.rs:175-193 -> quant::matmul, quant/mod.rs:223-304): activations are
 * quantised to int8 per 32 and dotted with the packed rows for Q8_0 and Q2_K..Q6_K;
 * Q4_0/F16/F32 dequantise. F32 is Weight::Full under `mmap = false`
 * (llama/mod.rs:376-381 -> simd::matmul): every weight is the exact dequantised f32. */
enum { GMOE_MATH_PACKED = 0, GMOE_MATH_F32 = 1 };

/* Expert tensor layout (llama/mod.rs:223-226): one stacked `..._exps` tensor with
 * expert e at rows [e*rows, (e+1)*rows), or one tensor per expert. */
enum { GMOE_LAYOUT_STACKED = 0, GMOE_LAYOUT_SPLIT = 1 };

typedef struct gmoe_ctx gmoe_ctx;

typedef struct gmoe_tensor {
  uint32_t qtype;               /* ggml type id */
  uint32_t layout;              /* GMOE_LAYOUT_* */
  const void* data;             /* STACKED: n_experts*rows packed rows */
  const void* const* experts;   /* SPLIT: n_experts pointers, each `rows` packed rows */
} gmoe_tensor;

/* One MoE FFN layer: the `Ffn::Moe` arm of llama/mod.rs:495-507. gate/up are
 * [d_ff x d_model] per expert, down is [d_model x d_ff] (core/mod.rs:181-184). */
typedef struct gmoe_layer_desc {
  uint32_t d_model, d_ff, n_experts, top_k;
  uint32_t gating, combine, math;
  const float* router;          /* ffn_gate_inp, [n_experts x d_model] f32 row-major */
  gmoe_tensor gate, up, down;
} gmoe_layer_desc;

typedef struct gmoe_slab_stats {
  uint64_t hits, misses, evictions; /* as cache::CacheStats (cache/mod.rs:34-40) */
  uint64_t entries, bytes, capacity;
  uint64_t h2d_bytes;               /* bytes staged host->HBM since init */
} gmoe_slab_stats;

/* ---- context ---- */

/* Open device `device` and reserve an HBM slab of `slab_bytes` for packed experts
 * (the L1 tier; cache::ExpertCache's byte budget, cache/mod.rs:18-22). */
gmoe_status gmoe_init(int device, uint64_t slab_bytes, gmoe_ctx** out);
void gmoe_shutdown(gmoe_ctx* ctx);
const char* gmoe_last_error(void);
/* The token id of the calling thread's last GMOE_ERR_INVALID_TOKEN, the Token that
 * GarudaError::InvalidToken carries (garuda/src/core/mod.rs:33-34); UINT32_MAX if none. */
uint32_t gmoe_last_invalid_token(void);
uint32_t gmoe_abi_version(void);

/* Register a layer. Validates dims and byte lengths (quant::byte_size,
 * quant/mod.rs:89-98), copies the router to HBM and stages as many experts into
 * the slab as fit (least recently used first out). The host expert bytes are
 * borrowed: they must stay valid until gmoe_layer_release, because an evicted
 * expert is staged again from them. */
gmoe_status gmoe_layer_register(gmoe_ctx* ctx, const gmoe_layer_desc* desc, uint32_t* layer_id);
gmoe_status gmoe_layer_release(gmoe_ctx* ctx, uint32_t layer_id);

/* The expert loader under the slab (core::ExpertLoader::load on an L1 miss,
 * core/mod.rs:215-223; MemoryManager::load_uncached, memory/mod.rs:114-146): fills
 * weights[0..2] with expert `expert`'s gate, up and down bytes in the descriptor's types,
 * row-major as in a split tensor, valid until the same expert is fetched again or the
 * source closes. A non-zero status fails the call that needed the expert. */
typedef gmoe_status (*gmoe_expert_fetch)(void* user, uint32_t expert, const void* weights[3]);
/* Register a layer whose experts come from `fetch` each time one is staged into the slab
 * (first routing, or again after an eviction). The descriptor's dims, types and router are
 * used as gmoe_layer_register uses them; its tensors' data and expert pointers are not
 * read, and nothing is staged until an expert is routed, prefetched or asked for. `user`
 * must stay valid until gmoe_layer_release. */
gmoe_status gmoe_layer_register_fetch(gmoe_ctx* ctx, const gmoe_layer_desc* desc, gmoe_expert_fetch fetch,
                                      void* user, uint32_t* layer_id);

/* ---- the hot path ---- */

/* feed_forward_batch for n tokens: hs is [n x d_model] (vector-major), out the same.
 * routed_ids/routed_w (may be NULL) receive each token's top_k experts in ranked
 * order, the ids the advisory predictor consumes (llama/mod.rs:951-962).
 * Synchronous; host pointers. */
gmoe_status gmoe_ffn_forward(gmoe_ctx* ctx, uint32_t layer_id, const float* hs, uint32_t n,
                             float* out, uint32_t* routed_ids, float* routed_w);

/* As gmoe_ffn_forward, with precomputed router logits [n x n_experts] in place of
 * the router matvec (llama/mod.rs:939). */
gmoe_status gmoe_ffn_forward_logits(gmoe_ctx* ctx, uint32_t layer_id, const float* hs,
                                    const float* logits, uint32_t n, float* out,
                                    uint32_t* routed_ids, float* routed_w);

/* Device-pointer form: every pointer is device memory, work is queued on `stream`
 * (a hipStream_t; NULL = the context's own stream) and the call returns without
 * waiting. Requires every expert of the layer to be resident (GMOE_ERR_CACHE
 * otherwise). Calls on one context share its scratch, so they must be ordered on
 * one stream. d_logits may be NULL. d_out may equal d_hs (the output overwrites the
 * input); otherwise the output must not overlap an input. */
gmoe_status gmoe_ffn_forward_async(gmoe_ctx* ctx, uint32_t layer_id, const float* d_hs,
                                   const float* d_logits, uint32_t n, float* d_out,
                                   uint32_t* d_routed_ids, float* d_routed_w, void* stream);

/* gmoe_ffn_forward_async without any allocation. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory during a call (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Its
 * scratch is a static device array of 64 MiB per GPU, set up when the library's first
 * context on that GPU opens and held until the process ends; no call allocates or frees.
 * A call whose scratch would exceed it is refused with GMOE_ERR_INFERENCE before any
 * device work (a Mixtral-shape layer, d 4096 / f 14336 / 8 experts, fits every batch of
 * up to 53 tokens; the 128-expert C4 layer fits 64). Every call on one GPU, from every
 * context and on every stream, shares that array: each call's stream waits (an event, no
 * allocation) until the previous call on the GPU has finished with it, so calls never
 * overlap on the array. A call made under stream capture does not take part in that
 * ordering (its graph's launches are ordered by the caller): two graphs holding such calls
 * must not run at the same time. Same arguments and results as gmoe_ffn_forward_async. */
gmoe_status gmoe_ffn_forward_noalloc(gmoe_ctx* ctx, uint32_t layer_id, const float* d_hs,
                                     const float* d_logits, uint32_t n, float* d_out,
                                     uint32_t* d_routed_ids, float* d_routed_w, void* stream);

/* ---- the L1 tier (core::ExpertLoader, core/mod.rs:215-223) ---- */
/* ExpertLoader::prefetch: stage the expert now (returns when it is resident). */
gmoe_status gmoe_expert_prefetch(gmoe_ctx* ctx, uint32_t layer_id, uint32_t expert);
int gmoe_expert_is_resident(gmoe_ctx* ctx, uint32_t layer_id, uint32_t expert);
/* ExpertLoader::unload: an expert queued for staging leaves the queue; one being staged
 * is waited for, then evicted. */
gmoe_status gmoe_expert_evict(gmoe_ctx* ctx, uint32_t layer_id, uint32_t expert);
gmoe_status gmoe_slab_get_stats(gmoe_ctx* ctx, gmoe_slab_stats* out);

/* Where an expert is on its way into the slab: gmoe_prefetch_step queues experts for the
 * context's staging thread, which stages them one at a time (PrefetchEngine::warm's
 * in-flight set and pool, prefetch/mod.rs:102-127). A forward that routes to a queued
 * expert takes it off the queue and stages it itself; one that routes to an expert being
 * staged waits for it. */
enum { GMOE_EXPERT_ABSENT = 0, GMOE_EXPERT_QUEUED = 1, GMOE_EXPERT_STAGING = 2, GMOE_EXPERT_RESIDENT = 3 };
int gmoe_expert_state(gmoe_ctx* ctx, uint32_t layer_id, uint32_t expert);
/* hold != 0: the staging thread starts no new expert (the one it is copying finishes);
 * queued experts stay queued until hold is lifted or a forward takes them. */
gmoe_status gmoe_prefetch_hold(gmoe_ctx* ctx, int hold);
/* Returns once the staging thread is idle: nothing being staged and, unless held, nothing
 * queued. */
gmoe_status gmoe_prefetch_wait(gmoe_ctx* ctx);

/* ---- dense projections (Weight::matmul_rows, llama/mod.rs:148-195) ----
 *
 * The attention projections and the output head (llama/mod.rs:743-757, :880, :1198,
 * :1240) through the expert kernels: a packed rows x cols matrix, tiled into device
 * memory of its own (outside the expert slab, never evicted). PACKED math quantises the
 * activations per 32 and dots them as quant::matmul does (quant/mod.rs:223-304); F32
 * math uses the exact dequantised weights (simd::matmul), on MFMA for prefill-sized
 * calls. A row's dot may be split over K and its slices added in order, so results
 * match the reference within the layer tolerance rather than bit for bit. */
typedef struct gmoe_dense_desc {
  uint32_t rows, cols;          /* out_features x in_features */
  uint32_t qtype, math;         /* ggml type id; GMOE_MATH_* */
  const void* data;             /* rows packed rows, quant::byte_size(qtype, cols) bytes each;
                                   copied during the call */
} gmoe_dense_desc;

gmoe_status gmoe_dense_register(gmoe_ctx* ctx, const gmoe_dense_desc* desc, uint32_t* dense_id);
gmoe_status gmoe_dense_release(gmoe_ctx* ctx, uint32_t dense_id);
/* Weight::matmul_rows(0, xs, n, out): xs [n x cols] -> out [n x rows], vector-major.
 * Synchronous; host pointers. */
gmoe_status gmoe_dense_forward(gmoe_ctx* ctx, uint32_t dense_id, const float* xs, uint32_t n, float* out);
/* Device-pointer form on `stream` (NULL: the context's stream); returns without waiting.
 * Shares the context's scratch with the layer calls: order them on one stream. */
gmoe_status gmoe_dense_forward_async(gmoe_ctx* ctx, uint32_t dense_id, const float* d_xs, uint32_t n,
                                     float* d_out, void* stream);
/* gmoe_dense_forward_async without its last step, the in-order sum of the K slices, for a
 * caller whose next launch adds them itself (the model step folds them into rope/append
 * and into the feed-forward's residual add). Writes *nsl <= GMOE_DENSE_MAX_SLICES slices
 * of [n x rows] to d_parts (slice s of row t at d_parts + (s * n + t) * rows; the caller
 * provides GMOE_DENSE_MAX_SLICES * n * rows floats); parts[0] + parts[1] + ... in that
 * order is gmoe_dense_forward_async's output bit for bit. No counterpart in the reference,
 * whose matmul_rows returns the finished rows; this is the split the model step uses. */
#define GMOE_DENSE_MAX_SLICES 8
gmoe_status gmoe_dense_forward_slices_async(gmoe_ctx* ctx, uint32_t dense_id, const float* d_xs, uint32_t n,
                                            float* d_parts, uint32_t* nsl, void* stream);

/* ---- GGUF checkpoints: the slab's source (garuda/src/gguf/mod.rs; llama/mod.rs:551-637) ----
 *
 * A parsed GGUF file: header, metadata and tensor descriptors, with the reference's
 * bounds rules (gguf/mod.rs:247-330): every length is checked against the bytes that
 * remain, counts are bounded by what those bytes could describe, so a malformed file
 * is an error (GMOE_ERR_MODEL, message prefixed "gguf: ") and never a crash or an
 * outsized allocation. Pure host code: no device, no context. */
typedef struct gmoe_gguf gmoe_gguf;

/* Metadata value types, as the file stores them (gguf/mod.rs:181-221). */
enum {
  GMOE_GGUF_U8 = 0, GMOE_GGUF_I8 = 1, GMOE_GGUF_U16 = 2, GMOE_GGUF_I16 = 3, GMOE_GGUF_U32 = 4,
  GMOE_GGUF_I32 = 5, GMOE_GGUF_F32 = 6, GMOE_GGUF_BOOL = 7, GMOE_GGUF_STRING = 8,
  GMOE_GGUF_ARRAY = 9, GMOE_GGUF_U64 = 10, GMOE_GGUF_I64 = 11, GMOE_GGUF_F64 = 12
};

typedef struct gmoe_gguf_header {
  uint32_t version;      /* 2 or 3 */
  uint64_t n_tensors;    /* tensor descriptors, in file order */
  uint64_t n_keys;       /* distinct metadata keys (a repeated key keeps its last value) */
  uint64_t data_offset;  /* start of the tensor data: the descriptors' end rounded up to
                            general.alignment (32 by default), Gguf::data_offset */
  uint64_t file_bytes;
} gmoe_gguf_header;

typedef struct gmoe_gguf_value {
  uint32_t type;         /* GMOE_GGUF_* */
  uint32_t elem_type;    /* ARRAY: the element type */
  uint64_t u;            /* integer types and BOOL: the value (signed ones sign-extended) */
  double f;              /* F32, F64 */
  const char* str;       /* STRING: the bytes, NUL-terminated, valid until gmoe_gguf_close */
  uint64_t len;          /* STRING: byte length; ARRAY: element count */
  const void* node;      /* the value inside the handle (for gmoe_gguf_array_item) */
} gmoe_gguf_value;

typedef struct gmoe_gguf_tensor_info {
  const char* name;      /* valid until gmoe_gguf_close */
  uint32_t n_dims;       /* 0..4 */
  uint32_t qtype;        /* raw ggml type id */
  uint64_t dims[4];      /* ggml order: dims[0] is the row length */
  uint64_t offset;       /* from the start of the tensor data (TensorInfo::offset) */
  uint64_t n_elements;
  uint64_t nbytes;       /* quant::byte_size of the tensor; 0 for a type this library has no
                            block layout for */
  const void* data;      /* its bytes inside the file; NULL when they run past the end */
} gmoe_gguf_tensor_info;

/* Map `path` read-only and parse it (Gguf::parse over the mapping). */
gmoe_status gmoe_gguf_open(const char* path, gmoe_gguf** out);
/* Parse `len` bytes at `bytes`, borrowed until gmoe_gguf_close. */
gmoe_status gmoe_gguf_parse(const void* bytes, uint64_t len, gmoe_gguf** out);
void gmoe_gguf_close(gmoe_gguf* g);
gmoe_status gmoe_gguf_get_header(const gmoe_gguf* g, gmoe_gguf_header* out);
/* The i-th metadata key in byte order (the reference's BTreeMap order). */
gmoe_status gmoe_gguf_key_at(const gmoe_gguf* g, uint64_t i, const char** key);
/* A metadata value keyed exactly (Gguf::get); GMOE_ERR_NOT_FOUND if absent. */
gmoe_status gmoe_gguf_get_value(const gmoe_gguf* g, const char* key, gmoe_gguf_value* out);
/* Element i of an ARRAY value read from the same handle (nested arrays to any depth). */
gmoe_status gmoe_gguf_array_item(const gmoe_gguf* g, const gmoe_gguf_value* array, uint64_t i,
                                 gmoe_gguf_value* out);
gmoe_status gmoe_gguf_tensor_at(const gmoe_gguf* g, uint64_t i, gmoe_gguf_tensor_info* out);
/* The first tensor named `name` (Gguf::tensor); GMOE_ERR_NOT_FOUND if none. */
gmoe_status gmoe_gguf_find_tensor(const gmoe_gguf* g, const char* name, gmoe_gguf_tensor_info* out);

/* The MoE layer `layer` of the checkpoint as a layer descriptor, as
 * LlamaBackend::from_gguf reads it (llama/mod.rs:569-607, load_weight :358-381,
 * pinned_weight :320-350): dimensions from {arch}.embedding_length,
 * .feed_forward_length, .expert_count, .expert_used_count and .block_count; the
 * stacked blk.L.ffn_{gate,up,down}_exps tensors when present, else the split
 * blk.L.ffn_{gate,up,down}.E tensors; router blk.L.ffn_gate_inp (F32, or F16 widened
 * exactly). Element counts and byte ranges are checked. The descriptor's pointers
 * point into the file (or into buffers the handle owns) and stay valid until
 * gmoe_gguf_close, so a layer registered from it must be released first. */
gmoe_status gmoe_gguf_layer_desc(gmoe_gguf* g, uint32_t layer, uint32_t gating, uint32_t combine,
                                 uint32_t math, gmoe_layer_desc* out);
/* File byte ranges of expert `expert`'s gate, up and down weights in layer `layer`
 * (ExpertWeight::byte_range, llama/mod.rs:250-269; expert_page_ranges :664-682). */
gmoe_status gmoe_gguf_expert_ranges(gmoe_gguf* g, uint32_t layer, uint32_t expert, uint64_t offset[3],
                                    uint64_t length[3]);

/* ---- the synthetic engine's expert tiers (memory/mod.rs:114-184, weights/mod.rs:17-164) ----
 *
 * garuda's MoeEngine (moe/mod.rs:67-112) pulls each routed expert through MemoryManager:
 * the L1 cache, else `expert_{id}.bin` in the L2 directory, else the same file in the L3
 * directory (promoted into L2), else a deterministic synthesis written to L2. Here the
 * HBM slab is L1 and a gmoe_l2 handle is the L2/L3 side. Each file is read as
 * weights::expert_from_bytes reads it: little-endian f32, gate [f x d], up [f x d], down
 * [d x f], exactly 3*f*d*4 bytes, every value finite (GMOE_ERR_MODEL with the reference's
 * message otherwise). An expert with no file is synthesised as weights::synthesize_expert
 * does and written to L2; a failed write or promotion is not an error (the weights are
 * held). Host code. */
typedef struct gmoe_l2 gmoe_l2;
typedef struct gmoe_l2_counts {
  uint64_t l2;           /* loads from an L2 file (TierCounts::l2) */
  uint64_t synthesised;  /* experts synthesised (TierCounts::synthesised) */
  uint64_t written;      /* synthesised experts materialised into L2 */
  uint64_t l3;           /* loads from an L3 file (TierCounts::l3) */
  uint64_t promoted;     /* L3 loads copied into L2 */
} gmoe_l2_counts;
/* MemoryTier below L1 (memory/mod.rs:17-24, locate :99-111): where a load would find it */
enum { GMOE_TIER_L2 = 1, GMOE_TIER_L3 = 2, GMOE_TIER_SYNTHESISED = 3 };

/* weights::seeded (weights/mod.rs:26-35): n values uniform in [-bound, bound] from the
 * splitmix64 stream of `seed`; the engine's shared weights use it with bound(fan_in) =
 * 1 / sqrt(fan_in) (:38-40) and the seeds of :43-51. */
gmoe_status gmoe_fill_seeded(uint64_t seed, uint64_t n, float bound, float* out);
/* Experts id_base .. id_base + n_experts - 1 of the directory `dir` (expert e of the layer
 * is file expert_{id_base + e}.bin). */
/* Every expert is loaded at open (the files stay mapped while the handle lives). */
gmoe_status gmoe_l2_open(const char* dir, uint32_t d_model, uint32_t d_ff, uint32_t n_experts, uint32_t id_base,
                         gmoe_l2** out);
/* MemoryManager::new with an L2 directory and an optional L3 one (l3_dir may be NULL:
 * no L3 tier): nothing is loaded at open; each gmoe_l2_fetch is one load_uncached. */
gmoe_status gmoe_tiers_open(const char* l2_dir, const char* l3_dir, uint32_t d_model, uint32_t d_ff,
                            uint32_t n_experts, uint32_t id_base, gmoe_l2** out);
void gmoe_l2_close(gmoe_l2* l2);
gmoe_status gmoe_l2_get_counts(const gmoe_l2* l2, gmoe_l2_counts* out);
/* MemoryManager::load_uncached (memory/mod.rs:114-146) for expert `expert` of the handle:
 * an L2 file, else an L3 file (written into L2), else a synthesis (written into L2),
 * counted per load. weights[0..2] receive its gate, up and down f32 values, valid until
 * the expert is fetched again or the handle closes. An expert outside the handle is
 * GMOE_ERR_MODEL, as ExpertLoader::load refuses it (:151-157). Thread-safe: concurrent
 * fetches of one expert load it one after another, so it is synthesised once. */
gmoe_status gmoe_l2_fetch(gmoe_l2* l2, uint32_t expert, const void* weights[3]);
/* MemoryManager::locate below L1: GMOE_TIER_L2, _L3 or _SYNTHESISED; -1 outside the handle */
int gmoe_l2_locate(const gmoe_l2* l2, uint32_t expert);
/* The tier's experts as a layer descriptor: split F32 tensors pointing into the handle
 * (valid until gmoe_l2_close, so a layer registered from it is released first), the
 * given router [n_experts x d_model], top_k, gating (the engine's Router types: MIXTRAL,
 * DEEPSEEK, QWEN) and combine order (the engine's is RANK_ORDER, moe/mod.rs:104-109),
 * math F32 (simd::matvec, moe/mod.rs:82-90). For a handle from gmoe_l2_open only. */
gmoe_status gmoe_l2_layer_desc(const gmoe_l2* l2, const float* router, uint32_t top_k, uint32_t gating,
                               uint32_t combine, gmoe_layer_desc* out);
/* The same layer registered with its experts fetched from the tiers when staged
 * (gmoe_layer_register_fetch over gmoe_l2_fetch): MoeEngine's lazy loads, an eviction
 * followed by a reload from L2. Any handle; it must outlive the layer. */
gmoe_status gmoe_l2_layer_register(gmoe_ctx* ctx, gmoe_l2* l2, const float* router, uint32_t top_k,
                                   uint32_t gating, uint32_t combine, uint32_t* layer_id);

/* ---- decode attention over a paged KV cache (llama/mod.rs:766-821, cache/mod.rs:143-600) ----
 *
 * A pool of device pages, each `block_size` positions of keys then values (f32, kv_dim =
 * n_kv_heads * head_dim wide), shared by every sequence and layer; each (sequence,
 * layer) has its own length and page table, as KVCacheState does per layer. An
 * attention call takes one token per entry (several entries of one sequence are its
 * consecutive positions, in order), rotates q and k by the token's position (simd::rope),
 * appends k and v, and attends over [start, position]: start is 0, or position + 1 -
 * sliding_window when a window is set (KVCacheState::attention_start). The context
 * window is max_positions; a call that would exceed it, or find no free page, is
 * refused before any device work (GarudaError::Cache). Spill to storage is not done: the
 * pool lives in HBM. */
typedef struct gmoe_kv gmoe_kv;
typedef struct gmoe_kv_desc {
  uint32_t n_layers, n_heads, n_kv_heads, head_dim;  /* head_dim even, <= 256; n_heads a multiple
                                                        of n_kv_heads, at most 16 per kv head */
  uint32_t block_size;      /* positions per page */
  uint32_t max_positions;   /* context window of a sequence */
  uint32_t sliding_window;  /* 0: attend to every earlier position */
  uint32_t max_seqs;        /* sequences open at once */
  uint64_t max_pages;       /* pages in the pool, over all sequences and layers */
  float rope_theta;
} gmoe_kv_desc;

gmoe_status gmoe_kv_create(gmoe_ctx* ctx, const gmoe_kv_desc* desc, gmoe_kv** out);
void gmoe_kv_destroy(gmoe_kv* kv);
gmoe_status gmoe_kv_seq_open(gmoe_kv* kv, uint32_t* seq);
/* Frees the sequence's pages (after queued device work has finished). */
gmoe_status gmoe_kv_seq_close(gmoe_kv* kv, uint32_t seq);
gmoe_status gmoe_kv_seq_len(const gmoe_kv* kv, uint32_t seq, uint32_t layer, uint32_t* len);
/* Pages of the pool no sequence holds (CacheStats-like accounting of the paged pool). */
gmoe_status gmoe_kv_free_pages(gmoe_kv* kv, uint64_t* pages);
/* Test entry (no counterpart in the reference): the next `count` reservations of attention
 * scratch for graph-replayed model steps fail with GMOE_ERR_DEVICE, as a failed device
 * allocation would, so that tests can check a failed step leaves every sequence as it was. */
gmoe_status gmoe_kv_fail_reserves(gmoe_kv* kv, uint32_t count);
/* Attention for n tokens in layer `layer`: q [n x n_heads*head_dim], k and v
 * [n x kv_dim] (projected, not yet rotated), context [n x n_heads*head_dim] out.
 * Synchronous; host pointers. */
gmoe_status gmoe_attention(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, const float* q,
                           const float* k, const float* v, float* context);
/* Device-pointer form on `stream` (NULL: the context's stream). Calls on one KV cache
 * must be ordered on one stream. */
gmoe_status gmoe_attention_async(gmoe_kv* kv, uint32_t layer, const uint32_t* seqs, uint32_t n, const float* d_q,
                                 const float* d_k, const float* d_v, float* d_context, void* stream);

/* ---- expert prediction and prefetch into the slab (predictor/mod.rs, prefetch/mod.rs) ----
 *
 * The reference's ExpertPredictor (predictor/mod.rs:15-134): a first-order Markov model,
 * transition counts C[prev][next] over global expert ids (layer * n_experts + expert),
 * saturating at 2^32 - 1. predict(current, k) ranks every q by sum over p in current of
 * C[p][q], keeps positive scores, orders them by score then id, and returns the first k;
 * cold, it returns nothing. Host code; thread-safe (one writer or many readers). */
typedef struct gmoe_predictor gmoe_predictor;
typedef struct gmoe_predict_stats {
  uint64_t correct, wasted, missed;  /* PredictStats (predictor/mod.rs:22-30) */
} gmoe_predict_stats;

gmoe_status gmoe_predictor_create(uint32_t n_experts, gmoe_predictor** out);  /* n_experts 0 acts as 1 */
void gmoe_predictor_destroy(gmoe_predictor* p);
/* ExpertPredictor::observe: every prev -> next pair counts once; ids >= n_experts are ignored. */
gmoe_status gmoe_predictor_observe(gmoe_predictor* p, const uint32_t* prev, uint32_t n_prev, const uint32_t* next,
                                   uint32_t n_next);
/* ExpertPredictor::predict: up to k ids into out (capacity k); *n_out receives the count. */
gmoe_status gmoe_predictor_predict(const gmoe_predictor* p, const uint32_t* current, uint32_t n_current,
                                   uint32_t k, uint32_t* out, uint32_t* n_out);
/* ExpertPredictor::score: each predicted id counts correct or wasted, each actual id
 * not predicted counts missed. */
gmoe_status gmoe_predictor_score(gmoe_predictor* p, const uint32_t* predicted, uint32_t n_predicted,
                                 const uint32_t* actual, uint32_t n_actual);
gmoe_status gmoe_predictor_stats(const gmoe_predictor* p, gmoe_predict_stats* out);
/* The transition table, n_experts^2 counts row-major: read it out (to save a learned
 * model) or load one back. */
gmoe_status gmoe_predictor_get_counts(const gmoe_predictor* p, uint32_t* counts, uint64_t n);
gmoe_status gmoe_predictor_set_counts(gmoe_predictor* p, const uint32_t* counts, uint64_t n);

/* PrefetchEngine::observe_step (prefetch/mod.rs:77-106) for layer `layer_id` whose
 * experts are ids [id_base, id_base + n_experts) of the predictor. It scores last step's
 * prediction against `used`, learns previous -> used, predicts up to `depth` ids into
 * `predicted` (*n_predicted receives the count) and stages the predicted experts of this
 * layer that are neither resident nor already on their way into the slab for the
 * context's staging thread, and returns without waiting for them (gmoe_expert_state,
 * gmoe_prefetch_wait). *launched and *skipped (may be NULL) count the queued and the
 * skipped ones. The staging thread makes room by evicting least recently used experts
 * other than this step's and the previous step's used ones and the predicted ones, after
 * the evicted layer's last queued call has finished; a prediction that finds no such room
 * is dropped (the forward stages it if it is routed). */
gmoe_status gmoe_prefetch_step(gmoe_ctx* ctx, gmoe_predictor* p, uint32_t layer_id, uint32_t id_base,
                               const uint32_t* previous, uint32_t n_previous, const uint32_t* used,
                               uint32_t n_used, const uint32_t* predicted_last, uint32_t n_predicted_last,
                               uint32_t depth, uint32_t* predicted, uint32_t* n_predicted, uint32_t* launched,
                               uint32_t* skipped);

/* ---- one decode step of a whole model (LlamaBackend::logits_batch, llama/mod.rs:1134-1206) ----
 *
 * The caller around the MoE layer: every sequence takes one new token. The step embeds
 * the tokens, runs each layer as layer_batch_over does (llama/mod.rs:851-893) — h =
 * rmsnorm(x) * attn_norm; q, k, v = the dense projections; attention over the paged KV
 * cache; x += wo(context); h = rmsnorm(x) * ffn_norm; x += the MoE layer — then
 * rmsnorm(x) * output_norm, the output head, and greedy sampling (runtime/mod.rs:98-105:
 * the first index of the largest logit). The weights are the library's own registered
 * objects; the model keeps their ids (release them after the model). The token table
 * and the norm weights are copied into device memory. */
typedef struct gmoe_model gmoe_model;
typedef struct gmoe_model_desc {
  uint32_t n_layers, d_model, vocab;  /* d_model a multiple of 4, at most 8192 */
  float rms_eps;
  gmoe_kv* kv;                  /* n_layers layers; its heads set the q and kv widths */
  const uint32_t* moe_layers;   /* [n_layers] gmoe_layer_register ids (d_model wide) */
  const uint32_t* wq;           /* [n_layers] dense ids: q_dim x d_model */
  const uint32_t* wk;           /* [n_layers] kv_dim x d_model */
  const uint32_t* wv;           /* [n_layers] kv_dim x d_model */
  const uint32_t* wo;           /* [n_layers] d_model x q_dim */
  uint32_t output;              /* dense id: vocab x d_model, or GMOE_OUTPUT_TIED: the head is
                                   token_embd itself (llama/mod.rs:565-571), under output_math */
  const float* attn_norm;       /* [n_layers][d_model] */
  const float* ffn_norm;        /* [n_layers][d_model] */
  const float* output_norm;     /* [d_model] */
  uint32_t token_embd_qtype;    /* ggml type id of the table's rows (any the slab takes) */
  const void* token_embd;       /* [vocab] rows of d_model values, quant::byte_size each; copied.
                                   F32 rows stay an f32 table; other types stay packed in HBM,
                                   a row dequantised per token (Weight::row, llama/mod.rs:198-212) */
  uint32_t output_math;         /* GMOE_MATH_* of a tied head */
} gmoe_model_desc;
#define GMOE_OUTPUT_TIED 0xFFFFFFFFu

gmoe_status gmoe_model_create(gmoe_ctx* ctx, const gmoe_model_desc* desc, gmoe_model** out);
void gmoe_model_destroy(gmoe_model* model);
/* Sequences seqs[i] (open in the model's KV cache, distinct) take tokens[i]; next[i] is
 * the greedy next token; logits ([n x vocab], host) may be NULL. 1 <= n <= 64. Refused
 * before any device work when a token is outside the vocabulary (GMOE_ERR_INVALID_TOKEN),
 * a sequence's window is exhausted or the pool lacks pages (GMOE_ERR_CACHE), or an
 * expert is not resident. Synchronous: returns when next (and logits) are written.
 * The step's launches are replayed from a HIP graph captured after the first step of each
 * batch size (the tokens and the attention entries are then read from device memory);
 * the results are those of the launches issued one by one. */
gmoe_status gmoe_model_decode(gmoe_model* model, uint32_t n, const uint32_t* seqs, const uint32_t* tokens,
                              uint32_t* next, float* logits);
/* A prompt through the model: LlamaBackend::forward_tail + logits_multi
 * (llama/mod.rs:1027-1116, :1223-1247) for sequence `seq`, whose n new tokens take its
 * next positions. The tokens run in chunks of up to 256 (DEFAULT_PREFILL_CHUNK), each
 * chunk layer-major: every layer over the whole chunk (its projections and MoE layer as
 * batched products, the MFMA paths where the batch allows), its attention causal over the
 * sequence. next[0..n_last) receive the greedy token after each of the last n_last
 * positions and logits ([n_last x vocab], host) their logits when not NULL; 1 <= n_last <=
 * min(n, 64). Refused before any layer runs when a token is outside the vocabulary, the
 * window or pool cannot take the n positions, or an expert is not resident; a step that
 * fails later leaves the sequence as it was. Synchronous. */
gmoe_status gmoe_model_prefill(gmoe_model* model, uint32_t seq, uint32_t n, const uint32_t* tokens,
                               uint32_t n_last, uint32_t* next, float* logits);
/* No counterpart in the reference (the execution strategy of gmoe_model_decode):
 * enable != 0 replays decode steps from a graph (the default), 0 issues every launch of
 * every step. gmoe_model_graph_ready says whether a graph for batch size n is held. */
gmoe_status gmoe_model_set_graphs(gmoe_model* model, int enable);
int gmoe_model_graph_ready(gmoe_model* model, uint32_t n);
/* Diagnostic, with no counterpart in the reference: gmoe_model_decode that also copies
 * every layer's activations into trace (host, gmoe_model_trace_floats(model, n) floats),
 * for checks of each layer against a restatement fed the device's own inputs. Per layer,
 * each block n rows: the residual x entering it, h = rmsnorm(x) * attn_norm, q [q_dim],
 * k [kv_dim], v [kv_dim] (before rotation), the attention context [q_dim], wo(context),
 * x after the attention's residual add, h = rmsnorm(x) * ffn_norm, the MoE layer's output;
 * then the final residual and rmsnorm(x) * output_norm. */
size_t gmoe_model_trace_floats(const gmoe_model* model, uint32_t n);
gmoe_status gmoe_model_decode_trace(gmoe_model* model, uint32_t n, const uint32_t* seqs, const uint32_t* tokens,
                                    uint32_t* next, float* logits, float* trace);

/* ---- single steps of the path, for parity tests (host pointers, synchronous) ---- */

/* quant::dequantize (quant/mod.rs:104-114) on the device: n_elems values of qtype. */
gmoe_status gmoe_dequant(gmoe_ctx* ctx, uint32_t qtype, const void* blocks, uint64_t nbytes,
                         uint64_t n_elems, float* out);

/* quant::matmul (quant/mod.rs:223-304) for math = PACKED, simd::matmul over the
 * dequantised rows for math = F32: out[b*rows + r] = dot(row r, xs[b]). */
gmoe_status gmoe_matmul(gmoe_ctx* ctx, uint32_t qtype, uint32_t math, const void* w,
                        uint64_t nbytes, uint32_t rows, uint32_t cols, const float* xs,
                        uint32_t n, float* out);

/* Router logits (when router != NULL; otherwise `x` already holds [n x ne] logits),
 * then gating: ids/w are [n x top_k] in ranked order; logits_out (may be NULL)
 * receives the [n x ne] logits. */
gmoe_status gmoe_route(gmoe_ctx* ctx, uint32_t gating, const float* router, const float* x,
                       uint32_t d, uint32_t ne, uint32_t top_k, uint32_t n, uint32_t* ids,
                       float* w, float* logits_out);

/* Routing inversion (llama/mod.rs:966-972) as a stable counting sort: offsets[ne+1],
 * and for each slot in [0, n*k): its token, its routing weight and its rank. */
gmoe_status gmoe_dispatch(gmoe_ctx* ctx, const uint32_t* ids, const float* w, uint32_t n,
                          uint32_t top_k, uint32_t ne, uint32_t* offsets, uint32_t* slot_token,
                          float* slot_weight, uint32_t* slot_rank);

/* The device exp used by softmax and SiLU, applied elementwise. */
gmoe_status gmoe_expf(gmoe_ctx* ctx, const float* x, uint64_t n, float* y);

/* ---- build-side data preparation (host code; the reference has no quantiser) ---- */

/* Quantise n f32 values (n a multiple of the block size) into `out`
 * (byte_size(qtype, n) bytes). Round-to-nearest min/max quantisers; see DESIGN. */
gmoe_status gmoe_quantize(uint32_t qtype, const float* x, uint64_t n, void* out, int threads);

/* n values of N(mean, std^2) from a counter-based splitmix64 stream keyed by seed. */
gmoe_status gmoe_fill_gaussian(uint64_t seed, float mean, float std, uint64_t n, float* out,
                               int threads);

/* ---- measurement ---- */

/* When on, every forward records HIP events around the dominant expert kernels on
 * the stream they run on; gmoe_kernel_time returns their accumulated milliseconds. */
gmoe_status gmoe_set_kernel_timing(gmoe_ctx* ctx, int on);
gmoe_status gmoe_kernel_time(gmoe_ctx* ctx, uint32_t which, double* total_ms, uint64_t* count);

#ifdef __cplusplus
}
#endif
#endif
