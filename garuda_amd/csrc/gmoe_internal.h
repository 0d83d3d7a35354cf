// gmoe_internal.h — shared between the HIP kernels (gmoe_kernels.hip) and the host
// runtime (gmoe_api.cpp). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <stddef.h>
#include <stdint.h>

namespace gmoe {

// ggml type ids (garuda/src/quant/mod.rs:22-30)
enum QType : uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12,
                        Q5_K = 13, Q6_K = 14 };

// (elements per block, bytes per block), quant/mod.rs:41-61. Returns false if unsupported.
inline bool block_layout(uint32_t t, uint32_t* elems, uint32_t* bytes) {
  switch (t) {
    case F32: *elems = 1; *bytes = 4; return true;
    case F16: *elems = 1; *bytes = 2; return true;
    case Q4_0: *elems = 32; *bytes = 18; return true;
    case Q8_0: *elems = 32; *bytes = 34; return true;
    case Q2_K: *elems = 256; *bytes = 84; return true;
    case Q3_K: *elems = 256; *bytes = 110; return true;
    case Q4_K: *elems = 256; *bytes = 144; return true;
    case Q5_K: *elems = 256; *bytes = 176; return true;
    case Q6_K: *elems = 256; *bytes = 210; return true;
  }
  return false;
}

// quant/mod.rs:379-381: types whose packed rows are dotted against int8 activations.
__host__ __device__ constexpr bool has_int8_kernel(uint32_t t) {
  return t == Q8_0 || t == Q2_K || t == Q3_K || t == Q4_K || t == Q5_K || t == Q6_K;
}

// The activation sums a packed dot of type qt reads, one 32-bit word each: f32 sums of 32
// values (Q4_K, Q5_K: the reference converts the i32 sum, which is exact below 2^24), f32
// sums of 16 (Q2_K), i32 sums of 16 times the type's offset (Q6_K -32, Q3_K -4: the dot's
// integer chain starts from it, so it adds the -32 or -4 times the sum that the reference
// subtracts; integer sums are exact in any order), or none (Q8_0). The activation
// quantisers write them in the form of the type that reads them, so that staging them is
// a copy; a row of K values has K / sum_width words.
enum SumKind { kSumNone = 0, kSumF32x32 = 1, kSumF32x16 = 2, kSumI32x16 = 3 };
__host__ __device__ constexpr int sum_kind_of(uint32_t qt) {
  return (qt == Q4_K || qt == Q5_K) ? kSumF32x32 : qt == Q2_K ? kSumF32x16 : (qt == Q6_K || qt == Q3_K) ? kSumI32x16 : kSumNone;
}
__host__ __device__ constexpr int32_t sum_offset_of(uint32_t qt) { return qt == Q6_K ? -32 : qt == Q3_K ? -4 : 1; }
__host__ __device__ constexpr uint32_t sum_width(int kind) { return kind == kSumF32x32 ? 32u : kind ? 16u : 0u; }

// ---------------------------------------------------------------------------------
// Tiled slab layout of an expert matrix (rows x cols, packed rows of blocks).
//
// A row is cut into units of G consecutive blocks (EU elements) stored as U bytes, U a
// multiple of 16: one block padded with zeros (Q4_K, Q5_K, Q6_K, Q3_K, Q2_K, F32), two
// F16 blocks of 32 values, or eight Q8_0/Q4_0 blocks repacked as their eight f16 scales
// (16 bytes) followed by their quant bytes, so every block's quants stay dword
// aligned. Rows are grouped in tiles of 64, and a tile stores its units one after
// another; within a unit, 16-byte piece p of row i of the tile sits at p*1024 + i*16.
// A wave that streams a tile therefore reads each unit as NP = U/16 fully coalesced
// 1 KiB loads, and lane i receives its own row's unit in registers. Rows past the end
// of the matrix and blocks past the end of a row are zero bytes.
// ---------------------------------------------------------------------------------
constexpr uint32_t kTileRows = 64;

struct Unit {
  uint32_t G;   // blocks per unit
  uint32_t EU;  // elements per unit
  uint32_t U;   // bytes per unit in the slab
  uint32_t B;   // bytes per block in the packed row
};

__host__ __device__ inline bool unit_of(uint32_t t, Unit* u) {
  switch (t) {
    case F32: *u = {1, 32, 128, 128}; return true;
    case F16: *u = {2, 64, 128, 64}; return true;
    case Q4_0: *u = {8, 256, 144, 18}; return true;
    case Q8_0: *u = {8, 256, 272, 34}; return true;
    case Q2_K: *u = {1, 256, 96, 84}; return true;
    case Q3_K: *u = {1, 256, 112, 110}; return true;
    case Q4_K: *u = {1, 256, 144, 144}; return true;
    case Q5_K: *u = {1, 256, 176, 176}; return true;
    case Q6_K: *u = {1, 256, 224, 210}; return true;
  }
  return false;
}

// Blocks in a row of `cols` elements (F32/F16 counted as blocks of 32 values).
__host__ __device__ inline uint32_t row_blocks(const Unit& u, uint32_t cols) { return cols / (u.EU / u.G); }
__host__ __device__ inline uint32_t row_units(const Unit& u, uint32_t cols) {
  return (row_blocks(u, cols) + u.G - 1) / u.G;
}
// Bytes of one 64-row tile and of the whole tiled matrix.
__host__ __device__ inline uint64_t tile_bytes(const Unit& u, uint32_t cols) {
  return (uint64_t)row_units(u, cols) * kTileRows * u.U;
}
__host__ __device__ inline uint64_t tiled_bytes(const Unit& u, uint32_t rows, uint32_t cols) {
  return (uint64_t)((rows + kTileRows - 1) / kTileRows) * tile_bytes(u, cols);
}

// Byte `b` of unit `un` of a row with `nblk` blocks: its offset in the packed row, or
// -1 where the unit holds padding.
__host__ __device__ inline int64_t unit_src_byte(uint32_t t, const Unit& u, uint32_t nblk, uint32_t un,
                                                 uint32_t b) {
  const uint64_t b0 = (uint64_t)un * u.G;  // first block of the unit
  if (t == Q8_0 || t == Q4_0) {
    uint32_t g, o;
    if (b < 16) {
      g = b / 2;
      o = b % 2;
    } else {
      const uint32_t qb = u.B - 2;  // quant bytes per block
      g = (b - 16) / qb;
      o = 2 + (b - 16) % qb;
    }
    if (g >= u.G || b0 + g >= nblk) return -1;
    return (int64_t)((b0 + g) * u.B + o);
  }
  const uint32_t g = b / u.B;
  if (g >= u.G || b0 + g >= nblk) return -1;
  return (int64_t)((b0 + g) * u.B + b % u.B);
}

// Q3_K units in the slab. A packed Q3_K block (quant/mod.rs:503-540, :840-875) keeps each
// value v = q2 + 4 * hbit (0..7; the quant is v - 4) in two bit planes, qs and hmask, and
// putting a word of four values together again from them takes four operations. Bytes
// 0..95 of a slab unit hold the same values regrouped (bytes 96..109, the scales and d,
// are the block's). With O(s, i) the word of values 4i..4i+3 of sub-block s (one a byte),
// chunk c (sub-blocks 8c..8c+7) fills bytes 48c..48c+47, and in it sub-group r
// (sub-blocks s0 = 8c + 4r .. s0 + 3) and lane half h (words i = 2h, 2h + 1) own three
// words T0, T1, T2, word Tk at byte 48c + 16 (x / 2) + 8h + 4 (x % 2), x = 3r + k:
//   T0 = O(s0, 2h)     | O(s0, 2h + 1) << 3     | (O(s0 + 3, 2h) & 3) << 6
//   T1 = O(s0 + 1, 2h) | O(s0 + 1, 2h + 1) << 3 | (O(s0 + 3, 2h + 1) & 3) << 6
//   T2 = O(s0 + 2, 2h) | O(s0 + 2, 2h + 1) << 3 | (O(s0 + 3, 2h) >> 2) << 6 | (O(s0 + 3, 2h + 1) >> 2) << 7
// (each shift within its byte). A word of sub-blocks s0..s0 + 2 then takes two operations
// and one of s0 + 3 four (q3s_pair), and the two halves of a 16-value MFMA step find
// their words 8 bytes apart in one 16-byte piece.
__host__ __device__ constexpr uint32_t q3s_word(uint32_t c, uint32_t h, uint32_t x) {
  return 12 * c + 4 * (x / 2) + 2 * h + x % 2;
}
// The words O(s, 2h), O(s, 2h + 1) of sub-block s = s0 + k of a Q3_K slab unit (values
// v = q2 + 4 * hbit, one a byte) from lane half h's three words t0, t1, t2 of its
// sub-group (q3s_word); k is a constant once the callers' loops unroll.
__host__ __device__ __forceinline__ void q3s_pair(uint32_t t0, uint32_t t1, uint32_t t2, int k, uint32_t& o0,
                                                  uint32_t& o1) {
  if (k == 3) {
    o0 = ((t0 >> 6) & 0x03030303u) | ((t2 >> 4) & 0x04040404u);
    o1 = ((t1 >> 6) & 0x03030303u) | ((t2 >> 5) & 0x04040404u);
  } else {
    const uint32_t t = k == 0 ? t0 : k == 1 ? t1 : t2;
    o0 = t & 0x07070707u;
    o1 = (t >> 3) & 0x07070707u;
  }
}
// Value l of sub-block s of packed Q3_K block blk, as v = q2 + 4 * hbit (the is-th
// sub-block of quant/mod.rs:520-533: shift 2j of qs byte 32 half + 16 (s % 2) + l, mask
// bit 4 half + j of hmask byte 16 (s % 2) + l).
__host__ __device__ inline uint32_t q3k_value(const uint8_t* blk, uint32_t s, uint32_t l) {
  const uint32_t half = s / 8, j = (s % 8) / 2, off = 16 * (s % 2);
  return ((blk[32 + 32 * half + off + l] >> (2 * j)) & 3u) | (((blk[off + l] >> (4 * half + j)) & 1u) << 2);
}
// Byte b < 96 of the slab unit of packed Q3_K block blk.
__host__ __device__ inline uint8_t q3s_byte(const uint8_t* blk, uint32_t b) {
  const uint32_t c = b / 48, rem = b % 48, x = 2 * (rem / 16) + (rem % 8) / 4, h = (rem % 16) / 8, e = b % 4;
  const uint32_t k = x % 3, s0 = 8 * c + 4 * (x / 3);
  auto o = [&](uint32_t s, uint32_t i) { return q3k_value(blk, s, 4 * i + e); };
  uint32_t v = o(s0 + k, 2 * h) | o(s0 + k, 2 * h + 1) << 3;
  if (k == 0) v |= (o(s0 + 3, 2 * h) & 3u) << 6;
  else if (k == 1) v |= (o(s0 + 3, 2 * h + 1) & 3u) << 6;
  else v |= (o(s0 + 3, 2 * h) >> 2) << 6 | (o(s0 + 3, 2 * h + 1) >> 2) << 7;
  return (uint8_t)v;
}

// One active expert of a call as the expert kernels read it, in a single load: the
// dispatch writes entry a for the a-th active expert (ascending id) and m = 0 for the
// entries after the last one.
struct ExpertWork {
  const uint8_t* w[3];  // tiled gate, up, down matrices
  uint32_t e;           // expert id
  uint32_t s0;          // first slot of its tokens
  uint32_t m;           // number of its tokens
  uint32_t pad;
};

// Per-call device buffers. Token-indexed arrays have n rows; slot-indexed ones nslot
// (n*k, or n*ne when the speculative front end may dispatch more than k experts a token).
struct FwdBufs {
  const float* hs;       // [n][d]
  const float* logits_in;// [n][ne] or null
  float* out;            // [n][d]
  uint32_t* ids;         // [n][k]
  float* w;              // [n][k]
  float* logits;         // [n][ne]
  int8_t* xq;            // [n][d]
  float* xs;             // [n][d/32]
  uint32_t* xsum;        // [n][d/sum_width]: sums in the gate/up type's form (sum_kind_of)
  uint32_t* offsets;     // [ne+1]
  uint32_t* active;      // [1 + ne]: count, then active expert ids ascending
  uint32_t* slot_tok;    // [n*k]
  float* slot_w;         // [n*k]
  uint32_t* slot_rank;   // [n*k]
  uint32_t* slot_of;     // [n*k]: (t, rank) -> slot
  ExpertWork* work;      // [ne] active experts for the expert kernels (may be null outside a layer call)
  // prefill (f32 math, MFMA): token tiles; activations and h in slot order as fp16
  // pairs (v = hi + lo, hi plane then lo plane) and their sums over 16 or 32 values
  uint32_t* ptile;       // [ptile_cap] (active slot << 16) | tile of kPfTok tokens; ~0u past the last tile
  uint32_t ptile_cap;
  _Float16* xh;          // [2][n*k][d]
  _Float16* xsh;         // [2][n*k][d/16]
  _Float16* hh;          // [2][n*k][f]
  _Float16* hsh;         // [2][n*k][f/16]
  // packed-math prefill (k_pq): the activation codes in slot order as fp16 in xh (one
  // plane), their per-token scales and sums transposed to [d/32][nkp] and [d/w][nkp]
  float* qxs;
  float* qxsum;
  uint32_t nkp;          // >= n*k + 64
  int8_t* hq;            // [n*k][f]
  float* hsc;            // [n*k][f/32]
  uint32_t* hsum;        // [n*k][f/sum_width]: sums in the down type's form
  float* hf;             // [n*k][f]
  float* y;              // [kMaxKsg][n*k][d] partial slices of the down product
  uint32_t* done;        // [1] workgroups of the front end that have finished; 0 between calls
  uint32_t nslot;        // rows of the slot-indexed arrays; y slices are nslot*d apart
  uint32_t* cand;        // [n][ne] speculative front end: each token's candidate experts, ~0u-padded
  uint32_t fuse_out;     // 1: the front end zeroes out and the down product adds into it
                         // (launch_down_atomic); no combine launch
  uint32_t spec;         // 1: slots hold candidate pairs; slot_of / slot_w hold the combine's
                         // (slot, weight) per (token, position in combine order), written by
                         // the exact routing (RouteArgs::comb_slot, comb_w)
  // speculative front end with nx: it first makes hs itself, as k_add_norm<true> does:
  // nx += the sum of ny's nsl_y K slices (ny_stride floats apart), hs = RMSNorm(nx) * nw
  float* nx;             // [n][d] residual, updated
  const float* ny;       // [nsl_y][..][d] slices, row t at ny + t * d
  const float* nw;       // [d]
  float* nh;             // [n][d] where hs is written (hs points there too)
  float neps;
  uint32_t nsl_y;
  uint64_t ny_stride;
};

// Exact routing carried by the gate/up launch of a speculative decode call: one extra
// workgroup per (token, expert) runs route_logit (gmoe_device.h). n = 0: none.
struct RouteArgs {
  const float* router;  // [ne][d]
  const float* hs;      // [n][d]
  float* logits;        // [n][ne]
  uint32_t* ids;        // [n][k]
  float* w;             // [n][k]
  uint32_t* tok_done;   // [n] logits finished per token; 0 between calls
  // The combine's inputs, in its order (ascending expert id, or rank with combine = 1):
  // each routed pair's slot among the candidate slots (offsets / slot_tok of the
  // speculative dispatch, ~0u if the candidates missed it) and its weight.
  const uint32_t* offsets;  // [ne+1]
  const uint32_t* slot_tok; // candidate slots' tokens, in token order per expert
  uint32_t* comb_slot;      // [n][k]
  float* comb_w;            // [n][k]
  uint32_t n, ne, k, d, gating, sec, combine;
  uint32_t self;  // 1: the gate/up launch also does the front end's work (one token)
};
// Values of d per LDS half in route_logit. It shares its launch's LDS size with the expert
// workgroups, so it is kept small (8 KB in all).
constexpr uint32_t kRouteSection = 1024;
inline uint32_t route_logit_lds(uint32_t k, uint32_t sec) { return (2 * sec + 2 * k) * 4; }

struct LayerDev {
  uint32_t d, f, ne, k, gating, combine, math;
  uint32_t qt_gate, qt_up, qt_down;
  const float* router;          // device [ne][d]
  const uint8_t* const* eptr;   // device [3][ne]: gate, up, down tiled matrix of each expert (null = absent)
};

// Scratch of the allocation-free forward: a static device array of this many bytes per
// GPU (gmoe_noalloc.hip); a call whose launch sequence needs more is refused.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
// Its address on `device` (the current device), looked up once per device.
hipError_t noalloc_scratch(int device, void** out);
// Orders the calls that share a device's array: noalloc_begin waits (on st) for the previous
// call's work and holds the device's lock until noalloc_end records this call's (neither
// under graph capture).
std::unique_lock<std::mutex> noalloc_begin(int device, hipStream_t st, hipError_t* err);
hipError_t noalloc_end(int device, hipStream_t st);

// The down product splits K over this many partial slices at most; FwdBufs::y holds
// kMaxKsg slices of [n*k][d]. A down workgroup has kDnKS waves, each its own K range.
constexpr uint32_t kMaxKsg = 8;
constexpr int kDnKS = 2;

// Expert products of one block type (gmoe_units.hip, built once per type).
template <int QT> hipError_t units_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, const RouteArgs& ra,
                                          hipStream_t st);
template <int QT> hipError_t units_down(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st);
// Whether a gate/up launch of this type can fold the speculative front end in (one token,
// RouteArgs::self; packed math with int8 h, the split gate/up's shapes).
template <int QT> bool units_self_ok(const LayerDev& L, uint32_t n);
// Down with the combine folded in (top-k <= 2, out zeroed by the front end beforehand).
template <int QT> hipError_t units_down_atomic(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);

// Prefill products (f32 math) on MFMA over token tiles of kPfTok (gmoe_prefill.hip,
// built once per type; F32 weights are not supported). prefill_ok says when the path
// applies. Sums of activations are kept per 32 values for Q4_K/Q5_K and per 16 for Q2_K
// (the widths of their min terms), none otherwise.
constexpr uint32_t kPfTok = 64;
constexpr uint32_t kPfMinSlots = 64;
__host__ __device__ constexpr uint32_t pf_sum_width(uint32_t qt) {
  return (qt == Q4_K || qt == Q5_K) ? 32u : qt == Q2_K ? 16u : 0u;
}
// Packed-math prefill on MFMA (gmoe_prefill.hip): the int8 types only. Activation sums
// are kept per 32 values (Q4_K, Q5_K) or 16 (Q2_K); the others need none (Q6_K's and
// Q3_K's MFMA operand carries the quant offset, Q8_0 has no min term).
__host__ __device__ constexpr uint32_t pq_sum_width(uint32_t qt) {
  return (qt == Q4_K || qt == Q5_K) ? 32u : qt == Q2_K ? 16u : 0u;
}
template <int QT> hipError_t pq_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
template <int QT> hipError_t prefill_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
template <int QT> hipError_t prefill_down(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg,
                                          hipStream_t st);
// K slices of the prefill down product (partial slices of y, added by the combine).
template <int QT> uint32_t prefill_down_slices(const LayerDev& L, const FwdBufs& B);
// Token tiles a call of n tokens can need at most.
inline uint32_t prefill_tiles_cap(uint32_t n, uint32_t k, uint32_t ne) { return (n * k) / kPfTok + ne + 1; }

// Launchers (gmoe_kernels.hip). All are asynchronous on `st` and validate nothing:
// the host runtime checks shapes before calling them.
hipError_t launch_dequant(uint32_t qtype, const uint8_t* blocks, size_t nblocks, float* out,
                          hipStream_t st);
hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t st);
// sums in the form the packed dot of type `reader` reads (sum_kind_of)
hipError_t launch_quant_act(const float* x, uint32_t n_tok, uint32_t K, int8_t* q, float* s,
                            uint32_t* sums, uint32_t reader, hipStream_t st);
hipError_t launch_route(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
hipError_t launch_dispatch(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
// Route + gate + int8 activation quantiser (when quant) + dispatch in one launch, for
// small decode batches (front_small_ok).
bool front_small_ok(const LayerDev& L, uint32_t n);
// dispatch = false: logits, ids and weights only (the exact half of the speculative front end)
hipError_t launch_front_small(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, bool dispatch,
                              hipStream_t st);
// The dispatch alone by one workgroup of eight waves (ne <= kParExperts: its LDS holds
// 12 words an expert), after a front end launched without it.
constexpr uint32_t kParExperts = 1024;
hipError_t launch_dispatch_par(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
// Calls of at least this many tokens run the small front end and its dispatch as two
// launches: the launch boundary orders the routing for the dispatch, where one launch
// needs a release fence per workgroup (measured: 56 us at 512 tokens).
constexpr uint32_t kFrontSplitTokens = 64;
// Front end for 64 < ne <= 256 experts: one wave per token gates it (given logits or the
// sequential dots) and quantises its activations; the last workgroup dispatches.
bool front_wide_ok(const LayerDev& L, uint32_t n);
hipError_t launch_front_wide(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, hipStream_t st);
// Speculative front end: router logits by a parallel dot with a rigorous bound on their
// distance to the sequential dot, every expert that can be among a token's top k, the
// int8 activation quantiser, and the dispatch of all (token, candidate) pairs.
constexpr uint32_t kSpecMaxSlots = 512;
bool spec_ok(const LayerDev& L, uint32_t n);
hipError_t launch_spec_front(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, hipStream_t st);
hipError_t launch_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, const RouteArgs& ra, hipStream_t st);
bool gateup_self_ok(const LayerDev& L, uint32_t n);
// ksg = 0: down_ksg(L, n * L.k)
hipError_t launch_down(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st, uint32_t ksg = 0);
uint32_t dense_ksg(const LayerDev& L);
hipError_t launch_combine(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st);
// The down product adding its weighted rows into the zeroed output (launch_down_atomic)
// applies for top-k <= 2 at decode batches up to kFuseMaxTokens: measured on the C2 layer
// as fast as the K-split down product at batches 1-8 with the combine launch gone (batch
// 8: 177.2 -> 171.5 us a layer call). An expert with more tokens than a workgroup stages
// at once re-streams its weights per chunk.
constexpr uint32_t kFuseMaxTokens = 8;
bool down_atomic_ok(const LayerDev& L, uint32_t n);
hipError_t launch_down_atomic(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
// Prefill path: whether it applies (f32 math, at least kPfMinSlots slots, supported
// types and shapes), the per-slot fp16 gather of the activations, and the products.
bool prefill_ok(const LayerDev& L, uint32_t n);
// Packed-math calls with enough tokens per expert run the products on MFMA: the
// activation codes gathered in slot order, gate/up by k_pq (bit-exact h and codes), the
// down product by k_pf on the dequantised h.
bool prefill_packed_ok(const LayerDev& L, uint32_t n);
hipError_t launch_gather_codes(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
hipError_t launch_pq_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
bool prefill_dense_ok(const LayerDev& L, uint32_t n);
hipError_t launch_dense_setup(ExpertWork* work, uint32_t* offsets, uint32_t* active, uint32_t* ptile,
                              uint32_t ptile_cap, uint32_t* slot_tok, const uint8_t* w, uint32_t n, hipStream_t st);
hipError_t launch_gather_f16(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
hipError_t launch_prefill_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
hipError_t launch_prefill_down(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st);
uint32_t prefill_ksg(const LayerDev& L, const FwdBufs& B);
// Number of partial slices launch_down writes for this layer and about `pairs` routed
// (token, expert) pairs (1 = y is final).
uint32_t down_ksg(const LayerDev& L, uint32_t pairs);
// out[i] = parts[i] + parts[count + i] + ... over ksg slices, in slice order.
hipError_t launch_reduce_parts(const float* parts, uint32_t ksg, size_t count, float* out, hipStream_t st);
// Rows [r0, r0 + nrows) of a packed matrix (raw rows of row_bytes each, r0 a multiple of
// 64) -> the tiles they make up in the tiled layout of the whole matrix at dst.
// ---- decode attention over a paged KV cache (gmoe_attn.hip) ----
struct AttnEntry {
  uint32_t* pages;  // the sequence's page table for this layer
  uint32_t pos;     // this token's position
  uint32_t start;   // first position it attends to (sliding window)
  uint32_t page;    // the page holding pos
  uint32_t fresh;   // 1: pos opens that page; the append records it in the table
};

constexpr uint32_t kAttnInline = 16;  // entries carried in the kernel arguments
struct AttnArgs {
  const AttnEntry* ent;  // [n] in device memory, or null: n <= kAttnInline entries in `inl`
  AttnEntry inl[kAttnInline];
  uint32_t n, n_heads, n_kv, hd, bs;
  float theta, scale;
  float* pool;           // page pool
  uint64_t page_floats;  // 2 * bs * kv_dim
  const float* q;        // [n][n_heads * hd]
  const float* k;        // [n][kv_dim]
  const float* v;        // [n][kv_dim]
  float* qr;             // [n][n_heads * hd] rotated q
  float* part;           // [n][n_heads][nchunk][hd + 2]: chunk partials (o, m, l)
  uint32_t nchunk;       // chunks of kAttnChunk positions per entry
  float* ctx;            // [n][n_heads * hd]
  uint32_t q_stride, kv_stride;  // floats between consecutive rows of q, and of k and v
  uint32_t nsl;                  // > 1: q, k and v are each the sum of nsl K slices of a dense
  uint64_t sl_stride;            //   product, sl_stride floats apart (added in slice order)
};

constexpr uint32_t kAttnChunk = 64, kAttnMaxGroup = 16, kAttnMaxHd = 256;
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);

// Decode-step glue (gmoe_glue.hip): embedding rows, residual add + RMSNorm * weight,
// greedy token. A decode step carries its tokens in the kernel arguments.
constexpr uint32_t kModelMaxBatch = 64;
constexpr int kNormVec = 8;  // float4 of a row per thread in k_add_norm: d_model <= 8192
struct GlueTokens {
  uint32_t tok[kModelMaxBatch];
};
hipError_t launch_embed(const GlueTokens& tk, uint32_t n, const float* table, uint32_t d, float* x, hipStream_t st);
hipError_t launch_embed_dev(const uint32_t* tok, uint32_t n, const float* table, uint32_t d, float* x, hipStream_t st);
// rows of a tiled dense weight of type qtype, dequantised (tokens from tk, or dtok when tk is null)
template <int QT>
hipError_t units_embed(const uint8_t* tiled, uint32_t cols, const GlueTokens* tk, const uint32_t* dtok, uint32_t n,
                       float* x, hipStream_t st);
hipError_t launch_embed_tiled(uint32_t qtype, const uint8_t* tiled, uint32_t cols, const GlueTokens* tk,
                              const uint32_t* dtok, uint32_t n, float* x, hipStream_t st);
hipError_t launch_add_norm(float* x, const float* y, const float* w, uint32_t n, uint32_t d, float eps, float* h,
                           hipStream_t st);
// the same with y the sum of nsl K slices [nsl][n][d] of a dense product (k_reduce_parts's sum)
hipError_t launch_add_norm_slices(float* x, const float* parts, uint32_t nsl, const float* w, uint32_t n, uint32_t d,
                                  float eps, float* h, hipStream_t st);
hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t vocab, uint32_t* next, hipStream_t st);

hipError_t launch_tile_rows(uint32_t qtype, const uint8_t* raw, uint32_t r0, uint32_t nrows, uint32_t rows,
                            uint32_t cols, uint8_t* dst, hipStream_t st);

}  // namespace gmoe
