// gmoe_internal.h — shared between the HIP kernels (gmoe_kernels.hip) and the host
// runtime (gmoe_api.cpp). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
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
inline bool has_int8_kernel(uint32_t t) {
  return t == Q8_0 || t == Q2_K || t == Q3_K || t == Q4_K || t == Q5_K || t == Q6_K;
}

// Rows of every packed matrix are stored in the slab at a pitch rounded up to 16 bytes,
// so each row starts 16-byte aligned whatever the block size.
inline size_t row_pitch(size_t row_bytes) { return (row_bytes + 15) & ~size_t(15); }

// Activations of one matrix product, in the format its kernel reads.
// int8 form (quant/mod.rs:331-345, :322-326): per token K int8 values, K/32 scales,
// K/16 sums of 16 (sums of 32 are the pairwise totals).
struct ActQ {
  const int8_t* q;     // [rows_of_tokens][K]
  const float* s;      // [..][K/32]
  const int32_t* s16;  // [..][K/16]
};

// Per-call device buffers. Token-indexed arrays have n rows; slot-indexed ones n*k.
struct FwdBufs {
  const float* hs;       // [n][d]
  const float* logits_in;// [n][ne] or null
  float* out;            // [n][d]
  uint32_t* ids;         // [n][k]
  float* w;              // [n][k]
  float* logits;         // [n][ne]
  int8_t* xq;            // [n][d]
  float* xs;             // [n][d/32]
  int32_t* x16;          // [n][d/16]
  uint32_t* offsets;     // [ne+1]
  uint32_t* active;      // [1 + ne]: count, then active expert ids ascending
  uint32_t* slot_tok;    // [n*k]
  float* slot_w;         // [n*k]
  uint32_t* slot_rank;   // [n*k]
  uint32_t* slot_of;     // [n*k]: (t, rank) -> slot
  int8_t* hq;            // [n*k][f]
  float* hsc;            // [n*k][f/32]
  int32_t* h16;          // [n*k][f/16]
  float* hf;             // [n*k][f]
  float* y;              // [kMaxKsg][n*k][d] partial slices of the down product
};

struct LayerDev {
  uint32_t d, f, ne, k, gating, combine, math;
  uint32_t qt_gate, qt_up, qt_down;
  const float* router;          // device [ne][d]
  const uint8_t* const* eptr;   // device [3][ne]: gate, up, down base of each expert (null = absent)
  uint32_t pitch_gate, pitch_up, pitch_down;
};

// The down product of the row kernels splits K over this many partial slices at most;
// FwdBufs::y holds kMaxKsg slices of [n*k][d].
constexpr uint32_t kMaxKsg = 8;

// Launchers (gmoe_kernels.hip). All are asynchronous on `st` and validate nothing:
// the host runtime checks shapes before calling them.
hipError_t launch_dequant(uint32_t qtype, const uint8_t* blocks, size_t nblocks, float* out,
                          hipStream_t st);
hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t st);
hipError_t launch_quant_act(const float* x, uint32_t n_tok, uint32_t K, int8_t* q, float* s,
                            int32_t* s16, hipStream_t st);
hipError_t launch_route(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
hipError_t launch_dispatch(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
// Route + gate + int8 activation quantiser (when quant) + dispatch in one launch, for
// small decode batches (front_small_ok).
bool front_small_ok(const LayerDev& L, uint32_t n);
hipError_t launch_front_small(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, hipStream_t st);
hipError_t launch_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
hipError_t launch_down(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
hipError_t launch_combine(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st);
// Number of partial slices launch_down writes for this layer and batch (1 = y is final).
uint32_t down_ksg(const LayerDev& L, uint32_t n);
// out[i] = parts[i] + parts[count + i] + ... over ksg slices, in slice order.
hipError_t launch_reduce_parts(const float* parts, uint32_t ksg, size_t count, float* out, hipStream_t st);
// Plain matrix product for gmoe_matmul: out[b*rows + r] = dot(row r, x[b]).
hipError_t launch_matmul(uint32_t qtype, uint32_t math, const uint8_t* w, size_t pitch,
                         uint32_t rows, uint32_t cols, const float* x, const int8_t* xq,
                         const float* xs, const int32_t* x16, uint32_t n, float* out,
                         hipStream_t st);

}  // namespace gmoe
