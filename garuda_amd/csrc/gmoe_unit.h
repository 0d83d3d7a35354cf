// gmoe_unit.h — the slab's units as the expert kernels see them: compile-time unit
// shapes (matching unit_of() in gmoe_internal.h), the dequantisation of a unit's
// 32-value groups, and the wave-wide stream of a tile's units into registers.
#pragma once

#include "gmoe_device.h"

namespace gmoe {

// Compile-time unit shape; matches unit_of().
template <int QT> struct UT_;
template <> struct UT_<F32> { static constexpr int G = 1, EU = 32, U = 128; };
template <> struct UT_<F16> { static constexpr int G = 2, EU = 64, U = 128; };
template <> struct UT_<Q4_0> { static constexpr int G = 8, EU = 256, U = 144; };
template <> struct UT_<Q8_0> { static constexpr int G = 8, EU = 256, U = 272; };
template <> struct UT_<Q2_K> { static constexpr int G = 1, EU = 256, U = 96; };
template <> struct UT_<Q3_K> { static constexpr int G = 1, EU = 256, U = 112; };
template <> struct UT_<Q4_K> { static constexpr int G = 1, EU = 256, U = 144; };
template <> struct UT_<Q5_K> { static constexpr int G = 1, EU = 256, U = 176; };
template <> struct UT_<Q6_K> { static constexpr int G = 1, EU = 256, U = 224; };

// 32-value group q of a unit, dequantised with the reference's arithmetic
// (quant/mod.rs:624-875). For the repacked Q8_0/Q4_0 units group q is block q, whose
// f16 scale is half q of dwords 0..3 and whose quants follow the 16 scale bytes.
template <int QT>
__device__ __forceinline__ void unit_deq32(const uint32_t* w, int q, float* out) {
  if constexpr (QT == Q8_0) {
    const float s = f16f(w[q / 2] >> (16 * (q % 2)));
    const uint32_t* qb = w + 4 + 8 * q;
#pragma unroll
    for (int i = 0; i < 32; i++) out[i] = s * (float)(int8_t)byte_of(qb, i);
  } else if constexpr (QT == Q4_0) {
    const float s = f16f(w[q / 2] >> (16 * (q % 2)));
    const uint32_t* qb = w + 4 + 4 * q;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      uint32_t b = byte_of(qb, i);
      out[i] = s * (float)((int)(b & 15u) - 8);
      out[i + 16] = s * (float)((int)(b >> 4) - 8);
    }
  } else if constexpr (QT == F16) {
    deq32<F16>(w + 16 * q, 0, out);
  } else if constexpr (QT == Q3_K) {  // deq32<Q3_K>'s arithmetic over the regrouped values
    const float d_all = f16f(w[27]);
    uint32_t sc4[4];
    q3k_scales(w[24], w[25], w[26], sc4);
#pragma unroll
    for (int sb = 0; sb < 2; sb++) {
      const int s = 2 * q + sb;
      uint32_t v[4];
      q3s_words(w, s, v);
      const float dl = d_all * (float)((int)(int8_t)byte_of(sc4, s) - 32);
#pragma unroll
      for (int l = 0; l < 16; l++) out[16 * sb + l] = dl * (float)((int)byte_of(v, l) - 4);
    }
  } else {
    deq32<QT>(w, q, out);
  }
}

template <int QT>
__host__ __device__ constexpr uint32_t unit_blocks(uint32_t cols) { return cols / (UT_<QT>::EU / UT_<QT>::G); }
template <int QT>
__host__ __device__ constexpr uint32_t unit_count(uint32_t cols) {
  return (unit_blocks<QT>(cols) + UT_<QT>::G - 1) / UT_<QT>::G;
}

// One wave's stream over units [u0, u1) of the tile at `tile`: prime() issues the first
// loads, run(body) calls body(u, w) with the lane's row unit u in w[] for every unit in
// order. Set s of the ring holds units u0+s, u0+s+D, ...; a set is reloaded right after
// its body, so D-1 units are in flight during body(u). D = 2 by default (a third set
// measured no faster and cost the body its registers); single-token gate/up uses 4. Every
// load is unconditional (the unit index is clamped to the last unit, a re-read the L2
// serves) and the loop always runs whole rounds of D, only the bodies past u1 being
// skipped: the loads pending at each use are then the same on every path and the
// compiler waits for exactly the set it uses. STRIDE > 1: the lane's units are u0,
// u0 + STRIDE, ... below u1 (u1 - u0 a multiple of STRIDE), and the lane's row is its
// own (src is the lane's first piece).
template <int QT, int D = 2, int STRIDE = 1>
struct UnitStream {
  static constexpr int NP = UT_<QT>::U / 16, NW = UT_<QT>::U / 4;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const uint8_t* src;
  uint32_t u0, u1, ulast;
  u32x4 g[D][NP];

  __device__ __forceinline__ UnitStream(const uint8_t* __restrict__ tile, uint32_t u0_, uint32_t u1_, uint32_t lane)
      : src(tile + lane * 16), u0(u0_), u1(u1_), ulast(u1_ > u0_ ? u1_ - STRIDE : u0_) {}
  // (STRIDE > 1: the lane's first piece given directly)
  __device__ __forceinline__ UnitStream(const uint8_t* __restrict__ first, uint32_t u0_, uint32_t u1_)
      : src(first), u0(u0_), u1(u1_), ulast(u1_ > u0_ ? u1_ - STRIDE : u0_) {}

  __device__ __forceinline__ void fetch(int s, uint32_t u) {
    const uint8_t* p = src + (size_t)min(u, ulast) * (NP * 1024);
#pragma unroll
    for (int q = 0; q < NP; q++) g[s][q] = *reinterpret_cast<const u32x4*>(p + q * 1024);
  }

  __device__ __forceinline__ void prime() {
    if (u0 >= u1) return;
#pragma unroll
    for (int s = 0; s < D; s++) fetch(s, u0 + s * STRIDE);
  }

  template <class Body>
  __device__ __forceinline__ void run(Body body) { run_range(u0, u1, body); }

  // The units [a, b) of the stream, a - u0 a multiple of D, the ring carried on from the
  // previous range (its loads of the range's first units are in flight).
  template <class Body>
  __device__ __forceinline__ void run_range(uint32_t a, uint32_t b, Body body) {
    if (u0 >= u1) return;
    for (uint32_t u = a; u < b; u += D * STRIDE) {
#pragma unroll
      for (int s = 0; s < D; s++) {
        if (u + s * STRIDE < u1) {
          uint32_t w[NW];
#pragma unroll
          for (int q = 0; q < NP; q++) {
            w[4 * q] = g[s][q].x; w[4 * q + 1] = g[s][q].y; w[4 * q + 2] = g[s][q].z; w[4 * q + 3] = g[s][q].w;
          }
          body(u + s * STRIDE, w);
        }
        fetch(s, u + (s + D) * STRIDE);
      }
    }
  }
};

}  // namespace gmoe
