// gmoe_units.hip — the expert products (gate/up with SwiGLU, down) over the tiled slab.
//
// Compiled once per block type, with -DGMOE_QT=<ggml type id>: each object holds the
// kernels of one type and the explicit instantiations of units_gateup/units_down for it,
// so the instantiations build in parallel.
//
// Reference semantics: llama/mod.rs:1002-1020 via quant::matmul (quant/mod.rs:223-304)
// under packed math, or simd::matmul over dequantised weights (simd/mod.rs:96-129).
#include "gmoe_device.h"

#ifndef GMOE_QT
#error "gmoe_units.hip is compiled once per block type with -DGMOE_QT=<type id>"
#endif

namespace gmoe {

// ---------------------------------------------------------------------------------
// Expert products over the tiled slab (layout in gmoe_internal.h).
//
// A workgroup owns one 64-row tile of an expert matrix and lane i owns row i of it. A
// wave streams the tile's units in K order: unit u arrives as NP coalesced 1 KiB loads
// that leave row i's U bytes in lane i's registers, with no exchange between lanes.
// Three register sets form a ring, so two units stay in flight while one is computed.
// The activations of the chunk of tokens being served sit in LDS (staged once per
// chunk) and are read as broadcasts.
// ---------------------------------------------------------------------------------

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
  } else {
    deq32<QT>(w, q, out);
  }
}

// quant/mod.rs:398-407 over a repacked Q8_0 unit: block g adds ws*xs*dot.
template <int TM>
__device__ __forceinline__ void pk_q80_unit(const uint32_t* w, uint32_t nvalid, const int8_t* const* x,
                                            const float* const* xs, float* acc, int m) {
#pragma unroll
  for (int g = 0; g < 8; g++) {
    if ((uint32_t)g < nvalid) {
      const float ws = f16f(w[g / 2] >> (16 * (g % 2)));
      const uint32_t* q = w + 4 + 8 * g;
#pragma unroll
      for (int t = 0; t < TM; t++) {
        if (t < m) {
          const uint32_t* xa = reinterpret_cast<const uint32_t*>(x[t] + 32 * g);
          int dt = 0;
#pragma unroll
          for (int i = 0; i < 8; i++) dt = sdot4(q[i], xa[i], dt);
          acc[t] += ws * xs[t][g] * (float)dt;
        }
      }
    }
  }
}

// One unit's contribution to each chunk member's row dot. x/xs/sm (packed) or x (f32)
// point at the unit's first element; nvalid = blocks of the unit inside the row.
template <int QT, int TM>
__device__ __forceinline__ void unit_packed(const uint32_t* w, uint32_t nvalid, const int8_t* const* x,
                                            const float* const* xs, const uint32_t* const* sm, float* acc, int m) {
  if constexpr (QT == Q8_0) pk_q80_unit<TM>(w, nvalid, x, xs, acc, m);
  else pk_block<QT, TM>(w, x, xs, sm, acc, m);
}

template <int QT, int TM>
__device__ __forceinline__ void unit_f32(const uint32_t* w, uint32_t nvalid, const float* const* x, float* acc, int m) {
  constexpr int NG = UT_<QT>::EU / 32, GPB = QT_<QT>::E / 32;  // groups per unit / per block
#pragma unroll
  for (int q = 0; q < NG; q++) {
    if (UT_<QT>::G == 1 || (uint32_t)(q / GPB) < nvalid) {
      float v[32];
      unit_deq32<QT>(w, q, v);
#pragma unroll
      for (int t = 0; t < TM; t++) {
        if (t < m) {
          const float4* xa = reinterpret_cast<const float4*>(x[t] + 32 * q);
          float a = acc[t];
#pragma unroll
          for (int i = 0; i < 8; i++) {
            float4 xv = xa[i];
            a = fmaf(v[4 * i], xv.x, a);
            a = fmaf(v[4 * i + 1], xv.y, a);
            a = fmaf(v[4 * i + 2], xv.z, a);
            a = fmaf(v[4 * i + 3], xv.w, a);
          }
          acc[t] = a;
        }
      }
    }
  }
}

struct RowIO {
  const uint8_t* const* eptr;
  const uint32_t* active;
  const uint32_t* offsets;
  const uint32_t* slot_tok;
};

// One wave's stream over units [u0, u1) of the tile at `tile`: prime() issues the first
// loads, run(body) calls body(u, w) with the lane's row unit u in w[] for every unit in
// order. Set s of the ring holds units u0+s, u0+s+3, ...; a set is reloaded right after
// its body, so units u+1 and u+2 are in flight during body(u). Every load is
// unconditional (the unit index is clamped to the last unit, a re-read the L2 serves)
// and the loop always runs whole rounds of three, only the bodies past u1 being
// skipped: the loads pending at each use are then the same on every path and the
// compiler waits for exactly the set it uses.
template <int QT>
struct UnitStream {
  static constexpr int NP = UT_<QT>::U / 16, NW = UT_<QT>::U / 4, D = 3;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const uint8_t* src;
  uint32_t u0, u1, ulast;
  u32x4 g[D][NP];

  __device__ __forceinline__ UnitStream(const uint8_t* __restrict__ tile, uint32_t u0_, uint32_t u1_, uint32_t lane)
      : src(tile + lane * 16), u0(u0_), u1(u1_), ulast(u1_ > u0_ ? u1_ - 1 : u0_) {}

  __device__ __forceinline__ void fetch(int s, uint32_t u) {
    const uint8_t* p = src + (size_t)min(u, ulast) * (NP * 1024);
#pragma unroll
    for (int q = 0; q < NP; q++) g[s][q] = *reinterpret_cast<const u32x4*>(p + q * 1024);
  }

  __device__ __forceinline__ void prime() {
    if (u0 >= u1) return;
#pragma unroll
    for (int s = 0; s < D; s++) fetch(s, u0 + s);
  }

  template <class Body>
  __device__ __forceinline__ void run(Body body) {
    if (u0 >= u1) return;
    for (uint32_t u = u0; u < u1; u += D) {
#pragma unroll
      for (int s = 0; s < D; s++) {
        if (u + s < u1) {
          uint32_t w[NW];
#pragma unroll
          for (int q = 0; q < NP; q++) {
            w[4 * q] = g[s][q].x; w[4 * q + 1] = g[s][q].y; w[4 * q + 2] = g[s][q].z; w[4 * q + 3] = g[s][q].w;
          }
          body(u + s, w);
        }
        fetch(s, u + s + D);
      }
    }
  }
};

// Activations of one token chunk over the elements [k0, k0+nelem) a workgroup reads,
// staged in LDS once and read by every lane as broadcasts. Packed: the int8 values, the
// per-32 scales and the sums in the type's form (sum_kind); f32: the values. `row[t]` is
// the token (gate/up) or slot (down) row of chunk member t in the activation arrays,
// whose rows are K long. Each array of a member is padded to 16 bytes.
template <int QT, bool PACKED>
struct ActLds {
  static constexpr uint32_t SW = sum_width(sum_kind<QT>());  // elements per sum word (0: none)
  __host__ __device__ static uint32_t qb(uint32_t nelem) { return (nelem + 15) & ~15u; }
  __host__ __device__ static uint32_t sb(uint32_t nelem) { return (nelem / 32 * 4 + 15) & ~15u; }
  __host__ __device__ static uint32_t hb(uint32_t nelem) { return SW ? (nelem / SW * 4 + 15) & ~15u : 0u; }
  __host__ __device__ static uint32_t bytes(uint32_t tm, uint32_t nelem) {
    if (PACKED) return tm * (qb(nelem) + sb(nelem) + hb(nelem));
    return tm * nelem * 4;
  }
};

template <int QT, int TM>
__device__ __forceinline__ void stage_packed(uint8_t* lds, uint32_t nelem, const int8_t* __restrict__ q,
                                             const float* __restrict__ s, const int32_t* __restrict__ s16,
                                             uint32_t K, const uint32_t* row, int m, uint32_t k0) {
  using A = ActLds<QT, true>;
  constexpr int KIND = sum_kind<QT>();
  const uint32_t qb = A::qb(nelem), sb = A::sb(nelem), hb = A::hb(nelem);
  int8_t* lq = reinterpret_cast<int8_t*>(lds);
  float* ls = reinterpret_cast<float*>(lds + TM * qb);
  uint32_t* lh = reinterpret_cast<uint32_t*>(lds + TM * qb + TM * sb);
  const uint32_t nq4 = nelem / 16, ns = nelem / 32;  // int8 values move 16 at a time
#pragma unroll
  for (int t = 0; t < TM; t++) {
    if (t < m) {
      const uint4* qs = reinterpret_cast<const uint4*>(q + (size_t)row[t] * K + k0);
      for (uint32_t c = threadIdx.x; c < nq4; c += blockDim.x) reinterpret_cast<uint4*>(lq + t * qb)[c] = qs[c];
      const float* ss = s + (size_t)row[t] * (K / 32) + k0 / 32;
      for (uint32_t c = threadIdx.x; c < ns; c += blockDim.x) ls[t * (sb / 4) + c] = ss[c];
      if constexpr (KIND != kSumNone) {
        const int32_t* src = s16 + (size_t)row[t] * (K / 16) + k0 / 16;
        for (uint32_t c = threadIdx.x; c < nelem / A::SW; c += blockDim.x) {
          uint32_t v;
          if constexpr (KIND == kSumF32x32) v = __float_as_uint((float)(src[2 * c] + src[2 * c + 1]));
          else if constexpr (KIND == kSumF32x16) v = __float_as_uint((float)src[c]);
          else v = (uint32_t)src[c];
          lh[t * (hb / 4) + c] = v;
        }
      }
    }
  }
}

template <int TM>
__device__ __forceinline__ void stage_f32(uint8_t* lds, uint32_t nelem, const float* __restrict__ x, uint32_t K,
                                          const uint32_t* row, int m, uint32_t k0) {
  float* lx = reinterpret_cast<float*>(lds);
  const uint32_t n4 = nelem / 4;
#pragma unroll
  for (int t = 0; t < TM; t++) {
    if (t < m) {
      const float4* xs = reinterpret_cast<const float4*>(x + (size_t)row[t] * K + k0);
      for (uint32_t c = threadIdx.x; c < n4; c += blockDim.x) reinterpret_cast<float4*>(lx + t * nelem)[c] = xs[c];
    }
  }
}

// Runs unit u's body over the staged activations, whose first element is unit ubase's.
template <int QT, int TM, bool PACKED>
__device__ __forceinline__ void staged_unit(const uint32_t* w, uint8_t* lds, uint32_t nelem, uint32_t u,
                                            uint32_t ubase, uint32_t nblk, float* acc, int m) {
  constexpr int EU = UT_<QT>::EU, G = UT_<QT>::G;
  const uint32_t off = (u - ubase) * EU;
  const uint32_t nvalid = G == 1 ? 1u : min((uint32_t)G, nblk - u * G);
  if constexpr (PACKED) {
    using A = ActLds<QT, true>;
    const uint32_t qb = A::qb(nelem), sb = A::sb(nelem), hb = A::hb(nelem);
    const int8_t* lq = reinterpret_cast<const int8_t*>(lds);
    const float* ls = reinterpret_cast<const float*>(lds + TM * qb);
    const uint32_t* lh = reinterpret_cast<const uint32_t*>(lds + TM * qb + TM * sb);
    const int8_t* xb[TM];
    const float* sbp[TM];
    const uint32_t* hbp[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) {
      xb[t] = lq + t * qb + off;
      sbp[t] = ls + t * (sb / 4) + off / 32;
      hbp[t] = lh + t * (hb / 4) + (A::SW ? off / A::SW : 0);
    }
    unit_packed<QT, TM>(w, nvalid, xb, sbp, hbp, acc, m);
  } else {
    const float* lx = reinterpret_cast<const float*>(lds);
    const float* xb[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) xb[t] = lx + t * nelem + off;
    unit_f32<QT, TM>(w, nvalid, xb, acc, m);
  }
}

template <int QT>
__host__ __device__ constexpr uint32_t unit_blocks(uint32_t cols) { return cols / (UT_<QT>::EU / UT_<QT>::G); }
template <int QT>
__host__ __device__ constexpr uint32_t unit_count(uint32_t cols) {
  return (unit_blocks<QT>(cols) + UT_<QT>::G - 1) / UT_<QT>::G;
}

// Gate/up: the workgroup's first KG waves stream the tile of the gate matrix, the next
// KG the same rows of the up matrix, wave j of a matrix taking the j-th of KG
// consecutive K ranges; each lane runs its row's dot over its range in K order and the
// KG partial sums are added in range order. h = silu(g)*u; under packed math h is then
// quantised per 32 rows for the down product (quant/mod.rs:331-345). With KG = 1, g
// and u are quant::matmul's row dots term for term (quant/mod.rs:266-279).
// grid.x = row tiles, grid.y = active-expert slot.
template <int QT, int TM, bool PACKED, int KG>
__global__ void __launch_bounds__(128 * KG, 2)
k_gu_units(RowIO io, uint32_t ne, uint32_t f, uint32_t d, const int8_t* __restrict__ xq, const float* __restrict__ xs,
           const int32_t* __restrict__ x16, const float* __restrict__ hs, int8_t* __restrict__ hq,
           float* __restrict__ hsc, int32_t* __restrict__ h16, float* __restrict__ hf) {
  constexpr int U = UT_<QT>::U;
  extern __shared__ uint4 dsm[];
  float* part = reinterpret_cast<float*>(dsm);  // [2*KG][TM][64] per-wave row sums
  uint8_t* acts = reinterpret_cast<uint8_t*>(part + 2 * KG * TM * 64);
  const uint32_t a = blockIdx.y;
  if (a >= io.active[0]) return;
  const uint32_t e = io.active[1 + a];
  const uint32_t s0 = io.offsets[e], m_all = io.offsets[e + 1] - s0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t mat = wave / KG, kp = wave % KG;
  const uint32_t r0 = blockIdx.x * kTileRows;
  const uint32_t nblk = unit_blocks<QT>(d), nunit = unit_count<QT>(d);
  const uint32_t u0 = nunit * kp / KG, u1 = nunit * (kp + 1) / KG;
  UnitStream<QT> st(io.eptr[mat * ne + e] + (size_t)blockIdx.x * nunit * kTileRows * U, u0, u1, lane);
  for (uint32_t c0 = 0; c0 < m_all; c0 += TM) {
    const int m = (int)min((uint32_t)TM, m_all - c0);
    st.prime();  // the weights' first loads overlap the staging of the activations
    uint32_t tok[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) tok[t] = io.slot_tok[s0 + c0 + (t < m ? t : 0)];
    if constexpr (PACKED) stage_packed<QT, TM>(acts, d, xq, xs, x16, d, tok, m, 0);
    else stage_f32<TM>(acts, d, hs, d, tok, m, 0);
    __syncthreads();
    float acc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc[t] = 0.0f;
    st.run([&](uint32_t u, const uint32_t* w) { staged_unit<QT, TM, PACKED>(w, acts, d, u, 0, nblk, acc, m); });
#pragma unroll
    for (int t = 0; t < TM; t++) part[(wave * TM + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (wave == 0) {
      const bool valid = r0 + (lane & 32) + 32 <= f;  // this lane's 32-row block lies inside d_ff
#pragma unroll
      for (int t = 0; t < TM; t++) {
        if (t < m) {
          float g = part[t * 64 + lane], u = part[(KG * TM + t) * 64 + lane];
#pragma unroll
          for (int j = 1; j < KG; j++) {
            g += part[(j * TM + t) * 64 + lane];
            u += part[((KG + j) * TM + t) * 64 + lane];
          }
          const float h = swiglu(g, u);
          const size_t slot = s0 + c0 + t;
          if (hf && r0 + lane < f) hf[slot * f + r0 + lane] = h;
          if (hq) quant_wave(h, lane, valid, hq + slot * f + r0, hsc + slot * (f / 32) + r0 / 32, h16 + slot * (f / 16) + r0 / 16);
        }
      }
    }
    __syncthreads();  // part[] and the staged activations are reused by the next chunk
  }
}

// Down: the row's units are split over gridDim.y workgroups of KS waves each. A
// workgroup adds its waves' partial sums in wave order and writes them to its own
// partial slice y[blockIdx.y]; the combine adds the slices in order.
// grid.x = row tiles of d_model, grid.y = K groups, grid.z = active-expert slot.
template <int QT, int TM, bool PACKED, int KS>
__global__ void __launch_bounds__(64 * KS, 2)
k_dn_units(RowIO io, uint32_t ne, uint32_t f, uint32_t d, uint32_t part_stride, const int8_t* __restrict__ hq,
           const float* __restrict__ hsc, const int32_t* __restrict__ h16, const float* __restrict__ hf,
           float* __restrict__ ypart) {
  constexpr int U = UT_<QT>::U, EU = UT_<QT>::EU;
  extern __shared__ uint4 dsm[];
  float* red = reinterpret_cast<float*>(dsm);  // [KS][TM][64]
  uint8_t* acts = reinterpret_cast<uint8_t*>(red + KS * TM * 64);
  const uint32_t a = blockIdx.z;
  if (a >= io.active[0]) return;
  const uint32_t e = io.active[1 + a];
  const uint32_t s0 = io.offsets[e], m_all = io.offsets[e + 1] - s0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t r0 = blockIdx.x * kTileRows;
  const uint32_t nblk = unit_blocks<QT>(f), nunit = unit_count<QT>(f);
  const uint32_t nsl = gridDim.y * KS, sl = blockIdx.y * KS + wave;
  const uint32_t u0 = (nunit * sl) / nsl, u1 = (nunit * (sl + 1)) / nsl;
  // the workgroup's unit range: its first wave's start to its last wave's end
  const uint32_t uw0 = (nunit * (blockIdx.y * KS)) / nsl, uw1 = (nunit * (blockIdx.y * KS + KS)) / nsl;
  const uint32_t nelem = min(uw1 * EU, f) - min(uw0 * EU, f);
  float* y = ypart + (size_t)blockIdx.y * part_stride;
  UnitStream<QT> st(io.eptr[2 * ne + e] + (size_t)blockIdx.x * nunit * kTileRows * U, u0, u1, lane);
  for (uint32_t c0 = 0; c0 < m_all; c0 += TM) {
    const int m = (int)min((uint32_t)TM, m_all - c0);
    st.prime();  // the weights' first loads overlap the staging of the activations
    uint32_t slot[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) slot[t] = s0 + c0 + (t < m ? t : 0);
    if (nelem) {
      if constexpr (PACKED) stage_packed<QT, TM>(acts, nelem, hq, hsc, h16, f, slot, m, uw0 * EU);
      else stage_f32<TM>(acts, nelem, hf, f, slot, m, uw0 * EU);
    }
    __syncthreads();
    float acc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc[t] = 0.0f;
    st.run([&](uint32_t u, const uint32_t* w) { staged_unit<QT, TM, PACKED>(w, acts, nelem, u, uw0, nblk, acc, m); });
#pragma unroll
    for (int t = 0; t < TM; t++) red[(wave * TM + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (wave == 0) {
      uint32_t row = r0 + lane;
#pragma unroll
      for (int t = 0; t < TM; t++) {
        float sacc = red[t * 64 + lane];
#pragma unroll
        for (int w2 = 1; w2 < KS; w2++) sacc += red[(w2 * TM + t) * 64 + lane];
        if (t < m && row < d) y[(size_t)(s0 + c0 + t) * d + row] = sacc;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------------

constexpr uint32_t kLdsBudget = 160 * 1024 - 2048;


template <class K>
static bool allow_lds(K kernel) {
  // raise the dynamic LDS limit of one instantiation (called once per instantiation)
  return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBudget) ==
         hipSuccess;
}

// largest chunk of tokens <= want whose staging fits the LDS budget
template <class F>
static int fit_tm(int want, F lds_of) {
  int tm = want;
  while (tm > 1 && lds_of((uint32_t)tm) > kLdsBudget) tm /= 2;
  return tm;
}

template <int QT, bool PACKED>
static uint32_t gu_lds(uint32_t tm, uint32_t kg, uint32_t d) {
  return 2 * kg * tm * 64 * 4 + ActLds<QT, PACKED>::bytes(tm, d);
}

template <int QT, int TM, bool PACKED, int KG>
static void go_gu(const LayerDev& L, const FwdBufs& B, dim3 g, hipStream_t st) {
  RowIO io{L.eptr, B.active, B.offsets, B.slot_tok};
  static const bool once = allow_lds(k_gu_units<QT, TM, PACKED, KG>);
  (void)once;
  const uint32_t lds = gu_lds<QT, PACKED>(TM, KG, L.d);
  hipLaunchKernelGGL((k_gu_units<QT, TM, PACKED, KG>), g, dim3(128 * KG), lds, st, io, L.ne, L.f, L.d, B.xq, B.xs,
                     B.x16, B.hs, B.hq, B.hsc, B.h16, B.hf);
}

// Waves per matrix of a gate/up workgroup: enough workgroups' waves to give every SIMD
// two, each wave still streaming at least 4 units (decode batches of one or two tokens
// are the ones that need it). Under packed math h is requantised per 32 values, and a
// g or u summed in another order can move a block's scale and with it every value of
// the block, so packed math keeps each row's dot in one wave, in K order.
template <int QT, bool PACKED>
static int pick_kg(const LayerDev& L, uint32_t n, int tm) {
  if (PACKED) return 1;
  const uint32_t waves = ((L.f + kTileRows - 1) / kTileRows) * min(L.ne, n * L.k) * 2;
  const uint32_t nunit = unit_count<QT>(L.d);
  int kg = 1;
  while (kg < (tm == 1 ? 4 : tm == 2 ? 2 : 1) && waves * kg < 2048 && nunit / (2 * kg) >= 4 &&
         gu_lds<QT, PACKED>(tm, 2 * kg, L.d) <= kLdsBudget)
    kg *= 2;
  return kg;
}

// Tokens per pass: the decode batch, capped at 8 (packed) or 4 (f32 math, whose body
// holds a dequantised group of 32 values besides the accumulators).
template <bool PACKED>
static inline int pick_tm(uint32_t n) {
  return n <= 1 ? 1 : n <= 2 ? 2 : (n <= 4 || !PACKED) ? 4 : 8;
}

template <int QT, bool PACKED>
static void go_gu_tm(const LayerDev& L, const FwdBufs& B, dim3 g, uint32_t n, hipStream_t st) {
  const int tm = fit_tm(pick_tm<PACKED>(n), [&](uint32_t t) { return gu_lds<QT, PACKED>(t, 1, L.d); });
  const int kg = pick_kg<QT, PACKED>(L, n, tm);
  if constexpr (!PACKED) {
    if (kg > 1) {
      switch (tm * 8 + kg) {
        case 1 * 8 + 2: go_gu<QT, 1, PACKED, 2>(L, B, g, st); return;
        case 1 * 8 + 4: go_gu<QT, 1, PACKED, 4>(L, B, g, st); return;
        default: go_gu<QT, 2, PACKED, 2>(L, B, g, st); return;
      }
    }
  }
  switch (tm) {
    case 1: go_gu<QT, 1, PACKED, 1>(L, B, g, st); break;
    case 2: go_gu<QT, 2, PACKED, 1>(L, B, g, st); break;
    case 4: go_gu<QT, 4, PACKED, 1>(L, B, g, st); break;
    default:
      if constexpr (PACKED) go_gu<QT, 8, PACKED, 1>(L, B, g, st);
      break;
  }
}

// LDS of the down product: a workgroup stages at most ceil(units/ksg) + 1 units
template <int QT, bool PACKED>
static uint32_t dn_lds(uint32_t tm, uint32_t f, uint32_t ksg) {
  const uint32_t span = min(((unit_count<QT>(f) + ksg - 1) / ksg + 1) * UT_<QT>::EU, f);
  return kDnKS * tm * 64 * 4 + ActLds<QT, PACKED>::bytes(tm, span);
}

template <int QT, int TM, bool PACKED>
static void go_dn(const LayerDev& L, const FwdBufs& B, dim3 g, uint32_t n, hipStream_t st) {
  RowIO io{L.eptr, B.active, B.offsets, B.slot_tok};
  static const bool once = allow_lds(k_dn_units<QT, TM, PACKED, kDnKS>);
  (void)once;
  const uint32_t lds = dn_lds<QT, PACKED>(TM, L.f, g.y);
  hipLaunchKernelGGL((k_dn_units<QT, TM, PACKED, kDnKS>), g, dim3(64 * kDnKS), lds, st, io, L.ne, L.f, L.d,
                     n * L.k * L.d, B.hq, B.hsc, B.h16, B.hf, B.y);
}

template <int QT, bool PACKED>
static void go_dn_tm(const LayerDev& L, const FwdBufs& B, dim3 g, int want, uint32_t n, hipStream_t st) {
  switch (fit_tm(want, [&](uint32_t t) { return dn_lds<QT, PACKED>(t, L.f, g.y); })) {
    case 1: go_dn<QT, 1, PACKED>(L, B, g, n, st); break;
    case 2: go_dn<QT, 2, PACKED>(L, B, g, n, st); break;
    case 4: go_dn<QT, 4, PACKED>(L, B, g, n, st); break;
    default:
      if constexpr (PACKED) go_dn<QT, 8, PACKED>(L, B, g, n, st);
      break;
  }
}

template <int QT>
hipError_t units_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  const dim3 g((L.f + kTileRows - 1) / kTileRows, min(L.ne, n * L.k));
  if constexpr (has_int8_kernel(QT)) {
    if (L.math == 0) go_gu_tm<QT, true>(L, B, g, n, st);
    else go_gu_tm<QT, false>(L, B, g, n, st);
  } else {
    go_gu_tm<QT, false>(L, B, g, n, st);
  }
  return hipGetLastError();
}

template <int QT>
hipError_t units_down(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st) {
  const dim3 g((L.d + kTileRows - 1) / kTileRows, ksg, min(L.ne, n * L.k));
  if constexpr (has_int8_kernel(QT)) {
    if (L.math == 0) go_dn_tm<QT, true>(L, B, g, pick_tm<true>(n), n, st);
    else go_dn_tm<QT, false>(L, B, g, pick_tm<false>(n), n, st);
  } else {
    go_dn_tm<QT, false>(L, B, g, pick_tm<false>(n), n, st);
  }
  return hipGetLastError();
}

template hipError_t units_gateup<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, hipStream_t);
template hipError_t units_down<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, uint32_t, hipStream_t);

}  // namespace gmoe
