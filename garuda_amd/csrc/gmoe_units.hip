// gmoe_units.hip — the expert products (gate/up with SwiGLU, down) over the tiled slab.
//
// Compiled once per block type, with -DGMOE_QT=<ggml type id>: each object holds the
// kernels of one type and the explicit instantiations of units_gateup/units_down for it,
// so the instantiations build in parallel.
//
// Reference semantics: llama/mod.rs:1002-1020 via quant::matmul (quant/mod.rs:223-304)
// under packed math, or simd::matmul over dequantised weights (simd/mod.rs:96-129).
#include "gmoe_unit.h"

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
// Register sets form a ring (two; four for single-token gate/up), so the next units'
// loads are in flight while one is computed.
// The activations of the chunk of tokens being served sit in LDS (staged once per
// chunk) and are read as broadcasts.
// ---------------------------------------------------------------------------------

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


// Activations of one chunk of tokens over the elements [k0, k0+nelem) a workgroup reads,
// staged in LDS once per chunk and read by every lane as broadcasts, token after token
// (`per_token` bytes each). Packed: the int8 values, the per-32 scales, and the sums in
// the type's form (sum_kind), each array padded to 16 bytes; f32: the values.
template <int QT, bool PACKED>
struct ActLds {
  static constexpr uint32_t SW = sum_width(sum_kind<QT>());  // elements per sum word (0: none)
  __host__ __device__ static uint32_t qb(uint32_t nelem) { return (nelem + 15) & ~15u; }
  __host__ __device__ static uint32_t sb(uint32_t nelem) { return (nelem / 32 * 4 + 15) & ~15u; }
  __host__ __device__ static uint32_t hb(uint32_t nelem) { return SW ? (nelem / SW * 4 + 15) & ~15u : 0u; }
  __host__ __device__ static uint32_t per_token(uint32_t nelem) {
    return PACKED ? qb(nelem) + sb(nelem) + hb(nelem) : nelem * 4;
  }
};

// Stages tokens 0..m-1 of a chunk. rows[t] (LDS) is token t's row in the activation
// arrays, whose rows are K long; the sums are already in the type's form (the quantisers
// write them so). Packed with q null: quantised here from the f32 rows x. Every thread
// issues up to four loads before it stores, over the chunk's tokens flattened, so the
// chunk costs about one memory round trip.
template <int QT, bool PACKED>
__device__ __forceinline__ void stage_acts(uint8_t* lds, uint32_t nelem, uint32_t m, const uint32_t* rows, uint32_t K,
                                           uint32_t k0, const int8_t* __restrict__ q, const float* __restrict__ s,
                                           const uint32_t* __restrict__ sums, const float* __restrict__ x) {
  using A = ActLds<QT, PACKED>;
  const uint32_t per = A::per_token(nelem), bd = blockDim.x;
  // copies n items of `width` elements of type T per token: item c of token t comes from
  // src(row, c) and goes to byte dst_off + c * sizeof(T) of the token's LDS region
  auto copy = [&](uint32_t n, uint32_t dst_off, auto src) {
    using T = decltype(src(0u, 0u));
    const uint32_t total = m * n;
    for (uint32_t i0 = threadIdx.x; i0 < total; i0 += 4 * bd) {
      T v[4];
      uint32_t at[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t i = i0 + j * bd;
        if (i < total) {
          const uint32_t t = i / n, c = i - t * n;
          v[j] = src(rows[t], c);
          at[j] = t * per + dst_off + c * (uint32_t)sizeof(T);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (i0 + j * bd < total) *reinterpret_cast<T*>(lds + at[j]) = v[j];
    }
  };
  if constexpr (PACKED) {
    constexpr int KIND = sum_kind<QT>();
    if (!q) {
      // f32 activations (a dense call): each thread quantises 32-blocks into the token's
      // LDS region with quant32's arithmetic, so the values match k_quant_act's bit for bit
      const uint32_t nb = nelem / 32, total = m * nb;
      for (uint32_t i = threadIdx.x; i < total; i += bd) {
        const uint32_t t = i / nb, b = i - t * nb;
        const float4* src = reinterpret_cast<const float4*>(x + (size_t)rows[t] * K + k0 + 32 * b);
        float v[32];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float4 f = src[j];
          v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
        }
        uint32_t pk[8];
        float sc;
        int s0, s1;
        quant32_regs(v, pk, &sc, &s0, &s1);
        uint8_t* tok = lds + t * per;
        uint4* qd = reinterpret_cast<uint4*>(tok + 32 * b);
        qd[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        qd[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        reinterpret_cast<float*>(tok + A::qb(nelem))[b] = sc;
        uint32_t* hs = reinterpret_cast<uint32_t*>(tok + A::qb(nelem) + A::sb(nelem));
        if constexpr (KIND == kSumF32x32) hs[b] = __float_as_uint((float)(s0 + s1));
        else if constexpr (KIND == kSumF32x16) {
          hs[2 * b] = __float_as_uint((float)s0);
          hs[2 * b + 1] = __float_as_uint((float)s1);
        } else if constexpr (KIND == kSumI32x16) {
          hs[2 * b] = (uint32_t)(sum_offset<QT>() * s0);
          hs[2 * b + 1] = (uint32_t)(sum_offset<QT>() * s1);
        }
      }
      return;
    }
    copy(nelem / 16, 0u, [&](uint32_t r, uint32_t c) {
      return reinterpret_cast<const uint4*>(q + (size_t)r * K + k0)[c];
    });
    copy(nelem / 32, A::qb(nelem), [&](uint32_t r, uint32_t c) { return s[(size_t)r * (K / 32) + k0 / 32 + c]; });
    if constexpr (KIND != kSumNone) {
      copy(nelem / A::SW, A::qb(nelem) + A::sb(nelem),
           [&](uint32_t r, uint32_t c) { return sums[(size_t)r * (K / A::SW) + k0 / A::SW + c]; });
    }
  } else {
    copy(nelem / 4, 0u, [&](uint32_t r, uint32_t c) {
      return reinterpret_cast<const float4*>(x + (size_t)r * K + k0)[c];
    });
  }
}

// Unit u's share of every token of the chunk (`my[t * 64]` holds token t's running row
// sum; token t's staged activations start at acts + t * per, whose first element is unit
// ubase's). Packed: the token loop runs over whole units, the row sum in a register
// across each (the unit's decoded quants and scales stay in registers across the loop;
// running the sub-block groups outermost instead, the sums read and written in LDS per
// group, measured slower: C4 225 -> 305 us). f32: the dequantised values of one 32-value
// group at a time, each group applied to every token, in group order.
template <int QT, bool PACKED, int PIPE = 0>
__device__ __forceinline__ void unit_tokens(const uint32_t* w, const uint8_t* acts, uint32_t per, uint32_t nelem,
                                            uint32_t u, uint32_t ubase, uint32_t nblk, float* my, uint32_t m) {
  if constexpr (PACKED) {
    using A = ActLds<QT, true>;
    constexpr int EU = UT_<QT>::EU, G = UT_<QT>::G;
    const uint32_t off = (u - ubase) * EU;
    const uint32_t nvalid = G == 1 ? 1u : min((uint32_t)G, nblk - u * G);
    const uint32_t o_s = A::qb(nelem) + off / 8, o_h = A::qb(nelem) + A::sb(nelem) + (A::SW ? off / A::SW * 4 : 0u);
    for (uint32_t t = 0; t < m; t++) {
      const uint8_t* tok = acts + t * per;
      float acc = my[t * 64];
      const PkTok a{reinterpret_cast<const int8_t*>(tok) + off, reinterpret_cast<const float*>(tok + o_s),
                    reinterpret_cast<const uint32_t*>(tok + o_h), &acc};
      pk_unit<QT, PIPE>(w, nvalid, 1u, [&](uint32_t) { return a; });
      my[t * 64] = acc;
    }
  } else {
    constexpr int NG = UT_<QT>::EU / 32, GPB = QT_<QT>::E / 32;  // groups per unit / per block
    const uint32_t off = (u - ubase) * UT_<QT>::EU;
    const uint32_t nvalid = UT_<QT>::G == 1 ? 1u : min((uint32_t)UT_<QT>::G, nblk - u * UT_<QT>::G);
#pragma unroll
    for (int q = 0; q < NG; q++) {
      if (UT_<QT>::G == 1 || (uint32_t)(q / GPB) < nvalid) {
        float v[32];
        unit_deq32<QT>(w, q, v);
        for (uint32_t t = 0; t < m; t++) {
          const float4* xa = reinterpret_cast<const float4*>(acts + t * per) + (off + 32 * q) / 4;
          float a = my[t * 64];
#pragma unroll
          for (int i = 0; i < 8; i++) {
            float4 xv = xa[i];
            a = fmaf(v[4 * i], xv.x, a);
            a = fmaf(v[4 * i + 1], xv.y, a);
            a = fmaf(v[4 * i + 2], xv.z, a);
            a = fmaf(v[4 * i + 3], xv.w, a);
          }
          my[t * 64] = a;
        }
      }
    }
  }
}

// Gate/up: wave 0 streams the tile of the gate matrix, wave 1 the same rows of the up
// matrix. The expert's tokens go in chunks of at most mt; for each unit the lane adds
// the unit's terms for every token of the chunk to that token's running row sum (kept
// in LDS between units), so each row's dot runs in K order and g and u are
// quant::matmul's row dots term for term (quant/mod.rs:266-279). h = silu(g)*u; under
// packed math h is then quantised per 32 rows for the down product
// (quant/mod.rs:331-345). grid.x = row tiles, grid.y = active-expert slot.
//
// With ra.n > 0 (speculative decode) the last row of the grid is the exact routing
// instead: workgroup x < n*ne runs route_logit for token x / ne, expert x % ne. The
// dispatcher starts it with the last wave of expert workgroups, whose tail hides it.
template <int QT, bool PACKED, int D, int TPW = 1, int PIPE = 0>
__global__ void __launch_bounds__(128 * TPW, D > 2 ? 1 : (TPW > 1 ? 3 : 2))
k_gu_units(const ExpertWork* __restrict__ work, uint32_t ne, const uint32_t* __restrict__ slot_tok, uint32_t f,
           uint32_t d, uint32_t mt, const int8_t* __restrict__ xq,
           const float* __restrict__ xs, const uint32_t* __restrict__ xsum, const float* __restrict__ hs,
           int8_t* __restrict__ hq, float* __restrict__ hsc, uint32_t* __restrict__ hsum, float* __restrict__ hf,
           int hkind, int32_t hoff, RouteArgs ra) {
  constexpr int U = UT_<QT>::U;
  extern __shared__ uint4 dsm[];
  if (ra.n) {
    if (blockIdx.y == gridDim.y - 1) {
      if (blockIdx.x < ra.n * ra.ne) route_logit(ra, blockIdx.x, reinterpret_cast<float*>(dsm));
      return;
    }
  }
  float* accs = reinterpret_cast<float*>(dsm);                 // [2 TPW][mt][64] running row sums
  uint32_t* rows = reinterpret_cast<uint32_t*>(accs + 2 * TPW * mt * 64);  // [mt] token of each chunk member
  uint8_t* acts = reinterpret_cast<uint8_t*>(rows + ((mt + 3) & ~3u));
  if (blockIdx.x * TPW * kTileRows >= f) return;  // (the routing row may widen the grid)
  // active experts y0, y0 + ny, ... (the grid is sized for the usual count; rare extra
  // candidates are taken by the same workgroups)
  const uint32_t y0 = blockIdx.y, ny = gridDim.y - (ra.n ? 1 : 0);
  for (uint32_t a = y0; a < ne; a += ny) {
  const ExpertWork* W = work + a;  // field by field: scalar loads
  const uint32_t m_all = W->m;
  if (m_all == 0) break;
  const uint32_t s0 = W->s0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // wave 2i streams gate, wave 2i+1 up, of tile TPW * blockIdx.x + i
  const uint32_t tile = blockIdx.x * TPW + wave / 2, r0 = tile * kTileRows;
  const bool tv = r0 < f;  // (a last workgroup of TPW > 1 may hold a tile past d_ff)
  const uint32_t nblk = unit_blocks<QT>(d), nunit = unit_count<QT>(d);
  const uint32_t per = ActLds<QT, PACKED>::per_token(d);
  float* my = accs + wave * mt * 64 + lane;  // token t's sum of this lane's row: my[t * 64]
  const uint8_t* mat = W->w[wave & 1];
  UnitStream<QT, D> st(mat + (size_t)(tv ? tile : 0) * nunit * kTileRows * U, 0, tv ? nunit : 0, lane);
  for (uint32_t c0 = 0; c0 < m_all; c0 += mt) {
    const uint32_t m = min(mt, m_all - c0);
    st.prime();  // the weights' first loads overlap the staging of the activations
    for (uint32_t t = threadIdx.x; t < m; t += blockDim.x) rows[t] = slot_tok[s0 + c0 + t];
    for (uint32_t t = 0; t < m; t++) my[t * 64] = 0.0f;
    __syncthreads();
    stage_acts<QT, PACKED>(acts, d, m, rows, d, 0, xq, xs, xsum, hs);
    __syncthreads();
    st.run([&](uint32_t u, const uint32_t* w) { unit_tokens<QT, PACKED, PIPE>(w, acts, per, d, u, 0, nblk, my, m); });
    __syncthreads();
    if ((wave & 1) == 0 && tv) {
      const bool valid = r0 + (lane & 32) + 32 <= f;  // this lane's 32-row block lies inside d_ff
      for (uint32_t t = 0; t < m; t++) {
        const float h = swiglu(my[t * 64], my[(mt + t) * 64]);  // the up wave's sums follow
        const size_t slot = s0 + c0 + t;
        if (hf && r0 + lane < f) hf[slot * f + r0 + lane] = h;
        if (hq)
          quant_wave(h, lane, valid, hq + slot * f + r0, hsc + slot * (f / 32) + r0 / 32,
                     hkind ? hsum + slot * (f / sum_width(hkind)) : nullptr, r0, hkind, hoff);
      }
    }
    __syncthreads();  // the sums and the staged activations are reused by the next chunk
  }
  }
}

// Terms a packed unit adds to a row's dot: one per sub-block (Q4_K, Q5_K: 8 of 32 values;
// Q6_K, Q3_K, Q2_K: 16 of 16), or one per block of the eight-block Q8_0 units.
template <int QT>
__host__ __device__ constexpr uint32_t unit_terms() {
  return (QT == Q4_K || QT == Q5_K || QT == Q8_0) ? 8u : 16u;
}

// Gate/up for single-token calls (decode batch 1): a workgroup of 8 waves takes one
// 64-row tile, waves 0-3 the gate matrix and waves 4-7 the up matrix, each wave a quarter
// of the K range. A wave holds a quarter of the units a one-wave stream would, so every
// SIMD keeps several streams in flight and their arithmetic overlaps the loads (two
// workgroups a CU). Bit-exact with k_gu_units: each wave writes its units' terms (pk_unit
// with PkTerms, every term evaluated as the reference writes it) to LDS, and waves 0 and
// 4 then add a row's terms in K order from 0.0, the reference's row dot
// (quant/mod.rs:266-279); h = silu(g) * u is quantised per 32 rows by wave 0.
// Measured on the C2 layer at one token: gate/up 33.9 -> 31.5 us a call. With two tokens
// (both tokens' terms in LDS: one workgroup a CU) the same split took 67 us against 55.
// With ra.n > 0 (speculative decode) the last row of the grid is the exact routing:
// workgroup x < n routes token x (route_token), hidden under the expert tiles.
// With SELF the call's front end is folded in: every workgroup computes the router's
// parallel dots and the candidate test itself (spec_dots, spec_candidates, as the
// speculative front end does), so it knows which candidate its slot streams without a
// dispatch through memory, and quantises the token into LDS itself (stage_acts from the
// f32 row: quant32's arithmetic, the front end's codes bit for bit). Workgroup x = 0 of
// each slot writes that slot's work record and pair for the down product; the routing
// workgroup zeroes the output the down product adds into and writes the dispatch
// summary (active experts, offsets, empty work records past the candidates).
// grid.x = row tiles of d_ff, grid.y = active-expert slot (+ the routing row).
struct SelfArgs {
  const uint8_t* const* eptr;  // [3][ne] tiled gate, up, down of each expert
  ExpertWork* work;
  uint32_t* slot_tok;
  uint32_t* active;
  uint32_t* offsets;
  float* out;  // zeroed for the down product that adds into it, or null
};

struct SplitArgs {
  const ExpertWork* work;
  const uint32_t* slot_tok;
  const int8_t* xq;
  const float* xs;
  const uint32_t* xsum;
  int8_t* hq;
  float* hsc;
  uint32_t* hsum;
  uint32_t ne, d, f, rsec;
  int hkind;
  int32_t hoff;
};
constexpr uint32_t kSplitWaves = 8, kSplitParts = 4;
constexpr int kSplitLoads = 8;  // float4 pairs a lane has in flight in its router dots (SELF)

template <int QT, bool SELF>
__global__ void __launch_bounds__(64 * kSplitWaves, 4) k_gu_split(SplitArgs A, RouteArgs ra, SelfArgs S) {
  constexpr int U = UT_<QT>::U, EU = UT_<QT>::EU;
  constexpr uint32_t NT = unit_terms<QT>();
  using Act = ActLds<QT, true>;
  extern __shared__ uint4 dsm[];
  __shared__ float s_lt[kSpecMaxExperts], s_la[kSpecMaxExperts];
  __shared__ uint32_t s_cl[kSpecMaxExperts], s_nc;
  __shared__ double s_sb[2 * kSpecMaxExperts];
  float* lds = reinterpret_cast<float*>(dsm);
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint32_t mat = wave / kSplitParts, part = wave % kSplitParts;
  const bool route_row = ra.n && blockIdx.y == gridDim.y - 1;
  const uint32_t nunit = unit_count<QT>(A.d), nterm = nunit * NT;
  const uint32_t u0 = nunit * part / kSplitParts, u1 = nunit * (part + 1) / kSplitParts;
  const size_t toff = (size_t)blockIdx.x * nunit * kTileRows * U;  // the tile's offset in a matrix
  UnitStream<QT, 1> st(reinterpret_cast<const uint8_t*>(A.work), u0, u0, lane);  // empty until set
  uint32_t nc = 0, pred = ~0u;  // SELF: the candidate count, slot blockIdx.y's predicted expert
  const uint8_t* ep = nullptr;  // SELF: lane e's expert matrix of this wave (wave 0: gate, up, down below)
  const uint8_t* ep3[3] = {nullptr, nullptr, nullptr};
  if constexpr (SELF) {
    if (route_row ? blockIdx.x != 0 : blockIdx.x * kTileRows >= A.f) return;
    if (lane < ra.ne) {
      ep = S.eptr[mat * ra.ne + lane];
      if (wave == 0)
        for (int p = 0; p < 3; p++) ep3[p] = S.eptr[p * ra.ne + lane];
    }
    spec_dots<kSplitLoads>(ra.router, ra.hs, ra.ne, ra.d, s_lt, s_la);
    __syncthreads();
    // the candidate test's usual outcome is the top k of the parallel logits: slot y's
    // predicted expert is the y-th lowest id among them, whose stream is primed before the
    // test (and primed again in the rare call where the test names another)
    if (!route_row) {
      const float le = lane < ra.ne ? s_lt[lane] : 0.0f;
      uint32_t r = 0;
      for (uint32_t j = 0; j < ra.ne; j++) {
        const float lj = s_lt[j];
        r += (lj > le || (lj == le && j < lane)) ? 1u : 0u;
      }
      const uint64_t top = __ballot(lane < ra.ne && r < ra.k);
      if ((uint32_t)__popcll(top) > blockIdx.y) {
        uint64_t m = top;
        for (uint32_t i = 0; i < blockIdx.y; i++) m &= m - 1;
        pred = (uint32_t)__ffsll((unsigned long long)m) - 1;
        if (blockIdx.x * kTileRows < A.f) {
          st = UnitStream<QT, 1>(reinterpret_cast<const uint8_t*>(__shfl(reinterpret_cast<uintptr_t>(ep), (int)pred)) + toff,
                                 u0, u1, lane);
          st.prime();
        }
      }
    }
    if (wave == 0) {
      bool c;
      uint32_t p;
      const uint32_t q = spec_candidates<kSplitLoads>(ra.ne, ra.k, ra.d, ra.gating, s_lt, s_la, s_sb, s_cl, lane, &c, &p);
      if (lane == 0) s_nc = q;
    }
    __syncthreads();
    nc = s_nc;
  }
  if (route_row) {
    if constexpr (SELF) {
      // the dispatch summary of the candidates, as the front end writes it for one token,
      // and the output rows the down product adds into
      if (wave == 0 && lane < ra.ne) {
        uint32_t below = 0;
        for (uint32_t j = 0; j < nc; j++) below += s_cl[j] < lane ? 1u : 0u;
        S.offsets[lane] = below;
        if (lane < nc) S.active[1 + lane] = s_cl[lane];
        if (lane >= nc) S.work[lane].m = 0;
        if (lane == 0) {
          S.offsets[ra.ne] = nc;
          S.active[0] = nc;
        }
      }
      if (S.out)
        for (uint32_t c = tid; c < ra.d; c += blockDim.x) S.out[c] = 0.0f;
      route_token(ra, 0, lds, A.rsec, nullptr, s_cl, nc);
    } else {
      if (blockIdx.x < ra.n) route_token(ra, blockIdx.x, lds, A.rsec, nullptr);
    }
    return;
  }
  const uint32_t r0 = blockIdx.x * kTileRows;
  if (r0 >= A.f) return;  // (the routing row may widen the grid)
  // LDS: terms [2 matrices][nterm][64], u's row sums [64], the token's row, and its staged
  // activations
  float* terms = lds;
  float* usum = terms + (size_t)2 * nterm * 64;
  uint32_t* rows = reinterpret_cast<uint32_t*>(usum + 64);
  uint8_t* acts = reinterpret_cast<uint8_t*>(rows + 4);
  // active experts y, y + ny, ... (the grid is sized for the usual count; rare extra
  // candidates are taken by the same workgroups)
  const uint32_t ny = gridDim.y - (ra.n ? 1 : 0);
  for (uint32_t a = blockIdx.y; a < (SELF ? nc : A.ne); a += ny) {
  const uint8_t* wmat;
  uint32_t s0;
  bool primed = false;  // the stream already holds this slot's expert (the prediction held)
  if constexpr (SELF) {  // slot a streams the a-th candidate; its one pair is slot a, token 0's
    const uint32_t e = s_cl[a];
    primed = a == blockIdx.y && e == pred;
    wmat = reinterpret_cast<const uint8_t*>(__shfl(reinterpret_cast<uintptr_t>(ep), (int)e));
    s0 = a;
    if (blockIdx.x == 0 && wave == 0) {
      const uint8_t* w3[3];
      for (int p = 0; p < 3; p++) w3[p] = reinterpret_cast<const uint8_t*>(__shfl(reinterpret_cast<uintptr_t>(ep3[p]), (int)e));
      if (lane == 0) {
        ExpertWork& W = S.work[a];
        for (int p = 0; p < 3; p++) W.w[p] = w3[p];
        W.e = e;
        W.s0 = a;
        W.m = 1;
        S.slot_tok[a] = 0;
      }
    }
  } else {
    const ExpertWork* W = A.work + a;
    if (W->m != 1) break;  // m = 0: past the last active expert (one token a call: m <= 1)
    wmat = W->w[mat];
    s0 = W->s0;
  }
  if (!primed) {
    st = UnitStream<QT, 1>(wmat + toff, u0, u1, lane);
    st.prime();  // the weights' first loads overlap the staging of the activations
  }
  if (tid == 0) rows[0] = SELF ? 0u : A.slot_tok[s0];
  __syncthreads();
  if constexpr (SELF) stage_acts<QT, true>(acts, A.d, 1u, rows, A.d, 0, nullptr, nullptr, nullptr, ra.hs);
  else stage_acts<QT, true>(acts, A.d, 1u, rows, A.d, 0, A.xq, A.xs, A.xsum, nullptr);
  __syncthreads();
  st.run([&](uint32_t u, const uint32_t* w) {
    const uint32_t off = u * EU;
    const PkTerms a{reinterpret_cast<const int8_t*>(acts) + off, reinterpret_cast<const float*>(acts + Act::qb(A.d) + off / 8),
                    reinterpret_cast<const uint32_t*>(acts + Act::qb(A.d) + Act::sb(A.d) + (Act::SW ? off / Act::SW * 4 : 0u)),
                    terms + ((size_t)mat * nterm + u * NT) * 64 + lane};
    pk_unit<QT>(w, 1u, 1u, [&](uint32_t) { return a; });
  });
  __syncthreads();
  // waves 0 (gate) and 4 (up): the row dot, its terms added in K order
  if (part == 0) {
    const float* tv = terms + (size_t)mat * nterm * 64 + lane;
    float acc = 0.0f;
    for (uint32_t j0 = 0; j0 < nterm; j0 += 16) {  // 16 loads in flight, then their adds
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = tv[(j0 + i) * 64];
#pragma unroll
      for (int i = 0; i < 16; i++) acc = acc + v[i];
    }
    if (mat == 1) usum[lane] = acc;
    else terms[lane] = acc;  // g, over its own first term (read back below by this wave)
  }
  __syncthreads();
  if (wave == 0) {
    const bool valid = r0 + (lane & 32) + 32 <= A.f;  // this lane's 32-row block lies inside d_ff
    const float h = swiglu(terms[lane], usum[lane]);
    quant_wave(h, lane, valid, A.hq + (size_t)s0 * A.f + r0, A.hsc + (size_t)s0 * (A.f / 32) + r0 / 32,
               A.hkind ? A.hsum + (size_t)s0 * (A.f / sum_width(A.hkind)) : nullptr, r0, A.hkind, A.hoff);
  }
  __syncthreads();  // the LDS is the next expert's
  }
}

// Down: the row's units are split over gridDim.y workgroups of KS unit ranges each. A
// workgroup adds its ranges' partial sums in range order and writes them to its own
// partial slice y[blockIdx.y]; the combine adds the slices in order. TS > 1: each range
// is streamed by TS waves, each for its share of the chunk's tokens (the same sums, each
// by fewer dependent steps a wave).
// grid.x = row tiles of d_model, grid.y = K groups, grid.z = active-expert slot.
template <int QT, bool PACKED, int KS, int RD = 2, int TS = 1>
__global__ void __launch_bounds__(64 * KS * TS, 2)
k_dn_units(const ExpertWork* __restrict__ work, uint32_t ne, uint32_t f, uint32_t d, uint32_t mt, uint32_t part_stride,
           const int8_t* __restrict__ hq, const float* __restrict__ hsc, const uint32_t* __restrict__ hsum,
           const float* __restrict__ hf, float* __restrict__ ypart) {
  constexpr int U = UT_<QT>::U, EU = UT_<QT>::EU;
  extern __shared__ uint4 dsm[];
  float* accs = reinterpret_cast<float*>(dsm);  // [KS][mt][64]
  uint32_t* rows = reinterpret_cast<uint32_t*>(accs + KS * mt * 64);  // [mt] slot of each chunk member
  uint8_t* acts = reinterpret_cast<uint8_t*>(rows + ((mt + 3) & ~3u));
  for (uint32_t a = blockIdx.z; a < ne; a += gridDim.z) {  // active experts, as in k_gu_units
  const ExpertWork* W = work + a;  // field by field: scalar loads
  const uint32_t m_all = W->m;
  if (m_all == 0) break;
  const uint32_t s0 = W->s0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t rg = TS > 1 ? wave % KS : wave, tg = TS > 1 ? wave / KS : 0u;  // unit range, token share
  const uint32_t r0 = blockIdx.x * kTileRows;
  const uint32_t nblk = unit_blocks<QT>(f), nunit = unit_count<QT>(f);
  const uint32_t nsl = gridDim.y * KS, sl = blockIdx.y * KS + rg;
  const uint32_t u0 = (nunit * sl) / nsl, u1 = (nunit * (sl + 1)) / nsl;
  // the workgroup's unit range: its first wave's start to its last wave's end
  const uint32_t uw0 = (nunit * (blockIdx.y * KS)) / nsl, uw1 = (nunit * (blockIdx.y * KS + KS)) / nsl;
  const uint32_t nelem = min(uw1 * EU, f) - min(uw0 * EU, f);
  const uint32_t per = ActLds<QT, PACKED>::per_token(nelem);
  float* y = ypart + (size_t)blockIdx.y * part_stride;
  float* my = accs + rg * mt * 64 + lane;
  UnitStream<QT, RD> st(W->w[2] + (size_t)blockIdx.x * nunit * kTileRows * U, u0, u1, lane);
  for (uint32_t c0 = 0; c0 < m_all; c0 += mt) {
    const uint32_t m = min(mt, m_all - c0);
    const uint32_t t0 = (m * tg) / TS, t1 = (m * (tg + 1)) / TS;  // the wave's tokens of the chunk
    st.prime();  // the weights' first loads overlap the staging of the activations
    for (uint32_t t = threadIdx.x; t < m; t += blockDim.x) rows[t] = s0 + c0 + t;
    for (uint32_t t = t0; t < t1; t++) my[t * 64] = 0.0f;
    __syncthreads();
    if (nelem) stage_acts<QT, PACKED>(acts, nelem, m, rows, f, uw0 * EU, hq, hsc, hsum, hf);
    __syncthreads();
    st.run([&](uint32_t u, const uint32_t* w) {
      unit_tokens<QT, PACKED>(w, acts + t0 * per, per, nelem, u, uw0, nblk, my + t0 * 64, t1 - t0);
    });
    __syncthreads();
    if (wave == 0) {
      const uint32_t row = r0 + lane;
      for (uint32_t t = 0; t < m; t++) {
        float sacc = accs[t * 64 + lane];
#pragma unroll
        for (int w2 = 1; w2 < KS; w2++) sacc += accs[(w2 * mt + t) * 64 + lane];
        if (row < d) y[(size_t)(s0 + c0 + t) * d + row] = sacc;
      }
    }
    __syncthreads();
  }
  }
}

// The part of a chunk of a down tile with the combine folded in that follows its set-up
// (stream primed, rows[] holding the chunk's slots, the lane's running sums zeroed, a
// barrier): stages the chunk's h, streams the wave's units, adds the waves' row sums in
// wave order and adds y * w into the zeroed output with an atomic add. A token's output
// element then receives exactly k <= 2 terms; float addition is commutative, so 0 + p1 +
// p2 is the same in either arrival order and the result is the combine's
// (llama/mod.rs:974-997, moe/mod.rs:104-109) bit for bit, run to run. Weights: slot_w[slot],
// or with spec set the exact routing's (slot, weight) per (token, position), a candidate
// slot no routed pair names adding nothing and a routed pair the candidates missed giving
// NaN, as the combine does.
struct DnAtomicArgs {
  uint32_t f, d, k, spec;
  const uint32_t* slot_tok;
  const uint32_t* slot_of;
  const float* slot_w;
  const int8_t* hq;
  const float* hsc;
  const uint32_t* hsum;
  const float* hf;
  float* out;
};

// PAIR: the workgroup's 32 rows, lanes l and l + 32 row r0 + l's sums over the even and
// the odd units.
template <int QT, bool PACKED, int KS, bool PAIR = false, class Stream>
__device__ __forceinline__ void dn_atomic_chunk(Stream& st, const DnAtomicArgs& A, const float* accs, float* my,
                                                const uint32_t* rows, uint8_t* acts, uint32_t mt, uint32_t m,
                                                uint32_t slot0, uint32_t r0) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t nblk = unit_blocks<QT>(A.f), per = ActLds<QT, PACKED>::per_token(A.f);
  stage_acts<QT, PACKED>(acts, A.f, m, rows, A.f, 0, A.hq, A.hsc, A.hsum, A.hf);
  __syncthreads();
  // wave 0, lane t < m: chunk member t's token and combine weight, loaded here so that
  // their latency hides behind the stream (m <= kFuseMaxTokens <= 64, k <= 2). fl: 1 the
  // slot is a routed pair's, 2 a routed pair of the token has no candidate slot (NaN).
  uint32_t rtok = 0, rfl = 0;
  float rwt = 0.0f;
  if (wave == 0 && lane < m) {
    const uint32_t slot = slot0 + lane;
    rtok = A.slot_tok[slot];
    if (A.spec) {
      uint32_t sl[2];
      float wv[2];
#pragma unroll
      for (uint32_t i = 0; i < 2; i++)
        if (i < A.k) {
          sl[i] = A.slot_of[(size_t)rtok * A.k + i];
          wv[i] = A.slot_w[(size_t)rtok * A.k + i];
        }
#pragma unroll
      for (uint32_t i = 0; i < 2; i++)
        if (i < A.k) {
          if (sl[i] == slot) {
            rfl |= 1u;
            rwt = wv[i];
          }
          if (sl[i] == ~0u) rfl |= 2u;
        }
    } else {
      rfl = 1u;
      rwt = A.slot_w[slot];
    }
  }
  st.run([&](uint32_t u, const uint32_t* w) { unit_tokens<QT, PACKED, 1>(w, acts, per, A.f, u, 0, nblk, my, m); });
  __syncthreads();
  if (wave == 0) {
    const uint32_t l = PAIR ? (lane & 31u) : lane, row = r0 + l;
    for (uint32_t t = 0; t < m; t++) {
      float y;
      if constexpr (PAIR) {  // waves in order, each its even units' sum then its odd units'
        y = accs[t * 64 + l] + accs[t * 64 + l + 32];
#pragma unroll
        for (int w2 = 1; w2 < KS; w2++) y += accs[(w2 * mt + t) * 64 + l] + accs[(w2 * mt + t) * 64 + l + 32];
      } else {
        y = accs[t * 64 + lane];
#pragma unroll
        for (int w2 = 1; w2 < KS; w2++) y += accs[(w2 * mt + t) * 64 + lane];
      }
      const uint32_t tok = lane_u(rtok, t), fl = lane_u(rfl, t);
      const float wt = __uint_as_float(lane_u(__float_as_uint(rwt), t));
      if (row < A.d && (!PAIR || lane < 32)) {
        if (fl & 1u) atomicAdd(A.out + (size_t)tok * A.d + row, y * wt);
        if (fl & 2u) atomicAdd(A.out + (size_t)tok * A.d + row, __int_as_float(0x7fc00000));
      }
    }
  }
  __syncthreads();
}

// Down with the combine folded in, for layers of top-k <= 2: a workgroup of KS waves takes
// one 64-row tile of one expert over the whole K range (wave w its w-th share of the
// units) and runs dn_atomic_chunk over its tokens.
// grid.x = row tiles of d, grid.z = active-expert slot.
// PAIR (grids of at most half as many workgroups as the chip has CUs, such as one token's
// two experts): a workgroup takes half a tile, 32 rows, and each wave's two half-waves
// stream alternate units of its share (lane l: row l % 32, units of parity l / 32), so
// every load is still a whole 1 KiB (two 512-byte runs) and twice as many CUs issue them.
// grid.x = 2 x row tiles.
template <int QT, bool PACKED, int KS, int RD = 2, bool PAIR = false>
__global__ void __launch_bounds__(64 * KS, 2)
k_dn_atomic(const ExpertWork* __restrict__ work, uint32_t ne, uint32_t mt, DnAtomicArgs A) {
  constexpr int U = UT_<QT>::U;
  extern __shared__ uint4 dsm[];
  float* accs = reinterpret_cast<float*>(dsm);  // [KS][mt][64]
  uint32_t* rows = reinterpret_cast<uint32_t*>(accs + KS * mt * 64);  // [mt] slot of each chunk member
  uint8_t* acts = reinterpret_cast<uint8_t*>(rows + ((mt + 3) & ~3u));
  for (uint32_t a = blockIdx.z; a < ne; a += gridDim.z) {
    const ExpertWork* W = work + a;
    const uint32_t m_all = W->m;
    if (m_all == 0) break;
    const uint32_t s0 = W->s0;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t nunit = unit_count<QT>(A.f);
    float* my = accs + wave * mt * 64 + lane;
    auto chunks = [&](auto& st, uint32_t r0) {
      for (uint32_t c0 = 0; c0 < m_all; c0 += mt) {
        const uint32_t m = min(mt, m_all - c0);
        st.prime();
        for (uint32_t t = threadIdx.x; t < m; t += blockDim.x) rows[t] = s0 + c0 + t;
        for (uint32_t t = 0; t < m; t++) my[t * 64] = 0.0f;
        __syncthreads();
        dn_atomic_chunk<QT, PACKED, KS, PAIR>(st, A, accs, my, rows, acts, mt, m, s0 + c0, r0);
      }
    };
    if constexpr (PAIR) {
      const uint32_t tx = blockIdx.x >> 1, hx = blockIdx.x & 1u, ph = lane >> 5, np = (nunit + 1) / 2;
      const uint32_t p0 = (np * wave) / KS, p1 = (np * (wave + 1)) / KS;
      const uint32_t u0 = 2 * p0 + ph;
      uint32_t u1 = 2 * p1 + ph;
      if (u1 > u0 && u1 - 2 >= nunit) u1 -= 2;  // an odd unit count: the last pair's odd half
      UnitStream<QT, RD, 2> st(W->w[2] + (size_t)tx * nunit * kTileRows * U + 512 * hx + 16 * (lane & 31u), u0, u1);
      chunks(st, tx * kTileRows + 32 * hx);
    } else {
      const uint32_t u0 = (nunit * wave) / KS, u1 = (nunit * (wave + 1)) / KS;
      UnitStream<QT, RD> st(W->w[2] + (size_t)blockIdx.x * nunit * kTileRows * U, u0, u1, lane);
      chunks(st, blockIdx.x * kTileRows);
    }
  }
}

// Token embeddings from a tiled dense weight (the token table kept packed): x[i] = row
// tok[i] dequantised, Weight::row (llama/mod.rs:198-212) -> quant::dequantize, with the
// same per-block arithmetic as every dequantiser here (bit for bit). Row t is lane t % 64
// of tile t / 64; a thread takes one 32-value group of one unit (its unit's pieces are
// read by every group of the unit, from L1 after the first). The tokens come from the
// kernel arguments, or from device memory (dtok) in steps replayed from a graph.
template <int QT>
__global__ void __launch_bounds__(256) k_embed_tiled(const uint8_t* __restrict__ tiled, uint32_t cols, GlueTokens tk,
                                                     const uint32_t* __restrict__ dtok, float* __restrict__ x) {
  constexpr int U = UT_<QT>::U, NP = U / 16, NW = U / 4, EU = UT_<QT>::EU, G = UT_<QT>::G;
  constexpr int NG = EU / 32, GPB = QT_<QT>::E / 32;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const uint32_t i = blockIdx.x;
  const uint32_t t = dtok ? dtok[i] : tk.tok[i];
  const uint32_t nunit = unit_count<QT>(cols), nblk = unit_blocks<QT>(cols);
  const uint8_t* row = tiled + (size_t)(t / kTileRows) * nunit * kTileRows * U + (t % kTileRows) * 16;
  float* dst = x + (size_t)i * cols;
  for (uint32_t j = threadIdx.x; j < nunit * NG; j += blockDim.x) {
    const uint32_t u = j / NG, q = j % NG;
    const uint32_t nvalid = G == 1 ? 1u : min((uint32_t)G, nblk - u * G);
    if (G > 1 && q / GPB >= nvalid) continue;  // past the row's last block
    uint32_t w[NW];
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(row + (size_t)u * NP * 1024 + p * 1024);
      w[4 * p] = v.x; w[4 * p + 1] = v.y; w[4 * p + 2] = v.z; w[4 * p + 3] = v.w;
    }
    float v[32];
    unit_deq32<QT>(w, (int)q, v);
    float4* o = reinterpret_cast<float4*>(dst + (size_t)u * EU + 32 * q);
#pragma unroll
    for (int c = 0; c < 8; c++) o[c] = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
  }
}

template <int QT>
hipError_t units_embed(const uint8_t* tiled, uint32_t cols, const GlueTokens* tk, const uint32_t* dtok, uint32_t n,
                       float* x, hipStream_t st) {
  GlueTokens a{};
  if (tk) a = *tk;
  hipLaunchKernelGGL(k_embed_tiled<QT>, dim3(n), dim3(256), 0, st, tiled, cols, a, dtok, x);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------------

constexpr uint32_t kLdsBudget = 160 * 1024 - 2048;
// Single-token calls stream gate/up with a ring of 4 unit sets: at one token the grid
// has fewer waves than SIMDs, so the registers cost no occupancy, and on the C2 layer the
// launch took 33.7 us instead of 35.4 (a ring of 2) or 37.3 (a ring of 1). Calls of at
// most one token an expert on average (n * k <= experts) take a ring of one set: 159
// VGPRs instead of 209, three waves a SIMD, so that the grid (with those few tokens an
// expert, chunks of LDS for six workgroups a CU) is resident in one round: C2 at batch 4
// 88.6 -> 82.5 us. With more tokens an expert the ring of two stays (batch 8: 106.8 us
// against 111.7-125 with a ring of one and chunks of 3-5 tokens).
constexpr uint32_t kDeepRingTokens = 1;
// Q3_K gate/up with more than one token an expert on average runs workgroups of two row
// tiles with a ring of one unit set: 164 VGPRs, three waves a SIMD, and the two tiles'
// four waves share one staging of the tokens, so three workgroups a CU still hold 8
// tokens (kChunkLds3). The C5 slice (Q3_K gate/up, batch 8) went from 172.4 to 164.7 us a
// call; the same for Q4_K (C2 batch 8: 168.0 -> 172.9 us a step) and Q6_K (C4: 189.3 ->
// 194.5 us) measured slower, so they keep one tile and two unit sets.
template <int QT>
constexpr bool gu_pairs() { return QT == Q3_K; }
// Unit sets in the gate/up ring from two tokens an expert on (one tile a workgroup): Q6_K's
// 224-byte units make a set of 56 registers a lane, and with one set (171 VGPRs against
// 247, two waves a SIMD either way) C4 (Q6_K gate/up, 4 tokens an expert) went from 189.7
// to 185.0 us a call on one box; Q4_K keeps two (C2 batch 8: 170.1 -> 172.4 us with one).
// Capped at three waves a SIMD (167 VGPRs, 2 spilled) Q6_K's took C4 to 191.2 us.
template <int QT>
constexpr int gu_ring() { return QT == Q6_K ? 1 : 2; }

template <class K>
static bool allow_lds(K kernel) {
  // raise the dynamic LDS limit of one instantiation (called once per instantiation)
  return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBudget) ==
         hipSuccess;
}

// Tokens per chunk: enough for the tokens an expert usually gets (twice the mean n*k/ne,
// at least 8), as far as their staged activations and running sums fit kChunkLds; an
// expert with more tokens takes several chunks, re-streaming its weights once per chunk.
// kChunkLds leaves four workgroups per CU, the most the expert kernels' registers (about
// 180-240 VGPRs: two waves per SIMD) allow anyway: on the C2 layer at batch 8, 8 tokens
// of 5.6 KB held the gate/up kernel to three (118 us), 7 tokens let it run four (112 us).
// Sizing for the whole batch instead would give every workgroup the LDS of n tokens and
// one workgroup per CU when experts are many and tokens per expert few.
constexpr uint32_t kChunkLds = 40 * 1024 - 64;
// gate/up workgroups of two row tiles: three a CU (twelve waves, three a SIMD)
constexpr uint32_t kChunkLds3 = 160 * 1024 / 3 - 512;
static uint32_t chunk_tokens_lds(const LayerDev& L, uint32_t n, uint32_t per_token_bytes, uint32_t budget) {
  const uint32_t usual = max(8u, 2 * ((n * L.k + L.ne - 1) / L.ne));
  const uint32_t fit = budget / per_token_bytes;  // 0 when one token needs more (then one, if it fits at all)
  return min(min(n, usual), fit ? fit : kLdsBudget / per_token_bytes);
}
static uint32_t chunk_tokens(const LayerDev& L, uint32_t n, uint32_t per_token_bytes) {
  return chunk_tokens_lds(L, n, per_token_bytes, kChunkLds);
}

// The split gate/up (k_gu_split) serves packed math at one token a call for the K-quant
// types, whose units are one block, when its LDS (every term of a row tile of both
// matrices) fits.
template <int QT>
static uint32_t split_lds(const LayerDev& L, const RouteArgs& ra, uint32_t* rsec) {
  const uint32_t nterm = unit_count<QT>(L.d) * unit_terms<QT>();
  size_t lds = (size_t)2 * nterm * 64 * 4 + 64 * 4 + 16 + ActLds<QT, true>::per_token(L.d);
  *rsec = 0;
  if (ra.n) {  // route_token's sections: the longest multiple of 64 values whose halves take <= 64 KB
    *rsec = min(L.d, ((64u * 1024u / (8u * L.ne)) - 4u) & ~63u);
    lds = max(lds, (size_t)route_token_lds(L.ne, L.k, *rsec) * 4);
  }
  return lds <= kLdsBudget ? (uint32_t)lds : 0u;
}

template <int QT>
static bool split_ok(const LayerDev& L, uint32_t n, const RouteArgs& ra) {
  if constexpr (UT_<QT>::G != 1 || !has_int8_kernel(QT)) {
    return false;
  } else {
    uint32_t rsec;
    const uint32_t nterm = unit_count<QT>(L.d) * unit_terms<QT>();
    return L.math == 0 && n == 1 && nterm % 16 == 0 && unit_count<QT>(L.d) >= kSplitParts &&
           (!ra.n || (ra.n == n && L.ne <= 64 && L.d % 64 == 0)) && split_lds<QT>(L, ra, &rsec) != 0;
  }
}

template <int QT>
static hipError_t go_gu_split(const LayerDev& L, const FwdBufs& B, uint32_t n, const RouteArgs& ra, hipStream_t st) {
  uint32_t rsec = 0;
  const uint32_t lds = split_lds<QT>(L, ra, &rsec);
  if (lds == 0 || n != 1 || (ra.self && (!ra.n || L.ne > kSpecMaxExperts))) return hipErrorInvalidValue;
  static const bool once = allow_lds(k_gu_split<QT, false>) && allow_lds(k_gu_split<QT, true>);
  (void)once;
  const uint32_t tiles = (L.f + kTileRows - 1) / kTileRows;
  const dim3 g(max(tiles, ra.n), min(L.ne, n * L.k) + (ra.n ? 1 : 0));
  const SplitArgs A{B.work, B.slot_tok, B.xq, B.xs, B.xsum, B.hq, B.hsc, B.hsum, L.ne, L.d, L.f, rsec,
                    sum_kind_of(L.qt_down), sum_offset_of(L.qt_down)};
  const SelfArgs S{L.eptr, B.work, B.slot_tok, B.active, B.offsets, B.fuse_out ? B.out : nullptr};
  if (ra.self) hipLaunchKernelGGL((k_gu_split<QT, true>), g, dim3(64 * kSplitWaves), lds, st, A, ra, S);
  else hipLaunchKernelGGL((k_gu_split<QT, false>), g, dim3(64 * kSplitWaves), lds, st, A, ra, S);
  return hipGetLastError();
}

template <int QT, bool PACKED, int D, int TPW = 1, int PIPE = 0>
static hipError_t go_gu(const LayerDev& L, const FwdBufs& B, uint32_t n, const RouteArgs& ra, hipStream_t st) {
  const uint32_t per = 2 * TPW * 64 * 4 + ActLds<QT, PACKED>::per_token(L.d) + 4;
  const uint32_t mt = TPW > 1 ? chunk_tokens_lds(L, n, per + 16, kChunkLds3) : chunk_tokens(L, n, per + 16);
  if (mt == 0) return hipErrorInvalidValue;
  static const bool once = allow_lds(k_gu_units<QT, PACKED, D, TPW, PIPE>);
  (void)once;
  const uint32_t tiles = (L.f + kTileRows * TPW - 1) / (kTileRows * TPW);
  uint32_t lds = mt * per + 16;
  if (ra.n) lds = max(lds, route_logit_lds(ra.k, ra.sec));
  const dim3 g(max(tiles, ra.n * ra.ne), min(L.ne, n * L.k) + (ra.n ? 1 : 0));
  hipLaunchKernelGGL((k_gu_units<QT, PACKED, D, TPW, PIPE>), g, dim3(128 * TPW), lds, st, B.work, L.ne, B.slot_tok, L.f,
                     L.d, mt, B.xq, B.xs, B.xsum, B.hs, B.hq, B.hsc, B.hsum, B.hf, sum_kind_of(L.qt_down),
                     sum_offset_of(L.qt_down), ra);
  return hipGetLastError();
}

template <int QT, bool PACKED, int RD, int TS = 1>
static hipError_t go_dn_rd(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st);

// Dense projections (one "expert" of weight 1) of a few hundred row tiles at most, from 4
// tokens on, stream each unit range with two waves, each for half the tokens: there the
// launch is a short chain per workgroup (one or two units a wave), and the tokens' dots
// run one after another in a wave. The 32000-row output head (500 row tiles, more
// workgroups than the chip holds) measured slower that way (55 -> 80 us), so it keeps one.
static bool dn_token_split(const LayerDev& L, uint32_t n) {
  return L.ne == 1 && n >= 4 && (L.d + kTileRows - 1) / kTileRows <= 128;
}

// The K-sliced down product (and the dense projections it runs) streams through a ring of
// one unit set, as the fused down does: C4 (Q8_0 down) 201 -> 189.6 us a call, the
// attention projections at batch 8 64.3 -> 60.7 us, the 32000-row output head 55.0 ->
// 52.9 us, against a ring of two on the same box.
template <int QT, bool PACKED>
static hipError_t go_dn(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st) {
  if constexpr (PACKED) {
    if (dn_token_split(L, n)) return go_dn_rd<QT, PACKED, 1, 2>(L, B, n, ksg, st);
  }
  return go_dn_rd<QT, PACKED, 1>(L, B, n, ksg, st);
}

template <int QT, bool PACKED, int RD, int TS>
static hipError_t go_dn_rd(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st) {
  // a workgroup stages at most ceil(units / ksg) + 1 units
  const uint32_t span = min(((unit_count<QT>(L.f) + ksg - 1) / ksg + 1) * UT_<QT>::EU, L.f);
  const uint32_t per = kDnKS * 64 * 4 + ActLds<QT, PACKED>::per_token(span) + 4;
  const uint32_t mt = chunk_tokens(L, n, per + 16);
  if (mt == 0) return hipErrorInvalidValue;
  static const bool once = allow_lds(k_dn_units<QT, PACKED, kDnKS, RD, TS>);
  (void)once;
  const dim3 g((L.d + kTileRows - 1) / kTileRows, ksg, min(L.ne, n * L.k));
  hipLaunchKernelGGL((k_dn_units<QT, PACKED, kDnKS, RD, TS>), g, dim3(64 * kDnKS * TS), mt * per + 16, st, B.work, L.ne, L.f, L.d, mt,
                     B.nslot * L.d, B.hq, B.hsc, B.hsum, B.hf, B.y);
  return hipGetLastError();
}

constexpr int kDnAtomicKS = 8;
// Grids of the fused down product up to this many workgroups (half of MI355X's 256 CUs)
// run in half tiles (k_dn_atomic's PAIR form), twice as many.
constexpr uint32_t kDnPairGrid = 128;

static_assert(kFuseMaxTokens <= 64, "k_dn_atomic keeps a chunk's tokens one a lane");

// The down product with the combine folded in streams its units through a ring of one set
// (RD = 1): the loads of a unit are issued right after the previous unit's body. Measured
// on the C2 layer against a ring of two: 22.6 -> 22.2 us at batch 1, 33.0 -> 31.8 at 2,
// 48.4 -> 46.4 at 4, 57.6 -> 56.1 at 8, the C5 slice 175.1 -> 172.6 us. Its workgroups
// carry 8 waves and the long K range of d_ff, so every SIMD holds several streams at once
// and a deeper ring only lengthens the wait for each wave's next unit.
template <int QT, bool PACKED, int RD>
static hipError_t go_dn_atomic_rd(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  if (L.k > 2 || n > kFuseMaxTokens) return hipErrorInvalidValue;
  const uint32_t per = kDnAtomicKS * 64 * 4 + ActLds<QT, PACKED>::per_token(L.f) + 4;
  const uint32_t mt = min(n, (kLdsBudget - 16) / per);
  if (mt == 0) return hipErrorInvalidValue;
  static const bool once = allow_lds(k_dn_atomic<QT, PACKED, kDnAtomicKS, RD>) &&
                           allow_lds(k_dn_atomic<QT, PACKED, kDnAtomicKS, RD, true>);
  (void)once;
  const uint32_t tiles = (L.d + kTileRows - 1) / kTileRows, slots = min(L.ne, n * L.k);
  const DnAtomicArgs A{L.f, L.d, L.k, B.spec, B.slot_tok, B.slot_of, B.slot_w, B.hq, B.hsc, B.hsum, B.hf, B.out};
  if (tiles * slots <= kDnPairGrid)
    hipLaunchKernelGGL((k_dn_atomic<QT, PACKED, kDnAtomicKS, RD, true>), dim3(2 * tiles, 1, slots),
                       dim3(64 * kDnAtomicKS), mt * per + 16, st, B.work, L.ne, mt, A);
  else
    hipLaunchKernelGGL((k_dn_atomic<QT, PACKED, kDnAtomicKS, RD>), dim3(tiles, 1, slots), dim3(64 * kDnAtomicKS),
                       mt * per + 16, st, B.work, L.ne, mt, A);
  return hipGetLastError();
}

template <int QT, bool PACKED>
static hipError_t go_dn_atomic(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  return go_dn_atomic_rd<QT, PACKED, 1>(L, B, n, st);
}

template <int QT>
hipError_t units_down_atomic(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  if constexpr (has_int8_kernel(QT)) {
    if (L.math == 0) return go_dn_atomic<QT, true>(L, B, n, st);
  }
  return go_dn_atomic<QT, false>(L, B, n, st);
}

template <int QT>
hipError_t units_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, const RouteArgs& ra, hipStream_t st) {
  if constexpr (has_int8_kernel(QT)) {
    if (L.math == 0) {
      if (B.hq && split_ok<QT>(L, n, ra)) return go_gu_split<QT>(L, B, n, ra, st);
      if (ra.self) return hipErrorInvalidValue;  // (the caller asked only where units_self_ok)
      if (n <= kDeepRingTokens) return go_gu<QT, true, 4>(L, B, n, ra, st);
      // Q4_K at half a token an expert or fewer: the dots read the codes a group ahead
      // (182 VGPRs, two waves a SIMD, which still hold such a grid in one round); up to
      // one token an expert, half a group ahead (167 VGPRs, three waves a SIMD)
      if constexpr (QT == Q4_K) {
        if (2 * n * L.k <= L.ne) return go_gu<QT, true, 1, 1, 1>(L, B, n, ra, st);
        if (n * L.k <= L.ne) return go_gu<QT, true, 1, 1, 2>(L, B, n, ra, st);
      }
      if (n * L.k <= L.ne) return go_gu<QT, true, 1>(L, B, n, ra, st);
      if constexpr (gu_pairs<QT>()) return go_gu<QT, true, 1, 2>(L, B, n, ra, st);
      return go_gu<QT, true, gu_ring<QT>()>(L, B, n, ra, st);
    }
  }
  return go_gu<QT, false, 2>(L, B, n, ra, st);
}

template <int QT>
bool units_self_ok(const LayerDev& L, uint32_t n) {
  RouteArgs ra{};
  ra.n = n;
  return L.qt_gate == QT && L.qt_up == QT && L.ne <= kSpecMaxExperts && split_ok<QT>(L, n, ra);
}

template <int QT>
hipError_t units_down(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st) {
  if constexpr (has_int8_kernel(QT)) {
    if (L.math == 0) return go_dn<QT, true>(L, B, n, ksg, st);
  }
  return go_dn<QT, false>(L, B, n, ksg, st);
}

template hipError_t units_gateup<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, const RouteArgs&, hipStream_t);
template hipError_t units_down<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, uint32_t, hipStream_t);
template bool units_self_ok<GMOE_QT>(const LayerDev&, uint32_t);
template hipError_t units_down_atomic<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, hipStream_t);
template hipError_t units_embed<GMOE_QT>(const uint8_t*, uint32_t, const GlueTokens*, const uint32_t*, uint32_t, float*,
                                         hipStream_t);

}  // namespace gmoe
