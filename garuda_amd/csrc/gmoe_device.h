// gmoe_device.h — device-side helpers shared by the gfx950 kernels: half decoding,
// the bit-exact expf, block traits, the dequantisers, the activation quantiser and
// the packed (int8-activation) block dots.
#pragma once

#include "gmoe_internal.h"

#include <math.h>

namespace gmoe {

// ---------------------------------------------------------------------------------
// Scalar helpers
// ---------------------------------------------------------------------------------

// quant/mod.rs:878-890. The hardware conversion is exact for every finite half and
// for infinities; NaN is canonicalised the way the reference builds it (f32::NAN,
// sign applied by negation).
__device__ __forceinline__ float f16f(uint32_t h) {
  h &= 0xffffu;
  if ((h & 0x7c00u) == 0x7c00u && (h & 0x3ffu)) return __uint_as_float((h & 0x8000u) ? 0xffc00000u : 0x7fc00000u);
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

// expf, reproducing the host libm the reference links (glibc >= 2.28 on x86-64 with
// FMA). Method: exp2f-table reduction of Szabolcs Nagy (ARM optimized-routines,
// 2017): x*N/ln2 = k + r, 2^(k/N) from a 32-entry table, 2^(r/N) by a cubic, all in
// double; the scaled product is fused into both of its uses as the FMA build does.
// Checked bit-for-bit against the host expf over every float in the finite range.
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

__device__ __forceinline__ float gm_expf(float x) {
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  const double kShift = 0x1.8p+52;
  const double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
  uint32_t ux = __float_as_uint(x);
  uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {                    // |x| >= 88 or NaN
    if (ux == 0xff800000u) return 0.0f;      // -inf
    if (abstop >= 0x7f8u) return x + x;      // inf or NaN
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;                         // underflow
  }
  double xd = (double)x;
  double kd = fma(kInvLn2N, xd, kShift);
  uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd -= kShift;
  double r = fma(kInvLn2N, xd, -kd);
  uint64_t t = kExp2Tab[ki % 32] + (ki << 47);
  double s = __longlong_as_double((long long)t);
  double z = fma(kC0, r, kC1);
  double r2 = r * r;
  double y = fma(kC2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

__device__ __forceinline__ float fdiv(float a, float b) { return __fdiv_rn(a, b); }

// simd::silu then simd::mul_assign (simd/mod.rs:161-163, :188-191).
__device__ __forceinline__ float swiglu(float g, float u) {
  float s = fdiv(g, 1.0f + gm_expf(-g));
  return s * u;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, int i) {
  return (w[i >> 2] >> ((i & 3) * 8)) & 0xffu;
}

// quant/mod.rs:656-664, on the 12 scale bytes held in w[0..2] (little endian).
__device__ __forceinline__ void scale_min_k4(const uint32_t* s3, int j, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = byte_of(s3, j) & 63u;
    m = byte_of(s3, j + 4) & 63u;
  } else {
    sc = (byte_of(s3, j + 4) & 0x0fu) | ((byte_of(s3, j - 4) >> 6) << 4);
    m = (byte_of(s3, j + 4) >> 4) | ((byte_of(s3, j) >> 6) << 4);
  }
}

// quant/mod.rs:812-833
__device__ __forceinline__ void q3k_scales(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t out[4]) {
  const uint32_t K1 = 0x03030303u, K2 = 0x0f0f0f0fu;
  out[0] = (a0 & K2) | ((a2 & K1) << 4);
  out[1] = (a1 & K2) | (((a2 >> 2) & K1) << 4);
  out[2] = ((a0 >> 4) & K2) | (((a2 >> 4) & K1) << 4);
  out[3] = ((a1 >> 4) & K2) | (((a2 >> 6) & K1) << 4);
}

// ---------------------------------------------------------------------------------
// Block traits, and loads of raw packed blocks as the dequantiser entry receives them:
// a block is 16-, 4- or 2-byte aligned depending on its size.
// ---------------------------------------------------------------------------------

template <int QT> struct QT_;
template <> struct QT_<Q4_K> { static constexpr int E = 256, B = 144, A = 16; };
template <> struct QT_<Q5_K> { static constexpr int E = 256, B = 176, A = 16; };
template <> struct QT_<Q6_K> { static constexpr int E = 256, B = 210, A = 2; };
template <> struct QT_<Q3_K> { static constexpr int E = 256, B = 110, A = 2; };
template <> struct QT_<Q2_K> { static constexpr int E = 256, B = 84, A = 4; };
template <> struct QT_<Q8_0> { static constexpr int E = 32, B = 34, A = 2; };
template <> struct QT_<Q4_0> { static constexpr int E = 32, B = 18, A = 2; };
// F32/F16 rows are handled 32 elements at a time.
template <> struct QT_<F16> { static constexpr int E = 32, B = 64, A = 16; };
template <> struct QT_<F32> { static constexpr int E = 32, B = 128, A = 16; };

template <int QT> constexpr int ndw() { return (QT_<QT>::B + 3) / 4; }

// Load block bytes p[0..B) into w[] (byte i of the block = byte i%4 of w[i/4]).
// 2-byte aligned blocks read one dword past the block; the slab pads every matrix.
template <int QT>
__device__ __forceinline__ void load_block(const uint8_t* __restrict__ p, uint32_t* w) {
  constexpr int B = QT_<QT>::B, A = QT_<QT>::A, N = ndw<QT>();
  if constexpr (A == 16) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < B / 16; i++) {
      u32x4 v = q[i];
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (A == 4) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = q[i];
  } else {
    uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
    uint32_t sh = (uint32_t)(a & 3);
    uint32_t prev = q[0];
#pragma unroll
    for (int i = 0; i < N; i++) {
      uint32_t nxt = q[i + 1];
      w[i] = __builtin_amdgcn_alignbyte(nxt, prev, sh);
      prev = nxt;
    }
  }
}

// ---------------------------------------------------------------------------------
// Dequantisation (bit-exact, quant/mod.rs:624-875). deq32<QT>(w, g, out) writes the
// 32 values of group g (elements 32g..32g+31 of the block, in the reference's element
// order) with the reference's arithmetic; deq<QT> is every group of a block.
// ---------------------------------------------------------------------------------

template <int QT> __device__ __forceinline__ void deq32(const uint32_t* w, int g, float* out);

template <> __device__ __forceinline__ void deq32<Q4_K>(const uint32_t* w, int g, float* out) {
  float d = f16f(w[0]), dmin = f16f(w[0] >> 16);
  uint32_t sc, m;
  scale_min_k4(w + 1, g, sc, m);
  float dl = d * (float)sc, ml = dmin * (float)m;
  const uint32_t* chunk = w + 4 + 8 * (g / 2);
#pragma unroll
  for (int l = 0; l < 32; l++) {
    uint32_t b = byte_of(chunk, l);
    out[l] = dl * (float)((g & 1) ? (b >> 4) : (b & 15u)) - ml;
  }
}

template <> __device__ __forceinline__ void deq32<Q5_K>(const uint32_t* w, int g, float* out) {
  float d = f16f(w[0]), dmin = f16f(w[0] >> 16);
  uint32_t sc, m;
  scale_min_k4(w + 1, g, sc, m);
  float dl = d * (float)sc, ml = dmin * (float)m;
  const uint32_t* qh = w + 4;
  const uint32_t* ql = w + 12 + 8 * (g / 2);
#pragma unroll
  for (int l = 0; l < 32; l++) {
    uint32_t b = byte_of(ql, l), hb = (byte_of(qh, l) >> g) & 1u;
    out[l] = dl * (float)(((g & 1) ? (b >> 4) : (b & 15u)) + 16u * hb) - ml;
  }
}

template <> __device__ __forceinline__ void deq32<Q6_K>(const uint32_t* w, int g, float* out) {
  float d = f16f(w[52]);  // bytes 208..209 are the low half of dword 52
  const int half = g / 4, quarter = g % 4;
#pragma unroll
  for (int l = 0; l < 32; l++) {
    uint32_t ql = byte_of(w, 64 * half + l + 32 * (quarter & 1));
    uint32_t qh = byte_of(w, 128 + 32 * half + l);
    int q = (int)(((quarter < 2) ? (ql & 15u) : (ql >> 4)) | (((qh >> (2 * quarter)) & 3u) << 4)) - 32;
    float s = (float)(int8_t)byte_of(w, 192 + 8 * half + l / 16 + 2 * quarter);
    out[l] = d * s * (float)q;
  }
}

template <> __device__ __forceinline__ void deq32<Q3_K>(const uint32_t* w, int g, float* out) {
  float d_all = f16f(w[27]);  // bytes 108..109
  uint32_t sc4[4];
  q3k_scales(w[24], w[25], w[26], sc4);  // scale bytes 96..107
  const int half = g / 4, j = g % 4;
  const uint32_t m = 1u << (4 * half + j);
#pragma unroll
  for (int l = 0; l < 32; l++) {
    int is = 8 * half + 2 * j + l / 16;
    float dl = d_all * (float)((int)(int8_t)byte_of(sc4, is) - 32);
    int hbit = (byte_of(w, l) & m) ? 0 : 4;
    int q = (int)((byte_of(w, 32 + 32 * half + l) >> (2 * j)) & 3u) - hbit;
    out[l] = dl * (float)q;
  }
}

template <> __device__ __forceinline__ void deq32<Q2_K>(const uint32_t* w, int g, float* out) {
  float d = f16f(w[20]), dmin = f16f(w[20] >> 16);  // bytes 80..83
  const int half = g / 4, j = g % 4;
#pragma unroll
  for (int l = 0; l < 32; l++) {
    uint32_t sc = byte_of(w, 8 * half + 2 * j + l / 16);
    float dl = d * (float)(sc & 15u), ml = dmin * (float)(sc >> 4);
    uint32_t q = (byte_of(w, 16 + 32 * half + l) >> (2 * j)) & 3u;
    out[l] = dl * (float)q - ml;
  }
}

template <> __device__ __forceinline__ void deq32<Q8_0>(const uint32_t* w, int, float* out) {
  float s = f16f(w[0]);
#pragma unroll
  for (int i = 0; i < 32; i++) out[i] = s * (float)(int8_t)byte_of(w, 2 + i);
}

template <> __device__ __forceinline__ void deq32<Q4_0>(const uint32_t* w, int, float* out) {
  float s = f16f(w[0]);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    uint32_t b = byte_of(w, 2 + i);
    out[i] = s * (float)((int)(b & 15u) - 8);
    out[i + 16] = s * (float)((int)(b >> 4) - 8);
  }
}

template <> __device__ __forceinline__ void deq32<F16>(const uint32_t* w, int, float* out) {
#pragma unroll
  for (int i = 0; i < 16; i++) {
    out[2 * i] = f16f(w[i]);
    out[2 * i + 1] = f16f(w[i] >> 16);
  }
}

template <> __device__ __forceinline__ void deq32<F32>(const uint32_t* w, int, float* out) {
#pragma unroll
  for (int i = 0; i < 32; i++) out[i] = __uint_as_float(w[i]);
}

template <int QT> __device__ __forceinline__ void deq(const uint32_t* w, float* out) {
#pragma unroll
  for (int g = 0; g < QT_<QT>::E / 32; g++) deq32<QT>(w, g, out + 32 * g);
}

// ---------------------------------------------------------------------------------
// Activation quantiser (quant/mod.rs:331-345, :322-326): one thread per 32-block.
// ---------------------------------------------------------------------------------

// The block's values packed four to a word, its scale, and the sums of its halves.
__device__ __forceinline__ void quant32_regs(const float* v, uint32_t* packed, float* scale_out, int* sum0_out,
                                             int* sum1_out) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
  float scale = fdiv(amax, 127.0f);
  float inv = scale > 0.0f ? fdiv(1.0f, scale) : 0.0f;
  int sum0 = 0, sum1 = 0;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    float r = roundf(v[j] * inv);
    int qi;
    if (r != r) qi = 0;
    else if (r < -127.0f) qi = -127;
    else if (r > 127.0f) qi = 127;
    else qi = (int)r;
    if (j < 16) sum0 += qi; else sum1 += qi;
    if ((j & 3) == 0) packed[j >> 2] = 0;
    packed[j >> 2] |= ((uint32_t)qi & 0xffu) << (8 * (j & 3));
  }
  *scale_out = scale;
  *sum0_out = sum0;
  *sum1_out = sum1;
}

// Block gb of an activation array (q and s point at the block's values and scale): its
// sums go to words of `sums` in the form `kind` / `off` (sum_kind_of, sum_offset_of).
__device__ __forceinline__ void quant32(const float* v, int8_t* q, float* s, uint32_t* sums, size_t gb, int kind,
                                        int32_t off) {
  uint32_t packed[8];
  float scale;
  int sum0, sum1;
  quant32_regs(v, packed, &scale, &sum0, &sum1);
  *s = scale;
  uint4* q4 = reinterpret_cast<uint4*>(q);
  q4[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  q4[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  if (kind == kSumF32x32) {
    sums[gb] = __float_as_uint((float)(sum0 + sum1));
  } else if (kind == kSumF32x16) {
    sums[2 * gb] = __float_as_uint((float)sum0);
    sums[2 * gb + 1] = __float_as_uint((float)sum1);
  } else if (kind == kSumI32x16) {
    sums[2 * gb] = (uint32_t)(off * sum0);
    sums[2 * gb + 1] = (uint32_t)(off * sum1);
  }
}

// quant32 over a wave: lane l holds value l%32 of block l/32 (two consecutive 32-blocks
// per wave). The block maximum and the sums of 16 are cross-lane reductions, which their
// order does not change (the maximum starts from 0, so NaN never wins, as in the serial
// fold); every lane then quantises its own value with quant32's arithmetic. Lanes
// l%4 == 0 store four packed values, lanes 0/32 the scales, lanes 0/32 (sums of 32) or
// 0/16/32/48 (sums of 16) the sums, in the form kind / off, at their words of the row
// `sums` of which the wave holds values r0 .. r0 + 63. `valid` (uniform over each 32-lane
// half) leaves blocks past the end of the row unwritten; every lane of the wave must call
// this.
// Cross-lane moves within a row of 16 lanes as DPP operand modifiers (a VALU operand, no
// LDS round trip as __shfl's ds_bpermute takes): lane i reads lane i ^ 1 (quad_perm
// [1,0,3,2]), i ^ 2 (quad_perm [2,3,0,1]), 7 - i within its 8 (row_half_mirror), 15 - i
// within its 16 (row_mirror), i + n within its row (row_shl:n; lanes past the row's end
// read 0).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140, kDppShl1 = 0x101;

// A lane's value and its xor-16 (xor-32) partner's: v_permlane16_swap (v_permlane32_swap)
// of v with itself leaves the two in the pair's halves, own and partner's in some order
// (checked on the device).
struct LanePair {
  float a, b;
};
__device__ __forceinline__ LanePair xor16_pair(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  return {__int_as_float(p[0]), __int_as_float(p[1])};
}
__device__ __forceinline__ LanePair xor32_pair(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return {__int_as_float(p[0]), __int_as_float(p[1])};
}

// Butterfly sum and maximum over a wave: every lane ends with the result. Each level
// combines two halves that hold the same bits in every lane (a + b and b + a are equal),
// so within a row of 16 the DPP mirrors stand in for xor 4 and xor 8, and the permlane
// swaps give xor 16 and xor 32: no level goes through LDS. Levels run from distance 1 up.
__device__ __forceinline__ float wave64_sum(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  LanePair p = xor16_pair(v);
  v = p.a + p.b;
  p = xor32_pair(v);
  return p.a + p.b;
}
__device__ __forceinline__ float wave64_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  LanePair p = xor16_pair(v);
  v = fmaxf(p.a, p.b);
  p = xor32_pair(v);
  return fmaxf(p.a, p.b);
}
// The same butterfly for an unsigned 64-bit maximum, each level moving the two halves
// (the permlane swaps leave both halves of a lane's pair in the same order).
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return ((uint64_t)(uint32_t)dpp_i<CTRL>((int)(v >> 32)) << 32) | (uint32_t)dpp_i<CTRL>((int)(uint32_t)v);
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t wave64_max_u64(uint64_t v) {
  v = max_u64(v, dpp_u64<kDppXor1>(v));
  v = max_u64(v, dpp_u64<kDppXor2>(v));
  v = max_u64(v, dpp_u64<kDppHalfMirror>(v));
  v = max_u64(v, dpp_u64<kDppMirror>(v));
  auto pl = __builtin_amdgcn_permlane16_swap((int)(uint32_t)v, (int)(uint32_t)v, false, false);
  auto ph = __builtin_amdgcn_permlane16_swap((int)(v >> 32), (int)(v >> 32), false, false);
  v = max_u64(((uint64_t)(uint32_t)ph[0] << 32) | (uint32_t)pl[0], ((uint64_t)(uint32_t)ph[1] << 32) | (uint32_t)pl[1]);
  pl = __builtin_amdgcn_permlane32_swap((int)(uint32_t)v, (int)(uint32_t)v, false, false);
  ph = __builtin_amdgcn_permlane32_swap((int)(v >> 32), (int)(v >> 32), false, false);
  return max_u64(((uint64_t)(uint32_t)ph[0] << 32) | (uint32_t)pl[0], ((uint64_t)(uint32_t)ph[1] << 32) | (uint32_t)pl[1]);
}

// One row's residual add and RMSNorm by the block's first 256 threads; every thread of
// the block calls it (it holds one barrier). With y, x += y first (written back); with SL,
// y is the sum of nsl K slices of a dense product `stride` floats apart, added in slice
// order (k_reduce_parts's sum), each float4's slice loads issued together. Then
// h = (x * scale) * w with scale = 1 / sqrt(mean(x^2) + eps), written to h and, when hl is
// given, to hl as well. A thread holds its kNormVec float4 of the row (d <= 4 * 256 *
// kNormVec) in registers, every load issued before any use. part: 4 floats of LDS.
template <bool SL>
__device__ __forceinline__ void add_norm_row(float* __restrict__ x, const float* __restrict__ y,
                                             const float* __restrict__ w, uint32_t d, float eps,
                                             float* __restrict__ h, float* hl, uint32_t nsl, size_t stride,
                                             float* part) {
  const uint32_t t = threadIdx.x, nv = t < 256 ? d / 4 : 0u;  // threads past 256 only meet the barrier
  float4* xr = reinterpret_cast<float4*>(x);
  const float4* yr = reinterpret_cast<const float4*>(y);
  const float4* wr = reinterpret_cast<const float4*>(w);
  float4* hr = reinterpret_cast<float4*>(h);
  float4 xv[kNormVec], yv[kNormVec];
#pragma unroll
  for (int r = 0; r < kNormVec; r++) {
    const uint32_t c = t + 256 * r;
    if (c < nv) xv[r] = xr[c];
  }
  if (yr) {
#pragma unroll
    for (int r = 0; r < kNormVec; r++) {
      const uint32_t c = t + 256 * r;
      if (c < nv) {
        if constexpr (SL) {
          float4 p[kMaxKsg];
#pragma unroll
          for (uint32_t g = 0; g < kMaxKsg; g++) p[g] = yr[c + (size_t)min(g, nsl - 1) * (stride / 4)];
          float4 a = p[0];
#pragma unroll
          for (uint32_t g = 1; g < kMaxKsg; g++)
            if (g < nsl) a = make_float4(a.x + p[g].x, a.y + p[g].y, a.z + p[g].z, a.w + p[g].w);
          yv[r] = a;
        } else {
          yv[r] = yr[c];
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kNormVec; r++) {
      const uint32_t c = t + 256 * r;
      if (c < nv) {
        xv[r] = make_float4(xv[r].x + yv[r].x, xv[r].y + yv[r].y, xv[r].z + yv[r].z, xv[r].w + yv[r].w);
        xr[c] = xv[r];
      }
    }
  }
  float sq = 0.0f;
#pragma unroll
  for (int r = 0; r < kNormVec; r++) {
    const uint32_t c = t + 256 * r;
    if (c < nv) {
      sq = sq + xv[r].x * xv[r].x;
      sq = sq + xv[r].y * xv[r].y;
      sq = sq + xv[r].z * xv[r].z;
      sq = sq + xv[r].w * xv[r].w;
    }
  }
  if (t < 256) {
    sq = wave64_sum(sq);
    if ((t & 63) == 0) part[t >> 6] = sq;
  }
  __syncthreads();
  const float mean = (part[0] + part[1] + part[2] + part[3]) / (float)d;
  const float scale = fdiv(1.0f, __fsqrt_rn(mean + eps));
#pragma unroll
  for (int r = 0; r < kNormVec; r++) {
    const uint32_t c = t + 256 * r;
    if (c < nv) {
      const float4 v = xv[r], g = wr[c];
      const float4 o = make_float4((v.x * scale) * g.x, (v.y * scale) * g.y, (v.z * scale) * g.z, (v.w * scale) * g.w);
      hr[c] = o;
      if (hl) reinterpret_cast<float4*>(hl)[c] = o;
    }
  }
}

__device__ __forceinline__ void quant_wave(float v, uint32_t lane, bool valid, int8_t* q, float* s, uint32_t* sums,
                                           uint32_t r0, int kind, int32_t off) {
  // the max over the lane's 32 (16 by DPP, then the other 16): after the two quad steps
  // every lane holds its quad's value, after the half mirror its 8's, after the mirror its 16's
  float a = fmaxf(0.0f, fabsf(v));
  a = fmaxf(a, dpp_f<kDppXor1>(a));
  a = fmaxf(a, dpp_f<kDppXor2>(a));
  a = fmaxf(a, dpp_f<kDppHalfMirror>(a));
  a = fmaxf(a, dpp_f<kDppMirror>(a));
  const LanePair ap = xor16_pair(a);
  a = fmaxf(ap.a, ap.b);
  const float scale = fdiv(a, 127.0f);
  const float inv = scale > 0.0f ? fdiv(1.0f, scale) : 0.0f;
  const float r = roundf(v * inv);
  const int qi = (r != r) ? 0 : r < -127.0f ? -127 : r > 127.0f ? 127 : (int)r;
  int sum = qi;  // over the lane's 16, the same way (integer: any order is exact)
  sum += dpp_i<kDppXor1>(sum);
  sum += dpp_i<kDppXor2>(sum);
  sum += dpp_i<kDppHalfMirror>(sum);
  sum += dpp_i<kDppMirror>(sum);
  const auto sp = __builtin_amdgcn_permlane16_swap(sum, sum, false, false);
  const int sum32 = sp[0] + sp[1];
  // lanes 4j pack lanes 4j .. 4j+3 (all in one row)
  const uint32_t b = (uint32_t)qi & 0xffu;
  const uint32_t word = b | ((uint32_t)dpp_i<kDppShl1>((int)b) << 8) | ((uint32_t)dpp_i<kDppShl1 + 1>((int)b) << 16) |
                        ((uint32_t)dpp_i<kDppShl1 + 2>((int)b) << 24);
  if (valid) {
    if ((lane & 3) == 0) reinterpret_cast<uint32_t*>(q)[lane / 4] = word;
    if ((lane & 31) == 0) s[lane / 32] = scale;
    if (kind == kSumF32x32) {
      if ((lane & 31) == 0) sums[(r0 + lane) / 32] = __float_as_uint((float)sum32);
    } else if (kind != kSumNone && (lane & 15) == 0) {
      sums[(r0 + lane) / 16] = kind == kSumF32x16 ? __float_as_uint((float)sum) : (uint32_t)(off * sum);
    }
  }
}

// ---------------------------------------------------------------------------------
// Packed (int8-activation) block dots. Each adds its block's sub-block terms to the
// running row sums of m tokens, in the reference's order, each term evaluated exactly as
// the reference writes it. tok(t) gives token t's view of the block (PkTok): x its int8
// activations, xs its per-32 scales, sm its activation sums in the form the type's dot
// reads them (sum_kind_of), acc its running sum. A sub-block group's quants are unpacked
// once, then every token takes that group's terms before the next group's are unpacked:
// only one group's unpacked quants are live, and each token still adds its terms in K
// order.
// ---------------------------------------------------------------------------------

struct PkTok {
  const int8_t* x;
  const float* xs;
  const uint32_t* sm;
  float* acc;
  // the block's i-th term (its sub-blocks in K order) is added to the running row sum
  __device__ __forceinline__ void put(int, float v) const { *acc += v; }
};

// The same view whose terms are kept instead of added: term i goes to out[i * 64] (one
// lane's column of a [term][64] array in LDS), to be added in K order later.
struct PkTerms {
  const int8_t* x;
  const float* xs;
  const uint32_t* sm;
  float* out;
  __device__ __forceinline__ void put(int i, float v) const { out[i * 64] = v; }
};

// The activation sums a packed dot reads: sum_kind_of / sum_offset_of (gmoe_internal.h).
template <int QT>
__host__ __device__ constexpr int sum_kind() { return sum_kind_of(QT); }
template <int QT>
__host__ __device__ constexpr int32_t sum_offset() { return sum_offset_of(QT); }

// quant/mod.rs:586-621
// PIPE 1: tokens outermost, each token's codes read one group (64 values) ahead of its
// dots; PIPE 2: half a group ahead, each group's low-nibble chain then its high-nibble
// chain (fewer registers: 167 VGPRs in gate/up, three waves a SIMD). The same operations
// in the same order either way (the two chains are separate sums). Measured: the down
// product with the combine and gate/up at half a token an expert take 1 (C2 batch 8
// down 56.3 -> 54.5 us, batch 2 92.6 -> 90.5 us), gate/up at up to one token an expert
// takes 2 (batch 4 134.1 -> 133.2 us); gate/up above that keeps the group-outer form.
template <int PIPE = 0, class Tok>
__device__ __forceinline__ void pk_q4k(const uint32_t* w, uint32_t m, Tok tok) {
  float d = f16f(w[0]), dmin = f16f(w[0] >> 16);
  if constexpr (PIPE == 2) {
    for (uint32_t t = 0; t < m; t++) {
      const auto a = tok(t);
      const uint4* xv = reinterpret_cast<const uint4*>(a.x);
      // half a group (32 codes, two uint4) in flight ahead of the chain that needs it
      uint4 xn0 = xv[0], xn1 = xv[1];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        uint32_t sc1, m1, sc2, m2;
        scale_min_k4(w + 1, 2 * c, sc1, m1);
        scale_min_k4(w + 1, 2 * c + 1, sc2, m2);
        uint4 x0 = xn0, x1 = xn1;
        xn0 = xv[4 * c + 2];
        xn1 = xv[4 * c + 3];
        const uint32_t lo_x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int dl = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) dl = sdot4(w[4 + 8 * c + i] & 0x0f0f0f0fu, lo_x[i], dl);
        x0 = xn0;
        x1 = xn1;
        if (c < 3) {
          xn0 = xv[4 * c + 4];
          xn1 = xv[4 * c + 5];
        }
        const uint32_t hi_x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int dh = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) dh = sdot4((w[4 + 8 * c + i] >> 4) & 0x0f0f0f0fu, hi_x[i], dh);
        const float s1 = __uint_as_float(a.sm[2 * c]), s2 = __uint_as_float(a.sm[2 * c + 1]);
        a.put(2 * c, a.xs[2 * c] * (d * (float)sc1 * (float)dl - dmin * (float)m1 * s1));
        a.put(2 * c + 1, a.xs[2 * c + 1] * (d * (float)sc2 * (float)dh - dmin * (float)m2 * s2));
      }
    }
    return;
  }
  if constexpr (PIPE == 1) {
    for (uint32_t t = 0; t < m; t++) {
      const auto a = tok(t);
      const uint4* xv = reinterpret_cast<const uint4*>(a.x);
      uint4 xn[4];
#pragma unroll
      for (int k = 0; k < 4; k++) xn[k] = xv[k];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        uint32_t xa[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          xa[4 * k] = xn[k].x; xa[4 * k + 1] = xn[k].y; xa[4 * k + 2] = xn[k].z; xa[4 * k + 3] = xn[k].w;
        }
        if (c < 3) {
#pragma unroll
          for (int k = 0; k < 4; k++) xn[k] = xv[4 * (c + 1) + k];
        }
        uint32_t sc1, m1, sc2, m2;
        scale_min_k4(w + 1, 2 * c, sc1, m1);
        scale_min_k4(w + 1, 2 * c + 1, sc2, m2);
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const uint32_t v = w[4 + 8 * c + i];
          dl = sdot4(v & 0x0f0f0f0fu, xa[i], dl);
          dh = sdot4((v >> 4) & 0x0f0f0f0fu, xa[8 + i], dh);
        }
        const float s1 = __uint_as_float(a.sm[2 * c]), s2 = __uint_as_float(a.sm[2 * c + 1]);
        a.put(2 * c, a.xs[2 * c] * (d * (float)sc1 * (float)dl - dmin * (float)m1 * s1));
        a.put(2 * c + 1, a.xs[2 * c + 1] * (d * (float)sc2 * (float)dh - dmin * (float)m2 * s2));
      }
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint32_t sc1, m1, sc2, m2;
    scale_min_k4(w + 1, 2 * c, sc1, m1);
    scale_min_k4(w + 1, 2 * c + 1, sc2, m2);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t v = w[4 + 8 * c + i];
      lo[i] = v & 0x0f0f0f0fu;
      hi[i] = (v >> 4) & 0x0f0f0f0fu;
    }
    for (uint32_t t = 0; t < m; t++) {
      const auto a = tok(t);
      const uint32_t* xa = reinterpret_cast<const uint32_t*>(a.x + 64 * c);
      int dl = 0, dh = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        dl = sdot4(lo[i], xa[i], dl);
        dh = sdot4(hi[i], xa[8 + i], dh);
      }
      const float s1 = __uint_as_float(a.sm[2 * c]), s2 = __uint_as_float(a.sm[2 * c + 1]);
      a.put(2 * c, a.xs[2 * c] * (d * (float)sc1 * (float)dl - dmin * (float)m1 * s1));
      a.put(2 * c + 1, a.xs[2 * c + 1] * (d * (float)sc2 * (float)dh - dmin * (float)m2 * s2));
    }
  }
}

// quant/mod.rs:454-495
template <class Tok>
__device__ __forceinline__ void pk_q5k(const uint32_t* w, uint32_t m, Tok tok) {
  float d = f16f(w[0]), dmin = f16f(w[0] >> 16);
  const uint32_t* qh = w + 4;
  const uint32_t* qs = w + 12;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    uint32_t sc1, m1, sc2, m2;
    scale_min_k4(w + 1, 2 * g, sc1, m1);
    scale_min_k4(w + 1, 2 * g + 1, sc2, m2);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t v = qs[8 * g + i], h = qh[i];
      lo[i] = (v & 0x0f0f0f0fu) | (((h >> (2 * g)) & 0x01010101u) << 4);
      hi[i] = ((v >> 4) & 0x0f0f0f0fu) | (((h >> (2 * g + 1)) & 0x01010101u) << 4);
    }
    for (uint32_t t = 0; t < m; t++) {
      const auto a = tok(t);
      const uint32_t* xa = reinterpret_cast<const uint32_t*>(a.x + 64 * g);
      int dl = 0, dh = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        dl = sdot4(lo[i], xa[i], dl);
        dh = sdot4(hi[i], xa[8 + i], dh);
      }
      const float s1 = __uint_as_float(a.sm[2 * g]), s2 = __uint_as_float(a.sm[2 * g + 1]);
      a.put(2 * g, a.xs[2 * g] * (d * (float)sc1 * (float)dl - dmin * (float)m1 * s1));
      a.put(2 * g + 1, a.xs[2 * g + 1] * (d * (float)sc2 * (float)dh - dmin * (float)m2 * s2));
    }
  }
}

// quant/mod.rs:417-445. Sub-block s (16 wide): q-32 is dotted as q then -32*sum.
template <class Tok>
__device__ __forceinline__ void pk_q6k(const uint32_t* w, uint32_t m, Tok tok) {
  float d = f16f(w[52]);
  for (uint32_t t = 0; t < m; t++) {  // each token's 16 sub-blocks, its codes read a sub-block ahead
    const auto a = tok(t);
    const uint4* xv = reinterpret_cast<const uint4*>(a.x);
    uint4 xn = xv[0];
#pragma unroll
    for (int s = 0; s < 16; s++) {
      const uint4 xc = xn;
      if (s < 15) xn = xv[s + 1];
      const int half = s / 8, quarter = (s % 8) / 2, l0 = 16 * (s % 2);
      uint32_t q[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int l = l0 + 4 * i;
        uint32_t ql = w[(64 * half + l + (quarter & 1) * 32) / 4];
        uint32_t qh = w[(128 + 32 * half + l) / 4];
        uint32_t lo4 = (quarter < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
        uint32_t hi2 = ((qh >> (2 * quarter)) & 0x03030303u) << 4;
        q[i] = lo4 | hi2;
      }
      const float sc = (float)(int8_t)byte_of(w, 192 + s);
      int dt = (int)a.sm[s];  // -32 * the sub-block's sum
      dt = sdot4(q[0], xc.x, dt);
      dt = sdot4(q[1], xc.y, dt);
      dt = sdot4(q[2], xc.z, dt);
      dt = sdot4(q[3], xc.w, dt);
      a.put(s, a.xs[s / 2] * d * sc * (float)dt);
    }
  }
}

// The four words of sub-block s of a Q3_K slab unit w.
__device__ __forceinline__ void q3s_words(const uint32_t* w, int s, uint32_t* q) {
  const uint32_t c = s / 8, x0 = 3 * ((s % 8) / 4);
#pragma unroll
  for (uint32_t h = 0; h < 2; h++)
    q3s_pair(w[q3s_word(c, h, x0)], w[q3s_word(c, h, x0 + 1)], w[q3s_word(c, h, x0 + 2)], s % 4, q[2 * h],
             q[2 * h + 1]);
}

// quant/mod.rs:503-540. q = ((qs >> shift) & 3) - (hmask bit ? 0 : 4), dotted as
// v = low2 | hbit << 2 (the slab unit's regrouped values, q3s_words) then -4*sum.
template <class Tok>
__device__ __forceinline__ void pk_q3k(const uint32_t* w, uint32_t m, Tok tok) {
  float d_all = f16f(w[27]);
  uint32_t sc4[4];
  q3k_scales(w[24], w[25], w[26], sc4);
  uint32_t q[16][4];
  float dl[16];
#pragma unroll
  for (int s = 0; s < 16; s++) {
    q3s_words(w, s, q[s]);
    dl[s] = d_all * (float)((int)(int8_t)byte_of(sc4, s) - 32);
  }
  for (uint32_t t = 0; t < m; t++) {  // each token's 16 sub-blocks, its codes read a sub-block ahead
    const auto a = tok(t);
    const uint4* xv = reinterpret_cast<const uint4*>(a.x);
    uint4 xn = xv[0];
#pragma unroll
    for (int s = 0; s < 16; s++) {
      const uint4 xc = xn;
      if (s < 15) xn = xv[s + 1];
      int dt = (int)a.sm[s];  // -4 * the sub-block's sum
      dt = sdot4(q[s][0], xc.x, dt);
      dt = sdot4(q[s][1], xc.y, dt);
      dt = sdot4(q[s][2], xc.z, dt);
      dt = sdot4(q[s][3], xc.w, dt);
      a.put(s, a.xs[s / 2] * dl[s] * (float)dt);
    }
  }
}

// quant/mod.rs:548-581
template <class Tok>
__device__ __forceinline__ void pk_q2k(const uint32_t* w, uint32_t m, Tok tok) {
  float d = f16f(w[20]), dmin = f16f(w[20] >> 16);
#pragma unroll
  for (int s = 0; s < 16; s++) {
    const int half = s / 8, j = (s % 8) / 2, o = 16 * (s % 2);
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = (w[(16 + 32 * half + o) / 4 + i] >> (2 * j)) & 0x03030303u;
    uint32_t sc = byte_of(w, s);
    float dl = d * (float)(sc & 15u), ml = dmin * (float)(sc >> 4);
    for (uint32_t t = 0; t < m; t++) {
      const auto a = tok(t);
      const uint32_t* xa = reinterpret_cast<const uint32_t*>(a.x + 16 * s);
      int dt = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) dt = sdot4(q[i], xa[i], dt);
      a.put(s, a.xs[s / 2] * (dl * (float)dt - ml * __uint_as_float(a.sm[s])));
    }
  }
}

// quant/mod.rs:398-407 over a repacked Q8_0 unit of the slab (eight blocks: their f16
// scales in dwords 0..3, then their quants): block g adds ws*xs*dot. nvalid = blocks of
// the unit inside the row.
template <class Tok>
__device__ __forceinline__ void pk_q80_unit(const uint32_t* w, uint32_t nvalid, uint32_t m, Tok tok) {
#pragma unroll
  for (int g = 0; g < 8; g++) {
    if ((uint32_t)g < nvalid) {
      const float ws = f16f(w[g / 2] >> (16 * (g % 2)));
      const uint32_t* q = w + 4 + 8 * g;
      for (uint32_t t = 0; t < m; t++) {
        const auto a = tok(t);
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(a.x + 32 * g);
        int dt = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) dt = sdot4(q[i], xa[i], dt);
        a.put(g, ws * a.xs[g] * (float)dt);
      }
    }
  }
}

// One slab unit of a packed type against m tokens (nvalid: blocks of the unit inside the
// row, for the eight-block Q8_0 units).
template <int QT, int PIPE = 0, class Tok>
__device__ __forceinline__ void pk_unit(const uint32_t* w, uint32_t nvalid, uint32_t m, Tok tok) {
  if constexpr (QT == Q4_K) pk_q4k<PIPE>(w, m, tok);
  else if constexpr (QT == Q5_K) pk_q5k(w, m, tok);
  else if constexpr (QT == Q6_K) pk_q6k(w, m, tok);
  else if constexpr (QT == Q3_K) pk_q3k(w, m, tok);
  else if constexpr (QT == Q2_K) pk_q2k(w, m, tok);
  else if constexpr (QT == Q8_0) pk_q80_unit(w, nvalid, m, tok);
}

// ---------------------------------------------------------------------------------
// Ranking and gating
// ---------------------------------------------------------------------------------

// f32::total_cmp key
__device__ __forceinline__ int total_key(float f) {
  int i = __float_as_int(f);
  return i ^ (int)(((uint32_t)(i >> 31)) >> 1);
}

// rank order: llama = total_cmp descending, stable (llama/mod.rs:943);
// router = partial_cmp descending, equal -> lower id first (router/mod.rs:83-88). The
// router's comparator is no order once a logit is NaN (NaN compares Equal to every value,
// which is not transitive; Rust's sort_by then gives an unspecified order and may panic),
// so this build ranks a NaN logit after every number and NaNs among themselves by id: a
// strict total order that agrees with partial_cmp wherever that is one, so the counted
// ranks below are always a permutation.
__device__ __forceinline__ bool ranks_before(bool llama, float a, uint32_t ia, float b, uint32_t ib) {
  if (llama) {
    int ka = total_key(a), kb = total_key(b);
    return ka > kb || (ka == kb && ia < ib);
  }
  const bool na = a != a, nb = b != b;
  if (na || nb) return na == nb ? ia < ib : nb;
  if (a > b) return true;
  if (a < b) return false;
  return ia < ib;
}

// ---------------------------------------------------------------------------------
// Gating by one wave (ne <= 64: lane e holds expert e). It computes what gate_block does,
// with every ordered sum taken lane by lane in index order through readlane, so the
// arithmetic is the same; maxima, which no order changes, are cross-lane reductions.
// ---------------------------------------------------------------------------------

__device__ __forceinline__ float lane_f(float v, uint32_t l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)l));
}
__device__ __forceinline__ uint32_t lane_u(uint32_t v, uint32_t l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}

// The top-k weights after ranking: lane i < k holds the i-th ranked expert's value w
// (probability, or logit under Mixtral gating); returns its final weight
// (llama/mod.rs:945-949, router/mod.rs:91-115).
__device__ __forceinline__ float gate_topk_weights(uint32_t gating, uint32_t k, float w) {
  if (gating == 0) {  // llama/mod.rs:945-949
    float sum = -0.0f;
    for (uint32_t i = 0; i < k; i++) sum += lane_f(w, i);
    w *= sum > 0.0f ? fdiv(1.0f, sum) : fdiv(1.0f, (float)k);
  } else if (gating == 1) {  // router/mod.rs:91-97: softmax over the k kept logits
    float mx = -INFINITY;
    for (uint32_t i = 0; i < k; i++) mx = fmaxf(mx, lane_f(w, i));
    if (!isfinite(mx)) {
      w = fdiv(1.0f, (float)k);
    } else {
      w = gm_expf(w - mx);
      float sum = 0.0f;
      for (uint32_t i = 0; i < k; i++) sum += lane_f(w, i);
      w = (isfinite(sum) && sum > 0.0f) ? w * fdiv(1.0f, sum) : fdiv(1.0f, (float)k);
    }
  } else if (gating == 3) {  // router/mod.rs:102-115
    float sum = -0.0f;
    for (uint32_t i = 0; i < k; i++) sum += lane_f(w, i);
    w = sum > 0.0f ? fdiv(w, sum) : fdiv(1.0f, (float)k);
  }
  return w;
}

// gate_wave for up to 64*EPL experts: lane l holds experts l, l + 64, ... in x[0..EPL).
// Every ordered sum still runs over the experts in index order (readlane), so the
// arithmetic is gate_wave's. Lanes r < k receive the r-th ranked expert and its weight.
// `scratch` holds 2*k words of LDS.
template <int EPL>
__device__ void gate_wave_wide(uint32_t gating, uint32_t ne, uint32_t k, const float* x, uint32_t lane,
                               uint32_t* id_out, float* w_out, uint32_t* scratch) {
  const bool llama = gating == 0;
  float v[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j++) v[j] = x[j];
  if (gating == 0 || gating == 2 || gating == 3) {  // softmax over all experts (simd/mod.rs:132-158)
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPL; j++)
      if (64 * j + lane < ne) mx = fmaxf(mx, x[j]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float inv = -1.0f;  // uniform
    if (isfinite(mx)) {
#pragma unroll
      for (int j = 0; j < EPL; j++) v[j] = gm_expf(x[j] - mx);
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < EPL; j++)
        for (uint32_t l = 0; l < 64 && 64 * j + l < ne; l++) sum += lane_f(v[j], l);
      if (isfinite(sum) && sum > 0.0f) inv = fdiv(1.0f, sum);
    }
#pragma unroll
    for (int j = 0; j < EPL; j++) v[j] = inv < 0.0f ? fdiv(1.0f, (float)ne) : v[j] * inv;
  }
  float* tw = reinterpret_cast<float*>(scratch);
  uint32_t* ti = scratch + k;
  // The rank order (ranks_before) is a strict total order, so the r-th ranked expert is
  // the r-th pick of k rounds of a wave-wide maximum over the key (value key, then ~id,
  // so that ties go to the lower id).
  {
    uint64_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      const uint32_t e = 64 * j + lane;
      // order-preserving unsigned image of the rank order's value key: under partial_cmp
      // +0 and -0 are one value and a NaN comes after every number (0, below -inf's key)
      const uint32_t vk = llama ? (uint32_t)total_key(v[j]) ^ 0x80000000u
                          : v[j] != v[j] ? 0u
                                         : (uint32_t)total_key(v[j] == 0.0f ? 0.0f : v[j]) ^ 0x80000000u;
      key[j] = e < ne ? ((uint64_t)vk << 32) | (uint64_t)(0xffffffffu - e) : 0ull;
    }
    for (uint32_t r = 0; r < k; r++) {
      uint64_t best = 0ull;
#pragma unroll
      for (int j = 0; j < EPL; j++) best = key[j] > best ? key[j] : best;
      best = wave64_max_u64(best);  // DPP and permlane levels: no LDS round trip a level
      const uint32_t e = 0xffffffffu - (uint32_t)best;
#pragma unroll
      for (int j = 0; j < EPL; j++)
        if (key[j] == best && best != 0ull) {  // the owner records the pick
          tw[r] = v[j];
          ti[r] = e;
          key[j] = 0ull;
        }
    }
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");  // one wave: its DS writes land before these reads
  const float w = lane < k ? tw[lane] : 0.0f;
  *id_out = lane < k ? ti[lane] : 0u;
  *w_out = gate_topk_weights(gating, k, w);
}

// One token's routing from its logit x (lane e < ne). Lanes r < k receive the r-th
// ranked expert and its weight. `scratch` holds 2*k words of LDS.
__device__ void gate_wave(uint32_t gating, uint32_t ne, uint32_t k, float x, uint32_t lane, uint32_t* id_out,
                          float* w_out, uint32_t* scratch) {
  const bool llama = gating == 0;
  float v = x;
  if (gating == 0 || gating == 2 || gating == 3) {  // softmax over all experts (simd/mod.rs:132-158)
    float mx = -INFINITY;
    for (uint32_t e = 0; e < ne; e++) mx = fmaxf(mx, lane_f(x, e));
    if (isfinite(mx)) v = gm_expf(x - mx);
    float inv = -1.0f;  // uniform
    if (isfinite(mx)) {
      float sum = 0.0f;
      for (uint32_t e = 0; e < ne; e++) sum += lane_f(v, e);
      if (isfinite(sum) && sum > 0.0f) inv = fdiv(1.0f, sum);
    }
    v = inv < 0.0f ? fdiv(1.0f, (float)ne) : v * inv;
  }
  // rank = how many experts come before this one
  uint32_t r = 0;
  for (uint32_t o = 0; o < ne; o++)
    if (o != lane && ranks_before(llama, lane_f(v, o), o, v, lane)) r++;
  float* tw = reinterpret_cast<float*>(scratch);
  uint32_t* ti = scratch + k;
  if (lane < ne && r < k) {
    tw[r] = v;
    ti[r] = lane;
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");  // one wave: its DS writes land before these reads
  const float w = lane < k ? tw[lane] : 0.0f;
  *id_out = lane < k ? ti[lane] : 0u;
  *w_out = gate_topk_weights(gating, k, w);
}


// The combine's inputs of token t from its gating (id, w of lane < k): the pair's place in
// the combine's order (among the token's k ids when the combine runs in expert order)
// and its slot, found by binary search among the expert's candidate slots (~0u when the
// candidates missed it).
__device__ __forceinline__ void route_comb(const RouteArgs& r, uint32_t t, uint32_t id, float w, uint32_t lane) {
  uint32_t pos = lane;
  if (r.combine == 0) {
    pos = 0;
    for (uint32_t j = 0; j < r.k; j++) pos += lane_u(id, j) < id ? 1u : 0u;
  }
  if (lane < r.k) {
    uint32_t lo = r.offsets[id], hi = r.offsets[id + 1];
    const uint32_t end = hi;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) / 2;
      if (r.slot_tok[mid] < t) lo = mid + 1;
      else hi = mid;
    }
    r.comb_slot[(size_t)t * r.k + pos] = lo < end && r.slot_tok[lo] == t ? lo : ~0u;
    r.comb_w[(size_t)t * r.k + pos] = w;
  }
}

// ---------------------------------------------------------------------------------
// Exact router logit of one (token, expert) pair by one workgroup of two or more waves,
// then the token's gating by the last of its ne workgroups. Wave 1 puts the products w*h
// of a section of d into LDS (two halves: the next section while wave 0 adds the
// current one); lane 0 of wave 0 runs the chain, the reference's sequential f32 sum from
// -0.0 (simd/mod.rs:13-16). The logit goes to memory; the workgroup that brings the
// token's counter to ne (after a release fence) gates all ne logits (gate_wave) and puts
// the counter back to zero. lds holds 2 * sec floats and 2k words. Every thread of the
// workgroup must call this.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void route_logit(const RouteArgs& r, uint32_t x, float* lds) {
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint32_t ne = r.ne, d = r.d, sec = r.sec, nsec = (d + sec - 1) / sec;
  const uint32_t t = x / ne, e = x % ne;
  const float* hs = r.hs + (size_t)t * d;
  const float* wr = r.router + (size_t)e * d;
  uint32_t* scratch = reinterpret_cast<uint32_t*>(lds + 2 * sec);
  constexpr int kItems = 4;  // a 1024-value section is one pass of 64 lanes; few registers, as the launch sizes them for the expert workgroups
  auto produce = [&](uint32_t s) {
    const uint32_t k0 = s * sec, len4 = min(sec, d - k0) / 4;
    float* half = lds + (s & 1) * sec;
    for (uint32_t base = 0; base < len4; base += 64 * kItems) {
      float4 wv[kItems], xv[kItems];
#pragma unroll
      for (int i = 0; i < kItems; i++) {
        const uint32_t j = base + lane + 64 * i;
        if (j < len4) {
          wv[i] = reinterpret_cast<const float4*>(wr + k0)[j];
          xv[i] = reinterpret_cast<const float4*>(hs + k0)[j];
        }
      }
#pragma unroll
      for (int i = 0; i < kItems; i++) {
        const uint32_t j = base + lane + 64 * i;
        if (j < len4)
          reinterpret_cast<float4*>(half)[j] =
              make_float4(wv[i].x * xv[i].x, wv[i].y * xv[i].y, wv[i].z * xv[i].z, wv[i].w * xv[i].w);
      }
    }
  };
  if (wave == 1) produce(0);
  __syncthreads();
  float acc = -0.0f;
  for (uint32_t s = 0; s < nsec; s++) {
    if (wave == 0) {
      if (lane == 0) {
        const float4* src = reinterpret_cast<const float4*>(lds + (s & 1) * sec);
        const uint32_t len4 = min(sec, d - s * sec) / 4;
        for (uint32_t j = 0; j < len4; j++) {
          const float4 v = src[j];
          acc = acc + v.x;
          acc = acc + v.y;
          acc = acc + v.z;
          acc = acc + v.w;
        }
      }
    } else if (wave == 1 && s + 1 < nsec) {
      produce(s + 1);
    }
    __syncthreads();
  }
  if (wave != 0) return;
  if (lane == 0) r.logits[(size_t)t * ne + e] = acc;
  __threadfence();
  uint32_t prev = 0;
  if (lane == 0) prev = atomicAdd(r.tok_done + t, 1u);
  if (lane_u(prev, 0) != ne - 1) return;
  __threadfence();
  const float lg = lane < ne ? r.logits[(size_t)t * ne + lane] : 0.0f;
  uint32_t id;
  float w;
  gate_wave(r.gating, ne, r.k, lg, lane, &id, &w, scratch);
  if (lane < r.k) {
    r.ids[(size_t)t * r.k + lane] = id;
    r.w[(size_t)t * r.k + lane] = w;
  }
  route_comb(r, t, id, w, lane);
  if (lane == 0) r.tok_done[t] = 0;
}

// ---------------------------------------------------------------------------------
// Exact routing of one token by one workgroup of two or more waves: lane e of wave 0 runs
// expert e's chain, the reference's sequential f32 dot from -0.0 (simd/mod.rs:13-16),
// over the products w*h that the other waves put in LDS one section of d ahead (two
// halves of [ne][sec + 4]); lane e reads its products 32 at a time from two register
// buffers, each fetched one batch ahead. Then wave 0 gates the token (gate_wave), writes
// its logits, ids and weights and the combine's (slot, weight) pairs, and bumps `routed`
// (when given) after a release fence. With cand, the token's candidate experts in
// ascending id (LDS, nc of them, one token a call), a routed pair's slot is its
// expert's rank among them; otherwise the search of route_comb finds it (nothing with
// comb_slot null: the routing alone). sec: a
// multiple of 64 (d too), lds: route_token_lds floats.
// Every thread of the workgroup calls this; ne <= 64.
// ---------------------------------------------------------------------------------
__host__ __device__ inline uint32_t route_token_lds(uint32_t ne, uint32_t k, uint32_t sec) {
  return 2 * ne * (sec + 4) + 2 * k;
}

__device__ __forceinline__ void route_token(const RouteArgs& r, uint32_t t, float* lds, uint32_t sec,
                                            uint32_t* routed, const uint32_t* cand = nullptr, uint32_t nc = 0) {
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, np = blockDim.x - 64;
  const uint32_t ne = r.ne, d = r.d, row = sec + 4, nsec = (d + sec - 1) / sec;
  float* prod = lds;  // [2][ne][row]
  uint32_t* scratch = reinterpret_cast<uint32_t*>(lds + 2 * ne * row);
  const float* hs = r.hs + (size_t)t * d;
  constexpr int kItems = 4;  // float4 products a producer thread has in flight
  auto produce = [&](uint32_t s) {
    const uint32_t k0 = s * sec, len4 = min(sec, d - k0) / 4, total = ne * len4;
    float* half = prod + (s & 1) * ne * row;
    for (uint32_t base = tid - 64; base < total; base += np * kItems) {
      float4 wv[kItems], xv[kItems];
      uint32_t off[kItems];
#pragma unroll
      for (int i = 0; i < kItems; i++) {
        const uint32_t q = base + np * i;
        if (q < total) {
          const uint32_t e = q / len4, j = q - e * len4;
          wv[i] = reinterpret_cast<const float4*>(r.router + (size_t)e * d + k0)[j];
          xv[i] = reinterpret_cast<const float4*>(hs + k0)[j];
          off[i] = e * row + 4 * j;
        }
      }
#pragma unroll
      for (int i = 0; i < kItems; i++)
        if (base + np * i < total)
          *reinterpret_cast<float4*>(half + off[i]) =
              make_float4(wv[i].x * xv[i].x, wv[i].y * xv[i].y, wv[i].z * xv[i].z, wv[i].w * xv[i].w);
    }
  };
  if (wave != 0) produce(0);
  __syncthreads();
  float acc = -0.0f;
  for (uint32_t s = 0; s < nsec; s++) {
    if (wave == 0) {
      if (lane < ne) {
        const uint32_t nb = min(sec, d - s * sec) / 32;  // even: sections and d are multiples of 64
        const float4* src = reinterpret_cast<const float4*>(prod + (s & 1) * ne * row + lane * row);
        float4 ba[8], bb[8];
        auto fetch = [&](float4* dst, uint32_t b) {
#pragma unroll
          for (int u = 0; u < 8; u++) dst[u] = src[8 * b + u];
        };
        auto add = [&](const float4* v) {
#pragma unroll
          for (int u = 0; u < 8; u++) {
            acc = acc + v[u].x;
            acc = acc + v[u].y;
            acc = acc + v[u].z;
            acc = acc + v[u].w;
          }
        };
        fetch(ba, 0);
        for (uint32_t b = 0; b < nb; b += 2) {
          fetch(bb, b + 1);
          add(ba);
          fetch(ba, min(b + 2, nb - 1));  // the last round re-reads a batch it does not add
          add(bb);
        }
      }
    } else if (s + 1 < nsec) {
      produce(s + 1);
    }
    __syncthreads();
  }
  if (wave != 0) return;
  if (lane < ne) r.logits[(size_t)t * ne + lane] = acc;
  uint32_t id;
  float w;
  gate_wave(r.gating, ne, r.k, lane < ne ? acc : 0.0f, lane, &id, &w, scratch);
  if (lane < r.k) {
    r.ids[(size_t)t * r.k + lane] = id;
    r.w[(size_t)t * r.k + lane] = w;
  }
  if (!r.comb_slot) {  // the routing alone (k_route_tok)
  } else if (cand) {  // one token, its candidates cand[0..nc) (LDS): a routed pair's slot is its rank
    uint32_t p = lane;
    if (r.combine == 0) {
      p = 0;
      for (uint32_t j = 0; j < r.k; j++) p += lane_u(id, j) < id ? 1u : 0u;
    }
    if (lane < r.k) {
      uint32_t slot = ~0u;
      for (uint32_t j = 0; j < nc; j++)
        if (cand[j] == id) slot = j;
      r.comb_slot[(size_t)t * r.k + p] = slot;
      r.comb_w[(size_t)t * r.k + p] = w;
    }
  } else {
    route_comb(r, t, id, w, lane);
  }
  if (routed) {
    __threadfence();
    if (lane == 0) atomicAdd(routed, 1u);
  }
}

// ---------------------------------------------------------------------------------
// Speculative routing (decode). The exact router logit is d dependent f32 adds
// (simd/mod.rs:13-16); the expert products only need to know which experts to stream.
//  * logit L~_e: the same rounded products w*h summed as d/64-long lane sums and a
//    64-lane tree. With S the exact sum of the rounded products and A = sum |products|,
//    recursive summation gives |L_seq - S| <= g(d-1) A and the tree |L~ - S| <= g(m) A,
//    m = d/64 + 4 KB + 7 (every lane addition, zero padding included, and the 6 tree
//    levels; KB float4 pairs a lane loads at a time), g(m) = m u / (1 - m u), u = 2^-24;
//    so |L~ - L_seq| <= delta_e.
//  * candidates: expert e is left out only when at least k others certainly rank before
//    it, L~_j - delta_j > L~_e + delta_e + eps_e; eps_e keeps their probabilities apart
//    after expf and the normalisation, so the exact order puts them first whatever the
//    tie rule. Non-finite logits, or fewer than k experts safely above expf's underflow,
//    make every expert a candidate. The exact top k is therefore a subset.
// ---------------------------------------------------------------------------------
constexpr uint32_t kSpecMaxExperts = 64;

__device__ __forceinline__ double sum_gamma(double m) {
  const double u = 0x1p-24;
  return m * u / (1.0 - m * u);
}

// Wave w of the workgroup takes experts w, w + waves, ...: lt[e] = the products' tree sum,
// la[e] = the sum of their magnitudes (LDS, written by lane 0). hs: the token's row. KB:
// float4 pairs a lane has in flight.
template <int KB>
__device__ __forceinline__ void spec_dots(const float* __restrict__ router, const float* hs, uint32_t ne, uint32_t d,
                                          float* lt, float* la) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const float4* xr = reinterpret_cast<const float4*>(hs);
  const uint32_t n4 = d / 4;
  for (uint32_t e = wave; e < ne; e += nw) {
    const float4* wr = reinterpret_cast<const float4*>(router + (size_t)e * d);
    float sm = 0.0f, ab = 0.0f;
    for (uint32_t j0 = 0; j0 < n4; j0 += 64 * KB) {  // lane j: float4 columns j, j + 64, ...
      float4 wv[KB], xv[KB];
#pragma unroll
      for (int i = 0; i < KB; i++) {
        const uint32_t j = j0 + lane + 64 * i;
        if (j < n4) {
          wv[i] = wr[j];
          xv[i] = xr[j];
        } else {
          wv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          xv[i] = wv[i];
        }
      }
#pragma unroll
      for (int i = 0; i < KB; i++) {
        const float p0 = wv[i].x * xv[i].x, p1 = wv[i].y * xv[i].y, p2 = wv[i].z * xv[i].z, p3 = wv[i].w * xv[i].w;
        sm = sm + p0; sm = sm + p1; sm = sm + p2; sm = sm + p3;
        ab = ab + fabsf(p0); ab = ab + fabsf(p1); ab = ab + fabsf(p2); ab = ab + fabsf(p3);
      }
    }
    sm = wave64_sum(sm);  // a tree of 6 levels, as the bound counts
    ab = wave64_sum(ab);
    if (lane == 0) {
      lt[e] = sm;
      la[e] = ab;
    }
  }
}

// One wave (lane e < ne: expert e), after lt/la are complete: the candidate test in
// double. Returns the number of candidates nc; cl[0..nc) (LDS) holds them in ascending id,
// *cand says whether this lane's expert is one and *pos its rank among them. sb: LDS of
// 2 * kSpecMaxExperts doubles. KB: that of the spec_dots that made lt and la.
template <int KB>
__device__ __forceinline__ uint32_t spec_candidates(uint32_t ne, uint32_t k, uint32_t d, uint32_t gating, const float* lt,
                                                    const float* la, double* sb, uint32_t* cl, uint32_t lane, bool* cand,
                                                    uint32_t* pos) {
  const double m_tree = (double)(d / 64 + 4 * KB + 7), m_seq = (double)d;
  const bool valid = lane < ne;
  const double Lt = valid ? (double)lt[lane] : 0.0;
  const double A = valid ? (double)la[lane] / (1.0 - sum_gamma(m_tree)) : 0.0;
  const double delta = (sum_gamma(m_seq) + sum_gamma(m_tree)) * A * (1.0 + 0x1p-20);
  const bool fin = !valid || (isfinite(Lt) && isfinite(delta));
  const double lo = Lt - delta, hi = Lt + delta;
  // every lane reads every expert's bounds from LDS, eight at a time with their loads
  // issued together (a shuffle per expert would wait out one LDS round trip each)
  if (valid) {
    sb[lane] = lo;
    sb[kSpecMaxExperts + lane] = hi;
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");  // one wave: its DS writes land before these reads
  // f(j, lo_j, hi_j) for j = 0 .. ne-1 in order
  auto each = [&](auto f) {
    for (uint32_t j0 = 0; j0 < ne; j0 += 8) {
      double l8[8], h8[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t j = min(j0 + i, ne - 1);
        l8[i] = sb[j];
        h8[i] = sb[kSpecMaxExperts + j];
      }
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (j0 + i < ne) f(j0 + i, l8[i], h8[i]);
    }
  };
  double maxhi = -INFINITY;
  each([&](uint32_t, double, double hj) { maxhi = fmax(maxhi, hj); });
  const bool all_fin = __ballot(!fin) == 0ull;
  // experts certainly clear of expf's underflow relative to the largest logit
  const uint32_t safe = (uint32_t)__popcll(__ballot(valid && lo - maxhi > -80.0));
  const bool all = !all_fin || (gating != 1 && safe < k);
  const double eps = 4e-6 * (1.0 + fabs(Lt) + fabs(maxhi));
  uint32_t above = 0;
  each([&](uint32_t j, double loj, double) {
    if (j != lane && loj > hi + eps) above++;
  });
  const bool c = valid && (all || above < k);
  const uint64_t cm = __ballot(c);
  const uint32_t p = (uint32_t)__popcll(cm & ((1ull << lane) - 1ull)), nc = (uint32_t)__popcll(cm);
  if (c) cl[p] = lane;
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");  // one wave: its DS writes land before these reads
  *cand = c;
  *pos = p;
  return nc;
}

}  // namespace gmoe
