// gmoe_kernels.hip — gfx950 kernels of the MoE feed-forward path.
//
// Reference semantics (hanumanit/garuda 0.31.0):
//   routing      llama/mod.rs:935-949 (softmax, stable top-k, renormalise) and
//                router/mod.rs:58-118 (Mixtral / DeepSeek / QwenMoe)
//   dispatch     llama/mod.rs:966-972 (members[e] in ascending token order)
//   experts      llama/mod.rs:1002-1020 via quant::matmul (quant/mod.rs:223-304) or
//                simd::matmul over dequantised weights (simd/mod.rs:96-129)
//   combine      llama/mod.rs:974-997 with simd::add_scaled (simd/mod.rs:182-185)
//
// Built with -ffp-contract=off: a multiply and an add are only fused where this file
// writes fmaf()/fma() itself, which it does only where the reference's result is
// unchanged by it (or where the path is tolerance-checked, the f32 expert products).
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
// Block traits and loads. Rows start 16-byte aligned (row pitch); a block inside a
// row is 16-, 4- or 2-byte aligned depending on its size.
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
// Dequantisation (bit-exact, quant/mod.rs:624-875). deq<QT>(w, out) writes the E
// values of one block in the reference's element order.
// ---------------------------------------------------------------------------------

template <int QT> __device__ __forceinline__ void deq(const uint32_t* w, float* out);

template <> __device__ __forceinline__ void deq<Q4_K>(const uint32_t* w, float* out) {
  float d = f16f(w[0]), dmin = f16f(w[0] >> 16);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint32_t sc1, m1, sc2, m2;
    scale_min_k4(w + 1, 2 * c, sc1, m1);
    scale_min_k4(w + 1, 2 * c + 1, sc2, m2);
    float d1 = d * (float)sc1, mn1 = dmin * (float)m1;
    float d2 = d * (float)sc2, mn2 = dmin * (float)m2;
#pragma unroll
    for (int l = 0; l < 32; l++) {
      uint32_t b = byte_of(w + 4 + 8 * c, l);
      out[64 * c + l] = d1 * (float)(b & 15u) - mn1;
      out[64 * c + 32 + l] = d2 * (float)(b >> 4) - mn2;
    }
  }
}

template <> __device__ __forceinline__ void deq<Q5_K>(const uint32_t* w, float* out) {
  float d = f16f(w[0]), dmin = f16f(w[0] >> 16);
  const uint32_t* qh = w + 4;
  const uint32_t* qs = w + 12;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    uint32_t sc1, m1, sc2, m2;
    scale_min_k4(w + 1, 2 * g, sc1, m1);
    scale_min_k4(w + 1, 2 * g + 1, sc2, m2);
    float d1 = d * (float)sc1, mn1 = dmin * (float)m1;
    float d2 = d * (float)sc2, mn2 = dmin * (float)m2;
#pragma unroll
    for (int l = 0; l < 32; l++) {
      uint32_t ql = byte_of(qs + 8 * g, l), h = byte_of(qh, l);
      uint32_t hi1 = (h >> (2 * g)) & 1u, hi2 = (h >> (2 * g + 1)) & 1u;
      out[64 * g + l] = d1 * (float)((ql & 15u) + 16u * hi1) - mn1;
      out[64 * g + 32 + l] = d2 * (float)((ql >> 4) + 16u * hi2) - mn2;
    }
  }
}

template <> __device__ __forceinline__ void deq<Q6_K>(const uint32_t* w, float* out) {
  float d = f16f(w[52]);  // bytes 208..209 are the low half of dword 52
#pragma unroll
  for (int half = 0; half < 2; half++) {
#pragma unroll
    for (int l = 0; l < 32; l++) {
      int is = l / 16;
      uint32_t ql0 = byte_of(w, 64 * half + l), ql1 = byte_of(w, 64 * half + l + 32);
      uint32_t qh = byte_of(w, 128 + 32 * half + l);
      int q1 = (int)((ql0 & 15u) | ((qh & 3u) << 4)) - 32;
      int q2 = (int)((ql1 & 15u) | (((qh >> 2) & 3u) << 4)) - 32;
      int q3 = (int)((ql0 >> 4) | (((qh >> 4) & 3u) << 4)) - 32;
      int q4 = (int)((ql1 >> 4) | (((qh >> 6) & 3u) << 4)) - 32;
      float s0 = (float)(int8_t)byte_of(w, 192 + 8 * half + is);
      float s2 = (float)(int8_t)byte_of(w, 192 + 8 * half + is + 2);
      float s4 = (float)(int8_t)byte_of(w, 192 + 8 * half + is + 4);
      float s6 = (float)(int8_t)byte_of(w, 192 + 8 * half + is + 6);
      out[128 * half + l] = d * s0 * (float)q1;
      out[128 * half + l + 32] = d * s2 * (float)q2;
      out[128 * half + l + 64] = d * s4 * (float)q3;
      out[128 * half + l + 96] = d * s6 * (float)q4;
    }
  }
}

template <> __device__ __forceinline__ void deq<Q3_K>(const uint32_t* w, float* out) {
  float d_all = f16f(w[27]);  // bytes 108..109
  uint32_t sc4[4];
  // scale bytes 96..107 = w[24..26]
  q3k_scales(w[24], w[25], w[26], sc4);
  int is = 0;
  uint32_t m = 1;
#pragma unroll
  for (int half = 0; half < 2; half++) {
    int shift = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int o = 0; o < 32; o += 16) {
        float dl = d_all * (float)((int)(int8_t)byte_of(sc4, is) - 32);
        is++;
#pragma unroll
        for (int l = 0; l < 16; l++) {
          int hbit = (byte_of(w, l + o) & m) ? 0 : 4;
          int q = (int)((byte_of(w, 32 + 32 * half + o + l) >> shift) & 3u) - hbit;
          out[128 * half + 32 * j + o + l] = dl * (float)q;
        }
      }
      shift += 2;
      m <<= 1;
    }
  }
}

template <> __device__ __forceinline__ void deq<Q2_K>(const uint32_t* w, float* out) {
  float d = f16f(w[20]), dmin = f16f(w[20] >> 16);  // bytes 80..83
  int is = 0;
#pragma unroll
  for (int half = 0; half < 2; half++) {
    int shift = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int o = 0; o < 32; o += 16) {
        uint32_t sc = byte_of(w, is);
        is++;
        float dl = d * (float)(sc & 15u), ml = dmin * (float)(sc >> 4);
#pragma unroll
        for (int l = 0; l < 16; l++) {
          uint32_t q = (byte_of(w, 16 + 32 * half + o + l) >> shift) & 3u;
          out[128 * half + 32 * j + o + l] = dl * (float)q - ml;
        }
      }
      shift += 2;
    }
  }
}

template <> __device__ __forceinline__ void deq<Q8_0>(const uint32_t* w, float* out) {
  float s = f16f(w[0]);
#pragma unroll
  for (int i = 0; i < 32; i++) out[i] = s * (float)(int8_t)byte_of(w, 2 + i);
}

template <> __device__ __forceinline__ void deq<Q4_0>(const uint32_t* w, float* out) {
  float s = f16f(w[0]);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    uint32_t b = byte_of(w, 2 + i);
    out[i] = s * (float)((int)(b & 15u) - 8);
    out[i + 16] = s * (float)((int)(b >> 4) - 8);
  }
}

template <> __device__ __forceinline__ void deq<F16>(const uint32_t* w, float* out) {
#pragma unroll
  for (int i = 0; i < 16; i++) {
    out[2 * i] = f16f(w[i]);
    out[2 * i + 1] = f16f(w[i] >> 16);
  }
}

template <> __device__ __forceinline__ void deq<F32>(const uint32_t* w, float* out) {
#pragma unroll
  for (int i = 0; i < 32; i++) out[i] = __uint_as_float(w[i]);
}

template <int QT>
__global__ void __launch_bounds__(256) k_dequant(const uint8_t* __restrict__ blocks, size_t nblocks,
                                                 float* __restrict__ out) {
  size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  uint32_t w[ndw<QT>()];
  const uint8_t* p = blocks + b * QT_<QT>::B;
  // The test buffer is a plain packed tensor: read byte-wise so no alignment is assumed.
#pragma unroll
  for (int i = 0; i < ndw<QT>(); i++) {
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (4 * i + j < QT_<QT>::B) v |= (uint32_t)p[4 * i + j] << (8 * j);
    w[i] = v;
  }
  float v[QT_<QT>::E];
  deq<QT>(w, v);
  float* o = out + b * QT_<QT>::E;
#pragma unroll
  for (int i = 0; i < QT_<QT>::E; i++) o[i] = v[i];
}

hipError_t launch_dequant(uint32_t qt, const uint8_t* blocks, size_t nb, float* out, hipStream_t st) {
  dim3 g((unsigned)((nb + 255) / 256)), b(256);
  switch (qt) {
#define DQ(T) case T: hipLaunchKernelGGL(k_dequant<T>, g, b, 0, st, blocks, nb, out); break;
    DQ(Q4_K) DQ(Q5_K) DQ(Q6_K) DQ(Q3_K) DQ(Q2_K) DQ(Q8_0) DQ(Q4_0)
#undef DQ
    case F16: {
      // one "block" here is 32 halfs = 64 bytes
      hipLaunchKernelGGL(k_dequant<F16>, g, b, 0, st, blocks, nb, out);
      break;
    }
    case F32:
      hipLaunchKernelGGL(k_dequant<F32>, g, b, 0, st, blocks, nb, out);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = gm_expf(x[i]);
}

hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Activation quantiser (quant/mod.rs:331-345, :322-326): one thread per 32-block.
// ---------------------------------------------------------------------------------

__device__ __forceinline__ void quant32(const float* v, int8_t* q, float* s, int32_t* s16) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
  float scale = fdiv(amax, 127.0f);
  *s = scale;
  float inv = scale > 0.0f ? fdiv(1.0f, scale) : 0.0f;
  int sum0 = 0, sum1 = 0;
  uint32_t packed[8];
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
  uint4* q4 = reinterpret_cast<uint4*>(q);
  q4[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  q4[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  s16[0] = sum0;
  s16[1] = sum1;
}

__global__ void __launch_bounds__(256) k_quant_act(const float* __restrict__ x, uint32_t nblk,
                                                   int8_t* __restrict__ q, float* __restrict__ s,
                                                   int32_t* __restrict__ s16) {
  uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblk) return;
  float v[32];
  const float4* p = reinterpret_cast<const float4*>(x + (size_t)b * 32);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float4 t = p[i];
    v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
  quant32(v, q + (size_t)b * 32, s + b, s16 + 2 * (size_t)b);
}

hipError_t launch_quant_act(const float* x, uint32_t n_tok, uint32_t K, int8_t* q, float* s,
                            int32_t* s16, hipStream_t st) {
  uint32_t nblk = n_tok * (K / 32);
  hipLaunchKernelGGL(k_quant_act, dim3((nblk + 255) / 256), dim3(256), 0, st, x, nblk, q, s, s16);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Routing. One workgroup per group of tokens; thread (token, expert) pairs compute the
// router logit as the reference's sequential f32 dot (simd/mod.rs:13-16: separate
// multiply and add, left to right, Iterator::sum starting at -0.0).
// ---------------------------------------------------------------------------------

// f32::total_cmp key
__device__ __forceinline__ int total_key(float f) {
  int i = __float_as_int(f);
  return i ^ (int)(((uint32_t)(i >> 31)) >> 1);
}

// rank order: llama = total_cmp descending, stable (llama/mod.rs:943);
// router = partial_cmp descending, unordered/equal -> lower id first (router/mod.rs:83-88).
__device__ __forceinline__ bool ranks_before(bool llama, float a, uint32_t ia, float b, uint32_t ib) {
  if (llama) {
    int ka = total_key(a), kb = total_key(b);
    return ka > kb || (ka == kb && ia < ib);
  }
  if (a > b) return true;
  if (a < b) return false;
  return ia < ib;
}

constexpr int kRouteThreads = 256;

// Sequential softmax pieces over `n` values held in LDS (simd/mod.rs:132-158),
// computed cooperatively: exps in parallel, the running sum by one lane in order.
__global__ void __launch_bounds__(kRouteThreads) k_route(LayerDev L, FwdBufs B, uint32_t n) {
  extern __shared__ float sm[];
  const uint32_t ne = L.ne, k = L.k, d = L.d;
  const uint32_t tpb = ne >= kRouteThreads ? 1u : kRouteThreads / ne;  // tokens per block
  const uint32_t t0 = blockIdx.x * tpb;
  float* lg = sm;                       // [tpb][ne] logits -> probabilities
  float* red = sm + tpb * ne;           // [tpb] scratch (max, inv)
  uint32_t* rk = reinterpret_cast<uint32_t*>(red + tpb);  // [tpb][ne] rank of each expert
  float* topw = reinterpret_cast<float*>(rk + tpb * ne);  // [tpb][k]
  uint32_t* topi = reinterpret_cast<uint32_t*>(topw + tpb * k);

  for (uint32_t p = threadIdx.x; p < tpb * ne; p += blockDim.x) {
    uint32_t tt = p / ne, e = p % ne, t = t0 + tt;
    float acc = 0.0f;
    if (t < n) {
      if (B.logits_in) {
        acc = B.logits_in[(size_t)t * ne + e];
      } else {
        const float4* wr = reinterpret_cast<const float4*>(L.router + (size_t)e * d);
        const float4* hr = reinterpret_cast<const float4*>(B.hs + (size_t)t * d);
        acc = -0.0f;
        for (uint32_t j = 0; j < d / 4; j++) {
          float4 a = wr[j], h = hr[j];
          float p0 = a.x * h.x, p1 = a.y * h.y, p2 = a.z * h.z, p3 = a.w * h.w;
          acc = acc + p0;
          acc = acc + p1;
          acc = acc + p2;
          acc = acc + p3;
        }
      }
      B.logits[(size_t)t * ne + e] = acc;
    }
    lg[p] = acc;
  }
  __syncthreads();

  const bool llama = L.gating == 0;
  const bool soft_all = L.gating == 0 || L.gating == 2 || L.gating == 3;
  if (soft_all) {
    // max (order-free), exps in parallel, sum in order
    if (threadIdx.x < tpb) {
      float mx = -INFINITY;
      for (uint32_t e = 0; e < ne; e++) mx = fmaxf(mx, lg[threadIdx.x * ne + e]);
      red[threadIdx.x] = mx;
    }
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < tpb * ne; p += blockDim.x) {
      float mx = red[p / ne];
      if (isfinite(mx)) lg[p] = gm_expf(lg[p] - mx);
    }
    __syncthreads();
    if (threadIdx.x < tpb) {
      float* x = lg + threadIdx.x * ne;
      float mx = red[threadIdx.x];
      float inv;
      if (!isfinite(mx)) {
        inv = -1.0f;  // uniform
      } else {
        float sum = 0.0f;
        for (uint32_t e = 0; e < ne; e++) sum += x[e];
        inv = (isfinite(sum) && sum > 0.0f) ? fdiv(1.0f, sum) : -1.0f;
      }
      red[threadIdx.x] = inv;
    }
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < tpb * ne; p += blockDim.x) {
      float inv = red[p / ne];
      lg[p] = inv < 0.0f ? fdiv(1.0f, (float)ne) : lg[p] * inv;
    }
    __syncthreads();
  }

  // rank of every expert: how many come before it
  for (uint32_t p = threadIdx.x; p < tpb * ne; p += blockDim.x) {
    uint32_t tt = p / ne, e = p % ne;
    const float* x = lg + tt * ne;
    float me = x[e];
    uint32_t r = 0;
    for (uint32_t o = 0; o < ne; o++)
      if (o != e && ranks_before(llama, x[o], o, me, e)) r++;
    rk[p] = r;
    if (r < k) {
      topw[tt * k + r] = me;
      topi[tt * k + r] = e;
    }
  }
  __syncthreads();

  if (threadIdx.x < tpb && t0 + threadIdx.x < n) {
    uint32_t tt = threadIdx.x, t = t0 + tt;
    float* w = topw + tt * k;
    if (L.gating == 0) {
      // llama/mod.rs:945-949
      float sum = -0.0f;
      for (uint32_t i = 0; i < k; i++) sum += w[i];
      float norm = sum > 0.0f ? fdiv(1.0f, sum) : fdiv(1.0f, (float)k);
      for (uint32_t i = 0; i < k; i++) w[i] *= norm;
    } else if (L.gating == 1) {
      // router/mod.rs:91-97: softmax over the k kept logits
      float mx = -INFINITY;
      for (uint32_t i = 0; i < k; i++) mx = fmaxf(mx, w[i]);
      if (!isfinite(mx)) {
        for (uint32_t i = 0; i < k; i++) w[i] = fdiv(1.0f, (float)k);
      } else {
        float sum = 0.0f;
        for (uint32_t i = 0; i < k; i++) {
          w[i] = gm_expf(w[i] - mx);
          sum += w[i];
        }
        if (isfinite(sum) && sum > 0.0f) {
          float inv = fdiv(1.0f, sum);
          for (uint32_t i = 0; i < k; i++) w[i] *= inv;
        } else {
          for (uint32_t i = 0; i < k; i++) w[i] = fdiv(1.0f, (float)k);
        }
      }
    } else if (L.gating == 3) {
      // router/mod.rs:102-115
      float sum = -0.0f;
      for (uint32_t i = 0; i < k; i++) sum += w[i];
      if (sum > 0.0f) {
        for (uint32_t i = 0; i < k; i++) w[i] = fdiv(w[i], sum);
      } else {
        for (uint32_t i = 0; i < k; i++) w[i] = fdiv(1.0f, (float)k);
      }
    }
    for (uint32_t i = 0; i < k; i++) {
      B.ids[(size_t)t * k + i] = topi[tt * k + i];
      B.w[(size_t)t * k + i] = w[i];
    }
  }
}

hipError_t launch_route(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  uint32_t tpb = L.ne >= kRouteThreads ? 1u : kRouteThreads / L.ne;
  size_t shm = (size_t)tpb * L.ne * 8 + tpb * 4 + (size_t)tpb * L.k * 8;
  hipLaunchKernelGGL(k_route, dim3((n + tpb - 1) / tpb), dim3(kRouteThreads), shm, st, L, B, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Dispatch: a stable counting sort of the (token, rank) pairs by expert id, which is
// exactly members[e] of llama/mod.rs:967-972 laid end to end. One workgroup.
// ---------------------------------------------------------------------------------

__global__ void __launch_bounds__(256) k_dispatch(LayerDev L, FwdBufs B, uint32_t n) {
  extern __shared__ uint32_t cnt[];  // [ne + 1]
  const uint32_t ne = L.ne, k = L.k, nk = n * k;
  for (uint32_t e = threadIdx.x; e < ne; e += blockDim.x) {
    uint32_t c = 0;
    for (uint32_t p = 0; p < nk; p++) c += B.ids[p] == e;
    cnt[e] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t off = 0, na = 0;
    for (uint32_t e = 0; e < ne; e++) {
      uint32_t c = cnt[e];
      cnt[e] = off;
      B.offsets[e] = off;
      if (c) B.active[1 + na++] = e;
      off += c;
    }
    B.offsets[ne] = off;
    B.active[0] = na;
  }
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < ne; e += blockDim.x) {
    uint32_t pos = cnt[e];
    for (uint32_t p = 0; p < nk; p++) {
      if (B.ids[p] == e) {
        B.slot_tok[pos] = p / k;
        B.slot_w[pos] = B.w[p];
        B.slot_rank[pos] = p % k;
        B.slot_of[p] = pos;
        pos++;
      }
    }
  }
}

hipError_t launch_dispatch(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(256), (L.ne + 1) * 4, st, L, B, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Packed (int8-activation) block dots. Each adds its block's sub-block terms to `acc`
// in the reference's order, each term evaluated exactly as the reference writes it.
// x: the block's int8 activations; xs: its per-32 scales; x16: its per-16 sums.
// ---------------------------------------------------------------------------------

template <int QT, int TM>
__device__ __forceinline__ void pk_dot(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                       const int32_t* const* x16, float* acc, int m);

// quant/mod.rs:586-621
template <>
__device__ __forceinline__ void pk_dot<Q4_K, 0>(const uint32_t*, const int8_t* const*, const float* const*,
                                                const int32_t* const*, float*, int) {}

template <int TM>
__device__ __forceinline__ void pk_q4k(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                       const int32_t* const* x16, float* acc, int m) {
  float d = f16f(w[0]), dmin = f16f(w[0] >> 16);
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
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < m) {
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(x[t] + 64 * c);
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          dl = sdot4(lo[i], xa[i], dl);
          dh = sdot4(hi[i], xa[8 + i], dh);
        }
        float s1 = (float)(x16[t][4 * c] + x16[t][4 * c + 1]);
        float s2 = (float)(x16[t][4 * c + 2] + x16[t][4 * c + 3]);
        acc[t] += xs[t][2 * c] * (d * (float)sc1 * (float)dl - dmin * (float)m1 * s1);
        acc[t] += xs[t][2 * c + 1] * (d * (float)sc2 * (float)dh - dmin * (float)m2 * s2);
      }
    }
  }
}

// quant/mod.rs:454-495
template <int TM>
__device__ __forceinline__ void pk_q5k(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                       const int32_t* const* x16, float* acc, int m) {
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
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < m) {
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(x[t] + 64 * g);
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          dl = sdot4(lo[i], xa[i], dl);
          dh = sdot4(hi[i], xa[8 + i], dh);
        }
        float s1 = (float)(x16[t][4 * g] + x16[t][4 * g + 1]);
        float s2 = (float)(x16[t][4 * g + 2] + x16[t][4 * g + 3]);
        acc[t] += xs[t][2 * g] * (d * (float)sc1 * (float)dl - dmin * (float)m1 * s1);
        acc[t] += xs[t][2 * g + 1] * (d * (float)sc2 * (float)dh - dmin * (float)m2 * s2);
      }
    }
  }
}

// quant/mod.rs:417-445. Sub-block s (16 wide): q-32 is dotted as q then -32*sum.
template <int TM>
__device__ __forceinline__ void pk_q6k(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                       const int32_t* const* x16, float* acc, int m) {
  float d = f16f(w[52]);
#pragma unroll
  for (int s = 0; s < 16; s++) {
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
    float sc = (float)(int8_t)byte_of(w, 192 + s);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < m) {
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(x[t] + 16 * s);
        int dt = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) dt = sdot4(q[i], xa[i], dt);
        dt -= 32 * x16[t][s];
        acc[t] += xs[t][s / 2] * d * sc * (float)dt;
      }
    }
  }
}

// quant/mod.rs:503-540. q = ((qs >> shift) & 3) - (hmask bit ? 0 : 4), dotted as
// (low2 | hbit << 2) then -4*sum.
template <int TM>
__device__ __forceinline__ void pk_q3k(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                       const int32_t* const* x16, float* acc, int m) {
  float d_all = f16f(w[27]);
  uint32_t sc4[4];
  q3k_scales(w[24], w[25], w[26], sc4);
#pragma unroll
  for (int s = 0; s < 16; s++) {
    const int half = s / 8, j = (s % 8) / 2, o = 16 * (s % 2);
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t qs = w[(32 + 32 * half + o) / 4 + i];
      uint32_t hm = w[o / 4 + i];
      q[i] = ((qs >> (2 * j)) & 0x03030303u) | (((hm >> (4 * half + j)) & 0x01010101u) << 2);
    }
    float dl = d_all * (float)((int)(int8_t)byte_of(sc4, s) - 32);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < m) {
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(x[t] + 16 * s);
        int dt = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) dt = sdot4(q[i], xa[i], dt);
        dt -= 4 * x16[t][s];
        acc[t] += xs[t][s / 2] * dl * (float)dt;
      }
    }
  }
}

// quant/mod.rs:548-581
template <int TM>
__device__ __forceinline__ void pk_q2k(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                       const int32_t* const* x16, float* acc, int m) {
  float d = f16f(w[20]), dmin = f16f(w[20] >> 16);
#pragma unroll
  for (int s = 0; s < 16; s++) {
    const int half = s / 8, j = (s % 8) / 2, o = 16 * (s % 2);
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = (w[(16 + 32 * half + o) / 4 + i] >> (2 * j)) & 0x03030303u;
    uint32_t sc = byte_of(w, s);
    float dl = d * (float)(sc & 15u), ml = dmin * (float)(sc >> 4);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < m) {
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(x[t] + 16 * s);
        int dt = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) dt = sdot4(q[i], xa[i], dt);
        acc[t] += xs[t][s / 2] * (dl * (float)dt - ml * (float)x16[t][s]);
      }
    }
  }
}

// quant/mod.rs:398-407. The 32 quant bytes start at byte 2 of the block.
template <int TM>
__device__ __forceinline__ void pk_q80(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                       const int32_t*const*, float* acc, int m) {
  float ws = f16f(w[0]);
  uint32_t q[8];
#pragma unroll
  for (int i = 0; i < 8; i++) q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
#pragma unroll
  for (int t = 0; t < TM; t++) {
    if (t < m) {
      const uint32_t* xa = reinterpret_cast<const uint32_t*>(x[t]);
      int dt = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) dt = sdot4(q[i], xa[i], dt);
      acc[t] += ws * xs[t][0] * (float)dt;
    }
  }
}

template <int QT, int TM>
__device__ __forceinline__ void pk_block(const uint32_t* w, const int8_t* const* x, const float* const* xs,
                                         const int32_t* const* x16, float* acc, int m) {
  if constexpr (QT == Q4_K) pk_q4k<TM>(w, x, xs, x16, acc, m);
  else if constexpr (QT == Q5_K) pk_q5k<TM>(w, x, xs, x16, acc, m);
  else if constexpr (QT == Q6_K) pk_q6k<TM>(w, x, xs, x16, acc, m);
  else if constexpr (QT == Q3_K) pk_q3k<TM>(w, x, xs, x16, acc, m);
  else if constexpr (QT == Q2_K) pk_q2k<TM>(w, x, xs, x16, acc, m);
  else if constexpr (QT == Q8_0) pk_q80<TM>(w, x, xs, x16, acc, m);
}

// f32 block dot: acc[t] += sum_i w_i * x[t][i] over the block's dequantised values.
template <int QT, int TM>
__device__ __forceinline__ void f32_block(const uint32_t* w, const float* const* x, float* acc, int m) {
  constexpr int E = QT_<QT>::E;
  float v[E];
  deq<QT>(w, v);
#pragma unroll
  for (int t = 0; t < TM; t++) {
    if (t < m) {
      const float4* xa = reinterpret_cast<const float4*>(x[t]);
      float a = acc[t];
#pragma unroll
      for (int i = 0; i < E / 4; i++) {
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

// ---------------------------------------------------------------------------------
// Gate/up, int8 activations, one lane per row. Each lane runs its row's whole dot in
// K order, so g and u come out bit-identical to quant::matmul's (quant/mod.rs:266-279)
// and so does the int8 h the down product reads. Wave 0 of a workgroup computes the
// gate rows, wave 1 the same up rows; h = silu(g)*u, then h is quantised per 32 rows.
// grid.x = row tiles of 64, grid.y = active-expert slot.
// ---------------------------------------------------------------------------------

constexpr int kGU_TM = 8;  // tokens per pass

template <int QT>
__global__ void __launch_bounds__(128) k_gateup_packed(LayerDev L, FwdBufs B) {
  __shared__ float su[kGU_TM][64];
  __shared__ float sh[kGU_TM][64];
  const uint32_t a = blockIdx.y;
  if (a >= B.active[0]) return;
  const uint32_t e = B.active[1 + a];
  const uint32_t s0 = B.offsets[e], m_all = B.offsets[e + 1] - s0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * 64 + lane;
  const bool valid = row < L.f;
  const uint32_t d = L.d, nblk = d / QT_<QT>::E;
  const uint8_t* W = L.eptr[(wave == 0 ? 0 : 1) * L.ne + e] + (size_t)(valid ? row : 0) *
                     (wave == 0 ? L.pitch_gate : L.pitch_up);

  for (uint32_t c0 = 0; c0 < m_all; c0 += kGU_TM) {
    const int m = (int)min((uint32_t)kGU_TM, m_all - c0);
    const int8_t* xq[kGU_TM];
    const float* xs[kGU_TM];
    const int32_t* x16[kGU_TM];
#pragma unroll
    for (int t = 0; t < kGU_TM; t++) {
      uint32_t tok = B.slot_tok[s0 + c0 + (t < m ? t : 0)];
      xq[t] = B.xq + (size_t)tok * d;
      xs[t] = B.xs + (size_t)tok * (d / 32);
      x16[t] = B.x16 + (size_t)tok * (d / 16);
    }
    float acc[kGU_TM];
#pragma unroll
    for (int t = 0; t < kGU_TM; t++) acc[t] = 0.0f;
    for (uint32_t bi = 0; bi < nblk; bi++) {
      uint32_t w[ndw<QT>()];
      load_block<QT>(W + (size_t)bi * QT_<QT>::B, w);
      const int8_t* xb[kGU_TM];
      const float* sb[kGU_TM];
      const int32_t* hb[kGU_TM];
#pragma unroll
      for (int t = 0; t < kGU_TM; t++) {
        xb[t] = xq[t] + bi * QT_<QT>::E;
        sb[t] = xs[t] + bi * (QT_<QT>::E / 32);
        hb[t] = x16[t] + bi * (QT_<QT>::E / 16);
      }
      pk_block<QT, kGU_TM>(w, xb, sb, hb, acc, m);
    }
    if (wave == 1) {
#pragma unroll
      for (int t = 0; t < kGU_TM; t++) su[t][lane] = acc[t];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int t = 0; t < kGU_TM; t++) sh[t][lane] = swiglu(acc[t], su[t][lane]);
    }
    __syncthreads();
    // h out: f32 copy and/or int8 per 32 rows, slot-indexed
    const uint32_t f = L.f;
    if (B.hf) {
      for (uint32_t p = threadIdx.x; p < (uint32_t)m * 64; p += blockDim.x) {
        uint32_t t = p / 64, r = p % 64, rr = blockIdx.x * 64 + r;
        if (rr < f) B.hf[(size_t)(s0 + c0 + t) * f + rr] = sh[t][r];
      }
    }
    if (B.hq) {
      for (uint32_t p = threadIdx.x; p < (uint32_t)m * 2; p += blockDim.x) {
        uint32_t t = p / 2, hb = p % 2, r0 = blockIdx.x * 64 + 32 * hb;
        if (r0 + 32 <= f) {
          size_t slot = s0 + c0 + t;
          quant32(&sh[t][32 * hb], B.hq + slot * f + r0, B.hsc + slot * (f / 32) + r0 / 32,
                  B.h16 + slot * (f / 16) + r0 / 16);
        }
      }
    }
    __syncthreads();
  }
}

// Gate/up with f32 activations (Weight::Full, and Q4_0/F16/F32 under Weight::Packed).
// Split K: LPR lanes per row, 64/LPR rows per wave, 4 waves = 32 rows per workgroup.
constexpr int kF_LPR = 8, kF_TM = 4;

template <int QT>
__global__ void __launch_bounds__(256) k_gateup_f32(LayerDev L, FwdBufs B) {
  __shared__ float sg[kF_TM][32];
  __shared__ float su[kF_TM][32];
  __shared__ float sh[kF_TM][32];
  const uint32_t a = blockIdx.y;
  if (a >= B.active[0]) return;
  const uint32_t e = B.active[1 + a];
  const uint32_t s0 = B.offsets[e], m_all = B.offsets[e + 1] - s0;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t g = lane % kF_LPR, rl = wave * (64 / kF_LPR) + lane / kF_LPR;  // 0..31
  const uint32_t row = blockIdx.x * 32 + rl;
  const bool valid = row < L.f;
  const uint32_t d = L.d, nblk = d / QT_<QT>::E;
  const uint8_t* Wg = L.eptr[0 * L.ne + e] + (size_t)(valid ? row : 0) * L.pitch_gate;
  const uint8_t* Wu = L.eptr[1 * L.ne + e] + (size_t)(valid ? row : 0) * L.pitch_up;
  const uint32_t f = L.f;
  for (uint32_t c0 = 0; c0 < m_all; c0 += kF_TM) {
    const int m = (int)min((uint32_t)kF_TM, m_all - c0);
    const float* xr[kF_TM];
#pragma unroll
    for (int t = 0; t < kF_TM; t++) xr[t] = B.hs + (size_t)B.slot_tok[s0 + c0 + (t < m ? t : 0)] * d;
    float ag[kF_TM], au[kF_TM];
#pragma unroll
    for (int t = 0; t < kF_TM; t++) ag[t] = au[t] = 0.0f;
    if (valid) {
      for (uint32_t bi = g; bi < nblk; bi += kF_LPR) {
        uint32_t w[ndw<QT>()];
        const float* xb[kF_TM];
#pragma unroll
        for (int t = 0; t < kF_TM; t++) xb[t] = xr[t] + bi * QT_<QT>::E;
        load_block<QT>(Wg + (size_t)bi * QT_<QT>::B, w);
        f32_block<QT, kF_TM>(w, xb, ag, m);
        load_block<QT>(Wu + (size_t)bi * QT_<QT>::B, w);
        f32_block<QT, kF_TM>(w, xb, au, m);
      }
    }
#pragma unroll
    for (int t = 0; t < kF_TM; t++) {
#pragma unroll
      for (int o = kF_LPR / 2; o > 0; o >>= 1) {
        ag[t] += __shfl_xor(ag[t], o, 64);
        au[t] += __shfl_xor(au[t], o, 64);
      }
    }
    if (g == 0) {
#pragma unroll
      for (int t = 0; t < kF_TM; t++) sh[t][rl] = swiglu(ag[t], au[t]);
    }
    __syncthreads();
    if (B.hf) {
      for (uint32_t p = threadIdx.x; p < (uint32_t)m * 32; p += blockDim.x) {
        uint32_t t = p / 32, r = p % 32, rr = blockIdx.x * 32 + r;
        if (rr < f) B.hf[(size_t)(s0 + c0 + t) * f + rr] = sh[t][r];
      }
    }
    if (B.hq) {
      for (uint32_t t = threadIdx.x; t < (uint32_t)m; t += blockDim.x) {
        uint32_t r0 = blockIdx.x * 32;
        if (r0 + 32 <= f) {
          size_t slot = s0 + c0 + t;
          quant32(&sh[t][0], B.hq + slot * f + r0, B.hsc + slot * (f / 32) + r0 / 32,
                  B.h16 + slot * (f / 16) + r0 / 16);
        }
      }
    }
    __syncthreads();
  }
  (void)sg;
  (void)su;
}

// ---------------------------------------------------------------------------------
// Down product: y[slot] = W_down[e] * h[slot]. Split K over LPR lanes per row, the
// partial sums of a row reduced across its lanes. grid.x = tiles of 32 rows.
// ---------------------------------------------------------------------------------

constexpr int kD_LPR = 8, kD_TM = 4;

template <int QT, bool PACKED>
__global__ void __launch_bounds__(256) k_down(LayerDev L, FwdBufs B) {
  const uint32_t a = blockIdx.y;
  if (a >= B.active[0]) return;
  const uint32_t e = B.active[1 + a];
  const uint32_t s0 = B.offsets[e], m_all = B.offsets[e + 1] - s0;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t g = lane % kD_LPR;
  const uint32_t row = blockIdx.x * 32 + wave * (64 / kD_LPR) + lane / kD_LPR;
  const bool valid = row < L.d;
  const uint32_t f = L.f, nblk = f / QT_<QT>::E;
  const uint8_t* W = L.eptr[2 * L.ne + e] + (size_t)(valid ? row : 0) * L.pitch_down;
  for (uint32_t c0 = 0; c0 < m_all; c0 += kD_TM) {
    const int m = (int)min((uint32_t)kD_TM, m_all - c0);
    float acc[kD_TM];
#pragma unroll
    for (int t = 0; t < kD_TM; t++) acc[t] = 0.0f;
    if (valid) {
      for (uint32_t bi = g; bi < nblk; bi += kD_LPR) {
        uint32_t w[ndw<QT>()];
        load_block<QT>(W + (size_t)bi * QT_<QT>::B, w);
        if constexpr (PACKED) {
          const int8_t* xb[kD_TM];
          const float* sb[kD_TM];
          const int32_t* hb[kD_TM];
#pragma unroll
          for (int t = 0; t < kD_TM; t++) {
            size_t slot = s0 + c0 + (t < m ? t : 0);
            xb[t] = B.hq + slot * f + bi * QT_<QT>::E;
            sb[t] = B.hsc + slot * (f / 32) + bi * (QT_<QT>::E / 32);
            hb[t] = B.h16 + slot * (f / 16) + bi * (QT_<QT>::E / 16);
          }
          pk_block<QT, kD_TM>(w, xb, sb, hb, acc, m);
        } else {
          const float* xb[kD_TM];
#pragma unroll
          for (int t = 0; t < kD_TM; t++) {
            size_t slot = s0 + c0 + (t < m ? t : 0);
            xb[t] = B.hf + slot * f + bi * QT_<QT>::E;
          }
          f32_block<QT, kD_TM>(w, xb, acc, m);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kD_TM; t++) {
#pragma unroll
      for (int o = kD_LPR / 2; o > 0; o >>= 1) acc[t] += __shfl_xor(acc[t], o, 64);
    }
    if (valid && g == 0) {
#pragma unroll
      for (int t = 0; t < kD_TM; t++)
        if (t < m) B.y[(size_t)(s0 + c0 + t) * L.d + row] = acc[t];
    }
  }
}

// ---------------------------------------------------------------------------------
// Combine: out[t] = sum over the token's experts of y*w, ascending expert id
// (llama/mod.rs:977-995) or routed rank (moe/mod.rs:104-109); add_scaled multiplies
// then adds, starting from the zeroed output.
// ---------------------------------------------------------------------------------

__global__ void __launch_bounds__(256) k_combine(LayerDev L, FwdBufs B, uint32_t n) {
  const uint32_t t = blockIdx.y, k = L.k, d = L.d;
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n || c >= d) return;
  uint32_t order[32];  // top_k <= 32, checked at registration
  for (uint32_t i = 0; i < k; i++) order[i] = i;
  if (L.combine == 0) {
    for (uint32_t i = 1; i < k; i++) {  // insertion sort of ranks by expert id
      uint32_t v = order[i], id = B.ids[(size_t)t * k + v];
      int j = (int)i - 1;
      while (j >= 0 && B.ids[(size_t)t * k + order[j]] > id) {
        order[j + 1] = order[j];
        j--;
      }
      order[j + 1] = v;
    }
  }
  float acc = 0.0f;
  for (uint32_t i = 0; i < k; i++) {
    uint32_t r = order[i];
    uint32_t slot = B.slot_of[(size_t)t * k + r];
    float wv = B.w[(size_t)t * k + r];
    acc = acc + B.y[(size_t)slot * d + c] * wv;
  }
  B.out[(size_t)t * d + c] = acc;
}

hipError_t launch_combine(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_combine, dim3((L.d + 255) / 256, n), dim3(256), 0, st, L, B, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Launch selection
// ---------------------------------------------------------------------------------

static inline bool packed_kernel(uint32_t math, uint32_t qt) {
  return math == 0 && has_int8_kernel(qt);
}

hipError_t launch_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  uint32_t ymax = min(L.ne, n * L.k);
  if (packed_kernel(L.math, L.qt_gate)) {
    dim3 g((L.f + 63) / 64, ymax), b(128);
    switch (L.qt_gate) {
#define GU(T) case T: hipLaunchKernelGGL(k_gateup_packed<T>, g, b, 0, st, L, B); break;
      GU(Q4_K) GU(Q5_K) GU(Q6_K) GU(Q3_K) GU(Q2_K) GU(Q8_0)
#undef GU
      default: return hipErrorInvalidValue;
    }
  } else {
    dim3 g((L.f + 31) / 32, ymax), b(256);
    switch (L.qt_gate) {
#define GU(T) case T: hipLaunchKernelGGL(k_gateup_f32<T>, g, b, 0, st, L, B); break;
      GU(Q4_K) GU(Q5_K) GU(Q6_K) GU(Q3_K) GU(Q2_K) GU(Q8_0) GU(Q4_0) GU(F16) GU(F32)
#undef GU
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

hipError_t launch_down(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  uint32_t ymax = min(L.ne, n * L.k);
  dim3 g((L.d + 31) / 32, ymax), b(256);
  if (packed_kernel(L.math, L.qt_down)) {
    switch (L.qt_down) {
#define DN(T) case T: hipLaunchKernelGGL((k_down<T, true>), g, b, 0, st, L, B); break;
      DN(Q4_K) DN(Q5_K) DN(Q6_K) DN(Q3_K) DN(Q2_K) DN(Q8_0)
#undef DN
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (L.qt_down) {
#define DN(T) case T: hipLaunchKernelGGL((k_down<T, false>), g, b, 0, st, L, B); break;
      DN(Q4_K) DN(Q5_K) DN(Q6_K) DN(Q3_K) DN(Q2_K) DN(Q8_0) DN(Q4_0) DN(F16) DN(F32)
#undef DN
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

// gmoe_matmul: one "expert" whose matrix is `w`, all n vectors routed to it; reuse the
// down kernel (split K) with an identity dispatch built on the host.
hipError_t launch_matmul(uint32_t qt, uint32_t math, const uint8_t* w, size_t pitch, uint32_t rows,
                         uint32_t cols, const float* x, const int8_t* xq, const float* xs,
                         const int32_t* x16, uint32_t n, float* out, hipStream_t st) {
  (void)qt; (void)math; (void)w; (void)pitch; (void)rows; (void)cols; (void)x; (void)xq;
  (void)xs; (void)x16; (void)n; (void)out; (void)st;
  return hipErrorNotSupported;
}

}  // namespace gmoe
