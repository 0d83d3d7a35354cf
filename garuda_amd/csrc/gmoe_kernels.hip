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

#include <type_traits>
#include <utility>

namespace gmoe {

static inline bool row_kernel_type(uint32_t qt) { return qt == Q4_K || qt == Q5_K || qt == F16 || qt == F32; }

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

// Gating of `tpb` tokens whose router logits sit in lg[tpb][ne] (LDS), for tokens
// t0.. t0+tpb-1 (those >= n are ignored). Softmax (simd/mod.rs:132-158) is computed
// cooperatively: max in any order (it is exact), exps in parallel, the running sum by
// one lane in order. Ranks by counting (a stable sort's positions). Every thread of the
// block must call this.
__device__ void gate_block(const LayerDev& L, const FwdBufs& B, float* lg, float* red, float* topw,
                           uint32_t* topi, uint32_t tpb, uint32_t t0, uint32_t n) {
  const uint32_t ne = L.ne, k = L.k;
  const bool llama = L.gating == 0;
  const bool soft_all = L.gating == 0 || L.gating == 2 || L.gating == 3;
  if (soft_all) {
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

// Router logits: one lane per (token, expert) pair runs the reference's sequential f32
// dot (simd/mod.rs:13-16: separate multiply and add, left to right, Iterator::sum
// starting at -0.0), then gate_block. Used when the fused decode kernel does not apply.
__global__ void __launch_bounds__(kRouteThreads) k_route(LayerDev L, FwdBufs B, uint32_t n) {
  extern __shared__ float sm[];
  const uint32_t ne = L.ne, k = L.k, d = L.d;
  const uint32_t tpb = ne >= kRouteThreads ? 1u : kRouteThreads / ne;  // tokens per block
  const uint32_t t0 = blockIdx.x * tpb;
  float* lg = sm;                       // [tpb][ne] logits -> probabilities
  float* red = sm + tpb * ne;           // [tpb] scratch (max, inv)
  float* topw = red + tpb;              // [tpb][k]
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
  gate_block(L, B, lg, red, topw, topi, tpb, t0, n);
}

// Dispatch body: a stable counting sort of the (token, rank) pairs by expert id, which is
// exactly members[e] of llama/mod.rs:967-972 laid end to end. One workgroup; cnt is
// [ne] in LDS; every thread must call this.
__device__ void dispatch_block(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t* cnt,
                               const uint32_t* ids, const float* wts) {
  const uint32_t ne = L.ne, k = L.k, nk = n * k;
  for (uint32_t e = threadIdx.x; e < ne; e += blockDim.x) {
    uint32_t c = 0;
    for (uint32_t p = 0; p < nk; p++) c += ids[p] == e;
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
      if (ids[p] == e) {
        B.slot_tok[pos] = p / k;
        B.slot_w[pos] = wts[p];
        B.slot_rank[pos] = p % k;
        B.slot_of[p] = pos;
        pos++;
      }
    }
  }
}

__global__ void __launch_bounds__(256) k_dispatch(LayerDev L, FwdBufs B, uint32_t n) {
  extern __shared__ uint32_t cnt[];  // [ne]
  dispatch_block(L, B, n, cnt, B.ids, B.w);
}

// ---------------------------------------------------------------------------------
// Fused decode front end: router logits, gating, the int8 activation quantiser and the
// dispatch in one workgroup of 512 threads, for n*ne <= 64 (one chain per lane of
// wave 0). The logits' products w*h (each rounded, as the reference multiplies before
// it adds) are made by waves 1..15 one K-chunk ahead into LDS; wave 0 only runs the 64
// sequential add chains over them, so the chain's latency is the adds alone.
// (The products are made by waves 1..7.)
// ---------------------------------------------------------------------------------

constexpr int kFrontKC = 128, kFrontPairs = 64, kFrontRows = 16, kFrontRing = 16, kFrontMaxCh = 32;
constexpr int kFrontProd = 512, kFrontThreads = 64 + kFrontProd;
constexpr int kFrontRow = kFrontKC + 4;  // padded LDS row (floats)

// Producer p owns one float4 column slot (row p / 32, float4 p % 32) of every K chunk of
// the (router rows ; token rows) operand matrix and loads it 16 chunks ahead into a
// register ring; each chunk is parked in LDS two chunks before its products are made.
// The chunk loop is fully unrolled so ring indices are compile-time.
__global__ void __launch_bounds__(kFrontThreads) k_front_small(LayerDev L, FwdBufs B, uint32_t n, int quant) {
  extern __shared__ float fs[];
  float* stage = fs;                                    // [2][kFrontRows][kFrontRow]
  float* prod = stage + 2 * kFrontRows * kFrontRow;     // [2][kFrontPairs][kFrontRow]
  float* lg = prod + 2 * kFrontPairs * kFrontRow;       // [n][ne]
  float* red = lg + kFrontPairs;                        // [n]
  float* topw = red + kFrontPairs;                      // [n][k]
  uint32_t* topi = reinterpret_cast<uint32_t*>(topw + kFrontPairs * 32);
  uint32_t* cnt = topi + kFrontPairs * 32;              // [ne]
  const uint32_t ne = L.ne, d = L.d, P = n * ne, R = ne + n;
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  if (B.logits_in) {
    for (uint32_t p = tid; p < P; p += blockDim.x) lg[p] = B.logits_in[p];
  } else {
    const uint32_t nch = d / kFrontKC;
    const bool producer = wave != 0;
    const uint32_t p = tid - 64, r = p / 32, c4 = p % 32;
    const bool slot = producer && r < R;
    const float4* src = reinterpret_cast<const float4*>(slot ? (r < ne ? L.router + (size_t)r * d
                                                                      : B.hs + (size_t)(r - ne) * d)
                                                             : L.router);
    // the ring is one 64-wide vector value: constant-index element accesses stay in VGPRs
    typedef float f32x64 __attribute__((ext_vector_type(64)));
    f32x64 ring = {};
    auto ring_put = [&](int i, float4 v) __attribute__((always_inline)) {
      ring[4 * i] = v.x; ring[4 * i + 1] = v.y; ring[4 * i + 2] = v.z; ring[4 * i + 3] = v.w;
    };
    auto ring_get = [&](int i) __attribute__((always_inline)) {
      return make_float4(ring[4 * i], ring[4 * i + 1], ring[4 * i + 2], ring[4 * i + 3]);
    };
#pragma unroll
    for (int c = 0; c < kFrontRing; c++)
      if (slot && (uint32_t)c < nch) ring_put(c, src[c * (kFrontKC / 4) + c4]);
    float acc = -0.0f;
    // prologue: park chunks 0 and 1, make chunk 0's products
#pragma unroll
    for (int c = 0; c < 2; c++) {
      if (slot && (uint32_t)c < nch) {
        *reinterpret_cast<float4*>(stage + (c * kFrontRows + r) * kFrontRow + 4 * c4) = ring_get(c);
        if ((uint32_t)(c + kFrontRing) < nch) ring_put(c, src[(c + kFrontRing) * (kFrontKC / 4) + c4]);
      }
    }
    __syncthreads();
    if (producer) {
#pragma unroll
      for (int q = 0; q < kFrontPairs * kFrontKC / 4 / kFrontProd; q++) {
        uint32_t g = p + kFrontProd * q, pr = g / (kFrontKC / 4), j = 4 * (g % (kFrontKC / 4));
        if (pr < P) {
          uint32_t t = pr / ne, e = pr % ne;
          float4 av = *reinterpret_cast<const float4*>(stage + e * kFrontRow + j);
          float4 hv = *reinterpret_cast<const float4*>(stage + (ne + t) * kFrontRow + j);
          *reinterpret_cast<float4*>(prod + pr * kFrontRow + j) =
              make_float4(av.x * hv.x, av.y * hv.y, av.z * hv.z, av.w * hv.w);
        }
      }
    }
    __syncthreads();
    // iteration c: wave 0 chains chunk c | producers make chunk c+1's products and park
    // chunk c+2 (whose LDS slot chunk c's products have finished with)
#pragma unroll
    for (int c = 0; c < kFrontMaxCh; c++) {
      if ((uint32_t)c < nch) {
        if (wave == 0) {
          if (lane < P) {
            const float* src2 = prod + (c & 1) * kFrontPairs * kFrontRow + lane * kFrontRow;
#pragma unroll
            for (int j0 = 0; j0 < kFrontKC; j0 += 32) {
              float4 v[8];
#pragma unroll
              for (int u = 0; u < 8; u++) v[u] = *reinterpret_cast<const float4*>(src2 + j0 + 4 * u);
#pragma unroll
              for (int u = 0; u < 8; u++) {
                acc = acc + v[u].x;
                acc = acc + v[u].y;
                acc = acc + v[u].z;
                acc = acc + v[u].w;
              }
            }
          }
        } else {
          if ((uint32_t)(c + 1) < nch) {
            const float* st = stage + ((c + 1) & 1) * kFrontRows * kFrontRow;
            float* dst = prod + ((c + 1) & 1) * kFrontPairs * kFrontRow;
#pragma unroll
            for (int q = 0; q < kFrontPairs * kFrontKC / 4 / kFrontProd; q++) {
              uint32_t g = p + kFrontProd * q, pr = g / (kFrontKC / 4), j = 4 * (g % (kFrontKC / 4));
              if (pr < P) {
                uint32_t t = pr / ne, e = pr % ne;
                float4 av = *reinterpret_cast<const float4*>(st + e * kFrontRow + j);
                float4 hv = *reinterpret_cast<const float4*>(st + (ne + t) * kFrontRow + j);
                *reinterpret_cast<float4*>(dst + pr * kFrontRow + j) =
                    make_float4(av.x * hv.x, av.y * hv.y, av.z * hv.z, av.w * hv.w);
              }
            }
          }
          if (slot && (uint32_t)(c + 2) < nch) {
            const int slot_i = (c + 2) % kFrontRing;
            *reinterpret_cast<float4*>(stage + ((c & 1) * kFrontRows + r) * kFrontRow + 4 * c4) = ring_get(slot_i);
            if ((uint32_t)(c + 2 + kFrontRing) < nch) ring_put(slot_i, src[(c + 2 + kFrontRing) * (kFrontKC / 4) + c4]);
          }
        }
        __syncthreads();
      }
    }
    if (wave == 0 && lane < P) lg[lane] = acc;
  }
  __syncthreads();
  for (uint32_t p = tid; p < P; p += blockDim.x) B.logits[p] = lg[p];
  gate_block(L, B, lg, red, topw, topi, n, 0, n);
  if (quant) {
    const uint32_t nblk = n * (d / 32);
    for (uint32_t b = tid; b < nblk; b += blockDim.x) {
      float v[32];
      const float4* src = reinterpret_cast<const float4*>(B.hs + (size_t)b * 32);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        float4 t4 = src[i];
        v[4 * i] = t4.x; v[4 * i + 1] = t4.y; v[4 * i + 2] = t4.z; v[4 * i + 3] = t4.w;
      }
      quant32(v, B.xq + (size_t)b * 32, B.xs + b, B.x16 + 2 * (size_t)b);
    }
  }
  __syncthreads();
  // gate_block leaves every token's ranked ids and weights in topi/topw ([n][k], LDS)
  dispatch_block(L, B, n, cnt, topi, topw);
}

bool front_small_ok(const LayerDev& L, uint32_t n) {
  return n * L.ne <= (uint32_t)kFrontPairs && L.ne + n <= (uint32_t)kFrontRows && L.k <= 32 &&
         L.d % kFrontKC == 0 && L.d <= (uint32_t)(kFrontKC * kFrontMaxCh);
}

hipError_t launch_front_small(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, hipStream_t st) {
  size_t shm = (size_t)(2 * kFrontRows * kFrontRow + 2 * kFrontPairs * kFrontRow + 2 * kFrontPairs +
                        2 * kFrontPairs * 32) * 4 + L.ne * 4;
  static bool attr = (hipFuncSetAttribute((const void*)k_front_small, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          160 * 1024 - 2048), true);
  (void)attr;
  hipLaunchKernelGGL(k_front_small, dim3(1), dim3(kFrontThreads), shm, st, L, B, n, quant);
  return hipGetLastError();
}

hipError_t launch_route(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  uint32_t tpb = L.ne >= kRouteThreads ? 1u : kRouteThreads / L.ne;
  size_t shm = (size_t)tpb * L.ne * 4 + tpb * 4 + (size_t)tpb * L.k * 8;
  hipLaunchKernelGGL(k_route, dim3((n + tpb - 1) / tpb), dim3(kRouteThreads), shm, st, L, B, n);
  return hipGetLastError();
}

hipError_t launch_dispatch(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(256), L.ne * 4, st, L, B, n);
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
#pragma unroll
  for (int g = 0; g < E / 32; g++) {
    float v[32];
    deq32<QT>(w, g, v);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if (t < m) {
        const float4* xa = reinterpret_cast<const float4*>(x[t] + 32 * g);
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
// Row-per-lane streaming kernels, for block types made of whole 16-byte pieces
// (Q4_K 144 B, Q5_K 176 B; F16/F32 rows walked 32 values = 64/128 B at a time).
//
// A workgroup owns 64 consecutive rows of one expert's matrix and lane i owns row i.
// A wave streams its rows one block-column ("step") at a time: the 64 blocks of a step
// are fetched with coalesced 16-byte loads (consecutive lanes read consecutive bytes of
// a row, 9 lanes per Q4_K block), parked in LDS, and each lane reads its own row's block
// back. Two steps are in flight while one is computed. The activations of a step are
// the same for every lane of the wave, so they arrive through scalar loads. Each lane
// runs its row's dot in K order.
// ---------------------------------------------------------------------------------

struct RowIO {
  const uint8_t* const* eptr;
  const uint32_t* active;
  const uint32_t* offsets;
  const uint32_t* slot_tok;
};

// One wave's streaming loop over blocks [j0, j1) of rows `W + row*pitch`, calling
// body(j, w) with the lane's own block j in w[]. T is the wave's LDS step buffer.
//
// D register sets form a ring: step j is parked from set j % D, whose loads are then
// reissued for step j + D, so D - 1 steps stay in flight while one is computed. Every
// fetch is unconditional (its block index is clamped to the last block, a re-read that
// the L2 serves) and the loop always runs whole rounds of D steps, with only the body
// of the steps past j1 skipped; the load count pending at each park is then the same on
// every path through the loop, and the compiler waits for exactly the set it parks
// instead of draining every load in flight.
template <int QT, int D = 3, class Body>
__device__ __forceinline__ void stream_rows(const uint8_t* __restrict__ W, uint32_t pitch, uint32_t r0,
                                            uint32_t nrows, uint32_t j0, uint32_t j1, uint4* T, uint32_t lane,
                                            Body body) {
  constexpr int B = QT_<QT>::B, P = B / 16, NW = B / 4;
  if (j0 >= j1) return;
  const uint8_t* src[P];
#pragma unroll
  for (int q = 0; q < P; q++) {
    uint32_t c = q * 64 + lane, row = c / P, piece = c % P;
    uint32_t rr = min(r0 + row, nrows - 1);
    src[q] = W + (size_t)rr * pitch + piece * 16;
  }
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4 g[D][P];
  const uint32_t jlast = j1 - 1;
  auto fetch = [&](u32x4* gg, uint32_t j) {
    const size_t off = (size_t)min(j, jlast) * B;
#pragma unroll
    for (int q = 0; q < P; q++) gg[q] = *reinterpret_cast<const u32x4*>(src[q] + off);
  };
  // Lanes of one wave hand blocks to each other through T. The LDS performs one wave's
  // DS instructions in issue order, so the hand-off only needs the compiler to keep the
  // stores before the other lanes' loads and the loads before the next step's stores:
  // an empty asm with a memory clobber. (A memory-model fence would also wait for
  // every global load in flight, draining the prefetch.)
  auto wave_sync = [] {
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  };
#pragma unroll
  for (int i = 0; i < D; i++) fetch(g[i], j0 + i);
  for (uint32_t j = j0; j < j1; j += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
#pragma unroll
      for (int q = 0; q < P; q++) T[q * 64 + lane] = make_uint4(g[i][q].x, g[i][q].y, g[i][q].z, g[i][q].w);
      fetch(g[i], j + i + D);
      wave_sync();
      uint32_t w[NW];
#pragma unroll
      for (int p = 0; p < P; p++) {
        uint4 v = T[lane * P + p];
        w[4 * p] = v.x; w[4 * p + 1] = v.y; w[4 * p + 2] = v.z; w[4 * p + 3] = v.w;
      }
      wave_sync();
      if (j + i < j1) body(j + i, w);
    }
  }
}

// Activations of one token chunk over the K blocks [j0, j0+span) a workgroup reads,
// staged in LDS once and read by every lane as broadcasts. Packed: int8 values, per-32
// scales and per-16 sums; f32: the values. `row[t]` is the token (gate/up) or slot
// (down) row of chunk member t in the activation arrays, whose rows are K long.
template <bool PACKED>
struct ActLds {
  static constexpr uint32_t bytes_per_elem_x16() { return PACKED ? 22u : 64u; }  // x16: 1 + 1/8 + 1/4 (q, s, s16) or 4
  // LDS bytes for tm tokens over span*E elements (each array rounded to 16 bytes)
  __host__ __device__ static uint32_t bytes(uint32_t tm, uint32_t nelem) {
    if (PACKED) return tm * (((nelem + 15) & ~15u) + ((nelem / 32 * 4 + 15) & ~15u) + ((nelem / 16 * 4 + 15) & ~15u));
    return tm * nelem * 4;
  }
};

template <int TM>
__device__ __forceinline__ void stage_packed(uint8_t* lds, uint32_t nelem, const int8_t* __restrict__ q,
                                             const float* __restrict__ s, const int32_t* __restrict__ s16,
                                             uint32_t K, const uint32_t* row, int m, uint32_t k0) {
  const uint32_t qb = (nelem + 15) & ~15u, sb = (nelem / 32 * 4 + 15) & ~15u, hb = (nelem / 16 * 4 + 15) & ~15u;
  int8_t* lq = reinterpret_cast<int8_t*>(lds);
  float* ls = reinterpret_cast<float*>(lds + TM * qb);
  int32_t* lh = reinterpret_cast<int32_t*>(lds + TM * qb + TM * sb);
  const uint32_t nq4 = nelem / 16;  // int8 values move 16 at a time (nelem is a multiple of 32)
  for (uint32_t i = threadIdx.x; i < (uint32_t)m * nq4; i += blockDim.x) {
    uint32_t t = i / nq4, c = i % nq4;
    reinterpret_cast<uint4*>(lq + t * qb)[c] = reinterpret_cast<const uint4*>(q + (size_t)row[t] * K + k0)[c];
  }
  const uint32_t ns = nelem / 32, nh = nelem / 16;
  for (uint32_t i = threadIdx.x; i < (uint32_t)m * ns; i += blockDim.x) {
    uint32_t t = i / ns, c = i % ns;
    ls[t * (sb / 4) + c] = s[(size_t)row[t] * (K / 32) + k0 / 32 + c];
  }
  for (uint32_t i = threadIdx.x; i < (uint32_t)m * nh; i += blockDim.x) {
    uint32_t t = i / nh, c = i % nh;
    lh[t * (hb / 4) + c] = s16[(size_t)row[t] * (K / 16) + k0 / 16 + c];
  }
}

template <int TM>
__device__ __forceinline__ void stage_f32(uint8_t* lds, uint32_t nelem, const float* __restrict__ x, uint32_t K,
                                          const uint32_t* row, int m, uint32_t k0) {
  float* lx = reinterpret_cast<float*>(lds);
  const uint32_t n4 = nelem / 4;
  for (uint32_t i = threadIdx.x; i < (uint32_t)m * n4; i += blockDim.x) {
    uint32_t t = i / n4, c = i % n4;
    reinterpret_cast<float4*>(lx + t * nelem)[c] = reinterpret_cast<const float4*>(x + (size_t)row[t] * K + k0)[c];
  }
}

// Runs the block body over the staged activations: block j (absolute) of chunk member t
// sits at element (j - jbase) * E of its staged row.
template <int QT, int TM, bool PACKED>
__device__ __forceinline__ void staged_block(const uint32_t* w, uint8_t* lds, uint32_t nelem, uint32_t j,
                                             uint32_t jbase, float* acc, int m) {
  constexpr int E = QT_<QT>::E;
  const uint32_t off = (j - jbase) * E;
  if constexpr (PACKED) {
    const uint32_t qb = (nelem + 15) & ~15u, sb = (nelem / 32 * 4 + 15) & ~15u, hb = (nelem / 16 * 4 + 15) & ~15u;
    const int8_t* lq = reinterpret_cast<const int8_t*>(lds);
    const float* ls = reinterpret_cast<const float*>(lds + TM * qb);
    const int32_t* lh = reinterpret_cast<const int32_t*>(lds + TM * qb + TM * sb);
    const int8_t* xb[TM];
    const float* sbp[TM];
    const int32_t* hbp[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) {
      xb[t] = lq + t * qb + off;
      sbp[t] = ls + t * (sb / 4) + off / 32;
      hbp[t] = lh + t * (hb / 4) + off / 16;
    }
    pk_block<QT, TM>(w, xb, sbp, hbp, acc, m);
  } else {
    const float* lx = reinterpret_cast<const float*>(lds);
    const float* xb[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) xb[t] = lx + t * nelem + off;
    f32_block<QT, TM>(w, xb, acc, m);
  }
}

// Dynamic LDS of the row kernels: [KS step tiles][misc floats][staged activations].
__host__ __device__ inline uint32_t row_tile_bytes(uint32_t qt_bytes, uint32_t ks) { return ks * 64 * qt_bytes; }

template <int QT, int TM, bool PACKED>
__global__ void __launch_bounds__(128)
k_gu_rows(RowIO io, uint32_t ne, uint32_t f, uint32_t d, uint32_t pitch_g, uint32_t pitch_u,
          const int8_t* __restrict__ xq, const float* __restrict__ xs, const int32_t* __restrict__ x16,
          const float* __restrict__ hs, int8_t* __restrict__ hq, float* __restrict__ hsc,
          int32_t* __restrict__ h16, float* __restrict__ hf) {
  constexpr int E = QT_<QT>::E, P = QT_<QT>::B / 16;
  extern __shared__ uint4 dsm[];
  uint4* tile0 = dsm;                                              // [2][64*P]
  float* su = reinterpret_cast<float*>(dsm + 2 * 64 * P);         // [TM][64]
  float* sh = su + TM * 64;                                        // [TM][64]
  uint8_t* acts = reinterpret_cast<uint8_t*>(sh + TM * 64);
  const uint32_t a = blockIdx.y;
  if (a >= io.active[0]) return;
  const uint32_t e = io.active[1 + a];
  const uint32_t s0 = io.offsets[e], m_all = io.offsets[e + 1] - s0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t r0 = blockIdx.x * 64;
  const uint8_t* W = io.eptr[wave * ne + e];
  const uint32_t pitch = wave ? pitch_u : pitch_g;
  const uint32_t nblk = d / E;
  for (uint32_t c0 = 0; c0 < m_all; c0 += TM) {
    const int m = (int)min((uint32_t)TM, m_all - c0);
    uint32_t tok[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) tok[t] = io.slot_tok[s0 + c0 + (t < m ? t : 0)];
    if constexpr (PACKED) stage_packed<TM>(acts, d, xq, xs, x16, d, tok, m, 0);
    else stage_f32<TM>(acts, d, hs, d, tok, m, 0);
    __syncthreads();
    float acc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc[t] = 0.0f;
    stream_rows<QT>(W, pitch, r0, f, 0, nblk, tile0 + wave * 64 * P, lane, [&](uint32_t j, const uint32_t* w) {
      staged_block<QT, TM, PACKED>(w, acts, d, j, 0, acc, m);
    });
    if (wave == 1) {
#pragma unroll
      for (int t = 0; t < TM; t++) su[t * 64 + lane] = acc[t];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int t = 0; t < TM; t++) sh[t * 64 + lane] = swiglu(acc[t], su[t * 64 + lane]);
    }
    __syncthreads();
    if (hf) {
      for (uint32_t p = threadIdx.x; p < (uint32_t)m * 64; p += blockDim.x) {
        uint32_t t = p / 64, r = p % 64, rr = r0 + r;
        if (rr < f) hf[(size_t)(s0 + c0 + t) * f + rr] = sh[t * 64 + r];
      }
    }
    if (hq) {
      for (uint32_t p = threadIdx.x; p < (uint32_t)m * 2; p += blockDim.x) {
        uint32_t t = p / 2, hb = p % 2, q0 = r0 + 32 * hb;
        if (q0 + 32 <= f) {
          size_t slot = s0 + c0 + t;
          quant32(&sh[t * 64 + 32 * hb], hq + slot * f + q0, hsc + slot * (f / 32) + q0 / 32, h16 + slot * (f / 16) + q0 / 16);
        }
      }
    }
    __syncthreads();
  }
}

// Down: the row's K range is split over gridDim.y workgroups of KS waves each. A
// workgroup adds its waves' partial sums in wave order and writes them to its own
// partial slice y[blockIdx.y]; the combine adds the slices in order.
// grid.x = tiles of 64 rows of d_model, grid.y = K groups, grid.z = active-expert slot.
template <int QT, int TM, bool PACKED, int KS>
__global__ void __launch_bounds__(64 * KS)
k_dn_rows(RowIO io, uint32_t ne, uint32_t f, uint32_t d, uint32_t pitch_d, uint32_t part_stride,
          const int8_t* __restrict__ hq, const float* __restrict__ hsc, const int32_t* __restrict__ h16,
          const float* __restrict__ hf, float* __restrict__ ypart) {
  constexpr int E = QT_<QT>::E, P = QT_<QT>::B / 16;
  extern __shared__ uint4 dsm[];
  uint4* tile0 = dsm;                                              // [KS][64*P]
  float* red = reinterpret_cast<float*>(dsm + KS * 64 * P);       // [KS][TM][64]
  uint8_t* acts = reinterpret_cast<uint8_t*>(red + KS * TM * 64);
  const uint32_t a = blockIdx.z;
  if (a >= io.active[0]) return;
  const uint32_t e = io.active[1 + a];
  const uint32_t s0 = io.offsets[e], m_all = io.offsets[e + 1] - s0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t r0 = blockIdx.x * 64;
  const uint8_t* W = io.eptr[2 * ne + e];
  const uint32_t nblk = f / E, nsl = gridDim.y * KS, sl = blockIdx.y * KS + wave;
  const uint32_t j0 = (nblk * sl) / nsl, j1 = (nblk * (sl + 1)) / nsl;
  // the workgroup's K range: its first wave's start to its last wave's end
  const uint32_t jw0 = (nblk * (blockIdx.y * KS)) / nsl, jw1 = (nblk * (blockIdx.y * KS + KS)) / nsl;
  const uint32_t nelem = (jw1 - jw0) * E;
  float* y = ypart + (size_t)blockIdx.y * part_stride;
  for (uint32_t c0 = 0; c0 < m_all; c0 += TM) {
    const int m = (int)min((uint32_t)TM, m_all - c0);
    uint32_t slot[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) slot[t] = s0 + c0 + (t < m ? t : 0);
    if (nelem) {
      if constexpr (PACKED) stage_packed<TM>(acts, nelem, hq, hsc, h16, f, slot, m, jw0 * E);
      else stage_f32<TM>(acts, nelem, hf, f, slot, m, jw0 * E);
    }
    __syncthreads();
    float acc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc[t] = 0.0f;
    stream_rows<QT>(W, pitch_d, r0, d, j0, j1, tile0 + wave * 64 * P, lane, [&](uint32_t j, const uint32_t* w) {
      staged_block<QT, TM, PACKED>(w, acts, nelem, j, jw0, acc, m);
    });
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
// Combine: out[t] = sum over the token's experts of y*w, ascending expert id
// (llama/mod.rs:977-995) or routed rank (moe/mod.rs:104-109); add_scaled multiplies
// then adds, starting from the zeroed output.
// ---------------------------------------------------------------------------------

__global__ void __launch_bounds__(256) k_combine(LayerDev L, FwdBufs B, uint32_t n, uint32_t ksg) {
  const uint32_t t = blockIdx.y, k = L.k, d = L.d;
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n || c >= d) return;
  const size_t part = (size_t)n * k * d;
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
    const float* yp = B.y + (size_t)slot * d + c;
    float yv = yp[0];
    for (uint32_t g = 1; g < ksg; g++) yv += yp[g * part];
    acc = acc + yv * wv;
  }
  B.out[(size_t)t * d + c] = acc;
}

hipError_t launch_combine(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_combine, dim3((L.d + 255) / 256, n), dim3(256), 0, st, L, B, n, down_ksg(L, n));
  return hipGetLastError();
}

__global__ void k_reduce_parts(const float* __restrict__ parts, uint32_t ksg, size_t count, float* __restrict__ out) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  float s = parts[i];
  for (uint32_t g = 1; g < ksg; g++) s += parts[i + g * count];
  out[i] = s;
}

hipError_t launch_reduce_parts(const float* parts, uint32_t ksg, size_t count, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_reduce_parts, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, parts, ksg, count, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Launch selection
// ---------------------------------------------------------------------------------

static inline bool packed_kernel(uint32_t math, uint32_t qt) {
  return math == 0 && has_int8_kernel(qt);
}

// tokens handled together per pass: enough for a decode batch, capped at 8
static inline int pick_tm(uint32_t n) { return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : 8; }

constexpr uint32_t kLdsBudget = 160 * 1024 - 2048;

template <int QT, bool PACKED>
static uint32_t gu_lds(uint32_t tm, uint32_t d) {
  return row_tile_bytes(QT_<QT>::B, 2) + 2 * tm * 64 * 4 + ActLds<PACKED>::bytes(tm, d);
}

template <class K>
static void allow_lds(K kernel, uint32_t bytes) {
  // raise the dynamic LDS limit of this instantiation once (idempotent, cheap)
  hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

template <int QT, int TM, bool PACKED>
static void go_gu_rows(const LayerDev& L, const FwdBufs& B, dim3 g, hipStream_t st) {
  RowIO io{L.eptr, B.active, B.offsets, B.slot_tok};
  uint32_t lds = gu_lds<QT, PACKED>(TM, L.d);
  static bool once = (allow_lds(k_gu_rows<QT, TM, PACKED>, kLdsBudget), true);
  (void)once;
  hipLaunchKernelGGL((k_gu_rows<QT, TM, PACKED>), g, dim3(128), lds, st, io, L.ne, L.f, L.d, L.pitch_gate,
                     L.pitch_up, B.xq, B.xs, B.x16, B.hs, B.hq, B.hsc, B.h16, B.hf);
}

// largest chunk of tokens <= want whose staging fits the LDS budget
template <class F>
static int fit_tm(int want, F lds_of) {
  int tm = want;
  while (tm > 1 && lds_of((uint32_t)tm) > kLdsBudget) tm /= 2;
  return tm;
}

template <int QT, bool PACKED>
static void go_gu_rows_tm(const LayerDev& L, const FwdBufs& B, dim3 g, int want, hipStream_t st) {
  int tm = fit_tm(want, [&](uint32_t t) { return gu_lds<QT, PACKED>(t, L.d); });
  switch (tm) {
    case 1: go_gu_rows<QT, 1, PACKED>(L, B, g, st); break;
    case 2: go_gu_rows<QT, 2, PACKED>(L, B, g, st); break;
    case 4: go_gu_rows<QT, 4, PACKED>(L, B, g, st); break;
    default: go_gu_rows<QT, 8, PACKED>(L, B, g, st); break;
  }
}

constexpr int kDnKS = 2;

// K groups of the row-kernel down product: enough workgroups to cover the chip twice
// over, each wave keeping at least 4 blocks to stream.
uint32_t down_ksg(const LayerDev& L, uint32_t n) {
  if (!row_kernel_type(L.qt_down)) return 1;
  uint32_t tiles = (L.d + 63) / 64, ymax = min(L.ne, n * L.k);
  uint32_t nblk = L.f / ((L.qt_down == F16 || L.qt_down == F32) ? 32u : 256u);
  uint32_t ksg = (512 + tiles * ymax - 1) / (tiles * ymax);
  uint32_t cap = max(1u, nblk / (kDnKS * 4));
  return max(1u, min(min(ksg, cap), (uint32_t)kMaxKsg));
}

template <int QT, bool PACKED>
static uint32_t dn_lds(uint32_t tm, uint32_t f, uint32_t ksg) {
  constexpr uint32_t E = QT_<QT>::E;
  uint32_t nblk = f / E, span = (nblk + ksg - 1) / ksg + 1;
  return row_tile_bytes(QT_<QT>::B, kDnKS) + kDnKS * tm * 64 * 4 + ActLds<PACKED>::bytes(tm, span * E);
}

template <int QT, int TM, bool PACKED>
static void go_dn_rows(const LayerDev& L, const FwdBufs& B, dim3 g, uint32_t n, hipStream_t st) {
  RowIO io{L.eptr, B.active, B.offsets, B.slot_tok};
  uint32_t lds = dn_lds<QT, PACKED>(TM, L.f, g.y);
  static bool once = (allow_lds(k_dn_rows<QT, TM, PACKED, kDnKS>, kLdsBudget), true);
  (void)once;
  hipLaunchKernelGGL((k_dn_rows<QT, TM, PACKED, kDnKS>), g, dim3(64 * kDnKS), lds, st, io, L.ne, L.f, L.d,
                     L.pitch_down, n * L.k * L.d, B.hq, B.hsc, B.h16, B.hf, B.y);
}

template <int QT, bool PACKED>
static void go_dn_rows_tm(const LayerDev& L, const FwdBufs& B, dim3 g, int want, uint32_t n, hipStream_t st) {
  int tm = fit_tm(want, [&](uint32_t t) { return dn_lds<QT, PACKED>(t, L.f, g.y); });
  switch (tm) {
    case 1: go_dn_rows<QT, 1, PACKED>(L, B, g, n, st); break;
    case 2: go_dn_rows<QT, 2, PACKED>(L, B, g, n, st); break;
    case 4: go_dn_rows<QT, 4, PACKED>(L, B, g, n, st); break;
    default: go_dn_rows<QT, 8, PACKED>(L, B, g, n, st); break;
  }
}

hipError_t launch_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  uint32_t ymax = min(L.ne, n * L.k);
  if (row_kernel_type(L.qt_gate)) {
    dim3 g((L.f + 63) / 64, ymax);
    int tm = pick_tm(n);
    bool pk = packed_kernel(L.math, L.qt_gate);
    switch (L.qt_gate) {
      case Q4_K: pk ? go_gu_rows_tm<Q4_K, true>(L, B, g, tm, st) : go_gu_rows_tm<Q4_K, false>(L, B, g, tm, st); break;
      case Q5_K: pk ? go_gu_rows_tm<Q5_K, true>(L, B, g, tm, st) : go_gu_rows_tm<Q5_K, false>(L, B, g, tm, st); break;
      case F16: go_gu_rows_tm<F16, false>(L, B, g, tm, st); break;
      case F32: go_gu_rows_tm<F32, false>(L, B, g, tm, st); break;
    }
    return hipGetLastError();
  }
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
  if (row_kernel_type(L.qt_down)) {
    dim3 g((L.d + 63) / 64, down_ksg(L, n), ymax);
    int tm = pick_tm(n);
    bool pk = packed_kernel(L.math, L.qt_down);
    switch (L.qt_down) {
      case Q4_K: pk ? go_dn_rows_tm<Q4_K, true>(L, B, g, tm, n, st) : go_dn_rows_tm<Q4_K, false>(L, B, g, tm, n, st); break;
      case Q5_K: pk ? go_dn_rows_tm<Q5_K, true>(L, B, g, tm, n, st) : go_dn_rows_tm<Q5_K, false>(L, B, g, tm, n, st); break;
      case F16: go_dn_rows_tm<F16, false>(L, B, g, tm, n, st); break;
      case F32: go_dn_rows_tm<F32, false>(L, B, g, tm, n, st); break;
    }
    return hipGetLastError();
  }
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
