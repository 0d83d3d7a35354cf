// gmoe_prefill.hip — prefill-sized expert products on MFMA, f32 math.
//
// Compiled once per block type, with -DGMOE_QT=<ggml type id>, like gmoe_units.hip.
//
// Reference semantics: llama/mod.rs:1002-1020 under Weight::Full (mmap = false): the
// weights are the dequantised f32 values (quant/mod.rs:624-875) and every product is an
// f32 dot (simd/mod.rs:96-129); layer outputs must stay within rtol 1e-3 / atol 1e-4 of
// it. A single fp16 (or bf16) MFMA pass rounds both operands and misses that bar, so
// the products are made exact instead:
//
//  * weights: a dequantised value is w = d * (sc * q) - dmin * m (K-quants) or d * q
//    (Q8_0/Q4_0, Q6_K with d*sc as d), with q a small integer. The integer part (sc * q,
//    or q) is exact in fp16 (|.| <= 1953 < 2048) and is the MFMA operand; the block
//    scale d (f32) multiplies the block's partial sums afterwards.
//  * activations: x = hi + lo, both fp16 (22 significant bits); two MFMAs per step.
//  * mins (Q4_K/Q5_K/Q2_K): the sum over sub-blocks of (dmin * m) * S, S the
//    sub-block's sum of x, is a GEMM of length K/32 (or K/16) run on MFMA with both
//    operands split (three passes).
//
// Every product is then an exact fp16 x fp16 product accumulated in f32, and the layer
// differs from the f32 reference by reordered f32 sums (~1e-6 relative).
//
// Work layout. The dispatch lists the call's token tiles (kPfTok = 64 tokens of one
// expert, in slot order) in B.ptile; blockIdx.y is a token tile. A workgroup has PF<QT>::NW
// waves (8; 4 for Q6_K), each owning 32 rows: gate/up
// workgroups take NW * 32 rows of f (both matrices: 256 for NW = 8), down workgroups NW *
// 64 rows of d. Each wave owns two 32-row MFMA row tiles (gate and up of its 32 rows, or
// two 32-row halves of its 64 down rows) and both 32-token tiles: 4 accumulators of 32x32,
// plus 4 of partial block sums. Per chunk of K (PF<QT>::KC values: 128; 64 for Q5_K and
// Q8_0, 32 for F16) the workgroup copies the chunk's raw 16-byte pieces of its rows (the
// slab's tiled layout makes each piece of 64 rows one 1 KiB run) and the tokens' hi/lo
// activations into LDS; a lane then decodes
// its row's 8 values of each 16-value K step straight into the MFMA B operand.
//
// v_mfma_f32_32x32x16_f16 (operand layout checked on the device): lane l supplies row
// l%32 of A and column l%32 of B, each with k = 8*(l/32) .. +7, and holds D[i][l%32] for
// i = 8*(r/4) + 4*(l/32) + r%4, r = 0..15. A is the tokens, B the weight rows, so a
// lane's 16 results share one weight row and one block scale.
#include <utility>

#include "gmoe_unit.h"

#ifndef GMOE_QT
#error "gmoe_prefill.hip is compiled once per block type with -DGMOE_QT=<type id>"
#endif

namespace gmoe {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kPfWaves = 4, kPfThreads = 64 * kPfWaves;

// f(integral_constant<int, I>) for I = 0 .. N-1, each call with I a constant.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------------------------
// Per-type shape: EU values per slab unit, KC values per LDS chunk, NPC 16-byte pieces
// of a unit that chunk c needs (piece(c, i) is the i-th), SU16 K16 steps per scale
// (0: the decoded values are the weights), SW the width of a min-term sub-block, NW
// waves per workgroup. A workgroup double-buffers its chunks, 2 x (NW * NPC KiB of
// weight pieces + 2 * kPfTok * KC * 2 bytes of activations), within the 160 KiB of LDS.
// Unit byte layouts are those of the packed blocks (quant/mod.rs:624-875); Q8_0/Q4_0
// units are eight blocks repacked as 8 f16 scales then the quants.
// ---------------------------------------------------------------------------------
template <int QT> struct PF;
template <> struct PF<Q4_K> {  // d dmin | scales[12] | qs[128]: sub-blocks 4c..4c+3 in pieces 1+4c..
  static constexpr int EU = 256, KC = 128, NPC = 5, SU16 = 16, SW = 32, NW = 8;
  static constexpr int piece(int c, int i) { return i == 0 ? 0 : 4 * c + i; }
};
template <> struct PF<Q5_K> {  // d dmin scales | qh[32] | qs[128]: sub-blocks 2c, 2c+1 in pieces 3+2c..
  static constexpr int EU = 256, KC = 64, NPC = 5, SU16 = 16, SW = 32, NW = 8;
  static constexpr int piece(int c, int i) { return i < 3 ? i : 2 * c + i; }
};
template <> struct PF<Q6_K> {  // ql[128] | qh[64] | scales[16] | d
  static constexpr int EU = 256, KC = 128, NPC = 8, SU16 = 1, SW = 0, NW = 4;
  static constexpr int piece(int c, int i) { return i < 4 ? 4 * c + i : i < 6 ? 8 + 2 * c + (i - 4) : 12 + (i - 6); }
};
template <> struct PF<Q3_K> {  // values regrouped (q3s_word): sub-blocks 8c.. in pieces 3c..3c+2 | scales[12] d
  static constexpr int EU = 256, KC = 128, NPC = 4, SU16 = 16, SW = 0, NW = 8;
  static constexpr int piece(int c, int i) { return i < 3 ? 3 * c + i : 6; }
};
template <> struct PF<Q2_K> {  // scales[16] | qs[64] | d dmin
  static constexpr int EU = 256, KC = 128, NPC = 4, SU16 = 16, SW = 16, NW = 8;
  static constexpr int piece(int c, int i) { return i == 0 ? 0 : i < 3 ? 1 + 2 * c + (i - 1) : 5; }
};
template <> struct PF<Q8_0> {  // 8 scales | 8 x 32 quants: blocks 2c, 2c+1 in pieces 1+4c..4+4c
  static constexpr int EU = 256, KC = 64, NPC = 5, SU16 = 2, SW = 0, NW = 8;
  static constexpr int piece(int c, int i) { return i == 0 ? 0 : 4 * c + i; }
};
template <> struct PF<Q4_0> {  // 8 scales | 8 x 16 quant bytes
  static constexpr int EU = 256, KC = 128, NPC = 5, SU16 = 2, SW = 0, NW = 8;
  static constexpr int piece(int c, int i) { return i == 0 ? 0 : 4 * c + i; }
};
template <> struct PF<F16> {  // 64 halves: values 32c.. in pieces 4c..4c+3
  static constexpr int EU = 64, KC = 32, NPC = 4, SU16 = 0, SW = 0, NW = 8;
  static constexpr int piece(int c, int i) { return 4 * c + i; }
};

template <int QT>
constexpr int pf_slot(int c, int p) {
  for (int i = 0; i < PF<QT>::NPC; i++)
    if (PF<QT>::piece(c, i) == p) return i;
  return -1;
}

// Byte OFF of the lane's unit, chunk C staged: row points at the row's piece in slot 0.
template <int QT, int C, int OFF>
__device__ __forceinline__ const uint8_t* pf_at(const uint8_t* row) {
  constexpr int sl = pf_slot<QT>(C, OFF / 16);
  static_assert(sl >= 0, "piece not staged for this chunk");
  return row + sl * 1024 + OFF % 16;
}
__device__ __forceinline__ u32x2 ld8(const uint8_t* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// 16 bytes at src -> LDS at dst + 16 * lane (dst the same for the whole wave).
__device__ __forceinline__ void lds_load16(const void* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

__device__ __forceinline__ half2_t h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ half2_t h2s(_Float16 v) { return half2_t{v, v}; }

// Four bytes b0..b3 (each < 1024) as fp16 pairs (1024 + b0, 1024 + b1), (1024 + b2,
// 1024 + b3): byte-permute each beside the exponent byte 0x64.
__device__ __forceinline__ void magic4(uint32_t b, half2_t& p0, half2_t& p1) {
  p0 = h2(__builtin_amdgcn_perm(b, 0x64646464u, 0x00050004u));
  p1 = h2(__builtin_amdgcn_perm(b, 0x64646464u, 0x00070006u));
}

// 8 bytes (two dwords) -> 8 fp16 values f(1024 + byte) with f(t) = fma(t, mul, add);
// exact when the result is an integer of magnitude <= 2048.
__device__ __forceinline__ half8 bytes_fma(u32x2 b, half2_t mul, half2_t add) {
  half8 o;
#pragma unroll
  for (int d = 0; d < 2; d++) {
    half2_t p0, p1;
    magic4(b[d], p0, p1);
    p0 = __builtin_elementwise_fma(p0, mul, add);
    p1 = __builtin_elementwise_fma(p1, mul, add);
    o[4 * d] = p0.x; o[4 * d + 1] = p0.y; o[4 * d + 2] = p1.x; o[4 * d + 3] = p1.y;
  }
  return o;
}

// 8 bytes (two dwords) -> 8 fp16 values byte * 2^-24: each byte beside a zero byte, the
// fp16 subnormal of that mantissa (exact for bytes < 1024). The MFMAs keep fp16
// subnormals under the kernels' default float mode (no flush-to-zero flag is set here);
// the packed-prefill tests compare every output bit for bit.
__device__ __forceinline__ half8 bytes_sub(u32x2 b) {
  half8 o;
#pragma unroll
  for (int d = 0; d < 2; d++) {
    const half2_t p0 = h2(__builtin_amdgcn_perm(0u, b[d], 0x0c010c00u));
    const half2_t p1 = h2(__builtin_amdgcn_perm(0u, b[d], 0x0c030c02u));
    o[4 * d] = p0.x; o[4 * d + 1] = p0.y; o[4 * d + 2] = p1.x; o[4 * d + 3] = p1.y;
  }
  return o;
}

__device__ __forceinline__ _Float16 fh(uint32_t v) { return (_Float16)(float)v; }
// The low half of v as f32 (a scale or min; non-finite ones give non-finite outputs).
__device__ __forceinline__ float f16v(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)v); }

// ---------------------------------------------------------------------------------
// Decoders: frag<C, S>(row, h) = the integer parts of values 16S + 8h .. +7 of the unit
// (K16 step S, staged in chunk C), as exact fp16; scale<C, S>(row) = the f32 factor of
// the scale group that step S closes; mins<C>(row, h, hi, lo) = -(dmin * m) of the
// lane's 8 min-term sub-blocks as an fp16 pair.
// ---------------------------------------------------------------------------------
template <int QT> struct Dec;

template <> struct Dec<Q4_K> {
  static constexpr int QT = Q4_K;
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    constexpr int sb = S / 2;
    constexpr bool high = sb & 1;
    const u32x4 hd = ld16(pf_at<QT, C, 0>(row));
    const uint32_t s3[3] = {hd.y, hd.z, hd.w};
    uint32_t sc, m;
    scale_min_k4(s3, sb, sc, m);
    u32x2 q = ld8(pf_at<QT, C, 16 + 32 * (sb / 2) + 16 * (S % 2)>(row) + 8 * h);
    const uint32_t mask = high ? 0xf0f0f0f0u : 0x0f0f0f0fu;
    q.x &= mask;
    q.y &= mask;
    // high nibbles stay in place (16q): scale by sc/16
    const _Float16 f = high ? fh(sc) * (_Float16)0.0625f : fh(sc);
    return bytes_fma(q, h2s(f), h2s(f * (_Float16)-1024.0f));
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t* row) {
    return f16v(ld16(pf_at<QT, C, 0>(row)).x);
  }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t* row, uint32_t h, half8& hi, half8& lo) {
    const u32x4 hd = ld16(pf_at<QT, C, 0>(row));
    const uint32_t s3[3] = {hd.y, hd.z, hd.w};
    const float dmin = f16v(hd.x >> 16);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      uint32_t sc, m;
      scale_min_k4(s3, j, sc, m);
      const float b = h ? 0.0f : -(dmin * (float)m);
      hi[j] = (_Float16)b;
      lo[j] = (_Float16)(b - (float)hi[j]);
    }
  }
};

template <> struct Dec<Q5_K> {
  static constexpr int QT = Q5_K;
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    constexpr int sb = S / 2;
    const u32x4 hd = ld16(pf_at<QT, C, 0>(row));
    const uint32_t s3[3] = {hd.y, hd.z, hd.w};
    uint32_t sc, m;
    scale_min_k4(s3, sb, sc, m);
    const u32x2 qh = ld8(pf_at<QT, C, 16 + 16 * (S % 2)>(row) + 8 * h);
    const u32x2 ql = ld8(pf_at<QT, C, 48 + 32 * (sb / 2) + 16 * (S % 2)>(row) + 8 * h);
    u32x2 b;
#pragma unroll
    for (int d = 0; d < 2; d++)
      b[d] = ((sb & 1 ? ql[d] >> 4 : ql[d]) & 0x0f0f0f0fu) | (((qh[d] >> sb) & 0x01010101u) << 4);
    const _Float16 f = fh(sc);
    return bytes_fma(b, h2s(f), h2s(f * (_Float16)-1024.0f));
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t* row) {
    return f16v(ld16(pf_at<QT, C, 0>(row)).x);
  }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t* row, uint32_t h, half8& hi, half8& lo) {
    const u32x4 hd = ld16(pf_at<QT, C, 0>(row));  // same header layout as Q4_K
    const uint32_t s3[3] = {hd.y, hd.z, hd.w};
    const float dmin = f16v(hd.x >> 16);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      uint32_t sc, m;
      scale_min_k4(s3, j, sc, m);
      const float b = h ? 0.0f : -(dmin * (float)m);
      hi[j] = (_Float16)b;
      lo[j] = (_Float16)(b - (float)hi[j]);
    }
  }
};

template <> struct Dec<Q6_K> {
  static constexpr int QT = Q6_K;
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    constexpr int n = S / 8, j4 = (S % 8) / 2;
    const u32x2 ql = ld8(pf_at<QT, C, 64 * n + 32 * (j4 % 2) + 16 * (S % 2)>(row) + 8 * h);
    const u32x2 qh = ld8(pf_at<QT, C, 128 + 32 * n + 16 * (S % 2)>(row) + 8 * h);
    u32x2 b;
#pragma unroll
    for (int d = 0; d < 2; d++)
      b[d] = ((j4 >= 2 ? ql[d] >> 4 : ql[d]) & 0x0f0f0f0fu) | (((qh[d] >> (2 * j4)) & 0x03030303u) << 4);
    return bytes_fma(b, h2s((_Float16)1.0f), h2s((_Float16)-1056.0f));  // q - 32
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t* row) {
    constexpr int n = S / 8, j4 = (S % 8) / 2, is = 8 * n + 2 * j4 + S % 2;
    const u32x4 sc = ld16(pf_at<QT, C, 192>(row));
    const float d = f16v(ld16(pf_at<QT, C, 208>(row)).x);
    const float s = (float)(int8_t)((sc[is / 4] >> (8 * (is % 4))) & 0xffu);
    return d * s;  // (d * sc) * q, as the reference orders it
  }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t*, uint32_t, half8&, half8&) {}
};

// Q3_K step S (sub-block S) of chunk C: lane half h's words O(S, 2h), O(S, 2h + 1) of the
// regrouped values v = q2 + 4 * hbit (q3s_word: the half's three words of the sub-group
// sit at bytes 48C + 16 (x / 2) + 4 (x % 2) + 8h of the unit).
template <int C, int S>
__device__ __forceinline__ u32x2 q3s_step(const uint8_t* row, uint32_t h) {
  constexpr int x0 = 3 * ((S % 8) / 4), k = S % 4;
  auto word = [&](auto xc) {
    constexpr int x = decltype(xc)::value;
    return *reinterpret_cast<const uint32_t*>(pf_at<Q3_K, C, 48 * C + 16 * (x / 2) + 4 * (x % 2)>(row) + 8 * h);
  };
  uint32_t b0, b1;
  if constexpr (k == 3) {
    q3s_pair(word(std::integral_constant<int, x0>{}), word(std::integral_constant<int, x0 + 1>{}),
             word(std::integral_constant<int, x0 + 2>{}), k, b0, b1);
  } else {
    const uint32_t t = word(std::integral_constant<int, x0 + k>{});
    q3s_pair(t, t, t, k, b0, b1);
  }
  return u32x2{b0, b1};
}

template <> struct Dec<Q3_K> {
  static constexpr int QT = Q3_K;
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    constexpr int is = S;
    const u32x4 tl = ld16(pf_at<QT, C, 96>(row));  // scales[12] | d
    uint32_t sc4[4];
    q3k_scales(tl.x, tl.y, tl.z, sc4);
    const int scs = (int)((sc4[is / 4] >> (8 * (is % 4))) & 0xffu) - 32;
    const u32x2 b = q3s_step<C, S>(row, h);  // q2 + 4 * hbit in [0, 7]; the value is b - 4
    half8 o;
    const half2_t s2 = h2s((_Float16)(float)scs);
#pragma unroll
    for (int d = 0; d < 2; d++) {
      half2_t p0, p1;
      magic4(b[d], p0, p1);
      p0 = (p0 - h2s((_Float16)1028.0f)) * s2;  // (b - 4) * (sc - 32): |.| <= 128
      p1 = (p1 - h2s((_Float16)1028.0f)) * s2;
      o[4 * d] = p0.x; o[4 * d + 1] = p0.y; o[4 * d + 2] = p1.x; o[4 * d + 3] = p1.y;
    }
    return o;
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t* row) {
    return f16v(ld16(pf_at<QT, C, 96>(row)).w);
  }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t*, uint32_t, half8&, half8&) {}
};

template <> struct Dec<Q2_K> {
  static constexpr int QT = Q2_K;
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    constexpr int n = S / 8, j4 = (S % 8) / 2, is = 8 * n + 2 * j4 + S % 2;
    const u32x2 qs = ld8(pf_at<QT, C, 16 + 32 * n + 16 * (S % 2)>(row) + 8 * h);
    const u32x4 scb = ld16(pf_at<QT, C, 0>(row));
    const uint32_t sc = (scb[is / 4] >> (8 * (is % 4))) & 15u;
    u32x2 b;
#pragma unroll
    for (int d = 0; d < 2; d++) b[d] = (qs[d] >> (2 * j4)) & 0x03030303u;
    const _Float16 f = fh(sc);
    return bytes_fma(b, h2s(f), h2s(f * (_Float16)-1024.0f));
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t* row) {
    return f16v(ld16(pf_at<QT, C, 80>(row)).x);
  }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t* row, uint32_t h, half8& hi, half8& lo) {
    const u32x4 scb = ld16(pf_at<QT, C, 0>(row));
    const float dmin = f16v(ld16(pf_at<QT, C, 80>(row)).x >> 16);
    const uint32_t w0 = h ? scb.z : scb.x, w1 = h ? scb.w : scb.y;  // sub-blocks 8h .. 8h+7
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t m = (((j < 4 ? w0 : w1) >> (8 * (j % 4))) & 0xffu) >> 4;
      const float b = -(dmin * (float)m);
      hi[j] = (_Float16)b;
      lo[j] = (_Float16)(b - (float)hi[j]);
    }
  }
};

template <> struct Dec<Q8_0> {
  static constexpr int QT = Q8_0;
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    u32x2 q = ld8(pf_at<QT, C, 16 + 32 * (S / 2) + 16 * (S % 2)>(row) + 8 * h);
    q.x ^= 0x80808080u;  // q + 128 as unsigned bytes
    q.y ^= 0x80808080u;
    return bytes_fma(q, h2s((_Float16)1.0f), h2s((_Float16)-1152.0f));
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t* row) {
    constexpr int b = S / 2;
    return f16v(ld16(pf_at<QT, C, 0>(row))[b / 2] >> (16 * (b % 2)));
  }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t*, uint32_t, half8&, half8&) {}
};

template <> struct Dec<Q4_0> {
  static constexpr int QT = Q4_0;
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    constexpr bool high = S & 1;  // values 16..31 of the block are the high nibbles
    u32x2 q = ld8(pf_at<QT, C, 16 + 16 * (S / 2)>(row) + 8 * h);
    const uint32_t mask = high ? 0xf0f0f0f0u : 0x0f0f0f0fu;
    q.x &= mask;
    q.y &= mask;
    // low: (1024 + q) - 1032; high: (1024 + 16q) / 16 - 72
    return high ? bytes_fma(q, h2s((_Float16)0.0625f), h2s((_Float16)-72.0f))
                : bytes_fma(q, h2s((_Float16)1.0f), h2s((_Float16)-1032.0f));
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t* row) {
    constexpr int b = S / 2;
    return f16v(ld16(pf_at<QT, C, 0>(row))[b / 2] >> (16 * (b % 2)));
  }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t*, uint32_t, half8&, half8&) {}
};

template <> struct Dec<F16> {
  template <int C, int S>
  static __device__ __forceinline__ half8 frag(const uint8_t* row, uint32_t h) {
    // values 16S + 8h .. are bytes 32S + 16h ..: piece 2S + h, slot 2S + h - 4C
    return __builtin_bit_cast(half8, ld16(row + (2 * S - 4 * C + h) * 1024));
  }
  template <int C, int S>
  static __device__ __forceinline__ float scale(const uint8_t*) { return 1.0f; }
  template <int C>
  static __device__ __forceinline__ void mins(const uint8_t*, uint32_t, half8&, half8&) {}
};

// ---------------------------------------------------------------------------------
// The kernel. GU: gate/up (rows of f, input x planes of width d, output h planes and,
// when the down type has mins, h sums of width swo). !GU: down (rows of d, input h of
// width f, units [u0, u1) of K per blockIdx.z slice, output y slice blockIdx.z).
// ---------------------------------------------------------------------------------
struct PfArgs {
  const ExpertWork* work;
  const uint32_t* ptile;
  const _Float16* in;     // [2][nk][K] hi, lo planes
  const _Float16* ins;    // [2][nk][K/SW] sums (types with mins)
  uint32_t nk, K, rows;   // slots, input width, output rows (f or d)
  uint32_t upk;           // down: units of K per slice
  _Float16* out;          // GU: [2][nk][rows] h planes
  _Float16* outs;         // GU: [2][nk][rows/swo] h sums, or null
  uint32_t swo;           // GU: width of the h sums (0: none)
  float* y;               // down: [slices][nk][rows]
};

// The (row block, token tile) of a workgroup of a gate/up grid (gridDim.x row blocks,
// gridDim.y token tiles). Workgroups go round-robin over the 8 XCDs, each with its own L2,
// and the token tiles of one expert read the same weight rows. With gridDim.x a multiple
// of 8, XCD c's sequence of workgroups is remapped to take one row block's token tiles one
// after another, so an expert's tiles of a row block run side by side on one XCD and the
// weights come from its L2 after the first; otherwise the launch's own order.
__device__ __forceinline__ void pf_block(uint32_t& bx, uint32_t& by) {
  bx = blockIdx.x;
  by = blockIdx.y;
  if (gridDim.x % 8 == 0) {
    const uint32_t L = blockIdx.y * gridDim.x + blockIdx.x, j = L / 8;
    bx = (j / gridDim.y) * 8 + L % 8;
    by = j % gridDim.y;
  }
}

template <int QT, bool GU>
__global__ void __launch_bounds__(64 * PF<QT>::NW) k_pf(PfArgs a) {
  using T = PF<QT>;
  using D = Dec<QT>;
  constexpr int NW = T::NW, NT = 64 * NW;
  constexpr int KC = T::KC, NCK = KC / 8, NPC = T::NPC, NCH = T::EU / KC, SPC = KC / 16;
  constexpr int U = UT_<QT>::U, NP = U / 16;
  constexpr uint32_t WROWS = 32 * NW * (GU ? 1 : 2);    // rows of a workgroup
  // min-term sums of a unit: NS halves per token and plane, staged with its last chunk
  constexpr int NS = T::SW ? T::EU / T::SW : 0;
  constexpr uint32_t WBYTES = NW * NPC * 1024, XBYTES = 2 * kPfTok * KC * 2, SBYTES = 2 * kPfTok * NS * 2;
  constexpr uint32_t BUF = WBYTES + XBYTES + SBYTES;
  constexpr int NX = 2 * (int)kPfTok * NCK / NT;        // activation loads per thread per chunk
  static_assert(2 * BUF <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * BUF];

  uint32_t bx = blockIdx.x, by = blockIdx.y;
  if constexpr (GU) pf_block(bx, by);
  const uint32_t pt = a.ptile[by];
  if (pt == ~0u) return;
  const ExpertWork* W = a.work + (pt >> 16);
  const uint32_t t0 = (pt & 0xffffu) * kPfTok;
  const uint32_t m = min(kPfTok, W->m - t0), s0 = W->s0 + t0;
  const uint32_t tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t K = a.K, nunit = K / T::EU;
  const uint32_t u0 = GU ? 0 : blockIdx.z * a.upk, u1 = GU ? nunit : min(nunit, u0 + a.upk);
  const size_t plane = (size_t)a.nk * K;

  // slab tiles of the workgroup's NW (matrix, tile) pairs: NW/2 gate tiles then NW/2 up
  // tiles (GU), or NW down tiles
  const size_t tile_bytes = (size_t)nunit * kTileRows * U;
  const uint8_t* m_lo = GU ? W->w[0] + (NW / 2) * bx * tile_bytes : W->w[2] + NW * bx * tile_bytes;
  const uint8_t* m_hi = GU ? W->w[1] + (NW / 2) * bx * tile_bytes : m_lo + (NW / 2) * tile_bytes;
  // the lane's row in each of its two row tiles (offsets into a weight buffer)
  uint32_t row[2];
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const uint32_t tm = GU ? rt * (NW / 2) + wave / 2 : wave, i = GU ? 32 * (wave % 2) + l32 : 32 * rt + l32;
    row[rt] = (tm * NPC * 64 + i) * 16;
  }
  // the lane's token row of its first 32-token tile in an activation buffer, and its
  // column swizzle (t % NCK, the same for both tiles), in bytes
  const uint32_t xrow = l32 * NCK * 16;
  uint32_t tsw = (l32 % NCK) * 16;

  // chunk (u, c) into buffer b: straight into LDS (global_load_lds: lane i of a wave
  // writes 16 bytes at the wave's base + 16 i); the wave's j-th batch is items
  // 64 wq + lane, wq = NW j + wave, at byte 16 * item of the buffer's part
  auto stage = [&](uint32_t u, auto cc, uint32_t b) {
    constexpr int C = decltype(cc)::value;
    uint8_t* wb = lds + b * BUF;
    uint8_t* xb = wb + WBYTES;
    // weight pieces: item (tm, pc, row i)
#pragma unroll
    for (int j = 0; j < NPC; j++) {
      const uint32_t wq = NW * j + wave, tm = wq / NPC, pc = wq % NPC;
      const uint8_t* src = (tm < NW / 2 ? m_lo : m_hi) + (tm % (NW / 2)) * tile_bytes;
      lds_load16(src + ((size_t)u * NP + (uint32_t)T::piece(C, (int)pc)) * 1024 + lane * 16, wb + 1024 * wq);
    }
    // activations: item (plane, token t, position); 16-byte column c of token t at
    // position c ^ (t % NCK)
    constexpr uint32_t RW = 64 / NCK;  // token rows per wave batch
    const uint32_t k0 = u * T::EU + C * KC;
#pragma unroll
    for (int j = 0; j < NX; j++) {
      const uint32_t wq = NW * j + wave, pl = wq / NCK;
      const uint32_t t = (RW * wq) % kPfTok + lane / NCK, c = (lane % NCK) ^ (t % NCK), tc = min(t, m - 1);
      lds_load16(a.in + pl * plane + ((s0 + tc) * K + k0 + 8 * c), xb + 1024 * wq);
    }
    if constexpr (NS != 0 && C == NCH - 1) {
      // the unit's sub-block sums: item (plane, token t, piece e) = sums 8e .. 8e+7 of
      // token t, at byte 16 * item of the sums part
      constexpr uint32_t NE8 = NS / 8, ITEMS = 2 * kPfTok * NE8;
      const uint32_t ns_row = K / T::SW;
#pragma unroll
      for (uint32_t j = 0; j < (ITEMS + NT - 1) / NT; j++) {
        const uint32_t wq = NW * j + wave;
        if (wq * 64 < ITEMS) {
          const uint32_t q = 64 * wq + lane, e = q % NE8, t = (q / NE8) % kPfTok, pl = q / (NE8 * kPfTok);
          const uint32_t tc = min(t, m - 1);
          lds_load16(a.ins + (size_t)pl * a.nk * ns_row + (size_t)(s0 + tc) * ns_row + u * NS + 8 * e,
                     xb + XBYTES + 1024 * wq);
        }
      }
    }
  };

  f32x16 acc[2][2], P[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = P[i][j][r] = 0.0f;
  const f32x16 zero = acc[0][0];
  const bool two = m > 32;  // the second 32-token tile holds tokens

  // one barrier per chunk: chunk k computes from buffer k % 2 while chunk k+1 loads into
  // the other; the barrier after it says both that every wave is done reading buffer
  // k % 2 and that every wave's loads of chunk k+1 have landed
  if (u0 < u1) stage(u0, std::integral_constant<int, 0>{}, 0);  // a slice past the end writes zeros
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // the main loop compiled twice, with and without the second 32-token tile, so that no
  // branch splits a chunk's steps and the scheduler can overlap one step's LDS reads and
  // weight decode with the previous step's MFMAs
  auto main_loop = [&](auto twoc) {
    constexpr bool TWO = decltype(twoc)::value;
    for (uint32_t u = u0; u < u1; u++) {
      static_for<NCH>([&](auto cc) {
        constexpr int C = decltype(cc)::value;
        const uint32_t b = (NCH % 2 == 0) ? (uint32_t)(C % 2) : ((u - u0) * NCH + C) % 2;
        if constexpr (C + 1 < NCH) {
          stage(u, std::integral_constant<int, C + 1>{}, b ^ 1);
        } else {
          if (u + 1 < u1) stage(u + 1, std::integral_constant<int, 0>{}, b ^ 1);
        }
        const uint8_t* wb = lds + b * BUF;
        const uint8_t* xb = wb + WBYTES;
        asm volatile("" : "+v"(tsw));  // per-step addresses are made here, not kept across chunks
        static_for<SPC>([&](auto ss) {
          constexpr int SL = decltype(ss)::value, S = C * SPC + SL;
          half8 bw[2], ax[2][2];
  #pragma unroll
          for (int rt = 0; rt < 2; rt++) bw[rt] = D::template frag<C, S>(wb + row[rt], h);
          const uint32_t pos = ((2 * SL + h) * 16) ^ tsw;
  #pragma unroll
          for (int tt = 0; tt < 2; tt++)
  #pragma unroll
            for (int pl = 0; pl < 2; pl++)
              ax[tt][pl] = *reinterpret_cast<const half8*>(xb + xrow + pos + (pl * kPfTok + 32 * tt) * NCK * 16);
  #pragma unroll
          for (int rt = 0; rt < 2; rt++)
  #pragma unroll
            for (int tt = 0; tt < 2; tt++) {
              if (tt == 1 && !TWO) continue;  // a tile of at most 32 tokens: its second half is padding
              if constexpr (T::SU16 == 0) {
                acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[tt][0], bw[rt], acc[rt][tt], 0, 0, 0);
                acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[tt][1], bw[rt], acc[rt][tt], 0, 0, 0);
              } else {
                const f32x16 c0 = (S % T::SU16 == 0) ? zero : P[rt][tt];
                P[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[tt][0], bw[rt], c0, 0, 0, 0);
                P[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[tt][1], bw[rt], P[rt][tt], 0, 0, 0);
              }
            }
          if constexpr (T::SU16 != 0) {
            if constexpr ((S + 1) % T::SU16 == 0) {
  #pragma unroll
              for (int rt = 0; rt < 2; rt++) {
                const float sc = D::template scale<C, S>(wb + row[rt]);
  #pragma unroll
                for (int tt = 0; tt < 2; tt++)
                  if (tt == 0 || TWO)
  #pragma unroll
                    for (int r = 0; r < 16; r++) acc[rt][tt][r] = __builtin_fmaf(sc, P[rt][tt][r], acc[rt][tt][r]);
              }
            }
            // short scale groups: keep the scheduler from overlapping the next group's
            // partial sums with these (two live sets of P do not fit the registers)
            if constexpr (T::SU16 <= 2) __builtin_amdgcn_sched_barrier(0);
          }
        });
        if constexpr (T::SW != 0 && C == NCH - 1) {
          // min term of unit u: -sum over its sub-blocks of (dmin*m) * S, three MFMA passes
          half8 bh[2], bl[2];
  #pragma unroll
          for (int rt = 0; rt < 2; rt++) D::template mins<C>(wb + row[rt], h, bh[rt], bl[rt]);
          const uint8_t* sb = xb + XBYTES;
  #pragma unroll
          for (int tt = 0; tt < 2; tt++) {
            if (tt == 1 && !TWO) continue;
            // sums 8h'.. of token t (h' = h with 16 sub-blocks; with 8 the upper lanes' B is zero)
            const uint32_t t = 32 * tt + l32, e = NS == 16 ? h : 0;
            const half8 sh = *reinterpret_cast<const half8*>(sb + ((0 * kPfTok + t) * (NS / 8) + e) * 16);
            const half8 sl = *reinterpret_cast<const half8*>(sb + ((1 * kPfTok + t) * (NS / 8) + e) * 16);
  #pragma unroll
            for (int rt = 0; rt < 2; rt++) {
              acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh, bh[rt], acc[rt][tt], 0, 0, 0);
              acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sl, bh[rt], acc[rt][tt], 0, 0, 0);
              acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh, bl[rt], acc[rt][tt], 0, 0, 0);
            }
          }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      });
    }
  };
  if (two) main_loop(std::true_type{});
  else main_loop(std::false_type{});

  // epilogue
#pragma unroll
  for (int tt = 0; tt < 2; tt++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const uint32_t t = 32 * tt + 8 * (r / 4) + 4 * h + (r % 4);
      if constexpr (GU) {
        const uint32_t fr = bx * WROWS + 32 * wave + l32;
        const float hv = swiglu(acc[0][tt][r], acc[1][tt][r]);
        const _Float16 hi = (_Float16)hv, lo = (_Float16)(hv - (float)hi);
        if (t < m) {
          const size_t o = (size_t)(s0 + t) * a.rows + fr;
          a.out[o] = hi;
          a.out[o + (size_t)a.nk * a.rows] = lo;
        }
        if (a.swo) {  // sums of h over swo consecutive rows (lanes): the down min term's S
          float sm = hv;  // offsets fixed at compile time, so the 32 reductions overlap
#pragma unroll
          for (int o = 1; o <= 8; o <<= 1) sm += __shfl_xor(sm, o, 64);
          if (a.swo == 32) sm += __shfl_xor(sm, 16, 64);
          if (t < m && (l32 % a.swo) == 0) {
            const uint32_t ns = a.rows / a.swo;
            const size_t o = (size_t)(s0 + t) * ns + fr / a.swo;
            const _Float16 shi = (_Float16)sm;
            a.outs[o] = shi;
            a.outs[o + (size_t)a.nk * ns] = (_Float16)(sm - (float)shi);
          }
        }
      } else {
        float* y = a.y + (size_t)blockIdx.z * a.nk * a.rows;
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
          const uint32_t dr = bx * WROWS + 64 * wave + 32 * rt + l32;
          if (t < m) y[(size_t)(s0 + t) * a.rows + dr] = acc[rt][tt][r];
        }
      }
    }
}

// ---------------------------------------------------------------------------------
// Packed math on MFMA: quant::matmul's int8 path (quant/mod.rs:223-304, the q*_dot
// kernels :398-621) for prefill-sized calls, the arithmetic of Weight::Packed under
// mmap = true.
//
// The reference splits every row dot into sub-blocks (32 values for Q4_K/Q5_K/Q8_0, 16
// for Q6_K/Q3_K/Q2_K), takes each sub-block's integer dot of the raw quants with the
// int8 activations, and adds one float term per sub-block to the row sum, in K order:
//   Q4_K, Q5_K, Q2_K:  acc += xs * ((d*sc) * dot - (dmin*m) * sum)
//   Q6_K:              acc += ((xs * d) * sc) * dot      (dot over q - 32)
//   Q3_K:              acc += (xs * (d*(sc-32))) * dot   (dot over q - 4*(1-hbit))
//   Q8_0:              acc += (ws * xs) * dot
// Here the integer dots come from fp16 MFMAs: the raw quants and the int8 activation
// codes are exact fp16 values and every partial sum is an integer below 2^24, so the
// f32 result of a sub-block's MFMA (one K16 step for 16-wide sub-blocks, two for
// 32-wide) is the reference's dot exactly. The float term is then evaluated per (row,
// token) exactly as the reference writes it and added in K order. With the whole K
// range in one workgroup (gate/up) the row sums are the reference's bit for bit, so h
// and its int8 requantisation are too; the down product splits K into slices that the
// combine adds in order (outputs then within rtol 1e-3 / atol 1e-4).
//
// Inputs: the activation codes in slot order as fp16 ([nk][K]), and the per-token
// factors transposed, [K/32][nkp] scales and [K/SW][nkp] sums (nkp >= nk + 64 so a
// token tile's 64 slots are always in bounds). Gate/up writes h's codes, scales and
// sums the same way for the down product.
// ---------------------------------------------------------------------------------
template <int QT> struct PQ;

// (d*sc, dmin*m) of sub-block SB from a Q4_K/Q5_K header (d, dmin, scales[12]).
template <int SB>
__device__ __forceinline__ void kq_rowf(u32x4 hd, float* rf) {
  const uint32_t s3[3] = {hd.y, hd.z, hd.w};
  uint32_t sc, m;
  scale_min_k4(s3, SB, sc, m);
  rf[0] = f16v(hd.x) * (float)sc;
  rf[1] = f16v(hd.x >> 16) * (float)m;
}

// Sub-block width SBW, activation-sum width SWS (0: the dot's operand carries the
// offset, or the type has no min term), and the per-row factors of sub-block SB of the
// unit staged in chunk C: rf[0], rf[1] as the term below reads them.
template <> struct PQ<Q4_K> {
  static constexpr int QT = Q4_K, SBW = 32, SWS = 32;
  template <int C, int S>
  static __device__ __forceinline__ half8 qfrag(const uint8_t* row, uint32_t h) {
    constexpr int sb = S / 2;
    constexpr bool high = sb & 1;
    u32x2 q = ld8(pf_at<QT, C, 16 + 32 * (sb / 2) + 16 * (S % 2)>(row) + 8 * h);
    const uint32_t mask = high ? 0xf0f0f0f0u : 0x0f0f0f0fu;
    q.x &= mask;
    q.y &= mask;
    // the quants as fp16 subnormals, q * 2^-24 (a high nibble in place, 16q * 2^-24): the
    // sub-block's dot comes out as dot * 2^-24 (2^-20), exact, and rowf scales d * sc by
    // the inverse power of two, so (d * sc) * dot is the same single rounding
    return bytes_sub(q);
  }
  template <int C, int SB>
  static __device__ __forceinline__ void rowf(const uint8_t* row, float* rf) {
    kq_rowf<SB>(ld16(pf_at<QT, C, 0>(row)), rf);
    rf[0] *= (SB & 1) ? 0x1p20f : 0x1p24f;
  }
  static __device__ __forceinline__ float term(float dot, const float* rf, float xs, float s) {
    return xs * (rf[0] * dot - rf[1] * s);
  }
};

template <> struct PQ<Q5_K> {
  static constexpr int QT = Q5_K, SBW = 32, SWS = 32;
  template <int C, int S>
  static __device__ __forceinline__ half8 qfrag(const uint8_t* row, uint32_t h) {
    constexpr int sb = S / 2;
    const u32x2 qh = ld8(pf_at<QT, C, 16 + 16 * (S % 2)>(row) + 8 * h);
    const u32x2 ql = ld8(pf_at<QT, C, 48 + 32 * (sb / 2) + 16 * (S % 2)>(row) + 8 * h);
    u32x2 b;
#pragma unroll
    for (int d = 0; d < 2; d++)
      b[d] = ((sb & 1 ? ql[d] >> 4 : ql[d]) & 0x0f0f0f0fu) | (((qh[d] >> sb) & 0x01010101u) << 4);
    return bytes_sub(b);  // q * 2^-24, as for Q4_K
  }
  template <int C, int SB>
  static __device__ __forceinline__ void rowf(const uint8_t* row, float* rf) {
    kq_rowf<SB>(ld16(pf_at<QT, C, 0>(row)), rf);
    rf[0] *= 0x1p24f;
  }
  static __device__ __forceinline__ float term(float dot, const float* rf, float xs, float s) {
    return xs * (rf[0] * dot - rf[1] * s);
  }
};

template <> struct PQ<Q6_K> {
  static constexpr int QT = Q6_K, SBW = 16, SWS = 0;
  template <int C, int S>
  static __device__ __forceinline__ half8 qfrag(const uint8_t* row, uint32_t h) {
    return Dec<Q6_K>::frag<C, S>(row, h);  // q - 32
  }
  template <int C, int SB>
  static __device__ __forceinline__ void rowf(const uint8_t* row, float* rf) {
    const u32x4 sc = ld16(pf_at<QT, C, 192>(row));
    rf[0] = f16v(ld16(pf_at<QT, C, 208>(row)).x);
    rf[1] = (float)(int8_t)((sc[SB / 4] >> (8 * (SB % 4))) & 0xffu);
  }
  static __device__ __forceinline__ float term(float dot, const float* rf, float xs, float) {
    return xs * rf[0] * rf[1] * dot;
  }
};

template <> struct PQ<Q3_K> {
  static constexpr int QT = Q3_K, SBW = 16, SWS = 0;
  template <int C, int S>
  static __device__ __forceinline__ half8 qfrag(const uint8_t* row, uint32_t h) {
    const u32x2 b = q3s_step<C, S>(row, h);  // q2 + 4 * hbit in [0, 7]; the quant is b - 4
    return bytes_fma(b, h2s((_Float16)1.0f), h2s((_Float16)-1028.0f));
  }
  template <int C, int SB>
  static __device__ __forceinline__ void rowf(const uint8_t* row, float* rf) {
    const u32x4 tl = ld16(pf_at<QT, C, 96>(row));  // scales[12] | d
    uint32_t sc4[4];
    q3k_scales(tl.x, tl.y, tl.z, sc4);
    const int scs = (int)(int8_t)((sc4[SB / 4] >> (8 * (SB % 4))) & 0xffu) - 32;
    rf[0] = f16v(tl.w) * (float)scs;
  }
  static __device__ __forceinline__ float term(float dot, const float* rf, float xs, float) {
    return xs * rf[0] * dot;
  }
};

template <> struct PQ<Q2_K> {
  static constexpr int QT = Q2_K, SBW = 16, SWS = 16;
  template <int C, int S>
  static __device__ __forceinline__ half8 qfrag(const uint8_t* row, uint32_t h) {
    constexpr int n = S / 8, j4 = (S % 8) / 2;
    const u32x2 qs = ld8(pf_at<QT, C, 16 + 32 * n + 16 * (S % 2)>(row) + 8 * h);
    u32x2 b;
#pragma unroll
    for (int d = 0; d < 2; d++) b[d] = (qs[d] >> (2 * j4)) & 0x03030303u;
    return bytes_sub(b);  // q * 2^-24, as for Q4_K
  }
  template <int C, int SB>
  static __device__ __forceinline__ void rowf(const uint8_t* row, float* rf) {
    const u32x4 scb = ld16(pf_at<QT, C, 0>(row));
    const uint32_t dd = ld16(pf_at<QT, C, 80>(row)).x;
    const uint32_t sc = (scb[SB / 4] >> (8 * (SB % 4))) & 0xffu;
    rf[0] = f16v(dd) * (float)(sc & 15u) * 0x1p24f;
    rf[1] = f16v(dd >> 16) * (float)(sc >> 4);
  }
  static __device__ __forceinline__ float term(float dot, const float* rf, float xs, float s) {
    return xs * (rf[0] * dot - rf[1] * s);
  }
};

template <> struct PQ<Q8_0> {
  static constexpr int QT = Q8_0, SBW = 32, SWS = 0;
  template <int C, int S>
  static __device__ __forceinline__ half8 qfrag(const uint8_t* row, uint32_t h) {
    return Dec<Q8_0>::frag<C, S>(row, h);  // the int8 quants
  }
  template <int C, int SB>
  static __device__ __forceinline__ void rowf(const uint8_t* row, float* rf) {
    rf[0] = f16v(ld16(pf_at<QT, C, 0>(row))[SB / 2] >> (16 * (SB % 2)));
  }
  static __device__ __forceinline__ float term(float dot, const float* rf, float xs, float) {
    return rf[0] * xs * dot;
  }
};

template <int QT> constexpr bool pq_type() {
  return QT == Q4_K || QT == Q5_K || QT == Q6_K || QT == Q3_K || QT == Q2_K || QT == Q8_0;
}

struct PqArgs {
  const ExpertWork* work;
  const uint32_t* ptile;
  const _Float16* in;   // [nk][K] activation codes
  const float* ins;     // [K/32][nkp] activation scales
  const float* insum;   // [K/SWS][nkp] activation sums (types with SWS)
  uint32_t nk, nkp, K, rows;
  // h dequantised (scale * q of its int8 requantisation) as fp16 hi/lo planes [2][nk][rows],
  // and its sums over swf rows as hi/lo planes [2][nk][rows/swf] (swf 0: none): the input
  // of the f32-math down product (k_pf)
  _Float16* outf;
  _Float16* outfs;
  uint32_t swf;
};

template <int QT>
__global__ void __launch_bounds__(64 * PF<QT>::NW) k_pq(PqArgs a) {
  using T = PF<QT>;
  using Q = PQ<QT>;
  constexpr int NW = T::NW, NT = 64 * NW;
  constexpr int KC = T::KC, NCK = KC / 8, NPC = T::NPC, NCH = T::EU / KC, SPC = KC / 16;
  constexpr int U = UT_<QT>::U, NP = U / 16;
  constexpr int SPS = Q::SBW / 16;                       // K16 steps per sub-block
  constexpr int NXS = KC / 32, NSM = Q::SWS ? KC / Q::SWS : 0;  // token factor rows per chunk
  constexpr uint32_t WROWS = 32 * NW;
  constexpr uint32_t WBYTES = NW * NPC * 1024, XBYTES = kPfTok * KC * 2, TBYTES = (NXS + NSM) * kPfTok * 4;
  constexpr uint32_t BUF = WBYTES + XBYTES + TBYTES;
  constexpr int NX = (int)kPfTok * NCK / NT;              // activation loads per thread per chunk
  static_assert(NX >= 1 && (int)kPfTok * NCK % NT == 0, "activation staging");
  static_assert(2 * BUF <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * BUF];

  uint32_t bx, by;
  pf_block(bx, by);
  const uint32_t pt = a.ptile[by];
  if (pt == ~0u) return;
  const ExpertWork* W = a.work + (pt >> 16);
  const uint32_t t0 = (pt & 0xffffu) * kPfTok;
  const uint32_t m = min(kPfTok, W->m - t0), s0 = W->s0 + t0;
  const uint32_t tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t K = a.K, nunit = K / T::EU;
  const uint32_t u0 = 0, u1 = nunit;

  // NW/2 gate tiles then NW/2 up tiles of 64 rows; wave w owns rows 32 (w % 2) .. of gate
  // tile w / 2 (rt = 0) and of the same up tile (rt = 1)
  const size_t tile_bytes = (size_t)nunit * kTileRows * U;
  const uint8_t* m_lo = W->w[0] + (NW / 2) * bx * tile_bytes;
  const uint8_t* m_hi = W->w[1] + (NW / 2) * bx * tile_bytes;
  uint32_t row[2];
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const uint32_t tm = rt * (NW / 2) + wave / 2, i = 32 * (wave % 2) + l32;
    row[rt] = (tm * NPC * 64 + i) * 16;
  }
  const uint32_t xrow = l32 * NCK * 16;
  uint32_t tsw = (l32 % NCK) * 16;

  auto stage = [&](uint32_t u, auto cc, uint32_t b) {
    constexpr int C = decltype(cc)::value;
    uint8_t* wb = lds + b * BUF;
    uint8_t* xb = wb + WBYTES;
    uint8_t* tb = xb + XBYTES;
#pragma unroll
    for (int j = 0; j < NPC; j++) {
      const uint32_t wq = NW * j + wave, tm = wq / NPC, pc = wq % NPC;
      const uint8_t* src = (tm < NW / 2 ? m_lo : m_hi) + (tm % (NW / 2)) * tile_bytes;
      lds_load16(src + ((size_t)u * NP + (uint32_t)T::piece(C, (int)pc)) * 1024 + lane * 16, wb + 1024 * wq);
    }
    // activation codes: item (token t, 16-byte column c at position c ^ (t % NCK))
    constexpr uint32_t RW = 64 / NCK;
    const uint32_t k0 = u * T::EU + C * KC;
#pragma unroll
    for (int j = 0; j < NX; j++) {
      const uint32_t wq = NW * j + wave;
      const uint32_t t = (RW * wq) % kPfTok + lane / NCK, c = (lane % NCK) ^ (t % NCK), tc = min(t, m - 1);
      lds_load16(a.in + ((size_t)(s0 + tc) * K + k0 + 8 * c), xb + 1024 * wq);
    }
    // token factors: row r of the chunk (scales, then sums) = 64 floats of slots s0..
#pragma unroll
    for (int j = 0; j < (NXS + NSM + NW - 1) / NW; j++) {
      const uint32_t r = NW * j + wave;
      if (r < (uint32_t)(NXS + NSM)) {
        const float* src = r < (uint32_t)NXS ? a.ins + (size_t)(k0 / 32 + r) * a.nkp
                                             : a.insum + (size_t)(k0 / (Q::SWS ? Q::SWS : 1) + r - NXS) * a.nkp;
        __builtin_amdgcn_global_load_lds(src + s0 + lane, (__attribute__((address_space(3))) void*)(tb + 256 * r), 4,
                                         0, 0);
      }
    }
  };

  f32x16 acc[2][2], P[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = P[i][j][r] = 0.0f;
  const f32x16 zero = acc[0][0];
  const bool two = m > 32;  // the second 32-token tile holds tokens

  if (u0 < u1) stage(u0, std::integral_constant<int, 0>{}, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (uint32_t u = u0; u < u1; u++) {
    static_for<NCH>([&](auto cc) {
      constexpr int C = decltype(cc)::value;
      const uint32_t b = (NCH % 2 == 0) ? (uint32_t)(C % 2) : ((u - u0) * NCH + C) % 2;
      if constexpr (C + 1 < NCH) {
        stage(u, std::integral_constant<int, C + 1>{}, b ^ 1);
      } else {
        if (u + 1 < u1) stage(u + 1, std::integral_constant<int, 0>{}, b ^ 1);
      }
      const uint8_t* wb = lds + b * BUF;
      const uint8_t* xb = wb + WBYTES;
      const float* tf = reinterpret_cast<const float*>(xb + XBYTES);
      asm volatile("" : "+v"(tsw));
      static_for<SPC>([&](auto ss) {
        constexpr int SL = decltype(ss)::value, S = C * SPC + SL;
        half8 bw[2], ax[2];
#pragma unroll
        for (int rt = 0; rt < 2; rt++) bw[rt] = Q::template qfrag<C, S>(wb + row[rt], h);
        const uint32_t pos = ((2 * SL + h) * 16) ^ tsw;
#pragma unroll
        for (int tt = 0; tt < 2; tt++) ax[tt] = *reinterpret_cast<const half8*>(xb + xrow + pos + 32 * tt * NCK * 16);
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
          P[rt][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[0], bw[rt], S % SPS == 0 ? zero : P[rt][0], 0, 0, 0);
          if (two)
            P[rt][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[1], bw[rt], S % SPS == 0 ? zero : P[rt][1], 0, 0, 0);
        }
        if constexpr ((S + 1) % SPS == 0) {
          // sub-block SB closes: its term for every (row, token), added in K order
          constexpr int SB = S / SPS;
          constexpr int EX = SL * 16 / 32, ES = Q::SWS ? SL * 16 / (Q::SWS ? Q::SWS : 1) : 0;
          float rf[2][2];
#pragma unroll
          for (int rt = 0; rt < 2; rt++) Q::template rowf<C, SB>(wb + row[rt], rf[rt]);
#pragma unroll
          for (int tt = 0; tt < 2; tt++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
              if (32 * tt + 8 * j < m) {
                const uint32_t t4 = 32 * tt + 8 * j + 4 * h;
                const float4 xs4 = *reinterpret_cast<const float4*>(tf + EX * kPfTok + t4);
                float4 s4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if constexpr (Q::SWS != 0) s4 = *reinterpret_cast<const float4*>(tf + (NXS + ES) * kPfTok + t4);
                const float xv[4] = {xs4.x, xs4.y, xs4.z, xs4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                  for (int rt = 0; rt < 2; rt++) {
                    const int r = 4 * j + i;
                    acc[rt][tt][r] = acc[rt][tt][r] + Q::term(P[rt][tt][r], rf[rt], xv[i], sv[i]);
                  }
              }
            }
          }
        }
      });
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    });
  }

  // epilogue
#pragma unroll
  for (int tt = 0; tt < 2; tt++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const uint32_t t = 32 * tt + 8 * (r / 4) + 4 * h + (r % 4);
      {
        // h = silu(g) * u, then quantised per 32 rows (the 32 lanes of this half) with
        // quant_wave's arithmetic (quant/mod.rs:331-345)
        const uint32_t fr = bx * WROWS + 32 * wave + l32;
        const float hv = swiglu(acc[0][tt][r], acc[1][tt][r]);
        float am = fmaxf(0.0f, fabsf(hv));
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
        const float scale = fdiv(am, 127.0f);
        const float inv = scale > 0.0f ? fdiv(1.0f, scale) : 0.0f;
        const float rq = roundf(hv * inv);
        const int qi = (rq != rq) ? 0 : rq < -127.0f ? -127 : rq > 127.0f ? 127 : (int)rq;
        // the dequantised activation the reference's down dot sees, scale * q, as fp16
        // hi/lo planes for the f32-math MFMA product (k_pf), and its sums over swf rows
        const float xv = scale * (float)qi;
        const _Float16 hi = (_Float16)xv, lo = (_Float16)(xv - (float)hi);
        float sf = xv;  // offsets fixed at compile time, so the 32 reductions overlap
        if (a.swf) {
#pragma unroll
          for (int o = 1; o <= 8; o <<= 1) sf += __shfl_xor(sf, o, 64);
          if (a.swf == 32) sf += __shfl_xor(sf, 16, 64);
        }
        if (t < m) {
          const size_t o = (size_t)(s0 + t) * a.rows + fr;
          a.outf[o] = hi;
          a.outf[o + (size_t)a.nk * a.rows] = lo;
          if (a.swf && (l32 % a.swf) == 0) {
            const uint32_t ns = a.rows / a.swf;
            const size_t os = (size_t)(s0 + t) * ns + fr / a.swf;
            const _Float16 shi = (_Float16)sf;
            a.outfs[os] = shi;
            a.outfs[os + (size_t)a.nk * ns] = (_Float16)(sf - (float)shi);
          }
        }
      }
    }
}

template <int QT>
uint32_t pf_rows(bool gu) {
  if constexpr (QT == F32) {
    return 0;
  } else {
    return 32u * PF<QT>::NW * (gu ? 1u : 2u);
  }
}

// The packed-math gate/up product (k_pq) of this block type; its down product is k_pf's.
template <int QT>
hipError_t pq_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  if constexpr (!pq_type<QT>()) {
    return hipErrorNotSupported;
  } else {
    if (L.f % pf_rows<QT>(true) || L.d % PF<QT>::EU) return hipErrorInvalidValue;
    PqArgs a{};
    a.work = B.work;
    a.ptile = B.ptile;
    a.in = B.xh;
    a.ins = B.qxs;
    a.insum = B.qxsum;
    a.nk = n * L.k;
    a.nkp = B.nkp;
    a.K = L.d;
    a.rows = L.f;
    a.outf = B.hh;
    a.outfs = B.hsh;
    a.swf = pf_sum_width(L.qt_down);
    hipLaunchKernelGGL((k_pq<QT>), dim3(L.f / pf_rows<QT>(true), B.ptile_cap), dim3(64 * PF<QT>::NW), 0, st, a);
    return hipGetLastError();
  }
}

template <int QT>
hipError_t prefill_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  if constexpr (QT == F32) {
    return hipErrorNotSupported;
  } else {
    if (L.f % pf_rows<QT>(true)) return hipErrorInvalidValue;
    PfArgs a{};
    a.work = B.work;
    a.ptile = B.ptile;
    a.in = B.xh;
    a.ins = B.xsh;
    a.nk = n * L.k;
    a.K = L.d;
    a.rows = L.f;
    a.out = B.hh;
    a.swo = pf_sum_width(L.qt_down);
    a.outs = a.swo ? B.hsh : nullptr;
    hipLaunchKernelGGL((k_pf<QT, true>), dim3(L.f / pf_rows<QT>(true), B.ptile_cap), dim3(64 * PF<QT>::NW), 0, st,
                       a);
    return hipGetLastError();
  }
}

// The down product's K slices: enough workgroups for about four rounds of one per CU
// over the token tiles the call can have, each slice keeping at least 8 units.
template <int QT>
uint32_t prefill_down_slices(const LayerDev& L, const FwdBufs& B) {
  if constexpr (QT == F32) {
    return 1;
  } else {
    const uint32_t tiles = (L.d / pf_rows<QT>(false)) * B.ptile_cap, nunit = L.f / PF<QT>::EU;
    uint32_t ks = (4 * 256 + tiles - 1) / tiles;
    ks = min(ks, max(1u, nunit / 8));
    return max(1u, min(ks, kMaxKsg));
  }
}

template <int QT>
hipError_t prefill_down(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st) {
  if constexpr (QT == F32) {
    return hipErrorNotSupported;
  } else {
    if (L.d % pf_rows<QT>(false) || ksg < 1 || ksg > kMaxKsg) return hipErrorInvalidValue;
    PfArgs a{};
    a.work = B.work;
    a.ptile = B.ptile;
    a.in = B.hh;
    a.ins = B.hsh;
    a.nk = n * L.k;
    a.K = L.f;
    a.rows = L.d;
    const uint32_t nunit = L.f / PF<QT>::EU;
    a.upk = (nunit + ksg - 1) / ksg;
    a.y = B.y;
    hipLaunchKernelGGL((k_pf<QT, false>), dim3(L.d / pf_rows<QT>(false), B.ptile_cap, ksg), dim3(64 * PF<QT>::NW),
                       0, st, a);
    return hipGetLastError();
  }
}

template uint32_t prefill_down_slices<GMOE_QT>(const LayerDev&, const FwdBufs&);
template hipError_t prefill_gateup<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, hipStream_t);
template hipError_t prefill_down<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, uint32_t, hipStream_t);
template hipError_t pq_gateup<GMOE_QT>(const LayerDev&, const FwdBufs&, uint32_t, hipStream_t);

}  // namespace gmoe
