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
#include "gmoe_device.h"

#include <math.h>

#include <type_traits>
#include <utility>

namespace gmoe {


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
// Staging: raw packed rows -> tiled layout. One thread writes one 16-byte piece,
// gathering its bytes through unit_src_byte.
// ---------------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
k_tile_rows(uint32_t qt, const uint8_t* __restrict__ raw, uint32_t r0, uint32_t nrows, uint32_t rows, uint32_t cols,
            uint8_t* __restrict__ dst, uint64_t npieces) {
  const uint64_t pi = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pi >= npieces) return;
  Unit un;
  unit_of(qt, &un);
  const uint32_t nblk = row_blocks(un, cols), nunit = row_units(un, cols), np = un.U / 16;
  const uint64_t rb = (uint64_t)nblk * un.B;
  const uint32_t i = (uint32_t)(pi % kTileRows);
  const uint64_t rest = pi / kTileRows;
  const uint32_t p = (uint32_t)(rest % np);
  const uint64_t tu = rest / np;  // tile-local unit index over the chunk's tiles
  const uint32_t u = (uint32_t)(tu % nunit), lt = (uint32_t)(tu / nunit);
  const uint32_t rl = lt * kTileRows + i, row = r0 + rl;
  uint32_t v[4] = {0, 0, 0, 0};
  if (rl < nrows && row < rows) {
    const uint8_t* src = raw + (uint64_t)rl * rb;
    for (uint32_t b = 0; b < 16; b++) {
      int64_t s = unit_src_byte(qt, un, nblk, u, p * 16 + b);
      if (s >= 0) v[b / 4] |= (uint32_t)src[s] << (8 * (b % 4));
    }
  }
  const uint64_t tile = r0 / kTileRows + lt;
  uint8_t* o = dst + ((tile * nunit + u) * np + p) * 1024 + (uint64_t)i * 16;
  *reinterpret_cast<uint4*>(o) = make_uint4(v[0], v[1], v[2], v[3]);
}

hipError_t launch_tile_rows(uint32_t qt, const uint8_t* raw, uint32_t r0, uint32_t nrows, uint32_t rows,
                            uint32_t cols, uint8_t* dst, hipStream_t st) {
  Unit un;
  if (!unit_of(qt, &un) || r0 % kTileRows) return hipErrorInvalidValue;
  const uint64_t tiles = (nrows + kTileRows - 1) / kTileRows;
  const uint64_t npieces = tiles * row_units(un, cols) * (un.U / 16) * kTileRows;
  if (!npieces) return hipSuccess;
  hipLaunchKernelGGL(k_tile_rows, dim3((unsigned)((npieces + 255) / 256)), dim3(256), 0, st, qt, raw, r0, nrows,
                     rows, cols, dst, npieces);
  return hipGetLastError();
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
// Expert-product dispatch by block type (the kernels live in gmoe_units.hip)
// ---------------------------------------------------------------------------------

// K groups of the down product: enough workgroups for two waves per SIMD (1024
// workgroups of kDnKS = 2 waves on 256 CUs), each wave keeping at least 4 units.
uint32_t down_ksg(const LayerDev& L, uint32_t n) {
  Unit un;
  if (!unit_of(L.qt_down, &un)) return 1;
  const uint32_t tiles = (L.d + kTileRows - 1) / kTileRows, ymax = min(L.ne, n * L.k);
  const uint32_t ksg = (1024 + tiles * ymax - 1) / (tiles * ymax);
  const uint32_t cap = max(1u, row_units(un, L.f) / (kDnKS * 4));
  return max(1u, min(min(ksg, cap), kMaxKsg));
}

hipError_t launch_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  switch (L.qt_gate) {
#define GU(T) case T: return units_gateup<T>(L, B, n, st);
    GU(Q4_K) GU(Q5_K) GU(Q6_K) GU(Q3_K) GU(Q2_K) GU(Q8_0) GU(Q4_0) GU(F16) GU(F32)
#undef GU
  }
  return hipErrorInvalidValue;
}

hipError_t launch_down(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  const uint32_t ksg = down_ksg(L, n);
  switch (L.qt_down) {
#define DN(T) case T: return units_down<T>(L, B, n, ksg, st);
    DN(Q4_K) DN(Q5_K) DN(Q6_K) DN(Q3_K) DN(Q2_K) DN(Q8_0) DN(Q4_0) DN(F16) DN(F32)
#undef DN
  }
  return hipErrorInvalidValue;
}

}  // namespace gmoe
