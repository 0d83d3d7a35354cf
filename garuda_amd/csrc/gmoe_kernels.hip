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
                                                   uint32_t* __restrict__ sums, int kind, int32_t off) {
  uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblk) return;
  float v[32];
  const float4* p = reinterpret_cast<const float4*>(x + (size_t)b * 32);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float4 t = p[i];
    v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
  quant32(v, q + (size_t)b * 32, s + b, sums, b, kind, off);
}

hipError_t launch_quant_act(const float* x, uint32_t n_tok, uint32_t K, int8_t* q, float* s,
                            uint32_t* sums, uint32_t reader, hipStream_t st) {
  uint32_t nblk = n_tok * (K / 32);
  hipLaunchKernelGGL(k_quant_act, dim3((nblk + 255) / 256), dim3(256), 0, st, x, nblk, q, s, sums,
                     sum_kind_of(reader), sum_offset_of(reader));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Routing. One workgroup per group of tokens; thread (token, expert) pairs compute the
// router logit as the reference's sequential f32 dot (simd/mod.rs:13-16: separate
// multiply and add, left to right, Iterator::sum starting at -0.0).
// ---------------------------------------------------------------------------------

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
        // the products of 16 float4 columns at a time, their loads issued together, then
        // added to the chain in order (the same sequential sum)
        constexpr uint32_t kRB = 16;
        const uint32_t n4 = d / 4;
        for (uint32_t j0 = 0; j0 < n4; j0 += kRB) {
          float4 a[kRB], h[kRB];
#pragma unroll
          for (uint32_t i = 0; i < kRB; i++) {
            const uint32_t j = min(j0 + i, n4 - 1);
            a[i] = wr[j];
            h[i] = hr[j];
          }
#pragma unroll
          for (uint32_t i = 0; i < kRB; i++) {
            if (j0 + i < n4) {
              const float p0 = a[i].x * h[i].x, p1 = a[i].y * h[i].y, p2 = a[i].z * h[i].z, p3 = a[i].w * h[i].w;
              acc = acc + p0;
              acc = acc + p1;
              acc = acc + p2;
              acc = acc + p3;
            }
          }
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
// exactly members[e] of llama/mod.rs:967-972 laid end to end. One workgroup of T
// threads; sm holds T + 3*ne + 2 words of LDS, whatever the number of pairs. Counts by
// LDS atomics, the active slots by rank of count, offsets by one wave's running scans,
// then every pair's slot = its expert's offset + the pairs of that expert before it
// (counted chunk of T pairs by chunk against an LDS copy of the chunk's ids, the counts
// of earlier chunks carried per expert). Every thread must call this.
__device__ void dispatch_block(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t* sm,
                               const uint32_t* ids, const float* wts) {
  const uint32_t ne = L.ne, k = L.k, nk = n * k, tid = threadIdx.x, T = blockDim.x;
  uint32_t* idl = sm;            // [T] ids of the chunk being placed
  uint32_t* cnt = sm + T;        // [ne] counts, then the running count of earlier chunks
  uint32_t* start = cnt + ne;    // [ne] offsets
  uint32_t* aidx = start + ne;   // [ne] active slot (~0u: inactive)
  uint32_t* tot = aidx + ne;     // [2] active experts, token tiles
  for (uint32_t e = tid; e < ne; e += T) cnt[e] = 0;
  __syncthreads();
  for (uint32_t p = tid; p < nk; p += T) atomicAdd(&cnt[ids[p]], 1u);
  __syncthreads();
  // active slot: experts by descending pair count, then ascending id, so that the expert
  // kernels' grids start the experts with the most tokens first
  for (uint32_t e = tid; e < ne; e += T) {
    const uint32_t c = cnt[e];
    uint32_t r = 0;
    if (c)
      for (uint32_t j = 0; j < ne; j++) {
        const uint32_t cj = cnt[j];
        r += (cj > c || (cj == c && j < e)) ? 1u : 0u;
      }
    aidx[e] = c ? r : ~0u;
  }
  __syncthreads();
  if (tid < 64) {  // running scans over the experts, 64 at a time
    const uint32_t lane = tid;
    uint32_t off = 0, na = 0, nt = 0;
    for (uint32_t e0 = 0; e0 < ne; e0 += 64) {
      const uint32_t e = e0 + lane;
      const uint32_t c = e < ne ? cnt[e] : 0u, act = c ? 1u : 0u;
      const uint32_t tl = B.ptile ? (c + kPfTok - 1) / kPfTok : 0u;
      uint32_t ic = c, ia = act, it = tl;  // inclusive scans
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t vc = __shfl_up(ic, o, 64), va = __shfl_up(ia, o, 64), vt = __shfl_up(it, o, 64);
        if (lane >= (uint32_t)o) {
          ic += vc;
          ia += va;
          it += vt;
        }
      }
      if (e < ne) {
        start[e] = off + ic - c;
        if (act && B.ptile) {
          const uint32_t a = aidx[e], t0 = nt + it - tl;
          for (uint32_t t = 0; t < tl; t++) B.ptile[t0 + t] = (a << 16) | t;
        }
      }
      off += __shfl(ic, 63, 64);
      na += __shfl(ia, 63, 64);
      nt += __shfl(it, 63, 64);
    }
    if (lane == 0) {
      tot[0] = na;
      tot[1] = nt;
      B.offsets[ne] = off;
      B.active[0] = na;
    }
  }
  __syncthreads();
  const uint32_t na = tot[0], nt = tot[1];
  for (uint32_t e = tid; e < ne; e += T) {
    B.offsets[e] = start[e];
    const uint32_t a = aidx[e];
    if (a != ~0u) {
      B.active[1 + a] = e;
      if (B.work) {
        ExpertWork& W = B.work[a];
        for (int q = 0; q < 3; q++) W.w[q] = L.eptr[q * ne + e];
        W.e = e;
        W.s0 = start[e];
        W.m = cnt[e];
      }
    }
  }
  if (B.work)
    for (uint32_t a = na + tid; a < ne; a += T) B.work[a].m = 0;
  if (B.ptile)
    for (uint32_t i = nt + tid; i < B.ptile_cap; i += T) B.ptile[i] = ~0u;
  __syncthreads();
  for (uint32_t e = tid; e < ne; e += T) cnt[e] = 0;  // now: pairs placed by earlier chunks
  __syncthreads();
  for (uint32_t c0 = 0; c0 < nk; c0 += T) {
    const uint32_t p = c0 + tid;
    if (p < nk) idl[tid] = ids[p];
    __syncthreads();
    uint32_t e = ~0u, pos = 0;
    if (p < nk) {
      e = idl[tid];
      uint32_t r = 0;
      for (uint32_t q = 0; q < tid; q++) r += idl[q] == e;
      pos = start[e] + cnt[e] + r;
    }
    __syncthreads();  // every pair of the chunk has read the carried counts and the chunk's ids
    if (p < nk) {
      atomicAdd(&cnt[e], 1u);
      B.slot_tok[pos] = p / k;
      B.slot_w[pos] = wts[p];
      B.slot_rank[pos] = p % k;
      B.slot_of[p] = pos;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------
// Wide front end (64 < ne <= 64 * kWideEPL experts): one workgroup of one wave per token
// gates it (lane l holds experts l, l + 64, ...: gate_wave_wide) from the given logits or
// the reference's sequential dots and quantises its activations; a second launch
// dispatches every pair (dispatch_par).
// ---------------------------------------------------------------------------------
constexpr int kWideEPL = 4, kWideWaves = 8, kWideThreads = 64 * kWideWaves;

// The stable counting sort of dispatch_block by one workgroup of W waves, each pair's
// position found without a scan over the pairs before it: per chunk of 64 pairs (a wave)
// the experts present are peeled one at a time by ballot, which gives each pair its rank
// among its expert's pairs in the chunk and the chunk's count per expert; the chunks of
// a round (W of them, in pair order) then add their counts per expert in chunk order to
// the running position. sm holds (4 + W) * ne + 2 words. Every thread must call this.
__device__ void dispatch_par(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t* sm) {
  const uint32_t ne = L.ne, k = L.k, nk = n * k, tid = threadIdx.x, T = blockDim.x, W = T / 64;
  const uint32_t wave = tid >> 6, lane = tid & 63;
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t* cnt = sm;             // [ne]
  uint32_t* start = cnt + ne;     // [ne]
  uint32_t* aidx = start + ne;    // [ne]
  uint32_t* run = aidx + ne;      // [ne] next position per expert
  uint32_t* lh = run + ne;        // [W][ne] a round's per-chunk counts, then bases
  uint32_t* tot = lh + W * ne;    // [2]
  // the first kParRounds rounds' pairs are read once, all loads issued together, and kept
  // for both the counts and the placement
  constexpr uint32_t kParRounds = 4;
  uint32_t cid[kParRounds];
  float cwt[kParRounds];
#pragma unroll
  for (uint32_t r = 0; r < kParRounds; r++) {
    const uint32_t p = r * T + tid;
    cid[r] = p < nk ? B.ids[p] : ~0u;
    cwt[r] = p < nk ? B.w[p] : 0.0f;
  }
  for (uint32_t e = tid; e < ne; e += T) cnt[e] = 0;
  __syncthreads();
#pragma unroll
  for (uint32_t r = 0; r < kParRounds; r++)
    if (cid[r] != ~0u) atomicAdd(&cnt[cid[r]], 1u);
  for (uint32_t p = kParRounds * T + tid; p < nk; p += T) atomicAdd(&cnt[B.ids[p]], 1u);
  __syncthreads();
  for (uint32_t e = tid; e < ne; e += T) {  // active slot: descending count, then id
    const uint32_t c = cnt[e];
    uint32_t r = 0;
    if (c)
#pragma unroll 8
      for (uint32_t j = 0; j < ne; j++) {
        const uint32_t cj = cnt[j];
        r += (cj > c || (cj == c && j < e)) ? 1u : 0u;
      }
    aidx[e] = c ? r : ~0u;
  }
  __syncthreads();
  if (wave == 0) {  // running scans over the experts, 64 at a time
    uint32_t off = 0, na = 0, nt = 0;
    for (uint32_t e0 = 0; e0 < ne; e0 += 64) {
      const uint32_t e = e0 + lane;
      const uint32_t c = e < ne ? cnt[e] : 0u, act = c ? 1u : 0u;
      const uint32_t tl = B.ptile ? (c + kPfTok - 1) / kPfTok : 0u;
      uint32_t ic = c, ia = act, it = tl;
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t vc = __shfl_up(ic, o, 64), va = __shfl_up(ia, o, 64), vt = __shfl_up(it, o, 64);
        if (lane >= (uint32_t)o) {
          ic += vc;
          ia += va;
          it += vt;
        }
      }
      if (e < ne) {
        start[e] = off + ic - c;
        if (act && B.ptile) {
          const uint32_t a = aidx[e], t0 = nt + it - tl;
          for (uint32_t t = 0; t < tl; t++) B.ptile[t0 + t] = (a << 16) | t;
        }
      }
      off += __shfl(ic, 63, 64);
      na += __shfl(ia, 63, 64);
      nt += __shfl(it, 63, 64);
    }
    if (lane == 0) {
      tot[0] = na;
      tot[1] = nt;
      B.offsets[ne] = off;
      B.active[0] = na;
    }
  }
  __syncthreads();
  const uint32_t na = tot[0], nt = tot[1];
  for (uint32_t e = tid; e < ne; e += T) {
    B.offsets[e] = start[e];
    run[e] = start[e];
    const uint32_t a = aidx[e];
    if (a != ~0u) {
      B.active[1 + a] = e;
      if (B.work) {
        ExpertWork& Wk = B.work[a];
        for (int q = 0; q < 3; q++) Wk.w[q] = L.eptr[q * ne + e];
        Wk.e = e;
        Wk.s0 = start[e];
        Wk.m = cnt[e];
      }
    }
  }
  if (B.work)
    for (uint32_t a = na + tid; a < ne; a += T) B.work[a].m = 0;
  if (B.ptile)
    for (uint32_t i = nt + tid; i < B.ptile_cap; i += T) B.ptile[i] = ~0u;
  for (uint32_t c0 = 0, rd = 0; c0 < nk; c0 += T, rd++) {
    for (uint32_t e = lane; e < ne; e += 64) lh[wave * ne + e] = 0;
    const uint32_t p = c0 + tid;
    uint32_t id = ~0u;
    float w = 0.0f;
    if (rd < kParRounds) {
#pragma unroll
      for (uint32_t r = 0; r < kParRounds; r++)
        if (r == rd) {
          id = cid[r];
          w = cwt[r];
        }
    } else if (p < nk) {
      id = B.ids[p];
      w = B.w[p];
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");  // the wave's zeros land before its counts
    // the lanes holding this lane's expert: one ballot per bit of the id (ids past the end
    // are ~0u and match only each other)
    uint64_t m = __ballot(id != ~0u);
    if (id == ~0u) m = ~m;
    for (uint32_t bit = 1; bit < ne; bit <<= 1) {
      const uint64_t b = __ballot((id & bit) != 0);
      m &= (id & bit) ? b : ~b;
    }
    const uint32_t lrank = (uint32_t)__popcll(m & below);
    if (id != ~0u && lrank == 0) lh[wave * ne + id] = (uint32_t)__popcll(m);
    __syncthreads();
    for (uint32_t e = tid; e < ne; e += T) {  // chunk bases in pair order
      uint32_t r = run[e];
      for (uint32_t v = 0; v < W; v++) {
        const uint32_t c = lh[v * ne + e];
        lh[v * ne + e] = r;
        r += c;
      }
      run[e] = r;
    }
    __syncthreads();
    if (id != ~0u) {
      const uint32_t pos = lh[wave * ne + id] + lrank;
      B.slot_tok[pos] = p / k;
      B.slot_w[pos] = w;
      B.slot_rank[pos] = p % k;
      B.slot_of[p] = pos;
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(64) k_front_wide(LayerDev L, FwdBufs B, uint32_t n, int quant) {
  __shared__ uint32_t gsc[64];  // gating scratch: 2k words (k <= 32)
  const uint32_t ne = L.ne, k = L.k, d = L.d, lane = threadIdx.x, t = blockIdx.x;
  const float* hs = B.hs + (size_t)t * d;
  // the quantiser's first block a lane (block `lane` of the row), loaded first so that its
  // latency hides behind the gating
  const uint32_t nblk = d / 32;
  const bool pre = quant && lane < nblk;
  float v0[32];
  if (pre) {
    const float4* src = reinterpret_cast<const float4*>(hs + (size_t)lane * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 t4 = src[i];
      v0[4 * i] = t4.x; v0[4 * i + 1] = t4.y; v0[4 * i + 2] = t4.z; v0[4 * i + 3] = t4.w;
    }
  }
  float x[kWideEPL];
#pragma unroll
  for (int j = 0; j < kWideEPL; j++) {
    const uint32_t e = 64 * j + lane;
    float acc = 0.0f;
    if (e < ne) {
      if (B.logits_in) {
        acc = B.logits_in[(size_t)t * ne + e];
      } else {  // simd/mod.rs:13-16: products added left to right from -0.0
        const float4* wr = reinterpret_cast<const float4*>(L.router + (size_t)e * d);
        const float4* hr = reinterpret_cast<const float4*>(hs);
        acc = -0.0f;
        for (uint32_t i = 0; i < d / 4; i++) {
          const float4 a = wr[i], h = hr[i];
          const float p0 = a.x * h.x, p1 = a.y * h.y, p2 = a.z * h.z, p3 = a.w * h.w;
          acc = acc + p0;
          acc = acc + p1;
          acc = acc + p2;
          acc = acc + p3;
        }
      }
      B.logits[(size_t)t * ne + e] = acc;
    }
    x[j] = acc;
  }
  uint32_t id;
  float w;
  gate_wave_wide<kWideEPL>(L.gating, ne, k, x, lane, &id, &w, gsc);
  if (lane < k) {
    B.ids[(size_t)t * k + lane] = id;
    B.w[(size_t)t * k + lane] = w;
  }
  if (pre) {
    const size_t gb = (size_t)t * nblk + lane;
    quant32(v0, B.xq + gb * 32, B.xs + gb, B.xsum, gb, sum_kind_of(L.qt_gate), sum_offset_of(L.qt_gate));
  }
  if (quant) {
    for (uint32_t b = lane + 64; b < nblk; b += 64) {
      float v[32];
      const float4* src = reinterpret_cast<const float4*>(hs + (size_t)b * 32);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float4 t4 = src[i];
        v[4 * i] = t4.x; v[4 * i + 1] = t4.y; v[4 * i + 2] = t4.z; v[4 * i + 3] = t4.w;
      }
      const size_t gb = (size_t)t * nblk + b;
      quant32(v, B.xq + gb * 32, B.xs + gb, B.xsum, gb, sum_kind_of(L.qt_gate), sum_offset_of(L.qt_gate));
    }
  }
}

// The dispatch alone (dispatch_par over the routing in memory), for ne <= kParExperts.
__global__ void __launch_bounds__(kWideThreads) k_dispatch_par(LayerDev L, FwdBufs B, uint32_t n) {
  extern __shared__ uint32_t dsm_par[];  // [(4 + kWideWaves) * ne + 2]
  dispatch_par(L, B, n, dsm_par);
}

hipError_t launch_dispatch_par(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  if (L.ne > kParExperts) return hipErrorInvalidValue;
  const size_t shm = ((4 + kWideWaves) * (size_t)L.ne + 2) * 4;
  static const bool attr =
      hipFuncSetAttribute((const void*)k_dispatch_par, hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024) ==
      hipSuccess;
  (void)attr;
  hipLaunchKernelGGL(k_dispatch_par, dim3(1), dim3(kWideThreads), shm, st, L, B, n);
  return hipGetLastError();
}

bool front_wide_ok(const LayerDev& L, uint32_t n) {
  return n >= 1 && L.ne > 64u && L.ne <= 64u * kWideEPL && L.k <= 32 && L.d % 32 == 0;
}

hipError_t launch_front_wide(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, hipStream_t st) {
  hipLaunchKernelGGL(k_front_wide, dim3(n), dim3(64), 0, st, L, B, n, quant);
  if (hipError_t e = hipGetLastError()) return e;
  return launch_dispatch_par(L, B, n, st);
}

constexpr uint32_t kDispatchThreads = 256;

__global__ void __launch_bounds__(kDispatchThreads) k_dispatch(LayerDev L, FwdBufs B, uint32_t n) {
  extern __shared__ uint32_t dsm_u32[];  // [kDispatchThreads + 3*ne + 2]
  dispatch_block(L, B, n, dsm_u32, B.ids, B.w);
}

// ---------------------------------------------------------------------------------
// Dispatch by one wave (ne <= 64: lane e holds expert e); its counts are cross-lane
// reductions, its positions running sums in index order.
// ---------------------------------------------------------------------------------

// Stable counting sort of the nk (token, rank) pairs by expert: members[e] of
// llama/mod.rs:967-972 laid end to end, as dispatch_block makes it. pair(p, &id, &w)
// reads pair p. Pairs go 64 at a time; per expert a ballot finds its pairs in the chunk
// and lane e keeps expert e's count, then its next free slot. Up to kWaveChunks chunks
// are read once, all loads issued together, and kept in registers for both passes (one
// memory round trip instead of two per chunk); longer lists are read chunk by chunk.
constexpr uint32_t kWaveChunks = 16;

template <class Ptr, class Pair>
__device__ void dispatch_wave(const FwdBufs& B, Ptr eptr, uint32_t ne, uint32_t k, uint32_t nk,
                              uint32_t lane, Pair pair, bool meta = true) {
  const uint64_t below = (1ull << lane) - 1ull;
  const bool cached = nk <= 64 * kWaveChunks;
  uint32_t cid[kWaveChunks];
  float cw[kWaveChunks];
  if (cached) {
#pragma unroll
    for (uint32_t c = 0; c < kWaveChunks; c++) {
      cid[c] = ~0u;
      cw[c] = 0.0f;
      if (64 * c + lane < nk) pair(64 * c + lane, &cid[c], &cw[c]);
    }
  }
  // f(c0, id, w) for every chunk in order, pair c0 + lane in (id, w) (id ~0u past the end)
  auto chunks = [&](auto f) {
    if (cached) {
#pragma unroll
      for (uint32_t c = 0; c < kWaveChunks; c++)
        if (64 * c < nk) f(64 * c, cid[c], cw[c]);
    } else {
      for (uint32_t c0 = 0; c0 < nk; c0 += 64) {
        uint32_t id = ~0u;
        float w = 0.0f;
        if (c0 + lane < nk) pair(c0 + lane, &id, &w);
        f(c0, id, w);
      }
    }
  };
  uint32_t cnt = 0;
  chunks([&](uint32_t, uint32_t id, float) {
    for (uint32_t e = 0; e < ne; e++) {
      const uint32_t c = (uint32_t)__popcll(__ballot(id == e));
      if (lane == e) cnt += c;
    }
  });
  uint32_t off = 0, run = 0;
  for (uint32_t e = 0; e < ne; e++) {
    if (lane == e) off = run;
    run += lane_u(cnt, e);
  }
  const uint64_t act = __ballot(lane < ne && cnt > 0);
  const uint32_t na = (uint32_t)__popcll(act);
  // active slot: experts by descending pair count, then ascending id. The expert
  // kernels' grids run the active slots in this order, so the experts with the most
  // tokens (the longest workgroups) start first and the short ones fill in behind them.
  uint32_t arank = 0;
  for (uint32_t e = 0; e < ne; e++) {
    const uint32_t ce = lane_u(cnt, e);
    arank += (ce > cnt || (ce == cnt && e < lane)) ? 1u : 0u;
  }
  if (lane < ne) {
    B.offsets[lane] = off;
    if (cnt > 0) {
      const uint32_t a = arank;
      B.active[1 + a] = lane;
      if (B.work) {
        ExpertWork& W = B.work[a];
        for (int p = 0; p < 3; p++) W.w[p] = eptr(p);
        W.e = lane;
        W.s0 = off;
        W.m = cnt;
      }
    }
    if (B.work && lane >= na) B.work[lane].m = 0;
  }
  if (lane == 0) {
    B.offsets[ne] = run;
    B.active[0] = na;
  }
  if (B.ptile) {  // token tiles of kPfTok per active expert, in slot order
    const uint32_t nt = (cnt + kPfTok - 1) / kPfTok;
    uint32_t t0 = 0, tr = 0;
    for (uint32_t e = 0; e < ne; e++) {
      if (lane == e) t0 = tr;
      tr += lane_u(nt, e);
    }
    if (lane < ne && cnt > 0) {
      const uint32_t a = arank;
      for (uint32_t t = 0; t < nt; t++) B.ptile[t0 + t] = (a << 16) | t;
    }
    for (uint32_t i = tr + lane; i < B.ptile_cap; i += 64) B.ptile[i] = ~0u;
  }
  chunks([&](uint32_t c0, uint32_t id, float w) {
    uint32_t pos = 0;
    const uint32_t p = c0 + lane;
    for (uint32_t e = 0; e < ne; e++) {
      const uint64_t m = __ballot(id == e);
      if (id == e) pos = lane_u(off, e) + (uint32_t)__popcll(m & below);
      if (lane == e) off += (uint32_t)__popcll(m);
    }
    if (id < ne) {  // pairs with id ~0u (no expert) are skipped
      B.slot_tok[pos] = p / k;
      if (meta) {
        B.slot_w[pos] = w;
        B.slot_rank[pos] = p % k;
        B.slot_of[p] = pos;
      }
    }
  });
}

// ---------------------------------------------------------------------------------
// Fused front end: router logits, gating, the int8 activation quantiser and the
// dispatch in one launch (ne <= 64 experts), tpw tokens a workgroup (front_tokens).
//
// A logit is the reference's sequential f32 dot (simd/mod.rs:13-16): products w*h, each
// rounded, added left to right from -0.0. Its latency is its d dependent adds, so wave
// 0 (lane l = token l / ne, expert l % ne: one chain per lane) does only those adds while
// eight producer waves make the products into LDS ahead of it. K is cut into sections as
// long as two LDS halves of [tpw * ne][section] allow, and the two sides meet at a
// barrier once per section: while wave 0 adds section s from one half, the producers
// fill the other with section s+1 (and quantise the tokens' activations during the last
// one). Wave 0 reads its products 32 at a time from two fixed register buffers, each
// batch fetched one batch ahead by an unconditional load, so it waits only for the batch
// it adds. Then wave w gates token w. The workgroup that finishes last (a device-wide
// counter taken after a release fence) does the dispatch over every token's routing and
// puts the counter back to zero.
// ---------------------------------------------------------------------------------

constexpr int kFrontExperts = 64, kFrontProdWaves = 8, kFrontThreads = 64 * (1 + kFrontProdWaves);
constexpr uint32_t kFrontProdBytes = 150 * 1024;  // both LDS halves of products (the rest: < 4 KB)
constexpr int kFrontItems = 12;                   // float4 products a producer lane has in flight
constexpr uint32_t kFrontMaxTok = 8;

// Tokens a workgroup: one until the workgroups would outnumber the CUs (the chains are
// latency-bound, so spreading them wins), then as many as keep about 256 workgroups,
// within the 64 lanes of the chain wave.
static inline uint32_t front_tokens(uint32_t ne, uint32_t n) {
  return min(min(kFrontMaxTok, max(1u, 64u / ne)), max(1u, n / 256u));
}

// Section length for `rows` chains: the longest multiple of 128 whose two halves fit.
static inline uint32_t front_section(uint32_t rows, uint32_t d) {
  const uint32_t sec = (kFrontProdBytes / (8 * rows) - 4) & ~127u;
  return sec < d ? sec : d;
}

__global__ void __launch_bounds__(kFrontThreads) k_front(LayerDev L, FwdBufs B, uint32_t n, int quant, int dispatch,
                                                          uint32_t sec, uint32_t tpw) {
  extern __shared__ float fs[];
  const uint32_t ne = L.ne, d = L.d, k = L.k, nr = tpw * ne, row = sec + 4;  // padded row of one chain
  const uint32_t t0 = blockIdx.x * tpw, ntok = min(tpw, n - t0);             // this workgroup's tokens
  float* prod = fs;                                                          // [2][nr][row]
  float* lg = prod + 2 * nr * row;                                           // [nr] logits
  uint32_t* scratch = reinterpret_cast<uint32_t*>(lg + nr);                  // [tpw][2k] gating
  uint32_t* last = scratch + tpw * 2 * k;                                     // [1] the last workgroup
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint32_t nsec = (d + sec - 1) / sec;
  // producer wave pw (1..8) makes the chains pw-1, pw-1+8, ... of the workgroup's valid
  // tokens; its items are (chain, float4 column) pairs, kFrontItems of them in flight per lane
  auto produce = [&](uint32_t s) {
    const uint32_t k0 = s * sec, len4 = min(sec, d - k0) / 4, c0 = wave - 1, nrv = ntok * ne;
    const uint32_t nch = c0 < nrv ? (nrv - c0 + kFrontProdWaves - 1) / kFrontProdWaves : 0;
    const uint32_t total = nch * len4;
    float* half = prod + (s & 1) * nr * row;
    for (uint32_t base = 0; base < total; base += 64 * kFrontItems) {
      float4 wv[kFrontItems], xv[kFrontItems];
      uint32_t off[kFrontItems];
#pragma unroll
      for (int i = 0; i < kFrontItems; i++) {
        const uint32_t q = base + lane + 64 * i;
        if (q < total) {
          const uint32_t cl = q / len4, j = q - cl * len4, ch = c0 + kFrontProdWaves * cl;
          const uint32_t tt = ch / ne, e = ch - tt * ne;
          wv[i] = reinterpret_cast<const float4*>(L.router + (size_t)e * d + k0)[j];
          xv[i] = reinterpret_cast<const float4*>(B.hs + (size_t)(t0 + tt) * d + k0)[j];
          off[i] = ch * row + 4 * j;
        }
      }
#pragma unroll
      for (int i = 0; i < kFrontItems; i++) {
        if (base + lane + 64 * i < total)
          *reinterpret_cast<float4*>(half + off[i]) =
              make_float4(wv[i].x * xv[i].x, wv[i].y * xv[i].y, wv[i].z * xv[i].z, wv[i].w * xv[i].w);
      }
    }
  };
  auto quantise = [&] {
    const uint32_t nblk = d / 32, items = ntok * nblk;
    for (uint32_t q = tid - 64; q < items; q += 64 * kFrontProdWaves) {
      const uint32_t tt = q / nblk, b = q - tt * nblk;
      float v[32];
      const float4* src = reinterpret_cast<const float4*>(B.hs + (size_t)(t0 + tt) * d + (size_t)b * 32);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        float4 t4 = src[i];
        v[4 * i] = t4.x; v[4 * i + 1] = t4.y; v[4 * i + 2] = t4.z; v[4 * i + 3] = t4.w;
      }
      const size_t gb = (size_t)(t0 + tt) * nblk + b;
      quant32(v, B.xq + gb * 32, B.xs + gb, B.xsum, gb, sum_kind_of(L.qt_gate), sum_offset_of(L.qt_gate));
    }
  };
  if (B.fuse_out)  // the down product adds into the tokens' output rows
    for (uint32_t c = tid; c < ntok * d; c += kFrontThreads) B.out[(size_t)t0 * d + c] = 0.0f;
  if (B.logits_in) {
    if (wave == 0 && lane < ntok * ne) lg[lane] = B.logits_in[(size_t)t0 * ne + lane];
    if (quant && wave != 0) quantise();
  } else {
    if (wave != 0) produce(0);
    __syncthreads();
    float acc = -0.0f;
    for (uint32_t s = 0; s < nsec; s++) {
      if (wave == 0) {
        if (lane < nr) {
          // nb batches of 8 float4; sections are multiples of 128 values, so nb is even
          const uint32_t nb = min(sec, d - s * sec) / 32;
          const float4* src = reinterpret_cast<const float4*>(prod + (s & 1) * nr * row + lane * row);
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
      } else if (quant) {
        quantise();
      }
      __syncthreads();
    }
    if (wave == 0 && lane < nr) lg[lane] = acc;
  }
  __syncthreads();
  // wave w gates token t0 + w
  if (wave < ntok) {
    const uint32_t t = t0 + wave;
    const float x = lane < ne ? lg[wave * ne + lane] : 0.0f;
    if (lane < ne) B.logits[(size_t)t * ne + lane] = x;
    uint32_t id;
    float w;
    gate_wave(L.gating, ne, k, x, lane, &id, &w, scratch + wave * 2 * k);
    if (lane < k) {
      B.ids[(size_t)t * k + lane] = id;
      B.w[(size_t)t * k + lane] = w;
    }
  }
  if (!dispatch) return;
  const auto pair = [&](uint32_t p, uint32_t* pid, float* pw) {
    *pid = B.ids[p];
    *pw = B.w[p];
  };
  if (gridDim.x == 1) {  // the only workgroup: its routing is in memory after the barrier
    __syncthreads();
    if (wave == 0) dispatch_wave(B, [&](int p) { return L.eptr[p * ne + lane]; }, ne, k, n * k, lane, pair);
    return;
  }
  // every workgroup's ids, weights and activation codes are in memory before its count
  // is taken: the barrier orders the waves' stores before thread 0's release fence
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    *last = atomicAdd(B.done, 1u) == gridDim.x - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (!*last || wave != 0) return;
  __threadfence();
  dispatch_wave(B, [&](int p) { return L.eptr[p * ne + lane]; }, ne, k, n * k, lane, pair);
  if (lane == 0) *B.done = 0;
}

bool front_small_ok(const LayerDev& L, uint32_t n) {
  return n >= 1 && L.ne <= (uint32_t)kFrontExperts && L.k <= 32 && L.d % 128 == 0;
}

hipError_t launch_front_small(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, bool dispatch,
                              hipStream_t st) {
  const uint32_t tpw = front_tokens(L.ne, n), sec = front_section(tpw * L.ne, L.d);
  const size_t shm = ((size_t)2 * tpw * L.ne * (sec + 4) + tpw * L.ne + (size_t)tpw * 2 * L.k + 1) * 4;
  static const bool attr =
      hipFuncSetAttribute((const void*)k_front, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  (void)attr;
  hipLaunchKernelGGL(k_front, dim3((n + tpw - 1) / tpw), dim3(kFrontThreads), shm, st, L, B, n, quant,
                     dispatch ? 1 : 0, sec, tpw);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Speculative front end (decode). The exact router logits are d dependent adds per
// (token, expert) (simd/mod.rs:13-16), a chain of ~10 us that the expert products need
// only to know which experts to stream. So the decode call runs k_front without its
// dispatch on a side stream, for the exact logits, ids and weights the combine uses, and
// this kernel on the call's stream:
//
//  * logit L~_e: the same rounded products w*h summed as d/64-long lane sums and a
//    64-lane tree. With S the exact sum of the rounded products and A = sum |products|,
//    recursive summation gives |L_seq - S| <= g(d-1) A and the tree |L~ - S| <= g(d/64+6) A
//    (g(m) = m u / (1 - m u), u = 2^-24), so |L~ - L_seq| <= delta_e.
//  * candidates: expert e is left out only when at least k others certainly rank before
//    it, L~_j - delta_j > L~_e + delta_e + eps_e; eps_e keeps their probabilities apart
//    after expf and the normalisation, so the exact order puts them first whatever the
//    tie rule. Non-finite logits, or fewer than k experts safely above expf's underflow,
//    make every expert a candidate. The exact top k is therefore a subset.
//  * the int8 quantiser of the token's activations (packed math), and the dispatch of the
//    (token, candidate) pairs by the last workgroup, as k_front does for the routed ones.
//
// The expert products then run on the candidate pairs (almost always exactly the routed
// ones), and the combine picks each routed (token, expert) pair's slot by search.
// ---------------------------------------------------------------------------------

constexpr int kSpecThreads = 512;
constexpr int kSpecFrontLoads = 16;  // float4 pairs a lane has in flight in a router dot
static_assert(kFrontExperts == (int)kSpecMaxExperts, "one expert a lane in the candidate test");

// NORM: the token's row of hs is made first, by the residual add and RMSNorm of
// add_norm_row (FwdBufs::nx ...), written to nh and kept in LDS, from where the logits
// and the quantiser read it.
template <bool NORM>
__global__ void __launch_bounds__(kSpecThreads) k_spec_front(LayerDev L, FwdBufs B, uint32_t n, int quant) {
  __shared__ float lt[kFrontExperts], la[kFrontExperts];
  __shared__ uint32_t cl[kFrontExperts];
  __shared__ double sb[2 * kFrontExperts];  // candidate test: lo, then hi, of each expert
  extern __shared__ float4 hrow[];          // NORM: the token's row of hs
  const uint32_t ne = L.ne, d = L.d, k = L.k, t = blockIdx.x;
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  if constexpr (NORM) {
    add_norm_row<true>(B.nx + (size_t)t * d, B.ny + (size_t)t * d, B.nw, d, B.neps, B.nh + (size_t)t * d,
                       reinterpret_cast<float*>(hrow), B.nsl_y, B.ny_stride, lt);
    __syncthreads();
  }
  const float* hs = NORM ? reinterpret_cast<const float*>(hrow) : B.hs + (size_t)t * d;
  // wave 0's slab pointers for the dispatch (lane e: expert e's gate, up, down), loaded
  // first; the output rows' zeroing and the quantiser's loads (threads of waves 1 on, the
  // activations of their 32-value block) follow the router dots' loads, whose results
  // the barrier waits for. Only the expert kernels read the quantised activations, so
  // those waves quantise after the barrier while wave 0 runs the candidate test and the
  // dispatch.
  const uint8_t* ep[3] = {nullptr, nullptr, nullptr};
  if (wave == 0 && lane < ne)
    for (int p = 0; p < 3; p++) ep[p] = L.eptr[p * ne + lane];
  spec_dots<kSpecFrontLoads>(L.router, hs, ne, d, lt, la);
  if (B.fuse_out)  // the down product adds into the token's output row
    for (uint32_t c = tid; c < d; c += kSpecThreads) B.out[(size_t)t * d + c] = 0.0f;
  const uint32_t nblk = d / 32, qb = tid - 64;  // block of thread tid >= 64
  float qv[32];
  const bool qown = quant && tid >= 64 && qb < nblk && nblk <= kSpecThreads - 64;
  if (qown) {
    const float4* src = reinterpret_cast<const float4*>(hs + (size_t)qb * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 t4 = src[i];
      qv[4 * i] = t4.x; qv[4 * i + 1] = t4.y; qv[4 * i + 2] = t4.z; qv[4 * i + 3] = t4.w;
    }
  }
  if (quant && nblk > kSpecThreads - 64) {  // (wide rows: every thread, before the barrier)
    for (uint32_t b = tid; b < nblk; b += kSpecThreads) {
      float v[32];
      const float4* src = reinterpret_cast<const float4*>(hs + (size_t)b * 32);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        float4 t4 = src[i];
        v[4 * i] = t4.x; v[4 * i + 1] = t4.y; v[4 * i + 2] = t4.z; v[4 * i + 3] = t4.w;
      }
      const size_t gb = (size_t)t * nblk + b;
      quant32(v, B.xq + gb * 32, B.xs + gb, B.xsum, gb, sum_kind_of(L.qt_gate), sum_offset_of(L.qt_gate));
    }
  }
  __syncthreads();
  if (wave != 0) {
    if (qown) {
      const size_t gb = (size_t)t * nblk + qb;
      quant32(qv, B.xq + gb * 32, B.xs + gb, B.xsum, gb, sum_kind_of(L.qt_gate), sum_offset_of(L.qt_gate));
    }
    return;
  }
  bool cand;
  uint32_t pos;
  const uint32_t nc = spec_candidates<kSpecFrontLoads>(ne, k, d, L.gating, lt, la, sb, cl, lane, &cand, &pos);
  const bool valid = lane < ne;
  const uint32_t my = lane < nc ? cl[lane] : ~0u;
  if (lane < ne) B.cand[(size_t)t * ne + lane] = my;
  if (n == 1) {
    // one token: what dispatch_wave makes of its candidate list, written directly. Every
    // candidate has one pair, so the experts of equal count go in ascending id order:
    // candidate e's active slot, first pair slot and token tile are all its rank pos
    // among the candidates, and its one pair is token 0's.
    if (valid) {
      B.offsets[lane] = pos;
      if (cand) {
        B.active[1 + pos] = lane;
        if (B.work) {
          ExpertWork& W = B.work[pos];
          for (int p = 0; p < 3; p++) W.w[p] = ep[p];
          W.e = lane;
          W.s0 = pos;
          W.m = 1;
        }
        B.slot_tok[pos] = 0;
      }
      if (B.work && lane >= nc) B.work[lane].m = 0;
    }
    if (lane == 0) {
      B.offsets[ne] = nc;
      B.active[0] = nc;
    }
    if (B.ptile) {
      if (cand) B.ptile[pos] = pos << 16;
      for (uint32_t i = nc + lane; i < B.ptile_cap; i += 64) B.ptile[i] = ~0u;
    }
    return;
  }
  __threadfence();
  uint32_t prev = 0;
  if (lane == 0) prev = atomicAdd(B.done, 1u);
  if (lane_u(prev, 0) == n - 1) {
    __threadfence();
    dispatch_wave(B, [&](int p) { return ep[p]; }, ne, ne, n * ne, lane, [&](uint32_t p, uint32_t* pid, float* pw) {
      *pid = B.cand[p];
      *pw = 0.0f;
    }, false);
    if (lane == 0) *B.done = 0;
  }
}

bool spec_ok(const LayerDev& L, uint32_t n) {
  return front_small_ok(L, n) && (uint64_t)n * L.ne <= kSpecMaxSlots && L.k <= L.ne;
}

hipError_t launch_spec_front(const LayerDev& L, const FwdBufs& B, uint32_t n, int quant, hipStream_t st) {
  if (B.nx) {
    if (B.nsl_y == 0 || B.nsl_y > kMaxKsg || L.d > 4 * 256 * kNormVec) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_spec_front<true>, dim3(n), dim3(kSpecThreads), L.d * 4, st, L, B, n, quant);
  } else {
    hipLaunchKernelGGL(k_spec_front<false>, dim3(n), dim3(kSpecThreads), 0, st, L, B, n, quant);
  }
  return hipGetLastError();
}

// Exact routing of one token a workgroup (route_token): lanes of wave 0 run the ne
// sequential chains (simd/mod.rs:13-16) over the products the other seven waves put in LDS
// a section ahead, then gate the token (gate_wave). For ne <= 64 and d a multiple of 64 it
// replaces k_route's one thread a chain, which waits for its loads a batch at a time (68
// us a single-token call at d 4096, 8 experts).
constexpr int kRouteTokThreads = 512;
__global__ void __launch_bounds__(kRouteTokThreads) k_route_tok(RouteArgs r) {
  extern __shared__ float rt_lds[];
  route_token(r, blockIdx.x, rt_lds, r.sec, nullptr);
}

hipError_t launch_route(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  if (!B.logits_in && L.ne <= 64 && L.d % 64 == 0) {
    RouteArgs r{};
    r.router = L.router;
    r.hs = B.hs;
    r.logits = B.logits;
    r.ids = B.ids;
    r.w = B.w;
    r.n = n;
    r.ne = L.ne;
    r.k = L.k;
    r.d = L.d;
    r.gating = L.gating;
    r.combine = L.combine;
    // sections: the longest multiple of 64 values (at most 1024, at least 64) whose two
    // halves of products fit 64 KB
    const uint32_t fit = (65536u / (8u * L.ne) - 4u) & ~63u;
    r.sec = std::min(L.d, std::max(64u, std::min(fit, 1024u)));
    const size_t lds = (size_t)route_token_lds(L.ne, L.k, r.sec) * 4;
    static const bool once = hipFuncSetAttribute((const void*)k_route_tok,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024) == hipSuccess;
    (void)once;
    hipLaunchKernelGGL(k_route_tok, dim3(n), dim3(kRouteTokThreads), lds, st, r);
    return hipGetLastError();
  }
  uint32_t tpb = L.ne >= kRouteThreads ? 1u : kRouteThreads / L.ne;
  size_t shm = (size_t)tpb * L.ne * 4 + tpb * 4 + (size_t)tpb * L.k * 8;
  hipLaunchKernelGGL(k_route, dim3((n + tpb - 1) / tpb), dim3(kRouteThreads), shm, st, L, B, n);
  return hipGetLastError();
}

hipError_t launch_dispatch(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  if (L.ne <= kParExperts) return launch_dispatch_par(L, B, n, st);
  const size_t shm = (kDispatchThreads + 3 * (size_t)L.ne + 2) * 4;
  if (shm > 160 * 1024) return hipErrorInvalidValue;  // registration bounds ne far below this
  static const bool attr =
      hipFuncSetAttribute((const void*)k_dispatch, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) ==
      hipSuccess;
  (void)attr;
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(kDispatchThreads), shm, st, L, B, n);
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
    if (qt == Q3_K && p < 6) {  // the regrouped values (q3s_byte); the unit is one block
      for (uint32_t b = 0; b < 16; b++) v[b / 4] |= (uint32_t)q3s_byte(src + (uint64_t)u * un.B, p * 16 + b) << (8 * (b % 4));
    } else {
      for (uint32_t b = 0; b < 16; b++) {
        int64_t s = unit_src_byte(qt, un, nblk, u, p * 16 + b);
        if (s >= 0) v[b / 4] |= (uint32_t)src[s] << (8 * (b % 4));
      }
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

// Decode-sized combines (k <= kCombK pairs a token): every slot, weight and slice value
// is loaded before the first add, so the kernel waits on two memory round trips (the
// slots, then the slices) instead of one per slice.
constexpr uint32_t kCombK = 8;

template <uint32_t KS>
__device__ __forceinline__ void combine_fast(const LayerDev& L, const FwdBufs& B, uint32_t t, uint32_t c,
                                             uint32_t ksg) {
  const uint32_t k = L.k, d = L.d;
  const size_t part = (size_t)B.nslot * d;
  uint32_t slot[kCombK], rk[kCombK];
  float wv[kCombK];
  if (B.spec) {
#pragma unroll
    for (uint32_t i = 0; i < kCombK; i++)
      if (i < k) {
        slot[i] = B.slot_of[(size_t)t * k + i];
        wv[i] = B.slot_w[(size_t)t * k + i];
      }
  } else {
    uint32_t id[kCombK];
#pragma unroll
    for (uint32_t i = 0; i < kCombK; i++)
      if (i < k) {
        id[i] = B.ids[(size_t)t * k + i];
        wv[i] = B.w[(size_t)t * k + i];
        slot[i] = B.slot_of[(size_t)t * k + i];
        rk[i] = i;
      }
    if (L.combine == 0) {  // ascending expert id: each rank's position among the token's ids
#pragma unroll
      for (uint32_t i = 0; i < kCombK; i++)
        if (i < k) {
          uint32_t pos = 0;
#pragma unroll
          for (uint32_t j = 0; j < kCombK; j++)
            if (j < k) pos += (id[j] < id[i] || (id[j] == id[i] && j < i)) ? 1u : 0u;
          rk[i] = pos;
        }
    }
  }
  float yv[kCombK][KS];
#pragma unroll
  for (uint32_t i = 0; i < kCombK; i++)
    if (i < k) {
      const bool ok = slot[i] != ~0u;
      const float* yp = B.y + (size_t)(ok ? slot[i] : 0u) * d + c;
#pragma unroll
      for (uint32_t g = 0; g < KS; g++) yv[i][g] = g < ksg ? yp[g * part] : 0.0f;
      if (!ok) yv[i][0] = __int_as_float(0x7fc00000);  // a pair the candidates missed: NaN
    }
  float ys[kCombK];  // each pair's down row: its slices added in order
#pragma unroll
  for (uint32_t i = 0; i < kCombK; i++)
    if (i < k) {
      float s = yv[i][0];
#pragma unroll
      for (uint32_t g = 1; g < KS; g++)
        if (g < ksg) s += yv[i][g];
      ys[i] = s;
    }
  float acc = 0.0f;
  // in combine order: position r holds the pair whose rank is r
#pragma unroll
  for (uint32_t r = 0; r < kCombK; r++)
    if (r < k) {
      float y = 0.0f, w = 0.0f;
#pragma unroll
      for (uint32_t i = 0; i < kCombK; i++)
        if (i < k && (B.spec ? i == r : rk[i] == r)) {
          y = ys[i];
          w = wv[i];
        }
      acc = acc + y * w;
    }
  B.out[(size_t)t * d + c] = acc;
}

__global__ void __launch_bounds__(256) k_combine(LayerDev L, FwdBufs B, uint32_t n, uint32_t ksg) {
  const uint32_t t = blockIdx.y, k = L.k, d = L.d;
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n || c >= d) return;
  if (k <= kCombK && ksg <= kMaxKsg) {
    combine_fast<kMaxKsg>(L, B, t, c, ksg);
    return;
  }
  const size_t part = (size_t)B.nslot * d;
  float acc = 0.0f;
  if (B.spec) {
    // the exact routing left (slot, weight) in combine order; slot ~0u: a pair the
    // candidates missed, which gives NaN (the candidate sets are supersets)
    for (uint32_t i = 0; i < k; i++) {
      const uint32_t slot = B.slot_of[(size_t)t * k + i];
      const float wv = B.slot_w[(size_t)t * k + i];
      float yv = __int_as_float(0x7fc00000);
      if (slot != ~0u) {
        const float* yp = B.y + (size_t)slot * d + c;
        yv = yp[0];
        for (uint32_t g = 1; g < ksg; g++) yv += yp[g * part];
      }
      acc = acc + yv * wv;
    }
    B.out[(size_t)t * d + c] = acc;
    return;
  }
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
  for (uint32_t i = 0; i < k; i++) {
    const uint32_t r = order[i];
    const float wv = B.w[(size_t)t * k + r];
    const uint32_t slot = B.slot_of[(size_t)t * k + r];
    const float* yp = B.y + (size_t)slot * d + c;
    float yv = yp[0];
    for (uint32_t g = 1; g < ksg; g++) yv += yp[g * part];
    acc = acc + yv * wv;
  }
  B.out[(size_t)t * d + c] = acc;
}

hipError_t launch_combine(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st) {
  hipLaunchKernelGGL(k_combine, dim3((L.d + 255) / 256, n), dim3(256), 0, st, L, B, n, ksg);
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

// K groups of the down product. Measured on the C2 layer (64 row tiles, 56 units): with
// up to 4 (token, expert) pairs, 4 groups; with more, as many as the rows allow (7), the
// down kernel then taking 61 us instead of 89 us at batch 8. Bounded to between about
// 1024 and 4096 workgroups (kDnKS = 2 waves each) and at least 4 units a wave.
uint32_t down_ksg(const LayerDev& L, uint32_t pairs) {
  Unit un;
  if (!unit_of(L.qt_down, &un)) return 1;
  const uint32_t tiles = (L.d + kTileRows - 1) / kTileRows, wgs = tiles * min(L.ne, pairs);
  uint32_t ksg = pairs <= 4 ? 4u : 8u;
  ksg = min(ksg, (4096 + wgs - 1) / wgs);
  ksg = max(ksg, (1024 + wgs - 1) / wgs);
  const uint32_t cap = max(1u, row_units(un, L.f) / (kDnKS * 4));
  return max(1u, min(min(ksg, cap), kMaxKsg));
}

bool gateup_self_ok(const LayerDev& L, uint32_t n) {
  switch (L.qt_gate) {
#define SO(T) case T: return units_self_ok<T>(L, n);
    SO(Q4_K) SO(Q5_K) SO(Q6_K) SO(Q3_K) SO(Q2_K) SO(Q8_0) SO(Q4_0) SO(F16) SO(F32)
#undef SO
  }
  return false;
}

hipError_t launch_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, const RouteArgs& ra, hipStream_t st) {
  switch (L.qt_gate) {
#define GU(T) case T: return units_gateup<T>(L, B, n, ra, st);
    GU(Q4_K) GU(Q5_K) GU(Q6_K) GU(Q3_K) GU(Q2_K) GU(Q8_0) GU(Q4_0) GU(F16) GU(F32)
#undef GU
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------
// Prefill (f32 math on MFMA, gmoe_prefill.hip)
// ---------------------------------------------------------------------------------

static bool prefill_type(uint32_t qt) {
  return qt == Q4_K || qt == Q5_K || qt == Q6_K || qt == Q3_K || qt == Q2_K || qt == Q8_0 || qt == Q4_0 ||
         qt == F16;
}

bool prefill_ok(const LayerDev& L, uint32_t n) {
  const uint32_t nk = n * L.k;
  // rows: gate/up workgroups take up to 256 rows of f, down ones up to 512 of d
  return L.math == 1 && nk >= kPfMinSlots && nk >= 4 * L.ne && L.qt_gate == L.qt_up && prefill_type(L.qt_gate) &&
         prefill_type(L.qt_down) && L.d % 512 == 0 && L.f % 256 == 0 && L.ne < 65536;
}

// A dense projection run through the down-product path: rows = L.d, width = L.f.
bool prefill_dense_ok(const LayerDev& L, uint32_t n) {
  return L.math == 1 && n >= kPfMinSlots && prefill_type(L.qt_down) && L.d % 512 == 0 && L.f % 256 == 0;
}

// The work list of a dense projection: one "expert" (the weight, tiled) holding all n
// tokens as slots 0..n-1, its token tiles, and the identity slot -> token map.
__global__ void __launch_bounds__(256) k_dense_setup(ExpertWork* __restrict__ work, uint32_t* __restrict__ offsets,
                                                     uint32_t* __restrict__ active, uint32_t* __restrict__ ptile,
                                                     uint32_t ptile_cap, uint32_t* __restrict__ slot_tok,
                                                     const uint8_t* w, uint32_t n) {
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    ExpertWork e;
    e.w[0] = e.w[1] = e.w[2] = w;
    e.e = 0;
    e.s0 = 0;
    e.m = n;
    e.pad = 0;
    work[0] = e;
    offsets[0] = 0;
    offsets[1] = n;
    active[0] = 1;
    active[1] = 0;
  }
  const uint32_t tiles = (n + kPfTok - 1) / kPfTok;
  if (ptile)
    for (uint32_t i = t; i < ptile_cap; i += blockDim.x) ptile[i] = i < tiles ? i : ~0u;
  if (slot_tok)
    for (uint32_t i = t; i < n; i += blockDim.x) slot_tok[i] = i;
}

hipError_t launch_dense_setup(ExpertWork* work, uint32_t* offsets, uint32_t* active, uint32_t* ptile,
                              uint32_t ptile_cap, uint32_t* slot_tok, const uint8_t* w, uint32_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_dense_setup, dim3(1), dim3(256), 0, st, work, offsets, active, ptile, ptile_cap, slot_tok, w, n);
  return hipGetLastError();
}

// The activations in slot order as fp16 pairs, x = hi + lo (hi = fp16(x), lo =
// fp16(x - hi)), hi plane then lo plane, and with sw > 0 the sums of each sw values
// (f32, left to right) as pairs the same way. One thread per 32 values.
__global__ void __launch_bounds__(256) k_gather_f16(const float* __restrict__ hs, const uint32_t* __restrict__ slot_tok,
                                                    uint32_t d, uint32_t nk, uint32_t sw, _Float16* __restrict__ xh,
                                                    _Float16* __restrict__ xsh) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  const uint32_t s = blockIdx.y, c = 32 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (c >= d) return;
  const float4* src = reinterpret_cast<const float4*>(hs + (size_t)slot_tok[s] * d + c);
  const size_t o = (size_t)s * d + c, plane = (size_t)nk * d;
  float sum[2] = {0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 a = src[2 * i], b = src[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    half8 hi, lo;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      hi[j] = (_Float16)v[j];
      lo[j] = (_Float16)(v[j] - (float)hi[j]);
      sum[i / 2] += v[j];
    }
    *reinterpret_cast<half8*>(xh + o + 8 * i) = hi;
    *reinterpret_cast<half8*>(xh + plane + o + 8 * i) = lo;
  }
  if (sw) {
    const uint32_t ns = d / sw, per = 32 / sw;
    const size_t so = (size_t)s * ns + c / sw, splane = (size_t)nk * ns;
    const float tot[2] = {sum[0] + sum[1], 0.0f};
    for (uint32_t i = 0; i < per; i++) {
      const float v = per == 1 ? tot[0] : sum[i];
      const _Float16 hi = (_Float16)v;
      xsh[so + i] = hi;
      xsh[splane + so + i] = (_Float16)(v - (float)hi);
    }
  }
}

hipError_t launch_gather_f16(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  const uint32_t nk = n * L.k;
  hipLaunchKernelGGL(k_gather_f16, dim3((L.d / 32 + 255) / 256, nk), dim3(256), 0, st, B.hs, B.slot_tok, L.d, nk,
                     pf_sum_width(L.qt_gate), B.xh, B.xsh);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Packed-math prefill (k_pq, gmoe_prefill.hip)
// ---------------------------------------------------------------------------------

static bool pq_type_rt(uint32_t qt) {
  return qt == Q4_K || qt == Q5_K || qt == Q6_K || qt == Q3_K || qt == Q2_K || qt == Q8_0;
}

// Tokens per expert from which the MFMA products beat the per-row decode kernels
// (whose cost grows with every token an expert gets, while a token tile's is fixed).
constexpr uint32_t kPqMinPerExpert = 16;

bool prefill_packed_ok(const LayerDev& L, uint32_t n) {
  const uint32_t nk = n * L.k;
  return L.math == 0 && nk >= kPfMinSlots && nk >= kPqMinPerExpert * L.ne && L.qt_gate == L.qt_up &&
         pq_type_rt(L.qt_gate) && pq_type_rt(L.qt_down) && L.d % 512 == 0 && L.f % 256 == 0 && L.ne < 65536;
}

// The int8 activation codes in slot order as fp16, their per-32 scales and their sums
// (the gate type's width) transposed to [K/w][nkp]. Threads: 64 slots x 4 blocks of 32.
__global__ void __launch_bounds__(256) k_gather_codes(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                      const uint32_t* __restrict__ xsum,
                                                      const uint32_t* __restrict__ slot_tok, uint32_t d, uint32_t nk,
                                                      uint32_t nkp, uint32_t sw, _Float16* __restrict__ xh,
                                                      float* __restrict__ qxs, float* __restrict__ qxsum) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  const uint32_t s = blockIdx.x * 64 + (threadIdx.x & 63), b = blockIdx.y * 4 + (threadIdx.x >> 6), nb = d / 32;
  if (s >= nk || b >= nb) return;
  const uint32_t t = slot_tok[s];
  const uint4* src = reinterpret_cast<const uint4*>(xq + (size_t)t * d + 32 * b);
  const uint4 q[2] = {src[0], src[1]};
  half8* dst = reinterpret_cast<half8*>(xh + (size_t)s * d + 32 * b);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint4 v = q[i / 2];
    const uint32_t w0 = (i % 2) ? v.z : v.x, w1 = (i % 2) ? v.w : v.y;
    half8 o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      o[j] = (_Float16)(float)(int8_t)(w0 >> (8 * j));
      o[4 + j] = (_Float16)(float)(int8_t)(w1 >> (8 * j));
    }
    dst[i] = o;
  }
  qxs[(size_t)b * nkp + s] = xs[(size_t)t * nb + b];
  if (sw == 32) {
    qxsum[(size_t)b * nkp + s] = __uint_as_float(xsum[(size_t)t * nb + b]);
  } else if (sw == 16) {
    qxsum[(size_t)(2 * b) * nkp + s] = __uint_as_float(xsum[(size_t)t * 2 * nb + 2 * b]);
    qxsum[(size_t)(2 * b + 1) * nkp + s] = __uint_as_float(xsum[(size_t)t * 2 * nb + 2 * b + 1]);
  }
}

hipError_t launch_gather_codes(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  const uint32_t nk = n * L.k;
  hipLaunchKernelGGL(k_gather_codes, dim3((nk + 63) / 64, (L.d / 32 + 3) / 4), dim3(256), 0, st, B.xq, B.xs, B.xsum,
                     B.slot_tok, L.d, nk, B.nkp, pq_sum_width(L.qt_gate), B.xh, B.qxs, B.qxsum);
  return hipGetLastError();
}

hipError_t launch_pq_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  switch (L.qt_gate) {
#define GU(T) case T: return pq_gateup<T>(L, B, n, st);
    GU(Q4_K) GU(Q5_K) GU(Q6_K) GU(Q3_K) GU(Q2_K) GU(Q8_0)
#undef GU
  }
  return hipErrorInvalidValue;
}

hipError_t launch_prefill_gateup(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  switch (L.qt_gate) {
#define GU(T) case T: return prefill_gateup<T>(L, B, n, st);
    GU(Q4_K) GU(Q5_K) GU(Q6_K) GU(Q3_K) GU(Q2_K) GU(Q8_0) GU(Q4_0) GU(F16)
#undef GU
  }
  return hipErrorInvalidValue;
}

hipError_t launch_prefill_down(const LayerDev& L, const FwdBufs& B, uint32_t n, uint32_t ksg, hipStream_t st) {
  switch (L.qt_down) {
#define DN(T) case T: return prefill_down<T>(L, B, n, ksg, st);
    DN(Q4_K) DN(Q5_K) DN(Q6_K) DN(Q3_K) DN(Q2_K) DN(Q8_0) DN(Q4_0) DN(F16)
#undef DN
  }
  return hipErrorInvalidValue;
}

uint32_t prefill_ksg(const LayerDev& L, const FwdBufs& B) {
  switch (L.qt_down) {
#define DN(T) case T: return prefill_down_slices<T>(L, B);
    DN(Q4_K) DN(Q5_K) DN(Q6_K) DN(Q3_K) DN(Q2_K) DN(Q8_0) DN(Q4_0) DN(F16)
#undef DN
  }
  return 1;
}

// K groups of a dense projection's down kernel (one matrix, no experts): enough for
// about 960 workgroups (near four per CU), each wave keeping at least one unit.
uint32_t dense_ksg(const LayerDev& L) {
  Unit un;
  if (!unit_of(L.qt_down, &un)) return 1;
  const uint32_t tiles = (L.d + kTileRows - 1) / kTileRows;
  const uint32_t ksg = (960 + tiles - 1) / tiles;
  const uint32_t cap = max(1u, row_units(un, L.f) / kDnKS);
  return max(1u, min(min(ksg, cap), kMaxKsg));
}

bool down_atomic_ok(const LayerDev& L, uint32_t n) { return L.k <= 2 && n >= 1 && n <= kFuseMaxTokens; }

hipError_t launch_down_atomic(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st) {
  switch (L.qt_down) {
#define DN(T) case T: return units_down_atomic<T>(L, B, n, st);
    DN(Q4_K) DN(Q5_K) DN(Q6_K) DN(Q3_K) DN(Q2_K) DN(Q8_0) DN(Q4_0) DN(F16) DN(F32)
#undef DN
  }
  return hipErrorInvalidValue;
}

hipError_t launch_embed_tiled(uint32_t qtype, const uint8_t* tiled, uint32_t cols, const GlueTokens* tk,
                              const uint32_t* dtok, uint32_t n, float* x, hipStream_t st) {
  switch (qtype) {
#define EM(T) case T: return units_embed<T>(tiled, cols, tk, dtok, n, x, st);
    EM(Q4_K) EM(Q5_K) EM(Q6_K) EM(Q3_K) EM(Q2_K) EM(Q8_0) EM(Q4_0) EM(F16) EM(F32)
#undef EM
  }
  return hipErrorInvalidValue;
}

hipError_t launch_down(const LayerDev& L, const FwdBufs& B, uint32_t n, hipStream_t st, uint32_t ksg_in) {
  const uint32_t ksg = ksg_in ? ksg_in : down_ksg(L, n * L.k);
  switch (L.qt_down) {
#define DN(T) case T: return units_down<T>(L, B, n, ksg, st);
    DN(Q4_K) DN(Q5_K) DN(Q6_K) DN(Q3_K) DN(Q2_K) DN(Q8_0) DN(Q4_0) DN(F16) DN(F32)
#undef DN
  }
  return hipErrorInvalidValue;
}

}  // namespace gmoe
