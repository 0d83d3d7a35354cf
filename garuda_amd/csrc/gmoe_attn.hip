// gmoe_attn.hip — grouped-query decode attention over a paged KV cache.
//
// Reference: LlamaBackend::attend_one (garuda/src/llama/mod.rs:766-821) and
// KVCacheState (cache/mod.rs:143-600). Per token: rotate q (every query head) and k
// (every kv head) by the token's position (simd::rope, simd/mod.rs:196-206), append k
// and v to the sequence's cache, and for each query head h attend over positions
// [start, pos] of kv head h / group: scores = q·k * (1/sqrt(hd)), softmax (simd.rs
// :132-158), context = sum of p_j * v_j. f32 throughout; the reductions run in
// parallel, so results match the reference within the layer tolerance.
//
// Device layout. Pages of `bs` positions: keys [n_kv][bs][hd] then values in the same
// layout, f32, so one kv head's rows of a page are contiguous. Each (sequence, layer) has
// a page table of `ppseq` page ids. A call's entries
// are tokens, each with its sequence's page table, its position and the position
// attention starts at; entries of one sequence come in position order, so the append
// kernel writes every entry's k and v before any attends (causal within the call).
#include "gmoe_device.h"

namespace gmoe {


// simd::rope for pair i of a head at position pos: the frequency theta^(-2i/hd) and
// the angle in f32 as the reference forms them.
__device__ __forceinline__ void rope_pair(float& a, float& b, uint32_t i, uint32_t hd, uint32_t pos, float theta) {
  const float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)hd);
  const float ang = (float)pos * freq;
  float s, c;
  sincosf(ang, &s, &c);
  const float x = a, y = b;
  a = x * c - y * s;
  b = x * s + y * c;
}

__device__ __forceinline__ AttnEntry entry(const AttnArgs& a, uint32_t i) { return a.ent ? a.ent[i] : a.inl[i]; }

// Key row of position p, kv head h (the value row is bs * kv_dim floats further on).
__device__ __forceinline__ const float* key_row(const AttnArgs& a, const AttnEntry& e, uint32_t p, uint32_t h) {
  return a.pool + (size_t)e.pages[p / a.bs] * a.page_floats + ((size_t)h * a.bs + p % a.bs) * a.hd;
}

// grid (n, ceil(pairs / 256)), pairs = (n_heads + n_kv) * hd / 2
// (x, y) = elements 2j, 2j+1 from p, each the sum of nsl K slices `stride` floats apart in
// slice order when nsl > 1 (k_reduce_parts's sum); the slice loads are issued together
// (indices clamped, the surplus ones not added)
__device__ __forceinline__ void ld_pair(const float* p, uint32_t j, uint32_t nsl, uint64_t stride, float& x, float& y) {
  if (nsl <= 1) {
    x = p[2 * j];
    y = p[2 * j + 1];
    return;
  }
  float vx[kMaxKsg], vy[kMaxKsg];
#pragma unroll
  for (uint32_t g = 0; g < kMaxKsg; g++) {
    const float* s = p + min(g, nsl - 1) * stride;
    vx[g] = s[2 * j];
    vy[g] = s[2 * j + 1];
  }
  x = vx[0];
  y = vy[0];
#pragma unroll
  for (uint32_t g = 1; g < kMaxKsg; g++)
    if (g < nsl) {
      x += vx[g];
      y += vy[g];
    }
}

__global__ void __launch_bounds__(256) k_rope_append(AttnArgs a) {
  const uint32_t i = blockIdx.x, half = a.hd / 2, kvd = a.n_kv * a.hd;
  const uint32_t pr = blockIdx.y * 256 + threadIdx.x, qpairs = a.n_heads * half;
  const AttnEntry e = entry(a, i);
  const uint32_t page = e.page, slot = e.pos % a.bs;
  if (e.fresh && pr == 0) e.pages[e.pos / a.bs] = page;  // read by the attention kernel after this one
  float* kp = a.pool + (size_t)page * a.page_floats + (size_t)slot * a.hd;  // head h at + h * bs * hd
  float* vp = kp + (size_t)a.bs * kvd;
  if (pr < qpairs) {
    const uint32_t h = pr / half, j = pr % half;
    const float* src = a.q + (size_t)i * a.q_stride + h * a.hd;
    float x, y;
    ld_pair(src, j, a.nsl, a.sl_stride, x, y);
    rope_pair(x, y, j, a.hd, e.pos, a.theta);
    float* dst = a.qr + (size_t)i * a.n_heads * a.hd + h * a.hd;
    dst[2 * j] = x;
    dst[2 * j + 1] = y;
  } else if (pr < qpairs + a.n_kv * half) {
    const uint32_t p2 = pr - qpairs, h = p2 / half, j = p2 % half;
    const float* src = a.k + (size_t)i * a.kv_stride + h * a.hd;
    float x, y;
    ld_pair(src, j, a.nsl, a.sl_stride, x, y);
    rope_pair(x, y, j, a.hd, e.pos, a.theta);
    const size_t hoff = (size_t)h * a.bs * a.hd;
    kp[hoff + 2 * j] = x;
    kp[hoff + 2 * j + 1] = y;
    const float* vs = a.v + (size_t)i * a.kv_stride + h * a.hd;
    float vx, vy;
    ld_pair(vs, j, a.nsl, a.sl_stride, vx, vy);
    vp[hoff + 2 * j] = vx;
    vp[hoff + 2 * j + 1] = vy;
  }
}

__device__ __forceinline__ float wave_max(float v) { return wave64_max(v); }
__device__ __forceinline__ float wave_sum(float v) { return wave64_sum(v); }

// grid (n, n_kv, nchunk), 256 threads: one chunk of kAttnChunk positions for the
// `group` query heads of one kv head. Thread t takes position j = t / 4 of the chunk and
// every fourth float4 column of its key and value rows from column t % 4 on, loaded from
// the page at once (the value loads' latency hides behind the scores). Scores: the
// thread's columns dotted with each head's q (in LDS), the four partial dots added by
// lane shuffles. The values go to an LDS tile [kAttnChunk][hd]; per head the chunk's max
// m, the sum l of exp(s - m) and o = sum of exp(s - m) * v go to part, o by float4
// columns with the positions split over the spare threads (parts added in order).
// Dynamic LDS: tile, q [G][hd], p [G][kAttnChunk], (m, l) [kAttnMaxGroup][2], o parts [256] float4.
inline uint32_t attn_lds_bytes(uint32_t G, uint32_t hd) {
  return (kAttnChunk * hd + G * hd + G * kAttnChunk + 2 * kAttnMaxGroup) * 4 + 256 * 16;
}

static_assert(kAttnChunk * 4 == 256, "four threads per position of a chunk");

template <int MAXHD>
__global__ void __launch_bounds__(256) k_attn_partial(AttnArgs a) {
  constexpr int NR = MAXHD / 16;  // float4 columns of a row per thread
  extern __shared__ float4 lds_v4[];
  float* lds_f = reinterpret_cast<float*>(lds_v4);
  const uint32_t i = blockIdx.x, h = blockIdx.y, c = blockIdx.z, t = threadIdx.x;
  const uint32_t G = a.n_heads / a.n_kv, hd = a.hd, kvd = a.n_kv * hd, q4 = hd / 4;
  float* tile = lds_f;                  // [kAttnChunk][hd] values
  float* qs = tile + kAttnChunk * hd;   // [G][hd]
  float* psb = qs + G * hd;             // [G][kAttnChunk]
  float* mlb = psb + G * kAttnChunk;    // [kAttnMaxGroup][2]
  float4* og = reinterpret_cast<float4*>(mlb + 2 * kAttnMaxGroup);  // [256]
  auto ps = [&](uint32_t g, uint32_t j) -> float& { return psb[g * kAttnChunk + j]; };
  auto ml = [&](uint32_t g, uint32_t k) -> float& { return mlb[2 * g + k]; };
  const AttnEntry e = entry(a, i);
  const uint32_t end = e.pos + 1, p0 = e.start + c * kAttnChunk;
  float* out = a.part + (((size_t)i * a.n_heads + h * G) * a.nchunk + c) * (hd + 2);
  const size_t gstride = (size_t)a.nchunk * (hd + 2);
  if (p0 >= end) {  // past the entry's span: an empty chunk
    if (t < G) {
      out[t * gstride + hd] = -INFINITY;
      out[t * gstride + hd + 1] = 0.0f;
    }
    return;
  }
  const uint32_t cnt = min(kAttnChunk, end - p0);
  const uint32_t j = t >> 2, qq = t & 3;
  const bool rowok = j < cnt;
  float4 kreg[NR], vreg[NR];
  {
    const float* kr = key_row(a, e, p0 + (rowok ? j : 0u), h);
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const uint32_t col = qq + 4 * r;
      kreg[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      vreg[r] = kreg[r];
      if (rowok && col < q4) {
        kreg[r] = *reinterpret_cast<const float4*>(kr + 4 * col);
        vreg[r] = *reinterpret_cast<const float4*>(kr + (size_t)a.bs * kvd + 4 * col);
      }
    }
  }
  {
    const float4* qsrc = reinterpret_cast<const float4*>(a.qr + (size_t)i * a.n_heads * hd + (size_t)h * G * hd);
    for (uint32_t x = t; x < G * q4; x += 256) reinterpret_cast<float4*>(qs)[x] = qsrc[x];
  }
  __syncthreads();
  // scores of position j, every head of the group
  float acc[kAttnMaxGroup];
#pragma unroll
  for (int g = 0; g < kAttnMaxGroup; g++) acc[g] = 0.0f;
#pragma unroll
  for (int r = 0; r < NR; r++) {
    const uint32_t col = qq + 4 * r;
    if (col < q4) {
      const float4 kv = kreg[r];
#pragma unroll
      for (int g = 0; g < kAttnMaxGroup; g++) {
        if ((uint32_t)g < G) {
          const float4 qv = reinterpret_cast<const float4*>(qs + g * hd)[col];
          float v = acc[g];
          v = fmaf(qv.x, kv.x, v);
          v = fmaf(qv.y, kv.y, v);
          v = fmaf(qv.z, kv.z, v);
          v = fmaf(qv.w, kv.w, v);
          acc[g] = v;
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < kAttnMaxGroup; g++) {
    if ((uint32_t)g < G) {
      float v = acc[g];
      v += dpp_f<kDppXor1>(v);
      v += dpp_f<kDppXor2>(v);
      if (qq == 0) ps(g, j) = rowok ? v * a.scale : -INFINITY;
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++) {
    const uint32_t col = qq + 4 * r;
    if (rowok && col < q4) reinterpret_cast<float4*>(tile + j * hd)[col] = vreg[r];
  }
  __syncthreads();
  // per head: max and sum over the chunk, one wave per head in turn. A NaN or +inf score
  // makes the reference's softmax uniform over the whole span (simd/mod.rs:132-158): the
  // chunk's max is then NaN, which the combine reads as that mark.
  const uint32_t lane = t & 63, w = t >> 6;
  for (uint32_t g = w; g < G; g += 4) {
    const float sc = ps(g, lane);  // kAttnChunk == 64: one position a lane
    const bool bad = __ballot(lane < cnt && (sc != sc || sc == INFINITY)) != 0ull;
    const float m = wave_max(sc);
    const float pv = lane < cnt && !bad ? gm_expf(sc - m) : 0.0f;
    ps(g, lane) = pv;
    const float l = wave_sum(pv);
    if (lane == 0) {
      ml(g, 0) = bad ? __int_as_float(0x7fc00000) : m;
      ml(g, 1) = l;
    }
  }
  __syncthreads();
  // o: item = (head, float4 column); with few items the positions split into parts
  const uint32_t items = G * q4;
  const float4* tile4 = reinterpret_cast<const float4*>(tile);
  auto pv_sum = [&](uint32_t item, uint32_t j0, uint32_t j1) {
    const uint32_t g = item / q4, d4 = item % q4;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t jj = j0; jj < j1; jj++) {
      const float p = ps(g, jj);
      const float4 v = tile4[jj * q4 + d4];
      o.x = fmaf(p, v.x, o.x);
      o.y = fmaf(p, v.y, o.y);
      o.z = fmaf(p, v.z, o.z);
      o.w = fmaf(p, v.w, o.w);
    }
    return o;
  };
  auto put = [&](uint32_t item, float4 o) {
    float* dst = out + (item / q4) * gstride + 4 * (item % q4);
    dst[0] = o.x; dst[1] = o.y; dst[2] = o.z; dst[3] = o.w;
  };
  if (items <= 128) {
    const uint32_t parts = items <= 64 ? 4u : 2u, span = kAttnChunk / parts;
    if (t < items * parts) {
      const uint32_t part = t / items, j0 = part * span;
      og[t] = pv_sum(t % items, min(j0, cnt), min(j0 + span, cnt));
    }
    __syncthreads();
    if (t < items) {
      float4 o = og[t];
      for (uint32_t part = 1; part < parts; part++) {
        const float4 v = og[part * items + t];
        o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
      }
      put(t, o);
    }
  } else {
    for (uint32_t x = t; x < items; x += 256) put(x, pv_sum(x, 0, cnt));
  }
  if (t < G) {
    out[t * gstride + hd] = ml(t, 0);
    out[t * gstride + hd + 1] = ml(t, 1);
  }
}

// The reference's softmax falls back to uniform weights when a score is NaN or +inf, or
// every score is -inf (simd/mod.rs:132-158); the context is then the values' plain mean,
// summed as add_scaled does (out += v * (1 / len), positions in order). Column d of
// query head hh; runs only on that rare input.
__device__ float attn_uniform(const AttnArgs& a, uint32_t i, uint32_t hh, uint32_t d) {
  const AttnEntry e = entry(a, i);
  const uint32_t kh = hh / (a.n_heads / a.n_kv), len = e.pos + 1 - e.start;
  const float u = fdiv(1.0f, (float)len);
  const size_t voff = (size_t)a.bs * a.n_kv * a.hd;
  float acc = 0.0f;
  for (uint32_t p = e.start; p <= e.pos; p++) acc = acc + key_row(a, e, p, kh)[voff + d] * u;
  return acc;
}

// grid (n, n_heads), 256 threads: the chunks merged, context = o / l, in one pass.
// Thread (g, d) with g < 256 / hd runs over the chunks c = g, g + 256 / hd, ... of column
// d (16 chunks in flight) with a running max: (M, L, O) is rescaled when a chunk's max
// exceeds M. The groups are then merged in group order. A chunk marked NaN (a NaN or
// +inf score), or no finite score at all, gives the uniform weights of attn_uniform.
__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a) {
  __shared__ float gm[256], gl[256], go[256];
  const uint32_t i = blockIdx.x, hh = blockIdx.y, t = threadIdx.x, hd = a.hd, row = hd + 2, nc = a.nchunk;
  const float* base = a.part + ((size_t)i * a.n_heads + hh) * nc * row;
  const uint32_t ng = 256 / hd, g = t / hd, d = t % hd;
  float M = -INFINITY, L = 0.0f, O = 0.0f;
  bool bad = false;
  if (g < ng) {
    constexpr int kIn = 16;
    for (uint32_t c0 = g; c0 < nc; c0 += kIn * ng) {
      float mv[kIn], lv[kIn], pv[kIn];
#pragma unroll
      for (int r = 0; r < kIn; r++) {
        const uint32_t c = c0 + r * ng;
        mv[r] = -INFINITY;
        if (c < nc) {
          const float* rc = base + (size_t)c * row;
          mv[r] = rc[hd];
          lv[r] = rc[hd + 1];
          pv[r] = rc[d];
        }
      }
#pragma unroll
      for (int r = 0; r < kIn; r++) {
        if (mv[r] != mv[r]) {  // a NaN or +inf score in that chunk
          bad = true;
          continue;
        }
        if (mv[r] == -INFINITY) continue;  // an empty chunk
        if (mv[r] > M) {
          const float f = gm_expf(M - mv[r]);  // 0 while M is -inf
          L = fmaf(L, f, lv[r]);
          O = fmaf(O, f, pv[r]);
          M = mv[r];
        } else {
          const float f = gm_expf(mv[r] - M);
          L = fmaf(lv[r], f, L);
          O = fmaf(pv[r], f, O);
        }
      }
    }
  }
  gm[t] = bad ? __int_as_float(0x7fc00000) : M;
  gl[t] = L;
  go[t] = O;
  __syncthreads();
  if (t < hd) {
    float Mt = gm[t], Lt = gl[t], Ot = go[t];
    bool bad_t = Mt != Mt;
    if (bad_t) Mt = -INFINITY;
    for (uint32_t k = 1; k < ng; k++) {
      const float m2 = gm[k * hd + t];
      if (m2 != m2) {
        bad_t = true;
        continue;
      }
      if (m2 == -INFINITY) continue;
      if (m2 > Mt) {
        const float f = gm_expf(Mt - m2);
        Lt = fmaf(Lt, f, gl[k * hd + t]);
        Ot = fmaf(Ot, f, go[k * hd + t]);
        Mt = m2;
      } else {
        const float f = gm_expf(m2 - Mt);
        Lt = fmaf(gl[k * hd + t], f, Lt);
        Ot = fmaf(go[k * hd + t], f, Ot);
      }
    }
    a.ctx[(size_t)i * a.n_heads * hd + hh * hd + t] =
        bad_t || Mt == -INFINITY ? attn_uniform(a, i, hh, t) : Ot / Lt;
  }
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
  const uint32_t pairs = (a.n_heads + a.n_kv) * a.hd / 2;
  hipLaunchKernelGGL(k_rope_append, dim3(a.n, (pairs + 255) / 256), dim3(256), 0, st, a);
  static const bool once =
      hipFuncSetAttribute((const void*)k_attn_partial<128>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)attn_lds_bytes(kAttnMaxGroup, 128)) == hipSuccess &&
      hipFuncSetAttribute((const void*)k_attn_partial<kAttnMaxHd>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)attn_lds_bytes(kAttnMaxGroup, kAttnMaxHd)) == hipSuccess;
  (void)once;
  const dim3 grid(a.n, a.n_kv, a.nchunk);
  const uint32_t lds = attn_lds_bytes(a.n_heads / a.n_kv, a.hd);
  if (a.hd <= 128) hipLaunchKernelGGL(k_attn_partial<128>, grid, dim3(256), lds, st, a);
  else hipLaunchKernelGGL(k_attn_partial<kAttnMaxHd>, grid, dim3(256), lds, st, a);
  hipLaunchKernelGGL(k_attn_combine, dim3(a.n, a.n_heads), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace gmoe
