// gmoe_glue.hip — the small per-token steps of a decode step around the MoE layer,
// dense projections and attention: embedding rows, RMSNorm with its weight (and the
// residual add before it), and greedy token choice.
//
// Reference: LlamaBackend::logits_batch / layer_batch_over (garuda/src/llama/mod.rs
// :1134-1206, :851-893): x = token_embd.row(token); per layer h = norm(x, attn_norm),
// x += wo(attention(h)), h = norm(x, ffn_norm), x += ffn(h); then norm(x, output_norm)
// and the output head. norm is simd::rmsnorm (simd/mod.rs:166-173: mean of squares,
// scale = 1 / sqrt(mean + eps), x *= scale) then mul_assign by the weight; add_assign
// is x += y. Greedy sampling (runtime/mod.rs:98-105) takes the first index of the
// largest value; NaN never wins and an all -inf (or NaN) row gives 0.
//
// The mean of squares is a parallel sum here (the reference's is sequential), so a
// norm matches the reference's within rounding, not bit for bit.
#include "gmoe_device.h"

namespace gmoe {

namespace {

__device__ __forceinline__ float glue_wave_sum(float v) { return wave64_sum(v); }

}  // namespace

// grid n, 256 threads: x[i] = table[tokens[i]] (f32 rows of width d)
__global__ void __launch_bounds__(256) k_embed(GlueTokens tk, const float* __restrict__ table, uint32_t d,
                                               float* __restrict__ x) {
  const uint32_t i = blockIdx.x;
  const float4* src = reinterpret_cast<const float4*>(table + (size_t)tk.tok[i] * d);
  float4* dst = reinterpret_cast<float4*>(x + (size_t)i * d);
  for (uint32_t c = threadIdx.x; c < d / 4; c += blockDim.x) dst[c] = src[c];
}

// The same with the tokens in device memory (a decode step replayed from a graph).
__global__ void __launch_bounds__(256) k_embed_dev(const uint32_t* __restrict__ tok, const float* __restrict__ table,
                                                   uint32_t d, float* __restrict__ x) {
  const uint32_t i = blockIdx.x;
  const float4* src = reinterpret_cast<const float4*>(table + (size_t)tok[i] * d);
  float4* dst = reinterpret_cast<float4*>(x + (size_t)i * d);
  for (uint32_t c = threadIdx.x; c < d / 4; c += blockDim.x) dst[c] = src[c];
}

// grid n, 256 threads: with y, x[i] += y[i] first (written back); then
// h[i] = (x[i] * scale) * w with scale = 1 / sqrt(mean(x[i]^2) + eps). A thread holds its
// kNormVec float4 of the row (d <= 4 * 256 * kNormVec, checked by the model) in
// registers, every load issued before any use. SL: y is the sum of nsl K slices of a
// dense product, `stride` floats apart, added in slice order (k_reduce_parts's sum) before
// it is added to x; a float4's slice loads are issued together (slice indices clamped,
// the surplus ones not added).
template <bool SL>
__global__ void __launch_bounds__(256) k_add_norm(float* __restrict__ x, const float* __restrict__ y,
                                                  const float* __restrict__ w, uint32_t d, float eps,
                                                  float* __restrict__ h, uint32_t nsl, size_t stride) {
  __shared__ float part[4];
  const uint32_t i = blockIdx.x;
  add_norm_row<SL>(x + (size_t)i * d, y ? y + (size_t)i * d : nullptr, w, d, eps, h + (size_t)i * d, nullptr, nsl,
                   stride, part);
}

// grid n, 256 threads: next[i] = the first index of row i's largest value
__global__ void __launch_bounds__(256) k_argmax(const float* __restrict__ logits, uint32_t vocab,
                                                uint32_t* __restrict__ next) {
  constexpr int U = 8;  // loads in flight per thread
  __shared__ float bvs[4];
  __shared__ uint32_t bis[4];
  const uint32_t i = blockIdx.x, t = threadIdx.x;
  const float* row = logits + (size_t)i * vocab;
  float bv = -INFINITY;
  uint32_t bi = ~0u;
  for (uint32_t c0 = t; c0 < vocab; c0 += 256 * U) {  // ascending: keeps the thread's first maximum
    float v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t c = c0 + 256 * u;
      v[u] = c < vocab ? row[c] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (v[u] > bv) {
        bv = v[u];
        bi = c0 + 256 * u;
      }
  }
  // larger value first, then the lower index (an index of ~0u found nothing)
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((t & 63) == 0) {
    bvs[t >> 6] = bv;
    bis[t >> 6] = bi;
  }
  __syncthreads();
  if (t == 0) {
    for (int k = 1; k < 4; k++)
      if (bvs[k] > bv || (bvs[k] == bv && bis[k] < bi)) {
        bv = bvs[k];
        bi = bis[k];
      }
    next[i] = bi == ~0u ? 0u : bi;
  }
}

hipError_t launch_embed(const GlueTokens& tk, uint32_t n, const float* table, uint32_t d, float* x, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(n), dim3(256), 0, st, tk, table, d, x);
  return hipGetLastError();
}

hipError_t launch_embed_dev(const uint32_t* tok, uint32_t n, const float* table, uint32_t d, float* x, hipStream_t st) {
  hipLaunchKernelGGL(k_embed_dev, dim3(n), dim3(256), 0, st, tok, table, d, x);
  return hipGetLastError();
}

hipError_t launch_add_norm(float* x, const float* y, const float* w, uint32_t n, uint32_t d, float eps, float* h,
                           hipStream_t st) {
  hipLaunchKernelGGL(k_add_norm<false>, dim3(n), dim3(256), 0, st, x, y, w, d, eps, h, 1u, (size_t)0);
  return hipGetLastError();
}

hipError_t launch_add_norm_slices(float* x, const float* parts, uint32_t nsl, const float* w, uint32_t n, uint32_t d,
                                  float eps, float* h, hipStream_t st) {
  if (nsl == 0 || nsl > kMaxKsg || d % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_add_norm<true>, dim3(n), dim3(256), 0, st, x, parts, w, d, eps, h, nsl, (size_t)n * d);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t vocab, uint32_t* next, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax, dim3(n), dim3(256), 0, st, logits, vocab, next);
  return hipGetLastError();
}

}  // namespace gmoe
