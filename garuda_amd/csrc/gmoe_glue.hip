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

__device__ __forceinline__ float glue_wave_sum(float v) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace

// grid n, 256 threads: x[i] = table[tokens[i]] (f32 rows of width d)
__global__ void __launch_bounds__(256) k_embed(GlueTokens tk, const float* __restrict__ table, uint32_t d,
                                               float* __restrict__ x) {
  const uint32_t i = blockIdx.x;
  const float4* src = reinterpret_cast<const float4*>(table + (size_t)tk.tok[i] * d);
  float4* dst = reinterpret_cast<float4*>(x + (size_t)i * d);
  for (uint32_t c = threadIdx.x; c < d / 4; c += blockDim.x) dst[c] = src[c];
}

// grid n, 256 threads: with y, x[i] += y[i] first (written back); then
// h[i] = (x[i] * scale) * w with scale = 1 / sqrt(mean(x[i]^2) + eps).
__global__ void __launch_bounds__(256) k_add_norm(float* __restrict__ x, const float* __restrict__ y,
                                                  const float* __restrict__ w, uint32_t d, float eps,
                                                  float* __restrict__ h) {
  __shared__ float part[4];
  const uint32_t i = blockIdx.x, t = threadIdx.x;
  float* xr = x + (size_t)i * d;
  const float* yr = y ? y + (size_t)i * d : nullptr;
  float sq = 0.0f;
  for (uint32_t c = t; c < d; c += 256) {
    float v = xr[c];
    if (yr) {
      v = v + yr[c];
      xr[c] = v;
    }
    sq = sq + v * v;
  }
  sq = glue_wave_sum(sq);
  if ((t & 63) == 0) part[t >> 6] = sq;
  __syncthreads();
  const float mean = (part[0] + part[1] + part[2] + part[3]) / (float)d;
  const float scale = fdiv(1.0f, __fsqrt_rn(mean + eps));
  float* hr = h + (size_t)i * d;
  for (uint32_t c = t; c < d; c += 256) hr[c] = (xr[c] * scale) * w[c];
}

// grid n, 256 threads: next[i] = the first index of row i's largest value
__global__ void __launch_bounds__(256) k_argmax(const float* __restrict__ logits, uint32_t vocab,
                                                uint32_t* __restrict__ next) {
  __shared__ float bvs[4];
  __shared__ uint32_t bis[4];
  const uint32_t i = blockIdx.x, t = threadIdx.x;
  const float* row = logits + (size_t)i * vocab;
  float bv = -INFINITY;
  uint32_t bi = ~0u;
  for (uint32_t c = t; c < vocab; c += 256) {  // ascending: keeps the thread's first maximum
    const float v = row[c];
    if (v > bv) {
      bv = v;
      bi = c;
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

hipError_t launch_add_norm(float* x, const float* y, const float* w, uint32_t n, uint32_t d, float eps, float* h,
                           hipStream_t st) {
  hipLaunchKernelGGL(k_add_norm, dim3(n), dim3(256), 0, st, x, y, w, d, eps, h);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t vocab, uint32_t* next, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax, dim3(n), dim3(256), 0, st, logits, vocab, next);
  return hipGetLastError();
}

}  // namespace gmoe
