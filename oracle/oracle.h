/*
 * oracle.h — CPU restatement of Garuda's mixture-of-experts feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * never as the thing measured or shipped. The product (garuda_amd/) does not
 * link, load or call it.
 *
 * Every function restates one function of the reference (hanumanit/garuda,
 * crate 0.31.0, Rust) in the reference's own operation order, so that float
 * results match bit for bit wherever the reference is deterministic:
 *   garuda/src/quant/mod.rs   block layouts, dequantisers, int8 activation
 *                             quantiser, packed-row int8 dot kernels
 *   garuda/src/simd/mod.rs    f32 dot/matvec/softmax/silu/add_scaled
 *   garuda/src/router/mod.rs  synthetic-engine gating variants
 *   garuda/src/llama/mod.rs   feed_forward_batch / expert_batch
 *   garuda/src/moe/mod.rs     synthetic engine moe_ffn / expert_ffn
 *   garuda/src/weights/mod.rs splitmix64 / seeded / synthesize_expert
 * It is compiled with -ffp-contract=off because rustc never fuses a multiply
 * and an add; `expf` is the host libm's, which is what Rust's f32::exp calls
 * on Linux.
 */
#ifndef GARUDA_ORACLE_H
#define GARUDA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, garuda/src/quant/mod.rs:22-30 */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q8_0 = 8, OR_Q2_K = 10,
       OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14 };

/* Status codes: 0 ok, 1 model error (bad type/length), 2 inference error (shape). */
int   or_block_layout(uint32_t qtype, size_t* elems, size_t* bytes);
int   or_byte_size(uint32_t qtype, size_t n, size_t* out);
float or_f16_to_f32(uint16_t h);
void  or_get_scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m);
void  or_unpack_q3_k_scales(const uint8_t* scale_bytes, int8_t out[16]);
int   or_dequant_into(uint32_t qtype, const uint8_t* raw, size_t raw_len, float* out, size_t n);
int   or_dequantize(uint32_t qtype, const uint8_t* raw, size_t raw_len, float* out, size_t n);

void  or_quantize_activation(const float* x, size_t n, int8_t* xq, float* xs);
void  or_block_sums(const int8_t* xq, size_t n, size_t width, int32_t* sums);
int   or_sum_width(uint32_t qtype);
int   or_has_int8_kernel(uint32_t qtype);
float or_int8_dot(uint32_t qtype, const uint8_t* row, const int8_t* xq, const float* xs,
                  const int32_t* sums);

/* Packed path: quant::matvec / quant::matmul (rows split over `threads` workers). */
int   or_matvec(uint32_t qtype, const uint8_t* w, size_t w_len, size_t rows, size_t cols,
                const float* x, float* out, int threads);
int   or_matmul(uint32_t qtype, const uint8_t* w, size_t w_len, size_t rows, size_t cols,
                const float* xs, size_t n, float* out, int threads);

/* simd::* */
float or_dot(const float* a, const float* b, size_t n);
void  or_simd_matvec(const float* m, size_t rows, size_t cols, const float* x, float* out,
                     int threads);
void  or_simd_matmul(const float* m, size_t rows, size_t cols, const float* xs, size_t n,
                     float* out, int threads);
void  or_softmax(float* x, size_t n);
void  or_expf(const float* x, size_t n, float* y);  /* host libm expf, elementwise */
void  or_silu(float* x, size_t n);
void  or_add_scaled(float* a, const float* b, size_t n, float k);
void  or_mul_assign(float* a, const float* b, size_t n);

/* Gating. kind: 0 llama (llama/mod.rs:938-949), 1 Mixtral, 2 DeepSeek, 3 QwenMoe
 * (router/mod.rs:58-118). `scores` holds the ne router logits and is consumed. */
void  or_gate(int kind, float* scores, int ne, int k, uint32_t* ids, float* w);

/* One MoE feed-forward layer. */
typedef struct {
  int d, f, ne, k;
  int gating;   /* as or_gate */
  int combine;  /* 0 ascending expert id (llama/mod.rs:977-995), 1 routed rank (moe/mod.rs:104-109) */
  int packed;   /* 1: Weight::Packed (mmap=true) -> quant::matmul; 0: Weight::Full -> simd::matmul */
  const float* router;          /* [ne * d] f32 */
  uint32_t qt_gate, qt_up, qt_down;
  const uint8_t* gate;          /* stacked: ne*f rows of byte_size(qt_gate, d) */
  const uint8_t* up;
  const uint8_t* down;          /* ne*d rows of byte_size(qt_down, f) */
  const float* gate_f32;        /* optional pre-dequantised copies for packed == 0 */
  const float* up_f32;
  const float* down_f32;
} or_moe_layer;

/* llama::LlamaBackend::feed_forward_batch for Ffn::Moe (llama/mod.rs:903-998).
 * logits: optional [n*ne] router logits that replace the router matvec.
 * ids/w: optional [n*k] outputs, the routed experts per token in ranked order. */
int or_feed_forward_batch(const or_moe_layer* L, const float* hs, int n, float* out,
                          uint32_t* ids, float* w, const float* logits, int threads);

/* weights/mod.rs:17-109 */
uint64_t or_splitmix64(uint64_t* state);
void  or_seeded(uint64_t seed, size_t n, float bound, float* out);
float or_bound(size_t fan_in);
void  or_synthesize_expert(uint32_t id, int d, int f, float* gate, float* up, float* down);

#ifdef __cplusplus
}
#endif
#endif
