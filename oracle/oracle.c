/*
 * oracle.c — CPU restatement of Garuda's MoE feed-forward path (test infrastructure).
 * See oracle.h for the rules this file follows. Each function names the reference
 * lines it restates; the arithmetic is kept in the reference's order.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define QK_K 256

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* quant/mod.rs:41-61 */
int or_block_layout(uint32_t t, size_t* elems, size_t* bytes) {
  size_t e, b;
  switch (t) {
    case OR_F32: e = 1; b = 4; break;
    case OR_F16: e = 1; b = 2; break;
    case OR_Q4_0: e = QK; b = 2 + QK / 2; break;
    case OR_Q8_0: e = QK; b = 2 + QK; break;
    case OR_Q2_K: e = QK_K; b = QK_K / 16 + QK_K / 4 + 2 + 2; break;
    case OR_Q3_K: e = QK_K; b = QK_K / 8 + QK_K / 4 + 12 + 2; break;
    case OR_Q4_K: e = QK_K; b = 2 + 2 + 12 + QK_K / 2; break;
    case OR_Q5_K: e = QK_K; b = 2 + 2 + 12 + QK_K / 8 + QK_K / 2; break;
    case OR_Q6_K: e = QK_K; b = QK_K / 2 + QK_K / 4 + QK_K / 16 + 2; break;
    default: return 1;
  }
  if (elems) *elems = e;
  if (bytes) *bytes = b;
  return 0;
}

/* quant/mod.rs:89-98 */
int or_byte_size(uint32_t t, size_t n, size_t* out) {
  size_t e, b;
  if (or_block_layout(t, &e, &b)) return 1;
  if (n % e != 0) return 1;
  *out = (n / e) * b;
  return 0;
}

/* quant/mod.rs:878-890. Every branch is exact in f32. */
float or_f16_to_f32(uint16_t h) {
  unsigned sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, mant = h & 0x3ff;
  float val;
  if (exp == 0 && mant == 0) val = 0.0f;
  else if (exp == 0) val = (float)mant * ldexpf(1.0f, -24);
  else if (exp == 0x1f && mant == 0) val = INFINITY;
  else if (exp == 0x1f) val = NAN;
  else val = (1.0f + (float)mant / 1024.0f) * ldexpf(1.0f, (int)exp - 15);
  return sign ? -val : val;
}

/* quant/mod.rs:656-664 */
void or_get_scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
    *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* quant/mod.rs:812-833 */
void or_unpack_q3_k_scales(const uint8_t* sb, int8_t out[16]) {
  const uint32_t KMASK1 = 0x03030303u, KMASK2 = 0x0f0f0f0fu;
  uint32_t aux[4];
  aux[0] = rd32(sb);
  aux[1] = rd32(sb + 4);
  aux[2] = rd32(sb + 8);
  uint32_t tmp = aux[2];
  aux[2] = ((aux[0] >> 4) & KMASK2) | (((tmp >> 4) & KMASK1) << 4);
  aux[3] = ((aux[1] >> 4) & KMASK2) | (((tmp >> 6) & KMASK1) << 4);
  aux[0] = (aux[0] & KMASK2) | ((tmp & KMASK1) << 4);
  aux[1] = (aux[1] & KMASK2) | (((tmp >> 2) & KMASK1) << 4);
  for (int k = 0; k < 4; k++)
    for (int b = 0; b < 4; b++) out[k * 4 + b] = (int8_t)((aux[k] >> (8 * b)) & 0xff);
}

/* quant/mod.rs:624-632 */
static void dq_q8_0(const uint8_t* raw, float* out, size_t n) {
  for (size_t bi = 0; bi < n / QK; bi++) {
    const uint8_t* blk = raw + bi * (2 + QK);
    float scale = or_f16_to_f32(rd16(blk));
    for (int i = 0; i < QK; i++) out[bi * QK + i] = scale * (float)(int8_t)blk[2 + i];
  }
}

/* quant/mod.rs:637-648 */
static void dq_q4_0(const uint8_t* raw, float* out, size_t n) {
  for (size_t b = 0; b < n / QK; b++) {
    const uint8_t* blk = raw + b * (2 + QK / 2);
    float scale = or_f16_to_f32(rd16(blk));
    for (int i = 0; i < QK / 2; i++) {
      int lo = (blk[2 + i] & 0x0F) - 8, hi = (blk[2 + i] >> 4) - 8;
      out[b * QK + i] = scale * (float)lo;
      out[b * QK + i + QK / 2] = scale * (float)hi;
    }
  }
}

/* quant/mod.rs:671-696 */
static void dq_q4_k(const uint8_t* raw, float* out, size_t n) {
  for (size_t bi = 0; bi < n / QK_K; bi++) {
    const uint8_t* b = raw + bi * 144;
    float d = or_f16_to_f32(rd16(b)), dmin = or_f16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4, *qs = b + 16;
    size_t w = bi * QK_K;
    int is = 0;
    for (int c = 0; c < 4; c++) {
      const uint8_t* chunk = qs + c * 32;
      uint8_t sc1, m1, sc2, m2;
      or_get_scale_min_k4(is, scales, &sc1, &m1);
      or_get_scale_min_k4(is + 1, scales, &sc2, &m2);
      float d1 = d * (float)sc1, mn1 = dmin * (float)m1;
      float d2 = d * (float)sc2, mn2 = dmin * (float)m2;
      for (int l = 0; l < 32; l++) out[w++] = d1 * (float)(chunk[l] & 0x0F) - mn1;
      for (int l = 0; l < 32; l++) out[w++] = d2 * (float)(chunk[l] >> 4) - mn2;
      is += 2;
    }
  }
}

/* quant/mod.rs:704-731 */
static void dq_q6_k(const uint8_t* raw, float* out, size_t n) {
  for (size_t bi = 0; bi < n / QK_K; bi++) {
    const uint8_t* blk = raw + bi * 210;
    float d = or_f16_to_f32(rd16(blk + 208));
    size_t sb = bi * QK_K;
    for (int half = 0; half < 2; half++) {
      const uint8_t* ql = blk + half * 64;
      const uint8_t* qh = blk + 128 + half * 32;
      const uint8_t* sc = blk + 192 + half * 8;
      size_t y = sb + half * 128;
      for (int l = 0; l < 32; l++) {
        int is = l / 16;
        int q1 = (int)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
        int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
        int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        out[y + l] = d * (float)(int8_t)sc[is] * (float)q1;
        out[y + l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
        out[y + l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
        out[y + l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
      }
    }
  }
}

/* quant/mod.rs:737-769 */
static void dq_q5_k(const uint8_t* raw, float* out, size_t n) {
  for (size_t bi = 0; bi < n / QK_K; bi++) {
    const uint8_t* b = raw + bi * 176;
    float d = or_f16_to_f32(rd16(b)), dmin = or_f16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    size_t w = bi * QK_K;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int g = 0; g < 4; g++) {
      const uint8_t* ql = qs + g * 32;
      uint8_t sc1, m1, sc2, m2;
      or_get_scale_min_k4(is, scales, &sc1, &m1);
      or_get_scale_min_k4(is + 1, scales, &sc2, &m2);
      float d1 = d * (float)sc1, mn1 = dmin * (float)m1;
      float d2 = d * (float)sc2, mn2 = dmin * (float)m2;
      for (int l = 0; l < 32; l++) {
        int hi = (qh[l] & u1) ? 16 : 0;
        out[w++] = d1 * (float)((ql[l] & 0x0F) + hi) - mn1;
      }
      for (int l = 0; l < 32; l++) {
        int hi = (qh[l] & u2) ? 16 : 0;
        out[w++] = d2 * (float)((ql[l] >> 4) + hi) - mn2;
      }
      is += 2;
      u1 = (uint8_t)(u1 << 2);
      u2 = (uint8_t)(u2 << 2);
    }
  }
}

/* quant/mod.rs:775-806 */
static void dq_q2_k(const uint8_t* raw, float* out, size_t n) {
  for (size_t bi = 0; bi < n / QK_K; bi++) {
    const uint8_t* b = raw + bi * 84;
    const uint8_t *scales = b, *qs = b + 16;
    float d = or_f16_to_f32(rd16(b + 80)), dmin = or_f16_to_f32(rd16(b + 82));
    size_t w = bi * QK_K;
    int is = 0;
    for (int half = 0; half < 2; half++) {
      const uint8_t* q = qs + half * 32;
      int shift = 0;
      for (int j = 0; j < 4; j++) {
        for (int off = 0; off < 32; off += 16) {
          uint8_t sc = scales[is++];
          float dl = d * (float)(sc & 0x0F), ml = dmin * (float)(sc >> 4);
          for (int l = 0; l < 16; l++) out[w++] = dl * (float)((q[off + l] >> shift) & 3) - ml;
        }
        shift += 2;
      }
    }
  }
}

/* quant/mod.rs:840-875 */
static void dq_q3_k(const uint8_t* raw, float* out, size_t n) {
  for (size_t bi = 0; bi < n / QK_K; bi++) {
    const uint8_t* b = raw + bi * 110;
    const uint8_t *hmask = b, *qs = b + 32;
    float d_all = or_f16_to_f32(rd16(b + 108));
    int8_t scales[16];
    or_unpack_q3_k_scales(b + 96, scales);
    size_t w = bi * QK_K;
    int is = 0;
    uint8_t m = 1;
    for (int half = 0; half < 2; half++) {
      const uint8_t* q = qs + half * 32;
      int shift = 0;
      for (int j = 0; j < 4; j++) {
        for (int off = 0; off < 32; off += 16) {
          float dl = d_all * (float)((int)scales[is++] - 32);
          for (int l = 0; l < 16; l++) {
            int hbit = (hmask[l + off] & m) ? 0 : 4;
            out[w++] = dl * (float)((int)((q[l + off] >> shift) & 3) - hbit);
          }
        }
        shift += 2;
        m = (uint8_t)(m << 1);
      }
    }
  }
}

/* quant/mod.rs:119-150 */
int or_dequant_into(uint32_t t, const uint8_t* raw, size_t raw_len, float* out, size_t n) {
  size_t expected;
  if (or_byte_size(t, n, &expected)) return 1;
  if (raw_len != expected) return 1;
  switch (t) {
    case OR_F32:
      for (size_t i = 0; i < n; i++) {
        uint32_t u = rd32(raw + 4 * i);
        memcpy(&out[i], &u, 4);
      }
      break;
    case OR_F16:
      for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(rd16(raw + 2 * i));
      break;
    case OR_Q8_0: dq_q8_0(raw, out, n); break;
    case OR_Q4_0: dq_q4_0(raw, out, n); break;
    case OR_Q2_K: dq_q2_k(raw, out, n); break;
    case OR_Q3_K: dq_q3_k(raw, out, n); break;
    case OR_Q4_K: dq_q4_k(raw, out, n); break;
    case OR_Q5_K: dq_q5_k(raw, out, n); break;
    case OR_Q6_K: dq_q6_k(raw, out, n); break;
    default: return 1;
  }
  return 0;
}

/* quant/mod.rs:104-114: as dequant_into, plus the non-finite refusal. */
int or_dequantize(uint32_t t, const uint8_t* raw, size_t raw_len, float* out, size_t n) {
  int rc = or_dequant_into(t, raw, raw_len, out, n);
  if (rc) return rc;
  for (size_t i = 0; i < n; i++)
    if (!isfinite(out[i])) return 1;
  return 0;
}

/* quant/mod.rs:331-345. Rust's f32::round is half-away-from-zero (C roundf); its
 * clamp keeps NaN and `as i8` maps NaN to 0. */
void or_quantize_activation(const float* x, size_t n, int8_t* xq, float* xs) {
  for (size_t b = 0; b < n / QK; b++) {
    const float* blk = x + b * QK;
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(blk[j]));
    float scale = amax / 127.0f;
    xs[b] = scale;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    for (int j = 0; j < QK; j++) {
      float v = roundf(blk[j] * inv);
      int8_t q;
      if (isnan(v)) q = 0;
      else if (v < -127.0f) q = -127;
      else if (v > 127.0f) q = 127;
      else q = (int8_t)v;
      xq[b * QK + j] = q;
    }
  }
}

/* quant/mod.rs:322-326 */
void or_block_sums(const int8_t* xq, size_t n, size_t width, int32_t* sums) {
  for (size_t b = 0; b < n / width; b++) {
    int32_t s = 0;
    for (size_t j = 0; j < width; j++) s += xq[b * width + j];
    sums[b] = s;
  }
}

/* quant/mod.rs:368-375 */
int or_sum_width(uint32_t t) {
  if (t == OR_Q4_K || t == OR_Q5_K) return 32;
  if (t == OR_Q2_K) return 16;
  return 0;
}

/* quant/mod.rs:379-381 */
int or_has_int8_kernel(uint32_t t) {
  return t == OR_Q8_0 || t == OR_Q2_K || t == OR_Q3_K || t == OR_Q4_K || t == OR_Q5_K ||
         t == OR_Q6_K;
}

/* simd/mod.rs:23-39 (exact integer sum, any order). */
static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int n) {
  int32_t s = 0;
  for (int i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
  return s;
}

/* quant/mod.rs:398-407 */
static float q8_0_dot(const uint8_t* row, size_t nblk, const int8_t* xq, const float* xs) {
  float sum = 0.0f;
  for (size_t b = 0; b < nblk; b++) {
    const uint8_t* blk = row + b * (2 + QK);
    float ws = or_f16_to_f32(rd16(blk));
    sum += ws * xs[b] * (float)dot_i8((const int8_t*)(blk + 2), xq + b * QK, QK);
  }
  return sum;
}

/* quant/mod.rs:417-445 */
static float q6_k_dot(const uint8_t* row, size_t nsb, const int8_t* xq, const float* xs) {
  float acc = 0.0f;
  int8_t q[QK_K];
  for (size_t bi = 0; bi < nsb; bi++) {
    const uint8_t* block = row + bi * 210;
    float d = or_f16_to_f32(rd16(block + 208));
    const uint8_t* sc = block + 192;
    for (int half = 0; half < 2; half++) {
      const uint8_t* ql = block + half * 64;
      const uint8_t* qh = block + 128 + half * 32;
      int y = half * 128;
      for (int l = 0; l < 32; l++) {
        q[y + l] = (int8_t)(((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32);
        q[y + l + 32] = (int8_t)(((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32);
        q[y + l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
        q[y + l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
      }
    }
    size_t base = bi * QK_K;
    for (int s = 0; s < 16; s++) {
      size_t off = base + s * 16;
      float dot = (float)dot_i8(q + s * 16, xq + off, 16);
      acc += xs[off / QK] * d * (float)(int8_t)sc[s] * dot;
    }
  }
  return acc;
}

/* quant/mod.rs:454-495 */
static float q5_k_dot(const uint8_t* row, size_t nsb, const int8_t* xq, const float* xs,
                      const int32_t* sums) {
  float acc = 0.0f;
  int8_t q[QK];
  for (size_t bi = 0; bi < nsb; bi++) {
    const uint8_t* block = row + bi * 176;
    float d = or_f16_to_f32(rd16(block)), dmin = or_f16_to_f32(rd16(block + 2));
    const uint8_t *scales = block + 4, *qh = block + 16, *qs = block + 48;
    size_t base = bi * 8;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int g = 0; g < 4; g++) {
      const uint8_t* ql = qs + g * 32;
      uint8_t sc1, m1, sc2, m2;
      or_get_scale_min_k4(is, scales, &sc1, &m1);
      or_get_scale_min_k4(is + 1, scales, &sc2, &m2);
      for (int l = 0; l < QK; l++) q[l] = (int8_t)((ql[l] & 0x0F) | ((qh[l] & u1) ? 16 : 0));
      size_t sb = base + is, off = sb * QK;
      float dot = (float)dot_i8(q, xq + off, QK);
      acc += xs[sb] * (d * (float)sc1 * dot - dmin * (float)m1 * (float)sums[sb]);
      for (int l = 0; l < QK; l++) q[l] = (int8_t)((ql[l] >> 4) | ((qh[l] & u2) ? 16 : 0));
      sb = sb + 1;
      off = sb * QK;
      dot = (float)dot_i8(q, xq + off, QK);
      acc += xs[sb] * (d * (float)sc2 * dot - dmin * (float)m2 * (float)sums[sb]);
      is += 2;
      u1 = (uint8_t)(u1 << 2);
      u2 = (uint8_t)(u2 << 2);
    }
  }
  return acc;
}

/* quant/mod.rs:503-540 */
static float q3_k_dot(const uint8_t* row, size_t nsb, const int8_t* xq, const float* xs) {
  float acc = 0.0f;
  int8_t q[16];
  for (size_t bi = 0; bi < nsb; bi++) {
    const uint8_t* block = row + bi * 110;
    const uint8_t *hmask = block, *qs = block + 32;
    float d_all = or_f16_to_f32(rd16(block + 108));
    int8_t scales[16];
    or_unpack_q3_k_scales(block + 96, scales);
    size_t base = bi * 16;
    int is = 0;
    uint8_t m = 1;
    for (int half = 0; half < 2; half++) {
      const uint8_t* qhp = qs + half * 32;
      int shift = 0;
      for (int j = 0; j < 4; j++) {
        for (int offset = 0; offset < 32; offset += 16) {
          float dl = d_all * (float)((int)scales[is] - 32);
          for (int l = 0; l < 16; l++) {
            int hbit = (hmask[l + offset] & m) ? 0 : 4;
            q[l] = (int8_t)(((qhp[l + offset] >> shift) & 3) - hbit);
          }
          size_t sb = base + is, off = sb * 16;
          float dot = (float)dot_i8(q, xq + off, 16);
          acc += xs[off / QK] * dl * dot;
          is += 1;
        }
        shift += 2;
        m = (uint8_t)(m << 1);
      }
    }
  }
  return acc;
}

/* quant/mod.rs:548-581 */
static float q2_k_dot(const uint8_t* row, size_t nsb, const int8_t* xq, const float* xs,
                      const int32_t* sums16) {
  float acc = 0.0f;
  int8_t q[16];
  for (size_t bi = 0; bi < nsb; bi++) {
    const uint8_t* block = row + bi * 84;
    const uint8_t *scales = block, *qs = block + 16;
    float d = or_f16_to_f32(rd16(block + 80)), dmin = or_f16_to_f32(rd16(block + 82));
    size_t base = bi * 16;
    int is = 0;
    for (int half = 0; half < 2; half++) {
      const uint8_t* qb = qs + half * 32;
      int shift = 0;
      for (int j = 0; j < 4; j++) {
        for (int offset = 0; offset < 32; offset += 16) {
          uint8_t sc = scales[is];
          float dl = d * (float)(sc & 0x0F), ml = dmin * (float)(sc >> 4);
          for (int l = 0; l < 16; l++) q[l] = (int8_t)((qb[l + offset] >> shift) & 3);
          size_t sb = base + is, off = sb * 16;
          float dot = (float)dot_i8(q, xq + off, 16);
          acc += xs[off / QK] * (dl * dot - ml * (float)sums16[sb]);
          is += 1;
        }
        shift += 2;
      }
    }
  }
  return acc;
}

/* quant/mod.rs:586-621 */
static float q4_k_dot(const uint8_t* row, size_t nsb, const int8_t* xq, const float* xs,
                      const int32_t* sums) {
  float acc = 0.0f;
  int8_t qlo[QK], qhi[QK];
  for (size_t bi = 0; bi < nsb; bi++) {
    const uint8_t* block = row + bi * 144;
    float d = or_f16_to_f32(rd16(block)), dmin = or_f16_to_f32(rd16(block + 2));
    const uint8_t *scales = block + 4, *qs = block + 16;
    size_t base = bi * 8;
    int is = 0;
    for (int c = 0; c < 4; c++) {
      const uint8_t* chunk = qs + c * 32;
      for (int i = 0; i < 32; i++) {
        qlo[i] = (int8_t)(chunk[i] & 0x0F);
        qhi[i] = (int8_t)(chunk[i] >> 4);
      }
      uint8_t sc1, m1, sc2, m2;
      or_get_scale_min_k4(is, scales, &sc1, &m1);
      or_get_scale_min_k4(is + 1, scales, &sc2, &m2);
      size_t sb = base + is, off = sb * QK;
      float dot = (float)dot_i8(qlo, xq + off, QK);
      acc += xs[sb] * (d * (float)sc1 * dot - dmin * (float)m1 * (float)sums[sb]);
      sb = sb + 1;
      off = sb * QK;
      dot = (float)dot_i8(qhi, xq + off, QK);
      acc += xs[sb] * (d * (float)sc2 * dot - dmin * (float)m2 * (float)sums[sb]);
      is += 2;
    }
  }
  return acc;
}

/* quant/mod.rs:384-394. `row` holds cols/elems whole blocks. */
static float int8_dot_n(uint32_t t, const uint8_t* row, size_t cols, const int8_t* xq,
                        const float* xs, const int32_t* sums) {
  switch (t) {
    case OR_Q8_0: return q8_0_dot(row, cols / QK, xq, xs);
    case OR_Q2_K: return q2_k_dot(row, cols / QK_K, xq, xs, sums);
    case OR_Q3_K: return q3_k_dot(row, cols / QK_K, xq, xs);
    case OR_Q4_K: return q4_k_dot(row, cols / QK_K, xq, xs, sums);
    case OR_Q5_K: return q5_k_dot(row, cols / QK_K, xq, xs, sums);
    case OR_Q6_K: return q6_k_dot(row, cols / QK_K, xq, xs);
  }
  return NAN;
}

/* Single-block entry used by tests: the row is exactly one super-block (or Q8_0 block). */
float or_int8_dot(uint32_t t, const uint8_t* row, const int8_t* xq, const float* xs,
                  const int32_t* sums) {
  size_t e;
  if (or_block_layout(t, &e, NULL) || !or_has_int8_kernel(t)) return NAN;
  return int8_dot_n(t, row, e, xq, xs, sums);
}

/* simd/mod.rs:13-16. Iterator::sum over f32 folds left to right; since Rust 1.82 it
 * starts from -0.0, which only decides the sign of an all-zero sum. */
float or_dot(const float* a, const float* b, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; i++) s += a[i] * b[i];
  return s;
}

/* ---- row-parallel driver (rayon's par_iter over rows; results are per row) ---- */

typedef void (*row_fn)(void* ctx, size_t r0, size_t r1);
typedef struct { row_fn fn; void* ctx; size_t r0, r1; } row_job;

static void* row_worker(void* p) {
  row_job* j = (row_job*)p;
  j->fn(j->ctx, j->r0, j->r1);
  return NULL;
}

static void par_rows(size_t rows, int threads, row_fn fn, void* ctx) {
  if (threads <= 1 || rows < 2) {
    fn(ctx, 0, rows);
    return;
  }
  if ((size_t)threads > rows) threads = (int)rows;
  pthread_t tid[256];
  row_job jobs[256];
  if (threads > 256) threads = 256;
  size_t per = (rows + threads - 1) / threads;
  int started = 0;
  for (int t = 0; t < threads; t++) {
    size_t r0 = t * per, r1 = r0 + per > rows ? rows : r0 + per;
    if (r0 >= r1) break;
    jobs[t] = (row_job){fn, ctx, r0, r1};
    if (pthread_create(&tid[t], NULL, row_worker, &jobs[t]) != 0) {
      fn(ctx, r0, r1);
      jobs[t].fn = NULL;
    }
    started = t + 1;
  }
  for (int t = 0; t < started; t++)
    if (jobs[t].fn) pthread_join(tid[t], NULL);
}

typedef struct {
  uint32_t t;
  const uint8_t* w;
  size_t row_bytes, cols, n;
  const int8_t* xq;
  const float* xs;
  const int32_t* sums;
  size_t sum_stride;
  const float* x;  /* f32 path */
  float* by_row;   /* [rows * n] */
} mm_ctx;

static void mm_int8_rows(void* p, size_t r0, size_t r1) {
  mm_ctx* c = (mm_ctx*)p;
  size_t sblocks = c->cols / QK;
  for (size_t r = r0; r < r1; r++)
    for (size_t b = 0; b < c->n; b++)
      c->by_row[r * c->n + b] =
          int8_dot_n(c->t, c->w + r * c->row_bytes, c->cols, c->xq + b * c->cols,
                     c->xs + b * sblocks, c->sums ? c->sums + b * c->sum_stride : NULL);
}

static void mm_f32_rows(void* p, size_t r0, size_t r1) {
  mm_ctx* c = (mm_ctx*)p;
  float* buf = (float*)malloc(c->cols * sizeof(float));
  for (size_t r = r0; r < r1; r++) {
    or_dequant_into(c->t, c->w + r * c->row_bytes, c->row_bytes, buf, c->cols);
    for (size_t b = 0; b < c->n; b++) c->by_row[r * c->n + b] = or_dot(buf, c->x + b * c->cols, c->cols);
  }
  free(buf);
}

/* quant/mod.rs:223-304 (and :158-206, which it equals for n == 1). */
int or_matmul(uint32_t t, const uint8_t* w, size_t w_len, size_t rows, size_t cols,
              const float* xs, size_t n, float* out, int threads) {
  size_t row_bytes;
  if (or_byte_size(t, cols, &row_bytes)) return 1;
  if (w_len != rows * row_bytes) return 1;
  if (n == 0) return 2;
  float* by_row = (float*)malloc(rows * n * sizeof(float));
  mm_ctx c = {t, w, row_bytes, cols, n, NULL, NULL, NULL, 0, xs, by_row};
  int8_t* xq = NULL;
  float* xsc = NULL;
  int32_t* sums = NULL;
  if (or_has_int8_kernel(t)) {
    xq = (int8_t*)malloc(n * cols);
    xsc = (float*)malloc(n * (cols / QK) * sizeof(float));
    for (size_t b = 0; b < n; b++) or_quantize_activation(xs + b * cols, cols, xq + b * cols, xsc + b * (cols / QK));
    int width = or_sum_width(t);
    if (width) {
      c.sum_stride = cols / width;
      sums = (int32_t*)malloc(n * c.sum_stride * sizeof(int32_t));
      or_block_sums(xq, n * cols, width, sums);
    }
    c.xq = xq;
    c.xs = xsc;
    c.sums = sums;
    par_rows(rows, threads, mm_int8_rows, &c);
  } else {
    par_rows(rows, threads, mm_f32_rows, &c);
  }
  for (size_t r = 0; r < rows; r++)
    for (size_t b = 0; b < n; b++) out[b * rows + r] = by_row[r * n + b];
  free(by_row);
  free(xq);
  free(xsc);
  free(sums);
  return 0;
}

int or_matvec(uint32_t t, const uint8_t* w, size_t w_len, size_t rows, size_t cols,
              const float* x, float* out, int threads) {
  return or_matmul(t, w, w_len, rows, cols, x, 1, out, threads);
}

typedef struct { const float* m; size_t cols, n; const float* xs; float* out; size_t rows; } sm_ctx;
static void sm_rows(void* p, size_t r0, size_t r1) {
  sm_ctx* c = (sm_ctx*)p;
  for (size_t r = r0; r < r1; r++)
    for (size_t b = 0; b < c->n; b++)
      c->out[b * c->rows + r] = or_dot(c->m + r * c->cols, c->xs + b * c->cols, c->cols);
}

/* simd/mod.rs:72-86 */
void or_simd_matvec(const float* m, size_t rows, size_t cols, const float* x, float* out, int threads) {
  or_simd_matmul(m, rows, cols, x, 1, out, threads);
}

/* simd/mod.rs:96-129: out[b*rows + r] = dot(m[r], xs[b]). */
void or_simd_matmul(const float* m, size_t rows, size_t cols, const float* xs, size_t n, float* out,
                    int threads) {
  sm_ctx c = {m, cols, n, xs, out, rows};
  par_rows(rows, threads, sm_rows, &c);
}

/* simd/mod.rs:132-158 */
void or_softmax(float* x, size_t n) {
  float max = -INFINITY;
  for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
  if (!isfinite(max)) {
    if (n) {
      float u = 1.0f / (float)n;
      for (size_t i = 0; i < n; i++) x[i] = u;
    }
    return;
  }
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - max);
    sum += x[i];
  }
  if (isfinite(sum) && sum > 0.0f) {
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
    return;
  }
  float u = 1.0f / (float)n;
  for (size_t i = 0; i < n; i++) x[i] = u;
}

void or_expf(const float* x, size_t n, float* y) {
  for (size_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* simd/mod.rs:161-163 */
void or_silu(float* x, size_t n) {
  for (size_t i = 0; i < n; i++) x[i] /= 1.0f + expf(-x[i]);
}

/* simd/mod.rs:182-185 */
void or_add_scaled(float* a, const float* b, size_t n, float k) {
  for (size_t i = 0; i < n; i++) a[i] += b[i] * k;
}

/* simd/mod.rs:188-191 */
void or_mul_assign(float* a, const float* b, size_t n) {
  for (size_t i = 0; i < n; i++) a[i] *= b[i];
}

/* f32::total_cmp key (Rust core): flip the magnitude bits of negatives. */
static inline int32_t total_key(float f) {
  int32_t i;
  memcpy(&i, &f, 4);
  i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
  return i;
}

/* Stable sort descending. llama: by total_cmp (llama/mod.rs:943, slice::sort_by is
 * stable so equal keys keep ascending id). Router: partial_cmp, equal values by id
 * ascending (router/mod.rs:83-88). The reference's comparator maps an unordered pair to
 * Equal, which is no order once a logit is NaN (Rust's sort_by then gives an unspecified
 * order, or panics): this restatement, like the device code, ranks a NaN after every
 * number and NaNs among themselves by id. That case is parity unpinned: nothing in the
 * reference fixes it. Insertion sort is stable and ne is small. */
static int before_llama(float a_s, float b_s) { return total_key(a_s) > total_key(b_s); }
static int before_router(uint32_t a_id, float a_s, uint32_t b_id, float b_s) {
  const int na = a_s != a_s, nb = b_s != b_s;
  if (na || nb) return na == nb ? a_id < b_id : nb;
  if (a_s > b_s) return 1;
  if (a_s < b_s) return 0;
  return a_id < b_id;  /* equal: id ascending */
}

void or_gate(int kind, float* scores, int ne, int k, uint32_t* ids, float* w) {
  uint32_t* rid = (uint32_t*)malloc(ne * sizeof(uint32_t));
  float* rs = (float*)malloc(ne * sizeof(float));
  if (kind == 0 || kind == 2 || kind == 3) or_softmax(scores, ne);
  for (int i = 0; i < ne; i++) {
    rid[i] = (uint32_t)i;
    rs[i] = scores[i];
  }
  for (int i = 1; i < ne; i++) {
    uint32_t id = rid[i];
    float s = rs[i];
    int j = i - 1;
    while (j >= 0 && (kind == 0 ? before_llama(s, rs[j]) : before_router(id, s, rid[j], rs[j]))) {
      rid[j + 1] = rid[j];
      rs[j + 1] = rs[j];
      j--;
    }
    rid[j + 1] = id;
    rs[j + 1] = s;
  }
  if (k > ne) k = ne;
  if (kind == 0) {
    /* llama/mod.rs:945-949 */
    float sum = -0.0f;
    for (int i = 0; i < k; i++) sum += rs[i];
    float norm = sum > 0.0f ? 1.0f / sum : 1.0f / (float)k;
    for (int i = 0; i < k; i++) rs[i] *= norm;
  } else if (kind == 1) {
    /* router/mod.rs:91-97: softmax over the k kept logits */
    or_softmax(rs, (size_t)k);
  } else if (kind == 3) {
    /* router/mod.rs:102-115 */
    float sum = -0.0f;
    for (int i = 0; i < k; i++) sum += rs[i];
    if (sum > 0.0f) {
      for (int i = 0; i < k; i++) rs[i] /= sum;
    } else {
      float u = 1.0f / (float)k;
      for (int i = 0; i < k; i++) rs[i] = u;
    }
  }
  for (int i = 0; i < k; i++) {
    ids[i] = rid[i];
    w[i] = rs[i];
  }
  free(rid);
  free(rs);
}

/* Weight::matmul_rows over one expert's rows of a stacked tensor (llama/mod.rs:148-195,
 * :233-245): packed -> quant::matmul, full -> simd::matmul on the dequantised copy. */
static int expert_matmul(const or_moe_layer* L, uint32_t qt, const uint8_t* w, const float* wf,
                         size_t e, size_t rows, size_t cols, const float* xs, size_t n, float* out,
                         int threads) {
  size_t row_bytes;
  if (or_byte_size(qt, cols, &row_bytes)) return 1;
  const uint8_t* ew = w + e * rows * row_bytes;
  if (L->packed) return or_matmul(qt, ew, rows * row_bytes, rows, cols, xs, n, out, threads);
  if (wf) {
    or_simd_matmul(wf + e * rows * cols, rows, cols, xs, n, out, threads);
    return 0;
  }
  float* deq = (float*)malloc(rows * cols * sizeof(float));
  int rc = or_dequant_into(qt, ew, rows * row_bytes, deq, rows * cols);
  if (!rc) or_simd_matmul(deq, rows, cols, xs, n, out, threads);
  free(deq);
  return rc;
}

/* llama/mod.rs:1002-1020 */
static int expert_batch(const or_moe_layer* L, size_t e, const float* hs, size_t n, float* out,
                        int threads) {
  size_t d = (size_t)L->d, f = (size_t)L->f;
  float* g = (float*)malloc(n * f * sizeof(float));
  float* u = (float*)malloc(n * f * sizeof(float));
  int rc = expert_matmul(L, L->qt_gate, L->gate, L->gate_f32, e, f, d, hs, n, g, threads);
  if (!rc) rc = expert_matmul(L, L->qt_up, L->up, L->up_f32, e, f, d, hs, n, u, threads);
  if (!rc) {
    or_silu(g, n * f);
    or_mul_assign(g, u, n * f);
    rc = expert_matmul(L, L->qt_down, L->down, L->down_f32, e, d, f, g, n, out, threads);
  }
  free(g);
  free(u);
  return rc;
}

/* llama/mod.rs:903-998 (Ffn::Moe arm). With combine == 1 the experts of each token are
 * applied in routed rank order instead, as MoeEngine::moe_ffn does (moe/mod.rs:98-112);
 * each expert still sees exactly the token's hidden state, so only the add order moves. */
int or_feed_forward_batch(const or_moe_layer* L, const float* hs, int n, float* out,
                          uint32_t* ids_out, float* w_out, const float* logits, int threads) {
  int d = L->d, ne = L->ne, k = L->k < 1 ? 1 : L->k;
  if (n <= 0 || k > ne) return 2;
  uint32_t* ids = (uint32_t*)malloc((size_t)n * k * sizeof(uint32_t));
  float* w = (float*)malloc((size_t)n * k * sizeof(float));
  float* scores = (float*)malloc((size_t)ne * sizeof(float));
  for (int t = 0; t < n; t++) {
    if (logits) memcpy(scores, logits + (size_t)t * ne, ne * sizeof(float));
    else or_simd_matvec(L->router, ne, d, hs + (size_t)t * d, scores, 1);
    or_gate(L->gating, scores, ne, k, ids + (size_t)t * k, w + (size_t)t * k);
  }
  free(scores);
  if (ids_out) memcpy(ids_out, ids, (size_t)n * k * sizeof(uint32_t));
  if (w_out) memcpy(w_out, w, (size_t)n * k * sizeof(float));

  /* llama/mod.rs:967-972: members[e] lists (t, w) in ascending t. */
  int* cnt = (int*)calloc(ne, sizeof(int));
  for (int t = 0; t < n; t++)
    for (int i = 0; i < k; i++) cnt[ids[(size_t)t * k + i]]++;

  memset(out, 0, (size_t)n * d * sizeof(float));
  float* yall = NULL;  /* rank-order combine needs every expert's rows first */
  int* slot = NULL;
  if (L->combine == 1) {
    yall = (float*)malloc((size_t)n * k * d * sizeof(float));
    slot = (int*)malloc((size_t)n * k * sizeof(int));
  }
  int rc = 0;
  float* gathered = (float*)malloc((size_t)n * d * sizeof(float));
  float* eout = (float*)malloc((size_t)n * d * sizeof(float));
  int* tok = (int*)malloc((size_t)n * sizeof(int));
  float* tw = (float*)malloc((size_t)n * sizeof(float));
  int* tr = (int*)malloc((size_t)n * sizeof(int));
  for (int e = 0; e < ne && !rc; e++) {
    if (!cnt[e]) continue;
    int m = 0;
    for (int t = 0; t < n; t++)
      for (int i = 0; i < k; i++)
        if (ids[(size_t)t * k + i] == (uint32_t)e) {
          tok[m] = t;
          tw[m] = w[(size_t)t * k + i];
          tr[m] = i;
          m++;
        }
    for (int i = 0; i < m; i++) memcpy(gathered + (size_t)i * d, hs + (size_t)tok[i] * d, d * sizeof(float));
    rc = expert_batch(L, (size_t)e, gathered, (size_t)m, eout, threads);
    if (rc) break;
    for (int i = 0; i < m; i++) {
      if (L->combine == 1) {
        memcpy(yall + ((size_t)tok[i] * k + tr[i]) * d, eout + (size_t)i * d, d * sizeof(float));
      } else {
        or_add_scaled(out + (size_t)tok[i] * d, eout + (size_t)i * d, (size_t)d, tw[i]);
      }
    }
  }
  if (!rc && L->combine == 1)
    for (int t = 0; t < n; t++)
      for (int i = 0; i < k; i++)
        or_add_scaled(out + (size_t)t * d, yall + ((size_t)t * k + i) * d, (size_t)d, w[(size_t)t * k + i]);
  free(gathered);
  free(eout);
  free(tok);
  free(tw);
  free(tr);
  free(cnt);
  free(ids);
  free(w);
  free(yall);
  free(slot);
  return rc;
}

/* weights/mod.rs:17-23 */
uint64_t or_splitmix64(uint64_t* state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* weights/mod.rs:26-35 */
void or_seeded(uint64_t seed, size_t n, float bound, float* out) {
  uint64_t state = seed;
  for (size_t i = 0; i < n; i++) {
    float u = (float)(or_splitmix64(&state) >> 40) / (float)(1u << 24);
    out[i] = (u * 2.0f - 1.0f) * bound;
  }
}

/* weights/mod.rs:38-40 */
float or_bound(size_t fan_in) { return 1.0f / sqrtf((float)fan_in); }

/* weights/mod.rs:98-109 */
void or_synthesize_expert(uint32_t id, int d, int f, float* gate, float* up, float* down) {
  const uint64_t EXPERT = 0x6761727564611000ull;
  uint64_t seed = EXPERT ^ ((uint64_t)id * 0x9E3779B97F4A7C15ull);
  or_seeded(seed, (size_t)f * d, or_bound((size_t)d), gate);
  or_seeded(seed ^ 0xAAAAAAAAull, (size_t)f * d, or_bound((size_t)d), up);
  or_seeded(seed ^ 0x55555555ull, (size_t)d * f, or_bound((size_t)f), down);
}
