// gmoe_quant.cpp — build-side data preparation: f32 -> GGUF block quantisers and a
// seeded Gaussian generator. The reference only decodes GGUF blocks (it ships no
// quantiser), so these are this project's own: plain min/max round-to-nearest
// quantisers whose output is any valid block of the format. Their only contract is
// that the reference decoders (garuda/src/quant/mod.rs:624-875) read them back with
// error within one quantisation step, which the tests check.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/garuda_moe.h"
#include "gmoe_internal.h"

using namespace gmoe;

namespace {

inline uint16_t to_f16(float v) {
  _Float16 h = (_Float16)v;  // round to nearest even
  uint16_t u;
  memcpy(&u, &h, 2);
  return u;
}
inline float from_f16(uint16_t u) {
  _Float16 h;
  memcpy(&h, &u, 2);
  return (float)h;
}
inline void put16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}
inline int nearest(float v) { return (int)lrintf(v); }
inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

// block_q8_0: d = amax/127, q = round(x/d)
void q8_0(const float* x, uint8_t* b) {
  float amax = 0;
  for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
  uint16_t dh = to_f16(amax / 127.0f);
  float d = from_f16(dh);
  put16(b, dh);
  for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)(d > 0 ? clampi(nearest(x[i] / d), -127, 127) : 0);
}

// block_q4_0: signed value of largest magnitude maps to -8
void q4_0(const float* x, uint8_t* b) {
  float amax = 0, mx = 0;
  for (int i = 0; i < 32; i++)
    if (std::fabs(x[i]) > amax) {
      amax = std::fabs(x[i]);
      mx = x[i];
    }
  uint16_t dh = to_f16(mx / -8.0f);
  float d = from_f16(dh);
  put16(b, dh);
  for (int i = 0; i < 16; i++) {
    int lo = d != 0 ? clampi(nearest(x[i] / d) + 8, 0, 15) : 8;
    int hi = d != 0 ? clampi(nearest(x[i + 16] / d) + 8, 0, 15) : 8;
    b[2 + i] = (uint8_t)(lo | (hi << 4));
  }
}

// Affine sub-blocks for Q4_K/Q5_K (8 of 32) and Q2_K (16 of 16): w = d*sc*q - dmin*m.
struct Affine {
  int sc[16], m[16];
  float d, dmin;
};

void affine_scales(const float* x, int nsub, int width, int qmax, int scmax, Affine& A, float* scale,
                   float* mn) {
  float maxsc = 0, maxm = 0;
  for (int s = 0; s < nsub; s++) {
    float lo = 0, hi = 0;  // the min is never above 0, so q = 0 can represent 0 exactly
    for (int i = 0; i < width; i++) {
      lo = std::min(lo, x[s * width + i]);
      hi = std::max(hi, x[s * width + i]);
    }
    scale[s] = (hi - lo) / qmax;
    mn[s] = -lo;
    maxsc = std::max(maxsc, scale[s]);
    maxm = std::max(maxm, mn[s]);
  }
  uint16_t dh = to_f16(maxsc / scmax), mh = to_f16(maxm / scmax);
  A.d = from_f16(dh);
  A.dmin = from_f16(mh);
  for (int s = 0; s < nsub; s++) {
    A.sc[s] = A.d > 0 ? clampi(nearest(scale[s] / A.d), 0, scmax) : 0;
    A.m[s] = A.dmin > 0 ? clampi(nearest(mn[s] / A.dmin), 0, scmax) : 0;
  }
}

// inverse of get_scale_min_k4 (quant/mod.rs:656-664)
void pack_k4(const int* sc, const int* m, uint8_t* s) {
  for (int i = 0; i < 4; i++) {
    s[i] = (uint8_t)((sc[i] & 63) | ((sc[4 + i] >> 4) << 6));
    s[4 + i] = (uint8_t)((m[i] & 63) | ((m[4 + i] >> 4) << 6));
    s[8 + i] = (uint8_t)((sc[4 + i] & 15) | ((m[4 + i] & 15) << 4));
  }
}

int affine_q(float v, float dl, float ml, int qmax) {
  return dl > 0 ? clampi(nearest((v + ml) / dl), 0, qmax) : 0;
}

void q4_k(const float* x, uint8_t* b) {
  Affine A;
  float scale[8], mn[8];
  affine_scales(x, 8, 32, 15, 63, A, scale, mn);
  put16(b, to_f16(A.d));
  put16(b + 2, to_f16(A.dmin));
  pack_k4(A.sc, A.m, b + 4);
  uint8_t* qs = b + 16;
  for (int c = 0; c < 4; c++) {
    int s1 = 2 * c, s2 = 2 * c + 1;
    float d1 = A.d * A.sc[s1], m1 = A.dmin * A.m[s1], d2 = A.d * A.sc[s2], m2 = A.dmin * A.m[s2];
    for (int l = 0; l < 32; l++) {
      int lo = affine_q(x[32 * s1 + l], d1, m1, 15), hi = affine_q(x[32 * s2 + l], d2, m2, 15);
      qs[32 * c + l] = (uint8_t)(lo | (hi << 4));
    }
  }
}

void q5_k(const float* x, uint8_t* b) {
  Affine A;
  float scale[8], mn[8];
  affine_scales(x, 8, 32, 31, 63, A, scale, mn);
  put16(b, to_f16(A.d));
  put16(b + 2, to_f16(A.dmin));
  pack_k4(A.sc, A.m, b + 4);
  uint8_t* qh = b + 16;
  uint8_t* qs = b + 48;
  memset(qh, 0, 32);
  for (int g = 0; g < 4; g++) {
    int s1 = 2 * g, s2 = 2 * g + 1;
    float d1 = A.d * A.sc[s1], m1 = A.dmin * A.m[s1], d2 = A.d * A.sc[s2], m2 = A.dmin * A.m[s2];
    for (int l = 0; l < 32; l++) {
      int q1 = affine_q(x[32 * s1 + l], d1, m1, 31), q2 = affine_q(x[32 * s2 + l], d2, m2, 31);
      qs[32 * g + l] = (uint8_t)((q1 & 15) | ((q2 & 15) << 4));
      if (q1 & 16) qh[l] |= (uint8_t)(1u << (2 * g));
      if (q2 & 16) qh[l] |= (uint8_t)(2u << (2 * g));
    }
  }
}

void q2_k(const float* x, uint8_t* b) {
  Affine A;
  float scale[16], mn[16];
  affine_scales(x, 16, 16, 3, 15, A, scale, mn);
  for (int s = 0; s < 16; s++) b[s] = (uint8_t)((A.sc[s] & 15) | ((A.m[s] & 15) << 4));
  uint8_t* qs = b + 16;
  memset(qs, 0, 64);
  // element order (dequant_q2_k): half h, shift 2j, offset o in {0,16}: sub-block 8h+2j+o/16
  for (int h = 0; h < 2; h++)
    for (int j = 0; j < 4; j++)
      for (int o = 0; o < 32; o += 16) {
        int s = 8 * h + 2 * j + o / 16;
        float dl = A.d * A.sc[s], ml = A.dmin * A.m[s];
        for (int l = 0; l < 16; l++) {
          int q = affine_q(x[16 * s + l], dl, ml, 3);
          qs[32 * h + o + l] |= (uint8_t)(q << (2 * j));
        }
      }
  put16(b + 80, to_f16(A.d));
  put16(b + 82, to_f16(A.dmin));
}

// Symmetric 16-wide sub-blocks with signed sub-scales (Q3_K: 6-bit offset 32, Q6_K: int8).
void sym_scales(const float* x, int qneg, int scmax, float& d, int* sc) {
  float smax = 0, s[16];
  for (int i = 0; i < 16; i++) {
    float amax = 0;
    for (int l = 0; l < 16; l++) amax = std::max(amax, std::fabs(x[16 * i + l]));
    s[i] = amax / qneg;
    smax = std::max(smax, s[i]);
  }
  d = from_f16(to_f16(smax / scmax));
  for (int i = 0; i < 16; i++) sc[i] = d > 0 ? clampi(nearest(s[i] / d), -scmax, scmax) : 0;
}

void q6_k(const float* x, uint8_t* b) {
  float d;
  int sc[16];
  sym_scales(x, 32, 127, d, sc);
  uint8_t* ql = b;
  uint8_t* qh = b + 128;
  memset(b, 0, 192);
  for (int i = 0; i < 16; i++) b[192 + i] = (uint8_t)(int8_t)sc[i];
  put16(b + 208, to_f16(d));
  for (int e = 0; e < 256; e++) {
    int s = e / 16;
    float dl = d * sc[s];
    int q = dl != 0 ? clampi(nearest(x[e] / dl), -32, 31) + 32 : 32;
    int half = e / 128, r = e % 128, quarter = r / 32, l = r % 32;
    uint8_t* qlh = ql + 64 * half;
    uint8_t* qhh = qh + 32 * half;
    if (quarter == 0) qlh[l] |= (uint8_t)(q & 15);
    if (quarter == 1) qlh[l + 32] |= (uint8_t)(q & 15);
    if (quarter == 2) qlh[l] |= (uint8_t)((q & 15) << 4);
    if (quarter == 3) qlh[l + 32] |= (uint8_t)((q & 15) << 4);
    qhh[l] |= (uint8_t)(((q >> 4) & 3) << (2 * quarter));
  }
}

void q3_k(const float* x, uint8_t* b) {
  float d;
  int sc[16];
  sym_scales(x, 4, 31, d, sc);
  uint8_t* hmask = b;
  uint8_t* qs = b + 32;
  memset(b, 0, 108);
  // pack 16 six-bit values (sc + 32), the inverse of unpack_q3_k_scales (quant/mod.rs:812-833)
  int u[16];
  for (int i = 0; i < 16; i++) u[i] = sc[i] + 32;
  for (int j = 0; j < 4; j++) {
    b[96 + j] = (uint8_t)((u[j] & 15) | ((u[8 + j] & 15) << 4));
    b[96 + 4 + j] = (uint8_t)((u[4 + j] & 15) | ((u[12 + j] & 15) << 4));
    b[96 + 8 + j] = (uint8_t)((u[j] >> 4) | ((u[4 + j] >> 4) << 2) | ((u[8 + j] >> 4) << 4) | ((u[12 + j] >> 4) << 6));
  }
  put16(b + 108, to_f16(d));
  // element order (dequant_q3_k): half h, j (shift 2j, mask bit 4h+j), offset o
  for (int h = 0; h < 2; h++)
    for (int j = 0; j < 4; j++)
      for (int o = 0; o < 32; o += 16) {
        int s = 8 * h + 2 * j + o / 16;
        float dl = d * sc[s];
        for (int l = 0; l < 16; l++) {
          int q = dl != 0 ? clampi(nearest(x[16 * s + l] / dl), -4, 3) : 0;
          int low, hb;
          if (q >= 0) { low = q; hb = 1; } else { low = q + 4; hb = 0; }
          qs[32 * h + o + l] |= (uint8_t)(low << (2 * j));
          if (hb) hmask[o + l] |= (uint8_t)(1u << (4 * h + j));
        }
      }
}

void quant_range(uint32_t qt, const float* x, uint64_t b0, uint64_t b1, uint8_t* out) {
  uint32_t E, B;
  block_layout(qt, &E, &B);
  for (uint64_t i = b0; i < b1; i++) {
    const float* xb = x + i * E;
    uint8_t* ob = out + i * B;
    switch (qt) {
      case F32: memcpy(ob, xb, 4); break;
      case F16: put16(ob, to_f16(*xb)); break;
      case Q8_0: q8_0(xb, ob); break;
      case Q4_0: q4_0(xb, ob); break;
      case Q4_K: q4_k(xb, ob); break;
      case Q5_K: q5_k(xb, ob); break;
      case Q6_K: q6_k(xb, ob); break;
      case Q3_K: q3_k(xb, ob); break;
      case Q2_K: q2_k(xb, ob); break;
    }
  }
}

template <class F>
void parallel(uint64_t n, int threads, F f) {
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  threads = (int)std::min<uint64_t>((uint64_t)threads, std::max<uint64_t>(1, n / 4096));
  if (threads <= 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> ts;
  uint64_t per = (n + threads - 1) / threads;
  for (int t = 0; t < threads; t++) {
    uint64_t a = t * per, b = std::min(n, a + per);
    if (a >= b) break;
    ts.emplace_back(f, a, b);
  }
  for (auto& t : ts) t.join();
}

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

extern "C" {

gmoe_status gmoe_quantize(uint32_t qt, const float* x, uint64_t n, void* out, int threads) {
  uint32_t E, B;
  if (!block_layout(qt, &E, &B)) return GMOE_ERR_MODEL;
  if (n % E) return GMOE_ERR_MODEL;
  if (!x || !out) return GMOE_ERR_INFERENCE;
  uint64_t nb = n / E;
  parallel(nb, threads, [&](uint64_t a, uint64_t b) { quant_range(qt, x, a, b, (uint8_t*)out); });
  return GMOE_OK;
}

// Value i is Box-Muller over outputs 2i and 2i+1 of the splitmix64 stream that starts at
// state `seed` (garuda/src/weights/mod.rs:17-23), computed by index so it parallelises.
gmoe_status gmoe_fill_gaussian(uint64_t seed, float mean, float stdv, uint64_t n, float* out, int threads) {
  if (!out) return GMOE_ERR_INFERENCE;
  parallel(n, threads, [&](uint64_t a, uint64_t b) {
    for (uint64_t i = a; i < b; i++) {
      uint64_t z1 = mix64(seed + (2 * i + 1) * 0x9E3779B97F4A7C15ull);
      uint64_t z2 = mix64(seed + (2 * i + 2) * 0x9E3779B97F4A7C15ull);
      double u1 = ((z1 >> 11) + 1) * 0x1.0p-53;  // (0, 1]
      double u2 = (z2 >> 11) * 0x1.0p-53;        // [0, 1)
      double g = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
      out[i] = (float)(mean + stdv * g);
    }
  });
  return GMOE_OK;
}

}  // extern "C"
