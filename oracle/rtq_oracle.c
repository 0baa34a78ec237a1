/*
 * rtq_oracle.c — CPU restatement of Rust_Trainer's frozen quantised-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker / the timed CPU baseline; never by the product library.
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off).
 * -ffp-contract=off because Rust (the reference and rie-core) never fuses a*b+c, so the
 * K-quant dequant `d1*q - m1` must round twice, as it does there.
 *
 * Parity pinning (what checks each function; see tests/test_oracle.py):
 *   Rng                     golden values recomputed from the SplitMix64 / Box-Muller definition
 *                           in numpy (float64 SplitMix is exact integer arithmetic).
 *   fp16                    numpy float16 conversion (RNE) over all 2^16 halves and random floats.
 *   quantise/dequant        hand-built known-answer blocks for every format (both 6-bit scale
 *                           packing halves of Q4_K, all four qh shifts of Q6_K) and round-trip bounds.
 *   activation quantisation closed-form tie cases and a numpy restatement.
 *   block isums             brute-force integer sums from the dequantised integer codes.
 *   forward                 f64 sum of the same f32-exact block terms (or_frozen_forward_f64).
 *   backward_input          dense dy . dequant(W) (tests/engine.rs:96-120) and the adjoint
 *                           identity <dy, x W^T> = <dy W, x> (src/frozen.rs:218-227).
 *   Linear                  f64 closed forms of src/linear.rs:84-118 and finite differences.
 * Parity against rie-core itself is unpinned: rie-core is not in this container.
 */
#define _GNU_SOURCE
#include "rtq_oracle.h"

#include <math.h>
#include <omp.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define QKK 256

/* ------------------------------------------------------------------ Rng */
/* src/tensor.rs:163-186 */
uint64_t or_rng_seed(uint64_t seed) { return seed ^ 0x9E3779B97F4A7C15ULL; }

uint64_t or_rng_next_u64(uint64_t* s) {
  *s += 0x9E3779B97F4A7C15ULL;
  uint64_t z = *s;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

float or_rng_uniform(uint64_t* s) { return (float)(or_rng_next_u64(s) >> 40) / (float)(1u << 24); }

float or_rng_normal(uint64_t* s) {
  float u1 = or_rng_uniform(s);
  if (u1 < 1e-12f) u1 = 1e-12f;
  float u2 = or_rng_uniform(s);
  const float pi = 3.14159265358979323846f; /* std::f32::consts::PI */
  return sqrtf(-2.0f * logf(u1)) * cosf(2.0f * pi * u2);
}

void or_rng_fill_normal(uint64_t* s, float* out, int64_t n, float std) {
  for (int64_t i = 0; i < n; i++) out[i] = or_rng_normal(s) * std;
}

void or_rng_fill_uniform_sym(uint64_t* s, float* out, int64_t n, float bound) {
  for (int64_t i = 0; i < n; i++) out[i] = (or_rng_uniform(s) * 2.0f - 1.0f) * bound;
}

/* ------------------------------------------------------------------ half */
uint16_t or_fp32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN, keep payload */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);                         /* >= 65520 -> inf */
  if (ax < 0x38800000u) {                                                            /* below 2^-14 */
    float af;
    memcpy(&af, &ax, 4);
    /* subnormal half: value / 2^-24 rounded to nearest even (exact scaling, then rint) */
    uint32_t m = (uint32_t)nearbyintf(af * 16777216.0f);
    return (uint16_t)(sign | m);
  }
  uint32_t e = (ax >> 23) - 127 + 15;
  uint32_t mant = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float or_fp16_to_fp32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else { /* subnormal: m * 2^-24, exact in f32 */
      float v = (float)m * (1.0f / 16777216.0f);
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e - 15 + 127) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* ------------------------------------------------------------------ blocks */
int64_t or_block_elems(int type) {
  switch (type) {
    case OR_F32:
    case OR_F16: return 1;
    case OR_Q4_0:
    case OR_Q8_0: return QK;
    case OR_Q4_K:
    case OR_Q6_K:
    case OR_Q8_K: return QKK;
  }
  return 0;
}

int64_t or_block_bytes(int type) {
  switch (type) {
    case OR_F32: return 4;
    case OR_F16: return 2;
    case OR_Q4_0: return 18;  /* fp16 d; u8 qs[16] */
    case OR_Q8_0: return 34;  /* fp16 d; i8 qs[32] */
    case OR_Q4_K: return 144; /* fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128] */
    case OR_Q6_K: return 210; /* u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d */
    case OR_Q8_K: return 292; /* f32 d; i8 qs[256]; i16 bsums[16] */
  }
  return 0;
}

int64_t or_row_bytes(int type, int64_t k) {
  int64_t be = or_block_elems(type);
  if (be == 0 || k % be) return -1;
  return k / be * or_block_bytes(type);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}

/* ggml nearest_int: round to nearest, ties to even, for |x| < 2^22 */
static inline int nearest_int(float x) { return (int)nearbyintf(x); }

/* Q4_0 reference quantiser (ggml): the signed element of largest |x| (first wins) maps to -8. */
static void quantize_q4_0_block(const float* x, uint8_t* b) {
  float amax = 0.0f, max = 0.0f;
  for (int j = 0; j < QK; j++) {
    float v = x[j];
    if (amax < fabsf(v)) {
      amax = fabsf(v);
      max = v;
    }
  }
  const float d = max / -8.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  wr16(b, or_fp32_to_fp16(d));
  for (int j = 0; j < QK / 2; j++) {
    const float x0 = x[j] * id;
    const float x1 = x[QK / 2 + j] * id;
    int q0 = (int8_t)(x0 + 8.5f); /* truncating cast, as the C reference does */
    int q1 = (int8_t)(x1 + 8.5f);
    if (q0 > 15) q0 = 15;
    if (q1 > 15) q1 = 15;
    b[2 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

/* Q8_0 reference quantiser (ggml): d = amax/127, q = roundf(x/d) (ties away from zero). */
static void quantize_q8_0_block(const float* x, uint8_t* b) {
  float amax = 0.0f;
  for (int j = 0; j < QK; j++) {
    float a = fabsf(x[j]);
    if (a > amax) amax = a;
  }
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  wr16(b, or_fp32_to_fp16(d));
  for (int j = 0; j < QK; j++) b[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

/*
 * Q4_K encoder.  ggml's own K-quant encoder (make_qkx2_quants' iterative search) is not in
 * this container; this is a documented valid encoder instead: per 32-element sub-block an
 * affine fit x ~ d*sc*q - dmin*m with q in [0,15], 6-bit sc and m, the super-block d / dmin
 * chosen so the largest sub-block scale / min maps to 63.  Parity never depends on the
 * encoder: the CPU oracle and the GPU consume the same bytes.
 */
static void quantize_q4_k_block(const float* x, uint8_t* b) {
  float scale[8], mins[8];
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; j++) {
    float mn = 0.0f, mx = x[32 * j];
    for (int l = 0; l < 32; l++) {
      float v = x[32 * j + l];
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    if (mx < mn) mx = mn;
    scale[j] = (mx - mn) / 15.0f;
    mins[j] = -mn;
    if (scale[j] > max_scale) max_scale = scale[j];
    if (mins[j] > max_min) max_min = mins[j];
  }
  uint16_t dh = or_fp32_to_fp16(max_scale / 63.0f);
  uint16_t mh = or_fp32_to_fp16(max_min / 63.0f);
  float d = or_fp16_to_fp32(dh), dmin = or_fp16_to_fp32(mh);
  int sc[8], m[8];
  for (int j = 0; j < 8; j++) {
    int s = d > 0.0f ? nearest_int(scale[j] / d) : 0;
    int mm = dmin > 0.0f ? nearest_int(mins[j] / dmin) : 0;
    sc[j] = s < 0 ? 0 : (s > 63 ? 63 : s);
    m[j] = mm < 0 ? 0 : (mm > 63 ? 63 : mm);
  }
  wr16(b, dh);
  wr16(b + 2, mh);
  uint8_t* s = b + 4;
  for (int j = 0; j < 4; j++) {
    s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
  }
  uint8_t L[256];
  for (int j = 0; j < 8; j++) {
    const float es = d * (float)sc[j];
    const float em = dmin * (float)m[j];
    for (int l = 0; l < 32; l++) {
      int q = es > 0.0f ? nearest_int((x[32 * j + l] + em) / es) : 0;
      L[32 * j + l] = (uint8_t)(q < 0 ? 0 : (q > 15 ? 15 : q));
    }
  }
  uint8_t* qs = b + 16;
  for (int c = 0; c < 4; c++)
    for (int l = 0; l < 32; l++) qs[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
}

/*
 * Q6_K encoder (documented valid encoder, see the Q4_K note): per 16-element sub-block the
 * signed element of largest |x| maps to -32; the sub-block scales are coded as int8 against a
 * super-block d chosen so the largest-magnitude scale maps to -128 (clamped to 127).
 */
static void quantize_q6_k_block(const float* x, uint8_t* b) {
  float scl[16];
  float max_scale = 0.0f, max_abs = 0.0f;
  for (int s = 0; s < 16; s++) {
    float amax = 0.0f, mx = 0.0f;
    for (int l = 0; l < 16; l++) {
      float v = x[16 * s + l];
      if (fabsf(v) > amax) {
        amax = fabsf(v);
        mx = v;
      }
    }
    scl[s] = mx / -32.0f;
    if (fabsf(scl[s]) > max_abs) {
      max_abs = fabsf(scl[s]);
      max_scale = scl[s];
    }
  }
  int8_t* scales = (int8_t*)(b + 192);
  float d = 0.0f;
  if (max_abs > 0.0f) {
    const float iscale = -128.0f / max_scale;
    uint16_t dh = or_fp32_to_fp16(1.0f / iscale);
    wr16(b + 208, dh);
    d = or_fp16_to_fp32(dh);
    for (int s = 0; s < 16; s++) {
      int v = nearest_int(iscale * scl[s]);
      scales[s] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
    }
  } else {
    wr16(b + 208, 0);
    for (int s = 0; s < 16; s++) scales[s] = 0;
  }
  uint8_t L[256];
  for (int s = 0; s < 16; s++) {
    const float es = d * (float)scales[s];
    for (int l = 0; l < 16; l++) {
      int q = es != 0.0f ? nearest_int(x[16 * s + l] / es) : 0;
      q = q < -32 ? -32 : (q > 31 ? 31 : q);
      L[16 * s + l] = (uint8_t)(q + 32);
    }
  }
  uint8_t* ql = b;
  uint8_t* qh = b + 128;
  for (int h = 0; h < 2; h++) {
    for (int l = 0; l < 32; l++) {
      const uint8_t q1 = L[128 * h + l], q2 = L[128 * h + l + 32];
      const uint8_t q3 = L[128 * h + l + 64], q4 = L[128 * h + l + 96];
      ql[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
      ql[64 * h + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
      qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  }
}

int or_quantize(int type, const float* x, int64_t n, void* out) {
  uint8_t* o = (uint8_t*)out;
  int64_t be = or_block_elems(type), bb = or_block_bytes(type);
  if (be == 0 || n % be) return -1;
  for (int64_t i = 0; i < n / be; i++) {
    const float* xb = x + i * be;
    uint8_t* b = o + i * bb;
    switch (type) {
      case OR_F32: memcpy(b, xb, 4); break;
      case OR_F16: wr16(b, or_fp32_to_fp16(*xb)); break;
      case OR_Q4_0: quantize_q4_0_block(xb, b); break;
      case OR_Q8_0: quantize_q8_0_block(xb, b); break;
      case OR_Q4_K: quantize_q4_k_block(xb, b); break;
      case OR_Q6_K: quantize_q6_k_block(xb, b); break;
      default: return -1;
    }
  }
  return 0;
}

/* 6-bit scale / min of sub-block j (0..7) of a Q4_K super-block */
static inline void q4k_scale_min(int j, const uint8_t* s, int* sc, int* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

/* signed integer code of element e of a Q6_K super-block (value = d * sc[e/16] * code) */
static inline int q6k_code(const uint8_t* b, int e) {
  const int h = e / 128, r = e % 128, m = r / 32, l = r % 32;
  const uint8_t* ql = b + 64 * h;
  const uint8_t* qh = b + 128 + 32 * h;
  int lo = (m & 1) ? ql[l + 32] : ql[l];
  lo = (m < 2) ? (lo & 0xF) : (lo >> 4);
  const int hi = (qh[l] >> (2 * m)) & 3;
  return (lo | (hi << 4)) - 32;
}

/* unsigned 4-bit code of element e of a Q4_K super-block */
static inline int q4k_code(const uint8_t* b, int e) {
  const uint8_t* qs = b + 16;
  const int c = e / 64, r = e % 64;
  return r < 32 ? (qs[32 * c + r] & 0xF) : (qs[32 * c + r - 32] >> 4);
}

int or_dequant_row(int type, const void* row, int64_t k, float* y) {
  const uint8_t* p = (const uint8_t*)row;
  int64_t be = or_block_elems(type), bb = or_block_bytes(type);
  if (be == 0 || k % be) return -1;
  for (int64_t i = 0; i < k / be; i++) {
    const uint8_t* b = p + i * bb;
    float* o = y + i * be;
    switch (type) {
      case OR_F32: memcpy(o, b, 4); break;
      case OR_F16: o[0] = or_fp16_to_fp32(rd16(b)); break;
      case OR_Q4_0: {
        const float d = or_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 16; j++) {
          o[j] = (float)((b[2 + j] & 0xF) - 8) * d;
          o[j + 16] = (float)((b[2 + j] >> 4) - 8) * d;
        }
        break;
      }
      case OR_Q8_0: {
        const float d = or_fp16_to_fp32(rd16(b));
        for (int j = 0; j < 32; j++) o[j] = (float)(int8_t)b[2 + j] * d;
        break;
      }
      case OR_Q4_K: {
        const float d = or_fp16_to_fp32(rd16(b)), dmin = or_fp16_to_fp32(rd16(b + 2));
        for (int j = 0; j < 8; j++) {
          int sc, m;
          q4k_scale_min(j, b + 4, &sc, &m);
          const float d1 = d * (float)sc, m1 = dmin * (float)m;
          for (int l = 0; l < 32; l++) o[32 * j + l] = d1 * (float)q4k_code(b, 32 * j + l) - m1;
        }
        break;
      }
      case OR_Q6_K: {
        const float d = or_fp16_to_fp32(rd16(b + 208));
        const int8_t* sc = (const int8_t*)(b + 192);
        for (int e = 0; e < 256; e++) o[e] = d * (float)sc[e / 16] * (float)q6k_code(b, e);
        break;
      }
      default: return -1;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ activations */
int or_act_type_for(int wtype) {
  switch (wtype) {
    case OR_Q4_0:
    case OR_Q8_0: return OR_Q8_0;
    case OR_Q4_K:
    case OR_Q6_K: return OR_Q8_K;
  }
  return OR_F32;
}

/* ggml quantize_row_q8_0 reference semantics (same as the Q8_0 weight quantiser) */
void or_quantize_acts_q8_0(const float* x, int64_t k, void* out) {
  uint8_t* o = (uint8_t*)out;
  for (int64_t i = 0; i < k / QK; i++) quantize_q8_0_block(x + i * QK, o + i * 34);
}

/* ggml quantize_row_q8_K reference semantics: the signed element of largest |x| maps to -127,
 * q = min(127, nearest_int(-127/max * x)), d = 1/iscale (f32), bsums over 16-element groups. */
void or_quantize_acts_q8_k(const float* x, int64_t k, void* out) {
  uint8_t* o = (uint8_t*)out;
  for (int64_t i = 0; i < k / QKK; i++) {
    const float* xb = x + i * QKK;
    uint8_t* b = o + i * 292;
    int8_t* qs = (int8_t*)(b + 4);
    int16_t bs[16];
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < QKK; j++) {
      float ax = fabsf(xb[j]);
      if (ax > amax) {
        amax = ax;
        max = xb[j];
      }
    }
    float d = 0.0f;
    if (amax == 0.0f) {
      memset(qs, 0, QKK);
    } else {
      const float iscale = -127.0f / max;
      for (int j = 0; j < QKK; j++) {
        int v = nearest_int(iscale * xb[j]);
        qs[j] = (int8_t)(v > 127 ? 127 : v);
      }
      d = 1.0f / iscale;
    }
    for (int g = 0; g < 16; g++) {
      int s = 0;
      for (int l = 0; l < 16; l++) s += qs[16 * g + l];
      bs[g] = (int16_t)s;
    }
    memcpy(b, &d, 4);
    memcpy(b + 260, bs, 32);
  }
}

/* ------------------------------------------------------------------ integer block dots */
int64_t or_isums_per_row(int wtype, int64_t k) {
  switch (wtype) {
    case OR_Q4_0:
    case OR_Q8_0: return k / QK;
    case OR_Q4_K: return 2 * (k / QKK);
    case OR_Q6_K: return k / QKK;
  }
  return 0;
}

int or_block_isums(int wtype, const void* wrow, const void* arow, int64_t k, int32_t* out) {
  const uint8_t* w = (const uint8_t*)wrow;
  const uint8_t* a = (const uint8_t*)arow;
  switch (wtype) {
    case OR_Q4_0:
      for (int64_t i = 0; i < k / QK; i++) {
        const uint8_t* wb = w + 18 * i;
        const int8_t* q8 = (const int8_t*)(a + 34 * i + 2);
        int32_t s = 0;
        for (int j = 0; j < 16; j++) s += ((wb[2 + j] & 0xF) - 8) * q8[j] + ((wb[2 + j] >> 4) - 8) * q8[j + 16];
        out[i] = s;
      }
      return 0;
    case OR_Q8_0:
      for (int64_t i = 0; i < k / QK; i++) {
        const int8_t* qw = (const int8_t*)(w + 34 * i + 2);
        const int8_t* q8 = (const int8_t*)(a + 34 * i + 2);
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += qw[j] * q8[j];
        out[i] = s;
      }
      return 0;
    case OR_Q4_K:
      for (int64_t i = 0; i < k / QKK; i++) {
        const uint8_t* wb = w + 144 * i;
        const int8_t* q8 = (const int8_t*)(a + 292 * i + 4);
        const int16_t* bs = (const int16_t*)(a + 292 * i + 260);
        int32_t s1 = 0, s2 = 0;
        for (int j = 0; j < 8; j++) {
          int sc, m, isum = 0;
          q4k_scale_min(j, wb + 4, &sc, &m);
          for (int l = 0; l < 32; l++) isum += q4k_code(wb, 32 * j + l) * q8[32 * j + l];
          s1 += sc * isum;
          s2 += m * (bs[2 * j] + bs[2 * j + 1]);
        }
        out[2 * i] = s1;
        out[2 * i + 1] = s2;
      }
      return 0;
    case OR_Q6_K:
      for (int64_t i = 0; i < k / QKK; i++) {
        const uint8_t* wb = w + 210 * i;
        const int8_t* sc = (const int8_t*)(wb + 192);
        const int8_t* q8 = (const int8_t*)(a + 292 * i + 4);
        int32_t s = 0;
        for (int g = 0; g < 16; g++) {
          int isum = 0;
          for (int l = 0; l < 16; l++) isum += q6k_code(wb, 16 * g + l) * q8[16 * g + l];
          s += sc[g] * isum;
        }
        out[i] = s;
      }
      return 0;
  }
  return -1;
}

/* ------------------------------------------------------------------ dense primitives */
/* dot_portable, src/tensor.rs:24-43: four interleaved partial sums */
float or_dot(const float* a, const float* b, int64_t n) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0, tail = 0;
  int64_t c = n / 4;
  for (int64_t i = 0; i < c; i++) {
    int64_t j = 4 * i;
    s0 += a[j] * b[j];
    s1 += a[j + 1] * b[j + 1];
    s2 += a[j + 2] * b[j + 2];
    s3 += a[j + 3] * b[j + 3];
  }
  for (int64_t j = 4 * c; j < n; j++) tail += a[j] * b[j];
  return (s0 + s1) + (s2 + s3) + tail;
}

static inline void axpy(float alpha, const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] += alpha * x[i];
}

static int nthr(int n) { return n > 0 ? n : 1; }

/* Timing support (not part of the restated algorithm): pins the threads of an OpenMP team of n -
   the calling thread and the pool threads that every later team of at most n reuses - one each to
   the CPUs of the process's affinity mask, in order, so timed runs do not migrate.  Returns the
   number of CPUs in the mask, or -1 if the mask cannot be read or set. */
int or_pin_threads(int n) {
  cpu_set_t allowed;
  if (sched_getaffinity(0, sizeof allowed, &allowed) != 0) return -1;
  int cpus[CPU_SETSIZE], ncpu = 0;
  for (int c = 0; c < CPU_SETSIZE; c++)
    if (CPU_ISSET(c, &allowed)) cpus[ncpu++] = c;
  if (ncpu == 0) return -1;
  int failed = 0;
#pragma omp parallel num_threads(nthr(n)) reduction(+ : failed)
  {
    cpu_set_t one;
    CPU_ZERO(&one);
    CPU_SET(cpus[omp_get_thread_num() % ncpu], &one);
    failed += sched_setaffinity(0, sizeof one, &one) != 0;
  }
  return failed ? -1 : ncpu;
}

/* out[m x n] = a[m x k] . b^T, b [n x k]  (src/tensor.rs:61-79) */
void or_matmul_nt(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* out, int nthreads) {
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
  for (int64_t i = 0; i < m; i++)
    for (int64_t j = 0; j < n; j++) out[i * n + j] = or_dot(a + i * k, b + j * k, k);
}

/* out[m x n] = a[m x k] . b[k x n]  (src/tensor.rs:81-101; zero coefficients skipped) */
void or_matmul_nn(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* out, int nthreads) {
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
  for (int64_t i = 0; i < m; i++) {
    float* o = out + i * n;
    for (int64_t j = 0; j < n; j++) o[j] = 0.0f;
    for (int64_t p = 0; p < k; p++) {
      const float av = a[i * k + p];
      if (av != 0.0f) axpy(av, b + p * n, o, n);
    }
  }
}

/* out[m x n] += a^T . b, a [k x m], b [k x n]  (src/tensor.rs:103-120) */
void or_matmul_tn_acc(float* out, const float* a, const float* b, int64_t k, int64_t m, int64_t n,
                      int nthreads) {
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
  for (int64_t i = 0; i < m; i++) {
    float* o = out + i * n;
    for (int64_t p = 0; p < k; p++) {
      const float av = a[p * m + i];
      if (av != 0.0f) axpy(av, b + p * n, o, n);
    }
  }
}

/* ------------------------------------------------------------------ trainer-native Q8_0
 * FrozenWeight::Q8_0 (src/frozen.rs:38-45): per 32-element block an f32 scale d = amax / 127 and
 * codes round(x / d) (Rust f32::round: halves away from zero, as C roundf), clamped to +-127
 * (src/frozen.rs:53-73).  Packed here as scales [n][k/32] then codes [n][k].  The forward is
 * q8_dot (src/frozen.rs:80-93: per block an f32 sum of q * x, then acc += d * s), the input
 * gradient q8_axpy per token and row (src/frozen.rs:96-108,156-166: a = g * d, blocks with
 * a == 0 skipped, y += a * q), row() is q8_axpy(1) into zeros (src/frozen.rs:172-176). */
int or_tq8_quantize(const float* w, int64_t n, int64_t k, void* out) {
  if (k % QK) return -2;
  const int64_t nb = k / QK;
  float* sc = (float*)out;
  int8_t* qs = (int8_t*)((uint8_t*)out + (size_t)(n * nb) * 4);
  for (int64_t b = 0; b < n * nb; b++) {
    const float* blk = w + b * QK;
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) amax = fmaxf(amax, fabsf(blk[i]));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    sc[b] = d;
    for (int i = 0; i < QK; i++) {
      float q = roundf(blk[i] * id);
      q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
      qs[b * QK + i] = (int8_t)q;
    }
  }
  return 0;
}

static float tq8_dot(const float* sc, const int8_t* qs, const float* x, int64_t k) {
  float acc = 0.0f;
  for (int64_t b = 0; b < k / QK; b++) {
    float s = 0.0f;
    for (int i = 0; i < QK; i++) s += (float)qs[b * QK + i] * x[b * QK + i];
    acc += sc[b] * s;
  }
  return acc;
}

static void tq8_axpy(float alpha, const float* sc, const int8_t* qs, float* y, int64_t k) {
  for (int64_t b = 0; b < k / QK; b++) {
    const float a = alpha * sc[b];
    if (a == 0.0f) continue;
    for (int i = 0; i < QK; i++) y[b * QK + i] += a * (float)qs[b * QK + i];
  }
}

static void tq8_views(const void* w, int64_t n, int64_t k, const float** sc, const int8_t** qs) {
  *sc = (const float*)w;
  *qs = (const int8_t*)((const uint8_t*)w + (size_t)(n * (k / QK)) * 4);
}

/* ------------------------------------------------------------------ FrozenMatmul */
static int supported_weight(int t) {
  return t == OR_F32 || t == OR_F16 || t == OR_Q4_0 || t == OR_Q8_0 || t == OR_Q4_K || t == OR_Q6_K ||
         t == OR_TQ8_0;
}

/* activation rows quantised once per call (QuantActs::prepare) */
static uint8_t* quantize_acts(int wtype, const float* x, int64_t t, int64_t k, int64_t* arow_bytes) {
  int at = or_act_type_for(wtype);
  int64_t rb = or_row_bytes(at, k);
  uint8_t* acts = (uint8_t*)malloc((size_t)(rb * t));
  for (int64_t i = 0; i < t; i++) {
    if (at == OR_Q8_0)
      or_quantize_acts_q8_0(x + i * k, k, acts + i * rb);
    else
      or_quantize_acts_q8_k(x + i * k, k, acts + i * rb);
  }
  *arow_bytes = rb;
  return acts;
}

/*
 * f32 epilogue over the integer block sums of one (row, token) pair.  rie-core's exact
 * accumulation order is unpinned (absent dependency); this follows ggml's scalar order:
 * per block sumf += (isum * d_w) * d_x, blocks in order; for Q4_K
 * sumf += (d*d_x)*S1 - (dmin*d_x)*S2; for Q6_K sumf += (d*d_x)*S.
 */
static float row_dot(int wtype, const uint8_t* wrow, const uint8_t* arow, int64_t k, int32_t* isums) {
  or_block_isums(wtype, wrow, arow, k, isums);
  float sumf = 0.0f;
  switch (wtype) {
    case OR_Q4_0:
    case OR_Q8_0: {
      const int64_t wb = wtype == OR_Q4_0 ? 18 : 34;
      for (int64_t i = 0; i < k / QK; i++) {
        const float dw = or_fp16_to_fp32(rd16(wrow + wb * i));
        const float dx = or_fp16_to_fp32(rd16(arow + 34 * i));
        sumf += ((float)isums[i] * dw) * dx;
      }
      break;
    }
    case OR_Q4_K:
      for (int64_t i = 0; i < k / QKK; i++) {
        float dx;
        memcpy(&dx, arow + 292 * i, 4);
        const float d = or_fp16_to_fp32(rd16(wrow + 144 * i)) * dx;
        const float dmin = or_fp16_to_fp32(rd16(wrow + 144 * i + 2)) * dx;
        sumf += d * (float)isums[2 * i] - dmin * (float)isums[2 * i + 1];
      }
      break;
    case OR_Q6_K:
      for (int64_t i = 0; i < k / QKK; i++) {
        float dx;
        memcpy(&dx, arow + 292 * i, 4);
        const float d = or_fp16_to_fp32(rd16(wrow + 210 * i + 208)) * dx;
        sumf += d * (float)isums[i];
      }
      break;
  }
  return sumf;
}

int or_frozen_forward(int wtype, const void* w, int64_t n, int64_t k, const float* x, int64_t t, float* y,
                      int nthreads) {
  if (!supported_weight(wtype)) return -1;
  if (wtype == OR_TQ8_0) { /* src/frozen.rs:121-136 */
    if (k % QK) return -2;
    const float* sc;
    const int8_t* qs;
    tq8_views(w, n, k, &sc, &qs);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < t; i++)
      for (int64_t o = 0; o < n; o++) y[i * n + o] = tq8_dot(sc + o * (k / QK), qs + o * k, x + i * k, k);
    return 0;
  }
  const int64_t wrb = or_row_bytes(wtype, k);
  if (wrb < 0) return -2;
  const uint8_t* W = (const uint8_t*)w;
  if (wtype == OR_F32 || wtype == OR_F16) {
    /* f32 / f16 weights skip activation quantisation: plain f32 dots */
#pragma omp parallel num_threads(nthr(nthreads))
    {
      float* row = (float*)malloc((size_t)k * 4);
#pragma omp for schedule(static)
      for (int64_t o = 0; o < n; o++) {
        or_dequant_row(wtype, W + o * wrb, k, row);
        for (int64_t i = 0; i < t; i++) y[i * n + o] = or_dot(x + i * k, row, k);
      }
      free(row);
    }
    return 0;
  }
  int64_t arb;
  uint8_t* acts = quantize_acts(wtype, x, t, k, &arb);
  const int64_t ni = or_isums_per_row(wtype, k);
#pragma omp parallel num_threads(nthr(nthreads))
  {
    int32_t* isums = (int32_t*)malloc((size_t)ni * 4);
#pragma omp for schedule(static)
    for (int64_t o = 0; o < n; o++)
      for (int64_t i = 0; i < t; i++) y[i * n + o] = row_dot(wtype, W + o * wrb, acts + i * arb, k, isums);
    free(isums);
  }
  free(acts);
  return 0;
}

int or_frozen_forward_f64(int wtype, const void* w, int64_t n, int64_t k, const float* x, int64_t t,
                          double* y) {
  if (!supported_weight(wtype)) return -1;
  if (wtype == OR_TQ8_0) { /* the same products, every sum in f64 */
    if (k % QK) return -2;
    const float* sc;
    const int8_t* qs;
    tq8_views(w, n, k, &sc, &qs);
    for (int64_t i = 0; i < t; i++)
      for (int64_t o = 0; o < n; o++) {
        double acc = 0;
        for (int64_t b = 0; b < k / QK; b++) {
          double s = 0;
          for (int j = 0; j < QK; j++) s += (double)qs[o * k + b * QK + j] * (double)x[i * k + b * QK + j];
          acc += (double)sc[o * (k / QK) + b] * s;
        }
        y[i * n + o] = acc;
      }
    return 0;
  }
  const int64_t wrb = or_row_bytes(wtype, k);
  if (wrb < 0) return -2;
  const uint8_t* W = (const uint8_t*)w;
  if (wtype == OR_F32 || wtype == OR_F16) {
    float* row = (float*)malloc((size_t)k * 4);
    for (int64_t o = 0; o < n; o++) {
      or_dequant_row(wtype, W + o * wrb, k, row);
      for (int64_t i = 0; i < t; i++) {
        double s = 0;
        for (int64_t j = 0; j < k; j++) s += (double)x[i * k + j] * (double)row[j];
        y[i * n + o] = s;
      }
    }
    free(row);
    return 0;
  }
  int64_t arb;
  uint8_t* acts = quantize_acts(wtype, x, t, k, &arb);
  const int64_t ni = or_isums_per_row(wtype, k);
  int32_t* is = (int32_t*)malloc((size_t)ni * 4);
  for (int64_t o = 0; o < n; o++) {
    const uint8_t* wr = W + o * wrb;
    for (int64_t i = 0; i < t; i++) {
      const uint8_t* ar = acts + i * arb;
      or_block_isums(wtype, wr, ar, k, is);
      double s = 0;
      if (wtype == OR_Q4_0 || wtype == OR_Q8_0) {
        const int64_t wb = wtype == OR_Q4_0 ? 18 : 34;
        for (int64_t b = 0; b < k / QK; b++)
          s += (double)is[b] * or_fp16_to_fp32(rd16(wr + wb * b)) * or_fp16_to_fp32(rd16(ar + 34 * b));
      } else {
        for (int64_t b = 0; b < k / QKK; b++) {
          float dx;
          memcpy(&dx, ar + 292 * b, 4);
          if (wtype == OR_Q4_K)
            s += (double)dx * ((double)or_fp16_to_fp32(rd16(wr + 144 * b)) * is[2 * b] -
                               (double)or_fp16_to_fp32(rd16(wr + 144 * b + 2)) * is[2 * b + 1]);
          else
            s += (double)dx * (double)or_fp16_to_fp32(rd16(wr + 210 * b + 208)) * is[b];
        }
      }
      y[i * n + o] = s;
    }
  }
  free(is);
  free(acts);
  return 0;
}

/* src/rie.rs:63-64 */
#define BWD_ROWS 32

/*
 * src/rie.rs:84-120: chunks of 32 rows are dequantised (no dy quantisation, straight-through),
 * each thread folds its chunks into a private [t x k] accumulator with f32 axpy, the per-thread
 * accumulators are reduced and added to dx.  The reduction order depends on the thread count,
 * as rayon's fold/reduce does in the reference.
 */
int or_frozen_backward_input(int wtype, const void* w, int64_t n, int64_t k, const float* dy, int64_t t,
                             float* dx, int nthreads) {
  if (!supported_weight(wtype)) return -1;
  if (wtype == OR_TQ8_0) { /* src/frozen.rs:155-166: per token, rows in order */
    if (k % QK) return -2;
    const float* sc;
    const int8_t* qs;
    tq8_views(w, n, k, &sc, &qs);
#pragma omp parallel for num_threads(nthr(nthreads)) schedule(static)
    for (int64_t i = 0; i < t; i++)
      for (int64_t o = 0; o < n; o++) {
        const float g = dy[i * n + o];
        if (g != 0.0f) tq8_axpy(g, sc + o * (k / QK), qs + o * k, dx + i * k, k);
      }
    return 0;
  }
  const int64_t wrb = or_row_bytes(wtype, k);
  if (wrb < 0) return -2;
  const uint8_t* W = (const uint8_t*)w;
  const int nt = nthr(nthreads);
  const int64_t nchunks = (n + BWD_ROWS - 1) / BWD_ROWS;
  float* accs = (float*)calloc((size_t)nt * t * k, 4);
#pragma omp parallel num_threads(nt)
  {
    const int tid = omp_get_thread_num();
    float* acc = accs + (size_t)tid * t * k;
    float* buf = (float*)malloc((size_t)BWD_ROWS * k * 4);
#pragma omp for schedule(static)
    for (int64_t c = 0; c < nchunks; c++) {
      const int64_t r0 = c * BWD_ROWS;
      const int64_t r1 = r0 + BWD_ROWS < n ? r0 + BWD_ROWS : n;
      for (int64_t r = r0; r < r1; r++) or_dequant_row(wtype, W + r * wrb, k, buf + (r - r0) * k);
      for (int64_t i = 0; i < t; i++)
        for (int64_t r = r0; r < r1; r++) {
          const float g = dy[i * n + r];
          if (g != 0.0f) axpy(g, buf + (r - r0) * k, acc + i * k, k);
        }
    }
    free(buf);
  }
  for (int th = 1; th < nt; th++) {
    const float* src = accs + (size_t)th * t * k;
    for (int64_t i = 0; i < t * k; i++) accs[i] += src[i];
  }
  for (int64_t i = 0; i < t * k; i++) dx[i] += accs[i];
  free(accs);
  return 0;
}

int or_frozen_row(int wtype, const void* w, int64_t n, int64_t k, int64_t r, float* out) {
  if (wtype == OR_TQ8_0) {
    if (k % QK || r < 0 || r >= n) return -2;
    const float* sc;
    const int8_t* qs;
    tq8_views(w, n, k, &sc, &qs);
    memset(out, 0, (size_t)k * 4);
    tq8_axpy(1.0f, sc + r * (k / QK), qs + r * k, out, k);
    return 0;
  }
  const int64_t wrb = or_row_bytes(wtype, k);
  if (wrb < 0 || r < 0 || r >= n) return -2;
  return or_dequant_row(wtype, (const uint8_t*)w + r * wrb, k, out);
}

/* ------------------------------------------------------------------ Linear + LoRA */
int or_linear_forward(int wtype, const void* w, int64_t n, int64_t k, const float* bias, int64_t rank,
                      float alpha, const float* A, const float* B, int lora_enabled, const float* x, int64_t t,
                      float* y, int nthreads) {
  int rc = or_frozen_forward(wtype, w, n, k, x, t, y, nthreads); /* src/linear.rs:76 */
  if (rc) return rc;
  if (bias) /* :77-83 */
    for (int64_t i = 0; i < t; i++)
      for (int64_t o = 0; o < n; o++) y[i * n + o] += bias[o];
  if (lora_enabled && rank > 0) { /* :84-91 */
    float* h = (float*)malloc((size_t)(t * rank) * 4);
    float* d = (float*)malloc((size_t)(t * n) * 4);
    or_matmul_nt(x, A, t, k, rank, h, nthreads);
    or_matmul_nt(h, B, t, rank, n, d, nthreads);
    const float s = alpha / (float)rank;
    for (int64_t i = 0; i < t * n; i++) y[i] += s * d[i];
    free(h);
    free(d);
  }
  return 0;
}

int or_linear_backward(int wtype, const void* w, int64_t n, int64_t k, int64_t rank, float alpha,
                       const float* A, const float* B, int lora_enabled, const float* x, const float* dy,
                       int64_t t, float* dx, float* ga, float* gb, int nthreads) {
  memset(dx, 0, (size_t)(t * k) * 4); /* src/linear.rs:100 */
  int rc = or_frozen_backward_input(wtype, w, n, k, dy, t, dx, nthreads);
  if (rc) return rc;
  if (lora_enabled && rank > 0) { /* :102-118 */
    const float s = alpha / (float)rank;
    float* h = (float*)malloc((size_t)(t * rank) * 4);
    float* sdy = (float*)malloc((size_t)(t * n) * 4);
    float* g = (float*)malloc((size_t)(t * rank) * 4);
    float* gx = (float*)malloc((size_t)(t * k) * 4);
    or_matmul_nt(x, A, t, k, rank, h, nthreads);
    for (int64_t i = 0; i < t * n; i++) sdy[i] = dy[i] * s;
    or_matmul_tn_acc(gb, sdy, h, t, n, rank, nthreads);
    or_matmul_nn(sdy, B, t, n, rank, g, nthreads);
    or_matmul_tn_acc(ga, g, x, t, rank, k, nthreads);
    or_matmul_nn(g, A, t, rank, k, gx, nthreads);
    for (int64_t i = 0; i < t * k; i++) dx[i] += gx[i];
    free(h);
    free(sdy);
    free(g);
    free(gx);
  }
  return 0;
}

/* ---- LM head + cross-entropy: Model::head (src/model.rs:561-609) ---- */

/* rmsnorm (src/ops.rs:14-36, fused_scale = false): y = (x * ir) * (w + off), ir = 1 / sqrt(dot(x, x) / d + eps) */
static void head_rmsnorm(const float* x, const float* w, int64_t d, float eps, float off, float* y, float* inv) {
  const float ms = or_dot(x, x, d) / (float)d;
  const float ir = 1.0f / sqrtf(ms + eps);
  *inv = ir;
  for (int64_t i = 0; i < d; i++) y[i] = x[i] * ir * (w[i] + off);
}

/* softmax_row (src/ops.rs:238-247): p = exp(v - max) in f32, normaliser summed in f64, p *= (f32)(1/s);
 * returns lse = max + (f32)ln(s) */
static float head_softmax_row(const float* row, int64_t v, float* p) {
  float m = -INFINITY;
  for (int64_t j = 0; j < v; j++) m = fmaxf(m, row[j]);
  double s = 0.0;
  for (int64_t j = 0; j < v; j++) {
    p[j] = expf(row[j] - m);
    s += (double)p[j];
  }
  const float inv = (float)(1.0 / s);
  for (int64_t j = 0; j < v; j++) p[j] *= inv;
  return m + (float)log(s);
}

int or_lm_head(int wtype, const void* w, int64_t V, int64_t d, const float* norm, float eps, float off,
               const float* x, int64_t t, const int32_t* pos, const int32_t* tok, const float* wts, int64_t n,
               int64_t chunk, float* logp, int64_t* hits, float* dx, int nthreads) {
  if (chunk < 1) chunk = 1;
  for (int64_t i = 0; i < n; i++)
    if (pos[i] < 0 || pos[i] >= t || tok[i] < 0 || tok[i] >= V) return -1; /* src/model.rs:575 assert */
  if (wts && dx) memset(dx, 0, (size_t)(t * d) * 4);
  int64_t nh = 0;
  float* xs = (float*)malloc((size_t)(chunk * d) * 4);
  float* ns = (float*)malloc((size_t)(chunk * d) * 4);
  float* inv = (float*)malloc((size_t)chunk * 4);
  float* logits = (float*)malloc((size_t)(chunk * V) * 4);
  float* p = (float*)malloc((size_t)V * 4);
  float* dns = (float*)malloc((size_t)(chunk * d) * 4);
  float* g = (float*)malloc((size_t)d * 4);
  int rc = 0;
  for (int64_t c0 = 0; c0 < n && !rc; c0 += chunk) {
    const int64_t m = n - c0 < chunk ? n - c0 : chunk;
    for (int64_t i = 0; i < m; i++) {
      memcpy(xs + i * d, x + (int64_t)pos[c0 + i] * d, (size_t)d * 4);
      head_rmsnorm(xs + i * d, norm, d, eps, off, ns + i * d, inv + i);
    }
    rc = or_frozen_forward(wtype, w, V, d, ns, m, logits, nthreads);
    if (rc) break;
    for (int64_t i = 0; i < m; i++) {
      float* row = logits + i * V;
      const float lse = head_softmax_row(row, V, p);
      const float tl = row[tok[c0 + i]];
      logp[c0 + i] = tl - lse;
      int all = 1;
      for (int64_t j = 0; j < V && all; j++) all = row[j] <= tl;
      nh += all;
      if (wts) { /* d(-w logp)/dlogits = w (softmax - onehot), written over the logits */
        const float wi = wts[c0 + i];
        for (int64_t j = 0; j < V; j++) row[j] = wi * p[j];
        row[tok[c0 + i]] -= wi;
      }
    }
    if (wts && dx) {
      memset(dns, 0, (size_t)(m * d) * 4);
      rc = or_frozen_backward_input(wtype, w, V, d, logits, m, dns, nthreads);
      if (rc) break;
      for (int64_t i = 0; i < m; i++) { /* rmsnorm_backward (src/ops.rs:39-56), then dx[pos] += dxs */
        const float* xr = xs + i * d;
        const float ir = inv[i];
        for (int64_t k = 0; k < d; k++) g[k] = dns[i * d + k] * (norm[k] + off);
        const float cc = or_dot(g, xr, d) * ir * ir * ir / (float)d;
        float* o = dx + (int64_t)pos[c0 + i] * d;
        for (int64_t k = 0; k < d; k++) o[k] += g[k] * ir - xr[k] * cc;
      }
    }
  }
  if (hits) *hits = nh;
  free(xs);
  free(ns);
  free(inv);
  free(logits);
  free(p);
  free(dns);
  free(g);
  return rc;
}
