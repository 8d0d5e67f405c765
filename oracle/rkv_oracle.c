/*
 * rkv_oracle.c -- CPU restatement of the reference's paged-Q8 KV path.
 *
 * TEST INFRASTRUCTURE ONLY (see rkv_oracle.h).  Build with
 * gcc -O2 -ffp-contract=off -fno-fast-math (oracle/Makefile).  All f32
 * arithmetic below is written in the reference's order; float expressions
 * stay float (x86-64 SSE, FLT_EVAL_METHOD == 0).
 */
#include "rkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- small helpers mirroring Rust `as` casts ----------------------------- */

/* Rust `f32 as i32` / `f64 as i32`: saturating, NaN -> 0. */
static int32_t sat_i32(double x) {
  if (isnan(x)) return 0;
  if (x >= 2147483647.0) return INT32_MAX;
  if (x <= -2147483648.0) return INT32_MIN;
  return (int32_t)x;
}
/* Rust `f64 as u16`: saturating, NaN -> 0. */
static uint16_t sat_u16(double x) {
  if (isnan(x) || x <= 0.0) return 0;
  if (x >= 65535.0) return 65535;
  return (uint16_t)x;
}
/* Rust `f32 as i8`: saturating, NaN -> 0. */
static int8_t sat_i8(float x) {
  if (isnan(x)) return 0;
  if (x >= 127.0f) return 127;
  if (x <= -128.0f) return -128;
  return (int8_t)x;
}

static uint32_t f32_bits(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return u;
}
static float bits_f32(uint32_t u) {
  float v;
  memcpy(&v, &u, 4);
  return v;
}

/* ---- generators --------------------------------------------------------- */

/* tools/repro-harness/src/main.rs:81-88 */
uint64_t rko_splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ULL;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

/* tools/repro-harness/src/main.rs:90-95 */
float rko_seeded_float(uint64_t index) {
  uint64_t x = index * 2654435761ULL + 1013904223ULL;
  uint32_t word = (uint32_t)rko_splitmix64(x);
  float num = (float)word;
  float den = (float)UINT32_MAX; /* u32::MAX as f32 == 4294967296.0f */
  float t = num / den;
  t = t * 8.0f;
  return t - 4.0f;
}

/* har/crates/har-serve/src/q4k.rs:109-120 */
void rko_lcg_values(float *out, size_t count, uint64_t seed) {
  uint64_t state = seed;
  for (size_t i = 0; i < count; ++i) {
    state = state * 6364136223846793005ULL + 1442695040888963407ULL;
    float u = (float)(uint32_t)(state >> 40) / (float)(1u << 24);
    out[i] = u - 0.5f;
  }
}

/* Counter-based N(0,1): pair k uses splitmix64(key + 2k) and
 * splitmix64(key + 2k + 1) as two 53-bit uniforms; Box-Muller in f64. */
void rko_normal_f32(float *out, size_t count, uint64_t seed) {
  const double two_pi = 6.283185307179586476925286766559;
  uint64_t key = rko_splitmix64(seed);
  for (size_t i = 0; i < count; i += 2) {
    uint64_t k = (uint64_t)(i / 2);
    uint64_t a = rko_splitmix64(key + 2 * k) >> 11;
    uint64_t b = rko_splitmix64(key + 2 * k + 1) >> 11;
    double u1 = ((double)a + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)b * (1.0 / 9007199254740992.0);         /* [0,1) */
    double r = sqrt(-2.0 * log(u1));
    out[i] = (float)(r * cos(two_pi * u2));
    if (i + 1 < count) out[i + 1] = (float)(r * sin(two_pi * u2));
  }
}

uint16_t rko_f32_to_bf16(float v) {
  uint32_t u = f32_bits(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}
float rko_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* ---- binary16 ------------------------------------------------------------ */

/* har/crates/r4kv/src/f16.rs:4-25 */
float rko_f16_to_f32(uint16_t bits) {
  uint32_t sign = ((uint32_t)(bits >> 15)) << 31;
  uint32_t exp = (bits >> 10) & 0x1f;
  uint32_t frac = bits & 0x3ff;
  uint32_t out;
  if (exp == 0) {
    if (frac == 0) {
      out = sign;
    } else {
      int t = 31 - __builtin_clz(frac); /* highest set bit index */
      int exp32 = 127 + t - 24;
      uint32_t mantissa = (frac << (23 - t)) & 0x007fffffu;
      out = sign | (((uint32_t)exp32 & 0xff) << 23) | mantissa;
    }
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (frac << 13);
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (frac << 13);
  }
  return bits_f32(out);
}

/* har/crates/har-serve/src/q4k.rs:22-50 */
float rko_f16_to_f32_harserve(uint8_t b0, uint8_t b1) {
  uint16_t bits = (uint16_t)(b0 | ((uint16_t)b1 << 8));
  uint32_t sign = (bits >> 15) & 1;
  uint32_t exp = (bits >> 10) & 0x1f;
  uint32_t frac = bits & 0x3ff;
  float value;
  if (exp == 0) {
    if (frac == 0) {
      value = 0.0f;
    } else {
      float m = (float)frac / 1024.0f;
      value = m * ldexpf(1.0f, -14); /* 2f32.powi(-14) */
    }
  } else if (exp == 31) {
    value = frac == 0 ? INFINITY : NAN;
  } else {
    float m = 1.0f + (float)frac / 1024.0f;
    value = m * ldexpf(1.0f, (int)exp - 15);
  }
  return sign == 1 ? -value : value;
}

/* har/crates/r4kv/src/f16.rs:27-86 */
uint16_t rko_f32_to_f16(float v) {
  uint32_t x = f32_bits(v);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  int32_t aexp = (int32_t)((x >> 23) & 0xff);
  uint32_t frac = x & 0x007fffffu;
  if (aexp == 0xff) return (uint16_t)(sign | 0x7c00 | (frac != 0 ? 0x0200 : 0));
  int32_t e = aexp - 127;
  uint32_t mant = frac | 0x00800000u;
  if (e > 15) return (uint16_t)(sign | 0x7c00);
  if (e >= -14) {
    uint32_t exp_h = (uint32_t)(e + 15);
    uint32_t keep = mant >> 13;
    uint32_t rem = mant & 0x1fff;
    uint32_t halfway = 0x1000;
    uint32_t r = keep;
    if (rem > halfway || (rem == halfway && (keep & 1) == 1)) r += 1;
    if (r >= 0x800) {
      uint32_t eo = exp_h + 1;
      if (eo >= 0x1f) return (uint16_t)(sign | 0x7c00);
      return (uint16_t)(sign | (eo << 10));
    }
    return (uint16_t)(sign | (exp_h << 10) | (r & 0x3ff));
  }
  if (aexp == 0 && frac == 0) return sign;
  int64_t sh = -(1 + (int64_t)e);
  if (sh >= 31) return sign;
  uint64_t m64 = mant;
  uint32_t whole = (uint32_t)(m64 >> sh);
  uint64_t rem = m64 & ((1ULL << sh) - 1);
  uint64_t halfway = 1ULL << (sh - 1);
  uint32_t kept = whole;
  if (rem > halfway || (rem == halfway && (whole & 1) == 1)) kept += 1;
  if (kept >= 0x400) return (uint16_t)(sign | (1 << 10));
  return (uint16_t)(sign | kept);
}

/* har/crates/har-serve/src/attention.rs:45-76 */
uint16_t rko_f32_to_f16_harserve(float value) {
  double v = (double)value;
  if (v == 0.0) return signbit(v) ? 0x8000 : 0;
  if (!isfinite(v)) {
    if (isnan(v)) return 0x7e00;
    return v > 0.0 ? 0x7c00 : 0xfc00;
  }
  int32_t exp = sat_i32(floor(log2(fabs(v))));
  if (exp < -14) {
    int32_t m = sat_i32(round(v / ldexp(1.0, -24)));
    uint16_t bits = (uint16_t)(m > 0 ? m : 0); /* m.max(0) as u16 */
    return v < 0.0 ? (uint16_t)(bits | 0x8000) : bits;
  }
  if (exp > 15) return v < 0.0 ? 0xfc00 : 0x7c00;
  uint16_t mantissa = sat_u16(round((v / ldexp(1.0, exp) - 1.0) * 1024.0));
  uint16_t bits = (uint16_t)((((uint16_t)(exp + 15)) << 10) | (mantissa & 0x3ff));
  return v < 0.0 ? (uint16_t)(bits | 0x8000) : bits;
}

/* ---- Q8_0 codecs ---------------------------------------------------------- */

/* har/crates/r4kv/src/quant.rs:45-90 (Fmt::Q8, max_code 127) */
static float q8_group_canonical(const float *src, uint8_t *dst) {
  float amax = 0.0f;
  for (int i = 0; i < RKO_Q8_GROUP; ++i) {
    float a = fabsf(src[i]);
    if (a > amax) amax = a;
  }
  float d = amax == 0.0f ? 0.0f : amax / 127.0f;
  float inv = d == 0.0f ? 0.0f : 1.0f / d;
  uint16_t h = rko_f32_to_f16(d);
  dst[0] = (uint8_t)(h & 0xff);
  dst[1] = (uint8_t)(h >> 8);
  float max_err = 0.0f;
  for (int i = 0; i < RKO_Q8_GROUP; ++i) {
    float v = src[i];
    int32_t q = sat_i32((double)roundf(v * inv));
    if (q < -127) q = -127;
    if (q > 127) q = 127;
    dst[2 + i] = (uint8_t)(int8_t)q;
    float dq = (float)q * d;
    float e = fabsf(v - dq);
    if (e > max_err) max_err = e;
  }
  return max_err;
}

/* har/crates/r4kv/src/quant.rs:138-170 (Fmt::Q8 branch) */
float rko_q8_encode(const float *src, size_t n, uint8_t *dst) {
  float worst = 0.0f;
  for (size_t g = 0; g < n / RKO_Q8_GROUP; ++g) {
    float err = q8_group_canonical(src + g * RKO_Q8_GROUP, dst + g * RKO_Q8_GROUP_BYTES);
    if (err > worst) worst = err;
  }
  return worst;
}

/* har/crates/har-serve/src/attention.rs:25-42 */
void rko_q8_quantize_harserve(const float *src, size_t n, uint8_t *dst) {
  for (size_t g = 0; g < n / RKO_Q8_GROUP; ++g) {
    const float *block = src + g * RKO_Q8_GROUP;
    uint8_t *out = dst + g * RKO_Q8_GROUP_BYTES;
    float max_abs = 0.0f;
    for (int i = 0; i < RKO_Q8_GROUP; ++i) max_abs = fmaxf(max_abs, fabsf(block[i]));
    float d = max_abs == 0.0f ? 0.0f : max_abs / 127.0f;
    uint16_t h = rko_f32_to_f16_harserve(d);
    out[0] = (uint8_t)(h & 0xff);
    out[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < RKO_Q8_GROUP; ++i) {
      int8_t q = 0;
      if (d != 0.0f) {
        float r = roundf(block[i] / d);
        /* f32::clamp(-127, 127) keeps NaN; `as i8` maps NaN to 0 */
        if (r < -127.0f) r = -127.0f;
        if (r > 127.0f) r = 127.0f;
        q = sat_i8(r);
      }
      out[2 + i] = (uint8_t)q;
    }
  }
}

/* har/crates/r4kv/src/quant.rs:173-225 (Fmt::Q8 branch) */
void rko_q8_decode(const uint8_t *src, size_t n, float *dst) {
  for (size_t g = 0; g < n / RKO_Q8_GROUP; ++g) {
    const uint8_t *b = src + g * RKO_Q8_GROUP_BYTES;
    float d = rko_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    for (int j = 0; j < RKO_Q8_GROUP; ++j) {
      int32_t c = (int8_t)b[2 + j];
      dst[g * RKO_Q8_GROUP + j] = (float)c * d;
    }
  }
}

/* har/crates/har-serve/src/attention.rs:79-90 */
void rko_q8_dequant_row(const uint8_t *row, size_t n, float *dst) {
  for (size_t b = 0; b < n / RKO_Q8_GROUP; ++b) {
    float d = rko_f16_to_f32_harserve(row[b * 34], row[b * 34 + 1]);
    for (int i = 0; i < RKO_Q8_GROUP; ++i) {
      int8_t q = (int8_t)row[b * 34 + 2 + i];
      dst[b * RKO_Q8_GROUP + i] = d * (float)q;
    }
  }
}

/* har/crates/r4kv/src/quant.rs:141-155 and 181-186 (Fmt::F16) */
void rko_f16_encode(const float *src, size_t n, uint16_t *dst) {
  for (size_t i = 0; i < n; ++i) dst[i] = rko_f32_to_f16(src[i]);
}
void rko_f16_decode(const uint16_t *src, size_t n, float *dst) {
  for (size_t i = 0; i < n; ++i) dst[i] = rko_f16_to_f32(src[i]);
}

/* har/crates/r4kv/src/quant.rs:228-245 */
void rko_roundtrip_stats(const float *src, size_t n, int fmt, float *decoded,
                         rko_group_stats *st) {
  if (fmt == 0) {
    uint16_t *enc = (uint16_t *)malloc(n * 2);
    rko_f16_encode(src, n, enc);
    rko_f16_decode(enc, n, decoded);
    free(enc);
  } else {
    uint8_t *enc = (uint8_t *)malloc(n / RKO_Q8_GROUP * RKO_Q8_GROUP_BYTES);
    rko_q8_encode(src, n, enc);
    rko_q8_decode(enc, n, decoded);
    free(enc);
  }
  st->max_abs_err = 0.0f;
  st->sum_sq_err = 0.0;
  st->sum_sq_ref = 0.0;
  for (size_t i = 0; i < n; ++i) {
    double e = (double)(src[i] - decoded[i]);
    if (fabs(e) > (double)st->max_abs_err) st->max_abs_err = (float)fabs(e);
    st->sum_sq_err += e * e;
    st->sum_sq_ref += (double)src[i] * (double)src[i];
  }
}

/* har/crates/r4kv/src/quant.rs:27-32 */
float rko_rel_rms(const rko_group_stats *st) {
  if (st->sum_sq_ref == 0.0) return 0.0f;
  return (float)sqrt(st->sum_sq_err / st->sum_sq_ref);
}

/* tools/repro-harness/src/main.rs:192-204 */
double rko_normalized_kl(const float *ref, const float *cand, size_t n) {
  double ref_sum = 0.0, cand_sum = 0.0;
  for (size_t i = 0; i < n; ++i) ref_sum += (double)ref[i];
  for (size_t i = 0; i < n; ++i) cand_sum += fmax((double)cand[i], 1.0e-12);
  double acc = 0.0;
  for (size_t i = 0; i < n; ++i) {
    double p = fmax((double)ref[i] / ref_sum, 1.0e-12);
    double q = fmax(fmax((double)cand[i], 1.0e-12) / cand_sum, 1.0e-12);
    acc += p * log(p / q);
  }
  return acc;
}

/* ---- reference (contiguous) flash decode ---------------------------------- */

static size_t row_bytes_of(int32_t head_dim) { return (size_t)head_dim / 32 * 34; }

/* har/crates/har-serve/src/attention.rs:92-94 */
static uint8_t byte_at(const uint32_t *words, size_t byte_offset) {
  return (uint8_t)((words[byte_offset >> 2] >> ((byte_offset & 3) * 8)) & 0xff);
}

/* har/crates/har-serve/src/attention.rs:98-112 */
float rko_q8_kv_value(const uint32_t *words, size_t row_word, size_t index) {
  size_t block_off = (index / 32) * 34;
  size_t byte_off = block_off + 2 + (index % 32);
  uint32_t scale_word = words[row_word + (block_off >> 2)];
  float h0 = rko_f16_to_f32_harserve((uint8_t)scale_word, (uint8_t)(scale_word >> 8));
  float h1 = rko_f16_to_f32_harserve((uint8_t)(scale_word >> 16), (uint8_t)(scale_word >> 24));
  float d = (block_off % 4 == 0) ? h0 : h1;
  return d * (float)(int8_t)byte_at(words, row_word * 4 + byte_off);
}

/* har/crates/har-serve/src/attention.rs:115-120 */
void rko_row_to_words(const uint8_t *row, size_t nbytes, uint32_t *words) {
  for (size_t i = 0; i + 3 < nbytes; i += 4)
    words[i / 4] = (uint32_t)row[i] | ((uint32_t)row[i + 1] << 8) |
                   ((uint32_t)row[i + 2] << 16) | ((uint32_t)row[i + 3] << 24);
}

/* har/crates/har-serve/src/attention.rs:169-215 */
void rko_flash_decode_online(const rko_fd_params *p, const uint32_t *k_words,
                             const uint32_t *v_words, const float *q, int32_t kvh,
                             float *m_out, float *l_out, float *o) {
  const int32_t D = p->head_dim;
  const size_t row_words = row_bytes_of(D) / 4;
  const size_t k_base = ((size_t)kvh * (size_t)p->seq_len) * row_words;
  const size_t v_base = k_base;
  float m = -INFINITY;
  float l = 0.0f;
  for (int32_t i = 0; i < D; ++i) o[i] = 0.0f;
  float *scores = (float *)malloc(sizeof(float) * (size_t)(p->chunk > 0 ? p->chunk : 1));
  float *o_c = (float *)malloc(sizeof(float) * (size_t)D);
  for (int32_t c = 0; c < p->seq_len; c += p->chunk) {
    int32_t n = p->seq_len - c < p->chunk ? p->seq_len - c : p->chunk;
    float chunk_max = -INFINITY;
    for (int32_t pp = 0; pp < n; ++pp) {
      size_t pos = (size_t)(c + pp);
      float s = 0.0f;
      for (int32_t i = 0; i < D; ++i)
        s += q[i] * rko_q8_kv_value(k_words, k_base + pos * row_words, (size_t)i);
      scores[pp] = s;
      chunk_max = fmaxf(chunk_max, s);
    }
    float l_c = 0.0f;
    for (int32_t i = 0; i < D; ++i) o_c[i] = 0.0f;
    for (int32_t pp = 0; pp < n; ++pp) {
      float e = expf(scores[pp] - chunk_max);
      size_t pos = (size_t)(c + pp);
      for (int32_t i = 0; i < D; ++i)
        o_c[i] += e * rko_q8_kv_value(v_words, v_base + pos * row_words, (size_t)i);
      l_c += e;
    }
    float m_new = fmaxf(m, chunk_max);
    float a = expf(m - m_new);
    float b = expf(chunk_max - m_new);
    for (int32_t i = 0; i < D; ++i) o[i] = o[i] * a + o_c[i] * b;
    l = l * a + l_c * b;
    m = m_new;
  }
  free(scores);
  free(o_c);
  *m_out = m;
  *l_out = l;
}

/* har/crates/har-serve/src/attention.rs:148-165 */
void rko_flash_decode_reference(const rko_fd_params *p, const uint32_t *k_words,
                                const uint32_t *v_words, const float *query,
                                float *out) {
  const int32_t D = p->head_dim;
  int32_t q_per_kv = p->q_heads / p->kv_heads;
  float *o = (float *)malloc(sizeof(float) * (size_t)D);
  for (int32_t qh = 0; qh < p->q_heads; ++qh) {
    int32_t kvh = qh / q_per_kv;
    float m, l;
    rko_flash_decode_online(p, k_words, v_words, query + (size_t)qh * D, kvh, &m, &l, o);
    for (int32_t i = 0; i < D; ++i) out[(size_t)qh * D + i] = o[i] / l;
  }
  free(o);
}

/* The reference loop above over n independent sequences (each with its own
 * contiguous K/V words and q_heads query rows), spread over `threads` OpenMP
 * threads by (sequence, q head); each head runs attention.rs:148-165
 * unchanged.  Used to time the CPU path on all host cores. */
void rko_flash_decode_reference_many(const rko_fd_params *p, int32_t n,
                                     const uint32_t *const *k_words,
                                     const uint32_t *const *v_words, const float *queries,
                                     float *out, int32_t threads) {
  const int32_t D = p->head_dim;
  const int32_t q_per_kv = p->q_heads / p->kv_heads;
  const int32_t total = n * p->q_heads;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (int32_t w = 0; w < total; ++w) {
    const int32_t s = w / p->q_heads, qh = w % p->q_heads;
    float *o = (float *)malloc(sizeof(float) * (size_t)D);
    float m, l;
    rko_flash_decode_online(p, k_words[s], v_words[s], queries + ((size_t)s * p->q_heads + qh) * D,
                            qh / q_per_kv, &m, &l, o);
    for (int32_t i = 0; i < D; ++i) out[((size_t)s * p->q_heads + qh) * D + i] = o[i] / l;
    free(o);
  }
}

/* har/crates/har-serve/src/attention.rs:219-250 */
void rko_flash_decode_bruteforce(const rko_fd_params *p, const uint32_t *k_words,
                                 const uint32_t *v_words, const float *q,
                                 int32_t kvh, float *o) {
  const int32_t D = p->head_dim;
  const size_t row_words = row_bytes_of(D) / 4;
  const size_t k_base = ((size_t)kvh * (size_t)p->seq_len) * row_words;
  const size_t v_base = k_base;
  float *scores = (float *)malloc(sizeof(float) * (size_t)(p->seq_len > 0 ? p->seq_len : 1));
  float max_s = -INFINITY;
  for (int32_t pp = 0; pp < p->seq_len; ++pp) {
    float s = 0.0f;
    for (int32_t i = 0; i < D; ++i)
      s += q[i] * rko_q8_kv_value(k_words, k_base + (size_t)pp * row_words, (size_t)i);
    scores[pp] = s;
    max_s = fmaxf(max_s, s);
  }
  float l = 0.0f;
  for (int32_t i = 0; i < D; ++i) o[i] = 0.0f;
  for (int32_t pp = 0; pp < p->seq_len; ++pp) {
    float e = expf(scores[pp] - max_s);
    for (int32_t i = 0; i < D; ++i)
      o[i] += e * rko_q8_kv_value(v_words, v_base + (size_t)pp * row_words, (size_t)i);
    l += e;
  }
  for (int32_t i = 0; i < D; ++i) o[i] /= l;
  free(scores);
}

/* attention.rs:182-204 per chunk, without the running combine */
int32_t rko_flash_decode_partials(const rko_fd_params *p, const uint32_t *k_words,
                                  const uint32_t *v_words, const float *q,
                                  int32_t kvh, float *cm, float *lc, float *oc) {
  const int32_t D = p->head_dim;
  int32_t nchunks = 0;
  rko_fd_params one = *p;
  for (int32_t c = 0; c < p->seq_len; c += p->chunk, ++nchunks) {
    /* A single-chunk run of attention.rs:169-215 over positions [c, c+n)
     * leaves (m, l, o) = (chunk_max, l_c, o_c) exactly (a = 0, b = 1). */
    int32_t n = p->seq_len - c < p->chunk ? p->seq_len - c : p->chunk;
    const size_t row_words = row_bytes_of(D) / 4;
    const size_t base = ((size_t)kvh * (size_t)p->seq_len + (size_t)c) * row_words;
    one.seq_len = n;
    one.chunk = n;
    /* kvh is folded into the base pointer: view the slice as kv head 0 */
    rko_flash_decode_online(&one, k_words + base, v_words + base, q, 0, &cm[nchunks],
                            &lc[nchunks], oc + (size_t)nchunks * D);
  }
  return nchunks;
}

/* attention.rs:205-212 applied across partials in order */
void rko_lse_combine(int32_t n, int32_t head_dim, const float *cm, const float *lc,
                     const float *oc, float *out, float *m_out, float *l_out) {
  float m = -INFINITY, l = 0.0f;
  float *o = (float *)calloc((size_t)head_dim, sizeof(float));
  for (int32_t c = 0; c < n; ++c) {
    float m_new = fmaxf(m, cm[c]);
    float a = expf(m - m_new);
    float b = expf(cm[c] - m_new);
    for (int32_t i = 0; i < head_dim; ++i)
      o[i] = o[i] * a + oc[(size_t)c * head_dim + i] * b;
    l = l * a + lc[c] * b;
    m = m_new;
  }
  for (int32_t i = 0; i < head_dim; ++i) out[i] = o[i] / l;
  if (m_out) *m_out = m;
  if (l_out) *l_out = l;
  free(o);
}

void rko_attention_f64(int32_t seq_len, int32_t head_dim, const uint32_t *k_words,
                       const uint32_t *v_words, const float *q, double *out) {
  const size_t row_words = row_bytes_of(head_dim) / 4;
  double *s = (double *)malloc(sizeof(double) * (size_t)(seq_len > 0 ? seq_len : 1));
  double mx = -INFINITY;
  for (int32_t p = 0; p < seq_len; ++p) {
    double acc = 0.0;
    for (int32_t i = 0; i < head_dim; ++i)
      acc += (double)q[i] * (double)rko_q8_kv_value(k_words, (size_t)p * row_words, (size_t)i);
    s[p] = acc;
    if (acc > mx) mx = acc;
  }
  double l = 0.0;
  for (int32_t i = 0; i < head_dim; ++i) out[i] = 0.0;
  for (int32_t p = 0; p < seq_len; ++p) {
    double e = exp(s[p] - mx);
    l += e;
    for (int32_t i = 0; i < head_dim; ++i)
      out[i] += e * (double)rko_q8_kv_value(v_words, (size_t)p * row_words, (size_t)i);
  }
  for (int32_t i = 0; i < head_dim; ++i) out[i] = l > 0.0 ? out[i] / l : 0.0;
  free(s);
}

/* ---- paged layout ----------------------------------------------------------
 * One layer of the pool is num_pages pages; a page holds page_tokens slots
 * for every kv head, K then V:  page = [kv_head][kind K|V][region].
 * region = codes (page_tokens*D bytes) then scales (page_tokens*D/32 f16).
 *   K codes: [slot][dim]                         (row-major, as the reference row)
 *   V codes: [slot/TT][dim][slot%TT]             (dim-major inside TT-slot tiles)
 *   scales : [slot/TT][block][pos(slot%TT)]  (K and V)
 * with TT = min(32, page_tokens); for TT == 32, pos(16m + 4g + r) = 8g + 4m + r
 * (m<2, g<4, r<4), for TT == 16 pos(t) = t.  Restated here independently of the HIP
 * source so the checker does not share code with the product. */

static int32_t tile_tokens(const rko_layout *L) {
  return L->page_tokens < 32 ? L->page_tokens : 32;
}
size_t rko_region_bytes(const rko_layout *L) {
  return (size_t)L->page_tokens * (size_t)L->head_dim +
         (size_t)L->page_tokens * (size_t)(L->head_dim / 32) * 2;
}
size_t rko_page_bytes(const rko_layout *L) {
  return (size_t)L->kv_heads * 2 * rko_region_bytes(L);
}
size_t rko_code_offset(const rko_layout *L, int kind, int32_t slot, int32_t dim) {
  const size_t D = (size_t)L->head_dim;
  if (kind == 0) return (size_t)slot * D + (size_t)dim;
  const int32_t TT = tile_tokens(L);
  return (size_t)(slot / TT) * D * (size_t)TT + (size_t)dim * (size_t)TT + (size_t)(slot % TT);
}
size_t rko_scale_offset(const rko_layout *L, int32_t slot, int32_t block) {
  const int32_t TT = tile_tokens(L);
  const size_t nb = (size_t)(L->head_dim / 32);
  int32_t t = slot % TT;
  if (TT == 32) {
    int32_t m = t / 16, g = (t / 4) % 4, r = t % 4;
    t = 8 * g + 4 * m + r;
  }
  return (size_t)L->page_tokens * (size_t)L->head_dim +
         2 * ((size_t)(slot / TT) * nb * (size_t)TT + (size_t)block * (size_t)TT + (size_t)t);
}
/* V codes are stored as x ^ 0x80 (unsigned x + 128), K codes as they are */
static uint8_t v_bias(int kind) { return kind == 1 ? 0x80 : 0x00; }
static size_t region_base(const rko_layout *L, int32_t page, int32_t kvh, int kind) {
  return (size_t)page * rko_page_bytes(L) + (size_t)(kvh * 2 + kind) * rko_region_bytes(L);
}

int32_t rko_paged_append(const rko_layout *L, uint8_t *pages,
                         const int32_t *block_tables, int32_t bt_stride,
                         const int32_t *seq_ids, const int32_t *positions,
                         int32_t n_rows, const float *k_src, const float *v_src,
                         int rule) {
  const int32_t D = L->head_dim;
  const int32_t nb = D / 32;
  uint8_t *row = (uint8_t *)malloc(row_bytes_of(D));
  for (int32_t r = 0; r < n_rows; ++r) {
    int32_t pos = positions[r];
    if (pos < 0 || pos / L->page_tokens >= bt_stride) { free(row); return -3; }
    int32_t page = block_tables[(size_t)seq_ids[r] * bt_stride + pos / L->page_tokens];
    if (page < 0 || page >= L->num_pages) { free(row); return -3; }
    int32_t slot = pos % L->page_tokens;
    for (int32_t h = 0; h < L->kv_heads; ++h) {
      for (int kind = 0; kind < 2; ++kind) {
        const float *src = (kind == 0 ? k_src : v_src) + ((size_t)r * L->kv_heads + h) * D;
        if (rule == 0) rko_q8_encode(src, (size_t)D, row);
        else rko_q8_quantize_harserve(src, (size_t)D, row);
        uint8_t *reg = pages + region_base(L, page, h, kind);
        for (int32_t b = 0; b < nb; ++b) {
          size_t so = rko_scale_offset(L, slot, b);
          reg[so] = row[b * 34];
          reg[so + 1] = row[b * 34 + 1];
          for (int32_t i = 0; i < 32; ++i)
            reg[rko_code_offset(L, kind, slot, b * 32 + i)] = row[b * 34 + 2 + i] ^ v_bias(kind);
        }
      }
    }
  }
  free(row);
  return 0;
}

int32_t rko_paged_gather(const rko_layout *L, const uint8_t *pages,
                         const int32_t *block_table, int32_t len, int kind,
                         uint8_t *out) {
  const int32_t D = L->head_dim;
  const int32_t nb = D / 32;
  const size_t rb = row_bytes_of(D);
  for (int32_t h = 0; h < L->kv_heads; ++h) {
    for (int32_t pos = 0; pos < len; ++pos) {
      int32_t page = block_table[pos / L->page_tokens];
      if (page < 0 || page >= L->num_pages) return -3;
      int32_t slot = pos % L->page_tokens;
      const uint8_t *reg = pages + region_base(L, page, h, kind);
      uint8_t *row = out + ((size_t)h * (size_t)len + (size_t)pos) * rb;
      for (int32_t b = 0; b < nb; ++b) {
        size_t so = rko_scale_offset(L, slot, b);
        row[b * 34] = reg[so];
        row[b * 34 + 1] = reg[so + 1];
        for (int32_t i = 0; i < 32; ++i)
          row[b * 34 + 2 + i] = reg[rko_code_offset(L, kind, slot, b * 32 + i)] ^ v_bias(kind);
      }
    }
  }
  return 0;
}

int32_t rko_paged_decode(const rko_layout *L, const uint8_t *pages,
                         const int32_t *block_tables, int32_t bt_stride,
                         const int32_t *seq_lens, const int32_t *seq_ids, int32_t batch,
                         int32_t q_len, int32_t q_heads, const float *q, float scale,
                         int32_t chunk, float *out) {
  const int32_t D = L->head_dim;
  const size_t rb = row_bytes_of(D);
  const int32_t q_per_kv = q_heads / L->kv_heads;
  float *qs = (float *)malloc(sizeof(float) * (size_t)D);
  float *o = (float *)malloc(sizeof(float) * (size_t)D);
  for (int32_t b = 0; b < batch; ++b) {
    int32_t seq = seq_ids[b];
    int32_t len = seq_lens[seq];
    const int32_t *bt = block_tables + (size_t)seq * bt_stride;
    size_t nbytes = (size_t)L->kv_heads * (size_t)(len > 0 ? len : 1) * rb;
    uint8_t *kr = (uint8_t *)malloc(nbytes);
    uint8_t *vr = (uint8_t *)malloc(nbytes);
    uint32_t *kw = (uint32_t *)malloc(nbytes);
    uint32_t *vw = (uint32_t *)malloc(nbytes);
    if (rko_paged_gather(L, pages, bt, len, 0, kr) != 0 ||
        rko_paged_gather(L, pages, bt, len, 1, vr) != 0) {
      free(kr); free(vr); free(kw); free(vw); free(qs); free(o);
      return -3;
    }
    rko_row_to_words(kr, (size_t)L->kv_heads * len * rb, kw);
    rko_row_to_words(vr, (size_t)L->kv_heads * len * rb, vw);
    for (int32_t j = 0; j < q_len; ++j) {
      int32_t n = len - q_len + j + 1; /* causal within the draft rows */
      for (int32_t qh = 0; qh < q_heads; ++qh) {
        int32_t kvh = qh / q_per_kv;
        const float *qsrc = q + (((size_t)b * q_len + j) * q_heads + qh) * D;
        float *dst = out + (((size_t)b * q_len + j) * q_heads + qh) * D;
        for (int32_t i = 0; i < D; ++i) qs[i] = qsrc[i] * scale;
        if (n <= 0) { /* shader rule (flash_decode_q8.comp:144-148): l == 0 -> 0 */
          for (int32_t i = 0; i < D; ++i) dst[i] = 0.0f;
          continue;
        }
        rko_fd_params pr = {q_heads, L->kv_heads, n, chunk, D};
        /* rows of kv head kvh start at kvh*len; view them as kv head 0 of an
         * n-position cache */
        size_t off = (size_t)kvh * (size_t)len * (rb / 4);
        float m, l;
        rko_flash_decode_online(&pr, kw + off, vw + off, qs, 0, &m, &l, o);
        for (int32_t i = 0; i < D; ++i) dst[i] = o[i] / l;
      }
    }
    free(kr); free(vr); free(kw); free(vw);
  }
  free(qs);
  free(o);
  return 0;
}

/* ---- R4KV page container ----------------------------------------------------- */

/* har/crates/r4kv/src/crc32c.rs:4-21 (table) and :23-31 (loop) */
uint32_t rko_crc32c(const uint8_t *data, size_t n) {
  static uint32_t table[256];
  static int ready = 0;
  if (!ready) {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1u) ? (0x82f63b78u ^ (c >> 1)) : (c >> 1);
      table[i] = c;
    }
    ready = 1;
  }
  uint32_t c = 0xffffffffu;
  for (size_t i = 0; i < n; ++i) c = table[(c ^ data[i]) & 0xffu] ^ (c >> 8);
  return c ^ 0xffffffffu;
}

/* page.rs:78-86 put_u16/put_u32/put_u64 (little endian) */
static void le_put(uint8_t *b, size_t off, uint64_t v, int bytes) {
  for (int i = 0; i < bytes; ++i) b[off + (size_t)i] = (uint8_t)(v >> (8 * i));
}

/* page.rs:100-126 */
void rko_r4kv_header_bytes(const rko_r4kv_header *h, uint8_t out[96]) {
  memset(out, 0, 96);
  le_put(out, 0, 0x52344B56u, 4); /* MAGIC "R4KV", page.rs:11 */
  le_put(out, 4, 1, 2);           /* VERSION, page.rs:12 */
  le_put(out, 6, h->flags, 2);
  le_put(out, 8, h->prefix_digest, 8);
  le_put(out, 16, h->token_start, 4);
  le_put(out, 20, h->token_count, 4);
  le_put(out, 24, h->pos_start, 4);
  le_put(out, 28, h->layer_lo, 2);
  le_put(out, 30, h->layer_hi, 2);
  out[32] = h->k_fmt;
  out[33] = h->v_fmt;
  le_put(out, 34, h->epoch, 4);
  le_put(out, 38, h->generation, 4);
  le_put(out, 42, h->payload_len, 8);
  le_put(out, 50, h->sketch_offset, 4);
  /* 54..92 reserved zeros */
  le_put(out, 92, rko_crc32c(out, 92), 4);
}

/* page.rs:213-224 */
void rko_r4kv_pack_page(const rko_r4kv_header *h, const uint8_t *body, size_t n, uint8_t *out) {
  rko_r4kv_header_bytes(h, out);
  if (n) memcpy(out + 96, body, n);
  le_put(out, 96 + n, rko_crc32c(body, n), 4);
}

