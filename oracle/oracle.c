/*
 * CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the contract and the parity status of each function.
 * Built with -ffp-contract=off: every float operation below rounds once, in
 * the order written, as the reference's Rust (which never contracts) does.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint32_t or_version(void) { return 1u; }

/* ------------------------------------------------------------------ */
/* scalar codecs                                                       */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: man * 2^-24 (exact in f32) */
    float v = (float)man * 0x1p-24f;
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t or_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) {
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | (man >> 13)); /* quiet NaN */
  }
  int32_t e = (int32_t)exp - 127;
  if (e > 15) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (e >= -14) {
    /* normal: keep 10 mantissa bits, RNE on the 13 dropped */
    uint32_t m = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint32_t he = (uint32_t)(e + 15);
    uint32_t out = (he << 10) | m;
    if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) out += 1; /* may carry */
    if (out >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | out);
  }
  /* subnormal half: value = sig * 2^(e-23), unit 2^-24 */
  if (e < -25) return (uint16_t)sign; /* < 2^-25: rounds to 0 (2^-25 tie too) */
  uint32_t sig = man | (exp ? 0x800000u : 0u);
  int shift = -e - 1; /* sig*2^(e-23)/2^-24 = sig * 2^(e+1) */
  /* e in [-25,-15] -> shift in [14,24] */
  uint32_t q = sig >> shift;
  uint32_t rem = sig & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
  uint32_t x = f2u(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  uint32_t round_bit = 0x8000u;
  if ((x & round_bit) && (x & (3u * round_bit - 1u)))
    return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}

float or_e4m3_to_f32(uint8_t code) {
  uint32_t sign = code >> 7;
  uint32_t exponent = (code >> 3) & 15u;
  uint32_t mantissa = code & 7u;
  float value;
  if (exponent == 0) {
    value = (float)mantissa * 0.001953125f;
  } else if (exponent == 15 && mantissa == 7) {
    value = 0.0f;
  } else {
    value = u2f((exponent + 120u) << 23) * (1.0f + (float)mantissa * 0.125f);
  }
  return sign ? -value : value;
}

float or_e4m3_to_f32_ocp(uint8_t code) {
  if ((code & 0x7f) == 0x7f) return NAN;
  return or_e4m3_to_f32(code);
}

/* Round the f32 magnitude `a` (finite, >= 0) to a binary format with `mbits`
 * mantissa bits, minimum normal exponent `emin` and largest finite value
 * `maxv`, saturating.  Returns the rounded value as f32 (exact). */
static float round_minifloat(float a, int mbits, int emin, float maxv) {
  if (a == 0.0f) return 0.0f;
  if (a >= maxv) return maxv;
  int e;
  (void)frexpf(a, &e); /* a = f * 2^e, f in [0.5,1) -> floor(log2 a) = e-1 */
  int el = e - 1;
  if (el < emin) el = emin; /* subnormal range: fixed quantum 2^(emin-mbits) */
  float quantum = ldexpf(1.0f, el - mbits);
  float units = a / quantum; /* exact: power-of-two division of a normal */
  float r = nearbyintf(units); /* RNE (default rounding mode) */
  float v = r * quantum;
  if (v > maxv) v = maxv;
  return v;
}

uint8_t or_f32_to_e4m3(float f) {
  if (isnan(f)) return 0x7f;
  uint8_t sign = signbit(f) ? 0x80 : 0x00;
  float a = fabsf(f);
  float v = round_minifloat(a, 3, -6, 448.0f);
  if (v == 0.0f) return sign;
  /* encode exact value v */
  int e;
  float fr = frexpf(v, &e); /* v = fr*2^e */
  int el = e - 1;
  if (el < -6) { /* subnormal: v = m * 2^-9 */
    int m = (int)(v * 512.0f);
    return (uint8_t)(sign | m);
  }
  int m = (int)((fr * 2.0f - 1.0f) * 8.0f);
  return (uint8_t)(sign | ((el + 7) << 3) | m);
}

static const float kE2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f,
                                4.0f, 6.0f, 0.0f, -0.5f, -1.0f, -1.5f,
                                -2.0f, -3.0f, -4.0f, -6.0f};

float or_e2m1_to_f32(uint8_t code) { return kE2M1[code & 15u]; }

uint8_t or_f32_to_e2m1(float f) {
  if (isnan(f)) return 0; /* not produced for finite inputs */
  uint8_t sign = signbit(f) ? 8 : 0;
  float v = round_minifloat(fabsf(f), 1, 0, 6.0f);
  for (uint8_t c = 0; c < 8; ++c)
    if (kE2M1[c] == v) return (uint8_t)(sign | c);
  return (uint8_t)(sign | 7);
}

float or_e8m0_to_f32(uint8_t e) {
  if (e == 0xff) return NAN;
  return ldexpf(1.0f, (int)e - 127);
}

/* Rust f32::round: half away from zero. */
static inline float round_away(float v) { return roundf(v); }

/* ------------------------------------------------------------------ */
/* W8A16                                                               */
/* ------------------------------------------------------------------ */
void or_w8a16_quantize(const float *w, int64_t n, int64_t k, int8_t *q,
                       float *scale_f32, uint16_t *scale_bf16) {
  for (int64_t r = 0; r < n; ++r) {
    const float *row = w + r * k;
    float max_abs = 0.0f;
    for (int64_t i = 0; i < k; ++i) {
      float a = fabsf(row[i]);
      /* Rust f32::max ignores a NaN operand */
      if (!(a <= max_abs) && !isnan(a)) max_abs = a;
    }
    float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    float inv_scale = 1.0f / scale;
    for (int64_t i = 0; i < k; ++i) {
      float v = round_away(row[i] * inv_scale);
      if (v < -127.0f) v = -127.0f;
      if (v > 127.0f) v = 127.0f;
      q[r * k + i] = isnan(v) ? 0 : (int8_t)v; /* Rust `as i8`: NaN -> 0 */
    }
    if (scale_f32) scale_f32[r] = scale;
    if (scale_bf16) scale_bf16[r] = or_f32_to_bf16(scale);
  }
}

static inline float load_scale(const void *scale, int is_bf16, int64_t i) {
  return is_bf16 ? or_bf16_to_f32(((const uint16_t *)scale)[i])
                 : ((const float *)scale)[i];
}

void or_w8a16_dequant(const int8_t *q, const void *scale, int scale_is_bf16,
                      int64_t n, int64_t k, float *out) {
  for (int64_t r = 0; r < n; ++r) {
    float s = load_scale(scale, scale_is_bf16, r);
    for (int64_t i = 0; i < k; ++i) out[r * k + i] = (float)q[r * k + i] * s;
  }
}

/* ------------------------------------------------------------------ */
/* GGUF Q8_0                                                           */
/* ------------------------------------------------------------------ */
static inline void put_u16(uint8_t *p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}
static inline uint16_t get_u16(const uint8_t *p) {
  return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

void or_q8_0_quantize(const float *w, int64_t n, int64_t k, uint8_t *blocks) {
  int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t b = 0; b < nb; ++b) {
      const float *xs = w + r * k + b * 32;
      uint8_t *blk = blocks + (r * nb + b) * 34;
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) {
        float a = fabsf(xs[i]);
        if (!(a <= amax) && !isnan(a)) amax = a;
      }
      float d = amax / 127.0f;
      float id = d != 0.0f ? 1.0f / d : 0.0f;
      put_u16(blk, or_f32_to_f16(d));
      for (int i = 0; i < 32; ++i) {
        float v = round_away(xs[i] * id);
        int iv;
        if (isnan(v)) iv = 0;
        else if (v > 127.0f) iv = 127;
        else if (v < -128.0f) iv = -128;
        else iv = (int)v;
        blk[2 + i] = (uint8_t)(int8_t)iv;
      }
    }
  }
}

void or_q8_0_dequant(const uint8_t *blocks, int64_t n, int64_t k, float *out) {
  int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t *blk = blocks + (r * nb + b) * 34;
      float d = or_f16_to_f32(get_u16(blk));
      for (int i = 0; i < 32; ++i)
        out[r * k + b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* ------------------------------------------------------------------ */
/* GGUF Q4_K                                                           */
/* ------------------------------------------------------------------ */
void or_q4_k_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* candle's nearest_int: f32::round (half away) then `as i32`. */
static inline int nearest_int(float v) {
  if (isnan(v)) return 0;
  float r = roundf(v);
  if (r >= 2147483647.0f) return 2147483647;
  if (r <= -2147483648.0f) return (-2147483647 - 1);
  return (int)r;
}

/* candle k_quants make_qkx1_quants(nmax, ntry, x) -> (scale, -min) */
static void make_qkx1_quants(int nmax, int ntry, const float *x, int n,
                             float *out_scale, float *out_min) {
  uint8_t l[32];
  memset(l, 0, sizeof(l));
  float min = x[0], max = x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < min) min = x[i];
    if (x[i] > max) max = x[i];
  }
  if (max == min) {
    *out_scale = 0.0f;
    *out_min = 0.0f;
    return;
  }
  if (min > 0.0f) min = 0.0f;
  float iscale = (float)nmax / (max - min);
  float scale = 1.0f / iscale;
  for (int it = 0; it < ntry; ++it) {
    float sumlx = 0.0f;
    int suml2 = 0;
    int did_change = 0;
    for (int i = 0; i < n; ++i) {
      int li = nearest_int(iscale * (x[i] - min));
      if (li < 0) li = 0;
      if (li > nmax) li = nmax;
      if ((uint8_t)li != l[i]) {
        l[i] = (uint8_t)li;
        did_change = 1;
      }
      sumlx += (x[i] - min) * (float)li;
      suml2 += li * li;
    }
    scale = sumlx / (float)suml2;
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)l[i];
    min = sum / (float)n;
    if (min > 0.0f) min = 0.0f;
    iscale = 1.0f / scale;
    if (!did_change) break;
  }
  *out_scale = scale;
  *out_min = -min;
}

void or_q4_k_quantize(const float *w, int64_t n, int64_t k, uint8_t *blocks) {
  int64_t nb = k / 256;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const float *x = w + r * k + b * 256;
      uint8_t *blk = blocks + (r * nb + b) * 144;
      uint8_t *scales = blk + 4;
      uint8_t *qs = blk + 16;
      float mins[8], scl[8];
      for (int j = 0; j < 8; ++j)
        make_qkx1_quants(15, 5, x + 32 * j, 32, &scl[j], &mins[j]);
      float max_scale = 0.0f, max_min = 0.0f;
      for (int j = 0; j < 8; ++j) {
        if (scl[j] > max_scale) max_scale = scl[j];
        if (mins[j] > max_min) max_min = mins[j];
      }
      float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
      float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
      memset(scales, 0, 12);
      for (int j = 0; j < 8; ++j) {
        int ls_i = nearest_int(inv_scale * scl[j]);
        int lm_i = nearest_int(inv_min * mins[j]);
        uint8_t ls = (uint8_t)(ls_i < 63 ? ls_i : 63);
        uint8_t lm = (uint8_t)(lm_i < 63 ? lm_i : 63);
        if (j < 4) {
          scales[j] = ls;
          scales[j + 4] = lm;
        } else {
          scales[j + 4] = (uint8_t)((ls & 0xf) | ((lm & 0xf) << 4));
          scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
          scales[j] |= (uint8_t)((lm >> 4) << 6);
        }
      }
      uint16_t dh = or_f32_to_f16(max_scale / 63.0f);
      uint16_t mh = or_f32_to_f16(max_min / 63.0f);
      put_u16(blk, dh);
      put_u16(blk + 2, mh);
      uint8_t L[256];
      memset(L, 0, sizeof(L));
      for (int j = 0; j < 8; ++j) {
        uint8_t sc, m;
        or_q4_k_scale_min(j, scales, &sc, &m);
        float d = or_f16_to_f32(dh) * (float)sc;
        if (d != 0.0f) {
          float dm = or_f16_to_f32(mh) * (float)m;
          for (int ii = 0; ii < 32; ++ii) {
            int lv = nearest_int((x[32 * j + ii] + dm) / d);
            if (lv < 0) lv = 0;
            if (lv > 15) lv = 15;
            L[32 * j + ii] = (uint8_t)lv;
          }
        }
      }
      for (int j = 0; j < 256; j += 64)
        for (int l = 0; l < 32; ++l)
          qs[j / 2 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    }
}

void or_q4_k_dequant(const uint8_t *blocks, int64_t n, int64_t k, float *out) {
  int64_t nb = k / 256;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t *blk = blocks + (r * nb + b) * 144;
      float d = or_f16_to_f32(get_u16(blk));
      float dmin = or_f16_to_f32(get_u16(blk + 2));
      const uint8_t *scales = blk + 4;
      const uint8_t *qs = blk + 16;
      float *y = out + r * k + b * 256;
      int is = 0;
      for (int j = 0; j < 256; j += 64) {
        const uint8_t *q = qs + j / 2;
        uint8_t sc, m;
        or_q4_k_scale_min(is, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        or_q4_k_scale_min(is + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[l] & 0xf) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[l] >> 4) - m2;
        is += 2;
      }
    }
}

void or_q6_k_dequant(const uint8_t *blocks, int64_t n, int64_t k, float *out) {
  int64_t nb = k / 256;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t *blk = blocks + (r * nb + b) * 210;
      const uint8_t *ql = blk, *qh = blk + 128;
      const int8_t *sc = (const int8_t *)(blk + 192);
      const float d = or_f16_to_f32(get_u16(blk + 208));
      float *y = out + r * k + b * 256;
      for (int h = 0; h < 2; ++h) {
        for (int l = 0; l < 32; ++l) {
          const int is = l / 16;
          const int q1 = (int)((ql[l] & 0xf) | (((qh[l] >> 0) & 3) << 4)) - 32;
          const int q2 = (int)((ql[l + 32] & 0xf) | (((qh[l] >> 2) & 3) << 4)) - 32;
          const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
          const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
          y[l] = d * (float)sc[is] * (float)q1;
          y[l + 32] = d * (float)sc[is + 2] * (float)q2;
          y[l + 64] = d * (float)sc[is + 4] * (float)q3;
          y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
      }
    }
}

/* ------------------------------------------------------------------ */
/* FP8                                                                 */
/* ------------------------------------------------------------------ */
void or_fp8_row_dequant(const uint8_t *q, const float *scale, int64_t n,
                        int64_t k, float *out) {
  for (int64_t r = 0; r < n; ++r)
    for (int64_t i = 0; i < k; ++i)
      out[r * k + i] = or_e4m3_to_f32(q[r * k + i]) * scale[r];
}

void or_fp8_block_quantize(const float *w, int64_t n, int64_t k, uint8_t *q,
                           float *scales) {
  int64_t nbn = (n + 127) / 128, nbk = (k + 127) / 128;
  for (int64_t bn = 0; bn < nbn; ++bn)
    for (int64_t bk = 0; bk < nbk; ++bk) {
      int64_t r1 = bn * 128 + 128 < n ? bn * 128 + 128 : n;
      int64_t c1 = bk * 128 + 128 < k ? bk * 128 + 128 : k;
      float amax = 0.0f;
      for (int64_t r = bn * 128; r < r1; ++r)
        for (int64_t c = bk * 128; c < c1; ++c) {
          float a = fabsf(w[r * k + c]);
          if (!(a <= amax) && !isnan(a)) amax = a;
        }
      float s = amax > 0.0f ? amax / 448.0f : 1.0f;
      float inv = 1.0f / s;
      scales[bn * nbk + bk] = s;
      for (int64_t r = bn * 128; r < r1; ++r)
        for (int64_t c = bk * 128; c < c1; ++c)
          q[r * k + c] = or_f32_to_e4m3(w[r * k + c] * inv);
    }
}

void or_fp8_block_dequant(const uint8_t *q, const float *scales, int64_t n,
                          int64_t k, float *out) {
  int64_t nbk = (k + 127) / 128;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t c = 0; c < k; ++c)
      out[r * k + c] =
          or_e4m3_to_f32(q[r * k + c]) * scales[(r / 128) * nbk + c / 128];
}

/* ------------------------------------------------------------------ */
/* NVFP4                                                               */
/* ------------------------------------------------------------------ */
int or_nvfp4_dequant(const uint8_t *packed, size_t packed_len,
                     const void *scales, size_t scales_len,
                     int scales_are_e4m3, float global_scale, int64_t n,
                     int64_t k, float *out, char *err, size_t err_size) {
  if (k % 16 != 0) {
    if (err) snprintf(err, err_size, "NVFP4 input dimension %lld is not divisible by group size 16", (long long)k);
    return -1;
  }
  size_t expected_packed = (size_t)(n * k / 2);
  if (packed_len != expected_packed) {
    if (err) snprintf(err, err_size, "NVFP4 packed weight has %zu bytes, expected %zu", packed_len, expected_packed);
    return -1;
  }
  int64_t gpr = k / 16;
  size_t expected_scales = (size_t)(n * gpr);
  if (scales_len != expected_scales) {
    if (err) snprintf(err, err_size, "NVFP4 weight scale has %zu values, expected %zu", scales_len, expected_scales);
    return -1;
  }
  for (int64_t r = 0; r < n; ++r)
    for (int64_t c = 0; c < k; ++c) {
      uint8_t byte = packed[r * (k / 2) + c / 2];
      uint8_t code = (c % 2 == 0) ? (byte & 0x0f) : (byte >> 4);
      float s = scales_are_e4m3
                    ? or_e4m3_to_f32(((const uint8_t *)scales)[r * gpr + c / 16])
                    : ((const float *)scales)[r * gpr + c / 16];
      out[r * k + c] = kE2M1[code] * s * global_scale;
    }
  return 0;
}

/* ------------------------------------------------------------------ */
/* MXFP4                                                               */
/* ------------------------------------------------------------------ */
static int floor_log2_f32(float a) { /* a > 0, finite */
  int e;
  (void)frexpf(a, &e);
  return e - 1;
}

static void mx_block(const float *x, int len, uint8_t *codes, uint8_t *scale) {
  float amax = 0.0f;
  for (int i = 0; i < len; ++i) {
    float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  int shared = amax > 0.0f ? floor_log2_f32(amax) - 2 : -127;
  if (shared < -127) shared = -127;
  if (shared > 127) shared = 127;
  *scale = (uint8_t)(shared + 127);
  for (int i = 0; i < len; ++i) codes[i] = or_f32_to_e2m1(ldexpf(x[i], -shared));
}

void or_mxfp4_quantize(const float *w, int64_t n, int64_t k, uint8_t *packed,
                       uint8_t *scales) {
  int64_t nb = k / 32;
  uint8_t codes[32];
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      mx_block(w + r * k + b * 32, 32, codes, &scales[r * nb + b]);
      for (int i = 0; i < 16; ++i)
        packed[r * (k / 2) + b * 16 + i] =
            (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
    }
}

void or_mxfp4_dequant(const uint8_t *packed, const uint8_t *scales, int64_t n,
                      int64_t k, float *out) {
  int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t c = 0; c < k; ++c) {
      uint8_t byte = packed[r * (k / 2) + c / 2];
      uint8_t code = (c % 2 == 0) ? (byte & 0x0f) : (byte >> 4);
      out[r * k + c] = kE2M1[code] * or_e8m0_to_f32(scales[r * nb + c / 32]);
    }
}

void or_act_fp8_quantize(const float *x, int64_t m, int64_t k, uint8_t *q,
                         float *scale) {
  for (int64_t r = 0; r < m; ++r) {
    float amax = 0.0f;
    for (int64_t i = 0; i < k; ++i) {
      float a = fabsf(x[r * k + i]);
      if (a > amax) amax = a;
    }
    float s = amax > 0.0f ? amax / 448.0f : 1.0f;
    float inv = 1.0f / s;
    scale[r] = s;
    for (int64_t i = 0; i < k; ++i) q[r * k + i] = or_f32_to_e4m3(x[r * k + i] * inv);
  }
}

void or_act_mxfp4_quantize(const float *x, int64_t m, int64_t k,
                           uint8_t *packed, uint8_t *scales) {
  or_mxfp4_quantize(x, m, k, packed, scales);
}

/* ------------------------------------------------------------------ */
/* products                                                            */
/* ------------------------------------------------------------------ */
void or_matmul_f64(const float *x, const float *w, int64_t m, int64_t n,
                   int64_t k, double *y) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      const float *xr = x + i * k, *wr = w + j * k;
      for (int64_t t = 0; t < k; ++t) acc += (double)xr[t] * (double)wr[t];
      y[i * n + j] = acc;
    }
}

void or_w8a16_linear(const float *x, const int8_t *q, const void *scale,
                     int scale_is_bf16, int64_t m, int64_t n, int64_t k,
                     float *y) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (int64_t t = 0; t < k; ++t) sum += (float)q[j * k + t] * x[i * k + t];
      y[i * n + j] = sum * load_scale(scale, scale_is_bf16, j);
    }
}

void or_local_q8_forward(const float *x, int64_t k, const int8_t *q,
                         const float *scale, int64_t n, float *y) {
  float x_max_abs = 0.0f;
  for (int64_t i = 0; i < k; ++i) {
    float a = fabsf(x[i]);
    if (!(a <= x_max_abs) && !isnan(a)) x_max_abs = a;
  }
  float x_scale = x_max_abs > 0.0f ? x_max_abs / 127.0f : 1.0f;
  float inv_x_scale = 1.0f / x_scale;
  if (k <= 0) {
    for (int64_t r = 0; r < n; ++r) y[r] = 0.0f * scale[r] * x_scale;
    return;
  }
  int8_t *xq = (int8_t *)malloc((size_t)k);
  for (int64_t i = 0; i < k; ++i) {
    float v = round_away(x[i] * inv_x_scale);
    if (v < -127.0f) v = -127.0f;
    if (v > 127.0f) v = 127.0f;
    xq[i] = isnan(v) ? 0 : (int8_t)v;
  }
  for (int64_t r = 0; r < n; ++r) {
    int32_t acc = 0;
    for (int64_t i = 0; i < k; ++i) acc += (int32_t)q[r * k + i] * (int32_t)xq[i];
    y[r] = (float)acc * scale[r] * x_scale;
  }
  free(xq);
}
