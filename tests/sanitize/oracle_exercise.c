/*
 * Runs every function of the CPU oracle (oracle/oracle.c) under
 * AddressSanitizer and UndefinedBehaviorSanitizer: buffers are allocated at
 * exactly the sizes the functions document, so an access one byte past a
 * row, block or scale array is reported.  Shapes cover one row, ragged
 * 128-blocks, the smallest and two format blocks along K; values include
 * zeros, NaN, +-inf, subnormals and large magnitudes.  Built and run by
 * tests/test_sanitizers.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/oracle.h"

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint32_t next32(void) {
  rng ^= rng << 13;
  rng ^= rng >> 7;
  rng ^= rng << 17;
  return (uint32_t)(rng >> 16);
}

static float special(int i) {
  switch (i % 13) {
    case 0: return 0.0f;
    case 1: return -0.0f;
    case 2: return NAN;
    case 3: return INFINITY;
    case 4: return -INFINITY;
    case 5: return 1e-40f;  /* subnormal */
    case 6: return 3.0e38f;
    case 7: return -448.0f;
    default: return ((int)(next32() % 2001) - 1000) * 1e-4f;
  }
}

static void *xmalloc(size_t n) {
  void *p = malloc(n ? n : 1);
  if (!p) abort();
  return p;
}

static float *fill(int64_t count, int with_specials) {
  float *w = (float *)xmalloc((size_t)count * sizeof(float));
  for (int64_t i = 0; i < count; ++i) w[i] = with_specials ? special((int)i) : ((int)(next32() % 2001) - 1000) * 1e-4f;
  return w;
}

static uint8_t *bytes(size_t n) {
  uint8_t *b = (uint8_t *)xmalloc(n);
  for (size_t i = 0; i < n; ++i) b[i] = (uint8_t)next32();
  return b;
}

static void run(int64_t n, int64_t k, int specials) {
  float *w = fill(n * k, specials);
  float *out = (float *)xmalloc((size_t)(n * k) * sizeof(float));
  /* W8A16 */
  int8_t *q = (int8_t *)xmalloc((size_t)(n * k));
  float *s32 = (float *)xmalloc((size_t)n * 4);
  uint16_t *sb = (uint16_t *)xmalloc((size_t)n * 2);
  or_w8a16_quantize(w, n, k, q, s32, sb);
  or_w8a16_dequant(q, s32, 0, n, k, out);
  or_w8a16_dequant(q, sb, 1, n, k, out);
  float *x = fill(3 * k, specials), *y = (float *)xmalloc((size_t)(3 * n) * 4);
  or_w8a16_linear(x, q, sb, 1, 3, n, k, y);
  or_local_q8_forward(x, k, q, s32, n, y);
  double *yd = (double *)xmalloc((size_t)(3 * n) * 8);
  or_matmul_f64(x, w, 3, n, k, yd);
  /* FP8 row / block */
  uint8_t *codes = bytes((size_t)(n * k));
  or_fp8_row_dequant(codes, s32, n, k, out);
  const int64_t nb = ((n + 127) / 128) * ((k + 127) / 128);
  float *bs = (float *)xmalloc((size_t)nb * 4);
  or_fp8_block_quantize(w, n, k, codes, bs);
  or_fp8_block_dequant(codes, bs, n, k, out);
  /* activation quantizers */
  uint8_t *xq = (uint8_t *)xmalloc((size_t)(3 * k));
  float *xs = (float *)xmalloc(3 * 4);
  or_act_fp8_quantize(x, 3, k, xq, xs);
  if (k % 32 == 0) {
    uint8_t *xp = (uint8_t *)xmalloc((size_t)(3 * k / 2)), *xe = (uint8_t *)xmalloc((size_t)(3 * k / 32));
    or_act_mxfp4_quantize(x, 3, k, xp, xe);
    /* GGUF Q8_0 and MXFP4 */
    uint8_t *b8 = (uint8_t *)xmalloc((size_t)(n * (k / 32) * 34));
    or_q8_0_quantize(w, n, k, b8);
    or_q8_0_dequant(b8, n, k, out);
    uint8_t *pk = (uint8_t *)xmalloc((size_t)(n * k / 2)), *e8 = (uint8_t *)xmalloc((size_t)(n * k / 32));
    or_mxfp4_quantize(w, n, k, pk, e8);
    or_mxfp4_dequant(pk, e8, n, k, out);
    free(xp); free(xe); free(b8); free(pk); free(e8);
  }
  if (k % 16 == 0) {
    /* NVFP4 with the right lengths, e4m3 and f32 scales, then wrong lengths (error path) */
    uint8_t *pk = bytes((size_t)(n * k / 2)), *se = bytes((size_t)(n * k / 16));
    float *sf = fill(n * k / 16, specials);
    char err[128];
    or_nvfp4_dequant(pk, (size_t)(n * k / 2), se, (size_t)(n * k / 16), 1, 0.5f, n, k, out, err, sizeof err);
    or_nvfp4_dequant(pk, (size_t)(n * k / 2), sf, (size_t)(n * k / 16) * 4, 0, 2.0f, n, k, out, err, sizeof err);
    if (or_nvfp4_dequant(pk, (size_t)(n * k / 2) - 1, se, (size_t)(n * k / 16), 1, 1.0f, n, k, out, err,
                         sizeof err) == 0)
      abort();
    free(pk); free(se); free(sf);
  }
  if (k % 256 == 0) {
    uint8_t *b4 = (uint8_t *)xmalloc((size_t)(n * (k / 256) * 144));
    or_q4_k_quantize(w, n, k, b4);
    or_q4_k_dequant(b4, n, k, out);
    uint8_t *b6 = bytes((size_t)(n * (k / 256) * 210));
    or_q6_k_dequant(b6, n, k, out);
    /* random Q4_K bytes as a file would hold them */
    uint8_t *r4 = bytes((size_t)(n * (k / 256) * 144));
    or_q4_k_dequant(r4, n, k, out);
    free(b4); free(b6); free(r4);
  }
  free(w); free(out); free(q); free(s32); free(sb); free(x); free(y); free(yd); free(codes); free(bs);
  free(xq); free(xs);
}

int main(void) {
  /* codecs over every code */
  for (int c = 0; c < 65536; ++c) {
    volatile float a = or_f16_to_f32((uint16_t)c), b = or_bf16_to_f32((uint16_t)c);
    (void)or_f32_to_f16(a);
    (void)or_f32_to_bf16(b);
  }
  for (int c = 0; c < 256; ++c) {
    volatile float a = or_e4m3_to_f32((uint8_t)c) + or_e4m3_to_f32_ocp((uint8_t)c) + or_e2m1_to_f32((uint8_t)(c & 15)) +
                       or_e8m0_to_f32((uint8_t)c);
    (void)a;
  }
  for (int i = 0; i < 4096; ++i) {
    const float f = special(i) * (float)(i % 7);
    (void)or_f32_to_e4m3(f);
    (void)or_f32_to_e2m1(f);
  }
  const int64_t shapes[][2] = {{1, 8}, {1, 16}, {1, 32}, {3, 256}, {2, 512}, {129, 136}, {130, 256}, {17, 1024}};
  for (unsigned i = 0; i < sizeof shapes / sizeof shapes[0]; ++i)
    for (int sp = 0; sp < 2; ++sp) run(shapes[i][0], shapes[i][1], sp);
  puts("oracle exercise done");
  return 0;
}
