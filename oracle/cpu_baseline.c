/*
 * CPU baseline for the quantized decode GEMV -- TEST/BENCH INFRASTRUCTURE.
 *
 * A multi-threaded restatement of the reference's host-side arithmetic
 * (dequantize on the fly, f32 dot per output row, rows split over worker
 * threads in chunks of 64 the way rayon par_chunks splits them in
 * qwen3_vl/text.rs:315-327).  It is timed by the benchmark's cpu_baseline
 * leg and checked against the scalar oracle by tests; the product never
 * calls it.  Unlike oracle.c it may reassociate the k-sum (eight partial
 * sums) so the compiler can vectorise it, as a tuned CPU path would.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define ROWS_PER_TASK 64

static inline float bf16f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float dot8(const float *a, const float *b, int64_t k) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= k; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] += a[i + j] * b[i + j];
  float s = 0.0f;
  for (int j = 0; j < 8; ++j) s += acc[j];
  for (; i < k; ++i) s += a[i] * b[i];
  return s;
}

/* y[m,n] (f32) = sum_k x[m,k] * dequant(w)[n,k]; x given as bf16 bits. */
void cb_w8a16_gemv(const uint16_t *x, int64_t m, int64_t k, const int8_t *q,
                   const uint16_t *scale_bf16, int64_t n, float *y,
                   int threads) {
  int64_t tasks = (n + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
#pragma omp parallel num_threads(threads)
  {
    int64_t mm = m < 8 ? m : 8;
    float *xbuf = (float *)malloc(sizeof(float) * (size_t)(k * (mm + 1)));
    float *xf[8];
    for (int64_t r = 0; r < mm; ++r) {
      xf[r] = xbuf + r * k;
      for (int64_t i = 0; i < k; ++i) xf[r][i] = bf16f(x[r * k + i]);
    }
    float *wf = xbuf + mm * k;
#pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < tasks; ++t) {
      int64_t r1 = (t + 1) * ROWS_PER_TASK < n ? (t + 1) * ROWS_PER_TASK : n;
      for (int64_t row = t * ROWS_PER_TASK; row < r1; ++row) {
        const int8_t *qr = q + row * k;
        for (int64_t i = 0; i < k; ++i) wf[i] = (float)qr[i];
        float s = bf16f(scale_bf16[row]);
        for (int64_t r = 0; r < mm; ++r) y[r * n + row] = dot8(xf[r], wf, k) * s;
      }
    }
    free(xbuf);
  }
}

void cb_q4_k_gemv(const uint16_t *x, int64_t m, int64_t k,
                  const uint8_t *blocks, int64_t n, float *y, int threads) {
  int64_t tasks = (n + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
  int64_t nb = k / 256;
#pragma omp parallel num_threads(threads)
  {
    int64_t mm = m < 8 ? m : 8;
    float *xbuf = (float *)malloc(sizeof(float) * (size_t)(k * (mm + 1)));
    float *xf[8];
    for (int64_t r = 0; r < mm; ++r) {
      xf[r] = xbuf + r * k;
      for (int64_t i = 0; i < k; ++i) xf[r][i] = bf16f(x[r * k + i]);
    }
    float *wf = xbuf + mm * k;
#pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < tasks; ++t) {
      int64_t r1 = (t + 1) * ROWS_PER_TASK < n ? (t + 1) * ROWS_PER_TASK : n;
      for (int64_t row = t * ROWS_PER_TASK; row < r1; ++row) {
        or_q4_k_dequant(blocks + row * nb * 144, 1, k, wf);
        for (int64_t r = 0; r < mm; ++r) y[r * n + row] = dot8(xf[r], wf, k);
      }
    }
    free(xbuf);
  }
}
