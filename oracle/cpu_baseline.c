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

/* Prefill: y[m,n] (f32) = sum_k x[m,k] * dequant(w)[n,k] for M rows, a
 * blocked f32 GEMM with on-the-fly dequantization.  The bf16 activations are
 * widened once; each task dequantizes 64 weight rows to f32 (the rayon
 * chunk size of qwen3_vl/text.rs:315-327) and multiplies them against all
 * M rows in 4 x 4 register tiles of 8-wide vector accumulators, so every
 * loaded x and w vector feeds four FMAs. */
typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float *p) {
  v8f v;
  memcpy(&v, p, sizeof v);
  return v;
}

static inline float hsum8(v8f v) {
  return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

void cb_w8a16_gemm(const uint16_t *x, int64_t m, int64_t k, const int8_t *q,
                   const uint16_t *scale_bf16, int64_t n, float *y,
                   int threads) {
  float *xf = (float *)malloc(sizeof(float) * (size_t)(m * k));
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < m * k; ++i) xf[i] = bf16f(x[i]);
  const int64_t tasks = (n + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
#pragma omp parallel num_threads(threads)
  {
    float *wf = (float *)malloc(sizeof(float) * (size_t)(ROWS_PER_TASK * k));
#pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < tasks; ++t) {
      const int64_t n0 = t * ROWS_PER_TASK;
      const int64_t nr = (n0 + ROWS_PER_TASK < n ? ROWS_PER_TASK : n - n0);
      for (int64_t r = 0; r < nr; ++r) {
        const int8_t *qr = q + (n0 + r) * k;
        for (int64_t i = 0; i < k; ++i) wf[r * k + i] = (float)qr[i];
      }
      for (int64_t m0 = 0; m0 < m; m0 += 4) {
        const int mr = (int)(m - m0 < 4 ? m - m0 : 4);
        for (int64_t j0 = 0; j0 < nr; j0 += 4) {
          const int jr = (int)(nr - j0 < 4 ? nr - j0 : 4);
          v8f acc[4][4];
          memset(acc, 0, sizeof acc);
          const float *xr[4], *wr[4];
          for (int a = 0; a < 4; ++a) {
            xr[a] = xf + (m0 + (a < mr ? a : 0)) * k;
            wr[a] = wf + (j0 + (a < jr ? a : 0)) * k;
          }
          for (int64_t kk = 0; kk + 8 <= k; kk += 8) {
            const v8f x0 = ld8(xr[0] + kk), x1 = ld8(xr[1] + kk), x2 = ld8(xr[2] + kk), x3 = ld8(xr[3] + kk);
            const v8f w0 = ld8(wr[0] + kk), w1 = ld8(wr[1] + kk), w2 = ld8(wr[2] + kk), w3 = ld8(wr[3] + kk);
            acc[0][0] += x0 * w0; acc[0][1] += x0 * w1; acc[0][2] += x0 * w2; acc[0][3] += x0 * w3;
            acc[1][0] += x1 * w0; acc[1][1] += x1 * w1; acc[1][2] += x1 * w2; acc[1][3] += x1 * w3;
            acc[2][0] += x2 * w0; acc[2][1] += x2 * w1; acc[2][2] += x2 * w2; acc[2][3] += x2 * w3;
            acc[3][0] += x3 * w0; acc[3][1] += x3 * w1; acc[3][2] += x3 * w2; acc[3][3] += x3 * w3;
          }
          for (int a = 0; a < mr; ++a)
            for (int b = 0; b < jr; ++b) {
              float sum = hsum8(acc[a][b]);
              for (int64_t kk = k & ~(int64_t)7; kk < k; ++kk) sum += xr[a][kk] * wr[b][kk];
              y[(m0 + a) * n + n0 + j0 + b] = sum * bf16f(scale_bf16[n0 + j0 + b]);
            }
        }
      }
    }
    free(wf);
  }
  free(xf);
}
