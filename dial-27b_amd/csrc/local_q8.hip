// Local q8 W8A8 decode (qwen3_vl/text.rs:291-336) on gfx950.
//
// The reference quantizes the [1,1,K] activation with one per-tensor scale
// (x_scale = amax/127, xq = clamp(round(x/x_scale))), takes an exact i32 dot
// with each int8 weight row and returns f32(acc) * scale[n] * x_scale.  The
// resident W8A16 tile (16 bytes per lane, k = 16g + j) is exactly the B
// operand of v_mfma_i32_16x16x64_i8, so the dot runs on the integer MFMA with
// the same exact i32 result; only the final two f32 multiplies round, in the
// reference order.
#include "tile_ops.hpp"

namespace dialq {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// One 256-thread block: amax, scale and the int8 activation vector.
__global__ __launch_bounds__(256) void k_local_q8_quant(const void *x, int dtype, int64_t K,
                                                        int64_t k_pad, int8_t *xq, float *xscale) {
  __shared__ float sh[8];
  float amax = 0.0f;
  for (int64_t i = threadIdx.x; i < K; i += 256) {
    float a = fabsf(load_in(x, i, dtype));
    amax = (a > amax) ? a : amax;
  }
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  float xs = amax > 0.0f ? amax / 127.0f : 1.0f;
  float inv = 1.0f / xs;
  for (int64_t i = threadIdx.x; i < k_pad; i += 256) {
    int8_t q = 0;
    if (i < K) {
      float v = roundf(load_in(x, i, dtype) * inv);
      v = fminf(fmaxf(v, -127.0f), 127.0f);
      q = (v == v) ? (int8_t)v : (int8_t)0;
    }
    xq[i] = q;
  }
  if (threadIdx.x == 0) *xscale = xs;
}

__global__ __launch_bounds__(1024) void k_local_q8_dot(WeightView w, const int8_t *xq,
                                                       const float *xscale, void *y, int y_dtype) {
  __shared__ int red[16 * 64 * 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t s = blockIdx.x, kc = w.k_chunks;
  i32x4 acc = {0, 0, 0, 0};
  for (int64_t c = wave; c < kc; c += W) {
    RawTile t = load_tile<DIALQ_FORMAT_W8A16>(w.tiles, s * kc + c, lane);
    u32x4 a = {0, 0, 0, 0};
    if (r == 0) a = *(const u32x4 *)(xq + c * 64 + 16 * g);
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                                __builtin_bit_cast(i32x4, t.a), acc, 0, 0, 0);
  }
  // row m = 0 of C sits in lanes g = 0, element 0
  red[wave * 64 + lane] = acc[0];
  __syncthreads();
  if (wave == 0 && g == 0) {
    int total = 0;
    for (int ww = 0; ww < W; ++ww) total += red[ww * 64 + lane];
    int64_t n = s * 16 + r;
    if (n < w.N) store_out(y, n, y_dtype, (float)total * w.row_scale[n] * (*xscale));
  }
}

hipError_t launch_local_q8(const WeightView &w, const void *x, int x_dtype, void *y, int y_dtype,
                           void *scratch, hipStream_t st) {
  int64_t k_pad = w.k_chunks * 64;
  int8_t *xq = (int8_t *)scratch;
  float *xs = (float *)((uint8_t *)scratch + ((k_pad + 255) / 256) * 256);
  k_local_q8_quant<<<1, 256, 0, st>>>(x, x_dtype, w.K, k_pad, xq, xs);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  int waves = 4;
  while (waves < 16 && w.n_strips * waves < 4096 && w.k_chunks >= (int64_t)waves * 16) waves *= 2;
  k_local_q8_dot<<<(unsigned)w.n_strips, 64 * waves, 0, st>>>(w, xq, xs, y, y_dtype);
  return hipGetLastError();
}

}  // namespace dialq
