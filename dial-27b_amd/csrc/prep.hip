// Load-time kernels: dense -> raw-format quantizers, raw -> resident
// repacker (and its inverse for export), and the dequantizer.
//
// The quantizers restate, on the device, the host arithmetic the reference
// runs at load time; every float operation is written out in the reference
// order and the library is built with -ffp-contract=off, so results are
// bit-identical to the reference's f32 arithmetic.
#include "common.hpp"
#include "kernels.hpp"

namespace dialq {

// ---------------------------------------------------------------------------
// dense input access
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dense_at(const void *w, int dtype, int64_t i) {
  return load_in(w, i, dtype);
}

// Rust `f32::max` fold that ignores NaN operands.
__device__ __forceinline__ float fmax_ignore_nan(float acc, float v) {
  return (v > acc) ? v : acc;
}

template <int BLOCK>
__device__ __forceinline__ float block_reduce_max(float v, float *sh) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = sh[0];
    for (int i = 1; i < BLOCK / 64; ++i) r = fmaxf(r, sh[i]);
    sh[BLOCK / 64] = r;
  }
  __syncthreads();
  float r = sh[BLOCK / 64];
  __syncthreads();
  return r;
}

// ---------------------------------------------------------------------------
// W8A16 per-row quantizer (worker_w8a16.rs:329-341)
//   amax = max |w| (NaN ignored); scale = amax > 0 ? amax/127 : 1;
//   inv = 1/scale; q = clamp(round_half_away(w*inv), -127, 127)
// One 256-thread block per row.  The max is order-independent, so the
// parallel reduction returns the same value as the sequential fold.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quant_w8a16(const void *w, int dtype, int64_t K,
                                                     int8_t *q, float *scale) {
  __shared__ float sh[8];
  int64_t row = blockIdx.x;
  float amax = 0.0f;
  for (int64_t i = threadIdx.x; i < K; i += 256)
    amax = fmax_ignore_nan(amax, fabsf(dense_at(w, dtype, row * K + i)));
  amax = block_reduce_max<256>(amax, sh);
  float s = amax > 0.0f ? amax / 127.0f : 1.0f;
  float inv = 1.0f / s;
  for (int64_t i = threadIdx.x; i < K; i += 256) {
    float v = roundf(dense_at(w, dtype, row * K + i) * inv);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    q[row * K + i] = (v == v) ? (int8_t)v : (int8_t)0;
  }
  if (threadIdx.x == 0) scale[row] = s;
}

// ---------------------------------------------------------------------------
// GGUF Q8_0 quantizer (candle BlockQ8_0::from_float, the ggml
// quantize_row_q8_0_reference algorithm): one thread per 32-value block.
// ---------------------------------------------------------------------------
__global__ void k_quant_q8_0(const void *w, int dtype, int64_t N, int64_t K, uint8_t *out) {
  int64_t nb = K / 32;
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= N * nb) return;
  int64_t row = b / nb, blk = b % nb;
  const int64_t base = row * K + blk * 32;
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = fmax_ignore_nan(amax, fabsf(dense_at(w, dtype, base + i)));
  float d = amax / 127.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint8_t *o = out + b * 34;
  uint16_t dh = f32_to_f16_bits(d);
  o[0] = (uint8_t)(dh & 0xff);
  o[1] = (uint8_t)(dh >> 8);
  for (int i = 0; i < 32; ++i) {
    float v = roundf(dense_at(w, dtype, base + i) * id);
    int iv = (v == v) ? (int)fminf(fmaxf(v, -128.0f), 127.0f) : 0;
    o[2 + i] = (uint8_t)(int8_t)iv;
  }
}

// ---------------------------------------------------------------------------
// GGUF Q4_K quantizer (candle BlockQ4K::from_float): make_qkx1_quants(15, 5)
// per 32-value sub-block, 6-bit scale/min packing, final re-quantization
// against the stored f16 scales.  One thread per 256-value super-block.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int nearest_int_away(float v) {
  if (!(v == v)) return 0;
  float r = roundf(v);
  if (r >= 2147483647.0f) return 2147483647;
  if (r <= -2147483648.0f) return (int)0x80000000;
  return (int)r;
}

__device__ void make_qkx1_quants(const float *x, float *out_scale, float *out_min) {
  const int nmax = 15, n = 32;
  uint8_t l[32];
  for (int i = 0; i < 32; ++i) l[i] = 0;
  float mn = x[0], mx = x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < mn) mn = x[i];
    if (x[i] > mx) mx = x[i];
  }
  if (mx == mn) {
    *out_scale = 0.0f;
    *out_min = 0.0f;
    return;
  }
  if (mn > 0.0f) mn = 0.0f;
  float iscale = (float)nmax / (mx - mn);
  float scale = 1.0f / iscale;
  for (int it = 0; it < 5; ++it) {
    float sumlx = 0.0f;
    int suml2 = 0;
    bool changed = false;
    for (int i = 0; i < n; ++i) {
      int li = nearest_int_away(iscale * (x[i] - mn));
      li = li < 0 ? 0 : (li > nmax ? nmax : li);
      if ((uint8_t)li != l[i]) {
        l[i] = (uint8_t)li;
        changed = true;
      }
      sumlx += (x[i] - mn) * (float)li;
      suml2 += li * li;
    }
    scale = sumlx / (float)suml2;
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)l[i];
    mn = sum / (float)n;
    if (mn > 0.0f) mn = 0.0f;
    iscale = 1.0f / scale;
    if (!changed) break;
  }
  *out_scale = scale;
  *out_min = -mn;
}

__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t *q, uint32_t &sc, uint32_t &m) {
  if (j < 4) {
    sc = q[j] & 63u;
    m = q[j + 4] & 63u;
  } else {
    sc = (q[j + 4] & 0xfu) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

__global__ __launch_bounds__(64) void k_quant_q4_k(const void *w, int dtype, int64_t N, int64_t K,
                                                   uint8_t *out) {
  int64_t nb = K / 256;
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= N * nb) return;
  int64_t row = b / nb, blk = b % nb;
  const int64_t base = row * K + blk * 256;
  float x[256];
  for (int i = 0; i < 256; ++i) x[i] = dense_at(w, dtype, base + i);
  float scl[8], mins[8];
  for (int j = 0; j < 8; ++j) make_qkx1_quants(x + 32 * j, &scl[j], &mins[j]);
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; ++j) {
    if (scl[j] > max_scale) max_scale = scl[j];
    if (mins[j] > max_min) max_min = mins[j];
  }
  float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  uint8_t scales[12];
  for (int i = 0; i < 12; ++i) scales[i] = 0;
  for (int j = 0; j < 8; ++j) {
    int lsi = nearest_int_away(inv_scale * scl[j]);
    int lmi = nearest_int_away(inv_min * mins[j]);
    uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
    uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
    if (j < 4) {
      scales[j] = ls;
      scales[j + 4] = lm;
    } else {
      scales[j + 4] = (uint8_t)((ls & 0xf) | ((lm & 0xf) << 4));
      scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
      scales[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  uint16_t dh = f32_to_f16_bits(max_scale / 63.0f);
  uint16_t mh = f32_to_f16_bits(max_min / 63.0f);
  uint8_t *o = out + b * 144;
  o[0] = (uint8_t)(dh & 0xff);
  o[1] = (uint8_t)(dh >> 8);
  o[2] = (uint8_t)(mh & 0xff);
  o[3] = (uint8_t)(mh >> 8);
  for (int i = 0; i < 12; ++i) o[4 + i] = scales[i];
  uint8_t L[256];
  for (int i = 0; i < 256; ++i) L[i] = 0;
  float dq = f16_bits_to_f32(dh), mq = f16_bits_to_f32(mh);
  for (int j = 0; j < 8; ++j) {
    uint32_t sc, m;
    q4k_scale_min(j, scales, sc, m);
    float d = dq * (float)sc;
    if (d != 0.0f) {
      float dm = mq * (float)m;
      for (int ii = 0; ii < 32; ++ii) {
        int lv = nearest_int_away((x[32 * j + ii] + dm) / d);
        L[32 * j + ii] = (uint8_t)(lv < 0 ? 0 : (lv > 15 ? 15 : lv));
      }
    }
  }
  for (int j = 0; j < 256; j += 64)
    for (int l = 0; l < 32; ++l) o[16 + j / 2 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
}

// ---------------------------------------------------------------------------
// FP8 E4M3 with one f32 scale per 128x128 block: s = amax>0 ? amax/448 : 1,
// q = e4m3_rne(w * (1/s)).  One 256-thread block per 128x128 block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quant_fp8_block(const void *w, int dtype, int64_t N,
                                                         int64_t K, uint8_t *q, float *scales) {
  __shared__ float sh[8];
  int64_t nbk = (K + 127) / 128;
  int64_t bn = blockIdx.x / nbk, bk = blockIdx.x % nbk;
  int64_t r0 = bn * 128, c0 = bk * 128;
  int64_t r1 = r0 + 128 < N ? r0 + 128 : N, c1 = c0 + 128 < K ? c0 + 128 : K;
  int64_t cols = c1 - c0, cnt = (r1 - r0) * cols;
  float amax = 0.0f;
  for (int64_t i = threadIdx.x; i < cnt; i += 256)
    amax = fmax_ignore_nan(amax, fabsf(dense_at(w, dtype, (r0 + i / cols) * K + c0 + i % cols)));
  amax = block_reduce_max<256>(amax, sh);
  float s = amax > 0.0f ? amax / 448.0f : 1.0f;
  float inv = 1.0f / s;
  for (int64_t i = threadIdx.x; i < cnt; i += 256) {
    int64_t idx = (r0 + i / cols) * K + c0 + i % cols;
    q[idx] = (uint8_t)f32_to_e4m3(dense_at(w, dtype, idx) * inv);
  }
  if (threadIdx.x == 0) scales[blockIdx.x] = s;
}

// ---------------------------------------------------------------------------
// MXFP4 (OCP MX v1.0): shared = max(floor(log2 amax) - 2, -127),
// p = e2m1_rne(v * 2^-shared).  One thread per 32-value block; also used for
// per-32 activation quantization.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int floor_log2_pos(float a) {
  uint32_t b = __float_as_uint(a);
  int e = (int)(b >> 23);
  if (e != 0) return e - 127;
  return (31 - __clz(b & 0x7fffffu)) - 149;  // subnormal
}

__device__ __forceinline__ void mx_quant32(const void *w, int dtype, int64_t base, uint8_t *packed,
                                           uint8_t *scale) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(dense_at(w, dtype, base + i)));
  int shared = amax > 0.0f ? floor_log2_pos(amax) - 2 : -127;
  shared = shared < -127 ? -127 : (shared > 127 ? 127 : shared);
  *scale = (uint8_t)(shared + 127);
  for (int i = 0; i < 16; ++i) {
    uint32_t lo = f32_to_e2m1(ldexpf(dense_at(w, dtype, base + 2 * i), -shared));
    uint32_t hi = f32_to_e2m1(ldexpf(dense_at(w, dtype, base + 2 * i + 1), -shared));
    packed[i] = (uint8_t)(lo | (hi << 4));
  }
}

__global__ void k_quant_mxfp4(const void *w, int dtype, int64_t N, int64_t K, uint8_t *packed,
                              uint8_t *scales) {
  int64_t nb = K / 32;
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= N * nb) return;
  int64_t row = b / nb, blk = b % nb;
  mx_quant32(w, dtype, row * K + blk * 32, packed + row * (K / 2) + blk * 16, scales + b);
}

// ---------------------------------------------------------------------------
// Repack / unpack.  Every resident byte either mirrors one raw byte or is
// padding (zero).  raw_index_tile / raw_index_aux give that raw byte index
// (or -1 for padding); repack gathers, unpack scatters back.
// ---------------------------------------------------------------------------
struct RepackGeom {
  int fmt;
  int64_t N, K, k_chunks;
  int chunk, lane_bytes, tile_bytes, aux_bytes;
};

// Q6_K tile byte b of (strip s, chunk c): plane b / 1024, lane (b / 16) % 64,
// byte j = b % 16 -> the ql (planes 0, 1) or qh (plane 2) byte of its
// super-block (layout in common.hpp).
__device__ __forceinline__ int64_t raw_index_q6k_tile(const RepackGeom &g, int64_t s, int64_t c, int b) {
  const int plane = b >> 10, lane = (b >> 4) & 63, j = b & 15;
  const int r = lane & 15, kg = lane >> 4;
  const int64_t n = s * 16 + r;
  if (n >= g.N || c >= g.K / 256) return -1;
  const int64_t blk = (n * (g.K / 256) + c) * 210;
  const int within = 32 * (j >> 3) + 8 * kg + (j & 7);
  return plane < 2 ? blk + 64 * plane + within : blk + 128 + within;
}

__device__ __forceinline__ int64_t raw_index_tile(const RepackGeom &g, int64_t i) {
  int64_t t = i / g.tile_bytes;
  int b = (int)(i % g.tile_bytes);
  int64_t s = t / g.k_chunks, c = t % g.k_chunks;
  if (g.fmt == DIALQ_FORMAT_Q6_K) return raw_index_q6k_tile(g, s, c, b);
  // inverse of tile_byte: plane b / 1024, lane (b / 16) % 64
  int lane = (b >> 4) & 63, j = (b >> 10) * 16 + (b & 15);
  int r = lane & 15, kg = lane >> 4;
  int64_t n = s * 16 + r;
  if (n >= g.N) return -1;
  switch (g.fmt) {
    case DIALQ_FORMAT_W8A16:
    case DIALQ_FORMAT_FP8_ROW: {
      int64_t k = c * 64 + kg * 16 + j;
      return k < g.K ? n * g.K + k : -1;
    }
    case DIALQ_FORMAT_FP8_BLOCK: {
      int64_t k = c * 128 + kg * 32 + j;
      return k < g.K ? n * g.K + k : -1;
    }
    case DIALQ_FORMAT_Q8_0: {
      int64_t blk = c * 2 + j / 8;
      if (blk >= g.K / 32) return -1;
      return (n * (g.K / 32) + blk) * 34 + 2 + kg * 8 + (j % 8);
    }
    case DIALQ_FORMAT_NVFP4:
    case DIALQ_FORMAT_MXFP4: {
      int64_t pb = c * 64 + kg * 16 + j;
      return pb < g.K / 2 ? n * (g.K / 2) + pb : -1;
    }
    case DIALQ_FORMAT_Q4_K: {
      if (c >= g.K / 256) return -1;
      return (n * (g.K / 256) + c) * 144 + 16 + 32 * (j / 8) + 8 * kg + (j % 8);
    }
  }
  return -1;
}

__device__ __forceinline__ int64_t raw_index_aux(const RepackGeom &g, int64_t i) {
  int64_t t = i / g.aux_bytes;
  int b = (int)(i % g.aux_bytes);
  int64_t s = t / g.k_chunks, c = t % g.k_chunks;
  switch (g.fmt) {
    case DIALQ_FORMAT_Q8_0: {
      int64_t n = s * 16 + b / 4;
      int64_t blk = c * 2 + (b % 4) / 2;
      if (n >= g.N || blk >= g.K / 32) return -1;
      return (n * (g.K / 32) + blk) * 34 + (b % 2);
    }
    case DIALQ_FORMAT_Q4_K: {
      int64_t n = s * 16 + b / 16;
      if (n >= g.N || c >= g.K / 256) return -1;
      return (n * (g.K / 256) + c) * 144 + (b % 16);
    }
    case DIALQ_FORMAT_Q6_K: {  // scales[16] per row, then d per row
      int64_t n = s * 16 + (b < 256 ? b / 16 : (b - 256) / 2);
      if (n >= g.N || c >= g.K / 256) return -1;
      return (n * (g.K / 256) + c) * 210 + (b < 256 ? 192 + b % 16 : 208 + (b - 256) % 2);
    }
    case DIALQ_FORMAT_NVFP4: {
      int64_t n = s * 16 + b / 8;
      int64_t grp = c * 8 + (b % 8);
      if (n >= g.N || grp >= g.K / 16) return -1;
      return n * (g.K / 16) + grp;
    }
    case DIALQ_FORMAT_MXFP4: {
      int64_t n = s * 16 + b / 4;
      int64_t blk = c * 4 + (b % 4);
      if (n >= g.N || blk >= g.K / 32) return -1;
      return n * (g.K / 32) + blk;
    }
  }
  return -1;
}

// E4M3 bytes that encode NaN decode to (signed) 0 in the reference's CUDA
// path (cuda_quant.rs:35-36,40); the resident copy stores them as the zero of
// the same sign so hardware converters can be used.
__device__ __forceinline__ uint8_t sanitize_e4m3(uint8_t v) {
  return ((v & 0x7f) == 0x7f) ? (uint8_t)(v & 0x80) : v;
}

__global__ void k_repack_tiles(RepackGeom g, const uint8_t *raw, uint8_t *tiles, int64_t total,
                               int sanitize) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t src = raw_index_tile(g, i);
    uint8_t v = src >= 0 ? raw[src] : (uint8_t)0;
    tiles[i] = sanitize ? sanitize_e4m3(v) : v;
  }
}

__global__ void k_unpack_tiles(RepackGeom g, const uint8_t *tiles, uint8_t *raw, int64_t total) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t dst = raw_index_tile(g, i);
    if (dst >= 0) raw[dst] = tiles[i];
  }
}

__global__ void k_repack_aux(RepackGeom g, const uint8_t *raw, uint8_t *aux, int64_t total,
                             int sanitize) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t src = raw_index_aux(g, i);
    uint8_t v = src >= 0 ? raw[src] : (uint8_t)0;
    aux[i] = sanitize ? sanitize_e4m3(v) : v;
  }
}

__global__ void k_unpack_aux(RepackGeom g, const uint8_t *aux, uint8_t *raw, int64_t total) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t dst = raw_index_aux(g, i);
    if (dst >= 0) raw[dst] = aux[i];
  }
}

// Per-row scales -> f32 [n_pad] (bf16 widened exactly; a single per-tensor
// scale is broadcast as quant.rs:418-425 does).
__global__ void k_row_scales(const void *src, int src_is_bf16, int64_t count, int64_t N,
                             int64_t n_pad, float *dst) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_pad) return;
  float v = 0.0f;
  if (i < N) {
    int64_t j = count == 1 ? 0 : i;
    v = src_is_bf16 ? bf16_bits_to_f32(((const uint16_t *)src)[j]) : ((const float *)src)[j];
  }
  dst[i] = v;
}

// ---------------------------------------------------------------------------
// Dequantize the resident weight to dense [N,K] (exact f32, then one RNE
// rounding for f16 / bf16 outputs).  One thread per element.
// ---------------------------------------------------------------------------
__global__ void k_dequant(DequantArgs a) {
  int64_t total = a.N * a.K;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t n = i / a.K, k = i % a.K;
    int64_t s = n / 16;
    int r = (int)(n % 16);
    int64_t c = k / a.chunk;
    int kk = (int)(k % a.chunk);
    const uint8_t *tile = a.tiles + (s * a.k_chunks + c) * a.tile_bytes;
    float v = 0.0f;
    switch (a.fmt) {
      case DIALQ_FORMAT_W8A16: {
        int kg = kk / 16, j = kk % 16;
        int8_t q = (int8_t)tile[(kg * 16 + r) * 16 + j];
        v = (float)q * a.row_scale[n];
        break;
      }
      case DIALQ_FORMAT_FP8_ROW: {
        int kg = kk / 16, j = kk % 16;
        v = e4m3_to_f32(tile[(kg * 16 + r) * 16 + j]) * a.row_scale[n];
        break;
      }
      case DIALQ_FORMAT_FP8_BLOCK: {
        int kg = kk / 32, j = kk % 32;
        v = e4m3_to_f32(tile[tile_byte(kg * 16 + r, j)]) * a.block_scale[(n / 128) * a.nbk + k / 128];
        break;
      }
      case DIALQ_FORMAT_Q8_0: {
        int h = kk / 32, within = kk % 32, kg = within / 8, j = within % 8;
        int8_t q = (int8_t)tile[(kg * 16 + r) * 16 + h * 8 + j];
        const uint8_t *aux = a.aux + (s * a.k_chunks + c) * 64 + r * 4 + h * 2;
        float d = f16_bits_to_f32((uint32_t)aux[0] | ((uint32_t)aux[1] << 8));
        v = d * (float)q;
        break;
      }
      case DIALQ_FORMAT_NVFP4:
      case DIALQ_FORMAT_MXFP4: {
        int kg = kk / 32, j = (kk % 32) / 2;
        uint8_t byte = tile[(kg * 16 + r) * 16 + j];
        uint32_t code = (kk & 1) ? (byte >> 4) : (byte & 15u);
        if (a.fmt == DIALQ_FORMAT_NVFP4) {
          float bs = e4m3_to_f32(a.aux[(s * a.k_chunks + c) * 128 + r * 8 + kk / 16]);
          v = e2m1_to_f32(code) * bs * a.global;
        } else {
          v = e2m1_to_f32(code) * e8m0_to_f32(a.aux[(s * a.k_chunks + c) * 64 + r * 4 + kk / 32]);
        }
        break;
      }
      case DIALQ_FORMAT_Q4_K: {
        int sub = kk / 32, val = kk % 32;  // sub-block, value within it
        int i4 = sub / 2, hi = sub & 1, kg = val / 8, j = val % 8;
        uint8_t byte = tile[tile_byte(kg * 16 + r, i4 * 8 + j)];
        uint32_t q = hi ? (byte >> 4) : (byte & 15u);
        const uint8_t *hdr = a.aux + (s * a.k_chunks + c) * 256 + r * 16;
        float d = f16_bits_to_f32((uint32_t)hdr[0] | ((uint32_t)hdr[1] << 8));
        float dmin = f16_bits_to_f32((uint32_t)hdr[2] | ((uint32_t)hdr[3] << 8));
        uint32_t sc, m;
        q4k_scale_min(sub, hdr + 4, sc, m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        v = d1 * (float)q - m1;
        break;
      }
      case DIALQ_FORMAT_Q6_K: {
        const int t6 = kk / 32, kg = (kk % 32) / 8, j = kk % 8;
        const int h = t6 >> 2, qd = t6 & 3;
        const uint8_t lb = tile[h * 1024 + (kg * 16 + r) * 16 + 8 * (qd & 1) + j];
        const uint8_t hb = tile[2048 + (kg * 16 + r) * 16 + 8 * h + j];
        const int q = (int)(((lb >> (4 * (qd >> 1))) & 15u) | (((hb >> (2 * qd)) & 3u) << 4));
        const uint8_t *aux = a.aux + (s * a.k_chunks + c) * 288;
        const float d = f16_bits_to_f32((uint32_t)aux[256 + 2 * r] | ((uint32_t)aux[257 + 2 * r] << 8));
        const float sc = (float)(int8_t)aux[r * 16 + kk / 16];
        v = d * sc * (float)(q - 32);  // exact: 11 + 8 + 6 significant bits
        break;
      }
    }
    store_out(a.out, i, a.out_dtype, v);
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline unsigned grid_for(int64_t total, int threads, int64_t cap = 65536) {
  int64_t g = (total + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

hipError_t launch_quantize(int fmt, const void *dense, int dtype, int64_t N, int64_t K,
                           void *raw_w, void *raw_s, hipStream_t st) {
  switch (fmt) {
    case DIALQ_FORMAT_W8A16:
      k_quant_w8a16<<<(unsigned)N, 256, 0, st>>>(dense, dtype, K, (int8_t *)raw_w, (float *)raw_s);
      break;
    case DIALQ_FORMAT_Q8_0: {
      int64_t nb = N * (K / 32);
      k_quant_q8_0<<<grid_for(nb, 256, 1 << 30), 256, 0, st>>>(dense, dtype, N, K, (uint8_t *)raw_w);
      break;
    }
    case DIALQ_FORMAT_Q4_K: {
      int64_t nb = N * (K / 256);
      k_quant_q4_k<<<grid_for(nb, 64, 1 << 30), 64, 0, st>>>(dense, dtype, N, K, (uint8_t *)raw_w);
      break;
    }
    case DIALQ_FORMAT_FP8_BLOCK: {
      int64_t blocks = ((N + 127) / 128) * ((K + 127) / 128);
      k_quant_fp8_block<<<(unsigned)blocks, 256, 0, st>>>(dense, dtype, N, K, (uint8_t *)raw_w,
                                                          (float *)raw_s);
      break;
    }
    case DIALQ_FORMAT_MXFP4: {
      int64_t nb = N * (K / 32);
      k_quant_mxfp4<<<grid_for(nb, 256, 1 << 30), 256, 0, st>>>(dense, dtype, N, K,
                                                                 (uint8_t *)raw_w, (uint8_t *)raw_s);
      break;
    }
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static RepackGeom make_geom(int fmt, int64_t N, int64_t K) {
  FormatGeom fg = format_geom(fmt);
  RepackGeom g;
  g.fmt = fmt;
  g.N = N;
  g.K = K;
  g.k_chunks = (K + fg.chunk - 1) / fg.chunk;
  g.chunk = fg.chunk;
  g.lane_bytes = fg.lane_bytes;
  g.tile_bytes = fg.tile_bytes;
  g.aux_bytes = fg.aux_bytes;
  return g;
}

hipError_t launch_repack(int fmt, int64_t N, int64_t K, const void *raw_w, const void *raw_s,
                         int scale_is_bf16, int64_t scale_count, uint8_t *tiles, uint8_t *aux,
                         float *row_scale, float *block_scale, hipStream_t st) {
  RepackGeom g = make_geom(fmt, N, K);
  int64_t strips = (N + 15) / 16;
  int64_t t_total = strips * g.k_chunks * g.tile_bytes;
  int sanitize = (fmt == DIALQ_FORMAT_FP8_ROW || fmt == DIALQ_FORMAT_FP8_BLOCK) ? 1 : 0;
  k_repack_tiles<<<grid_for(t_total, 256), 256, 0, st>>>(g, (const uint8_t *)raw_w, tiles, t_total,
                                                         sanitize);
  if (g.aux_bytes > 0) {
    int64_t a_total = strips * g.k_chunks * g.aux_bytes;
    // Q8_0 / Q4_K / Q6_K scales live inside the raw blocks; NVFP4 / MXFP4 in `raw_s`.
    const uint8_t *src = (fmt == DIALQ_FORMAT_Q8_0 || fmt == DIALQ_FORMAT_Q4_K || fmt == DIALQ_FORMAT_Q6_K)
                             ? (const uint8_t *)raw_w
                             : (const uint8_t *)raw_s;
    k_repack_aux<<<grid_for(a_total, 256), 256, 0, st>>>(g, src, aux, a_total,
                                                         fmt == DIALQ_FORMAT_NVFP4 ? 1 : 0);
  }
  if (fmt == DIALQ_FORMAT_W8A16 || fmt == DIALQ_FORMAT_FP8_ROW) {
    int64_t n_pad = strips * 16;
    k_row_scales<<<grid_for(n_pad, 256, 1 << 30), 256, 0, st>>>(raw_s, scale_is_bf16, scale_count, N,
                                                                n_pad, row_scale);
  } else if (fmt == DIALQ_FORMAT_FP8_BLOCK) {
    int64_t cnt = ((N + 127) / 128) * ((K + 127) / 128);
    hipError_t e = hipMemcpyAsync(block_scale, raw_s, cnt * sizeof(float), hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return e;
  }
  return hipGetLastError();
}

hipError_t launch_unpack(int fmt, int64_t N, int64_t K, const uint8_t *tiles, const uint8_t *aux,
                         void *raw_w, void *raw_s, hipStream_t st) {
  RepackGeom g = make_geom(fmt, N, K);
  int64_t strips = (N + 15) / 16;
  int64_t t_total = strips * g.k_chunks * g.tile_bytes;
  k_unpack_tiles<<<grid_for(t_total, 256), 256, 0, st>>>(g, tiles, (uint8_t *)raw_w, t_total);
  if (g.aux_bytes > 0) {
    int64_t a_total = strips * g.k_chunks * g.aux_bytes;
    uint8_t *dst = (fmt == DIALQ_FORMAT_Q8_0 || fmt == DIALQ_FORMAT_Q4_K || fmt == DIALQ_FORMAT_Q6_K)
                       ? (uint8_t *)raw_w
                       : (uint8_t *)raw_s;
    k_unpack_aux<<<grid_for(a_total, 256), 256, 0, st>>>(g, aux, dst, a_total);
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const DequantArgs &a, hipStream_t st) {
  k_dequant<<<grid_for(a.N * a.K, 256), 256, 0, st>>>(a);
  return hipGetLastError();
}

// Activation quantizers of the native prefill.
//   FP8 (per token): s = amax > 0 ? amax / 448 : 1, q = e4m3_rne(x * (1/s)).
//   MXFP4 (per 32-block): the E8M0 scale and E2M1 codes of mx_quant32.
// Both write [M, k_pad] (FP8 bytes / MXFP4 nibbles) with a zero tail past K.
// The weight formats make K a multiple of 8 (FP8_BLOCK) or 32 (MXFP4) and the
// C ABI makes x 16-byte aligned, so 8 activations come with one 16-byte (f16 /
// bf16) or 32-byte (f32) load and the codes leave 8 or 32 at a time.
template <int ACT>
__device__ __forceinline__ void load8(const void *x, int64_t e, float (&v)[8]) {
  if constexpr (ACT == DIALQ_F32) {
    const float4 a = *(const float4 *)((const float *)x + e), b = *(const float4 *)((const float *)x + e + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 u = *(const uint4 *)((const uint16_t *)x + e);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (ACT == DIALQ_BF16) {
        v[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
        v[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
      } else {
        v[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
        v[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
      }
    }
  }
}

// FP8: one 256-thread block per token.  G > 0 keeps the row's 8-value
// groups in registers (K <= 2048 * G), so the row is read once; G == 0 reads
// it twice (amax pass, then conversion).
// Four E4M3 codes, RNE, by the hardware converter.  For finite inputs of
// magnitude below 464 it agrees with f32_to_e4m3 (x / s never exceeds 448 by
// more than rounding); NaN takes f32_to_e4m3's code 0x7f.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  if (a != a || b != b || c != c || d != d)
    return f32_to_e4m3(a) | (f32_to_e4m3(b) << 8) | (f32_to_e4m3(c) << 16) | (f32_to_e4m3(d) << 24);
  uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)r, true);
}

template <int ACT, int G>
__global__ __launch_bounds__(256) void k_act_fp8_v8(const void *x, int64_t K, uint8_t *q, float *scale,
                                                    int64_t k_pad) {
  __shared__ float sh[8];
  const int64_t row = blockIdx.x, g8 = K / 8;
  float v[G > 0 ? G : 1][8];
  float amax = 0.0f;
  if constexpr (G > 0) {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int64_t g = threadIdx.x + 256 * i;
      if (g < g8) load8<ACT>(x, row * K + 8 * g, v[i]);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
    }
  } else {
    for (int64_t g = threadIdx.x; g < g8; g += 256) {
      load8<ACT>(x, row * K + 8 * g, v[0]);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[0][e]));
    }
  }
  amax = block_reduce_max<256>(amax, sh);
  const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
  const float inv = 1.0f / s;
  auto put = [&](int64_t g, const float (&u)[8]) {
    float t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = u[e] * inv;
    const uint2 out = {e4m3x4(t[0], t[1], t[2], t[3]), e4m3x4(t[4], t[5], t[6], t[7])};
    *(uint2 *)(q + row * k_pad + 8 * g) = out;
  };
  if constexpr (G > 0) {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int64_t g = threadIdx.x + 256 * i;
      if (g < g8) put(g, v[i]);
    }
  } else {
    for (int64_t g = threadIdx.x; g < g8; g += 256) {
      load8<ACT>(x, row * K + 8 * g, v[0]);
      put(g, v[0]);
    }
  }
  for (int64_t g = g8 + threadIdx.x; g < k_pad / 8; g += 256) *(uint2 *)(q + row * k_pad + 8 * g) = uint2{0u, 0u};
  if (threadIdx.x == 0) scale[row] = s;
}

// MXFP4: four lanes per 32-block, 8 activations each; the block's amax is
// combined across the four lanes with two butterfly shuffles.
template <int ACT>
__global__ __launch_bounds__(256) void k_act_mxfp4_v8(const void *x, int64_t M, int64_t K, int64_t k_pad,
                                                      uint8_t *packed, uint8_t *scales) {
  const int64_t per_row = k_pad / 8;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * per_row) return;  // M * per_row is a multiple of 4: whole blocks leave together
  const int64_t row = t / per_row, g = t % per_row;
  float v[8];
  if (8 * g < K) load8<ACT>(x, row * K + 8 * g, v);
  else
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.0f;
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  int shared = amax > 0.0f ? floor_log2_pos(amax) - 2 : -127;
  shared = shared < -127 ? -127 : (shared > 127 ? 127 : shared);
  bool nan = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) nan |= v[e] != v[e];
  uint32_t codes = 0;
  if (shared >= -126 && !nan) {
    // hardware E2M1 conversion of v / 2^shared (RNE, saturating at 6); the
    // scale is a normal f32 here, and NaN inputs take the path below
    const float sc = __builtin_bit_cast(float, (uint32_t)(shared + 127) << 23);
    codes = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(codes, v[0], v[1], sc, 0);
    codes = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(codes, v[2], v[3], sc, 1);
    codes = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(codes, v[4], v[5], sc, 2);
    codes = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(codes, v[6], v[7], sc, 3);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) codes |= f32_to_e2m1(ldexpf(v[e], -shared)) << (4 * e);
  }
  *(uint32_t *)(packed + row * (k_pad / 2) + 4 * g) = codes;
  if ((g & 3) == 0) scales[row * (k_pad / 32) + g / 4] = (uint8_t)(shared + 127);
}

template <int ACT>
static void act_fp8_dispatch(const void *x, int64_t M, int64_t K, int64_t k_pad, uint8_t *q, float *scale,
                             hipStream_t st) {
  const int64_t g = (K + 2047) / 2048;
  if (g <= 1) k_act_fp8_v8<ACT, 1><<<(unsigned)M, 256, 0, st>>>(x, K, q, scale, k_pad);
  else if (g <= 2) k_act_fp8_v8<ACT, 2><<<(unsigned)M, 256, 0, st>>>(x, K, q, scale, k_pad);
  else if (g <= 3) k_act_fp8_v8<ACT, 3><<<(unsigned)M, 256, 0, st>>>(x, K, q, scale, k_pad);
  else if (g <= 4) k_act_fp8_v8<ACT, 4><<<(unsigned)M, 256, 0, st>>>(x, K, q, scale, k_pad);
  else if (g <= 6) k_act_fp8_v8<ACT, 6><<<(unsigned)M, 256, 0, st>>>(x, K, q, scale, k_pad);
  else if (g <= 9) k_act_fp8_v8<ACT, 9><<<(unsigned)M, 256, 0, st>>>(x, K, q, scale, k_pad);
  else k_act_fp8_v8<ACT, 0><<<(unsigned)M, 256, 0, st>>>(x, K, q, scale, k_pad);
}

// bf16 activations as f16 for the GGUF (Q4_K, Q8_0) prefill's f16 MFMA kernel.  Row m is
// scaled by 2^-e_m, e_m the exponent that puts max|x_m| in [2^14, 2^15)
// (clamped to [-120, 127]), and rounded to f16: exact for every value that
// lands in f16's normal range, i.e. down to 2^-29 of the row's maximum (bf16
// carries 8 significant bits); smaller ones keep what f16 subnormals hold
// (absolute error <= 2^-25 * 2^e_m).  rs[m] = 2^e_m multiplies the row's
// outputs.  A row of zeros, or one holding an infinity, keeps e_m = 0; NaN
// stays NaN.
__global__ __launch_bounds__(256) void k_x_f16_rows(const uint16_t *x, int64_t K, uint16_t *xh, float *rs) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const uint16_t *row = x + m * K;
  float mx = 0.0f;
  for (int64_t k = (int64_t)threadIdx.x * 8; k < K; k += 256 * 8) {
    const u32x4 v = *(const u32x4 *)(row + k);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      mx = fmaxf(mx, fmaxf(fabsf(bf16_bits_to_f32(v[i] & 0xffffu)), fabsf(bf16_bits_to_f32(v[i] >> 16))));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.0f && mx <= 3.4028235e38f) {
    int ex;
    (void)__builtin_frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
    e = ex - 15;
    e = e < -120 ? -120 : (e > 127 ? 127 : e);
  }
  const float sc = __builtin_ldexpf(1.0f, -e);
  uint16_t *out = xh + m * K;
  for (int64_t k = (int64_t)threadIdx.x * 8; k < K; k += 256 * 8) {
    const u32x4 v = *(const u32x4 *)(row + k);
    u32x4 h;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      h[i] = (uint32_t)f32_to_f16_bits(bf16_bits_to_f32(v[i] & 0xffffu) * sc) |
             ((uint32_t)f32_to_f16_bits(bf16_bits_to_f32(v[i] >> 16) * sc) << 16);
    *(u32x4 *)(out + k) = h;
  }
  if (threadIdx.x == 0) rs[m] = __builtin_ldexpf(1.0f, e);
}

hipError_t launch_x_f16_rows(const void *x, int64_t M, int64_t K, uint16_t *xh, float *rs, hipStream_t st) {
  if (K % 8 != 0 || ((uintptr_t)x & 15u) != 0 || ((uintptr_t)xh & 15u) != 0 || M > 0x7fffffffLL)
    return hipErrorInvalidValue;
  if (M > 0) k_x_f16_rows<<<(unsigned)M, 256, 0, st>>>((const uint16_t *)x, K, xh, rs);
  return hipGetLastError();
}

hipError_t launch_act_fp8(const void *x, int dtype, int64_t M, int64_t K, int64_t k_pad, uint8_t *q,
                          float *scale, hipStream_t st) {
  if (K % 8 != 0 || k_pad % 8 != 0 || ((uintptr_t)x & 15u) != 0 || ((uintptr_t)q & 7u) != 0)
    return hipErrorInvalidValue;
  if (dtype == DIALQ_BF16) act_fp8_dispatch<DIALQ_BF16>(x, M, K, k_pad, q, scale, st);
  else if (dtype == DIALQ_F16) act_fp8_dispatch<DIALQ_F16>(x, M, K, k_pad, q, scale, st);
  else act_fp8_dispatch<DIALQ_F32>(x, M, K, k_pad, q, scale, st);
  return hipGetLastError();
}

hipError_t launch_act_mxfp4(const void *x, int dtype, int64_t M, int64_t K, int64_t k_pad,
                            uint8_t *packed, uint8_t *scales, hipStream_t st) {
  if (K % 32 != 0 || k_pad % 32 != 0 || ((uintptr_t)x & 15u) != 0 || ((uintptr_t)packed & 3u) != 0)
    return hipErrorInvalidValue;
  const dim3 grid = grid_for(M * (k_pad / 8), 256, 1 << 30);
  if (dtype == DIALQ_BF16) k_act_mxfp4_v8<DIALQ_BF16><<<grid, 256, 0, st>>>(x, M, K, k_pad, packed, scales);
  else if (dtype == DIALQ_F16) k_act_mxfp4_v8<DIALQ_F16><<<grid, 256, 0, st>>>(x, M, K, k_pad, packed, scales);
  else k_act_mxfp4_v8<DIALQ_F32><<<grid, 256, 0, st>>>(x, M, K, k_pad, packed, scales);
  return hipGetLastError();
}

}  // namespace dialq
