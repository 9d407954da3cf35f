// Shared definitions for the dialq HIP kernels (gfx950 / CDNA4 only).
//
// Resident (device) weight layout, shared by the repacker, the decode GEMV,
// the prefill GEMM and the dequantizer:
//
//   The N x K weight is cut into 16-row strips and CHUNK-wide k chunks.
//   Tile (strip s, chunk c) is TILE bytes, contiguous, tiles ordered
//   strip-major: tiles[(s * k_chunks + c) * TILE].  Inside a tile, lane l of
//   a 64-wide wavefront owns row r = l % 16 and k-group g = l / 16.  Its
//   bytes sit in 1 KB planes: byte j of lane l at (j / 16) * 1024 + 16 l +
//   j % 16 (tile_byte), so each 16-byte load instruction of a wave reads one
//   contiguous KB (a 32-byte lane at offset 32 l would spread each
//   instruction over 2 KB: 24 % slower FP8_BLOCK decode).  That lane -> (row,
//   k-group) map is the operand layout of v_mfma_*_16x16x32 (bf16/f16, B
//   operand) and of v_mfma_scale_f32_16x16x128_f8f6f4, so tiles go straight
//   from HBM into MFMA registers without an LDS round trip.
//
//   Per-format k map of a lane's bytes (k relative to the chunk start):
//     W8A16, FP8_ROW  CHUNK 64,  16 B: k = 16g + j                 (j < 16)
//     Q8_0            CHUNK 64,  16 B: bytes 0-7 : block 0, k = 8g + j
//                                       bytes 8-15: block 1, k = 32 + 8g + j
//     FP8_BLOCK       CHUNK 128, 32 B (two planes): k = 32g + j  (j < 32)
//     NVFP4, MXFP4    CHUNK 128, 16 B: k = 32g + j, two codes per byte,
//                                       low nibble first (raw byte order)
//     Q4_K            CHUNK 256, 32 B (two planes): bytes 8i..8i+7 = qs[32i + 8g + j]
//                                       (i < 4): low nibbles are sub-block 2i,
//                                       high nibbles sub-block 2i+1
//     Q6_K            CHUNK 256, 48 B in three 1 KB planes (plane p holds
//                                       bytes 16l..16l+15 for lane l):
//                                       plane h < 2: bytes 8i+j = ql[64h + 32i
//                                       + 8g + j] (i < 2); plane 2: bytes 8h+j
//                                       = qh[32h + 8g + j].  Value k = 32t + 8g
//                                       + j (t = 4h + qd) is the nibble qd >> 1
//                                       of ql byte i = qd & 1 with bits 2qd of
//                                       the qh byte on top
//   Scales that vary along k live in an aux array in the same tile order
//   (aux[(s * k_chunks + c) * AUX + ...]):
//     Q8_0   AUX 64 : u32 per row r = {f16 d(block 0), f16 d(block 1)}
//     Q4_K   AUX 256: 16 B per row = the block header {d, dmin, scales[12]}
//     Q6_K   AUX 288: 16 B per row = the i8 scales[16]; then 2 B per row = d
//     NVFP4  AUX 128: 8 E4M3 group scales per row (k/16)
//     MXFP4  AUX 64 : 4 E8M0 block scales per row (k/32)
//   Per-row scales (W8A16, FP8_ROW) are an f32 array of n_strips*16 values;
//   FP8_BLOCK keeps its [ceil(N/128), ceil(K/128)] f32 grid.
//   Padding rows / k beyond the logical size hold zero codes and zero
//   scales, so they contribute exact zeros.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dialq.h"

namespace dialq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

struct FormatGeom {
  int chunk;       // k per tile
  int lane_bytes;  // bytes per lane per tile
  int tile_bytes;  // 64 * lane_bytes
  int aux_bytes;   // per-tile k-varying scale bytes
  int k_align;     // required K multiple of the raw format
};

__host__ __device__ inline FormatGeom format_geom(int fmt) {
  switch (fmt) {
    case DIALQ_FORMAT_W8A16:
    case DIALQ_FORMAT_FP8_ROW:
      return {64, 16, 1024, 0, 8};
    case DIALQ_FORMAT_Q8_0:
      return {64, 16, 1024, 64, 32};
    case DIALQ_FORMAT_FP8_BLOCK:
      return {128, 32, 2048, 0, 8};
    case DIALQ_FORMAT_NVFP4:
      return {128, 16, 1024, 128, 16};
    case DIALQ_FORMAT_MXFP4:
      return {128, 16, 1024, 64, 32};
    case DIALQ_FORMAT_Q4_K:
      return {256, 32, 2048, 256, 256};
    case DIALQ_FORMAT_Q6_K:
      return {256, 48, 3072, 288, 256};
    default:
      return {0, 0, 0, 0, 0};
  }
}

// Offset of byte j of lane l inside a tile (the plane layout above).
__host__ __device__ inline int tile_byte(int lane, int j) { return (j >> 4) * 1024 + lane * 16 + (j & 15); }

// ---- scalar conversions (device) ------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
// RNE; a NaN keeps its upper bits and is made quiet.  Written as a select so
// that it compiles to straight-line code.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t rne = (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
  const uint32_t nan = (x >> 16) | 0x40u;
  return (uint16_t)(((x & 0x7fffffffu) > 0x7f800000u) ? nan : rne);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, v);
}

// E4M3 decode with the reference CUDA semantics (cuda_quant.rs:27-41):
// subnormals m*2^-9, the NaN codes 0x7f / 0xff decode to 0.
__device__ __forceinline__ float e4m3_to_f32(uint32_t code) {
  uint32_t e = (code >> 3) & 15u, m = code & 7u;
  float v;
  if (e == 0) {
    v = (float)m * 0.001953125f;
  } else if (e == 15 && m == 7) {
    v = 0.0f;
  } else {
    v = __uint_as_float((e + 120u) << 23) * (1.0f + (float)m * 0.125f);
  }
  return (code & 0x80u) ? -v : v;
}

// E2M1 table of quant.rs:16-18 (code 8 decodes to +0.0 there).
__device__ __forceinline__ float e2m1_to_f32(uint32_t code) {
  const float tab[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                         0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
  return tab[code & 15u];
}

__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  // 2^(e-127); e = 0 is 2^-127 (a subnormal f32), e = 255 is NaN.
  if (e == 255u) return __uint_as_float(0x7fc00000u);
  if (e == 0u) return __uint_as_float(0x00400000u);
  return __uint_as_float(e << 23);
}

// f32 -> E4M3FN, round-to-nearest-even, saturating at +-448.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  uint32_t x = __float_as_uint(f);
  uint32_t sign = (x >> 24) & 0x80u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return 0x7fu;
  float a = __uint_as_float(ax);
  if (a >= 448.0f) return sign | 0x7eu;
  int e = (int)(ax >> 23) - 127;  // floor(log2 a) for normal a
  if (e < -6) e = -6;             // subnormal quantum 2^-9
  float quantum = __uint_as_float((uint32_t)(e - 3 + 127) << 23);
  float inv_quantum = __uint_as_float((uint32_t)(3 - e + 127) << 23);
  float units = __builtin_rintf(a * inv_quantum);  // exact scaling, then RNE
  float v = units * quantum;
  if (v == 0.0f) return sign;
  uint32_t vb = __float_as_uint(v);
  int ve = (int)(vb >> 23) - 127;
  if (ve < -6) return sign | (uint32_t)(v * 512.0f);
  uint32_t mant = (vb >> 20) & 7u;
  return sign | ((uint32_t)(ve + 7) << 3) | mant;
}

// f32 -> E2M1, RNE, saturating at +-6.
__device__ __forceinline__ uint32_t f32_to_e2m1(float f) {
  uint32_t x = __float_as_uint(f);
  uint32_t sign = (x >> 28) & 8u;
  float a = __uint_as_float(x & 0x7fffffffu);
  if (!(a == a)) return 0u;
  if (a >= 6.0f) return sign | 7u;
  uint32_t ax = __float_as_uint(a);
  int e = (int)(ax >> 23) - 127;
  if (e < 0) e = 0;  // subnormal quantum 0.5
  float quantum = __uint_as_float((uint32_t)(e - 1 + 127) << 23);
  float inv_quantum = __uint_as_float((uint32_t)(1 - e + 127) << 23);
  float v = __builtin_rintf(a * inv_quantum) * quantum;
  uint32_t code;
  if (v < 0.75f) code = v == 0.0f ? 0u : 1u;
  else if (v < 1.25f) code = 2u;
  else if (v < 1.75f) code = 3u;
  else if (v < 2.5f) code = 4u;
  else if (v < 3.5f) code = 5u;
  else if (v < 5.0f) code = 6u;
  else code = 7u;
  return sign | code;
}

// Pack the high halves of two f32 (exact bf16 values) into a bf16 pair.
__device__ __forceinline__ uint32_t pack_bf16_trunc(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Store one output element of the given dtype.
__device__ __forceinline__ void store_out(void *y, int64_t idx, int dtype, float v) {
  if (dtype == DIALQ_BF16) {
    ((uint16_t *)y)[idx] = f32_to_bf16_bits(v);
  } else if (dtype == DIALQ_F16) {
    ((uint16_t *)y)[idx] = f32_to_f16_bits(v);
  } else {
    ((float *)y)[idx] = v;
  }
}

__device__ __forceinline__ float load_in(const void *x, int64_t idx, int dtype) {
  if (dtype == DIALQ_BF16) return bf16_bits_to_f32(((const uint16_t *)x)[idx]);
  if (dtype == DIALQ_F16) return f16_bits_to_f32(((const uint16_t *)x)[idx]);
  return ((const float *)x)[idx];
}

}  // namespace dialq
