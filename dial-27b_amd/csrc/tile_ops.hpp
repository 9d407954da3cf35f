// Per-format tile operations shared by the decode GEMV and the prefill GEMM.
//
// A resident tile (see common.hpp) is loaded by one wavefront, one 16- or
// 32-byte piece per lane, and unpacked in registers into exact bf16 B
// operands of v_mfma_f32_16x16x32_bf16 (BOps), together with the per-lane
// scale factors of the lane's weight row n = lane % 16.  bops_mac then
// multiply-accumulates those operands against NX activation operands
// (XOp, lane l = row m = l % 16 of x) into the f32x4 accumulator
// C[m = 4(l/16)+i][n = l%16].
//
// Exactness: every weight code is converted to an exact bf16 value (int8,
// E4M3, E2M1 times an E4M3 or E8M0 scale, Q4_K / Q6_K codes offset by 128), so
// the products are exact and only the fp32 accumulation order differs from
// the oracle.  Scales that cannot be folded exactly into a bf16 operand
// (Q8_0's f16 d, Q4_K's d*sc and dmin*m, Q6_K's d*sc, FP8_BLOCK's f32 block scale) are
// applied to the f32 partial product of their own k block.
#pragma once

#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace dialq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

// ---- activation operands ----------------------------------------------------
// ACT = DIALQ_BF16: one bf16 part.  DIALQ_F16 / DIALQ_F32: bf16 hi + lo parts
// (exact for f16, 2^-17 relative for f32), two MFMAs per product.
// kActF16N: f16 activations taken as they are by f16 MFMAs, against weight
// operands built in f16 (the prefill GEMMs; every code except MXFP4's
// E8M0-scaled values is exact in f16).
constexpr int kActF16N = 16;

template <int ACT>
struct XOp {
  u32x4 hi;
  u32x4 lo;
};
template <>
struct XOp<DIALQ_BF16> {
  u32x4 hi;
};
template <>
struct XOp<kActF16N> {
  u32x4 hi;
};

template <int ACT>
struct ActTraits {
  static constexpr int PARTS = (ACT == DIALQ_BF16 || ACT == kActF16N) ? 1 : 2;
  static constexpr int BYTES = (ACT == DIALQ_F32) ? 4 : 2;
  static constexpr bool F16OP = ACT == kActF16N;  // weight operands in f16
};

__device__ __forceinline__ void split_f32(float v, uint32_t &h, uint32_t &l) {
  uint32_t b = __float_as_uint(v);
  h = b >> 16;  // truncation is the exact high part
  l = f32_to_bf16_bits(v - __uint_as_float(b & 0xffff0000u));
}

// 8 consecutive activations starting at element `idx` -> operand parts.
template <int ACT>
__device__ __forceinline__ XOp<ACT> x8_from_global(const void *x, int64_t idx) {
  XOp<ACT> r;
  if constexpr (ACT == DIALQ_BF16) {
    r.hi = *(const u32x4 *)((const uint16_t *)x + idx);
  } else if constexpr (ACT == DIALQ_F16) {
    u32x4 raw = *(const u32x4 *)((const uint16_t *)x + idx);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t h0, l0, h1, l1;
      split_f32(f16_bits_to_f32(raw[i] & 0xffffu), h0, l0);
      split_f32(f16_bits_to_f32(raw[i] >> 16), h1, l1);
      r.hi[i] = h0 | (h1 << 16);
      r.lo[i] = l0 | (l1 << 16);
    }
  } else {
    u32x8 raw = *(const u32x8 *)((const float *)x + idx);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t h0, l0, h1, l1;
      split_f32(__uint_as_float(raw[2 * i]), h0, l0);
      split_f32(__uint_as_float(raw[2 * i + 1]), h1, l1);
      r.hi[i] = h0 | (h1 << 16);
      r.lo[i] = l0 | (l1 << 16);
    }
  }
  return r;
}

template <int ACT>
__device__ __forceinline__ XOp<ACT> load_x8(const void *x, int64_t m, int64_t k, int64_t M,
                                            int64_t K) {
  if (m < M && k < K) return x8_from_global<ACT>(x, m * K + k);
  XOp<ACT> r;
  r.hi = (u32x4){0, 0, 0, 0};
  if constexpr (ACT != DIALQ_BF16) r.lo = (u32x4){0, 0, 0, 0};
  return r;
}

// Unconditional variant: always loads (from a clamped, valid address) and
// zeroes the result for rows >= M or k >= K, so no branch surrounds the load.
template <int ACT>
__device__ __forceinline__ XOp<ACT> load_x8_clamped(const void *x, int64_t m, int64_t k, int64_t M,
                                                    int64_t K) {
  const bool ok = (m < M) && (k < K);
  const int64_t mc = m < M ? m : M - 1, kcl = k < K ? k : K - 8;
  XOp<ACT> r = x8_from_global<ACT>(x, mc * K + kcl);
  const u32x4 z = {0, 0, 0, 0};
  r.hi = ok ? r.hi : z;
  if constexpr (ACT != DIALQ_BF16) r.lo = ok ? r.lo : z;
  return r;
}

template <int ACT>
__device__ __forceinline__ f32x4 mfma_x(const XOp<ACT> &a, u32x4 b, f32x4 c) {
  if constexpr (ACT == kActF16N) {
    return mfma_f16(a.hi, b, c);
  } else {
    c = mfma_bf16(a.hi, b, c);
    if constexpr (ACT != DIALQ_BF16) c = mfma_bf16(a.lo, b, c);
    return c;
  }
}

// One MFMA on a one-part activation operand and a weight operand of the
// same type.
template <int ACT>
__device__ __forceinline__ f32x4 mfma_op(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (ACT == kActF16N) return mfma_f16(a, b, c);
  else return mfma_bf16(a, b, c);
}

// ---- buffer loads -----------------------------------------------------------
// Raw buffer loads through a resource descriptor whose size is the valid byte
// range: an offset at or past the end returns zeros without a memory access,
// so masked-off lanes, rows >= M and chunks past a segment need no branch.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;  // offset guaranteed out of range

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bload1(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}
// Streaming variants (cache policy nt) for data read once per launch: the
// resident weight tiles and their scales.
constexpr int kNT = 2;
// Device-coherent read (cache policy sc1) of data other workgroups wrote
// with agent-scope stores.
constexpr int kSC1 = 16;
__device__ __forceinline__ u32x4 sload16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kNT));
}
__device__ __forceinline__ uint32_t sload4(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kNT);
}
__device__ __forceinline__ uint32_t sload2(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, kNT);
}
__device__ __forceinline__ uint32_t sload1(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, kNT);
}

// Raw activation bytes for one 8-element operand (16 B for bf16/f16, 32 B
// for f32), converted to operand parts at use time.
template <int ACT>
struct XRaw {
  u32x4 a;
  u32x4 b;  // f32 only
};
template <int ACT>
__device__ __forceinline__ XRaw<ACT> xraw_load(rsrc_t r, uint32_t off) {
  XRaw<ACT> v;
  v.a = bload16(r, off);
  if constexpr (ACT == DIALQ_F32) v.b = bload16(r, off + 16);
  return v;
}
template <int ACT>
__device__ __forceinline__ XOp<ACT> xraw_to_op(const XRaw<ACT> &v) {
  XOp<ACT> o;
  if constexpr (ACT == DIALQ_BF16 || ACT == kActF16N) {
    o.hi = v.a;
  } else if constexpr (ACT == DIALQ_F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t h0, l0, h1, l1;
      split_f32(f16_bits_to_f32(v.a[i] & 0xffffu), h0, l0);
      split_f32(f16_bits_to_f32(v.a[i] >> 16), h1, l1);
      o.hi[i] = h0 | (h1 << 16);
      o.lo[i] = l0 | (l1 << 16);
    }
  } else {
    const uint32_t f[8] = {v.a[0], v.a[1], v.a[2], v.a[3], v.b[0], v.b[1], v.b[2], v.b[3]};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t h0, l0, h1, l1;
      split_f32(__uint_as_float(f[2 * i]), h0, l0);
      split_f32(__uint_as_float(f[2 * i + 1]), h1, l1);
      o.hi[i] = h0 | (h1 << 16);
      o.lo[i] = l0 | (l1 << 16);
    }
  }
  return o;
}

// ---- weight code -> exact bf16 --------------------------------------------
__device__ __forceinline__ u32x4 i8x8_to_bf16(uint32_t d0, uint32_t d1) {
  u32x4 r;
  uint32_t d[2] = {d0, d1};
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    float f0 = (float)((int32_t)(d[w] << 24) >> 24);
    float f1 = (float)((int32_t)(d[w] << 16) >> 24);
    float f2 = (float)((int32_t)(d[w] << 8) >> 24);
    float f3 = (float)((int32_t)d[w] >> 24);
    r[2 * w] = pack_bf16_trunc(f0, f1);
    r[2 * w + 1] = pack_bf16_trunc(f2, f3);
  }
  return r;
}

__device__ __forceinline__ u32x4 e4m3x8_to_bf16(uint32_t d0, uint32_t d1) {
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
  r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
  r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
  return r;
}

// 8 E2M1 codes (low nibble first) times an f32 scale whose product with
// any E2M1 value is exact in bf16 (an E4M3 or E8M0 value): decode to f32,
// multiply (exact), keep the high half.
__device__ __forceinline__ u32x4 e2m1x8_to_bf16(uint32_t d, float scale) {
  u32x4 r;
  f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0);
  f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1);
  f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2);
  f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3);
  r[0] = pack_bf16_trunc(v0[0] * scale, v0[1] * scale);
  r[1] = pack_bf16_trunc(v1[0] * scale, v1[1] * scale);
  r[2] = pack_bf16_trunc(v2[0] * scale, v2[1] * scale);
  r[3] = pack_bf16_trunc(v3[0] * scale, v3[1] * scale);
  return r;
}

// 8 E2M1 codes times a power-of-two scale (an E8M0 value) -> bf16, one
// v_cvt_scalef32_pk_bf16_fp4 per pair (exact: 2 significant bits).
__device__ __forceinline__ u32x4 e2m1x8_pow2_to_bf16(uint32_t d, float scale) {
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0));
  r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2));
  r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3));
  return r;
}

// ---- weight code -> exact f16 (kActF16N) ------------------------------------
__device__ __forceinline__ uint32_t pack_f16_exact(float lo, float hi) {
  // both values are exact in f16, so rounding toward zero changes nothing
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

__device__ __forceinline__ u32x4 i8x8_to_f16(uint32_t d0, uint32_t d1) {
  u32x4 r;
  uint32_t d[2] = {d0, d1};
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    float f0 = (float)((int32_t)(d[w] << 24) >> 24);
    float f1 = (float)((int32_t)(d[w] << 16) >> 24);
    float f2 = (float)((int32_t)(d[w] << 8) >> 24);
    float f3 = (float)((int32_t)d[w] >> 24);
    r[2 * w] = pack_f16_exact(f0, f1);
    r[2 * w + 1] = pack_f16_exact(f2, f3);
  }
  return r;
}

__device__ __forceinline__ u32x4 e4m3x8_to_f16(uint32_t d0, uint32_t d1) {
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, false));
  r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d0, 1.0f, true));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, false));
  r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(d1, 1.0f, true));
  return r;
}

// E2M1 times an E4M3 scale: at most 5 significant bits between 2^-10 and
// 2688, exact in f16.
__device__ __forceinline__ u32x4 e2m1x8_to_f16(uint32_t d, float scale) {
  u32x4 r;
  f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0);
  f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1);
  f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2);
  f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3);
  r[0] = pack_f16_exact(v0[0] * scale, v0[1] * scale);
  r[1] = pack_f16_exact(v1[0] * scale, v1[1] * scale);
  r[2] = pack_f16_exact(v2[0] * scale, v2[1] * scale);
  r[3] = pack_f16_exact(v3[0] * scale, v3[1] * scale);
  return r;
}

// Byte-code pairs with a constant high byte: 0x43 gives bf16 (128 + q),
// 0x64 gives f16 (1024 + q), q < 256.
template <bool F16>
__device__ __forceinline__ u32x4 bytes8_off(uint32_t a, uint32_t b) {
  constexpr uint32_t HI = F16 ? 0x64646464u : 0x43434343u;
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(HI, a, 0x04010400u);
  r[1] = __builtin_amdgcn_perm(HI, a, 0x04030402u);
  r[2] = __builtin_amdgcn_perm(HI, b, 0x04010400u);
  r[3] = __builtin_amdgcn_perm(HI, b, 0x04030402u);
  return r;
}

// 8 nibbles (shift 0 = low, 4 = high) of two dwords -> bf16 (128 + q), or
// f16 (1024 + q).
template <bool F16 = false>
__device__ __forceinline__ u32x4 nib8_off(uint32_t d0, uint32_t d1, int shift) {
  return bytes8_off<F16>((d0 >> shift) & 0x0f0f0f0fu, (d1 >> shift) & 0x0f0f0f0fu);
}
__device__ __forceinline__ u32x4 nib8_to_bf16_off128(uint32_t d0, uint32_t d1, int shift) {
  return nib8_off<false>(d0, d1, shift);
}

// Q6_K slice t of a lane (8 values k = 32t + 8g + j): 6-bit codes q from the
// ql plane of half t/4 (bytes 8(qd&1).., nibble qd>>1) and the qh plane
// (bytes 8h.., bits 2qd), qd = t%4, as bf16 (128 + q) or f16 (1024 + q).
template <bool F16 = false>
__device__ __forceinline__ u32x4 q6x8_off(const u32x4 &ql, const u32x4 &qh, int t) {
  const int h = t >> 2, qd = t & 3, i = qd & 1;
  const int ns = 4 * (qd >> 1), hs = 2 * qd;
  uint32_t q[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const uint32_t hb = hs <= 4 ? (qh[2 * h + w] << (4 - hs)) : (qh[2 * h + w] >> (hs - 4));
    q[w] = ((ql[2 * i + w] >> ns) & 0x0f0f0f0fu) | (hb & 0x30303030u);
  }
  return bytes8_off<F16>(q[0], q[1]);
}
__device__ __forceinline__ u32x4 q6x8_to_bf16_off128(const u32x4 &ql, const u32x4 &qh, int t) {
  return q6x8_off<false>(ql, qh, t);
}

// Signed byte i of a dword as f32.
__device__ __forceinline__ float sbyte_f32(uint32_t d, int i) {
  return (float)((int32_t)(d << (24 - 8 * i)) >> 24);
}

// ---- format traits -----------------------------------------------------------
// CHUNK: k per tile; LANE: bytes per lane; NX: MFMA k-slices per tile;
// xk(t, g): k offset (within the chunk) of slice t for lane group g.
template <int FMT>
struct FmtTraits;
template <>
struct FmtTraits<DIALQ_FORMAT_W8A16> {
  static constexpr int CHUNK = 64, LANE = 16, NX = 2;
  __device__ static int xk(int t, int g) { return 16 * g + 8 * t; }
};
template <>
struct FmtTraits<DIALQ_FORMAT_FP8_ROW> {
  static constexpr int CHUNK = 64, LANE = 16, NX = 2;
  __device__ static int xk(int t, int g) { return 16 * g + 8 * t; }
};
template <>
struct FmtTraits<DIALQ_FORMAT_Q8_0> {
  static constexpr int CHUNK = 64, LANE = 16, NX = 2;
  __device__ static int xk(int t, int g) { return 32 * t + 8 * g; }
};
template <>
struct FmtTraits<DIALQ_FORMAT_FP8_BLOCK> {
  static constexpr int CHUNK = 128, LANE = 32, NX = 4;
  __device__ static int xk(int t, int g) { return 32 * g + 8 * t; }
};
template <>
struct FmtTraits<DIALQ_FORMAT_NVFP4> {
  static constexpr int CHUNK = 128, LANE = 16, NX = 4;
  __device__ static int xk(int t, int g) { return 32 * g + 8 * t; }
};
template <>
struct FmtTraits<DIALQ_FORMAT_MXFP4> {
  static constexpr int CHUNK = 128, LANE = 16, NX = 4;
  __device__ static int xk(int t, int g) { return 32 * g + 8 * t; }
};
template <>
struct FmtTraits<DIALQ_FORMAT_Q4_K> {
  static constexpr int CHUNK = 256, LANE = 32, NX = 8;
  __device__ static int xk(int t, int g) { return 32 * t + 8 * g; }
};
template <>
struct FmtTraits<DIALQ_FORMAT_Q6_K> {  // LANE: 16 B in each of three 1 KB planes
  static constexpr int CHUNK = 256, LANE = 48, NX = 8;
  __device__ static int xk(int t, int g) { return 32 * t + 8 * g; }
};

struct RawTile {
  u32x4 a;
  u32x4 b;       // second 16 bytes (LANE == 32 formats)
  uint32_t s0;   // per-lane scale bits: Q8_0 d pair, NVFP4 E4M3 pair,
                 // MXFP4 E8M0, FP8_BLOCK f32 block scale
  u32x4 hdr;     // Q4_K super-block header {d, dmin, scales[12]}; Q6_K qh plane
  u32x4 sc;      // Q6_K i8 scales[16] of the lane's row (d in s0)
};

template <int FMT>
__device__ __forceinline__ RawTile load_tile(const uint8_t *tiles, int64_t tile_idx, int lane) {
  constexpr int LANE = FmtTraits<FMT>::LANE;
  const uint8_t *p = tiles + tile_idx * (64 * LANE) + lane * 16;  // plane 0 (and plane 1 at +1 KB)
  RawTile r;
  r.a = __builtin_nontemporal_load((const u32x4 *)p);
  if constexpr (LANE == 32)
    r.b = __builtin_nontemporal_load((const u32x4 *)(p + 1024));
  else
    r.b = (u32x4){0, 0, 0, 0};
  return r;
}

// B operands of one tile plus the lane row's scale factors.
template <int FMT>
struct BOps {
  u32x4 b[FmtTraits<FMT>::NX];
  float s1[FmtTraits<FMT>::NX];  // Q8_0: d per block; Q4_K: d*sc; FP8_BLOCK: s;
                                 // Q6_K: d*sc of the slice's upper sub-block
  float s2[FmtTraits<FMT>::NX];  // Q4_K: 128*d*sc + dmin*m; Q6_K: d*(sc_lo - sc_hi)
};

// `t` must carry the lane row's scales (gemv tile_fill / gemm gemm_tile).
// F16: operands in f16 for kActF16N (the k-quant codes offset by 1024
// instead of 128).
template <int FMT, bool F16 = false>
__device__ __forceinline__ BOps<FMT> make_bops(const RawTile &t) {
  static_assert(!F16 || FMT != DIALQ_FORMAT_MXFP4, "E8M0-scaled codes leave the f16 range");
  BOps<FMT> o;
  auto i8 = [](uint32_t a, uint32_t b) { return F16 ? i8x8_to_f16(a, b) : i8x8_to_bf16(a, b); };
  auto e4 = [](uint32_t a, uint32_t b) { return F16 ? e4m3x8_to_f16(a, b) : e4m3x8_to_bf16(a, b); };
  if constexpr (FMT == DIALQ_FORMAT_W8A16) {
    o.b[0] = i8(t.a[0], t.a[1]);
    o.b[1] = i8(t.a[2], t.a[3]);
  } else if constexpr (FMT == DIALQ_FORMAT_FP8_ROW) {
    o.b[0] = e4(t.a[0], t.a[1]);
    o.b[1] = e4(t.a[2], t.a[3]);
  } else if constexpr (FMT == DIALQ_FORMAT_Q8_0) {
    const uint32_t dd = t.s0;
    o.s1[0] = f16_bits_to_f32(dd & 0xffffu);
    o.s1[1] = f16_bits_to_f32(dd >> 16);
    o.b[0] = i8(t.a[0], t.a[1]);
    o.b[1] = i8(t.a[2], t.a[3]);
  } else if constexpr (FMT == DIALQ_FORMAT_FP8_BLOCK) {
    o.s1[0] = __uint_as_float(t.s0);
    o.b[0] = e4(t.a[0], t.a[1]);
    o.b[1] = e4(t.a[2], t.a[3]);
    o.b[2] = e4(t.b[0], t.b[1]);
    o.b[3] = e4(t.b[2], t.b[3]);
  } else if constexpr (FMT == DIALQ_FORMAT_NVFP4) {
    const uint32_t sb = t.s0;
    float g0 = e4m3_to_f32(sb & 0xffu), g1 = e4m3_to_f32(sb >> 8);
    o.b[0] = F16 ? e2m1x8_to_f16(t.a[0], g0) : e2m1x8_to_bf16(t.a[0], g0);
    o.b[1] = F16 ? e2m1x8_to_f16(t.a[1], g0) : e2m1x8_to_bf16(t.a[1], g0);
    o.b[2] = F16 ? e2m1x8_to_f16(t.a[2], g1) : e2m1x8_to_bf16(t.a[2], g1);
    o.b[3] = F16 ? e2m1x8_to_f16(t.a[3], g1) : e2m1x8_to_bf16(t.a[3], g1);
  } else if constexpr (FMT == DIALQ_FORMAT_MXFP4) {
    float sc = e8m0_to_f32(t.s0);
#pragma unroll
    for (int i = 0; i < 4; ++i) o.b[i] = e2m1x8_pow2_to_bf16(t.a[i], sc);
  } else if constexpr (FMT == DIALQ_FORMAT_Q4_K) {
    const u32x4 h = t.hdr;
    float d = f16_bits_to_f32(h[0] & 0xffffu), dmin = f16_bits_to_f32(h[0] >> 16);
    uint32_t sc8[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) sc8[i] = (h[1 + i / 4] >> (8 * (i % 4))) & 0xffu;
    const uint32_t qd[8] = {t.a[0], t.a[1], t.a[2], t.a[3], t.b[0], t.b[1], t.b[2], t.b[3]};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t scj, mj;
      if (j < 4) {
        scj = sc8[j] & 63u;
        mj = sc8[j + 4] & 63u;
      } else {
        scj = (sc8[j + 4] & 0xfu) | ((sc8[j - 4] >> 6) << 4);
        mj = (sc8[j + 4] >> 4) | ((sc8[j] >> 6) << 4);
      }
      float s1 = d * (float)scj;
      o.s1[j] = s1;
      o.s2[j] = __builtin_fmaf(F16 ? 1024.0f : 128.0f, s1, dmin * (float)mj);
      const int i4 = j >> 1;
      o.b[j] = nib8_off<F16>(qd[2 * i4], qd[2 * i4 + 1], (j & 1) ? 4 : 0);
    }
  } else if constexpr (FMT == DIALQ_FORMAT_Q6_K) {
    const float d = f16_bits_to_f32(t.s0 & 0xffffu);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o.b[j] = q6x8_off<F16>(j < 4 ? t.a : t.b, t.hdr, j);
      // sub-blocks 2j (lanes g < 2) and 2j + 1 (g >= 2): bytes 2j, 2j+1
      const float lo = sbyte_f32(t.sc[j >> 1], 2 * (j & 1)), hi = sbyte_f32(t.sc[j >> 1], 2 * (j & 1) + 1);
      o.s1[j] = d * hi;
      o.s2[j] = d * (lo - hi);
    }
  }
  return o;
}

// acc += (x slices) . (weight tile) for one 16-row group of x; the k-quants
// can take the slices T0 .. T0 + TN - 1 only (xo[0] is slice T0).
template <int FMT, int ACT, int T0 = 0, int TN = FmtTraits<FMT>::NX>
__device__ __forceinline__ void bops_mac(const BOps<FMT> &o, const XOp<ACT> *xo, f32x4 &acc) {
  static_assert(T0 == 0 && TN == FmtTraits<FMT>::NX || FMT == DIALQ_FORMAT_Q4_K || FMT == DIALQ_FORMAT_Q6_K,
                "slice ranges are for the k-quants");
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (FMT == DIALQ_FORMAT_W8A16 || FMT == DIALQ_FORMAT_FP8_ROW ||
                FMT == DIALQ_FORMAT_NVFP4 || FMT == DIALQ_FORMAT_MXFP4) {
#pragma unroll
    for (int t = 0; t < FmtTraits<FMT>::NX; ++t) acc = mfma_x<ACT>(xo[t], o.b[t], acc);
  } else if constexpr (FMT == DIALQ_FORMAT_Q8_0) {
    f32x4 p0 = mfma_x<ACT>(xo[0], o.b[0], zero);
    f32x4 p1 = mfma_x<ACT>(xo[1], o.b[1], zero);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc[i] = __builtin_fmaf(o.s1[1], p1[i], __builtin_fmaf(o.s1[0], p0[i], acc[i]));
  } else if constexpr (FMT == DIALQ_FORMAT_FP8_BLOCK) {
    f32x4 p = zero;
#pragma unroll
    for (int t = 0; t < 4; ++t) p = mfma_x<ACT>(xo[t], o.b[t], p);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(o.s1[0], p[i], acc[i]);
  } else if constexpr (FMT == DIALQ_FORMAT_Q4_K) {
    constexpr uint32_t ONE = ActTraits<ACT>::F16OP ? 0x3c003c00u : 0x3f803f80u;  // 1.0 pairs
    const u32x4 ones = {ONE, ONE, ONE, ONE};
#pragma unroll
    for (int j = T0; j < T0 + TN; ++j) {
      f32x4 pq = mfma_x<ACT>(xo[j - T0], o.b[j], zero);
      f32x4 px = mfma_x<ACT>(xo[j - T0], ones, zero);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i] = __builtin_fmaf(o.s1[j], pq[i], __builtin_fmaf(-o.s2[j], px[i], acc[i]));
    }
  } else if constexpr (FMT == DIALQ_FORMAT_Q6_K) {
    // A 32-k slice spans two 16-value sub-blocks with their own scales:
    // lanes g < 2 hold the lower one.  With P = x.(128 + q) and C = sum(x),
    // over the whole slice (a) and over the lower sub-block only (l):
    // y += s_hi*(Pa - 160 Ca) + (s_lo - s_hi)*(Pl - 160 Cl)  (1056 for the
    // f16 operands, whose codes are offset by 1024).
    constexpr uint32_t ONE = ActTraits<ACT>::F16OP ? 0x3c003c00u : 0x3f803f80u;
    constexpr float OFF = ActTraits<ACT>::F16OP ? 1056.0f : 160.0f;
    const u32x4 ones = {ONE, ONE, ONE, ONE};
    const u32x4 z4 = {0, 0, 0, 0};
    const bool lower = (threadIdx.x & 32) == 0;
#pragma unroll
    for (int j = T0; j < T0 + TN; ++j) {
      const XOp<ACT> &xj = xo[j - T0];
      XOp<ACT> xl;
      xl.hi = lower ? xj.hi : z4;
      if constexpr (ActTraits<ACT>::PARTS == 2) xl.lo = lower ? xj.lo : z4;
      const f32x4 pa = mfma_x<ACT>(xj, o.b[j], zero), ca = mfma_x<ACT>(xj, ones, zero);
      const f32x4 pl = mfma_x<ACT>(xl, o.b[j], zero), cl = mfma_x<ACT>(xl, ones, zero);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ua = __builtin_fmaf(-OFF, ca[i], pa[i]), ul = __builtin_fmaf(-OFF, cl[i], pl[i]);
        acc[i] = __builtin_fmaf(o.s1[j], ua, __builtin_fmaf(o.s2[j], ul, acc[i]));
      }
    }
  }
}

// ---- output stores -------------------------------------------------------------
// The y dtype is dispatched once per workgroup: body(YDtype<DIALQ_BF16>{}) and
// its siblings each carry a compile-time dtype, so the per-element stores are
// plain conversions and stores without branches.
template <int YT>
struct YDtype {
  static constexpr int value = YT;
  typedef typename std::conditional<YT == DIALQ_F32, float, uint16_t>::type T;
  __device__ static __forceinline__ T conv(float v) {
    if constexpr (YT == DIALQ_BF16) return f32_to_bf16_bits(v);
    else if constexpr (YT == DIALQ_F16) return f32_to_f16_bits(v);
    else return v;
  }
};
template <typename F>
__device__ __forceinline__ void with_y_dtype(int y_dtype, F &&body) {
  if (y_dtype == DIALQ_BF16) body(YDtype<DIALQ_BF16>{});
  else if (y_dtype == DIALQ_F16) body(YDtype<DIALQ_F16>{});
  else body(YDtype<DIALQ_F32>{});
}

// silu(g) * u in f32, silu(g) = g / (1 + exp(-g)) (candle_nn::ops::silu),
// from the unrounded gate and up sums; one rounding at the store.
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int FMT>
__device__ __forceinline__ float epilogue_scale(const WeightView &w, int64_t n) {
  if constexpr (FMT == DIALQ_FORMAT_W8A16 || FMT == DIALQ_FORMAT_FP8_ROW) return w.row_scale[n];
  if constexpr (FMT == DIALQ_FORMAT_NVFP4) return w.global;
  return 1.0f;
}

}  // namespace dialq
