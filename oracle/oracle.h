/*
 * CPU oracle for the quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code; only tests/, the smoke check and the CPU-baseline leg of
 * the benchmark use it, as the checker.  Every function restates the
 * reference arithmetic it cites (paths relative to the DIAL-27B source tree)
 * in plain C, scalar, with FMA contraction disabled so results are
 * bit-defined.
 *
 * Parity status per function is listed in the comment above it:
 *   "pinned by ..."  names the independent check in tests/ that would fail
 *                    on a dropped term, a wrong index or a wrong rounding;
 *   "parity unpinned" marks what no fixture or closed form in the reference
 *                    can pin (the candle Q4_K scale/min search).
 */
#ifndef DIALQ_ORACLE_H
#define DIALQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint32_t or_version(void);

/* ---- scalar codecs -------------------------------------------------- */
/* IEEE binary16 / bfloat16 <-> binary32, round-to-nearest-even (the `half`
 * crate 2.7.1 semantics used by candle's to_dtype).  Pinned against numpy
 * float16 and torch bfloat16 over edge cases and random bit patterns. */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);

/* E4M3 decode as the reference CUDA kernels do it
 * (qwen3_8/cuda_quant.rs:27-41): subnormal m*2^-9, exp=15&m=7 (NaN) -> 0.
 * Pinned against torch.float8_e4m3fn for all 254 non-NaN codes and the
 * reference KATs (quant.rs:545-619). */
float or_e4m3_to_f32(uint8_t code);
/* OCP E4M3FN decode (float8 crate, host path): NaN codes stay NaN. */
float or_e4m3_to_f32_ocp(uint8_t code);
/* f32 -> E4M3FN, round-to-nearest-even, saturating to +-448, NaN -> 0x7f.
 * Pinned against torch's float8_e4m3fn cast on every midpoint and random
 * values within range. */
uint8_t or_f32_to_e4m3(float f);
/* E2M1 table (qwen3_8/quant.rs:16-18).  Pinned by the NVFP4 KATs. */
float or_e2m1_to_f32(uint8_t code);
/* f32 -> E2M1, RNE, saturating to +-6 (OCP MX v1.0 conversion).  Pinned by
 * brute-force nearest-with-ties-to-even over every midpoint. */
uint8_t or_f32_to_e2m1(float f);
/* E8M0 -> 2^(e-127); 0xff is NaN (OCP MX v1.0 5.4). */
float or_e8m0_to_f32(uint8_t e);

/* ---- W8A16 per-row int8 ----------------------------------------------
 * Quantizer of CudaW8A16Linear::from_linear (qwen3_vl/worker_w8a16.rs:
 * 329-341); the local-q8 path uses the same quantizer
 * (qwen3_vl/text.rs:270-281).  amax = fold(max |w|); scale = amax>0 ?
 * amax/127 : 1; q = clamp(round_half_away(w * (1/scale)), -127, 127).
 * scale_bf16 (nullable) receives bf16_rne(scale), the bf16 storage of
 * the same scale; q is always computed against the f32 scale.
 * Pinned by closed-form invariants (argmax -> +-127, ties away from zero,
 * zero rows) in tests/test_oracle_formats.py. */
void or_w8a16_quantize(const float *w, int64_t n, int64_t k, int8_t *q,
                       float *scale_f32, uint16_t *scale_bf16);
/* out[n,k] = f32(q) * scale[n]   (scale_is_bf16: scale holds bf16 bits) */
void or_w8a16_dequant(const int8_t *q, const void *scale, int scale_is_bf16,
                      int64_t n, int64_t k, float *out);

/* ---- GGUF Q8_0: 34-byte blocks {f16 d; i8 qs[32]} --------------------
 * candle-core 0.11 BlockQ8_0::from_float (not vendored; the same
 * algorithm as ggml quantize_row_q8_0_reference): d = amax/127,
 * id = d ? 1/d : 0, qs = round_half_away(x*id), stored d = f16(d).
 * Pinned by the GGUF block layout and closed-form invariants. */
void or_q8_0_quantize(const float *w, int64_t n, int64_t k, uint8_t *blocks);
void or_q8_0_dequant(const uint8_t *blocks, int64_t n, int64_t k, float *out);

/* ---- GGUF Q4_K: 144-byte super-blocks {f16 d; f16 dmin; u8 scales[12];
 * u8 qs[128]} --------------------------------------------------------
 * Dequant (candle BlockQ4K::to_float, the GGUF Q4_K block format):
 * per 64-value group, y = (d*sc)*q - (dmin*m), low nibbles
 * first.  Pinned by hand-built blocks with known (d, dmin, sc, m, q).
 * Quantizer: candle BlockQ4K::from_float with make_qkx1_quants(15, 5) and
 * nearest_int = round-half-away.  Parity unpinned: the reference holds no
 * Q4_K byte fixture and candle is not vendored; only round-trip bounds are
 * checked. */
void or_q4_k_quantize(const float *w, int64_t n, int64_t k, uint8_t *blocks);
void or_q4_k_dequant(const uint8_t *blocks, int64_t n, int64_t k, float *out);
void or_q4_k_scale_min(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);

/* ---- GGUF Q6_K: 210-byte super-blocks {u8 ql[128]; u8 qh[64];
 * i8 scales[16]; f16 d} ------------------------------------------------
 * The second block type of a Q4_K_M file (qwen3_vl/worker_gguf.rs:536-540,
 * docs/worker_gguf.md:3-5).  Dequant restates the GGUF Q6_K block format
 * (ggml's dequantize_row_q6_K, which candle-core 0.11 BlockQ6K::to_float
 * reproduces; neither is in the reference tree): per 128-value half h and
 * l < 32, value 32*qd + l of the half is the 4-bit field qd>>1 of
 * ql[64h + l + 32*(qd&1)] with bits 2qd..2qd+1 of qh[32h + l] on top,
 * q - 32, times d * scales[8h + 2qd + l/16].  Products are exact in f32
 * (11 + 8 + 6 significant bits).  Pinned against an element-wise encoder
 * written from the same layout description (tests/test_oracle_formats.py)
 * and invariants (zero d, constant codes); parity with candle's own
 * element order is unpinned (no Q6_K fixture exists in the reference). */
void or_q6_k_dequant(const uint8_t *blocks, int64_t n, int64_t k, float *out);

/* ---- FP8 E4M3 ---------------------------------------------------------
 * Reference layout (cuda_quant.rs:58-65): u8[n,k] with one f32 scale per
 * row (a per-tensor scale is broadcast, quant.rs:418-425).
 * out = e4m3(q) * scale[n].  Pinned by quant.rs:596-619 KAT. */
void or_fp8_row_dequant(const uint8_t *q, const float *scale, int64_t n,
                        int64_t k, float *out);
/* 128x128-block layout: scales[(n/128) * ceil(k/128) + k/128], f32.
 * s = amax>0 ? amax/448 : 1; q = e4m3_rne(w * (1/s)).  Closed form. */
void or_fp8_block_quantize(const float *w, int64_t n, int64_t k, uint8_t *q,
                           float *scales);
void or_fp8_block_dequant(const uint8_t *q, const float *scales, int64_t n,
                          int64_t k, float *out);

/* ---- NVFP4 (reference FP4): packed u8[n, k/2] low nibble = even k, group
 * scale per 16, global f32 (quant.rs:160-208; cuda_quant.rs:43-56).
 * out = (E2M1[code] * group_scale) * global.
 * scales_are_e4m3 = 1: scales hold E4M3 bytes decoded as the CUDA path
 * does; 0: scales are f32 (host path).  Returns -1 on a length error and
 * writes the reference's message.  Pinned by quant.rs:527-594,650-680. */
int or_nvfp4_dequant(const uint8_t *packed, size_t packed_len,
                     const void *scales, size_t scales_len,
                     int scales_are_e4m3, float global_scale, int64_t n,
                     int64_t k, float *out, char *err, size_t err_size);

/* ---- MXFP4 (OCP MX v1.0): packed u8[n, k/2] low nibble = even k, one
 * E8M0 per 32 along k.  shared = max(floor(log2 amax) - 2, -127);
 * p = e2m1_rne(w / 2^shared).  Closed form. */
void or_mxfp4_quantize(const float *w, int64_t n, int64_t k, uint8_t *packed,
                       uint8_t *scales);
void or_mxfp4_dequant(const uint8_t *packed, const uint8_t *scales, int64_t n,
                      int64_t k, float *out);

/* ---- activation quantizers used by native fp8/fp4 prefill ------------
 * Per-token FP8: s[m] = amax>0 ? amax/448 : 1; q = e4m3_rne(x * (1/s)). */
void or_act_fp8_quantize(const float *x, int64_t m, int64_t k, uint8_t *q,
                         float *scale);
/* Per-32 MXFP4 along k, identical to or_mxfp4_quantize on x rows. */
void or_act_mxfp4_quantize(const float *x, int64_t m, int64_t k,
                           uint8_t *packed, uint8_t *scales);

/* ---- products ----------------------------------------------------------
 * y[m,n] = sum_k x[m,k] * w[n,k], accumulated in double (the fp32-or-better
 * oracle); pinned against numpy matmul. */
void or_matmul_f64(const float *x, const float *w, int64_t m, int64_t n,
                   int64_t k, double *y);
/* W8A16 kernel arithmetic (worker_w8a16.rs:146-184): per output,
 * fp32 sum over k of f32(q)*x, then * scale[n] (scale applied after the
 * sum).  Sequential-k fp32 accumulation. */
void or_w8a16_linear(const float *x, const int8_t *q, const void *scale,
                     int scale_is_bf16, int64_t m, int64_t n, int64_t k,
                     float *y);
/* Local q8 W8A8 decode (qwen3_vl/text.rs:291-336): x_scale = amax/127 (1 if
 * 0), xq = clamp(round(x/x_scale)), acc = i32 dot, y = f32(acc)*scale*xs.
 * Pinned: the integer dot is checked against numpy int64. */
void or_local_q8_forward(const float *x, int64_t k, const int8_t *q,
                         const float *scale, int64_t n, float *y);

#ifdef __cplusplus
}
#endif
#endif
