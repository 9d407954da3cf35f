/*
 * dialq -- C ABI of the MI355X (gfx950) quantized-linear library.
 *
 * This is the drop-in boundary for DIAL's quantized linear layer: the entry
 * points below are what a thin Rust FFI crate behind dial-core's
 * TextLinear / QuantLinear (candle CustomOp1) call sites binds.  The
 * conventions follow the reference's only C ABI, the GGML adapter
 * (backends/qwen38_ggml/adapter.h:8-46): an ABI-version export, opaque owned
 * handles, `char *error, size_t error_size` out-parameters, int 0 / -1
 * status, and a `device_io` flag that says whether buffers are device
 * (HIP) pointers or host pointers.  Nothing here throws across the ABI.
 *
 * Threading: calls on different handles may run concurrently.  Calls on one
 * handle are stream-ordered; callers serialize forward calls that share a
 * handle across streams (each handle owns one scratch area), and never
 * destroy a handle while a forward on it is in flight.
 *
 * Weight layout: W is [out_dim (N), in_dim (K)] row-major (out x in), as in
 * the reference (worker_w8a16.rs:294-297, cuda_quant.rs:289-358).  x is
 * [rows (M), K] row-major contiguous; y is [M, N].
 */
#ifndef DIALQ_H
#define DIALQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DIALQ_ABI_VERSION 1u

/* Weight formats.  The raw byte layouts are the reference's (or GGUF's /
 * OCP MX's) storage layouts; dialq_linear_create repacks them into the
 * device-resident tiled layout. */
enum dialq_format {
  /* int8 [N,K] + one scale per row, f32 (worker_w8a16.rs:294-297) or bf16 */
  DIALQ_FORMAT_W8A16 = 1,
  /* GGUF Q8_0: [N, K/32] blocks of {f16 d; i8 qs[32]} (34 B) */
  DIALQ_FORMAT_Q8_0 = 2,
  /* GGUF Q4_K: [N, K/256] super-blocks {f16 d, dmin; u8 scales[12]; u8 qs[128]} */
  DIALQ_FORMAT_Q4_K = 3,
  /* E4M3 [N,K] + f32 scale per row, or one per tensor (cuda_quant.rs:58-65) */
  DIALQ_FORMAT_FP8_ROW = 4,
  /* E4M3 [N,K] + f32 scale per 128x128 block, [ceil(N/128), ceil(K/128)] */
  DIALQ_FORMAT_FP8_BLOCK = 5,
  /* NVFP4: E2M1 [N, K/2] (low nibble = even k) + E4M3 scale per 16 + f32
   * global (cuda_quant.rs:43-56, quant.rs:160-208) */
  DIALQ_FORMAT_NVFP4 = 6,
  /* MXFP4 (OCP MX v1.0): E2M1 [N, K/2] + E8M0 scale per 32 along K */
  DIALQ_FORMAT_MXFP4 = 7,
  /* GGUF Q6_K: [N, K/256] super-blocks {u8 ql[128]; u8 qh[64]; i8 scales[16];
   * f16 d} (210 B), w = d * scales[k/16] * (q6 - 32); the second type of a
   * Q4_K_M file (worker_gguf.rs:536-540, docs/worker_gguf.md:3-5) */
  DIALQ_FORMAT_Q6_K = 8
};

enum dialq_dtype { DIALQ_F32 = 0, DIALQ_F16 = 1, DIALQ_BF16 = 2 };

/* desc.flags */
#define DIALQ_FLAG_GLOBAL_IS_DIVISOR 0x1 /* NVFP4 compressed-tensors: the
  stored global scale is a divisor; the multiplier is 1/global
  (quant.rs:322-329, quant.rs:407-412) */
#define DIALQ_FLAG_WEIGHT_ONLY_PREFILL 0x2 /* FP8_BLOCK / MXFP4: keep the
  weight-only bf16 product for prefill instead of quantizing activations
  for the native fp8 / fp4 MFMA product */

typedef struct dialq_linear_desc {
  int32_t format;      /* enum dialq_format */
  int32_t scale_dtype; /* W8A16: DIALQ_F32 or DIALQ_BF16; else ignored */
  int64_t out_dim;     /* N */
  int64_t in_dim;      /* K */
  float global_scale;  /* NVFP4 global scale (see DIALQ_FLAG_GLOBAL_IS_DIVISOR) */
  int32_t flags;
} dialq_linear_desc;

/* Kernel selection for dialq_linear_forward_ex. */
enum dialq_path {
  DIALQ_PATH_AUTO = 0,        /* GEMV for rows <= 16; above, GEMM_NATIVE for
                                 FP8_BLOCK / MXFP4 (unless
                                 DIALQ_FLAG_WEIGHT_ONLY_PREFILL), GEMM for
                                 the other formats (W8A16 / FP8_ROW split
                                 along K while their tiles are few) */
  DIALQ_PATH_GEMV = 1,        /* decode kernel, any rows (loops over row groups) */
  DIALQ_PATH_GEMM = 2,        /* weight-only MFMA GEMM (bf16/f16 operands) */
  DIALQ_PATH_GEMM_NATIVE = 3  /* FP8_BLOCK / MXFP4: activations quantized per
                                 token (fp8) or per 32 (MXFP4), fp8/fp4 MFMA */
};

/* Replaces the NVRTC kernel-availability checks of
 * worker_w8a16.rs:236-289 / cuda_quant.rs:214-267 and the adapter's
 * dial_ggml_abi_version (adapter.h:16). */
uint32_t dialq_abi_version(void);

/* Upload and repack pre-quantized weights.  Replaces the constructors
 * CudaQuantLinear::nvfp4 / ::fp8 (cuda_quant.rs:289-358, including their
 * length checks and messages) and the upload half of
 * CudaW8A16Linear::from_linear (worker_w8a16.rs:343-350).
 *   weight / weight_bytes: raw format bytes (layout per enum dialq_format)
 *   scales / scale_bytes:  W8A16: N f32|bf16; FP8_ROW: N or 1 f32;
 *                          FP8_BLOCK: ceil(N/128)*ceil(K/128) f32;
 *                          NVFP4: N*K/16 E4M3 bytes; MXFP4: N*K/32 E8M0 bytes;
 *                          Q8_0 / Q4_K / Q6_K: NULL, 0 (scales live in the blocks)
 *   host_io: 1 = weight/scales are host pointers, 0 = device pointers
 *   stream:  hipStream_t (NULL = default stream); the call synchronizes it
 * Returns an owned handle, or NULL with a message in `error`. */
void *dialq_linear_create(const dialq_linear_desc *desc, const void *weight,
                          size_t weight_bytes, const void *scales,
                          size_t scale_bytes, int device, int host_io,
                          void *stream, char *error, size_t error_size);

/* Quantize a dense [N,K] weight on the GPU and keep it resident.
 * W8A16 replaces CudaW8A16Linear::from_linear (worker_w8a16.rs:302-366: the
 * reference downloads the F16 weight, quantizes per row on the host and
 * uploads; here the same per-row arithmetic runs on the device).  Q8_0 and
 * Q4_K replace candle's QTensor::quantize (called at worker_gguf.rs:641,657
 * and ggml_tests.rs:83-84).  FP8_BLOCK and MXFP4 quantize round-to-nearest-
 * even with one f32 scale per 128x128 block / one E8M0 scale per 32.
 *   dense: [N,K] of dense_dtype (F32, F16 or BF16); host pointer if
 *   host_io = 1, else a device pointer. */
void *dialq_linear_quantize(const dialq_linear_desc *desc, const void *dense,
                            int32_t dense_dtype, int device, int host_io,
                            void *stream, char *error, size_t error_size);

/* Free a handle (Drop of CudaW8A16Linear / CudaQuantLinear). NULL is a no-op. */
void dialq_linear_destroy(void *linear);

/* Bytes the reference would count as resident for this weight: the formula
 * of CudaQuantLinear::resident_bytes (cuda_quant.rs:360-371) for NVFP4
 * (N*K/2 + N*K/16 + 4) and FP8_ROW (N*K + 4N), of from_linear's summary for
 * W8A16 (N*K + N*sizeof(scale), worker_w8a16.rs:351), and the packed format
 * size for the others. */
uint64_t dialq_linear_resident_bytes(const void *linear);

/* Bytes actually held on the device (tiles + scales + scratch). */
uint64_t dialq_linear_device_bytes(const void *linear);

/* Copy the handle's description out. */
int dialq_linear_describe(const void *linear, dialq_linear_desc *desc);

/* Forward y = x W^T.  Replaces CudaW8A16Linear::forward + cuda_fwd
 * (worker_w8a16.rs:368-386,402-475), CudaQuantLinear::forward + cuda_fwd
 * (cuda_quant.rs:373-391,406-499) and the GGUF QMatMul::forward call of
 * forward_worker_gguf (worker_gguf.rs:574-611).
 *   x: [rows, K] of x_dtype (F16, BF16 or F32), contiguous, at any address
 *      (a view at any start offset, as candle's contiguous layouts allow,
 *      worker_w8a16.rs:419); the kernels read from a 16-byte-aligned base,
 *      so a device x at any other address is first copied, on `stream`,
 *      into an aligned staging buffer the handle owns and grows (outside
 *      stream capture, like every per-handle scratch buffer)
 *   y: [rows, N] of y_dtype (F16, BF16 or F32), written in full; aligned to
 *      its element size
 *   device_io: 1 = x / y are device pointers (asynchronous on `stream`);
 *              0 = host pointers (copied in and out; synchronous)
 * Per-handle scratch (the decode workspace, the native prefill's activation
 * codes and partials, the staged x) grows on the first call of a larger
 * shape: that call synchronizes `stream` and allocates, and fails with a
 * message if `stream` is capturing -- capture after one eager call of the
 * same shape.
 * rows == 0 is a successful no-op.  Returns 0, or -1 with a message. */
int dialq_linear_forward(void *linear, const void *x, int32_t x_dtype,
                         int64_t rows, void *y, int32_t y_dtype, void *stream,
                         int device_io, char *error, size_t error_size);

/* As dialq_linear_forward with an explicit kernel choice (enum dialq_path). */
int dialq_linear_forward_ex(void *linear, const void *x, int32_t x_dtype,
                            int64_t rows, void *y, int32_t y_dtype,
                            int32_t path, void *stream, int device_io,
                            char *error, size_t error_size);

/* Grouped forward over n handles that share their input:
 *   y = cat([x W_0^T, x W_1^T, ..., x W_{n-1}^T], -1),  y: [rows, sum N_j]
 * Replaces QkvProjection::Split::forward and MlpGateUpProjection::Split::
 * forward (qwen3_vl/text.rs:1093-1101, :451-455: q / k / v or gate / up
 * TextLinear::forward on one x, then Tensor::cat along the last dim), the
 * projections the GGUF worker builds (text.rs:1387-1425).  All handles must
 * have the same in_dim and device.  The decode path runs the strips of up
 * to four consecutive same-format members in one launch (x staged once per
 * workgroup, one launch's fill and drain instead of one per member); the
 * prefill paths run the column tiles of up to four consecutive same-format
 * members in one GEMM launch (W8A16, FP8_ROW, Q4_K, Q8_0 and Q6_K with
 * bf16 / f16 x; FP8_BLOCK and MXFP4 native on x quantized once; the first
 * member's scratch serves the launch).  A grouped launch splits its sums along K
 * from the group's tile count, so a member may differ from its own forward
 * by f32 rounding.  Other cases run one launch per member, each writing
 * its columns of y, with the same kernels and results as
 * dialq_linear_forward_ex per member.  Other arguments as
 * dialq_linear_forward_ex (x at any address; y aligned to its element
 * size; per-handle scratch grows outside stream capture only). */
int dialq_linear_forward_group(void *const *linears, int32_t n, const void *x,
                               int32_t x_dtype, int64_t rows, void *y,
                               int32_t y_dtype, int32_t path, void *stream,
                               int device_io, char *error, size_t error_size);

/* Allocation-free forward; no counterpart in the reference.  For callers
 * that cannot allocate device memory during the call: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  The same
 * kernels as dialq_linear_forward_ex (device pointers only, device_io = 1),
 * with every scratch buffer -- decode workspace and counters, the native
 * prefill's activation codes, split-K partials and tile counters, the
 * aligned copy of a misaligned x -- taken from one static 32 MiB array per
 * device (held from the first call on that device until the process ends)
 * instead of the handle's grown buffers.  The call allocates and frees
 * nothing.  Sizes beyond the array (e.g. native prefill of 1024 rows at
 * K = 17408 plus split-K partials over 32 MiB, or an out_dim above 262112
 * rows) return -1 with a message naming the bytes needed; a prefill whose
 * last round of tiles would be split along K with partials that do not fit
 * runs that round whole instead (equal to dialq_linear_forward_ex to f32
 * rounding rather than bit for bit).  The array is
 * shared by every call on a device: calls that overlap on one device (two
 * streams, two host threads) race; serialize them.  The first call on a
 * device looks the array up and clears its counters: make it outside
 * stream capture. */
int dialq_linear_forward_noalloc(void *linear, const void *x, int32_t x_dtype,
                                 int64_t rows, void *y, int32_t y_dtype,
                                 int32_t path, void *stream, char *error,
                                 size_t error_size);

/* Fused gate_up projection with the SwiGLU epilogue: for a weight whose rows
 * [0, N/2) are the MLP's gate and [N/2, N) its up projection (the
 * MlpGateUpProjection::Fused weight, qwen3_vl/text.rs:424-469),
 *   y[m, j] = silu(g[m, j]) * u[m, j],  g = x W[0:N/2]^T,  u = x W[N/2:N]^T,
 * silu(g) = g / (1 + exp(-g)), computed in f32 from the unrounded products
 * and rounded once to y_dtype.  Replaces gate_up_proj.forward followed by
 * Mlp::mlp_mid_from_gate_up (qwen3_vl/text.rs:816-820: narrow, silu, mul).
 *   y: [rows, N/2] of y_dtype.  N must be a multiple of 128.
 * Paths and the other arguments as dialq_linear_forward_ex. */
int dialq_linear_forward_swiglu(void *linear, const void *x, int32_t x_dtype,
                                int64_t rows, void *y, int32_t y_dtype,
                                int32_t path, void *stream, int device_io,
                                char *error, size_t error_size);

/* Token selection over one row of logits, after the lm_head.  Replaces the
 * selection steps of sample_remote_logits / FastLogitsProcessor::sample
 * (qwen3_vl/qwen3_vl.rs:130-174,282-323): the repeat penalty
 * (apply_repeat_penalty_in_place, :225-240: the logit of each distinct
 * context id below vocab divided by the penalty when >= 0, else multiplied),
 * the greedy argmax, the top-k candidates and the softmax normaliser of
 * softmax_in_place (:325-345).
 *   logits: [vocab] of dtype; repeat_ids: HOST array of n_repeat ids (used
 *   only when repeat_penalty != 1)
 *   rule: DIALQ_SELECT_FIRST_MAX -- candle's argmax (the reference's greedy
 *         device path): -0 == +0, NaN never chosen, ties to the smaller index;
 *         DIALQ_SELECT_TOTAL_LAST_MAX -- max_by(f32::total_cmp) (its host
 *         path): IEEE total order, ties to the larger index
 *   k: 1 .. DIALQ_SELECT_MAX_K; out_idx[k], out_val[k]: indices and
 *      (penalised) logits in descending order of the rule
 *   temperature > 0: out_stats = {M, S}, M = max over the vocabulary of
 *      logit / temperature, S = sum of exp(logit / temperature - M), so that
 *      softmax_in_place's probability of candidate i is
 *      exp(out_val[i] / temperature - M) / S; otherwise out_stats = {-inf, 0}
 *   workspace: device memory of dialq_logits_select_workspace_bytes(vocab,
 *      n_repeat) bytes (device_io = 1); NULL lets the call allocate its own
 *      and synchronise
 *   device_io: 1 = logits and outputs are device pointers on `device`,
 *      asynchronous on `stream` (synchronous when repeat ids are uploaded);
 *      0 = host pointers, synchronous. */
enum dialq_select_rule { DIALQ_SELECT_FIRST_MAX = 0, DIALQ_SELECT_TOTAL_LAST_MAX = 1 };
#define DIALQ_SELECT_MAX_K 256
size_t dialq_logits_select_workspace_bytes(int64_t vocab, int64_t n_repeat);
int dialq_logits_select(const void *logits, int32_t dtype, int64_t vocab,
                        const uint32_t *repeat_ids, int64_t n_repeat,
                        float repeat_penalty, float temperature, int32_t rule,
                        int64_t k, uint32_t *out_idx, float *out_val,
                        float *out_stats, void *workspace,
                        size_t workspace_bytes, int32_t device, void *stream,
                        int device_io, char *error, size_t error_size);

/* Dequantize the resident weight into a dense [N,K] matrix of out_dtype
 * (F32, F16 or BF16, each rounded once to nearest-even from the exact f32
 * value).  Replaces QMatMul::dequantize_f16 (worker_w8a16.rs:125, used by
 * build_worker_gguf_fp16_prefill_linear, worker_gguf.rs:425-452) and the
 * host decoders load_nvfp4 / load_fp8 / decode_nvfp4_values
 * (quant.rs:160-208,252-363). */
int dialq_linear_dequantize(const void *linear, void *out, int32_t out_dtype,
                            void *stream, int device_io, char *error,
                            size_t error_size);

/* Export the raw (reference-layout) weight and scale bytes of a handle, e.g.
 * after dialq_linear_quantize.  Sizes must equal the format's raw sizes.
 * Host buffers; synchronous. */
int dialq_linear_export(const void *linear, void *weight, size_t weight_bytes,
                        void *scales, size_t scale_bytes, char *error,
                        size_t error_size);

/* Local q8 decode (qwen3_vl/text.rs:291-336): W8A8 with a per-tensor int8
 * activation scale, exact int32 dot, y = f32(acc) * scale[n] * x_scale.
 * Requires a W8A16 handle with f32 scales and rows == 1. */
int dialq_local_q8_forward(void *linear, const void *x, int32_t x_dtype,
                           int64_t rows, void *y, int32_t y_dtype,
                           void *stream, int device_io, char *error,
                           size_t error_size);

/* Test hook; no counterpart in the reference.  Sets how many polls without
 * progress the decode kernel's work-queue waits make before giving up
 * (process-wide; a negative value restores the default of 4194304).  A
 * launch that gives up still ends normally but leaves an incomplete output:
 * it marks its handle, and the next forward on that handle returns -1 with
 * a message and resets the handle's queue counters.  For tests of that
 * failure path only. */
void dialq_debug_set_wait_limit(int64_t polls);

/* Test hook; no counterpart in the reference.  The number of grouped decode
 * and prefill launches (dialq_linear_forward_group members run as one
 * kernel) this process has made, so that tests can tell a grouped launch
 * from the per-member fallback, whose outputs are the same to rounding. */
int64_t dialq_debug_grouped_launches(void);

#ifdef __cplusplus
}
#endif
#endif /* DIALQ_H */
