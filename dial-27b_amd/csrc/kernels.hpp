// Internal launcher interface between the C ABI (dialq.cpp) and the HIP
// kernels.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dialq {

struct DequantArgs {
  int fmt;
  int64_t N, K, k_chunks, nbk;
  int chunk, tile_bytes;
  const uint8_t *tiles;
  const uint8_t *aux;
  const float *row_scale;
  const float *block_scale;
  float global;
  void *out;
  int out_dtype;
};

// Weights one grouped prefill launch covers (members that share x and K).
constexpr int kGemmMaxGroup = 4;

// Everything a product kernel needs to read one resident weight.
struct WeightView {
  int fmt;
  int64_t N, K;
  int64_t n_strips, k_chunks, nbk;
  const uint8_t *tiles;
  const uint8_t *aux;
  const float *row_scale;    // W8A16, FP8_ROW: [n_strips*16]
  const float *block_scale;  // FP8_BLOCK: [ceil(N/128), nbk]
  float global;              // NVFP4 multiplier (1 otherwise)
  // 0: y = x W^T.  > 0: W is a fused gate_up weight whose rows [0, I) are
  // the gate and [I, 2I) the up projection, I = 16 * pair, and the product
  // writes y[m, j] = silu(gate[m, j]) * up[m, j], j < I (the MLP's
  // mlp_mid_from_gate_up, qwen3_vl/text.rs:816-820).
  int64_t pair = 0;
  // Output row stride in elements; 0 = the natural width (N, or I for the
  // SwiGLU product).  A member of a grouped forward writes its columns of
  // the concatenated [M, sum N] output: y points at its first column and
  // ldy is the sum.
  int64_t ldy = 0;
};

// Row stride of the output a product kernel writes.
__host__ __device__ inline int64_t out_ld(const WeightView &w) {
  return w.ldy ? w.ldy : (w.pair ? w.pair * 16 : w.N);
}

hipError_t launch_quantize(int fmt, const void *dense, int dtype, int64_t N, int64_t K, void *raw_w,
                           void *raw_s, hipStream_t st);
hipError_t launch_repack(int fmt, int64_t N, int64_t K, const void *raw_w, const void *raw_s,
                         int scale_is_bf16, int64_t scale_count, uint8_t *tiles, uint8_t *aux,
                         float *row_scale, float *block_scale, hipStream_t st);
hipError_t launch_unpack(int fmt, int64_t N, int64_t K, const uint8_t *tiles, const uint8_t *aux,
                         void *raw_w, void *raw_s, hipStream_t st);
hipError_t launch_dequant(const DequantArgs &a, hipStream_t st);
hipError_t launch_act_fp8(const void *x, int dtype, int64_t M, int64_t K, int64_t k_pad, uint8_t *q,
                          float *scale, hipStream_t st);
hipError_t launch_act_mxfp4(const void *x, int dtype, int64_t M, int64_t K, int64_t k_pad,
                            uint8_t *packed, uint8_t *scales, hipStream_t st);
// bf16 rows [M, K] -> f16 rows scaled by 2^-e_m so that each row's maximum
// sits in [2^14, 2^15); rs[m] = 2^e_m (the GGUF prefill's f16 kernel on bf16
// activations).  K % 8 == 0.
hipError_t launch_x_f16_rows(const void *x, int64_t M, int64_t K, uint16_t *xh, float *rs, hipStream_t st);

// Decode GEMV: y[M,N] = x[M,K] W^T for any M (16 rows per pass).
// ws: gemv_workspace_bytes(w, x_dtype, M) of scratch (exactly what the
// launches pick, often 0); cnt: n_strips + 2 ints that are
// zero before the call and are left zero after it.  err: a host-visible int
// (device address) that a launch sets to 1 when one of the work queue's
// bounded waits gives up -- its output is then incomplete and cnt may be
// left non-zero.  The resident tiles must be smaller than 2 GiB (32-bit
// buffer offsets).
size_t gemv_workspace_bytes(const WeightView &w, int x_dtype, int64_t M);
hipError_t launch_gemv(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y,
                       int y_dtype, float *ws, size_t ws_bytes, int *cnt, int *err, hipStream_t st);
// One decode launch over the strips of n (2..4) weights that share x (the
// same format and K): member j writes [M, N_j] through ys[j] with its view's
// output stride.  Returns hipErrorNotSupported, launching nothing, where the
// grouped kernel does not apply (activations too large to stage, SwiGLU,
// mixed formats); the caller then launches per member.
hipError_t launch_gemv_group(const WeightView *ws, void *const *ys, int n, const void *x, int x_dtype, int64_t M,
                             int y_dtype, hipStream_t st);
// Grouped decode launches made by this process (a test hook: a group that
// fell back to one launch per member leaves it unchanged).
int64_t gemv_grouped_launches();
// Polls without progress before a bounded wait of the work queue gives up
// (process-wide; < 0 restores the default).
void set_gemv_wait_limit(int64_t polls);
int gemv_wait_limit();
// Prefill GEMM with weight-only dequantization (bf16 / f16 MFMA operands).
// Launches with fewer tiles than workgroup slots split each tile along K,
// launches whose last round of tiles is at most half full split that
// round's tiles (`tail`: false keeps them whole); both need
// gemm_workspace(M, w, x_dtype) of scratch: `part` (partial tiles) and
// `cnt` (per-tile counters, zero before the call and left zero after it).
// The launch plans its split within the `part` bytes it is given, so a
// buffer sized without the tail split runs without it.
void gemm_workspace(int64_t M, const WeightView &w, int x_dtype, size_t &part_bytes, size_t &cnt_count,
                    bool tail = true);
// yrow: per-row output multipliers (k_gemm_kq only; null = 1).
hipError_t launch_gemm(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y, int y_dtype, float *part,
                       size_t part_bytes, int *cnt, size_t cnt_count, hipStream_t st, const float *yrow = nullptr);
// Grouped prefill over n (2..kGemmMaxGroup) weights of one format and K that
// share x: one launch over all members' column tiles, member j writing
// [M, N_j] through ys[j] with its view's output stride.  The 32x32 kernels
// (W8A16, FP8_ROW; Q4_K and Q8_0 with bf16 / f16 x) and the native kernel (FP8_BLOCK,
// MXFP4 on x quantized once).  *_group_workspace returns false, and the
// launchers hipErrorNotSupported (launching nothing), where no grouped
// kernel applies; the caller then launches per member.
bool gemm_group_workspace(int64_t M, const WeightView *ws, int n, int x_dtype, size_t &part_bytes, size_t &cnt_count);
hipError_t launch_gemm_group(const WeightView *ws, void *const *ys, int n, const void *x, int x_dtype, int64_t M,
                             int y_dtype, float *part, size_t part_bytes, int *cnt, size_t cnt_count, hipStream_t st,
                             const float *yrow = nullptr);
bool native_group_workspace(int64_t M, const WeightView *ws, int n, size_t &part_bytes, size_t &cnt_count);
hipError_t launch_gemm_native_group(const WeightView *ws, void *const *ys, int n, const uint8_t *xq, const void *xs,
                                    int64_t M, int64_t k_pad, int y_dtype, float *part, size_t part_bytes, int *cnt,
                                    size_t cnt_count, hipStream_t st);
// Grouped prefill launches made by this process (a test hook).
int64_t gemm_grouped_launches();
// Native low-precision prefill: FP8_BLOCK with per-token fp8 activations,
// MXFP4 with per-32 MXFP4 activations.  `xq` / `xs` are the quantized
// activations (codes and scales) produced by launch_act_*.  Split tiles (few
// tiles, or the last partial round's: `tail`) need native_workspace(M, w) of
// scratch: `part` (partial tiles) and `cnt` (per-tile counters, zero before
// the call and left zero after it).  As for launch_gemm, the launch plans
// its split within the `part` bytes it is given.
void native_workspace(int64_t M, const WeightView &w, size_t &part_bytes, size_t &cnt_count, bool tail = true);
hipError_t launch_gemm_native(const WeightView &w, const uint8_t *xq, const void *xs, int64_t M,
                              int64_t k_pad, void *y, int y_dtype, float *part, size_t part_bytes, int *cnt,
                              size_t cnt_count, hipStream_t st);
// Token selection over one row of logits (repeat penalty, top-k keys,
// softmax statistics); k <= 256.  ids: distinct context tokens below vocab.
size_t select_workspace_bytes(int64_t vocab);
hipError_t launch_select(const void *logits, int dtype, int64_t vocab, const uint32_t *ids, int n_ids, float penalty,
                         float temperature, int rule, int k, void *ws, size_t ws_bytes, uint32_t *out_idx,
                         float *out_val, float *out_stats, hipStream_t st);
// Compute units of the current device (cached at first use).
int device_cus();
// Local q8 W8A8 decode (one row).
hipError_t launch_local_q8(const WeightView &w, const void *x, int x_dtype, void *y, int y_dtype,
                           void *scratch, hipStream_t st);

}  // namespace dialq
