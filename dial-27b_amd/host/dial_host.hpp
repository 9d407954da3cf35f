// Host-side operator layer of DIAL's quantized linear, above the dialq C ABI.
//
// It mirrors the reference's Rust interfaces for this path: same type and
// function names, the same argument meaning, the same routing and the same
// error texts where the reference has them.
//   QuantLinear, linear_no_bias, configure_quant_linear,
//   quant_linear_summary                          qwen3_8/quant.rs:20-139,466-519
//   RocmQuantLinear (CudaQuantLinear)             qwen3_8/cuda_quant.rs:289-391
//   TextLinear, W8A16Linear (CudaW8A16Linear),
//   configure_worker_w8a16_from_args              qwen3_vl/worker_w8a16.rs:15-140,302-386
//   GgufMatMul (candle QMatMul), forward_worker_gguf,
//   configure_worker_gguf_from_args,
//   load_worker_gguf_linear,
//   worker_gguf_prefill_for_dims                  qwen3_vl/worker_gguf.rs:65-197,388-522,574-611
// (paths relative to dial-core/src/models).
//
// Differences, all MI355X-side:
//   * the device is ROCm (HIP) and "cuda" modes read "rocm";
//   * activations may be F16, BF16 or F32, where the reference kernels take
//     F16 only (the mode gates accept f16 and bf16 runtimes);
//   * every quantized product, quantizer and dequantizer runs in libdialq on
//     the GPU; the dense fallbacks multiply with rocBLAS.  Nothing on this
//     path computes on the CPU.
// Tensors own host or device (hipMalloc) memory; all GPU work is issued on
// the default stream, and calls that return host data synchronise it.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

namespace dial {

class Error : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

enum class DType { F32 = 0, F16 = 1, BF16 = 2, U8 = 3 };
const char *dtype_name(DType t);  // "F32", "F16", "BF16", "U8" (candle's Debug names)
size_t dtype_size(DType t);

struct Device {
  enum Kind { Cpu, Rocm };
  Kind kind = Cpu;
  int ordinal = 0;
  static Device cpu() { return Device{}; }
  static Device rocm(int ordinal = 0) { return Device{Rocm, ordinal}; }
  bool is_rocm() const { return kind == Rocm; }
  bool operator==(const Device &o) const { return kind == o.kind && (kind == Cpu || ordinal == o.ordinal); }
  std::string debug() const;  // "Cpu" / "Rocm(0)"
};

// Owned, contiguous, row-major buffer on the host or on a ROCm device.
class Tensor {
 public:
  Tensor() = default;
  static Tensor from_host(const void *data, DType dtype, std::vector<int64_t> dims);
  static Tensor empty(DType dtype, std::vector<int64_t> dims, Device device);
  Tensor to_device(Device device) const;
  std::vector<uint8_t> host_bytes() const;  // synchronous copy to the host
  Tensor reshape(std::vector<int64_t> dims) const;  // shares storage

  DType dtype() const { return dtype_; }
  const std::vector<int64_t> &dims() const { return dims_; }
  Device device() const { return device_; }
  int64_t elem_count() const;
  size_t nbytes() const { return (size_t)elem_count() * dtype_size(dtype_); }
  void *data() { return ptr_.get(); }
  const void *data() const { return ptr_.get(); }
  bool defined() const { return (bool)ptr_; }
  std::string dims_debug() const;  // "[1, 1, 4096]"

 private:
  DType dtype_ = DType::F32;
  std::vector<int64_t> dims_;
  Device device_;
  std::shared_ptr<uint8_t> ptr_;
};

// candle_nn::Linear: y = x W^T (+ b).  Weight [out, in] on a ROCm device;
// forward multiplies with rocBLAS (f32 accumulation).
class Linear {
 public:
  Linear() = default;
  Linear(Tensor weight, std::optional<Tensor> bias = std::nullopt);
  Tensor forward(const Tensor &x) const;
  const Tensor &weight() const { return weight_; }
  const std::optional<Tensor> &bias() const { return bias_; }

 private:
  Tensor weight_;
  std::optional<Tensor> bias_;
};

// candle VarBuilder stand-in: named tensors under a prefix, with the target
// runtime dtype and device.
class VarStore {
 public:
  VarStore(DType dtype, Device device) : dtype_(dtype), device_(device) {}
  void insert(const std::string &full_name, Tensor t);
  VarStore pp(const std::string &sub) const;  // push a prefix component
  bool contains_tensor(const std::string &name) const;
  const Tensor &get(const std::string &name) const;  // raises if absent
  const std::string &prefix() const { return prefix_; }
  DType dtype() const { return dtype_; }
  Device device() const { return device_; }

 private:
  std::string full(const std::string &name) const;
  std::shared_ptr<std::map<std::string, Tensor>> tensors_ = std::make_shared<std::map<std::string, Tensor>>();
  std::string prefix_;
  DType dtype_;
  Device device_;
};

// Warnings and info lines the reference sends to `log`; the last warning is
// kept for callers that surface it.
std::string last_warning();

// ---- libdialq handle -------------------------------------------------------
struct DialqHandle;  // owns one resident quantized weight

// ---- Qwen3.8 QuantLinear (qwen3_8/quant.rs, cuda_quant.rs) -----------------
class RocmQuantLinear {
 public:
  // CudaQuantLinear::nvfp4: packed [out, in/2] E2M1 bytes (low nibble = even
  // k), scales [out, in/16] E4M3 bytes, global multiplier.
  static std::shared_ptr<RocmQuantLinear> nvfp4(const std::vector<uint8_t> &packed,
                                                const std::vector<uint8_t> &scales, float global_scale,
                                                int64_t in_dim, int64_t out_dim, Device device);
  // CudaQuantLinear::fp8: weight [out, in] E4M3 bytes, one f32 scale per row.
  static std::shared_ptr<RocmQuantLinear> fp8(const std::vector<uint8_t> &weight, const std::vector<float> &scales,
                                              int64_t in_dim, int64_t out_dim, Device device);
  size_t resident_bytes() const;
  Tensor forward(const Tensor &x) const;
  int64_t in_dim() const { return in_dim_; }
  int64_t out_dim() const { return out_dim_; }

 private:
  std::shared_ptr<DialqHandle> h_;
  int64_t in_dim_ = 0, out_dim_ = 0;
};

enum class Qwen38QuantLinear { Dense, Auto, Rocm };

class QuantLinear {
 public:
  static QuantLinear dense(Linear l);
  static QuantLinear rocm(std::shared_ptr<RocmQuantLinear> l);
  Tensor forward(const Tensor &input) const;
  bool is_quantized_rocm() const { return (bool)rocm_; }
  const Linear &dense_linear() const;  // raises unless the dense variant

 private:
  std::optional<Linear> dense_;
  std::shared_ptr<RocmQuantLinear> rocm_;
};

void configure_quant_linear(Qwen38QuantLinear requested, Device device, DType dtype);
std::optional<std::pair<size_t, size_t>> quant_linear_summary();  // (linears, resident bytes)
QuantLinear linear_no_bias(int64_t input_size, int64_t output_size, const VarStore &vb);

// ---- Qwen3-VL worker linears (worker_w8a16.rs, worker_gguf.rs) --------------
class W8A16Linear {
 public:
  // CudaW8A16Linear::from_linear: per-row int8 of an F16 device weight.
  static std::shared_ptr<W8A16Linear> from_linear(const std::string &name, const Linear &linear);
  Tensor forward(const Tensor &x) const;
  size_t resident_bytes() const;
  int64_t in_dim() const { return in_dim_; }
  int64_t out_dim() const { return out_dim_; }

 private:
  std::shared_ptr<DialqHandle> h_;
  int64_t in_dim_ = 0, out_dim_ = 0;
};

// candle QMatMul stand-in for GGUF Q8_0 / Q4_K weights.
class GgufMatMul {
 public:
  enum Kind { Q8_0 = 2, Q4_K = 3, Q6_K = 8 };  // dialq format ids
  // Raw GGUF blocks (34 B per 32 / 144 B per 256 / 210 B per 256 along each
  // row), shape [out, in].
  static std::shared_ptr<GgufMatMul> from_blocks(Kind kind, const std::vector<uint8_t> &blocks, int64_t out_dim,
                                                 int64_t in_dim, Device device);
  // The same from blocks already on the device (a U8 tensor of the raw
  // block bytes), repacked there without a host copy.
  static std::shared_ptr<GgufMatMul> from_device_blocks(Kind kind, const Tensor &blocks, int64_t out_dim,
                                                        int64_t in_dim);
  // QTensor::quantize of a dense [out, in] tensor (host or device).
  static std::shared_ptr<GgufMatMul> quantize(Kind kind, const Tensor &dense, Device device);
  Tensor forward(const Tensor &x) const;  // output dtype = input dtype
  Tensor dequantize_f16() const;           // [out, in] F16 on the device
  int64_t in_dim() const { return in_dim_; }
  int64_t out_dim() const { return out_dim_; }

 private:
  std::shared_ptr<DialqHandle> h_;
  int64_t in_dim_ = 0, out_dim_ = 0;
};

class TextLinear {
 public:
  static TextLinear from_dense(const std::string &name, Linear dense);
  static TextLinear gguf(const std::string &name, std::shared_ptr<GgufMatMul> matmul);
  Tensor forward(const Tensor &x) const;
  Tensor gguf_dequantize_f16_weight() const;
  TextLinear with_gguf_fp16_prefill(Linear prefill) const;
  bool is_w8a16() const { return (bool)w8a16_; }
  bool is_gguf() const { return (bool)gguf_; }
  bool is_dense() const { return dense_.has_value() && !gguf_; }

 private:
  std::string name_;
  std::optional<Linear> dense_;  // Dense, or the GGUF fp16 prefill copy
  std::shared_ptr<GgufMatMul> gguf_;
  std::shared_ptr<W8A16Linear> w8a16_;
};

void configure_worker_w8a16_from_args(bool requested, bool worker_mode, Device device, DType dtype);
bool worker_w8a16_enabled();
std::optional<std::pair<size_t, size_t>> worker_w8a16_summary();
// configure_worker_gguf_from_args (worker_gguf.rs:65-180): opens and parses
// the GGUF file (host/gguf.hpp), checks general.architecture == "qwen3vl"
// and qwen3vl.block_count against the model config, and keeps the source
// for load_worker_gguf_linear.  Worker mode only; ROCm device, F16 or BF16
// runtime.
void configure_worker_gguf_from_args(const std::optional<std::string> &path, bool fp16_prefill, bool output_head,
                                     bool sample_token, bool worker_mode, Device device, DType dtype,
                                     int64_t num_hidden_layers);
bool worker_gguf_enabled();
bool worker_gguf_fp16_prefill_enabled();
bool worker_gguf_output_head_requested();
bool worker_gguf_sample_token_requested();
// (GGUF linears, their raw bytes, FP16 prefill linears, their bytes)
std::optional<std::tuple<size_t, size_t, size_t, size_t>> worker_gguf_summary();
// load_worker_gguf_linear (worker_gguf.rs:462-522): tensor
// blk.{layer}.{suffix}.weight, shape [out_dim, in_dim], uploaded and
// repacked (Q8_0, Q4_K, Q6_K), warmed once per GGUF dtype.  nullopt when no
// GGUF source is configured.
std::optional<TextLinear> load_worker_gguf_linear(std::optional<int64_t> layer_idx, const std::string &tensor_suffix,
                                                  int64_t in_dim, int64_t out_dim);
bool worker_gguf_prefill_for_dims(const std::vector<int64_t> &dims);
Tensor forward_worker_gguf(const GgufMatMul &matmul, const Tensor &x);
// build_worker_gguf_fp16_prefill_linear (worker_gguf.rs:425-452): the F16
// dequantized weights of GGUF linears, rows concatenated (fused QKV /
// gate_up), as one dense linear.
Linear build_worker_gguf_fp16_prefill_linear(const std::string &name, const std::vector<TextLinear> &sources);

// ---- worker GGUF output head (worker_gguf.rs:197-383) ------------------------
struct SamplingRequest;  // sampling.hpp
// f32 -> f16 bits, round to nearest even (half::f16::from_f32), as the output
// head converts output_norm.weight.
uint16_t f32_to_f16_bits(float f);
struct OutputHeadConfig {
  int64_t hidden_size = 0, vocab_size = 0, num_hidden_layers = 0;
  double rms_norm_eps = 1e-6;
};
// load_worker_gguf_output_head (worker_gguf.rs:197-310): when the head was
// requested and this worker owns the final layer, loads output_norm.weight
// (as F16, candle's gguf_tensor_to_f16) and output.weight -- or the tied
// token_embd.weight -- as a quantized lm_head (Q8_0 / Q4K / Q6K, streamed to
// the device in chunks), with the reference's shape checks and messages.
void load_worker_gguf_output_head(const OutputHeadConfig &cfg, bool owns_final_layer);
bool worker_gguf_output_head_enabled();
bool worker_gguf_sample_token_enabled();
// maybe_forward_worker_gguf_output_head (:342-383): nullopt without a head
// or for another block; else the last position's RMS-normalised hidden
// state times the lm_head -- F16 logits [1, vocab] -- or, with
// --worker-gguf-sample-token, the token sample_remote_logits draws.
struct OutputHeadResult {
  std::optional<Tensor> logits;
  std::optional<uint32_t> token;
};
std::optional<OutputHeadResult> maybe_forward_worker_gguf_output_head(const Tensor &x,
                                                                      std::optional<int64_t> final_request_block_idx,
                                                                      const SamplingRequest *sampling);

}  // namespace dial
