// Host-side operator layer above the dialq C ABI (see dial_host.hpp).
#include "dial_host.hpp"

#include <hip/hip_runtime_api.h>
#include <rocblas/rocblas.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <mutex>
#include <shared_mutex>
#include <sstream>

#include "dialq.h"
#include "gguf.hpp"
#include "sampling.hpp"

namespace dial {

namespace {

[[noreturn]] void bail(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw Error(buf);
}

void hip_ok(hipError_t e, const char *what) {
  if (e != hipSuccess) bail("%s failed: %s", what, hipGetErrorString(e));
}

std::mutex g_log_mu;
std::string g_last_warning;

void log_warn(const std::string &msg) {
  std::lock_guard<std::mutex> lk(g_log_mu);
  g_last_warning = msg;
  if (getenv("DIAL_LOG")) fprintf(stderr, "[WARN] %s\n", msg.c_str());
}
void log_info(const std::string &msg) {
  if (getenv("DIAL_LOG")) fprintf(stderr, "[INFO] %s\n", msg.c_str());
}

int dialq_dtype_of(DType t) {
  switch (t) {
    case DType::F32: return DIALQ_F32;
    case DType::F16: return DIALQ_F16;
    case DType::BF16: return DIALQ_BF16;
    default: bail("dtype %s has no dialq equivalent", dtype_name(t));
  }
}

// Format conversions of checkpoint values at load time (bit level).
float f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = s;
    } else {  // subnormal: m * 2^-24
      float f = (float)m * 5.9604644775390625e-08f;
      uint32_t fb;
      std::memcpy(&fb, &f, 4);
      bits = s | fb;
    }
  } else if (e == 31) {
    bits = s | 0x7f800000u | (m << 13);
  } else {
    bits = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}
// f32 -> f16, round to nearest even (overflow to inf, NaN kept quiet).
uint16_t f32_to_f16_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 rounds to inf
  if (ax < 0x38800000u) {  // below 2^-14: subnormal steps of 2^-24
    float v;
    std::memcpy(&v, &ax, 4);
    return (uint16_t)(sign | (uint32_t)std::nearbyint(v * 16777216.0f));
  }
  uint32_t r = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}
float bf16_to_f32(uint16_t h) {
  const uint32_t bits = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// Host values of a float tensor (F32 / F16 / BF16) as f32.
std::vector<float> values_f32(const Tensor &t) {
  const std::vector<uint8_t> b = t.host_bytes();
  const int64_t n = t.elem_count();
  std::vector<float> v((size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    switch (t.dtype()) {
      case DType::F32: std::memcpy(&v[i], b.data() + 4 * i, 4); break;
      case DType::F16: { uint16_t h; std::memcpy(&h, b.data() + 2 * i, 2); v[i] = f16_to_f32(h); break; }
      case DType::BF16: { uint16_t h; std::memcpy(&h, b.data() + 2 * i, 2); v[i] = bf16_to_f32(h); break; }
      default: bail("expected a float tensor, got %s", dtype_name(t.dtype()));
    }
  }
  return v;
}

// E4M3FN value of each code (OCP; 0x7f / 0xff are NaN).
const float *e4m3_table() {
  static float tab[256];
  static std::once_flag once;
  std::call_once(once, [] {
    for (int c = 0; c < 256; ++c) {
      const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
      float v;
      if (e == 15 && m == 7) v = NAN;
      else if (e == 0) v = std::ldexp((float)m, -9);
      else v = std::ldexp(1.0f + (float)m / 8.0f, e - 7);
      tab[c] = s ? -v : v;
    }
  });
  return tab;
}

// Raw E4M3 bytes of a tensor: U8 tensors are the bytes themselves
// (candle F8E4M3 storage); float tensors must hold E4M3 values exactly
// (candle's to_dtype(F8E4M3) of such values is lossless), else an error.
std::vector<uint8_t> e4m3_bytes(const Tensor &t, const std::string &what) {
  if (t.dtype() == DType::U8) return t.host_bytes();
  const std::vector<float> v = values_f32(t);
  const float *tab = e4m3_table();
  std::vector<uint8_t> out(v.size());
  for (size_t i = 0; i < v.size(); ++i) {
    int found = -1;
    for (int c = 0; c < 256 && found < 0; ++c)
      if (tab[c] == v[i] && (v[i] != 0.0f || std::signbit(tab[c]) == std::signbit(v[i]))) found = c;
    if (found < 0) bail("%s value %g is not representable in E4M3", what.c_str(), (double)v[i]);
    out[i] = (uint8_t)found;
  }
  return out;
}

rocblas_handle blas_handle(int device) {
  static std::mutex mu;
  static std::map<int, rocblas_handle> handles;
  std::lock_guard<std::mutex> lk(mu);
  auto it = handles.find(device);
  if (it != handles.end()) return it->second;
  rocblas_handle h;
  if (rocblas_create_handle(&h) != rocblas_status_success) bail("rocblas_create_handle failed");
  handles[device] = h;
  return h;
}

struct DeviceScope {
  int prev = 0;
  explicit DeviceScope(const Device &d) {
    hip_ok(hipGetDevice(&prev), "hipGetDevice");
    if (d.is_rocm() && d.ordinal != prev) hip_ok(hipSetDevice(d.ordinal), "hipSetDevice");
  }
  ~DeviceScope() { (void)hipSetDevice(prev); }
};

}  // namespace

uint16_t f32_to_f16_bits(float f) { return f32_to_f16_rne(f); }

// ---- basics ---------------------------------------------------------------
const char *dtype_name(DType t) {
  switch (t) {
    case DType::F32: return "F32";
    case DType::F16: return "F16";
    case DType::BF16: return "BF16";
    case DType::U8: return "U8";
  }
  return "?";
}
size_t dtype_size(DType t) { return t == DType::F32 ? 4 : (t == DType::U8 ? 1 : 2); }

std::string Device::debug() const {
  return kind == Cpu ? std::string("Cpu") : "Rocm(" + std::to_string(ordinal) + ")";
}

std::string last_warning() {
  std::lock_guard<std::mutex> lk(g_log_mu);
  return g_last_warning;
}

int64_t Tensor::elem_count() const {
  int64_t n = 1;
  for (int64_t d : dims_) n *= d;
  return n;
}

std::string Tensor::dims_debug() const {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < dims_.size(); ++i) o << (i ? ", " : "") << dims_[i];
  o << "]";
  return o.str();
}

Tensor Tensor::empty(DType dtype, std::vector<int64_t> dims, Device device) {
  Tensor t;
  t.dtype_ = dtype;
  t.dims_ = std::move(dims);
  t.device_ = device;
  const size_t n = std::max<size_t>(t.nbytes(), 1);
  if (device.is_rocm()) {
    DeviceScope ds(device);
    void *p = nullptr;
    hip_ok(hipMalloc(&p, n), "hipMalloc");
    t.ptr_ = std::shared_ptr<uint8_t>((uint8_t *)p, [](uint8_t *q) { (void)hipFree(q); });
  } else {
    t.ptr_ = std::shared_ptr<uint8_t>(new uint8_t[n](), std::default_delete<uint8_t[]>());
  }
  return t;
}

Tensor Tensor::from_host(const void *data, DType dtype, std::vector<int64_t> dims) {
  Tensor t = empty(dtype, std::move(dims), Device::cpu());
  if (t.nbytes()) std::memcpy(t.data(), data, t.nbytes());
  return t;
}

Tensor Tensor::to_device(Device device) const {
  if (device == device_) return *this;
  Tensor t = empty(dtype_, dims_, device);
  if (!nbytes()) return t;
  if (device.is_rocm() && !device_.is_rocm()) {
    DeviceScope ds(device);
    hip_ok(hipMemcpy(t.data(), data(), nbytes(), hipMemcpyHostToDevice), "hipMemcpy H2D");
  } else if (!device.is_rocm() && device_.is_rocm()) {
    DeviceScope ds(device_);
    hip_ok(hipMemcpy(t.data(), data(), nbytes(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
  } else {
    hip_ok(hipMemcpy(t.data(), data(), nbytes(), hipMemcpyDeviceToDevice), "hipMemcpy D2D");
  }
  return t;
}

std::vector<uint8_t> Tensor::host_bytes() const {
  std::vector<uint8_t> out(nbytes());
  if (out.empty()) return out;
  if (device_.is_rocm()) {
    DeviceScope ds(device_);
    hip_ok(hipMemcpy(out.data(), data(), nbytes(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
  } else {
    std::memcpy(out.data(), data(), nbytes());
  }
  return out;
}

Tensor Tensor::reshape(std::vector<int64_t> dims) const {
  Tensor t = *this;
  t.dims_ = std::move(dims);
  if (t.elem_count() != elem_count()) bail("cannot reshape %s to %s", dims_debug().c_str(), t.dims_debug().c_str());
  return t;
}

// ---- Linear (dense, rocBLAS) -------------------------------------------------
Linear::Linear(Tensor weight, std::optional<Tensor> bias) : weight_(std::move(weight)), bias_(std::move(bias)) {}

Tensor Linear::forward(const Tensor &x) const {
  if (bias_) bail("dense linear with bias is not part of the quantized-linear path");
  if (!weight_.device().is_rocm() || !x.device().is_rocm()) bail("dense linear runs on a ROCm device");
  if (weight_.dims().size() != 2) bail("linear weight must be 2-D, got %s", weight_.dims_debug().c_str());
  const int64_t n = weight_.dims()[0], k = weight_.dims()[1];
  if (x.dims().empty() || x.dims().back() != k)
    bail("shape mismatch in linear: x %s, weight %s", x.dims_debug().c_str(), weight_.dims_debug().c_str());
  if (x.dtype() != weight_.dtype())
    bail("dtype mismatch in linear: x %s, weight %s", dtype_name(x.dtype()), dtype_name(weight_.dtype()));
  const int64_t m = x.elem_count() / k;
  std::vector<int64_t> od = x.dims();
  od.back() = n;
  Tensor y = Tensor::empty(x.dtype(), od, x.device());
  if (m == 0) return y;
  rocblas_datatype t;
  switch (x.dtype()) {
    case DType::F16: t = rocblas_datatype_f16_r; break;
    case DType::BF16: t = rocblas_datatype_bf16_r; break;
    case DType::F32: t = rocblas_datatype_f32_r; break;
    default: bail("dense linear does not support %s", dtype_name(x.dtype()));
  }
  DeviceScope ds(x.device());
  const float alpha = 1.0f, beta = 0.0f;
  // row-major y[m,n] = x[m,k] W[n,k]^T  ==  column-major y^T = W^T' x^T
  const rocblas_status st = rocblas_gemm_ex(
      blas_handle(x.device().ordinal), rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)n,
      (rocblas_int)m, (rocblas_int)k, &alpha, weight_.data(), t, (rocblas_int)k, x.data(), t, (rocblas_int)k, &beta,
      y.data(), t, (rocblas_int)n, y.data(), t, (rocblas_int)n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0,
      0);
  if (st != rocblas_status_success) bail("rocblas_gemm_ex failed: %s", rocblas_status_to_string(st));
  return y;
}

// ---- VarStore ---------------------------------------------------------------
std::string VarStore::full(const std::string &name) const { return prefix_.empty() ? name : prefix_ + "." + name; }
void VarStore::insert(const std::string &full_name, Tensor t) { (*tensors_)[full_name] = std::move(t); }
VarStore VarStore::pp(const std::string &sub) const {
  VarStore v = *this;
  v.prefix_ = full(sub);
  return v;
}
bool VarStore::contains_tensor(const std::string &name) const { return tensors_->count(full(name)) != 0; }
const Tensor &VarStore::get(const std::string &name) const {
  auto it = tensors_->find(full(name));
  if (it == tensors_->end()) bail("cannot find tensor %s", full(name).c_str());
  return it->second;
}

// ---- libdialq handles -------------------------------------------------------
struct DialqHandle {
  void *h = nullptr;
  int device = 0;
  ~DialqHandle() {
    if (h) dialq_linear_destroy(h);
  }
};

namespace {

std::shared_ptr<DialqHandle> dq_create(int fmt, int scale_dtype, int64_t out_dim, int64_t in_dim, float global,
                                       int flags, const void *w, size_t wb, const void *s, size_t sb, Device dev) {
  dialq_linear_desc d{fmt, scale_dtype, out_dim, in_dim, global, flags};
  char err[512];
  void *h = dialq_linear_create(&d, w, wb, s, sb, dev.ordinal, 1, nullptr, err, sizeof err);
  if (!h) throw Error(err);
  auto r = std::make_shared<DialqHandle>();
  r->h = h;
  r->device = dev.ordinal;
  return r;
}

std::shared_ptr<DialqHandle> dq_quantize(int fmt, int scale_dtype, const Tensor &dense, Device dev) {
  if (dense.dims().size() != 2) bail("quantizer expects a 2-D weight, got %s", dense.dims_debug().c_str());
  dialq_linear_desc d{fmt, scale_dtype, dense.dims()[0], dense.dims()[1], 1.0f, 0};
  char err[512];
  const bool host = !dense.device().is_rocm();
  void *h = dialq_linear_quantize(&d, dense.data(), dialq_dtype_of(dense.dtype()), dev.ordinal, host ? 1 : 0,
                                  nullptr, err, sizeof err);
  if (!h) throw Error(err);
  auto r = std::make_shared<DialqHandle>();
  r->h = h;
  r->device = dev.ordinal;
  return r;
}

// y[.., N] = x[.., K] W^T through the handle; output dtype = input dtype.
Tensor dq_forward(const DialqHandle &h, const Tensor &x, int64_t in_dim, int64_t out_dim) {
  const int64_t rows = x.elem_count() / in_dim;
  std::vector<int64_t> od = x.dims();
  od.back() = out_dim;
  Tensor y = Tensor::empty(x.dtype(), od, x.device());
  char err[512];
  const int rc = dialq_linear_forward(h.h, x.data(), dialq_dtype_of(x.dtype()), rows, y.data(),
                                      dialq_dtype_of(x.dtype()), nullptr, 1, err, sizeof err);
  if (rc != 0) throw Error(err);
  return y;
}

Tensor dq_dequantize(const DialqHandle &h, DType dtype, int64_t out_dim, int64_t in_dim, Device dev) {
  Tensor w = Tensor::empty(dtype, {out_dim, in_dim}, dev);
  char err[512];
  if (dialq_linear_dequantize(h.h, w.data(), dialq_dtype_of(dtype), nullptr, 1, err, sizeof err) != 0)
    throw Error(err);
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return w;
}

void check_rocm_input(const Tensor &x, const char *what) {
  if (!x.device().is_rocm()) bail("%s is only available on ROCm", what);
  if (x.dtype() == DType::U8) bail("%s expects F16, BF16 or F32 input, got %s", what, dtype_name(x.dtype()));
}

}  // namespace

// ---- RocmQuantLinear (CudaQuantLinear, cuda_quant.rs:289-391) ---------------
std::shared_ptr<RocmQuantLinear> RocmQuantLinear::nvfp4(const std::vector<uint8_t> &packed,
                                                        const std::vector<uint8_t> &scales, float global_scale,
                                                        int64_t in_dim, int64_t out_dim, Device device) {
  if (!device.is_rocm()) bail("NVFP4 QuantLinear requires ROCm");
  // in_dim % 16, packed and scale lengths are checked by dialq_linear_create
  // with the reference's messages.
  auto r = std::make_shared<RocmQuantLinear>();
  r->h_ = dq_create(DIALQ_FORMAT_NVFP4, DIALQ_F32, out_dim, in_dim, global_scale, 0, packed.data(), packed.size(),
                    scales.data(), scales.size(), device);
  r->in_dim_ = in_dim;
  r->out_dim_ = out_dim;
  return r;
}

std::shared_ptr<RocmQuantLinear> RocmQuantLinear::fp8(const std::vector<uint8_t> &weight,
                                                      const std::vector<float> &scales, int64_t in_dim,
                                                      int64_t out_dim, Device device) {
  if (!device.is_rocm()) bail("FP8 QuantLinear requires ROCm");
  if (weight.size() != (size_t)(out_dim * in_dim)) bail("invalid FP8 weight length %zu", weight.size());
  if (scales.size() != (size_t)out_dim) bail("invalid FP8 scale length %zu", scales.size());
  auto r = std::make_shared<RocmQuantLinear>();
  r->h_ = dq_create(DIALQ_FORMAT_FP8_ROW, DIALQ_F32, out_dim, in_dim, 1.0f, 0, weight.data(), weight.size(),
                    scales.data(), scales.size() * sizeof(float), device);
  r->in_dim_ = in_dim;
  r->out_dim_ = out_dim;
  return r;
}

size_t RocmQuantLinear::resident_bytes() const { return (size_t)dialq_linear_resident_bytes(h_->h); }

Tensor RocmQuantLinear::forward(const Tensor &x) const {
  check_rocm_input(x, "Qwen3.8 QuantLinear");
  if (x.dims().empty() || x.dims().back() != in_dim_)
    bail("Qwen3.8 QuantLinear expected last dim %lld, got %s", (long long)in_dim_, x.dims_debug().c_str());
  return dq_forward(*h_, x, in_dim_, out_dim_);
}

// ---- QuantLinear (quant.rs:20-139) ------------------------------------------
QuantLinear QuantLinear::dense(Linear l) {
  QuantLinear q;
  q.dense_ = std::move(l);
  return q;
}
QuantLinear QuantLinear::rocm(std::shared_ptr<RocmQuantLinear> l) {
  QuantLinear q;
  q.rocm_ = std::move(l);
  return q;
}
Tensor QuantLinear::forward(const Tensor &input) const {
  return rocm_ ? rocm_->forward(input) : dense_->forward(input);
}
const Linear &QuantLinear::dense_linear() const {
  if (!dense_) bail("expected the dense fallback");
  return *dense_;
}

namespace {
constexpr uint8_t QUANT_DENSE = 0, QUANT_ROCM_AUTO = 1, QUANT_ROCM_REQUIRED = 2;
std::atomic<uint8_t> g_quant_mode{QUANT_DENSE};
std::atomic<size_t> g_quant_count{0}, g_quant_bytes{0};

void register_rocm_quant_linear(const std::string &name, size_t bytes) {
  const size_t count = g_quant_count.fetch_add(1) + 1;
  const size_t total = g_quant_bytes.fetch_add(bytes) + bytes;
  if (count == 1 || count % 32 == 0) {
    char b[256];
    snprintf(b, sizeof b, "Qwen3.8 ROCm QuantLinear progress: last=%s linears=%zu resident=%.1f MiB", name.c_str(),
             count, total / 1048576.0);
    log_info(b);
  }
}

// try_cuda_nvfp4 (quant.rs:381-423)
std::shared_ptr<RocmQuantLinear> try_rocm_nvfp4(int64_t input_size, int64_t output_size, const VarStore &vb) {
  std::string weight_name, global_name;
  bool invert = false;
  if (vb.contains_tensor("weight_packed") && vb.contains_tensor("weight_global_scale")) {
    weight_name = "weight_packed";
    global_name = "weight_global_scale";
    invert = true;
  } else if (vb.contains_tensor("weight_scale_2")) {
    weight_name = "weight";
    global_name = "weight_scale_2";
  } else {
    bail("%s is not an NVFP4 linear", vb.prefix().c_str());
  }
  const Tensor &packed = vb.get(weight_name);
  if (packed.dtype() != DType::U8) bail("%s.%s must be U8 packed E2M1", vb.prefix().c_str(), weight_name.c_str());
  const std::vector<uint8_t> scales = e4m3_bytes(vb.get("weight_scale"), vb.prefix() + ".weight_scale");
  const std::vector<float> global = values_f32(vb.get(global_name));
  if (global.size() != 1 || global[0] == 0.0f) {
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < global.size(); ++i) o << (i ? ", " : "") << global[i];
    o << "]";
    bail("%s %s must contain one non-zero value, got %s", vb.prefix().c_str(), global_name.c_str(), o.str().c_str());
  }
  const float g = invert ? 1.0f / global[0] : global[0];
  return RocmQuantLinear::nvfp4(packed.host_bytes(), scales, g, input_size, output_size, vb.device());
}

// try_cuda_fp8 (quant.rs:425-447)
std::shared_ptr<RocmQuantLinear> try_rocm_fp8(int64_t input_size, int64_t output_size, const VarStore &vb) {
  const std::vector<uint8_t> weight = e4m3_bytes(vb.get("weight"), vb.prefix() + ".weight");
  std::vector<float> scales = values_f32(vb.get("weight_scale"));
  if (scales.size() == 1) scales.assign((size_t)output_size, scales[0]);
  else if ((int64_t)scales.size() != output_size)
    bail("FP8 weight_scale for %s contains %zu values, expected 1 or %lld", vb.prefix().c_str(), scales.size(),
         (long long)output_size);
  return RocmQuantLinear::fp8(weight, scales, input_size, output_size, vb.device());
}

// Dense fallbacks (load_nvfp4 / load_compressed_tensors_nvfp4 / load_fp8 /
// load_tensor, quant.rs:252-379): decoded on the GPU by libdialq into the
// runtime dtype.
Tensor load_nvfp4_dense(const VarStore &vb, int64_t input_size, int64_t output_size, const std::string &weight_name,
                        const std::string &global_name, bool divisor) {
  const Tensor &packed = vb.get(weight_name);
  const std::vector<float> global = values_f32(vb.get(global_name));
  if (global.size() != 1) {
    if (divisor)
      bail("compressed-tensors weight_global_scale for %s contains %zu values, expected 1", vb.prefix().c_str(),
           global.size());
    bail("NVFP4 weight_scale_2 for %s contains %zu values, expected 1", vb.prefix().c_str(), global.size());
  }
  if (divisor && global[0] == 0.0f)
    bail("compressed-tensors weight_global_scale for %s is zero", vb.prefix().c_str());
  if (input_size % 16 != 0)
    bail("NVFP4 input dimension %lld is not divisible by group size 16", (long long)input_size);
  const std::vector<uint8_t> pk = packed.host_bytes();
  const int64_t expected_packed = output_size * input_size / 2;
  if ((int64_t)pk.size() != expected_packed)
    bail("NVFP4 packed weight has %zu bytes, expected %lld", pk.size(), (long long)expected_packed);
  const Tensor &sc = vb.get("weight_scale");
  const int64_t expected_scales = output_size * (input_size / 16);
  if (sc.elem_count() != expected_scales)
    bail("NVFP4 weight scale has %lld values, expected %lld", (long long)sc.elem_count(), (long long)expected_scales);
  const std::vector<uint8_t> scales = e4m3_bytes(sc, vb.prefix() + ".weight_scale");
  const Device dev = vb.device().is_rocm() ? vb.device() : Device::rocm(0);
  auto h = dq_create(DIALQ_FORMAT_NVFP4, DIALQ_F32, output_size, input_size, global[0],
                     divisor ? DIALQ_FLAG_GLOBAL_IS_DIVISOR : 0, pk.data(), pk.size(), scales.data(), scales.size(),
                     dev);
  return dq_dequantize(*h, vb.dtype(), output_size, input_size, dev);
}

Tensor load_fp8_dense(const VarStore &vb, int64_t input_size, int64_t output_size) {
  std::vector<uint8_t> weight = e4m3_bytes(vb.get("weight"), vb.prefix() + ".weight");
  if ((int64_t)weight.size() != output_size * input_size)
    bail("shape mismatch for %s.weight, expected [%lld, %lld]", vb.prefix().c_str(), (long long)output_size,
         (long long)input_size);
  std::vector<float> scales = values_f32(vb.get("weight_scale"));
  if (scales.size() == 1) scales.assign((size_t)output_size, scales[0]);
  else if ((int64_t)scales.size() != output_size)
    bail("FP8 weight_scale for %s contains %zu values, expected 1 or %lld", vb.prefix().c_str(), scales.size(),
         (long long)output_size);
  const Device dev = vb.device().is_rocm() ? vb.device() : Device::rocm(0);
  // The device format wants in_dim % 8 == 0; pad each row with zero codes
  // and keep the first input_size columns of the decoded weight.
  const int64_t kp = (input_size + 7) / 8 * 8;
  if (kp != input_size) {
    std::vector<uint8_t> padded((size_t)(output_size * kp), 0);
    for (int64_t r = 0; r < output_size; ++r)
      std::memcpy(&padded[(size_t)(r * kp)], &weight[(size_t)(r * input_size)], (size_t)input_size);
    weight.swap(padded);
  }
  auto h = dq_create(DIALQ_FORMAT_FP8_ROW, DIALQ_F32, output_size, kp, 1.0f, 0, weight.data(), weight.size(),
                     scales.data(), scales.size() * sizeof(float), dev);
  Tensor full = dq_dequantize(*h, vb.dtype(), output_size, kp, dev);
  if (kp == input_size) return full;
  Tensor w = Tensor::empty(vb.dtype(), {output_size, input_size}, dev);
  const size_t es = dtype_size(vb.dtype());
  DeviceScope ds(dev);
  hip_ok(hipMemcpy2D(w.data(), (size_t)input_size * es, full.data(), (size_t)kp * es, (size_t)input_size * es,
                     (size_t)output_size, hipMemcpyDeviceToDevice),
         "hipMemcpy2D");
  return w;
}
}  // namespace

void configure_quant_linear(Qwen38QuantLinear requested, Device device, DType dtype) {
  const bool supported_runtime = device.is_rocm() && (dtype == DType::F16 || dtype == DType::BF16);
  uint8_t mode;
  switch (requested) {
    case Qwen38QuantLinear::Dense: mode = QUANT_DENSE; break;
    case Qwen38QuantLinear::Auto: mode = supported_runtime ? QUANT_ROCM_AUTO : QUANT_DENSE; break;
    case Qwen38QuantLinear::Rocm:
      if (!supported_runtime)
        bail("--qwen38-quant-linear rocm requires a ROCm device and --dtype f16 or bf16 (device=%s, dtype=%s)",
             device.debug().c_str(), dtype_name(dtype));
      mode = QUANT_ROCM_REQUIRED;
      break;
    default: mode = QUANT_DENSE;
  }
  g_quant_mode.store(mode);
  g_quant_count.store(0);
  g_quant_bytes.store(0);
  if (mode == QUANT_DENSE) log_info("Qwen3.8 QuantLinear: dense compatibility mode");
  else if (mode == QUANT_ROCM_AUTO)
    log_info("Qwen3.8 QuantLinear: ROCm auto W4A16/W8A16 mode (quantized weights remain device-resident)");
  else log_info("Qwen3.8 QuantLinear: ROCm W4A16/W8A16 required mode (startup fails instead of dense fallback)");
}

std::optional<std::pair<size_t, size_t>> quant_linear_summary() {
  if (g_quant_mode.load() == QUANT_DENSE) return std::nullopt;
  return std::make_pair(g_quant_count.load(), g_quant_bytes.load());
}

// linear_no_bias (quant.rs:466-519)
QuantLinear linear_no_bias(int64_t input_size, int64_t output_size, const VarStore &vb) {
  const uint8_t mode = g_quant_mode.load();
  const bool is_nvfp4 = (vb.contains_tensor("weight_packed") && vb.contains_tensor("weight_global_scale")) ||
                        vb.contains_tensor("weight_scale_2");
  const bool is_fp8 = !is_nvfp4 && vb.contains_tensor("weight_scale");
  if (mode != QUANT_DENSE && (is_nvfp4 || is_fp8)) {
    try {
      auto linear = is_nvfp4 ? try_rocm_nvfp4(input_size, output_size, vb) : try_rocm_fp8(input_size, output_size, vb);
      register_rocm_quant_linear(vb.prefix(), linear->resident_bytes());
      return QuantLinear::rocm(linear);
    } catch (const Error &e) {
      if (mode == QUANT_ROCM_REQUIRED) throw;
      g_quant_mode.store(QUANT_DENSE);
      log_warn("Qwen3.8 ROCm QuantLinear unavailable for " + vb.prefix() + ": " + e.what() +
               "; disabling it for this process and using dense fallback");
    }
  }
  Tensor weight;
  if (vb.contains_tensor("weight_packed") && vb.contains_tensor("weight_global_scale")) {
    weight = load_nvfp4_dense(vb, input_size, output_size, "weight_packed", "weight_global_scale", true);
  } else if (vb.contains_tensor("weight_scale_2")) {
    weight = load_nvfp4_dense(vb, input_size, output_size, "weight", "weight_scale_2", false);
  } else if (vb.contains_tensor("weight_scale")) {
    weight = load_fp8_dense(vb, input_size, output_size);
  } else {
    const Tensor &w = vb.get("weight");
    if (w.dims() != std::vector<int64_t>{output_size, input_size})
      bail("shape mismatch for %s.weight, expected [%lld, %lld], got %s", vb.prefix().c_str(),
           (long long)output_size, (long long)input_size, w.dims_debug().c_str());
    if (w.dtype() != vb.dtype()) bail("%s.weight is %s, runtime dtype is %s", vb.prefix().c_str(),
                                      dtype_name(w.dtype()), dtype_name(vb.dtype()));
    weight = w.to_device(vb.device().is_rocm() ? vb.device() : Device::rocm(0));
  }
  return QuantLinear::dense(Linear(weight));
}

// ---- worker W8A16 (worker_w8a16.rs) -----------------------------------------
namespace {
std::atomic<bool> g_w8a16_enabled{false};
std::atomic<size_t> g_w8a16_count{0}, g_w8a16_bytes{0};
std::atomic<bool> g_gguf_fp16_prefill{false};
}  // namespace

void configure_worker_w8a16_from_args(bool requested, bool worker_mode, Device device, DType dtype) {
  const bool gguf = worker_gguf_enabled();
  const bool supported_dtype = dtype == DType::F16 || dtype == DType::BF16;
  const bool enabled = requested && !gguf && worker_mode && device.is_rocm() && supported_dtype;
  g_w8a16_enabled.store(enabled);
  if (requested && gguf)
    log_warn("both worker W8A16 and GGUF were requested; GGUF takes precedence and W8A16 is disabled");
  else if (requested && !worker_mode) log_info("worker W8A16 ignored in master mode; master weights remain unchanged");
  else if (requested && !device.is_rocm())
    log_warn("worker W8A16 requested on a non-ROCm device; falling back to dense weights");
  else if (requested && !supported_dtype)
    log_warn(std::string("worker W8A16 requires --dtype f16 or bf16 (got ") + dtype_name(dtype) +
             "); falling back to dense weights");
  else if (enabled)
    log_info("worker W8A16 enabled: ROCm linear weights use row-wise int8, activations/outputs keep their dtype");
}

bool worker_w8a16_enabled() { return g_w8a16_enabled.load(); }

std::optional<std::pair<size_t, size_t>> worker_w8a16_summary() {
  if (!worker_w8a16_enabled()) return std::nullopt;
  return std::make_pair(g_w8a16_count.load(), g_w8a16_bytes.load());
}

std::shared_ptr<W8A16Linear> W8A16Linear::from_linear(const std::string &name, const Linear &linear) {
  if (linear.bias()) bail("W8A16 only supports bias-free linear layers");
  const Tensor &w = linear.weight();
  if (w.dtype() != DType::F16 && w.dtype() != DType::BF16)
    bail("expected F16 weight, got %s", dtype_name(w.dtype()));
  if (!w.device().is_rocm()) bail("W8A16 ROCm linear requires a ROCm weight tensor");
  if (w.dims().size() != 2) bail("W8A16 weight must be 2-D, got %s", w.dims_debug().c_str());
  auto r = std::make_shared<W8A16Linear>();
  // f32 scales, as CudaW8A16Linear keeps them (worker_w8a16.rs:321-351)
  r->h_ = dq_quantize(DIALQ_FORMAT_W8A16, DIALQ_F32, w, w.device());
  r->out_dim_ = w.dims()[0];
  r->in_dim_ = w.dims()[1];
  const size_t bytes = r->resident_bytes();
  const size_t count = g_w8a16_count.fetch_add(1) + 1;
  g_w8a16_bytes.fetch_add(bytes);
  if (count == 1 || count % 32 == 0) log_info("worker W8A16 converted " + name);
  return r;
}

size_t W8A16Linear::resident_bytes() const { return (size_t)dialq_linear_resident_bytes(h_->h); }

Tensor W8A16Linear::forward(const Tensor &x) const {
  if (x.dtype() != DType::F16 && x.dtype() != DType::BF16)
    bail("W8A16 expects F16 activation, got %s", dtype_name(x.dtype()));
  if (!x.device().is_rocm()) bail("W8A16 linear is only available on ROCm");
  if (x.dims().empty() || x.dims().back() != in_dim_)
    bail("W8A16 input mismatch: expected last dim %lld, got %s", (long long)in_dim_, x.dims_debug().c_str());
  return dq_forward(*h_, x, in_dim_, out_dim_);
}

// ---- GGUF (worker_gguf.rs) --------------------------------------------------
std::shared_ptr<GgufMatMul> GgufMatMul::from_blocks(Kind kind, const std::vector<uint8_t> &blocks, int64_t out_dim,
                                                    int64_t in_dim, Device device) {
  if (!device.is_rocm()) bail("GGUF QMatMul requires a ROCm device");
  auto r = std::make_shared<GgufMatMul>();
  r->h_ = dq_create((int)kind, DIALQ_F32, out_dim, in_dim, 1.0f, 0, blocks.data(), blocks.size(), nullptr, 0, device);
  r->out_dim_ = out_dim;
  r->in_dim_ = in_dim;
  return r;
}

std::shared_ptr<GgufMatMul> GgufMatMul::from_device_blocks(Kind kind, const Tensor &blocks, int64_t out_dim,
                                                           int64_t in_dim) {
  if (!blocks.device().is_rocm()) bail("GGUF device blocks must be on a ROCm device");
  auto r = std::make_shared<GgufMatMul>();
  dialq_linear_desc d{(int)kind, DIALQ_F32, out_dim, in_dim, 1.0f, 0};
  char err[512];
  void *h = dialq_linear_create(&d, blocks.data(), blocks.nbytes(), nullptr, 0, blocks.device().ordinal, 0, nullptr,
                                err, sizeof err);
  if (!h) throw Error(err);
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");  // the repack has read `blocks`
  r->h_ = std::make_shared<DialqHandle>();
  r->h_->h = h;
  r->h_->device = blocks.device().ordinal;
  r->out_dim_ = out_dim;
  r->in_dim_ = in_dim;
  return r;
}

std::shared_ptr<GgufMatMul> GgufMatMul::quantize(Kind kind, const Tensor &dense, Device device) {
  if (!device.is_rocm()) bail("GGUF QMatMul requires a ROCm device");
  auto r = std::make_shared<GgufMatMul>();
  r->h_ = dq_quantize((int)kind, DIALQ_F32, dense, device);
  r->out_dim_ = dense.dims()[0];
  r->in_dim_ = dense.dims()[1];
  return r;
}

Tensor GgufMatMul::forward(const Tensor &x) const {
  check_rocm_input(x, "GGUF QMatMul");
  if (x.dims().empty() || x.dims().back() != in_dim_)
    bail("shape mismatch in GGUF matmul: x %s, weight [%lld, %lld]", x.dims_debug().c_str(), (long long)out_dim_,
         (long long)in_dim_);
  return dq_forward(*h_, x, in_dim_, out_dim_);
}

Tensor GgufMatMul::dequantize_f16() const {
  return dq_dequantize(*h_, DType::F16, out_dim_, in_dim_, Device::rocm(h_->device));
}

// ---- GGUF worker source (worker_gguf.rs:19-25,65-197,388-397,462-572) -------
namespace {
struct WorkerGgufSource {
  std::string path;
  gguf::Content content;
  std::mutex file_mu;  // the file position is shared: reads are serialized
  std::ifstream file;
  Device device;
};
std::shared_mutex g_gguf_mu;
std::shared_ptr<WorkerGgufSource> g_gguf_source;
std::atomic<bool> g_gguf_output_head{false}, g_gguf_sample_token{false};
std::atomic<size_t> g_gguf_count{0}, g_gguf_bytes{0}, g_gguf_prefill_count{0}, g_gguf_prefill_bytes{0};
std::atomic<unsigned> g_gguf_warmed{0};
// Drops the loaded output head and re-arms its route log (defined with the
// head's state below).
void reset_output_head();

std::shared_ptr<WorkerGgufSource> gguf_source() {
  std::shared_lock<std::shared_mutex> lk(g_gguf_mu);
  return g_gguf_source;
}

// warmup_worker_gguf (worker_gguf.rs:524-572): the first linear of each GGUF
// dtype runs one F16 decode row and one 9-row F32 prefill, so the kernels'
// first-launch cost is paid at load time.  DIAL_WORKER_GGUF_WARMUP=0 (or
// false / FALSE / no / NO) skips it.
void warmup_worker_gguf(const GgufMatMul &mm, gguf::GgmlDType dtype, int64_t in_dim, Device device) {
  if (const char *e = getenv("DIAL_WORKER_GGUF_WARMUP")) {
    const std::string v = e;
    if (v == "0" || v == "false" || v == "FALSE" || v == "no" || v == "NO") return;
  }
  const unsigned bit = dtype == gguf::GgmlDType::Q4K ? 1u : dtype == gguf::GgmlDType::Q6K ? 2u : 4u;
  if (g_gguf_warmed.fetch_or(bit) & bit) return;
  try {
    std::vector<uint16_t> z16((size_t)in_dim, 0);
    Tensor decode = Tensor::from_host(z16.data(), DType::F16, {1, 1, in_dim}).to_device(device);
    Tensor out = forward_worker_gguf(mm, decode);
    if (out.dtype() != DType::F16)
      bail("GGUF F16 decode warmup returned %s, expected F16", dtype_name(out.dtype()));
    std::vector<float> z32((size_t)(9 * in_dim), 0.0f);
    Tensor prefill = Tensor::from_host(z32.data(), DType::F32, {1, 9, in_dim}).to_device(device);
    (void)mm.forward(prefill);
    DeviceScope ds(device);
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  } catch (...) {
    g_gguf_warmed.fetch_and(~bit);
    throw;
  }
  log_info(std::string("worker GGUF ROCm warmup complete: dtype=") + gguf::ggml_dtype_name(dtype) +
           " decode=F16/direct seq=1 fallback=F32 seq=9");
}
}  // namespace

void configure_worker_gguf_from_args(const std::optional<std::string> &path, bool fp16_prefill, bool output_head,
                                     bool sample_token, bool worker_mode, Device device, DType dtype,
                                     int64_t num_hidden_layers) {
  g_gguf_fp16_prefill.store(false);
  g_gguf_output_head.store(false);
  g_gguf_sample_token.store(false);
  {
    std::unique_lock<std::shared_mutex> lk(g_gguf_mu);
    g_gguf_source.reset();
  }
  // the reference clears the output-head slot and its route-logged flag on
  // every configure (worker_gguf.rs:78-84), so a reconfigure never keeps a
  // stale head (and its resident lm_head) routing logits
  reset_output_head();
  if (!worker_mode) {
    if (path || fp16_prefill || output_head || sample_token)
      log_info("worker GGUF options ignored in master mode; master weights remain unchanged");
    return;
  }
  if (!path) {
    if (fp16_prefill || output_head || sample_token)
      bail("--worker-gguf-fp16-prefill/--worker-gguf-output-head requires --worker-quantized-gguf");
    return;
  }
  if (!device.is_rocm()) bail("--worker-quantized-gguf currently requires a ROCm worker");
  if (dtype != DType::F16 && dtype != DType::BF16)
    bail("--worker-quantized-gguf requires --dtype f16 or bf16 so DIAL activation and KV-cache contracts remain "
         "unchanged");
  if (sample_token && !output_head)
    bail("--worker-gguf-sample-token true requires --worker-gguf-output-head true");

  auto src = std::make_shared<WorkerGgufSource>();
  src->path = *path;
  src->device = device;
  src->file.open(*path, std::ios::binary);
  if (!src->file) bail("cannot open worker GGUF %s: %s", path->c_str(), std::strerror(errno));
  try {
    src->file.seekg(0, std::ios::end);
    const uint64_t size = (uint64_t)src->file.tellg();
    src->file.seekg(0);
    src->content = gguf::Content::read(src->file, size);
  } catch (const Error &e) {
    bail("cannot parse worker GGUF %s: %s", path->c_str(), e.what());
  }
  const gguf::Value *arch = src->content.get("general.architecture");
  if (!arch) bail("worker GGUF %s is missing general.architecture", path->c_str());
  if (arch->type != gguf::ValueType::String || arch->s != "qwen3vl")
    bail("worker GGUF %s has unsupported architecture metadata %s; expected qwen3vl", path->c_str(),
         arch->debug().c_str());
  if (const gguf::Value *bc = src->content.get("qwen3vl.block_count")) {
    uint64_t block_count;
    try {
      block_count = bc->to_u64();
    } catch (const Error &e) {
      bail("invalid qwen3vl.block_count: %s", e.what());
    }
    if ((int64_t)block_count != num_hidden_layers)
      bail("worker GGUF block count %llu does not match Hugging Face config %lld", (unsigned long long)block_count,
           (long long)num_hidden_layers);
  }
  g_gguf_count.store(0);
  g_gguf_bytes.store(0);
  g_gguf_warmed.store(0);
  g_gguf_prefill_count.store(0);
  g_gguf_prefill_bytes.store(0);
  {
    std::unique_lock<std::shared_mutex> lk(g_gguf_mu);
    g_gguf_source = src;
  }
  g_gguf_fp16_prefill.store(fp16_prefill);
  g_gguf_output_head.store(output_head);
  g_gguf_sample_token.store(sample_token);
  log_info("worker GGUF enabled: file=" + *path + " format=Ollama/llama.cpp activations=" + dtype_name(dtype) +
           " kv_cache=" + dtype_name(dtype));
  if (fp16_prefill)
    log_info("worker GGUF hybrid enabled: prefill=fused-FP16 decode=GGUF (both resident; routing by sequence length)");
}

bool worker_gguf_enabled() { return (bool)gguf_source(); }
bool worker_gguf_fp16_prefill_enabled() { return g_gguf_fp16_prefill.load(); }
bool worker_gguf_output_head_requested() { return g_gguf_output_head.load(); }
bool worker_gguf_sample_token_requested() { return g_gguf_sample_token.load(); }

std::optional<std::tuple<size_t, size_t, size_t, size_t>> worker_gguf_summary() {
  if (!worker_gguf_enabled()) return std::nullopt;
  return std::make_tuple(g_gguf_count.load(), g_gguf_bytes.load(), g_gguf_prefill_count.load(),
                         g_gguf_prefill_bytes.load());
}

// Streams a GGUF tensor to the device in 8 MiB chunks (the host holds one
// chunk, as adapter.cpp:198-227 reads) and repacks it as a quantized matmul.
std::shared_ptr<GgufMatMul> upload_gguf_matmul(WorkerGgufSource &src, const std::string &name,
                                               const gguf::TensorInfo &info, int64_t out_dim, int64_t in_dim) {
  GgufMatMul::Kind kind;
  switch (info.ggml_dtype) {
    case gguf::GgmlDType::Q8_0: kind = GgufMatMul::Q8_0; break;
    case gguf::GgmlDType::Q4K: kind = GgufMatMul::Q4_K; break;
    case gguf::GgmlDType::Q6K: kind = GgufMatMul::Q6_K; break;
    default:
      bail("worker GGUF tensor %s has dtype %s; the ROCm GGUF path takes Q8_0, Q4K and Q6K", name.c_str(),
           gguf::ggml_dtype_name(info.ggml_dtype));
  }
  const size_t nbytes = (size_t)info.size_in_bytes();
  Tensor dev_blocks = Tensor::empty(DType::U8, {(int64_t)nbytes}, src.device);
  {
    std::lock_guard<std::mutex> lk(src.file_mu);
    DeviceScope ds(src.device);
    src.content.tensor_chunks(src.file, name, (size_t)8 << 20, [&](const uint8_t *p, size_t off, size_t n) {
      hip_ok(hipMemcpy((uint8_t *)dev_blocks.data() + off, p, n, hipMemcpyHostToDevice), "hipMemcpy");
    });
  }
  return GgufMatMul::from_device_blocks(kind, dev_blocks, out_dim, in_dim);
}

std::optional<TextLinear> load_worker_gguf_linear(std::optional<int64_t> layer_idx, const std::string &tensor_suffix,
                                                  int64_t in_dim, int64_t out_dim) {
  std::shared_ptr<WorkerGgufSource> src = gguf_source();
  if (!src) return std::nullopt;
  if (!layer_idx) bail("worker GGUF requires a numeric transformer layer name");
  const std::string name = "blk." + std::to_string(*layer_idx) + "." + tensor_suffix + ".weight";
  auto it = src->content.tensor_infos.find(name);
  if (it == src->content.tensor_infos.end())
    bail("worker GGUF %s has no tensor %s", src->path.c_str(), name.c_str());
  const gguf::TensorInfo &info = it->second;
  if (info.dims != std::vector<int64_t>{out_dim, in_dim}) {
    std::string d = "[";
    for (size_t i = 0; i < info.dims.size(); ++i) d += (i ? ", " : "") + std::to_string(info.dims[i]);
    bail("worker GGUF tensor %s shape %s], expected [%lld, %lld]", name.c_str(), d.c_str(), (long long)out_dim,
         (long long)in_dim);
  }
  std::shared_ptr<GgufMatMul> mm = upload_gguf_matmul(*src, name, info, out_dim, in_dim);
  warmup_worker_gguf(*mm, info.ggml_dtype, in_dim, src->device);
  g_gguf_count.fetch_add(1);
  g_gguf_bytes.fetch_add((size_t)info.size_in_bytes());
  log_info("loaded worker GGUF tensor " + name + " dtype=" + gguf::ggml_dtype_name(info.ggml_dtype));
  return TextLinear::gguf(name, mm);
}

// ---- worker GGUF output head (worker_gguf.rs:197-383) -------------------------
namespace {
struct OutputHead {
  std::vector<float> norm;  // output_norm.weight, F16 values (gguf_tensor_to_f16)
  double eps = 1e-6;
  std::shared_ptr<GgufMatMul> output;
  int64_t final_block_idx = 0;
  Device device;
};
std::shared_mutex g_head_mu;
std::shared_ptr<OutputHead> g_head;
std::atomic<bool> g_head_route_logged{false};

void reset_output_head() {
  {
    std::unique_lock<std::shared_mutex> lk(g_head_mu);
    g_head.reset();
  }
  g_head_route_logged.store(false);
}

std::shared_ptr<OutputHead> output_head() {
  std::shared_lock<std::shared_mutex> lk(g_head_mu);
  return g_head;
}

bool warmup_disabled() {
  const char *e = getenv("DIAL_WORKER_GGUF_WARMUP");
  if (!e) return false;
  const std::string v = e;
  return v == "0" || v == "false" || v == "FALSE" || v == "no" || v == "NO";
}

// forward_output_head (:333-345): the last position of [1, seq, hidden] (or
// the [1, hidden] row), candle_nn::RmsNorm -- f32 sum of squares, x * rsqrt(
// mean + eps) * w, rounded to the activation dtype -- then the lm_head.  The
// one hidden row is normalised on the host (a few KB each way per token).
Tensor forward_output_head(const OutputHead &head, const Tensor &x) {
  const std::vector<int64_t> &d = x.dims();
  int64_t row_off;
  if (d.size() == 3 && d[0] == 1 && d[1] > 0) row_off = (d[1] - 1) * d[2];
  else if (d.size() == 2 && d[0] == 1) row_off = 0;
  else bail("worker GGUF output head expects [1, seq, hidden] or [1, hidden], got %s", x.dims_debug().c_str());
  const int64_t hidden = d.back();
  if (hidden != (int64_t)head.norm.size())
    bail("worker GGUF output head: hidden size %lld, output_norm.weight has %lld", (long long)hidden,
         (long long)head.norm.size());
  if (x.dtype() != DType::F16 && x.dtype() != DType::BF16 && x.dtype() != DType::F32)
    bail("worker GGUF output head: unsupported activation dtype %s", dtype_name(x.dtype()));
  const size_t es = dtype_size(x.dtype());
  std::vector<uint8_t> row((size_t)hidden * es);
  const uint8_t *src = (const uint8_t *)x.data() + (size_t)row_off * es;
  if (x.device().is_rocm()) {
    DeviceScope ds(x.device());
    hip_ok(hipMemcpy(row.data(), src, row.size(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
  } else {
    std::memcpy(row.data(), src, row.size());
  }
  std::vector<float> v((size_t)hidden);
  for (int64_t i = 0; i < hidden; ++i) {
    uint16_t h;
    switch (x.dtype()) {
      case DType::F32: std::memcpy(&v[i], row.data() + 4 * i, 4); break;
      case DType::F16: std::memcpy(&h, row.data() + 2 * i, 2); v[i] = f16_to_f32(h); break;
      default: std::memcpy(&h, row.data() + 2 * i, 2); v[i] = bf16_to_f32(h); break;
    }
  }
  float ss = 0.0f;
  for (float a : v) ss += a * a;
  const float scale = 1.0f / std::sqrt(ss / (float)hidden + (float)head.eps);
  for (int64_t i = 0; i < hidden; ++i) {
    const float y = v[i] * scale * head.norm[i];
    switch (x.dtype()) {
      case DType::F32: std::memcpy(row.data() + 4 * i, &y, 4); break;
      case DType::F16: { const uint16_t h = f32_to_f16_rne(y); std::memcpy(row.data() + 2 * i, &h, 2); break; }
      default: {
        uint32_t b;
        std::memcpy(&b, &y, 4);
        const uint16_t h = std::isnan(y) ? (uint16_t)0x7fc0u : (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
        std::memcpy(row.data() + 2 * i, &h, 2);
        break;
      }
    }
  }
  Tensor normalized = Tensor::from_host(row.data(), x.dtype(), {1, hidden}).to_device(head.device);
  return forward_worker_gguf(*head.output, normalized);
}
}  // namespace

void load_worker_gguf_output_head(const OutputHeadConfig &cfg, bool owns_final_layer) {
  {
    std::unique_lock<std::shared_mutex> lk(g_head_mu);
    g_head.reset();
  }
  if (!worker_gguf_output_head_requested()) return;
  if (!owns_final_layer) {
    log_info("worker GGUF output head not loaded: this Worker does not own the final layer");
    return;
  }
  std::shared_ptr<WorkerGgufSource> src = gguf_source();
  if (!src) bail("worker GGUF source is not configured");
  const auto dims_str = [](const std::vector<int64_t> &dims) {
    std::string s = "[";
    for (size_t i = 0; i < dims.size(); ++i) s += (i ? ", " : "") + std::to_string(dims[i]);
    return s + "]";
  };
  const std::string norm_name = "output_norm.weight";
  auto ni = src->content.tensor_infos.find(norm_name);
  if (ni == src->content.tensor_infos.end())
    bail("worker GGUF %s has no tensor %s", src->path.c_str(), norm_name.c_str());
  if (ni->second.dims != std::vector<int64_t>{cfg.hidden_size})
    bail("worker GGUF tensor %s shape %s, expected [%lld]", norm_name.c_str(), dims_str(ni->second.dims).c_str(),
         (long long)cfg.hidden_size);
  std::string output_name;
  if (src->content.tensor_infos.count("output.weight")) {
    output_name = "output.weight";
  } else if (src->content.tensor_infos.count("token_embd.weight")) {
    log_info("worker GGUF output.weight missing; using tied token_embd.weight");
    output_name = "token_embd.weight";
  } else {
    bail("worker GGUF %s has neither output.weight nor token_embd.weight", src->path.c_str());
  }
  const gguf::TensorInfo &oi = src->content.tensor_infos.at(output_name);
  if (oi.dims != std::vector<int64_t>{cfg.vocab_size, cfg.hidden_size})
    bail("worker GGUF tensor %s shape %s, expected [%lld, %lld]", output_name.c_str(), dims_str(oi.dims).c_str(),
         (long long)cfg.vocab_size, (long long)cfg.hidden_size);

  auto head = std::make_shared<OutputHead>();
  const gguf::GgmlDType norm_dtype = ni->second.ggml_dtype;
  std::vector<uint8_t> nb;
  {
    std::lock_guard<std::mutex> lk(src->file_mu);
    nb = src->content.tensor_bytes(src->file, norm_name);
  }
  head->norm.resize((size_t)cfg.hidden_size);
  for (int64_t i = 0; i < cfg.hidden_size; ++i) {
    float f;
    uint16_t h;
    switch (norm_dtype) {
      case gguf::GgmlDType::F32: std::memcpy(&f, nb.data() + 4 * i, 4); break;
      case gguf::GgmlDType::F16: std::memcpy(&h, nb.data() + 2 * i, 2); f = f16_to_f32(h); break;
      case gguf::GgmlDType::BF16: std::memcpy(&h, nb.data() + 2 * i, 2); f = bf16_to_f32(h); break;
      default:
        bail("worker GGUF tensor %s has dtype %s; expected F32, F16 or BF16", norm_name.c_str(),
             gguf::ggml_dtype_name(norm_dtype));
    }
    head->norm[i] = f16_to_f32(f32_to_f16_rne(f));
  }
  head->eps = cfg.rms_norm_eps;
  head->output = upload_gguf_matmul(*src, output_name, oi, cfg.vocab_size, cfg.hidden_size);
  head->final_block_idx = cfg.num_hidden_layers > 0 ? cfg.num_hidden_layers - 1 : 0;
  head->device = src->device;
  warmup_worker_gguf(*head->output, oi.ggml_dtype, cfg.hidden_size, src->device);
  if (!warmup_disabled()) {
    std::vector<uint16_t> z((size_t)cfg.hidden_size, 0);
    Tensor hidden = Tensor::from_host(z.data(), DType::F16, {1, 1, cfg.hidden_size}).to_device(src->device);
    (void)forward_output_head(*head, hidden);
    DeviceScope ds(src->device);
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
    log_info("worker GGUF output head warmup complete");
  }
  {
    std::unique_lock<std::shared_mutex> lk(g_head_mu);
    g_head = head;
  }
  char msg[512];
  snprintf(msg, sizeof msg,
           "worker GGUF output head loaded: norm=%s norm_dtype=%s output=%s dtype=%s shape=[%lld, %lld] "
           "quantized_memory=%.1f MiB return_dtype=F16",
           norm_name.c_str(), gguf::ggml_dtype_name(norm_dtype), output_name.c_str(),
           gguf::ggml_dtype_name(oi.ggml_dtype), (long long)cfg.vocab_size, (long long)cfg.hidden_size,
           (double)oi.size_in_bytes() / 1048576.0);
  log_info(msg);
}

bool worker_gguf_output_head_enabled() { return (bool)output_head(); }
bool worker_gguf_sample_token_enabled() { return worker_gguf_output_head_enabled() && g_gguf_sample_token.load(); }

std::optional<OutputHeadResult> maybe_forward_worker_gguf_output_head(const Tensor &x,
                                                                      std::optional<int64_t> final_request_block_idx,
                                                                      const SamplingRequest *sampling) {
  std::shared_ptr<OutputHead> head = output_head();
  if (!head) return std::nullopt;
  if (final_request_block_idx != head->final_block_idx) return std::nullopt;
  OutputHeadResult r;
  Tensor logits = forward_output_head(*head, x);
  if (!g_head_route_logged.exchange(true))
    log_info("worker GGUF output-head route selected: final_block=" + std::to_string(head->final_block_idx) +
             " hidden_shape=" + x.dims_debug() + " logits_shape=" + logits.dims_debug() +
             " logits_dtype=" + dtype_name(logits.dtype()));
  if (worker_gguf_sample_token_enabled()) {
    if (!sampling)
      bail("GGUF remote sampling is enabled but the Master did not send sampling parameters; rebuild and restart "
           "both endpoints");
    try {
      r.token = sample_remote_logits(logits, *sampling);
    } catch (const Error &e) {
      bail("remote sampling failed: %s", e.what());
    }
    return r;
  }
  r.logits = std::move(logits);
  return r;
}

// worker_gguf_prefill_for_dims (worker_gguf.rs:399-406): dims [.., seq, hidden]
bool worker_gguf_prefill_for_dims(const std::vector<int64_t> &dims) {
  const int64_t seq_len = dims.size() >= 2 ? dims[dims.size() - 2] : 1;
  return seq_len > 1;
}

// forward_worker_gguf (worker_gguf.rs:574-611).  The reference routes
// rows <= 8 to candle's direct MMVQ and casts larger inputs to F32 around
// QMatMul; here the library takes F16 / BF16 / F32 at any row count (GEMV
// up to 64 rows, GEMM above), so both routes call it with the caller's dtype
// and return that dtype.
Tensor forward_worker_gguf(const GgufMatMul &matmul, const Tensor &x) { return matmul.forward(x); }

Linear build_worker_gguf_fp16_prefill_linear(const std::string &name, const std::vector<TextLinear> &sources) {
  if (sources.empty()) bail("cannot build empty FP16 GGUF prefill projection");
  std::vector<Tensor> parts;
  int64_t rows = 0, in_dim = -1;
  for (const TextLinear &src : sources) {
    parts.push_back(src.gguf_dequantize_f16_weight());
    const Tensor &w = parts.back();
    if (in_dim >= 0 && w.dims()[1] != in_dim)
      bail("%s: source input dims differ (%lld vs %lld)", name.c_str(), (long long)w.dims()[1], (long long)in_dim);
    in_dim = w.dims()[1];
    rows += w.dims()[0];
  }
  Tensor fused = Tensor::empty(DType::F16, {rows, in_dim}, parts[0].device());
  size_t off = 0;
  for (const Tensor &w : parts) {
    DeviceScope ds(w.device());
    hip_ok(hipMemcpy(fused.data() ? (uint8_t *)fused.data() + off : nullptr, w.data(), w.nbytes(),
                     hipMemcpyDeviceToDevice),
           "hipMemcpy D2D");
    off += w.nbytes();
  }
  g_gguf_prefill_count.fetch_add(1);
  g_gguf_prefill_bytes.fetch_add(fused.nbytes());
  log_info("built worker GGUF FP16 prefill projection " + name + " shape=" + fused.dims_debug());
  return Linear(fused);
}

// ---- TextLinear (worker_w8a16.rs:65-140) --------------------------------------
TextLinear TextLinear::from_dense(const std::string &name, Linear dense) {
  TextLinear t;
  t.name_ = name;
  if (worker_w8a16_enabled()) {
    try {
      t.w8a16_ = W8A16Linear::from_linear(name, dense);
      return t;
    } catch (const Error &e) {
      log_warn("worker W8A16 conversion failed for " + name + ": " + e.what() + "; falling back to dense F16");
    }
  }
  t.dense_ = std::move(dense);
  return t;
}

TextLinear TextLinear::gguf(const std::string &name, std::shared_ptr<GgufMatMul> matmul) {
  TextLinear t;
  t.name_ = name;
  t.gguf_ = std::move(matmul);
  return t;
}

Tensor TextLinear::forward(const Tensor &x) const {
  if (w8a16_) return w8a16_->forward(x);
  if (gguf_) {
    if (dense_ && worker_gguf_prefill_for_dims(x.dims())) return dense_->forward(x);
    return forward_worker_gguf(*gguf_, x);
  }
  return dense_->forward(x);
}

Tensor TextLinear::gguf_dequantize_f16_weight() const {
  if (!gguf_) bail("FP16 GGUF prefill requires a GGUF linear");
  return gguf_->dequantize_f16();
}

TextLinear TextLinear::with_gguf_fp16_prefill(Linear prefill) const {
  TextLinear t = *this;
  if (gguf_) t.dense_ = std::move(prefill);
  return t;
}

}  // namespace dial
