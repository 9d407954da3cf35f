// Python bindings of the host operator layer (dial_host.hpp), for tests.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <fstream>

#include "dial_host.hpp"
#include "gguf.hpp"
#include "safetensors.hpp"
#include "sampling.hpp"

namespace py = pybind11;
using namespace dial;

namespace {

DType dtype_of_array(const py::array &a, std::optional<DType> hint) {
  if (hint) return *hint;
  const py::dtype d = a.dtype();
  if (d.is(py::dtype::of<float>())) return DType::F32;
  if (d.kind() == 'f' && d.itemsize() == 2) return DType::F16;
  if (d.is(py::dtype::of<uint8_t>())) return DType::U8;
  throw Error("pass dtype= for host arrays of " + std::string(py::str(d)));
}

Tensor tensor_from_numpy(const py::array &a, std::optional<DType> dtype) {
  const DType t = dtype_of_array(a, dtype);
  py::array c = py::array::ensure(a, py::array::c_style);
  if ((size_t)c.itemsize() != dtype_size(t)) throw Error("array item size does not match the dtype");
  std::vector<int64_t> dims(c.shape(), c.shape() + c.ndim());
  return Tensor::from_host(c.data(), t, dims);
}

py::array tensor_to_numpy(const Tensor &t) {
  const std::vector<uint8_t> b = t.host_bytes();
  std::vector<py::ssize_t> shape(t.dims().begin(), t.dims().end());
  py::dtype d = t.dtype() == DType::F32  ? py::dtype::of<float>()
                : t.dtype() == DType::F16 ? py::dtype("float16")
                : t.dtype() == DType::U8  ? py::dtype::of<uint8_t>()
                                          : py::dtype::of<uint16_t>();  // BF16 bits
  py::array out(d, shape);
  if (!b.empty()) std::memcpy(out.mutable_data(), b.data(), b.size());
  return out;
}

py::object gguf_value_to_py(const gguf::Value &v) {
  switch (v.type) {
    case gguf::ValueType::U8:
    case gguf::ValueType::U16:
    case gguf::ValueType::U32:
    case gguf::ValueType::U64:
      return py::int_(v.u);
    case gguf::ValueType::I8:
    case gguf::ValueType::I16:
    case gguf::ValueType::I32:
    case gguf::ValueType::I64:
      return py::int_(v.i);
    case gguf::ValueType::F32:
    case gguf::ValueType::F64:
      return py::float_(v.f);
    case gguf::ValueType::Bool:
      return py::bool_(v.u != 0);
    case gguf::ValueType::String:
      return py::str(v.s);
    case gguf::ValueType::Array: {
      py::list l;
      for (const gguf::Value &e : v.arr) l.append(gguf_value_to_py(e));
      return l;
    }
  }
  return py::none();
}

// The parsed header of a GGUF file: version, tensor_data_offset, metadata
// {key: (type id, value)} and tensors {name: (ggml dtype name, dims, offset)}.
py::dict gguf_read(const std::string &path) {
  const gguf::Content c = gguf::read_file(path);
  py::dict meta, tensors, out;
  for (const auto &kv : c.metadata)
    meta[py::str(kv.first)] = py::make_tuple((uint32_t)kv.second.type, gguf_value_to_py(kv.second));
  for (const auto &kv : c.tensor_infos)
    tensors[py::str(kv.first)] =
        py::make_tuple(gguf::ggml_dtype_name(kv.second.ggml_dtype), kv.second.dims, kv.second.offset);
  out["version"] = c.version;
  out["tensor_data_offset"] = c.tensor_data_offset;
  out["metadata"] = meta;
  out["tensors"] = tensors;
  return out;
}

// Content::tensor_chunks over a file: (the concatenated bytes, [(offset, count)]).
py::tuple gguf_tensor_chunks(const std::string &path, const std::string &name, size_t chunk) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw Error("cannot open " + path);
  f.seekg(0, std::ios::end);
  const uint64_t size = (uint64_t)f.tellg();
  f.seekg(0);
  const gguf::Content c = gguf::Content::read(f, size);
  std::string all;
  py::list pieces;
  c.tensor_chunks(f, name, chunk, [&](const uint8_t *p, size_t off, size_t n) {
    all.append((const char *)p, n);
    pieces.append(py::make_tuple(off, n));
  });
  return py::make_tuple(py::bytes(all), pieces);
}

py::bytes gguf_tensor_bytes(const std::string &path, const std::string &name) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw Error("cannot open " + path);
  f.seekg(0, std::ios::end);
  const uint64_t size = (uint64_t)f.tellg();
  f.seekg(0);
  const gguf::Content c = gguf::Content::read(f, size);
  const std::vector<uint8_t> b = c.tensor_bytes(f, name);
  return py::bytes((const char *)b.data(), b.size());
}

}  // namespace

PYBIND11_MODULE(dialq_host, m) {
  m.doc() = "Host operator layer of DIAL's quantized linear (C++ above the dialq C ABI)";
  py::register_exception<Error>(m, "DialError", PyExc_RuntimeError);

  py::enum_<DType>(m, "DType")
      .value("F32", DType::F32)
      .value("F16", DType::F16)
      .value("BF16", DType::BF16)
      .value("U8", DType::U8);

  py::class_<Device>(m, "Device")
      .def_static("cpu", &Device::cpu)
      .def_static("rocm", &Device::rocm, py::arg("ordinal") = 0)
      .def("is_rocm", &Device::is_rocm)
      .def("__repr__", &Device::debug);

  py::class_<Tensor>(m, "Tensor")
      .def_static("from_numpy", &tensor_from_numpy, py::arg("array"), py::arg("dtype") = py::none())
      .def("to_device", &Tensor::to_device)
      .def("numpy", &tensor_to_numpy)
      .def_property_readonly("dims", [](const Tensor &t) { return t.dims(); })
      .def_property_readonly("dtype", &Tensor::dtype)
      .def_property_readonly("device", &Tensor::device)
      .def("reshape", &Tensor::reshape);

  py::class_<Linear>(m, "Linear")
      .def(py::init<Tensor>())
      .def("forward", &Linear::forward)
      .def("weight", &Linear::weight);

  py::class_<VarStore>(m, "VarStore")
      .def(py::init<DType, Device>())
      .def("insert", &VarStore::insert)
      .def("get", &VarStore::get)
      .def("load_safetensors", [](VarStore &vs, const std::vector<std::string> &paths) {
        safetensors::load_into(vs, paths);
      })
      .def("pp", &VarStore::pp)
      .def("contains_tensor", &VarStore::contains_tensor)
      .def_property_readonly("prefix", &VarStore::prefix);

  py::class_<RocmQuantLinear, std::shared_ptr<RocmQuantLinear>>(m, "RocmQuantLinear")
      .def_static("nvfp4", &RocmQuantLinear::nvfp4)
      .def_static("fp8", &RocmQuantLinear::fp8)
      .def("resident_bytes", &RocmQuantLinear::resident_bytes)
      .def("forward", &RocmQuantLinear::forward);

  py::enum_<Qwen38QuantLinear>(m, "Qwen38QuantLinear")
      .value("Dense", Qwen38QuantLinear::Dense)
      .value("Auto", Qwen38QuantLinear::Auto)
      .value("Rocm", Qwen38QuantLinear::Rocm);

  py::class_<QuantLinear>(m, "QuantLinear")
      .def("forward", &QuantLinear::forward)
      .def("is_quantized_rocm", &QuantLinear::is_quantized_rocm)
      .def("dense_weight", [](const QuantLinear &q) { return q.dense_linear().weight(); });

  m.def("configure_quant_linear", &configure_quant_linear);
  m.def("quant_linear_summary", &quant_linear_summary);
  m.def("linear_no_bias", &linear_no_bias);

  py::class_<W8A16Linear, std::shared_ptr<W8A16Linear>>(m, "W8A16Linear")
      .def_static("from_linear", &W8A16Linear::from_linear)
      .def("forward", &W8A16Linear::forward)
      .def("resident_bytes", &W8A16Linear::resident_bytes);

  py::class_<GgufMatMul, std::shared_ptr<GgufMatMul>> gg(m, "GgufMatMul");
  py::enum_<GgufMatMul::Kind>(gg, "Kind")
      .value("Q8_0", GgufMatMul::Q8_0)
      .value("Q4_K", GgufMatMul::Q4_K)
      .value("Q6_K", GgufMatMul::Q6_K);
  gg.def_static("from_blocks", &GgufMatMul::from_blocks)
      .def_static("quantize", &GgufMatMul::quantize)
      .def("forward", &GgufMatMul::forward)
      .def("dequantize_f16", &GgufMatMul::dequantize_f16);

  py::class_<TextLinear>(m, "TextLinear")
      .def_static("from_dense", &TextLinear::from_dense)
      .def_static("gguf", &TextLinear::gguf)
      .def("forward", &TextLinear::forward)
      .def("gguf_dequantize_f16_weight", &TextLinear::gguf_dequantize_f16_weight)
      .def("with_gguf_fp16_prefill", &TextLinear::with_gguf_fp16_prefill)
      .def("is_w8a16", &TextLinear::is_w8a16)
      .def("is_gguf", &TextLinear::is_gguf)
      .def("is_dense", &TextLinear::is_dense);

  m.def("configure_worker_w8a16_from_args", &configure_worker_w8a16_from_args);
  m.def("worker_w8a16_enabled", &worker_w8a16_enabled);
  m.def("worker_w8a16_summary", &worker_w8a16_summary);
  m.def("configure_worker_gguf_from_args", &configure_worker_gguf_from_args, py::arg("path"),
        py::arg("fp16_prefill"), py::arg("output_head"), py::arg("sample_token"), py::arg("worker_mode"),
        py::arg("device"), py::arg("dtype"), py::arg("num_hidden_layers"));
  m.def("worker_gguf_enabled", &worker_gguf_enabled);
  m.def("worker_gguf_fp16_prefill_enabled", &worker_gguf_fp16_prefill_enabled);
  m.def("worker_gguf_output_head_requested", &worker_gguf_output_head_requested);
  m.def("worker_gguf_sample_token_requested", &worker_gguf_sample_token_requested);
  m.def("worker_gguf_summary", &worker_gguf_summary);
  m.def("load_worker_gguf_linear", &load_worker_gguf_linear);
  m.def("gguf_read", &gguf_read);
  m.def("safetensors_read_header", [](const std::string &path) {
    const safetensors::Header h = safetensors::read_header(path);
    py::dict tensors;
    for (const auto &kv : h.tensors)
      tensors[py::str(kv.first)] = py::make_tuple(kv.second.dtype, kv.second.shape, kv.second.begin, kv.second.end);
    py::dict out;
    out["data_start"] = h.data_start;
    out["tensors"] = tensors;
    out["metadata"] = h.metadata;
    return out;
  });
  m.def("safetensors_paths_from_index", &safetensors::paths_from_index);
  m.def("gguf_tensor_bytes", &gguf_tensor_bytes);
  m.def("gguf_tensor_chunks", &gguf_tensor_chunks);
  m.def("worker_gguf_prefill_for_dims", &worker_gguf_prefill_for_dims);
  m.def("forward_worker_gguf", &forward_worker_gguf);
  m.def("build_worker_gguf_fp16_prefill_linear", &build_worker_gguf_fp16_prefill_linear);
  m.def("last_warning", &last_warning);
  py::class_<OutputHeadConfig>(m, "OutputHeadConfig")
      .def(py::init([](int64_t hidden_size, int64_t vocab_size, int64_t num_hidden_layers, double rms_norm_eps) {
             return OutputHeadConfig{hidden_size, vocab_size, num_hidden_layers, rms_norm_eps};
           }),
           py::arg("hidden_size"), py::arg("vocab_size"), py::arg("num_hidden_layers"), py::arg("rms_norm_eps") = 1e-6);
  m.def("f32_to_f16_bits", [](py::array_t<float, py::array::c_style | py::array::forcecast> a) {
    py::array_t<uint16_t> out(a.size());
    const float *src = a.data();
    uint16_t *dst = out.mutable_data();
    for (py::ssize_t i = 0; i < a.size(); ++i) dst[i] = f32_to_f16_bits(src[i]);
    return out;
  });
  m.def("load_worker_gguf_output_head", &load_worker_gguf_output_head, py::arg("cfg"), py::arg("owns_final_layer"));
  m.def("worker_gguf_output_head_enabled", &worker_gguf_output_head_enabled);
  m.def("worker_gguf_sample_token_enabled", &worker_gguf_sample_token_enabled);
  // None, a logits Tensor, or the sampled token as an int.
  m.def(
      "maybe_forward_worker_gguf_output_head",
      [](const Tensor &x, std::optional<int64_t> final_request_block_idx,
         std::optional<SamplingRequest> sampling) -> py::object {
        auto r = maybe_forward_worker_gguf_output_head(x, final_request_block_idx, sampling ? &*sampling : nullptr);
        if (!r) return py::none();
        if (r->token) return py::int_(*r->token);
        return py::cast(*r->logits);
      },
      py::arg("x"), py::arg("final_request_block_idx"), py::arg("sampling") = py::none());

  py::class_<SamplingRequest>(m, "SamplingRequest")
      .def(py::init([](uint64_t seed, uint64_t sample_index, double temperature, std::optional<uint64_t> top_k,
                       std::optional<double> top_p, float repeat_penalty, std::vector<uint32_t> repeat_context) {
             return SamplingRequest{seed, sample_index, temperature, top_k, top_p, repeat_penalty,
                                    std::move(repeat_context)};
           }),
           py::arg("seed") = 0, py::arg("sample_index") = 0, py::arg("temperature") = 0.0,
           py::arg("top_k") = py::none(), py::arg("top_p") = py::none(), py::arg("repeat_penalty") = 1.0f,
           py::arg("repeat_context") = std::vector<uint32_t>{})
      .def_readwrite("seed", &SamplingRequest::seed)
      .def_readwrite("sample_index", &SamplingRequest::sample_index)
      .def_readwrite("temperature", &SamplingRequest::temperature)
      .def_readwrite("top_k", &SamplingRequest::top_k)
      .def_readwrite("top_p", &SamplingRequest::top_p)
      .def_readwrite("repeat_penalty", &SamplingRequest::repeat_penalty)
      .def_readwrite("repeat_context", &SamplingRequest::repeat_context);
  m.def("sample_remote_logits", &sample_remote_logits);
  m.def("sampling_mode", &sampling_mode);
  m.def("last_sample_used_host_logits", &last_sample_used_host_logits);
  m.def("chacha_block", [](std::array<uint32_t, 8> key, uint32_t counter, std::array<uint32_t, 3> nonce, int rounds) {
    return ChaChaRng::block(key, counter, nonce, rounds);
  });
  m.def("rng_u32_stream", [](uint64_t seed, int n) {
    ChaChaRng r = ChaChaRng::seed_from_u64(seed);
    std::vector<uint32_t> out((size_t)n);
    for (auto &v : out) v = r.next_u32();
    return out;
  });
  m.def("sample_weighted", [](const std::vector<float> &w, uint64_t seed) {
    ChaChaRng r = ChaChaRng::seed_from_u64(seed);
    return sample_weighted(w, r);
  });
}
