// GGUF file reader: the subset of candle-core 0.11's
// `quantized::gguf_file` that the reference's GGUF worker uses
// (qwen3_vl/worker_gguf.rs:113-114 Content::read, :484-505 tensor_infos /
// Content::tensor, :116-140 metadata lookups; paths relative to
// dial-core/src/models).  candle-core is a third-party crate that is not part
// of the reference tree; this is a restatement of the published GGUF layout
// (versions 1-3, little endian) with candle's conventions:
//
//   header   u32 magic "GGUF" (0x46554747 read little endian), u32 version,
//            tensor count and metadata count (u32 in v1, u64 in v2/v3)
//   metadata key string, u32 value type, value; strings are a length
//            (u32 in v1, u64 after) plus bytes, with trailing NUL bytes
//            dropped; arrays are u32 element type, length, elements
//   tensors  name string, u32 n_dims, dims (u32 in v1, u64 after, ggml order
//            ne0 = the contiguous dimension), u32 ggml type, u64 offset
//   data     starts at the end of the tensor infos rounded up to
//            general.alignment (default 32); tensor offsets are relative to it
//
// Shapes are reported the way candle reports them: the ggml dims reversed,
// so a linear weight stored with ne = [in, out] has dims [out, in].
#pragma once

#include <cstdint>
#include <functional>
#include <istream>
#include <map>
#include <string>
#include <vector>

namespace dial {
namespace gguf {

// ggml tensor types that GGUF files name (ggml numbering).
enum class GgmlDType : uint32_t {
  F32 = 0,
  F16 = 1,
  Q4_0 = 2,
  Q4_1 = 3,
  Q5_0 = 6,
  Q5_1 = 7,
  Q8_0 = 8,
  Q8_1 = 9,
  Q2K = 10,
  Q3K = 11,
  Q4K = 12,
  Q5K = 13,
  Q6K = 14,
  Q8K = 15,
  BF16 = 30,
};
bool ggml_dtype_known(uint32_t t);
const char *ggml_dtype_name(GgmlDType t);  // candle's Debug names: "Q4K", "Q8_0", "F16" ...
int64_t ggml_block_size(GgmlDType t);      // elements per block (1 for F32/F16/BF16)
int64_t ggml_type_size(GgmlDType t);       // bytes per block

enum class ValueType : uint32_t {
  U8 = 0,
  I8 = 1,
  U16 = 2,
  I16 = 3,
  U32 = 4,
  I32 = 5,
  F32 = 6,
  Bool = 7,
  String = 8,
  Array = 9,
  U64 = 10,
  I64 = 11,
  F64 = 12,
};

struct Value {
  ValueType type = ValueType::U8;
  uint64_t u = 0;  // U8/U16/U32/U64, Bool
  int64_t i = 0;   // I8/I16/I32/I64
  double f = 0.0;  // F32/F64
  std::string s;   // String
  std::vector<Value> arr;
  ValueType arr_type = ValueType::U8;

  // candle's to_u64: unsigned integers and bools widen, anything else fails
  uint64_t to_u64() const;
  uint32_t to_u32() const;  // U8/U16/U32 only
  const std::string &to_string() const;
  std::string debug() const;  // candle-style: U32(36), String("qwen3vl"), Array([...])
};

struct TensorInfo {
  GgmlDType ggml_dtype = GgmlDType::F32;
  std::vector<int64_t> dims;  // candle order: reversed ggml ne
  uint64_t offset = 0;        // from Content::tensor_data_offset
  int64_t elem_count() const;
  // bytes of the tensor's blocks; raises when the element count is not a
  // whole number of blocks (candle TensorInfo::read)
  int64_t size_in_bytes() const;
};

struct Content {
  uint32_t version = 0;
  std::map<std::string, Value> metadata;
  std::map<std::string, TensorInfo> tensor_infos;
  uint64_t tensor_data_offset = 0;
  uint64_t file_size = 0;

  // Parses header, metadata and tensor infos from the start of `in`.
  // `file_size` bounds every length read from the file.
  static Content read(std::istream &in, uint64_t file_size);
  // The raw bytes of tensor `name` (the range Content::tensor reads).
  std::vector<uint8_t> tensor_bytes(std::istream &in, const std::string &name) const;
  // The same bytes in chunks of at most `chunk` bytes, each handed to
  // sink(data, offset, count) in order: the host holds one chunk at a time
  // (the reference's GGML adapter streams assigned tensors in 8 MiB chunks,
  // backends/qwen38_ggml/adapter.cpp:198-227).  Returns the tensor's size.
  size_t tensor_chunks(std::istream &in, const std::string &name, size_t chunk,
                       const std::function<void(const uint8_t *, size_t, size_t)> &sink) const;
  const Value *get(const std::string &key) const;
};

// Opens and parses a file (Content::read on a File).
Content read_file(const std::string &path);

}  // namespace gguf
}  // namespace dial
