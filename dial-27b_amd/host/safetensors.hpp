// safetensors checkpoint reader for the quantized-linear loaders.
//
// The reference reads Hugging Face checkpoints through candle's
// VarBuilder::from_mmaped_safetensors (utils/mod.rs:114-135) over the files
// named by model.safetensors.index.json (load_safetensors_paths_from_index,
// utils/mod.rs:76-110); linear_no_bias then looks tensors up by name
// (qwen3_8/quant.rs:466-519).  Here the same files fill a VarStore that
// dial::linear_no_bias reads.  Layout (safetensors format): u64 little-endian
// header length N, N bytes of JSON {name: {"dtype", "shape", "data_offsets":
// [begin, end]}, "__metadata__": {...}}, then the data; offsets are relative
// to the end of the header.
//
// Dtypes kept: F32, F16, BF16 (as such), U8, I8 and F8_E4M3 (raw bytes in a
// U8 tensor: the E4M3 codes NVFP4 / FP8 checkpoints carry, which the loaders
// read bit for bit as the reference's load_fp8_raw does, quant.rs:220-232).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "dial_host.hpp"

namespace dial {
namespace safetensors {

struct TensorInfo {
  std::string dtype;           // "F32", "F8_E4M3", ...
  std::vector<int64_t> shape;  // row-major dims
  uint64_t begin = 0, end = 0; // byte range after the header
};

struct Header {
  uint64_t data_start = 0;  // 8 + header length
  std::map<std::string, TensorInfo> tensors;
  std::map<std::string, std::string> metadata;  // "__metadata__" (string values)
};

// Parses the header of `path` and checks every tensor's byte range against
// its dtype and shape and against the file size.
Header read_header(const std::string &path);

// Loads every tensor of the files into `vs` (names unchanged), on the host.
// Tensors of other dtypes (I64, F64, BOOL, ...) are skipped, as no quantized
// linear reads them.
void load_into(VarStore &vs, const std::vector<std::string> &paths);

// load_safetensors_paths_from_index (utils/mod.rs:76-110): the distinct
// files of the index's "weight_map", joined to the index's directory.
std::vector<std::string> paths_from_index(const std::string &index_json);

}  // namespace safetensors
}  // namespace dial
