// GGUF file reader (see gguf.hpp for the layout it follows).
#include "gguf.hpp"

#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

#include "dial_host.hpp"

namespace dial {
namespace gguf {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint64_t kDefaultAlignment = 32;

[[noreturn]] void fail(const std::string &msg) { throw Error(msg); }

// Sequential little-endian reader over an istream with a byte budget.
class Reader {
 public:
  Reader(std::istream &in, uint64_t size) : in_(in), size_(size) {}
  uint64_t pos() const { return pos_; }
  uint64_t left() const { return size_ - pos_; }
  void bytes(void *dst, uint64_t n) {
    if (n > left()) fail("unexpected end of GGUF file at byte " + std::to_string(pos_));
    if (n && !in_.read((char *)dst, (std::streamsize)n)) fail("GGUF read failed at byte " + std::to_string(pos_));
    pos_ += n;
  }
  template <typename T>
  T get() {
    T v;
    bytes(&v, sizeof(T));  // host and file are both little endian
    return v;
  }
  uint64_t len(uint32_t version) { return version == 1 ? get<uint32_t>() : get<uint64_t>(); }
  std::string str(uint32_t version) {
    const uint64_t n = len(version);
    if (n > left()) fail("GGUF string length " + std::to_string(n) + " runs past the end of the file");
    std::string s(n, '\0');
    bytes(&s[0], n);
    while (!s.empty() && s.back() == '\0') s.pop_back();  // some writers NUL-terminate
    return s;
  }

 private:
  std::istream &in_;
  uint64_t size_;
  uint64_t pos_ = 0;
};

uint64_t min_value_bytes(ValueType t) {
  switch (t) {
    case ValueType::U8:
    case ValueType::I8:
    case ValueType::Bool:
      return 1;
    case ValueType::U16:
    case ValueType::I16:
      return 2;
    case ValueType::U32:
    case ValueType::I32:
    case ValueType::F32:
      return 4;
    case ValueType::String:  // length only
    case ValueType::U64:
    case ValueType::I64:
    case ValueType::F64:
      return 4;
    case ValueType::Array:
      return 8;
  }
  return 1;
}

ValueType value_type(uint32_t t) {
  if (t > 12) fail("unknown GGUF metadata value type " + std::to_string(t));
  return (ValueType)t;
}

Value read_value(Reader &r, ValueType t, uint32_t version, int depth) {
  Value v;
  v.type = t;
  switch (t) {
    case ValueType::U8: v.u = r.get<uint8_t>(); break;
    case ValueType::I8: v.i = r.get<int8_t>(); break;
    case ValueType::U16: v.u = r.get<uint16_t>(); break;
    case ValueType::I16: v.i = r.get<int16_t>(); break;
    case ValueType::U32: v.u = r.get<uint32_t>(); break;
    case ValueType::I32: v.i = r.get<int32_t>(); break;
    case ValueType::U64: v.u = r.get<uint64_t>(); break;
    case ValueType::I64: v.i = r.get<int64_t>(); break;
    case ValueType::F32: v.f = r.get<float>(); break;
    case ValueType::F64: v.f = r.get<double>(); break;
    case ValueType::Bool: {
      const uint8_t b = r.get<uint8_t>();
      if (b > 1) fail("unexpected GGUF bool value " + std::to_string(b));
      v.u = b;
      break;
    }
    case ValueType::String: v.s = r.str(version); break;
    case ValueType::Array: {
      if (depth > 8) fail("GGUF metadata arrays nested too deeply");
      v.arr_type = value_type(r.get<uint32_t>());
      const uint64_t n = r.len(version);
      if (n > r.left() / min_value_bytes(v.arr_type))
        fail("GGUF array length " + std::to_string(n) + " runs past the end of the file");
      v.arr.reserve(n);
      for (uint64_t i = 0; i < n; ++i) v.arr.push_back(read_value(r, v.arr_type, version, depth + 1));
      break;
    }
  }
  return v;
}

}  // namespace

bool ggml_dtype_known(uint32_t t) { return (t <= 15 && t != 4 && t != 5) || t == 30; }

const char *ggml_dtype_name(GgmlDType t) {
  switch (t) {
    case GgmlDType::F32: return "F32";
    case GgmlDType::F16: return "F16";
    case GgmlDType::BF16: return "BF16";
    case GgmlDType::Q4_0: return "Q4_0";
    case GgmlDType::Q4_1: return "Q4_1";
    case GgmlDType::Q5_0: return "Q5_0";
    case GgmlDType::Q5_1: return "Q5_1";
    case GgmlDType::Q8_0: return "Q8_0";
    case GgmlDType::Q8_1: return "Q8_1";
    case GgmlDType::Q2K: return "Q2K";
    case GgmlDType::Q3K: return "Q3K";
    case GgmlDType::Q4K: return "Q4K";
    case GgmlDType::Q5K: return "Q5K";
    case GgmlDType::Q6K: return "Q6K";
    case GgmlDType::Q8K: return "Q8K";
  }
  return "?";
}

// Block geometry of each ggml type: elements per block, bytes per block.
int64_t ggml_block_size(GgmlDType t) {
  switch (t) {
    case GgmlDType::F32:
    case GgmlDType::F16:
    case GgmlDType::BF16:
      return 1;
    case GgmlDType::Q4_0:
    case GgmlDType::Q4_1:
    case GgmlDType::Q5_0:
    case GgmlDType::Q5_1:
    case GgmlDType::Q8_0:
    case GgmlDType::Q8_1:
      return 32;
    default:
      return 256;  // the k-quants
  }
}

int64_t ggml_type_size(GgmlDType t) {
  switch (t) {
    case GgmlDType::F32: return 4;
    case GgmlDType::F16: return 2;
    case GgmlDType::BF16: return 2;
    case GgmlDType::Q4_0: return 2 + 16;        // d, 32 nibbles
    case GgmlDType::Q4_1: return 2 + 2 + 16;    // d, m, 32 nibbles
    case GgmlDType::Q5_0: return 2 + 4 + 16;    // d, high bits, nibbles
    case GgmlDType::Q5_1: return 2 + 2 + 4 + 16;
    case GgmlDType::Q8_0: return 2 + 32;        // d, 32 int8
    case GgmlDType::Q8_1: return 2 + 2 + 32;    // d, s, 32 int8
    case GgmlDType::Q2K: return 16 + 64 + 2 + 2;
    case GgmlDType::Q3K: return 32 + 64 + 12 + 2;
    case GgmlDType::Q4K: return 2 + 2 + 12 + 128;
    case GgmlDType::Q5K: return 2 + 2 + 12 + 32 + 128;
    case GgmlDType::Q6K: return 128 + 64 + 16 + 2;
    case GgmlDType::Q8K: return 4 + 256 + 2 * 16;
  }
  return 0;
}

uint64_t Value::to_u64() const {
  switch (type) {
    case ValueType::U8:
    case ValueType::U16:
    case ValueType::U32:
    case ValueType::U64:
    case ValueType::Bool:
      return u;
    default:
      fail("not a u64 or upcastable to u64 " + debug());
  }
}

uint32_t Value::to_u32() const {
  switch (type) {
    case ValueType::U8:
    case ValueType::U16:
    case ValueType::U32:
      return (uint32_t)u;
    default:
      fail("not a u32 " + debug());
  }
}

const std::string &Value::to_string() const {
  if (type != ValueType::String) fail("not a string " + debug());
  return s;
}

std::string Value::debug() const {
  std::ostringstream o;
  switch (type) {
    case ValueType::U8: o << "U8(" << u << ")"; break;
    case ValueType::I8: o << "I8(" << i << ")"; break;
    case ValueType::U16: o << "U16(" << u << ")"; break;
    case ValueType::I16: o << "I16(" << i << ")"; break;
    case ValueType::U32: o << "U32(" << u << ")"; break;
    case ValueType::I32: o << "I32(" << i << ")"; break;
    case ValueType::U64: o << "U64(" << u << ")"; break;
    case ValueType::I64: o << "I64(" << i << ")"; break;
    case ValueType::F32: o << "F32(" << f << ")"; break;
    case ValueType::F64: o << "F64(" << f << ")"; break;
    case ValueType::Bool: o << "Bool(" << (u ? "true" : "false") << ")"; break;
    case ValueType::String: o << "String(\"" << s << "\")"; break;
    case ValueType::Array: {
      o << "Array([";
      for (size_t k = 0; k < arr.size() && k < 8; ++k) o << (k ? ", " : "") << arr[k].debug();
      if (arr.size() > 8) o << ", ...";
      o << "])";
      break;
    }
  }
  return o.str();
}

int64_t TensorInfo::elem_count() const {
  int64_t n = 1;
  for (int64_t d : dims) n *= d;
  return n;
}

int64_t TensorInfo::size_in_bytes() const {
  const int64_t n = elem_count(), bs = ggml_block_size(ggml_dtype);
  if (n % bs != 0)
    fail("the number of elements " + std::to_string(n) + " is not divisible by the block size " + std::to_string(bs));
  return n / bs * ggml_type_size(ggml_dtype);
}

Content Content::read(std::istream &in, uint64_t file_size) {
  Reader r(in, file_size);
  const uint32_t magic = r.get<uint32_t>();
  if (magic != kMagic) {
    char buf[16];
    std::snprintf(buf, sizeof buf, "%08x", magic);
    fail(std::string("unknown magic ") + buf);
  }
  Content c;
  c.version = r.get<uint32_t>();
  if (c.version < 1 || c.version > 3) fail("unknown GGUF version " + std::to_string(c.version));
  const uint64_t n_tensors = r.len(c.version), n_kv = r.len(c.version);
  // every entry takes at least 8 bytes of the file
  if (n_tensors > r.left() / 8 || n_kv > r.left() / 8) fail("GGUF header counts run past the end of the file");
  for (uint64_t k = 0; k < n_kv; ++k) {
    std::string key = r.str(c.version);
    const ValueType t = value_type(r.get<uint32_t>());
    c.metadata[key] = read_value(r, t, c.version, 0);
  }
  for (uint64_t k = 0; k < n_tensors; ++k) {
    std::string name = r.str(c.version);
    const uint32_t n_dims = r.get<uint32_t>();
    if (n_dims > 8) fail("tensor " + name + " has " + std::to_string(n_dims) + " dimensions");
    std::vector<int64_t> dims(n_dims);
    uint64_t elems = 1;
    for (uint32_t d = 0; d < n_dims; ++d) {
      const uint64_t v = c.version == 1 ? r.get<uint32_t>() : r.get<uint64_t>();
      if (v > (uint64_t)1 << 40) fail("tensor " + name + " has an invalid dimension " + std::to_string(v));
      if (v != 0 && elems > ((uint64_t)1 << 50) / v) fail("tensor " + name + " has too many elements");
      elems *= v;
      dims[n_dims - 1 - d] = (int64_t)v;  // candle reverses the ggml order
    }
    const uint32_t ty = r.get<uint32_t>();
    if (!ggml_dtype_known(ty)) fail("unknown dtype for tensor " + std::to_string(ty));
    TensorInfo ti;
    ti.ggml_dtype = (GgmlDType)ty;
    ti.dims = std::move(dims);
    ti.offset = r.get<uint64_t>();
    c.tensor_infos[name] = std::move(ti);
  }
  uint64_t alignment = kDefaultAlignment;
  if (const Value *a = c.get("general.alignment")) {
    switch (a->type) {
      case ValueType::U8:
      case ValueType::U16:
      case ValueType::U32:
        alignment = a->u;
        break;
      case ValueType::I8:
      case ValueType::I16:
      case ValueType::I32:
        if (a->i >= 0) alignment = (uint64_t)a->i;
        break;
      default:
        break;
    }
  }
  if (alignment == 0 || alignment > ((uint64_t)1 << 30)) fail("invalid general.alignment " + std::to_string(alignment));
  c.tensor_data_offset = (r.pos() + alignment - 1) / alignment * alignment;
  c.file_size = file_size;
  return c;
}

std::vector<uint8_t> Content::tensor_bytes(std::istream &in, const std::string &name) const {
  auto it = tensor_infos.find(name);
  if (it == tensor_infos.end()) fail("cannot find tensor info for " + name);
  const TensorInfo &ti = it->second;
  const int64_t n = ti.size_in_bytes();
  if (ti.offset > file_size || tensor_data_offset > file_size - ti.offset ||
      (uint64_t)n > file_size - tensor_data_offset - ti.offset)
    fail("truncated GGUF tensor " + name + ": " + std::to_string(n) + " bytes at offset " +
         std::to_string(tensor_data_offset + ti.offset) + " of a " + std::to_string(file_size) + "-byte file");
  std::vector<uint8_t> out((size_t)n);
  in.clear();
  in.seekg((std::streamoff)(tensor_data_offset + ti.offset));
  if (!in || (n && !in.read((char *)out.data(), (std::streamsize)n)))
    fail("truncated GGUF tensor " + name + ": " + std::to_string(n) + " bytes at offset " +
         std::to_string(tensor_data_offset + ti.offset));
  return out;
}

size_t Content::tensor_chunks(std::istream &in, const std::string &name, size_t chunk,
                              const std::function<void(const uint8_t *, size_t, size_t)> &sink) const {
  auto it = tensor_infos.find(name);
  if (it == tensor_infos.end()) fail("cannot find tensor info for " + name);
  if (chunk == 0) fail("chunk size must be positive");
  const TensorInfo &ti = it->second;
  const uint64_t n = (uint64_t)ti.size_in_bytes();
  if (ti.offset > file_size || tensor_data_offset > file_size - ti.offset || n > file_size - tensor_data_offset - ti.offset)
    fail("truncated GGUF tensor " + name + ": " + std::to_string(n) + " bytes at offset " +
         std::to_string(tensor_data_offset + ti.offset) + " of a " + std::to_string(file_size) + "-byte file");
  in.clear();
  in.seekg((std::streamoff)(tensor_data_offset + ti.offset));
  std::vector<uint8_t> buf((size_t)(n < chunk ? n : chunk));
  for (uint64_t off = 0; off < n;) {
    const size_t count = (size_t)((n - off) < chunk ? (n - off) : chunk);
    if (!in || !in.read((char *)buf.data(), (std::streamsize)count))
      fail("truncated GGUF tensor " + name + ": " + std::to_string(n) + " bytes at offset " +
           std::to_string(tensor_data_offset + ti.offset));
    sink(buf.data(), (size_t)off, count);
    off += count;
  }
  return (size_t)n;
}

const Value *Content::get(const std::string &key) const {
  auto it = metadata.find(key);
  return it == metadata.end() ? nullptr : &it->second;
}

Content read_file(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail("cannot open " + path);
  f.seekg(0, std::ios::end);
  const uint64_t size = (uint64_t)f.tellg();
  f.seekg(0);
  return Content::read(f, size);
}

}  // namespace gguf
}  // namespace dial
