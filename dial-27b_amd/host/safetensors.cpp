// safetensors checkpoint reader (see safetensors.hpp).
#include "safetensors.hpp"

#include <algorithm>
#include <cstring>
#include <fstream>
#include <set>

namespace dial {
namespace safetensors {

namespace {

[[noreturn]] void fail(const std::string &msg) { throw Error(msg); }

// Minimal JSON reader for safetensors headers and index files: objects,
// arrays, strings (with escapes), integers, true / false / null.
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  int64_t num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json *get(const std::string &k) const {
    for (const auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class Parser {
 public:
  explicit Parser(const std::string &s) : s_(s) {}
  Json parse() {
    Json v = value(0);
    ws();
    if (i_ != s_.size()) err("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void err(const char *what) { fail(std::string("invalid JSON: ") + what + " at byte " + std::to_string(i_)); }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  bool lit(const char *t) {
    const size_t n = std::strlen(t);
    if (s_.compare(i_, n, t) == 0) {
      i_ += n;
      return true;
    }
    return false;
  }
  static void utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xc0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      out += (char)(0xe0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3f));
      out += (char)(0x80 | (cp & 0x3f));
    } else {
      out += (char)(0xf0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3f));
      out += (char)(0x80 | ((cp >> 6) & 0x3f));
      out += (char)(0x80 | (cp & 0x3f));
    }
  }
  uint32_t hex4() {
    if (i_ + 4 > s_.size()) err("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else err("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    if (i_ >= s_.size() || s_[i_] != '"') err("expected a string");
    ++i_;
    std::string out;
    while (true) {
      if (i_ >= s_.size()) err("unterminated string");
      const char c = s_[i_++];
      if (c == '"') break;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) err("unterminated escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xd800 && cp < 0xdc00 && lit("\\u")) {  // surrogate pair
            const uint32_t lo = hex4();
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          utf8(out, cp);
          break;
        }
        default: err("bad escape");
      }
    }
    return out;
  }
  Json value(int depth) {
    if (depth > 32) err("nesting too deep");
    ws();
    if (i_ >= s_.size()) err("unexpected end");
    Json v;
    const char c = s_[i_];
    if (c == '{') {
      v.kind = Json::Obj;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == '}') {
        ++i_;
        return v;
      }
      while (true) {
        ws();
        std::string k = string();
        ws();
        if (i_ >= s_.size() || s_[i_] != ':') err("expected ':'");
        ++i_;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (i_ < s_.size() && s_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < s_.size() && s_[i_] == '}') {
          ++i_;
          return v;
        }
        err("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Json::Arr;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == ']') {
        ++i_;
        return v;
      }
      while (true) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (i_ < s_.size() && s_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < s_.size() && s_[i_] == ']') {
          ++i_;
          return v;
        }
        err("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Json::Str;
      v.str = string();
      return v;
    }
    if (lit("true")) {
      v.kind = Json::Bool;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.kind = Json::Bool;
      return v;
    }
    if (lit("null")) return v;
    if (c == '-' || (c >= '0' && c <= '9')) {
      v.kind = Json::Num;
      const size_t st = i_;
      if (s_[i_] == '-') ++i_;
      while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
      if (i_ < s_.size() && (s_[i_] == '.' || s_[i_] == 'e' || s_[i_] == 'E')) err("non-integer number");
      if (i_ - st > 19) err("integer out of range");
      v.num = std::stoll(s_.substr(st, i_ - st));
      return v;
    }
    err("unexpected character");
  }
  const std::string &s_;
  size_t i_ = 0;
};

int64_t dtype_bytes(const std::string &d) {
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
  if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  fail("unknown safetensors dtype " + d);
}

std::string read_file(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail("can't open " + path);
  return std::string(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

}  // namespace

Header read_header(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail("can't open " + path);
  f.seekg(0, std::ios::end);
  const uint64_t size = (uint64_t)f.tellg();
  f.seekg(0);
  uint64_t n = 0;
  if (size < 8 || !f.read((char *)&n, 8)) fail(path + ": too short for a safetensors header");
  if (n > size - 8 || n > ((uint64_t)100 << 20)) fail(path + ": header length " + std::to_string(n) + " is invalid");
  std::string text((size_t)n, '\0');
  if (n && !f.read(&text[0], (std::streamsize)n)) fail(path + ": truncated header");
  const Json j = Parser(text).parse();
  if (j.kind != Json::Obj) fail(path + ": header is not a JSON object");
  Header h;
  h.data_start = 8 + n;
  const uint64_t data_bytes = size - h.data_start;
  for (const auto &kv : j.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != Json::Obj) fail(path + ": __metadata__ is not an object");
      for (const auto &m : kv.second.obj)
        if (m.second.kind == Json::Str) h.metadata[m.first] = m.second.str;
      continue;
    }
    const Json &t = kv.second;
    const Json *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
    if (t.kind != Json::Obj || !dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off ||
        off->kind != Json::Arr || off->arr.size() != 2)
      fail(path + ": malformed entry for tensor " + kv.first);
    TensorInfo ti;
    ti.dtype = dt->str;
    int64_t elems = 1;
    for (const Json &d : sh->arr) {
      if (d.kind != Json::Num || d.num < 0) fail(path + ": bad shape for tensor " + kv.first);
      if (d.num != 0 && elems > ((int64_t)1 << 50) / d.num) fail(path + ": tensor " + kv.first + " has too many elements");
      ti.shape.push_back(d.num);
      elems *= d.num;
    }
    if (off->arr[0].kind != Json::Num || off->arr[1].kind != Json::Num || off->arr[0].num < 0 ||
        off->arr[1].num < off->arr[0].num)
      fail(path + ": bad data_offsets for tensor " + kv.first);
    ti.begin = (uint64_t)off->arr[0].num;
    ti.end = (uint64_t)off->arr[1].num;
    if (ti.end > data_bytes) fail(path + ": tensor " + kv.first + " runs past the end of the file");
    if ((int64_t)(ti.end - ti.begin) != elems * dtype_bytes(ti.dtype))
      fail(path + ": tensor " + kv.first + " has " + std::to_string(ti.end - ti.begin) + " bytes, its " + ti.dtype +
           " shape needs " + std::to_string(elems * dtype_bytes(ti.dtype)));
    h.tensors[kv.first] = ti;
  }
  return h;
}

void load_into(VarStore &vs, const std::vector<std::string> &paths) {
  for (const std::string &path : paths) {
    const Header h = read_header(path);
    std::ifstream f(path, std::ios::binary);
    if (!f) fail("can't open " + path);
    for (const auto &kv : h.tensors) {
      const TensorInfo &ti = kv.second;
      DType dt;
      if (ti.dtype == "F32") dt = DType::F32;
      else if (ti.dtype == "F16") dt = DType::F16;
      else if (ti.dtype == "BF16") dt = DType::BF16;
      else if (ti.dtype == "U8" || ti.dtype == "I8" || ti.dtype == "F8_E4M3") dt = DType::U8;
      else continue;
      std::vector<uint8_t> buf((size_t)(ti.end - ti.begin));
      f.clear();
      f.seekg((std::streamoff)(h.data_start + ti.begin));
      if (!buf.empty() && !f.read((char *)buf.data(), (std::streamsize)buf.size()))
        fail(path + ": truncated data for tensor " + kv.first);
      vs.insert(kv.first, Tensor::from_host(buf.data(), dt, ti.shape));
    }
  }
}

std::vector<std::string> paths_from_index(const std::string &index_json) {
  const Json j = Parser(read_file(index_json)).parse();
  const Json *wm = j.kind == Json::Obj ? j.get("weight_map") : nullptr;
  if (!wm) fail("no weight map in " + index_json);
  if (wm->kind != Json::Obj) fail("weight map in " + index_json + " is not a map");
  std::set<std::string> files;
  for (const auto &kv : wm->obj)
    if (kv.second.kind == Json::Str) files.insert(kv.second.str);
  const size_t slash = index_json.find_last_of('/');
  const std::string dir = slash == std::string::npos ? std::string(".") : index_json.substr(0, slash);
  std::vector<std::string> out;
  for (const std::string &file : files) out.push_back(dir + "/" + file);
  return out;
}

}  // namespace safetensors
}  // namespace dial
