// Feeds files to the host layer's checkpoint readers -- the GGUF reader
// (dial::gguf::read_file + tensor_bytes) and the safetensors reader
// (dial::safetensors::read_header + load_into, on the host) -- under
// AddressSanitizer and UndefinedBehaviorSanitizer.  Every file is expected
// to parse or to fail with a dial::Error; a crash, an out-of-bounds access
// or undefined behaviour is reported by the sanitizers and fails the run.
// Built and run by tests/test_sanitizers.py over valid, truncated and
// corrupted files.
#include <cstdio>
#include <exception>
#include <fstream>
#include <string>

#include "../../dial-27b_amd/host/gguf.hpp"
#include "../../dial-27b_amd/host/safetensors.hpp"

int main(int argc, char **argv) {
  int parsed = 0, rejected = 0;
  for (int i = 1; i < argc; ++i) {
    const std::string path = argv[i];
    const bool is_gguf = path.size() > 5 && path.compare(path.size() - 5, 5, ".gguf") == 0;
    try {
      if (is_gguf) {
        dial::gguf::Content c = dial::gguf::read_file(path);
        std::ifstream f(path, std::ios::binary);
        for (const auto &kv : c.tensor_infos) (void)c.tensor_bytes(f, kv.first);
      } else {
        dial::safetensors::Header h = dial::safetensors::read_header(path);
        (void)h;
        dial::VarStore vs(dial::DType::F32, dial::Device::cpu());
        dial::safetensors::load_into(vs, {path});
      }
      ++parsed;
    } catch (const std::exception &) {
      ++rejected;
    }
  }
  std::printf("parsed %d rejected %d\n", parsed, rejected);
  return 0;
}
