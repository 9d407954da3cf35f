"""AddressSanitizer / UndefinedBehaviorSanitizer runs of the CPU-side code
(tests/sanitize/): the oracle's every function at exact buffer sizes, and
the host layer's GGUF and safetensors readers -- which take offsets,
lengths and shapes from untrusted files -- over valid files and thousands
of truncated and corrupted ones.  A file may be rejected (dial::Error);
nothing may read out of bounds, overflow or otherwise hit undefined
behaviour.  Host code only: the sanitized binaries are built with g++ /
gcc and never touch a GPU."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


@pytest.fixture(scope="module")
def built():
    if not os.path.exists(os.path.join(ROOT, "dial-27b_amd", "lib", "libdialq.so")):
        pytest.skip("libdialq.so is not built (run __graft_entry__.build())")
    r = subprocess.run(["make", "-s", "-j2", "-C", SAN], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    return os.path.join(SAN, "_build")


def _run(binary, args=(), env=ENV):
    r = subprocess.run([binary, *args], capture_output=True, text=True, timeout=600, env=env)
    report = [l for l in r.stderr.splitlines() if "Sanitizer" in l or "runtime error" in l]
    assert r.returncode == 0 and not report, (r.returncode, report[:5], r.stderr[-2000:])
    return r.stdout


def test_binaries_carry_the_sanitizers(built):
    # a build that lost its -fsanitize flags would pass the runs below
    # without checking anything
    for b in ("oracle_exercise", "parsers_fuzz"):
        libs = subprocess.run(["ldd", os.path.join(built, b)], capture_output=True, text=True).stdout
        assert "libasan" in libs and "libubsan" in libs, (b, libs)


def test_oracle_under_sanitizers(built):
    assert "oracle exercise done" in _run(os.path.join(built, "oracle_exercise"))


def _gguf_corpus(tmp_path):
    from gguf_writer import write_gguf
    import oracle as O
    rng = np.random.default_rng(0)
    meta = [("general.architecture", "STRING", "qwen3vl"), ("qwen3vl.block_count", "U32", 2),
            ("tokenizer.ggml.tokens", "ARRAY", ("STRING", ["a", "bb", "ccc"])),
            ("nested", "ARRAY", ("ARRAY", [("U8", [1, 2]), ("F32", [0.5])])), ("general.alignment", "U32", 64)]
    w = rng.normal(0, 0.02, (4, 256)).astype(np.float32)
    tensors = [("blk.0.attn_q.weight", "Q4K", [4, 256], O.q4_k_quantize(w).tobytes()),
               ("blk.0.attn_k.weight", "Q8_0", [4, 256], O.q8_0_quantize(w).tobytes()),
               ("blk.0.ffn_down.weight", "Q6K", [2, 256], O.q6_k_random_blocks(2, 256, 1).tobytes()),
               ("output_norm.weight", "F32", [256], np.ones(256, np.float32).tobytes())]
    files = []
    for version in (1, 2, 3):
        p = tmp_path / f"valid_v{version}.gguf"
        write_gguf(str(p), meta, tensors, version=version)
        files.append(p)
    base = files[-1].read_bytes()
    # every truncation in the header region and a spread through the data
    cuts = list(range(0, min(len(base), 700))) + list(range(700, len(base), 97))
    for i in cuts:
        p = tmp_path / f"trunc_{i}.gguf"
        p.write_bytes(base[:i])
        files.append(p)
    # byte and word corruptions of the header region: counts, string and
    # array lengths, dimensions, types, offsets
    for i in range(1500):
        b = bytearray(base)
        pos = int(rng.integers(0, min(len(b), 800)))
        if i % 3 == 0:
            b[pos] = int(rng.integers(0, 256))
        elif i % 3 == 1:
            big = [0, 1, 2 ** 31, 2 ** 32 - 1, 2 ** 40, 2 ** 63, 2 ** 64 - 1]
            b[pos:pos + 8] = struct.pack("<Q", big[int(rng.integers(0, len(big)))])
        else:
            small = [0, 7, 13, 255, 2 ** 31, 2 ** 32 - 1]
            b[pos:pos + 4] = struct.pack("<I", small[int(rng.integers(0, len(small)))])
        p = tmp_path / f"corrupt_{i}.gguf"
        p.write_bytes(bytes(b[:len(base)]))
        files.append(p)
    return files


def _safetensors_corpus(tmp_path):
    import torch
    from safetensors.torch import save_file
    rng = np.random.default_rng(1)
    ts = {"a.weight_packed": torch.randint(0, 255, (4, 8), dtype=torch.uint8),
          "a.weight_scale": torch.rand(4, 2, dtype=torch.float32),
          "b.weight": torch.randn(3, 5).to(torch.bfloat16), "c.weight": torch.randn(2, 2).to(torch.float16),
          "d.weight": torch.randn(4, 4).to(torch.float8_e4m3fn), "e": torch.arange(6, dtype=torch.int64)}
    p0 = tmp_path / "valid.safetensors"
    save_file(ts, str(p0), metadata={"format": "pt"})
    base = p0.read_bytes()
    files = [p0]
    n = struct.unpack("<Q", base[:8])[0]
    for i in list(range(0, min(len(base), n + 8 + 16))) + list(range(n + 8 + 16, len(base), 11)):
        p = tmp_path / f"trunc_{i}.safetensors"
        p.write_bytes(base[:i])
        files.append(p)
    hdr = json.loads(base[8:8 + n])
    data = base[8 + n:]
    for i in range(600):
        h = json.loads(json.dumps(hdr))
        name = list(k for k in h if k != "__metadata__")[i % 6]
        choice = i % 6
        if choice == 0:
            h[name]["data_offsets"] = [int(rng.integers(-5, 2 ** 20)), int(rng.integers(-5, 2 ** 20))]
        elif choice == 1:
            h[name]["shape"] = [int(v) for v in rng.integers(-3, 2 ** 16, int(rng.integers(0, 5)))]
        elif choice == 2:
            h[name]["dtype"] = str(rng.choice(["F32", "BF16", "U8", "F8_E4M3", "I8", "XYZ", "", "F64"]))
        elif choice == 3:
            h[name]["data_offsets"] = [2 ** 63, 2 ** 64 - 1] if i % 12 == 3 else [2 ** 64 + 5, -1]
        elif choice == 4:
            h[name] = "not an object"
        else:
            h[name]["shape"] = [2 ** 31, 2 ** 31, 4]
        hb = json.dumps(h).encode()
        p = tmp_path / f"corrupt_{i}.safetensors"
        p.write_bytes(struct.pack("<Q", len(hb)) + hb + data)
        files.append(p)
    for i in range(300):  # raw byte flips of the JSON header and the length word
        b = bytearray(base)
        pos = int(rng.integers(0, n + 8))
        b[pos] = int(rng.integers(0, 256))
        p = tmp_path / f"flip_{i}.safetensors"
        p.write_bytes(bytes(b))
        files.append(p)
    return files


def test_checkpoint_readers_under_sanitizers(built, tmp_path):
    files = _gguf_corpus(tmp_path) + _safetensors_corpus(tmp_path)
    out = ""
    for i in range(0, len(files), 500):  # bounded argument lists
        out += _run(os.path.join(built, "parsers_fuzz"), [str(p) for p in files[i:i + 500]])
    parsed = sum(int(l.split()[1]) for l in out.splitlines() if l.startswith("parsed"))
    rejected = sum(int(l.split()[3]) for l in out.splitlines() if l.startswith("parsed"))
    assert parsed + rejected == len(files)
    assert parsed >= 4 and rejected >= len(files) // 2, (parsed, rejected)
