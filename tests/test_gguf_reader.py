"""GGUF file reader and the GGUF worker's configuration gate, CPU only.

The reader (dial-27b_amd/host/gguf.cpp) stands in for candle-core 0.11's
gguf_file::Content, which the reference calls at qwen3_vl/worker_gguf.rs:113
(read), :484-505 (tensor_infos, Content::tensor) and :116-140 (metadata).
candle is not in the reference tree, so the files here come from an
independent writer (tests/gguf_writer.py) built from the GGUF layout, shaped
like the reference's own fixture (qwen3_8/ggml_tests.rs:72-212: architecture
string, U32 hyper-parameters, F32 values, Q4K / Q8_0 / F32 tensors).  The
configuration checks follow configure_worker_gguf_from_args
(worker_gguf.rs:65-180) and load_worker_gguf_linear (:462-522) up to the
upload, which needs the GPU (tests/test_gpu_host_layer.py covers it).
"""
import numpy as np
import pytest

import dialq.host as H
from gguf_writer import GGML, tensor_nbytes, write_gguf

ROCM = H.Device.rocm(0)


def _raw(ggml, dims, seed):
    return np.random.default_rng(seed).integers(0, 256, tensor_nbytes(ggml, dims), dtype=np.uint8).tobytes()


def _tiny(path, arch="qwen3vl", block_count=("U32", 2), version=3, alignment=32, nul=False, extra_meta=(),
          tensors=None, **kw):
    meta = [("general.architecture", "STRING", arch)] if arch is not None else []
    if block_count is not None:
        meta.append(("qwen3vl.block_count", block_count[0], block_count[1]))
    meta += [("qwen3vl.embedding_length", "U32", 256), ("qwen3vl.rope.freq_base", "F32", 5e6)]
    if alignment != 32:
        meta.append(("general.alignment", "U32", alignment))
    meta += list(extra_meta)
    if tensors is None:
        tensors = [("blk.0.ffn_gate.weight", "Q4K", [512, 256], _raw("Q4K", [512, 256], 1)),
                   ("blk.0.ffn_down.weight", "Q8_0", [256, 512], _raw("Q8_0", [256, 512], 2)),
                   ("blk.0.attn_v.weight", "Q6K", [128, 256], _raw("Q6K", [128, 256], 3)),
                   ("blk.0.attn_q.weight", "F16", [64, 256], _raw("F16", [64, 256], 5)),
                   ("blk.0.attn_norm.weight", "F32", [256], _raw("F32", [256], 4))]
    start = write_gguf(str(path), meta, tensors, version=version, alignment=alignment, nul_strings=nul, **kw)
    return meta, tensors, start


@pytest.mark.parametrize("version", [1, 2, 3])
def test_reads_header_metadata_and_tensor_infos(tmp_path, version):
    p = tmp_path / "tiny.gguf"
    meta, tensors, start = _tiny(p, version=version, extra_meta=[
        ("t.u8", "U8", 7), ("t.i8", "I8", -7), ("t.u16", "U16", 65535), ("t.i16", "I16", -300),
        ("t.i32", "I32", -5), ("t.u64", "U64", 2 ** 40), ("t.i64", "I64", -2 ** 40), ("t.f64", "F64", 0.1),
        ("t.bool", "BOOL", True), ("t.arr", "ARRAY", ("STRING", ["a", "bc", ""])),
        ("t.nested", "ARRAY", ("ARRAY", [("U32", [1, 2]), ("U32", [])]))])
    c = H.gguf_read(str(p))
    assert c["version"] == version
    assert c["tensor_data_offset"] == start and start % 32 == 0
    got = c["metadata"]
    assert got["general.architecture"] == (8, "qwen3vl")
    assert got["qwen3vl.block_count"] == (4, 2)
    assert got["qwen3vl.rope.freq_base"][1] == pytest.approx(5e6)
    assert got["t.u8"] == (0, 7) and got["t.i8"] == (1, -7) and got["t.u16"] == (2, 65535)
    assert got["t.i16"] == (3, -300) and got["t.i32"] == (5, -5) and got["t.u64"] == (10, 2 ** 40)
    assert got["t.i64"] == (11, -2 ** 40) and got["t.f64"] == (12, 0.1) and got["t.bool"] == (7, True)
    assert got["t.arr"] == (9, ["a", "bc", ""])
    assert got["t.nested"] == (9, [[1, 2], []])
    ti = c["tensors"]
    # candle reports dims outer-first: [out, in] for a linear (ggml ne = [in, out])
    assert ti["blk.0.ffn_gate.weight"][:2] == ("Q4K", [512, 256])
    assert ti["blk.0.ffn_down.weight"][:2] == ("Q8_0", [256, 512])
    assert ti["blk.0.attn_v.weight"][:2] == ("Q6K", [128, 256])
    assert ti["blk.0.attn_norm.weight"][:2] == ("F32", [256])
    for name, ggml, dims, raw in tensors:
        assert H.gguf_tensor_bytes(str(p), name) == raw
    blob = p.read_bytes()
    for name, ggml, dims, raw in tensors:  # offsets are relative to the data start
        off = start + ti[name][2]
        assert ti[name][2] % 32 == 0 and blob[off:off + len(raw)] == raw


def test_tensor_chunks_stream_the_same_bytes(tmp_path):
    """Content::tensor_chunks (the loader's bounded-memory path) hands the
    tensor over in order, each piece at most the chunk size."""
    p = tmp_path / "c.gguf"
    meta, tensors, start = _tiny(p)
    for name, ggml, dims, raw in tensors:
        for chunk in (1, 100, 4096, 1 << 23):
            got, pieces = H.gguf_tensor_chunks(str(p), name, chunk)
            assert got == raw
            assert all(n <= chunk for _, n in pieces)
            assert [o for o, _ in pieces] == list(range(0, len(raw), chunk))
    _tiny(p, tensors=[("x.weight", "Q8_0", [2, 32], bytes(68))], truncate=10)
    with pytest.raises(H.DialError, match="truncated GGUF tensor x.weight"):
        H.gguf_tensor_chunks(str(p), "x.weight", 16)


def test_alignment_and_nul_terminated_strings(tmp_path):
    p = tmp_path / "a.gguf"
    meta, tensors, start = _tiny(p, alignment=256, nul=True)
    c = H.gguf_read(str(p))
    assert c["tensor_data_offset"] == start and start % 256 == 0
    assert c["metadata"]["general.architecture"][1] == "qwen3vl"  # trailing NUL dropped
    assert "blk.0.ffn_gate.weight" in c["tensors"]
    for name, ggml, dims, raw in tensors:
        assert H.gguf_tensor_bytes(str(p), name) == raw


def test_reader_errors(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + bytes(20))
    with pytest.raises(H.DialError, match="unknown magic"):
        H.gguf_read(str(p))
    p.write_bytes(b"GGUF" + (4).to_bytes(4, "little") + bytes(16))
    with pytest.raises(H.DialError, match="unknown GGUF version 4"):
        H.gguf_read(str(p))
    _tiny(p, tensors=[])
    blob = p.read_bytes()
    p.write_bytes(blob[:40])
    with pytest.raises(H.DialError, match="end of"):
        H.gguf_read(str(p))
    _tiny(p, tensors=[("x.weight", "Q8_0", [2, 32], bytes(68))], ggml_type_ids={"x.weight": 4})
    with pytest.raises(H.DialError, match="unknown dtype for tensor 4"):
        H.gguf_read(str(p))
    _tiny(p, tensors=[("x.weight", "Q8_0", [2, 32], bytes(68))], truncate=10)
    with pytest.raises(H.DialError, match="truncated GGUF tensor x.weight"):
        H.gguf_tensor_bytes(str(p), "x.weight")
    _tiny(p, tensors=[("x.weight", "Q8_0", [2, 32], bytes(68))])
    with pytest.raises(H.DialError, match="cannot find tensor info for y.weight"):
        H.gguf_tensor_bytes(str(p), "y.weight")
    # sizes come from the file: element counts that overflow and alignments
    # that cannot be honoured are refused before anything is allocated
    _tiny(p, tensors=[("x.weight", "F32", [2 ** 30, 2 ** 30], b"")], check_sizes=False)
    with pytest.raises(H.DialError, match="too many elements"):
        H.gguf_read(str(p))
    _tiny(p, tensors=[("x.weight", "F32", [2 ** 20, 64], b"")], check_sizes=False)
    with pytest.raises(H.DialError, match="truncated GGUF tensor x.weight"):
        H.gguf_tensor_bytes(str(p), "x.weight")
    _tiny(p, tensors=[], extra_meta=[("general.alignment", "U32", 0)])
    with pytest.raises(H.DialError, match="invalid general.alignment 0"):
        H.gguf_read(str(p))


def _configure(path, **kw):
    args = dict(fp16_prefill=False, output_head=False, sample_token=False, worker_mode=True, device=ROCM,
                dtype=H.DType.F16, num_hidden_layers=2)
    args.update(kw)
    H.configure_worker_gguf_from_args(str(path) if path is not None else None, **args)


def test_configure_gates_and_metadata_checks(tmp_path):
    p = tmp_path / "w.gguf"
    _tiny(p)
    try:
        _configure(p, worker_mode=False)  # master mode ignores the options
        assert not H.worker_gguf_enabled() and H.worker_gguf_summary() is None
        with pytest.raises(H.DialError, match="requires --worker-quantized-gguf"):
            _configure(None, fp16_prefill=True)
        _configure(None)
        assert not H.worker_gguf_enabled()
        with pytest.raises(H.DialError, match="requires a ROCm worker"):
            _configure(p, device=H.Device.cpu())
        with pytest.raises(H.DialError, match="requires --dtype f16 or bf16"):
            _configure(p, dtype=H.DType.F32)
        with pytest.raises(H.DialError, match="sample-token true requires --worker-gguf-output-head true"):
            _configure(p, sample_token=True)
        with pytest.raises(H.DialError, match="cannot open worker GGUF"):
            _configure(tmp_path / "missing.gguf")
        bad = tmp_path / "bad.gguf"
        bad.write_bytes(b"nope" + bytes(28))
        with pytest.raises(H.DialError, match="cannot parse worker GGUF .*unknown magic"):
            _configure(bad)
        _tiny(bad, arch="llama")
        with pytest.raises(H.DialError, match=r'unsupported architecture metadata String\("llama"\); expected qwen3vl'):
            _configure(bad)
        _tiny(bad, arch=None)
        with pytest.raises(H.DialError, match="is missing general.architecture"):
            _configure(bad)
        _tiny(bad, block_count=("U32", 3))
        with pytest.raises(H.DialError, match="block count 3 does not match Hugging Face config 2"):
            _configure(bad)
        _tiny(bad, block_count=("F32", 2.0))
        with pytest.raises(H.DialError, match="invalid qwen3vl.block_count"):
            _configure(bad)
        for bc in (("U64", 2), ("U8", 2)):  # unsigned widths widen (candle to_u64)
            _tiny(bad, block_count=bc)
            _configure(bad)
            assert H.worker_gguf_enabled()
        _configure(p, fp16_prefill=True, output_head=True, sample_token=True, dtype=H.DType.BF16)
        assert H.worker_gguf_enabled() and H.worker_gguf_fp16_prefill_enabled()
        assert H.worker_gguf_output_head_requested() and H.worker_gguf_sample_token_requested()
        assert H.worker_gguf_summary() == (0, 0, 0, 0)
        # GGUF takes precedence over the W8A16 worker path (worker_w8a16.rs:15-44)
        H.configure_worker_w8a16_from_args(True, True, ROCM, H.DType.F16)
        assert not H.worker_w8a16_enabled()
        assert "GGUF takes precedence" in H.last_warning()
    finally:
        _configure(None)
    assert not H.worker_gguf_enabled()


def test_load_linear_lookup_errors(tmp_path):
    p = tmp_path / "w.gguf"
    _tiny(p)
    assert H.load_worker_gguf_linear(0, "ffn_gate", 256, 512) is None  # no source configured
    try:
        _configure(p)
        with pytest.raises(H.DialError, match="requires a numeric transformer layer name"):
            H.load_worker_gguf_linear(None, "ffn_gate", 256, 512)
        with pytest.raises(H.DialError, match="has no tensor blk.1.ffn_gate.weight"):
            H.load_worker_gguf_linear(1, "ffn_gate", 256, 512)
        with pytest.raises(H.DialError, match=r"blk.0.ffn_gate.weight shape \[512, 256\], expected \[256, 512\]"):
            H.load_worker_gguf_linear(0, "ffn_gate", 512, 256)
        with pytest.raises(H.DialError, match="has dtype F16; the ROCm GGUF path takes Q8_0, Q4K and Q6K"):
            H.load_worker_gguf_linear(0, "attn_q", 256, 64)
    finally:
        _configure(None)


def test_block_geometry_table():
    # bytes per block of the types a Q4_K_M file mixes (ggml block layouts)
    assert GGML["Q4K"][2] == 2 + 2 + 12 + 128
    assert GGML["Q6K"][2] == 128 + 64 + 16 + 2
    assert GGML["Q8_0"][2] == 2 + 32
