"""safetensors checkpoint reader of the host layer, CPU only.

The reference loads Hugging Face checkpoints through candle's
VarBuilder::from_mmaped_safetensors over the files listed in
model.safetensors.index.json (utils/mod.rs:76-135); linear_no_bias then
reads tensors by name (qwen3_8/quant.rs:466-519).  The files here are
written by the `safetensors` library itself (an independent writer of the
format), with the dtypes NVFP4 / FP8 checkpoints use: U8 packed codes,
F8_E4M3 scales and weights, F32 / BF16 / F16 scales and dense weights."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import dialq.host as H


def _tensors():
    g = torch.Generator().manual_seed(0)
    return {
        "model.layers.0.mlp.down_proj.weight": torch.randint(0, 256, (4, 8), generator=g, dtype=torch.uint8),
        "model.layers.0.mlp.down_proj.weight_scale": torch.randn(4, 1, generator=g).to(torch.float8_e4m3fn),
        "model.layers.0.mlp.down_proj.weight_scale_2": torch.tensor([0.25]),
        "model.layers.0.self_attn.o_proj.weight": torch.randn(3, 5, generator=g).to(torch.bfloat16),
        "model.layers.0.self_attn.q_proj.weight": torch.randn(2, 6, generator=g).to(torch.float16),
        "model.layers.0.input_layernorm.weight": torch.randint(-128, 127, (7,), generator=g, dtype=torch.int8),
        "step": torch.tensor([3], dtype=torch.int64),  # a dtype no linear reads: skipped
    }


def _raw(t):
    return t.contiguous().view(torch.uint8).numpy().tobytes() if t.dtype != torch.uint8 else t.numpy().tobytes()


def test_header_matches_the_written_file(tmp_path):
    p = tmp_path / "model.safetensors"
    ts = _tensors()
    save_file(ts, str(p), metadata={"format": "pt", "quant_method": "modelopt"})
    h = H.safetensors_read_header(str(p))
    blob = p.read_bytes()
    n = struct.unpack("<Q", blob[:8])[0]
    ref = json.loads(blob[8:8 + n])
    assert h["data_start"] == 8 + n
    assert h["metadata"] == {"format": "pt", "quant_method": "modelopt"}
    dt = {torch.uint8: "U8", torch.float8_e4m3fn: "F8_E4M3", torch.float32: "F32", torch.bfloat16: "BF16",
          torch.float16: "F16", torch.int8: "I8", torch.int64: "I64"}
    assert set(h["tensors"]) == set(ts)
    for name, t in ts.items():
        dtype, shape, begin, end = h["tensors"][name]
        assert dtype == dt[t.dtype] == ref[name]["dtype"]
        assert shape == list(t.shape) == ref[name]["shape"]
        assert [begin, end] == ref[name]["data_offsets"]
        assert blob[8 + n + begin:8 + n + end] == _raw(t)


def test_load_into_var_store_keeps_bits(tmp_path):
    p = tmp_path / "model.safetensors"
    ts = _tensors()
    save_file(ts, str(p))
    vs = H.VarStore(H.DType.F16, H.Device.rocm(0))
    vs.load_safetensors([str(p)])
    want = {H.DType.U8: [torch.uint8, torch.float8_e4m3fn, torch.int8], H.DType.F32: [torch.float32],
            H.DType.BF16: [torch.bfloat16], H.DType.F16: [torch.float16]}
    for name, t in ts.items():
        if t.dtype == torch.int64:
            assert not vs.contains_tensor(name)
            continue
        got = vs.get(name)
        assert got.dims == list(t.shape)
        assert any(t.dtype in v for k, v in want.items() if k == got.dtype), (name, got.dtype)
        assert got.numpy().tobytes() == _raw(t), name
    # E4M3 codes arrive as their bytes, as load_fp8_raw keeps them (quant.rs:220-232)
    s = vs.get("model.layers.0.mlp.down_proj.weight_scale").numpy().ravel()
    assert list(s) == list(ts["model.layers.0.mlp.down_proj.weight_scale"].view(torch.uint8).ravel().numpy())
    assert vs.pp("model.layers.0.mlp").pp("down_proj").contains_tensor("weight_scale_2")


def test_index_lists_distinct_shards(tmp_path):
    # utils/mod.rs:76-110
    idx = tmp_path / "model.safetensors.index.json"
    idx.write_text(json.dumps({"metadata": {"total_size": 10}, "weight_map": {
        "a.weight": "model-00002-of-00002.safetensors", "b.weight": "model-00001-of-00002.safetensors",
        "c.weight": "model-00002-of-00002.safetensors"}}))
    assert H.safetensors_paths_from_index(str(idx)) == [
        f"{tmp_path}/model-00001-of-00002.safetensors", f"{tmp_path}/model-00002-of-00002.safetensors"]
    idx.write_text(json.dumps({"metadata": {}}))
    with pytest.raises(H.DialError, match="no weight map in"):
        H.safetensors_paths_from_index(str(idx))
    idx.write_text(json.dumps({"weight_map": ["x"]}))
    with pytest.raises(H.DialError, match="is not a map"):
        H.safetensors_paths_from_index(str(idx))


def test_malformed_files_are_rejected(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(b"\x01\x02")
    with pytest.raises(H.DialError, match="too short"):
        H.safetensors_read_header(str(p))
    hdr = json.dumps({"w": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(8))  # 8 of 16 data bytes
    with pytest.raises(H.DialError, match="runs past the end"):
        H.safetensors_read_header(str(p))
    hdr = json.dumps({"w": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 16]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(16))
    with pytest.raises(H.DialError, match="shape needs 24"):
        H.safetensors_read_header(str(p))
    p.write_bytes(struct.pack("<Q", 5) + b"{\"w\":")
    with pytest.raises(H.DialError, match="invalid JSON"):
        H.safetensors_read_header(str(p))
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(H.DialError, match="header length"):
        H.safetensors_read_header(str(p))
    # a shape whose element count overflows is refused, not wrapped round
    hdr = json.dumps({"w": {"dtype": "F32", "shape": [2 ** 40, 2 ** 40, 16], "data_offsets": [0, 0]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr)
    with pytest.raises(H.DialError, match="too many elements"):
        H.safetensors_read_header(str(p))
