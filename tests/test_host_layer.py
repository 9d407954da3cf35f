"""Host operator layer (C++ above the C ABI), CPU-only checks: the mode gates,
the GGUF hybrid routing rule and the error paths of linear_no_bias that fail
before any device work.  Mirrors the reference's own tests where it has them:
worker_gguf.rs:628-634 (hybrid routing), quant.rs:539-543 (NVFP4 length
error); the mode gates follow quant.rs:27-62 and worker_w8a16.rs:15-44."""
import numpy as np
import pytest

import dialq.host as H


def test_quant_linear_mode_gate():
    # quant.rs:27-62: the device-resident mode needs the GPU runtime
    with pytest.raises(H.DialError, match="requires a ROCm device and --dtype f16 or bf16"):
        H.configure_quant_linear(H.Qwen38QuantLinear.Rocm, H.Device.cpu(), H.DType.F16)
    with pytest.raises(H.DialError, match=r"dtype=F32"):
        H.configure_quant_linear(H.Qwen38QuantLinear.Rocm, H.Device.rocm(0), H.DType.F32)
    H.configure_quant_linear(H.Qwen38QuantLinear.Auto, H.Device.cpu(), H.DType.F16)
    assert H.quant_linear_summary() is None  # Auto on a CPU runtime is dense
    H.configure_quant_linear(H.Qwen38QuantLinear.Auto, H.Device.rocm(0), H.DType.BF16)
    assert H.quant_linear_summary() == (0, 0)
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, H.Device.rocm(0), H.DType.F16)
    assert H.quant_linear_summary() is None


def test_worker_w8a16_gate():
    # worker_w8a16.rs:15-44: master mode, non-GPU devices and unsupported
    # dtypes keep dense weights (GGUF precedence: test_gguf_reader.py)
    H.configure_worker_gguf_from_args(None, False, False, False, True, H.Device.rocm(0), H.DType.F16, 1)
    H.configure_worker_w8a16_from_args(True, False, H.Device.rocm(0), H.DType.F16)
    assert not H.worker_w8a16_enabled()
    H.configure_worker_w8a16_from_args(True, True, H.Device.cpu(), H.DType.F16)
    assert not H.worker_w8a16_enabled()
    assert "non-ROCm device" in H.last_warning()
    H.configure_worker_w8a16_from_args(True, True, H.Device.rocm(0), H.DType.F32)
    assert not H.worker_w8a16_enabled()
    assert "got F32" in H.last_warning()
    H.configure_worker_w8a16_from_args(True, True, H.Device.rocm(0), H.DType.F16)
    assert H.worker_w8a16_enabled()
    assert H.worker_w8a16_summary() is not None
    H.configure_worker_w8a16_from_args(False, True, H.Device.rocm(0), H.DType.F16)
    assert not H.worker_w8a16_enabled()


def test_hybrid_routing_uses_fp16_only_for_multi_token_inputs():
    # worker_gguf.rs:628-634
    assert not H.worker_gguf_prefill_for_dims([1, 1, 4096])
    assert H.worker_gguf_prefill_for_dims([1, 2, 4096])
    assert H.worker_gguf_prefill_for_dims([1, 224, 4096])
    assert not H.worker_gguf_prefill_for_dims([1, 4096])


def _vb(dtype=H.DType.F32):
    return H.VarStore(dtype, H.Device.rocm(0))


def test_rejects_invalid_nvfp4_shapes():
    # quant.rs:539-543: 7 packed bytes for a 1 x 16 weight
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, H.Device.rocm(0), H.DType.F32)
    vb = _vb()
    vb.insert("layer.weight", H.Tensor.from_numpy(np.zeros((1, 7), np.uint8)))
    vb.insert("layer.weight_scale", H.Tensor.from_numpy(np.ones((1, 1), np.float32)))
    vb.insert("layer.weight_scale_2", H.Tensor.from_numpy(np.ones(1, np.float32)))
    with pytest.raises(H.DialError, match="expected 8"):
        H.linear_no_bias(16, 1, vb.pp("layer"))


def test_fp8_scale_count_and_representability_errors():
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, H.Device.rocm(0), H.DType.F32)
    vb = _vb()
    vb.insert("layer.weight", H.Tensor.from_numpy(np.array([[1, 2], [3, 4]], np.float32)))
    vb.insert("layer.weight_scale", H.Tensor.from_numpy(np.array([1, 2, 3], np.float32)))
    with pytest.raises(H.DialError, match="contains 3 values, expected 1 or 2"):
        H.linear_no_bias(2, 2, vb.pp("layer"))
    vb2 = _vb()
    vb2.insert("layer.weight", H.Tensor.from_numpy(np.array([[0.3, 2], [3, 4]], np.float32)))
    vb2.insert("layer.weight_scale", H.Tensor.from_numpy(np.array([1.0], np.float32)))
    with pytest.raises(H.DialError, match="not representable in E4M3"):
        H.linear_no_bias(2, 2, vb2.pp("layer"))


def test_compressed_tensors_zero_global_is_rejected():
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, H.Device.rocm(0), H.DType.F32)
    vb = _vb()
    vb.insert("layer.weight_packed", H.Tensor.from_numpy(np.full((1, 8), 0x92, np.uint8)))
    vb.insert("layer.weight_scale", H.Tensor.from_numpy(np.array([[2.0]], np.float32)))
    vb.insert("layer.weight_global_scale", H.Tensor.from_numpy(np.array([0.0], np.float32)))
    with pytest.raises(H.DialError, match="weight_global_scale for layer is zero"):
        H.linear_no_bias(16, 1, vb.pp("layer"))


def test_worker_gguf_output_head_load_errors(tmp_path):
    # worker_gguf.rs:197-265: the gates and the shape / presence checks of
    # load_worker_gguf_output_head, all raised before any device work
    from gguf_writer import write_gguf
    rocm = H.Device.rocm(0)
    cfg = H.OutputHeadConfig(hidden_size=32, vocab_size=4, num_hidden_layers=2)
    meta = [("general.architecture", "STRING", "qwen3vl"), ("qwen3vl.block_count", "U32", 2)]
    ones = np.ones(32, np.float32).tobytes()
    q8 = bytes(4 * 34)

    def configure(tensors, head=True):
        path = tmp_path / f"head{len(list(tmp_path.iterdir()))}.gguf"
        write_gguf(str(path), meta, tensors)
        H.configure_worker_gguf_from_args(str(path), False, head, False, True, rocm, H.DType.F16, 2)

    try:
        configure([("output_norm.weight", "F32", [32], ones)], head=False)
        H.load_worker_gguf_output_head(cfg, True)  # not requested: nothing to do
        assert not H.worker_gguf_output_head_enabled()
        assert H.maybe_forward_worker_gguf_output_head(H.Tensor.from_numpy(np.zeros((1, 32), np.float32)), 1) is None
        configure([("output_norm.weight", "F32", [32], ones)])
        H.load_worker_gguf_output_head(cfg, False)  # another worker owns the final layer
        assert not H.worker_gguf_output_head_enabled()
        configure([("output.weight", "Q8_0", [4, 32], q8)])
        with pytest.raises(H.DialError, match="has no tensor output_norm.weight"):
            H.load_worker_gguf_output_head(cfg, True)
        configure([("output_norm.weight", "F32", [16], bytes(64))])
        with pytest.raises(H.DialError, match=r"output_norm.weight shape \[16\], expected \[32\]"):
            H.load_worker_gguf_output_head(cfg, True)
        configure([("output_norm.weight", "F32", [32], ones)])
        with pytest.raises(H.DialError, match="has neither output.weight nor token_embd.weight"):
            H.load_worker_gguf_output_head(cfg, True)
        configure([("output_norm.weight", "F32", [32], ones), ("token_embd.weight", "Q8_0", [5, 32], bytes(5 * 34))])
        with pytest.raises(H.DialError, match=r"token_embd.weight shape \[5, 32\], expected \[4, 32\]"):
            H.load_worker_gguf_output_head(cfg, True)
        assert not H.worker_gguf_output_head_enabled()
        path = tmp_path / "nohead.gguf"
        write_gguf(str(path), meta, [])
        with pytest.raises(H.DialError, match="requires --worker-gguf-output-head"):
            H.configure_worker_gguf_from_args(str(path), False, False, True, True, rocm, H.DType.F16, 2)
    finally:
        H.configure_worker_gguf_from_args(None, False, False, False, True, rocm, H.DType.F16, 1)


def test_f32_to_f16_rounding_matches_numpy():
    # the F16 conversion of output_norm.weight (gguf_tensor_to_f16,
    # worker_gguf.rs:681-696 checks 1..4): round to nearest even, against
    # numpy's float16 cast on ties, subnormals, overflow, signed zeros, inf
    # and every 13-bit tail pattern of a few exponents
    base = np.array([1.0, 2.0, 3.0, 4.0, 0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                     6.1035156e-05, 6.0e-05, 5.9604645e-08, 2.9802322e-08, 2.98e-08, 8.9e-08, -1.5e-06],
                    np.float32)
    bits = (np.arange(1 << 13, dtype=np.uint32)[:, None] | (np.array([103, 112, 127, 140], np.uint32) << 23))
    tails = bits.ravel().view(np.float32)
    x = np.concatenate([base, tails, -tails, np.random.default_rng(0).normal(0, 50, 4096).astype(np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(H.f32_to_f16_bits(x), want)
    nan = H.f32_to_f16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7c00) == 0x7c00 and (nan & 0x3ff) != 0
