"""Host operator layer on the GPU: the reference's own tests for this path,
run through the C++ layer (which calls the C ABI; dense fallbacks multiply
with rocBLAS).

  quant.rs:527-537, 545-680   linear_no_bias loads and decodes (dense mode)
  cuda_quant.rs:507-552       NVFP4 / FP8 quantized linears vs dense, rows {1, 7}
  worker_w8a16.rs:483-516     W8A16 TextLinear vs dense, rows {1, 9}
  worker_gguf.rs:636-752      Q4_K decode keeps F16; fused FP16 prefill ==
                              separate; hybrid keeps Q4_K for one token
"""
import numpy as np
import pytest

import dialq.host as H

pytestmark = pytest.mark.gpu
ROCM = H.Device.rocm(0)


def _t(a, dtype=None):
    return H.Tensor.from_numpy(np.ascontiguousarray(a), dtype)


def _dense_values(q):
    return q.dense_weight().numpy().astype(np.float32).ravel().tolist()


def _nvfp4_store(compressed, dtype=H.DType.F32):
    vb = H.VarStore(dtype, ROCM)
    if compressed:
        vb.insert("layer.weight_packed", _t(np.full((1, 8), 0x92, np.uint8)))
        vb.insert("layer.weight_global_scale", _t(np.array([4.0], np.float32)))
    else:
        vb.insert("layer.weight", _t(np.full((1, 8), 0x92, np.uint8)))
        vb.insert("layer.weight_scale_2", _t(np.array([4.0], np.float32)))
    vb.insert("layer.weight_scale", _t(np.array([[2.0]], np.float32)))
    return vb


def test_linear_no_bias_dense_loads(torch_dev):
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, ROCM, H.DType.F32)
    # quant.rs:564-594 (ModelOpt NVFP4)
    q = H.linear_no_bias(16, 1, _nvfp4_store(False).pp("layer"))
    assert not q.is_quantized_rocm()
    assert _dense_values(q) == [8.0, -4.0] * 8
    # quant.rs:650-680 (compressed-tensors, reciprocal global)
    q = H.linear_no_bias(16, 1, _nvfp4_store(True).pp("layer"))
    assert _dense_values(q) == [0.5, -0.25] * 8
    # quant.rs:596-619 (FP8 with per-output scale)
    vb = H.VarStore(H.DType.F32, ROCM)
    vb.insert("layer.weight", _t(np.array([[1, 2], [3, 4]], np.float32)))
    vb.insert("layer.weight_scale", _t(np.array([2.0, 0.5], np.float32)))
    q = H.linear_no_bias(2, 2, vb.pp("layer"))
    assert _dense_values(q) == [2.0, 4.0, 1.5, 2.0]
    # quant.rs:621-648 (f32 scales with an F16 runtime)
    vb = H.VarStore(H.DType.F16, ROCM)
    vb.insert("layer.weight", _t(np.array([[1, 2], [3, 4]], np.float32)))
    vb.insert("layer.weight_scale", _t(np.array([2.0, 0.5], np.float32)))
    q = H.linear_no_bias(2, 2, vb.pp("layer"))
    assert q.dense_weight().dtype == H.DType.F16
    assert _dense_values(q) == [2.0, 4.0, 1.5, 2.0]
    # a plain dense weight
    vb = H.VarStore(H.DType.F32, ROCM)
    vb.insert("layer.weight", _t(np.array([[1, 2], [3, 4]], np.float32)))
    q = H.linear_no_bias(2, 2, vb.pp("layer"))
    assert _dense_values(q) == [1.0, 2.0, 3.0, 4.0]


def test_decodes_low_nibble_before_high_nibble_and_applies_group_scales(torch_dev):
    # quant.rs:527-537: packed[0] = 0x92, packed[8] = 0x65, scales [2, 0.5], global 4
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, ROCM, H.DType.F32)
    packed = np.zeros((1, 16), np.uint8)
    packed[0, 0], packed[0, 8] = 0x92, 0x65
    vb = H.VarStore(H.DType.F32, ROCM)
    vb.insert("l.weight", _t(packed))
    vb.insert("l.weight_scale", _t(np.array([[2.0, 0.5]], np.float32)))
    vb.insert("l.weight_scale_2", _t(np.array([4.0], np.float32)))
    d = H.linear_no_bias(32, 1, vb.pp("l")).dense_weight().numpy().ravel()
    assert (d[0], d[1], d[16], d[17]) == (8.0, -4.0, 6.0, 8.0)


def test_auto_mode_keeps_quantized_and_matches_dense(torch_dev):
    for compressed in (False, True):
        H.configure_quant_linear(H.Qwen38QuantLinear.Dense, ROCM, H.DType.F16)
        dense = H.linear_no_bias(16, 1, _nvfp4_store(compressed, H.DType.F16).pp("layer"))
        H.configure_quant_linear(H.Qwen38QuantLinear.Auto, ROCM, H.DType.F16)
        quant = H.linear_no_bias(16, 1, _nvfp4_store(compressed, H.DType.F16).pp("layer"))
        assert quant.is_quantized_rocm()
        assert H.quant_linear_summary()[0] == 1
        x = _t(np.cos(np.arange(3 * 16) * 0.3).astype(np.float16).reshape(3, 16)).to_device(ROCM)
        a = quant.forward(x).numpy().astype(np.float32)
        b = dense.forward(x).numpy().astype(np.float32)
        assert np.abs(a - b).max() <= 1e-2 * max(1.0, np.abs(b).max())
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, ROCM, H.DType.F16)


def test_required_mode_raises_instead_of_falling_back(torch_dev):
    H.configure_quant_linear(H.Qwen38QuantLinear.Rocm, ROCM, H.DType.F16)
    vb = H.VarStore(H.DType.F16, ROCM)
    vb.insert("layer.weight", _t(np.zeros((1, 7), np.uint8)))  # wrong packed length
    vb.insert("layer.weight_scale", _t(np.array([[0x38]], np.uint8)))
    vb.insert("layer.weight_scale_2", _t(np.array([1.0], np.float32)))
    with pytest.raises(H.DialError, match="invalid NVFP4 packed weight length 7"):
        H.linear_no_bias(16, 1, vb.pp("layer"))
    # Auto mode falls back to dense with a warning (and the length error of
    # the dense decoder)
    H.configure_quant_linear(H.Qwen38QuantLinear.Auto, ROCM, H.DType.F16)
    with pytest.raises(H.DialError, match="expected 8"):
        H.linear_no_bias(16, 1, vb.pp("layer"))
    assert "using dense fallback" in H.last_warning()
    H.configure_quant_linear(H.Qwen38QuantLinear.Dense, ROCM, H.DType.F16)


def test_quant_linears_match_dense_reference(torch_dev):
    # cuda_quant.rs:507-552
    in_dim, out_dim = 32, 3
    nvfp4 = H.RocmQuantLinear.nvfp4([0x22] * (out_dim * in_dim // 2), [0x38] * (out_dim * in_dim // 16),
                                    0.5, in_dim, out_dim, ROCM)
    fp8 = H.RocmQuantLinear.fp8([0x38] * (out_dim * in_dim), [0.5] * out_dim, in_dim, out_dim, ROCM)
    assert nvfp4.resident_bytes() == out_dim * in_dim // 2 + out_dim * in_dim // 16 + 4
    assert fp8.resident_bytes() == out_dim * in_dim + 4 * out_dim
    dense = H.Linear(_t(np.full((out_dim, in_dim), 0.5, np.float16)).to_device(ROCM))
    for rows in (1, 7):
        x = _t(np.sin(np.arange(rows * in_dim) * 0.07).astype(np.float16).reshape(rows, in_dim)).to_device(ROCM)
        expected = dense.forward(x).numpy().astype(np.float32)
        for lin in (nvfp4, fp8):
            actual = lin.forward(x).numpy().astype(np.float32)
            assert np.abs(expected - actual).max() < 0.02


def test_w8a16_text_linear_matches_dense_for_decode_and_prefill(torch_dev):
    # worker_w8a16.rs:483-516
    in_dim, out_dim = 64, 37
    idx = np.arange(out_dim * in_dim, dtype=np.float32)
    w = (np.sin(idx * 0.037) * 0.25 + ((idx % 11) - 5.0) * 0.002).astype(np.float16).reshape(out_dim, in_dim)
    dense = H.Linear(_t(w).to_device(ROCM))
    H.configure_worker_gguf_from_args(None, False, False, False, True, ROCM, H.DType.F16, 1)
    H.configure_worker_w8a16_from_args(True, True, ROCM, H.DType.F16)
    lin = H.TextLinear.from_dense("test.linear", dense)
    assert lin.is_w8a16()
    for rows in (1, 9):
        x = _t(np.cos(np.arange(rows * in_dim) * 0.071).astype(np.float32) * 0.5).reshape([1, rows, in_dim])
        x = _t(x.numpy().astype(np.float16)).to_device(ROCM)
        expected = dense.forward(x).numpy().astype(np.float32)
        actual = lin.forward(x).numpy().astype(np.float32)
        assert actual.shape == (1, rows, out_dim)
        assert np.abs(expected - actual).max() < 0.04, rows
    # W8A16 rejects F32 activations like the reference
    with pytest.raises(H.DialError, match="W8A16 expects F16 activation, got F32"):
        lin.forward(_t(np.zeros((1, in_dim), np.float32)).to_device(ROCM))
    H.configure_worker_w8a16_from_args(False, True, ROCM, H.DType.F16)
    assert H.TextLinear.from_dense("test.dense", dense).is_dense()


def _q4k_linear(offset):
    # worker_gguf.rs:636-647: Q4_K (2, 256) of (((i + off) % 37) - 18) / 19
    v = ((((np.arange(512) + offset) % 37).astype(np.float32) - 18.0) / 19.0).reshape(2, 256)
    return H.TextLinear.gguf(f"test.{offset}", H.GgufMatMul.quantize(H.GgufMatMul.Kind.Q4_K, _t(v), ROCM))


def test_q4k_decode_keeps_f16_activations(torch_dev):
    v = (((np.arange(512) % 37).astype(np.float32) - 18.0) / 19.0).reshape(2, 256)
    mm = H.GgufMatMul.quantize(H.GgufMatMul.Kind.Q4_K, _t(v), ROCM)
    x = _t(((np.arange(256) % 29 - 14.0) / 15.0).astype(np.float16).reshape(1, 1, 256)).to_device(ROCM)
    out = H.forward_worker_gguf(mm, x)
    assert out.dtype == H.DType.F16 and out.dims == [1, 1, 2]
    assert np.isfinite(out.numpy().astype(np.float32)).all()


def test_fused_fp16_prefill_matches_separate_dequantized_q4k_projections(torch_dev):
    first, second = _q4k_linear(0), _q4k_linear(11)
    first_dense = H.Linear(first.gguf_dequantize_f16_weight())
    second_dense = H.Linear(second.gguf_dequantize_f16_weight())
    fused = H.build_worker_gguf_fp16_prefill_linear("test.fused", [first, second])
    x = _t(((np.arange(768) % 23 - 11.0) / 12.0).astype(np.float16).reshape(1, 3, 256)).to_device(ROCM)
    expected = np.concatenate([first_dense.forward(x).numpy(), second_dense.forward(x).numpy()], axis=-1)
    actual = fused.forward(x).numpy()
    assert np.array_equal(actual.view(np.uint16), expected.view(np.uint16))


def test_hybrid_linear_keeps_q4k_for_single_token_decode(torch_dev):
    linear = _q4k_linear(7)
    fp16 = H.Linear(linear.gguf_dequantize_f16_weight())
    hybrid = linear.with_gguf_fp16_prefill(fp16)
    x = _t(((np.arange(256) % 29 - 14.0) / 15.0).astype(np.float16).reshape(1, 1, 256)).to_device(ROCM)
    expected = linear.forward(x).numpy()
    actual = hybrid.forward(x).numpy()
    assert np.array_equal(actual.view(np.uint16), expected.view(np.uint16))
    # several tokens take the dense FP16 copy
    x3 = _t(((np.arange(768) % 29 - 14.0) / 15.0).astype(np.float16).reshape(1, 3, 256)).to_device(ROCM)
    assert np.array_equal(hybrid.forward(x3).numpy().view(np.uint16), fp16.forward(x3).numpy().view(np.uint16))


def test_worker_gguf_file_linears_load_and_match_oracle(tmp_path, torch_dev):
    # worker_gguf.rs:65-180 (configure), 462-522 (load_worker_gguf_linear),
    # 524-572 (warm-up per GGUF dtype), 388-397 (summary), 425-452 (FP16
    # prefill copy): a Q4_K_M-style file mixing Q4K, Q6K and Q8_0 linears
    import oracle as O
    from gguf_writer import write_gguf
    rng = np.random.default_rng(5)
    h, i = 256, 512
    gate = O.q4_k_quantize(rng.normal(0, 0.02, (i, h)).astype(np.float32))
    up = O.q6_k_random_blocks(i, h, seed=7)
    down = O.q8_0_quantize(rng.normal(0, 0.02, (h, i)).astype(np.float32))
    deq = {"ffn_gate": O.q4_k_dequant(gate, i, h), "ffn_up": O.q6_k_dequant(up, i, h),
           "ffn_down": O.q8_0_dequant(down, h, i)}
    path = tmp_path / "tiny-q4_k_m.gguf"
    write_gguf(str(path), [("general.architecture", "STRING", "qwen3vl"), ("qwen3vl.block_count", "U32", 1)],
               [("blk.0.ffn_gate.weight", "Q4K", [i, h], gate.tobytes()),
                ("blk.0.ffn_up.weight", "Q6K", [i, h], up.tobytes()),
                ("blk.0.ffn_down.weight", "Q8_0", [h, i], down.tobytes())])
    try:
        H.configure_worker_gguf_from_args(str(path), True, False, False, True, ROCM, H.DType.F16, 1)
        lins = {name: H.load_worker_gguf_linear(0, name, *dims)
                for name, dims in (("ffn_gate", (h, i)), ("ffn_up", (h, i)), ("ffn_down", (i, h)))}
        assert all(l.is_gguf() for l in lins.values())
        assert H.worker_gguf_summary() == (3, gate.nbytes + up.nbytes + down.nbytes, 0, 0)
        for name, lin in lins.items():
            k = deq[name].shape[1]
            for rows in (1, 7):
                x = O.round_f16(rng.normal(0, 1, (rows, k)).astype(np.float32))
                out = lin.forward(_t(x.astype(np.float16).reshape(1, rows, k)).to_device(ROCM))
                assert out.dtype == H.DType.F16 and out.dims == [1, rows, deq[name].shape[0]]
                ref = O.round_f16(O.matmul_f64(x, deq[name]).astype(np.float32))
                assert O.rel_l2(out.numpy().astype(np.float32).reshape(rows, -1), ref) <= 1e-3, (name, rows)
            # the F16 prefill copy is the dequantized weight, rounded once
            w16 = lin.gguf_dequantize_f16_weight().numpy()
            assert np.array_equal(w16, O.round_f16(deq[name]).astype(np.float16))
        fused = H.build_worker_gguf_fp16_prefill_linear("blk.0.gate_up", [lins["ffn_gate"], lins["ffn_up"]])
        assert fused.weight().dims == [2 * i, h]
        assert H.worker_gguf_summary()[2:] == (1, 2 * i * h * 2)
    finally:
        H.configure_worker_gguf_from_args(None, False, False, False, True, ROCM, H.DType.F16, 1)


def test_linear_no_bias_from_safetensors_checkpoint(tmp_path, torch_dev):
    # The reference's KATs (quant.rs:564-594 ModelOpt NVFP4, 650-680
    # compressed-tensors NVFP4, 596-619 FP8 per-row) stored the way real
    # checkpoints store them -- U8 packed codes, F8_E4M3 weights and group
    # scales, F32 global / row scales -- in a safetensors file read by the
    # host layer's reader, then decoded dense and run quantized.
    import torch
    from safetensors.torch import save_file
    e4 = torch.float8_e4m3fn
    path = tmp_path / "model.safetensors"
    save_file({
        "model.layers.0.mlp.down_proj.weight": torch.full((1, 8), 0x92, dtype=torch.uint8),
        "model.layers.0.mlp.down_proj.weight_scale": torch.tensor([[2.0]]).to(e4),
        "model.layers.0.mlp.down_proj.weight_scale_2": torch.tensor([4.0]),
        "model.layers.0.mlp.up_proj.weight_packed": torch.full((1, 8), 0x92, dtype=torch.uint8),
        "model.layers.0.mlp.up_proj.weight_scale": torch.tensor([[2.0]]).to(e4),
        "model.layers.0.mlp.up_proj.weight_global_scale": torch.tensor([4.0]),
        "model.layers.0.self_attn.q_proj.weight": torch.tensor([[1.0, 2.0], [3.0, 4.0]]).to(e4),
        "model.layers.0.self_attn.q_proj.weight_scale": torch.tensor([2.0, 0.5]),
    }, str(path))
    try:
        H.configure_quant_linear(H.Qwen38QuantLinear.Dense, ROCM, H.DType.F32)
        vb = H.VarStore(H.DType.F32, ROCM)
        vb.load_safetensors([str(path)])
        layer = vb.pp("model").pp("layers").pp("0")
        assert _dense_values(H.linear_no_bias(16, 1, layer.pp("mlp").pp("down_proj"))) == [8.0, -4.0] * 8
        assert _dense_values(H.linear_no_bias(16, 1, layer.pp("mlp").pp("up_proj"))) == [0.5, -0.25] * 8
        assert _dense_values(H.linear_no_bias(2, 2, layer.pp("self_attn").pp("q_proj"))) == [2.0, 4.0, 1.5, 2.0]
        H.configure_quant_linear(H.Qwen38QuantLinear.Rocm, ROCM, H.DType.F16)
        vb16 = H.VarStore(H.DType.F16, ROCM)
        vb16.load_safetensors([str(path)])
        q = H.linear_no_bias(16, 1, vb16.pp("model.layers.0.mlp.down_proj"))
        assert q.is_quantized_rocm()
        x = _t(np.cos(np.arange(2 * 16) * 0.3).astype(np.float16).reshape(2, 16)).to_device(ROCM)
        got = q.forward(x).numpy().astype(np.float32).ravel()
        want = (np.cos(np.arange(2 * 16) * 0.3).astype(np.float16).astype(np.float64).reshape(2, 16)
                @ np.array([8.0, -4.0] * 8))
        assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max()
    finally:
        H.configure_quant_linear(H.Qwen38QuantLinear.Dense, ROCM, H.DType.F16)


def _head_ref(O, x_last, w16, deq, eps):
    # candle_nn::RmsNorm in f32 rounded to F16, then the quantized lm_head
    normed = O.round_f16(O.rms_norm(x_last.astype(np.float64), w16, eps).astype(np.float32))
    return O.matmul_f64(normed, deq)


def test_worker_gguf_output_head_matches_oracle(tmp_path, torch_dev):
    # worker_gguf.rs:754-787 (output_head_uses_last_hidden_and_quantized_
    # projection: Q4_K (2, 256) of (((i + 17) % 37) - 18) / 19, unit F16
    # norm, input (1, 3, 256) of ((i % 31) - 15) / 16, final block 35) read
    # from a GGUF file, then a tied token_embd.weight head with a learned norm
    # whose sampled-token route (:366-381) returns the argmax at temperature 0
    import oracle as O
    from gguf_writer import write_gguf
    meta = [("general.architecture", "STRING", "qwen3vl"), ("qwen3vl.block_count", "U32", 36)]
    v = ((((np.arange(512) + 17) % 37).astype(np.float32) - 18.0) / 19.0).reshape(2, 256)
    q4 = O.q4_k_quantize(v)
    path = tmp_path / "head-q4k.gguf"
    write_gguf(str(path), meta, [("output_norm.weight", "F32", [256], np.ones(256, np.float32).tobytes()),
                                 ("output.weight", "Q4K", [2, 256], q4.tobytes())])
    x = ((np.arange(768) % 31).astype(np.float32) - 15.0) / 16.0
    x16 = x.astype(np.float16).reshape(1, 3, 256)
    try:
        H.configure_worker_gguf_from_args(str(path), False, True, False, True, ROCM, H.DType.F16, 36)
        H.load_worker_gguf_output_head(H.OutputHeadConfig(256, 2, 36, 1e-6), True)
        assert H.worker_gguf_output_head_enabled() and not H.worker_gguf_sample_token_enabled()
        xt = _t(x16).to_device(ROCM)
        assert H.maybe_forward_worker_gguf_output_head(xt, 34) is None
        assert H.maybe_forward_worker_gguf_output_head(xt, None) is None
        got = H.maybe_forward_worker_gguf_output_head(xt, 35)
        assert got.dtype == H.DType.F16 and got.dims == [1, 2]
        ref = _head_ref(O, x16[0, 2:3].astype(np.float32), np.ones(256), O.q4_k_dequant(q4, 2, 256), 1e-6)
        assert O.rel_l2(got.numpy().astype(np.float32), O.round_f16(ref.astype(np.float32))) <= 1e-3
        # the [1, hidden] form is the same row
        row = H.maybe_forward_worker_gguf_output_head(_t(x16[0, 2:3].copy()).to_device(ROCM), 35)
        assert np.array_equal(row.numpy().view(np.uint16), got.numpy().view(np.uint16))
        with pytest.raises(H.DialError, match=r"expects \[1, seq, hidden\] or \[1, hidden\], got \[2, 256\]"):
            H.maybe_forward_worker_gguf_output_head(_t(x16[0, :2].copy()).to_device(ROCM), 35)

        rng = np.random.default_rng(9)
        hid, vocab = 512, 1000
        emb = O.q8_0_quantize(rng.normal(0, 0.05, (vocab, hid)).astype(np.float32))
        norm = rng.normal(1.0, 0.2, hid).astype(np.float32)
        path2 = tmp_path / "head-tied-q8.gguf"
        write_gguf(str(path2), meta, [("output_norm.weight", "F32", [hid], norm.tobytes()),
                                      ("token_embd.weight", "Q8_0", [vocab, hid], emb.tobytes())])
        H.configure_worker_gguf_from_args(str(path2), False, True, True, True, ROCM, H.DType.F16, 36)
        H.load_worker_gguf_output_head(H.OutputHeadConfig(hid, vocab, 36, 1e-5), True)
        assert H.worker_gguf_sample_token_enabled()
        xs = O.round_f16(rng.normal(0, 1, (1, 4, hid)).astype(np.float32))
        xt = _t(xs.astype(np.float16)).to_device(ROCM)
        with pytest.raises(H.DialError, match="did not send sampling parameters"):
            H.maybe_forward_worker_gguf_output_head(xt, 35)
        ref = _head_ref(O, xs[0, 3:4], O.round_f16(norm), O.q8_0_dequant(emb, vocab, hid), 1e-5)
        token = H.maybe_forward_worker_gguf_output_head(xt, 35, H.SamplingRequest(seed=1, temperature=0.0))
        assert isinstance(token, int)
        top2 = np.sort(ref[0])[-2:]
        assert top2[1] - top2[0] > 1e-2  # a clear winner, so rounding cannot flip it
        assert token == int(np.argmax(ref[0]))
    finally:
        H.configure_worker_gguf_from_args(None, False, False, False, True, ROCM, H.DType.F16, 1)
        H.load_worker_gguf_output_head(H.OutputHeadConfig(1, 1, 1), True)
        assert not H.worker_gguf_output_head_enabled()


def test_reconfigure_drops_a_loaded_output_head(tmp_path, torch_dev):
    # configure_worker_gguf_from_args clears the output-head slot and its
    # route-logged flag on every call (worker_gguf.rs:78-84): after a
    # reconfigure with output_head = false, in master mode or without a file,
    # no stale head keeps routing logits, with no load_worker_gguf_output_head
    # call in between
    import oracle as O
    from gguf_writer import write_gguf
    meta = [("general.architecture", "STRING", "qwen3vl"), ("qwen3vl.block_count", "U32", 36)]
    v = ((((np.arange(512) + 17) % 37).astype(np.float32) - 18.0) / 19.0).reshape(2, 256)
    path = tmp_path / "head.gguf"
    write_gguf(str(path), meta, [("output_norm.weight", "F32", [256], np.ones(256, np.float32).tobytes()),
                                 ("output.weight", "Q4K", [2, 256], O.q4_k_quantize(v).tobytes())])
    x16 = (((np.arange(256) % 31).astype(np.float32) - 15.0) / 16.0).astype(np.float16).reshape(1, 1, 256)
    reconfigure = [
        (str(path), False, False, False, True),   # same file, output head off
        (None, False, False, False, False),       # master mode
        (None, False, False, False, True),        # worker without a GGUF file
    ]
    try:
        for args in reconfigure:
            H.configure_worker_gguf_from_args(str(path), False, True, False, True, ROCM, H.DType.F16, 36)
            H.load_worker_gguf_output_head(H.OutputHeadConfig(256, 2, 36, 1e-6), True)
            assert H.worker_gguf_output_head_enabled()
            assert H.maybe_forward_worker_gguf_output_head(_t(x16).to_device(ROCM), 35) is not None
            H.configure_worker_gguf_from_args(*args, ROCM, H.DType.F16, 36)
            assert not H.worker_gguf_output_head_enabled(), args
            assert not H.worker_gguf_sample_token_enabled(), args
            assert H.maybe_forward_worker_gguf_output_head(_t(x16).to_device(ROCM), 35) is None, args
    finally:
        H.configure_worker_gguf_from_args(None, False, False, False, True, ROCM, H.DType.F16, 1)


@pytest.mark.parametrize("dtype", ["F16", "BF16", "F32"])
def test_dense_gguf_output_head_is_refused_with_a_message(tmp_path, dtype, torch_dev):
    # the ROCm GGUF path multiplies Q8_0 / Q4K / Q6K heads (the Q4_K_M and
    # Q8_0 exports the reference's docs use); a dense lm_head in the file is
    # refused at load time with a message naming the tensor and its dtype,
    # never at the first token
    from gguf_writer import write_gguf
    meta = [("general.architecture", "STRING", "qwen3vl"), ("qwen3vl.block_count", "U32", 36)]
    npd = {"F16": np.float16, "F32": np.float32}.get(dtype)
    raw = (np.zeros((4, 256), npd).tobytes() if npd is not None else np.zeros((4, 256), np.uint16).tobytes())
    path = tmp_path / f"head-{dtype}.gguf"
    write_gguf(str(path), meta, [("output_norm.weight", "F32", [256], np.ones(256, np.float32).tobytes()),
                                 ("output.weight", dtype, [4, 256], raw)])
    try:
        H.configure_worker_gguf_from_args(str(path), False, True, False, True, ROCM, H.DType.F16, 36)
        with pytest.raises(H.DialError, match=f"output.weight has dtype {dtype}; the ROCm GGUF path takes "
                                              "Q8_0, Q4K and Q6K"):
            H.load_worker_gguf_output_head(H.OutputHeadConfig(256, 4, 36, 1e-6), True)
        assert not H.worker_gguf_output_head_enabled()
    finally:
        H.configure_worker_gguf_from_args(None, False, False, False, True, ROCM, H.DType.F16, 1)
