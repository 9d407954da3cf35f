"""The reference's own GPU tests, restated against the HIP path:
worker_w8a16.rs:483-516, cuda_quant.rs:507-552 and
examples/qwen38_quant_smoke.rs (f16 activations and outputs, max-abs bars
against a dense f16 linear)."""
import json
import math
import os

import numpy as np
import pytest

import dialq as dq
import oracle as O

pytestmark = pytest.mark.gpu
KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def _dense_f16_linear(x_f16, w_f16):
    """candle's dense f16 Linear: f16 operands, wide accumulation, f16 out."""
    y = x_f16.astype(np.float64) @ w_f16.astype(np.float64).T
    return y.astype(np.float32).astype(np.float16).astype(np.float32)


def _forward_f16(lin, x_f16, torch_dev, path=dq.PATH_AUTO):
    import torch
    xt = torch.from_numpy(x_f16).to(torch_dev)
    yt = torch.empty(x_f16.shape[0], lin.out_dim, dtype=torch.float16, device=torch_dev)
    lin.forward(xt, yt, path=path)
    torch.cuda.synchronize()
    return yt.float().cpu().numpy()


@pytest.mark.parametrize("path", [dq.PATH_AUTO, dq.PATH_GEMV, dq.PATH_GEMM], ids=["auto", "gemv", "gemm"])
def test_w8a16_matches_dense(path, torch_dev):
    import torch
    k = KATS["w8a16_dense_match"]
    n, kk = k["out_dim"], k["in_dim"]
    w = np.array([math.sin(i * 0.037) * 0.25 + ((i % 11) - 5.0) * 0.002 for i in range(n * kk)],
                 np.float32).reshape(n, kk).astype(np.float16)
    lin = dq.Linear.quantize(dq.W8A16, torch.from_numpy(w).to(torch_dev), scale_dtype=dq.F32)
    for rows in k["rows"]:
        x = np.array([math.cos(i * 0.071) * 0.5 for i in range(rows * kk)], np.float32)
        x = x.reshape(rows, kk).astype(np.float16)
        got = _forward_f16(lin, x, torch_dev, path)
        assert np.abs(got - _dense_f16_linear(x, w)).max() < k["max_abs"], rows


def test_cuda_quant_linears_match_dense(torch_dev):
    k = KATS["cuda_quant_dense_match"]
    n, kk = k["out_dim"], k["in_dim"]
    nv = dq.Linear.create(dq.NVFP4, n, kk, np.full(n * kk // 2, k["nvfp4_packed_byte"], np.uint8),
                          np.full(n * kk // 16, k["nvfp4_scale_byte"], np.uint8),
                          global_scale=k["nvfp4_global"])
    f8 = dq.Linear.create(dq.FP8_ROW, n, kk, np.full(n * kk, k["fp8_byte"], np.uint8),
                          np.full(n, k["fp8_scale"], np.float32))
    w = np.full((n, kk), k["dense_value"], np.float16)
    for rows in k["rows"]:
        x = np.array([math.sin(i * 0.07) for i in range(rows * kk)], np.float32).reshape(rows, kk).astype(np.float16)
        want = _dense_f16_linear(x, w)
        for lin in (nv, f8):
            assert np.abs(_forward_f16(lin, x, torch_dev) - want).max() < k["max_abs"]


def test_quant_smoke_example(torch_dev):
    k = KATS["quant_smoke"]
    n, kk = k["out_dim"], k["in_dim"]
    packed = np.array([k["packed_pattern"][i % 8] for i in range(n * kk // 2)], np.uint8)
    scales = np.array([k["scale_pattern"][i % 6] for i in range(n * kk // 16)], np.uint8)
    nv = dq.Linear.create(dq.NVFP4, n, kk, packed, scales, global_scale=k["nvfp4_global"])
    nv_dense = O.nvfp4_dequant(packed, scales, k["nvfp4_global"], n, kk, scales_are_e4m3=True)
    fp8 = np.array([k["fp8_pattern"][i % 8] for i in range(n * kk)], np.uint8)
    fs = np.array(k["fp8_scales"], np.float32)
    f8 = dq.Linear.create(dq.FP8_ROW, n, kk, fp8, fs)
    f8_dense = O.e4m3_to_f32(fp8, ocp=True).reshape(n, kk) * fs[:, None]
    for rows in k["rows"]:
        x = np.array([math.sin(i * 0.07) for i in range(rows * kk)], np.float32).reshape(rows, kk).astype(np.float16)
        for lin, dense in ((nv, nv_dense), (f8, f8_dense)):
            want = _dense_f16_linear(x, dense.astype(np.float16))
            assert np.abs(_forward_f16(lin, x, torch_dev) - want).max() < k["max_abs"]


def test_compressed_tensors_global_divisor(torch_dev):
    """quant.rs:322-329: weight_global_scale is a divisor; multiplier = 1/g."""
    import torch
    k = KATS["compressed_tensors_nvfp4"]
    lin = dq.Linear.create(dq.NVFP4, k["out_dim"], k["in_dim"], np.array(k["packed"], np.uint8),
                           O.f32_to_e4m3(np.array(k["scales_f32"], np.float32)).astype(np.uint8),
                           global_scale=k["global_divisor"], flags=dq.FLAG_GLOBAL_IS_DIVISOR)
    out = torch.empty(k["out_dim"], k["in_dim"], dtype=torch.float32, device=torch_dev)
    lin.dequantize(out)
    assert list(out.cpu().numpy().ravel()) == k["expect"]


def test_modelopt_nvfp4_dequant(torch_dev):
    import torch
    k = KATS["modelopt_nvfp4"]
    lin = dq.Linear.create(dq.NVFP4, k["out_dim"], k["in_dim"], np.array(k["packed"], np.uint8),
                           O.f32_to_e4m3(np.array(k["scales_f32"], np.float32)).astype(np.uint8),
                           global_scale=k["global_scale"])
    out = torch.empty(k["out_dim"], k["in_dim"], dtype=torch.float32, device=torch_dev)
    lin.dequantize(out)
    assert list(out.cpu().numpy().ravel()) == k["expect"]


def test_fp8_per_row_dequant(torch_dev):
    import torch
    k = KATS["fp8_per_row_scale"]
    codes = O.f32_to_e4m3(np.array(k["weight_values"], np.float32)).astype(np.uint8)
    lin = dq.Linear.create(dq.FP8_ROW, k["out_dim"], k["in_dim"] * 4, np.repeat(codes.reshape(2, 2), 4, 1),
                           np.array(k["scales"], np.float32))
    out = torch.empty(k["out_dim"], k["in_dim"] * 4, dtype=torch.float32, device=torch_dev)
    lin.dequantize(out)
    got = out.cpu().numpy()[:, ::4].ravel()
    assert list(got) == k["expect"]
