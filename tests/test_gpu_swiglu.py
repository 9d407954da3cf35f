"""GPU parity of the fused gate_up projection with the SwiGLU epilogue
(dialq_linear_forward_swiglu) against the oracle: the fp64 product of the
exact activations and the dequantized fused weight, then oracle.swiglu
(Mlp::mlp_mid_from_gate_up, qwen3_vl/text.rs:816-820), rounded to the output
dtype.

Bars as for the plain products: 1e-3 relative L2 for the weight-only paths
(decode GEMV and the bf16 GEMMs), 2e-3 for the native fp8 / fp4 prefill,
whose oracle applies the same activation quantizer.  Intermediate widths
I = 64 and 192 leave the last column tile of every GEMM kernel partly empty
(8 strips per half), and I = 192 starts the up half inside a 128-row FP8
block."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import empty_out, exact_inputs, make_weight, to_torch

pytestmark = pytest.mark.gpu

ALL_FORMATS = [dq.W8A16, dq.Q8_0, dq.Q4_K, dq.Q6_K, dq.FP8_ROW, dq.FP8_BLOCK, dq.NVFP4, dq.MXFP4]
TOL_BF16 = 1e-3
TOL_LOWP = 2e-3


def _rounded(y, y_dtype):
    y = np.asarray(y, np.float32)
    if y_dtype == dq.BF16:
        return O.round_bf16(y)
    if y_dtype == dq.F16:
        return O.round_f16(y)
    return y


def _fused(fmt, inter, k, seed):
    raw, scales, ckw, deq = make_weight(fmt, 2 * inter, k, seed)
    return dq.Linear.create(fmt, 2 * inter, k, raw, scales, **ckw), deq


def _native_x(fmt, x):
    if fmt == dq.FP8_BLOCK:
        q, s = O.act_fp8_quantize(x)
        return O.e4m3_to_f32(q) * s[:, None]
    p, s = O.act_mxfp4_quantize(x)
    return O.mxfp4_dequant(p, s)


def _check(lin, deq, m, path, x_dtype, y_dtype, dev, seed, native=None):
    import torch
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (m, lin.in_dim)).astype(np.float32)
    xe = exact_inputs(x, x_dtype)
    yt = empty_out(m, lin.out_dim // 2, y_dtype, dev)
    lin.forward_swiglu(to_torch(x, x_dtype, dev), yt, path=path)
    torch.cuda.synchronize()
    got = yt.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    xr = _native_x(native, xe) if native else xe
    if lin.desc.format in (dq.Q4_K, dq.Q8_0, dq.Q6_K) and path == dq.PATH_GEMM and x_dtype != dq.F32:
        deq = O.round_f16(deq)  # the GGUF prefill multiplies the f16-dequantized weight
    ref = _rounded(O.swiglu(O.matmul_f64(xr, deq)), y_dtype)
    return O.rel_l2(got, ref)


@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_swiglu_decode_gemv(fmt, torch_dev):
    """Decode: one workgroup per gate / up strip pair, 1..16 rows per pass and
    a second pass at 20 rows; staged and unstaged activations (K = 512 and
    K = 8192 at 16 rows)."""
    for inter, k in ((192, 512), (64, 8192)):
        lin, deq = _fused(fmt, inter, k, seed=200 + fmt)
        for m in (1, 3, 8, 16, 20):
            rel = _check(lin, deq, m, dq.PATH_GEMV, dq.BF16, dq.BF16, torch_dev, seed=m)
            assert rel <= TOL_BF16, (dq.FORMAT_NAMES[fmt], inter, k, m, rel)


@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_swiglu_prefill_gemm(fmt, torch_dev):
    """Weight-only prefill GEMM: gate waves and up waves of one column tile
    meet in LDS; ragged row tiles (M = 100) and a full one (M = 256)."""
    for inter in (64, 192):
        lin, deq = _fused(fmt, inter, 768, seed=220 + fmt)
        for m in (100, 256):
            rel = _check(lin, deq, m, dq.PATH_GEMM, dq.BF16, dq.BF16, torch_dev, seed=m)
            assert rel <= TOL_BF16, (dq.FORMAT_NAMES[fmt], inter, m, rel)


@pytest.mark.parametrize("fmt", [dq.FP8_BLOCK, dq.MXFP4], ids=["fp8_block", "mxfp4"])
def test_swiglu_native_prefill(fmt, torch_dev):
    """Native fp8 / fp4 prefill, whole tiles (K = 640) and split-K tiles whose
    last-arriving piece runs the epilogue (K = 8192)."""
    for inter, k, ms in ((192, 640, (100, 256)), (64, 8192, (45, 300))):
        lin, deq = _fused(fmt, inter, k, seed=240 + fmt)
        for m in ms:
            rel = _check(lin, deq, m, dq.PATH_GEMM_NATIVE, dq.BF16, dq.BF16, torch_dev, seed=m, native=fmt)
            assert rel <= TOL_LOWP, (dq.FORMAT_NAMES[fmt], inter, k, m, rel)


@pytest.mark.parametrize("x_dtype,y_dtype", [(dq.F16, dq.F32), (dq.F32, dq.F16)], ids=["f16-f32", "f32-f16"])
def test_swiglu_dtypes(x_dtype, y_dtype, torch_dev):
    lin, deq = _fused(dq.W8A16, 128, 512, seed=260)
    for m, path in ((2, dq.PATH_GEMV), (130, dq.PATH_GEMM)):
        rel = _check(lin, deq, m, path, x_dtype, y_dtype, torch_dev, seed=m)
        assert rel <= TOL_BF16, (m, path, rel)


def test_swiglu_auto_path_matches_fused_then_silu(torch_dev):
    """PATH_AUTO against the plain fused product followed by silu * up on the
    host, the reference's unfused sequence (gate_up_proj.forward, narrow,
    silu, mul), both in f32."""
    import torch
    lin, _ = _fused(dq.Q4_K, 256, 1024, seed=270)
    for m in (1, 7, 96):
        rng = np.random.default_rng(m)
        x = to_torch(rng.normal(0, 1, (m, 1024)).astype(np.float32), dq.BF16, torch_dev)
        gu = empty_out(m, 512, dq.F32, torch_dev)
        lin.forward(x, gu)
        fused = empty_out(m, 256, dq.F32, torch_dev)
        lin.forward_swiglu(x, fused)
        torch.cuda.synchronize()
        want = O.swiglu(gu.cpu().numpy())
        assert O.rel_l2(fused.cpu().numpy(), want) <= 1e-5, m


def test_swiglu_rejects_unaligned_width(torch_dev):
    raw, scales, ckw, _ = make_weight(dq.W8A16, 96, 256, 1)
    lin = dq.Linear.create(dq.W8A16, 96, 256, raw, scales, **ckw)
    import torch
    x = torch.zeros(1, 256, dtype=torch.bfloat16, device=torch_dev)
    y = torch.zeros(1, 48, dtype=torch.bfloat16, device=torch_dev)
    with pytest.raises(dq.DialqError, match="multiple of 128"):
        lin.forward_swiglu(x, y)
