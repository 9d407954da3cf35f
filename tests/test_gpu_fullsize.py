"""Parity at the full benchmark shapes: 8B-class GGUF matvec (12288x4096,
4096x12288), the 8B W8A16 layer, the 27B layer (hidden 5120, q 6144,
k/v 1024, o 5120x6144, gate/up 17408x5120, down 5120x17408) in W8A16 /
Q4_K / FP8-128 / MXFP4 at decode and prefill row counts.

Weights are N(0, 0.02) quantized on the GPU (the quantizers are bit-exact
against the oracle at small sizes, test_gpu_parity.py); the exported raw
bytes of a random sample of 96 output rows are dequantized by the oracle and
multiplied in fp64, so the full-size check stays cheap on the CPU."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import exact_inputs, to_torch

pytestmark = pytest.mark.gpu

SAMPLE = 96

SHAPES_8B_GGUF = [(12288, 4096), (4096, 12288)]
SHAPES_8B_LAYER = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288)]
SHAPES_27B = [(6144, 5120), (1024, 5120), (5120, 6144), (17408, 5120), (5120, 17408)]


def _oracle_rows(fmt, w, s, rows, n, k):
    """Dequantize `rows` of the exported raw weight with the oracle."""
    if fmt == dq.W8A16:
        return O.w8a16_dequant(w[rows], s[rows])
    if fmt == dq.Q8_0:
        return O.q8_0_dequant(w[rows], len(rows), k)
    if fmt == dq.Q4_K:
        return O.q4_k_dequant(w[rows], len(rows), k)
    if fmt == dq.FP8_BLOCK:
        out = O.e4m3_to_f32(w[rows].ravel()).reshape(len(rows), k)
        return out * np.repeat(s[rows // 128], 128, 1)[:, :k]
    if fmt == dq.MXFP4:
        return O.mxfp4_dequant(w[rows], s[rows])
    raise ValueError(fmt)


def _check_quantizer_bytes(fmt, dense_rows, w, s, rows):
    """The device quantizer's exported bytes for the sampled rows against the
    oracle's quantizer on the same dense values.  FP8-128 scales cover
    128-row blocks, so its sample is whole blocks (`rows` is then a range of
    block-aligned rows)."""
    if fmt == dq.W8A16:
        q, _, sb = O.w8a16_quantize(dense_rows)
        assert np.array_equal(w[rows], q) and np.array_equal(np.asarray(s)[rows].view(np.uint16), sb)
    elif fmt == dq.Q8_0:
        assert np.array_equal(w[rows], O.q8_0_quantize(dense_rows))
    elif fmt == dq.Q4_K:
        assert np.array_equal(w[rows], O.q4_k_quantize(dense_rows))
    elif fmt == dq.MXFP4:
        p, sx = O.mxfp4_quantize(dense_rows)
        assert np.array_equal(w[rows], p) and np.array_equal(np.asarray(s)[rows], sx)
    elif fmt == dq.FP8_BLOCK:
        q, sx = O.fp8_block_quantize(dense_rows)
        assert np.array_equal(w[rows], q)
        assert np.array_equal(np.asarray(s)[rows[0] // 128:rows[-1] // 128 + 1].view(np.uint32), sx.view(np.uint32))
    else:
        raise ValueError(fmt)


def _check(fmt, n, k, m, torch_dev, path=dq.PATH_AUTO, tol=1e-3, native=False, seed=0, quant_bytes=True):
    import torch
    g = torch.Generator(device=torch_dev).manual_seed(seed)
    wd = torch.randn(n, k, device=torch_dev, generator=g, dtype=torch.float32) * 0.02
    lin = dq.Linear.quantize(fmt, wd, scale_dtype=dq.BF16)
    rng = np.random.default_rng(seed + m)
    rows = np.sort(rng.choice(n, SAMPLE, replace=False))
    if quant_bytes:
        # the dense values of the sampled rows (whole 128-row blocks for
        # FP8-128: the first and the last block row) stay on the host
        if fmt == dq.FP8_BLOCK:
            qrows = np.concatenate([np.arange(b * 128, b * 128 + 128) for b in sorted({0, (n - 1) // 128})])
            qrows = qrows[qrows < n]
        else:
            qrows = rows
        dense_rows = wd[torch.from_numpy(qrows).to(torch_dev)].cpu().numpy()
    del wd
    w, s = lin.export()
    if quant_bytes:
        if fmt == dq.FP8_BLOCK:
            for b in sorted({0, (n - 1) // 128}):
                sel = (qrows >= b * 128) & (qrows < b * 128 + 128)
                _check_quantizer_bytes(fmt, dense_rows[sel], w, s, qrows[sel])
        else:
            _check_quantizer_bytes(fmt, dense_rows, w, s, qrows)
    deq = _oracle_rows(fmt, w, s, rows, n, k)
    x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
    xt = to_torch(x, dq.BF16, torch_dev)
    yt = torch.empty(m, n, dtype=torch.bfloat16, device=torch_dev)
    lin.forward(xt, yt, path=path)
    torch.cuda.synchronize()
    got = yt[:, torch.from_numpy(rows).to(torch_dev)].float().cpu().numpy()
    if native:
        if fmt == dq.FP8_BLOCK:
            q, sx = O.act_fp8_quantize(x)
            x = O.e4m3_to_f32(q.ravel()).reshape(m, k) * sx[:, None]
        else:
            p, sx = O.act_mxfp4_quantize(x)
            x = O.mxfp4_dequant(p, sx)
    ref = O.round_bf16((x.astype(np.float64) @ deq.astype(np.float64).T).astype(np.float32))
    rel = O.rel_l2(got, ref)
    assert rel <= tol, (dq.FORMAT_NAMES[fmt], n, k, m, rel)


@pytest.mark.parametrize("shape", SHAPES_8B_GGUF, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("fmt", [dq.Q4_K, dq.Q8_0], ids=["q4_k", "q8_0"])
def test_gguf_matvec_8b(fmt, shape, torch_dev):
    for m in (1, 4, 8):
        _check(fmt, shape[0], shape[1], m, torch_dev)


def test_w8a16_decode_6144x2048(torch_dev):
    _check(dq.W8A16, 6144, 2048, 1, torch_dev)


@pytest.mark.parametrize("shape", SHAPES_8B_LAYER, ids=lambda s: f"{s[0]}x{s[1]}")
def test_w8a16_prefill_8b_layer(shape, torch_dev):
    for m in (512, 2048):
        _check(dq.W8A16, shape[0], shape[1], m, torch_dev)


@pytest.mark.parametrize("shape", SHAPES_27B, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("fmt", [dq.W8A16, dq.Q4_K], ids=["w8a16", "q4_k"])
def test_27b_layer_sweep(fmt, shape, torch_dev):
    for m in (1, 8, 256, 2048):
        _check(fmt, shape[0], shape[1], m, torch_dev)


@pytest.mark.parametrize("shape", SHAPES_27B, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("fmt", [dq.FP8_BLOCK, dq.MXFP4], ids=["fp8_block", "mxfp4"])
def test_27b_lowp_decode_and_prefill(fmt, shape, torch_dev):
    _check(fmt, shape[0], shape[1], 1, torch_dev)
    _check(fmt, shape[0], shape[1], 1024, torch_dev, tol=2e-3, native=True)


@pytest.mark.parametrize("shape", SHAPES_8B_GGUF + [(5120, 17408), (1024, 5120)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_q6_k_full_size(shape, torch_dev):
    # Q6_K comes from GGUF files only (no quantizer on the path): seeded
    # random blocks, created through the C ABI's repacker
    import torch
    n, k = shape
    blocks = O.q6_k_random_blocks(n, k, seed=n + k)
    lin = dq.Linear.create(dq.Q6_K, n, k, blocks, None)
    rng = np.random.default_rng(n)
    rows = np.sort(rng.choice(n, SAMPLE, replace=False))
    deq = O.q6_k_dequant(blocks[rows], SAMPLE, k)
    for m in (1, 4, 8, 256):
        x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
        yt = torch.empty(m, n, dtype=torch.bfloat16, device=torch_dev)
        lin.forward(to_torch(x, dq.BF16, torch_dev), yt)
        torch.cuda.synchronize()
        got = yt[:, torch.from_numpy(rows).to(torch_dev)].float().cpu().numpy()
        ref = O.round_bf16((x.astype(np.float64) @ deq.astype(np.float64).T).astype(np.float32))
        assert O.rel_l2(got, ref) <= 1e-3, (n, k, m)


@pytest.mark.parametrize("fmt", [dq.W8A16, dq.MXFP4], ids=["w8a16", "mxfp4"])
def test_lm_head_27b(fmt, torch_dev):
    # the quantized output head (vocab 248320 x hidden 5120,
    # qwen3_8/model.rs:433-438): 1.27 GB of W8A16 tiles, the largest GEMV
    for m in (1, 8):
        _check(fmt, 248320, 5120, m, torch_dev)
