"""dialq_linear_forward_group: y = cat([x W_j^T], -1) for handles that share
x, the replacement of QkvProjection::Split / MlpGateUpProjection::Split
(qwen3_vl/text.rs:1093-1101, :451-455).  Every member's columns must equal
its own dialq_linear_forward_ex output bit for bit -- the grouped decode
launch runs the same per-strip arithmetic with the same waves per strip
(see test_group_27b_shapes for the one exception), the other paths the same
kernels with a strided output -- for decode row counts (one grouped launch),
prefill row counts (one launch per member), mixed formats, more members than
one launch takes, misaligned and host inputs, and the full 27B q / k / v and
gate / up shapes."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import make_weight, reference_product, to_torch

pytestmark = pytest.mark.gpu

TDT = {dq.F32: "float32", dq.F16: "float16", dq.BF16: "bfloat16"}


def _members(fmts, ns, k, seed):
    lins, deqs = [], []
    for i, (fmt, n) in enumerate(zip(fmts, ns)):
        raw, scales, kw, deq = make_weight(fmt, n, k, seed=seed + i)
        lins.append(dq.Linear.create(fmt, n, k, raw, scales, **kw))
        deqs.append(deq)
    return lins, deqs


def _separate(lins, x, y_dtype, path, dev):
    import torch
    outs = []
    for lin in lins:
        y = torch.full((x.shape[0], lin.out_dim), float("nan"), device=dev, dtype=getattr(torch, TDT[y_dtype]))
        lin.forward(x, y, path=path)
        outs.append(y)
    return torch.cat(outs, dim=1)


def _bits(t):
    import torch
    return t.view(torch.int16) if t.dtype != torch.float32 else t.view(torch.int32)


@pytest.mark.parametrize("fmts", [(dq.W8A16,) * 3, (dq.Q4_K,) * 3, (dq.MXFP4,) * 2, (dq.Q6_K,) * 2,
                                  (dq.W8A16, dq.Q8_0, dq.W8A16)],
                         ids=["w8a16_qkv", "q4k_qkv", "mxfp4_gate_up", "q6k_pair", "mixed"])
@pytest.mark.parametrize("rows", [1, 3, 8, 16, 40, 200])
def test_group_equals_separate(fmts, rows, torch_dev):
    import torch
    k = 512
    ns = [384, 64, 64][:len(fmts)] if len(fmts) == 3 else [320, 320]
    lins, deqs = _members(fmts, ns, k, seed=11 * rows)
    x = O.round_bf16(np.random.default_rng(rows).normal(0, 1, (rows, k)).astype(np.float32))
    for x_dtype in (dq.BF16, dq.F16, dq.F32):
        xt = to_torch(x, x_dtype, torch_dev)
        want = _separate(lins, xt, dq.BF16, dq.PATH_AUTO, torch_dev)
        got = torch.full_like(want, float("nan"))
        dq.forward_group(lins, xt, got)
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(want)), (x_dtype, rows)
    # and against the weight-only oracle, where the product is weight-only
    # (MXFP4 above 64 rows takes the native path, which quantizes x too)
    if not (rows > 64 and dq.MXFP4 in fmts):
        ref = np.concatenate([reference_product(x, d, dq.BF16) for d in deqs], axis=1)
        assert O.rel_l2(got.float().cpu().numpy(), ref) <= 1e-3


def test_group_native_prefill_and_output_dtypes(torch_dev):
    import torch
    k = 1024
    lins, _ = _members((dq.FP8_BLOCK, dq.FP8_BLOCK), (256, 128), k, seed=3)
    x = to_torch(O.round_bf16(np.random.default_rng(1).normal(0, 1, (300, k)).astype(np.float32)), dq.BF16,
                 torch_dev)
    for y_dtype in (dq.BF16, dq.F16, dq.F32):
        for path in (dq.PATH_GEMM_NATIVE, dq.PATH_GEMM):
            want = _separate(lins, x, y_dtype, path, torch_dev)
            got = torch.full_like(want, float("nan"))
            dq.forward_group(lins, x, got, path=path)
            torch.cuda.synchronize()
            assert torch.equal(_bits(got), _bits(want)), (y_dtype, path)


def test_group_of_more_members_than_one_launch(torch_dev):
    # six members: a grouped launch of four, then one of two
    import torch
    k = 256
    lins, _ = _members((dq.W8A16,) * 6, (48, 16, 160, 32, 64, 96), k, seed=5)
    x = to_torch(O.round_bf16(np.random.default_rng(2).normal(0, 1, (2, k)).astype(np.float32)), dq.BF16, torch_dev)
    want = _separate(lins, x, dq.BF16, dq.PATH_GEMV, torch_dev)
    got = torch.full_like(want, float("nan"))
    dq.forward_group(lins, x, got, path=dq.PATH_GEMV)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


def test_group_misaligned_and_host_inputs(torch_dev):
    import torch
    k = 512
    lins, deqs = _members((dq.W8A16,) * 3, (384, 64, 64), k, seed=9)
    x = O.round_bf16(np.random.default_rng(4).normal(0, 1, (1, k)).astype(np.float32))
    want = _separate(lins, to_torch(x, dq.BF16, torch_dev), dq.BF16, dq.PATH_GEMV, torch_dev)
    buf = torch.empty(k + 9, device=torch_dev, dtype=torch.bfloat16)
    xv = buf[1:1 + k].view(1, k)
    xv.copy_(to_torch(x, dq.BF16, torch_dev))
    got = torch.full_like(want, float("nan"))
    dq.forward_group(lins, xv, got)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))
    # host buffers: staged over PCIe, same kernels
    yh = np.full((1, 512), np.nan, np.float32)
    dq.forward_group(lins, x, yh, x_dtype=dq.F32, y_dtype=dq.F32)
    ref = np.concatenate([reference_product(x, d, dq.F32) for d in deqs], axis=1)
    assert O.rel_l2(yh, ref) <= 1e-5


def test_group_rejects_mismatched_members(torch_dev):
    import torch
    a, _ = _members((dq.W8A16,), (64,), 512, seed=1)
    b, _ = _members((dq.W8A16,), (64,), 256, seed=2)
    x = torch.zeros(1, 512, device=torch_dev, dtype=torch.bfloat16)
    y = torch.zeros(1, 128, device=torch_dev, dtype=torch.bfloat16)
    with pytest.raises(dq.DialqError, match="handle 1 has in_dim 256, handle 0 has 512"):
        dq.forward_group(a + b, x, y)


@pytest.mark.parametrize("group", [[6144, 1024, 1024], [17408, 17408]], ids=["qkv", "gate_up"])
@pytest.mark.parametrize("fmt", [dq.W8A16, dq.Q4_K, dq.MXFP4], ids=lambda f: dq.FORMAT_NAMES[f])
def test_group_27b_shapes(group, fmt, torch_dev):
    # A strip's sum is split over the waves of its workgroup (tile t goes to
    # wave t mod W).  Alone, k and v (64 strips, fewer than the CUs) launch
    # with 8 waves; in the q / k / v launch (512 strips) every strip runs with
    # the 4 waves q uses alone, so k and v agree with their own forward to
    # f32 rounding, not bit for bit.  q, gate and up are bit-exact.
    import torch
    k = 5120
    g = torch.Generator(device=torch_dev).manual_seed(7)
    lins = [dq.Linear.quantize(fmt, torch.randn(n, k, device=torch_dev, generator=g) * 0.02, scale_dtype=dq.BF16)
            for n in group]
    for rows in (1, 8):
        x = torch.randn(rows, k, device=torch_dev, generator=g).to(torch.bfloat16)
        want = _separate(lins, x, dq.BF16, dq.PATH_GEMV, torch_dev)
        got = torch.full_like(want, float("nan"))
        dq.forward_group(lins, x, got, path=dq.PATH_GEMV)
        torch.cuda.synchronize()
        off = 0
        for lin in lins:
            a, b = got[:, off:off + lin.out_dim], want[:, off:off + lin.out_dim]
            if lin.out_dim // 16 >= 256 or len(group) == 2:
                assert torch.equal(_bits(a), _bits(b)), (rows, lin.out_dim)
            else:
                assert O.rel_l2(a.float().cpu().numpy(), b.float().cpu().numpy()) <= 2e-4, (rows, lin.out_dim)
            off += lin.out_dim
