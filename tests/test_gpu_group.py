"""dialq_linear_forward_group: y = cat([x W_j^T], -1) for handles that share
x, the replacement of QkvProjection::Split / MlpGateUpProjection::Split
(qwen3_vl/text.rs:1093-1101, :451-455).  Paths that run one launch per
member (mixed formats, prefill formats without a grouped kernel) must
equal each member's own dialq_linear_forward_ex output bit for bit (the
same kernels with a strided output).  A grouped launch -- decode, or
prefill of W8A16 / FP8_ROW / Q4_K, Q8_0 and Q6_K (bf16, f16 x) / FP8_BLOCK and MXFP4
native -- sizes its split along K from all the group's tiles, so a
member's f32 sum may be split differently than in its own launch: those
columns must agree with its own forward to f32 rounding (rel-L2 <= 2e-4 in
bf16) and with the oracle (<= 1e-3).  Covered: decode row counts, prefill
row counts, mixed formats, more members than one launch takes, misaligned
and host inputs, the full 27B q / k / v and gate / up shapes."""
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


def _agree(got, want, exact, what):
    """Bit-exact for per-member launches; f32 rounding for a grouped one."""
    import torch
    if exact:
        assert torch.equal(_bits(got), _bits(want)), what
    else:
        assert O.rel_l2(got.float().cpu().numpy(), want.float().cpu().numpy()) <= 2e-4, what


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
        # decode: one grouped launch per row group of 16 (8 for the k-quants
        # at M <= 8); prefill: one launch where a grouped kernel exists
        prefill_grouped = fmts[0] in (dq.W8A16, dq.MXFP4) or (fmts[0] in (dq.Q4_K, dq.Q6_K) and x_dtype != dq.F32)
        grouped = len(set(fmts)) == 1 and (rows <= 16 or prefill_grouped)
        xt = to_torch(x, x_dtype, torch_dev)
        want = _separate(lins, xt, dq.BF16, dq.PATH_AUTO, torch_dev)
        got = torch.full_like(want, float("nan"))
        before = dq.grouped_launches()
        dq.forward_group(lins, xt, got)
        torch.cuda.synchronize()
        assert (dq.grouped_launches() > before) == grouped, (rows, fmts, x_dtype)
        _agree(got, want, not grouped, (x_dtype, rows))
    # and against the weight-only oracle, where the product is weight-only
    # (MXFP4 above 16 rows takes the native path, which quantizes x too)
    if not (rows > 16 and dq.MXFP4 in fmts):
        ref = np.concatenate([reference_product(x, d, dq.BF16) for d in deqs], axis=1)
        assert O.rel_l2(got.float().cpu().numpy(), ref) <= 1e-3


def test_group_native_prefill_and_output_dtypes(torch_dev):
    # native: one grouped launch on x quantized once; weight-only FP8_BLOCK
    # (k_gemm): one launch per member, bit for bit
    import torch
    k = 1024
    lins, _ = _members((dq.FP8_BLOCK, dq.FP8_BLOCK), (256, 128), k, seed=3)
    x = to_torch(O.round_bf16(np.random.default_rng(1).normal(0, 1, (300, k)).astype(np.float32)), dq.BF16,
                 torch_dev)
    for y_dtype in (dq.BF16, dq.F16, dq.F32):
        for path in (dq.PATH_GEMM_NATIVE, dq.PATH_GEMM):
            want = _separate(lins, x, y_dtype, path, torch_dev)
            got = torch.full_like(want, float("nan"))
            before = dq.grouped_launches()
            dq.forward_group(lins, x, got, path=path)
            torch.cuda.synchronize()
            grouped = path == dq.PATH_GEMM_NATIVE
            assert (dq.grouped_launches() == before + 1) == grouped, (y_dtype, path)
            _agree(got, want, not grouped, (y_dtype, path))


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
    _agree(got, want, False, "six members")


def test_group_misaligned_and_host_inputs(torch_dev):
    import torch
    k = 512
    lins, deqs = _members((dq.W8A16,) * 3, (384, 64, 64), k, seed=9)
    x = O.round_bf16(np.random.default_rng(4).normal(0, 1, (1, k)).astype(np.float32))
    want = _separate(lins, to_torch(x, dq.BF16, torch_dev), dq.BF16, dq.PATH_GEMV, torch_dev)
    buf = torch.empty(k + 9, device=torch_dev, dtype=torch.bfloat16)
    xv = buf[1:1 + k].view(1, k)
    xv.copy_(to_torch(x, dq.BF16, torch_dev))
    aligned = torch.full_like(want, float("nan"))
    dq.forward_group(lins, to_torch(x, dq.BF16, torch_dev), aligned)
    got = torch.full_like(want, float("nan"))
    dq.forward_group(lins, xv, got)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(aligned))  # the same grouped launch on the same values
    _agree(got, want, False, "misaligned")
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
    with pytest.raises(dq.DialqError, match="handle 1 is the same handle as 0"):
        dq.forward_group(a + a, x, y)


@pytest.mark.parametrize("group", [[6144, 1024, 1024], [17408, 17408]], ids=["qkv", "gate_up"])
@pytest.mark.parametrize("fmt", [dq.W8A16, dq.Q4_K, dq.MXFP4], ids=lambda f: dq.FORMAT_NAMES[f])
def test_group_27b_shapes(group, fmt, torch_dev):
    # one grouped launch per row group: every member agrees with its own
    # forward to f32 rounding (its strips may be split into k pieces and over
    # waves differently), and with the oracle on sampled rows
    import torch
    k = 5120
    g = torch.Generator(device=torch_dev).manual_seed(7)
    lins = [dq.Linear.quantize(fmt, torch.randn(n, k, device=torch_dev, generator=g) * 0.02, scale_dtype=dq.BF16)
            for n in group]
    for rows in (1, 8):
        x = torch.randn(rows, k, device=torch_dev, generator=g).to(torch.bfloat16)
        want = _separate(lins, x, dq.BF16, dq.PATH_GEMV, torch_dev)
        got = torch.full_like(want, float("nan"))
        before = dq.grouped_launches()
        dq.forward_group(lins, x, got, path=dq.PATH_GEMV)
        torch.cuda.synchronize()
        if rows == 1:  # the benchmark's decode: must be one grouped launch
            assert dq.grouped_launches() == before + 1
        _agree(got, want, False, rows)


@pytest.mark.parametrize("group", [[6144, 1024, 1024], [17408, 17408]], ids=["qkv", "gate_up"])
@pytest.mark.parametrize("fmt,x_dtype,path", [(dq.W8A16, dq.BF16, dq.PATH_GEMM), (dq.FP8_ROW, dq.BF16, dq.PATH_GEMM),
                                              (dq.Q4_K, dq.F16, dq.PATH_GEMM), (dq.Q4_K, dq.BF16, dq.PATH_GEMM),
                                              (dq.Q8_0, dq.BF16, dq.PATH_GEMM),
                                              (dq.FP8_BLOCK, dq.BF16, dq.PATH_GEMM_NATIVE),
                                              (dq.MXFP4, dq.BF16, dq.PATH_GEMM_NATIVE)],
                         ids=["w8a16", "fp8_row", "q4_k_f16", "q4_k_bf16", "q8_0_bf16", "fp8_block", "mxfp4"])
def test_group_prefill_27b_shapes(group, fmt, x_dtype, path, torch_dev):
    # prefill of DIAL's split projections: one grouped launch over every
    # member's column tiles (small and large row counts: split along K or
    # not), each member within f32 rounding of its own forward
    import torch
    k = 5120
    g = torch.Generator(device=torch_dev).manual_seed(17)
    lins = []
    for n in group:
        if fmt == dq.FP8_ROW:
            raw, scales, kw, _ = make_weight(dq.FP8_ROW, n, k, seed=n)
            lins.append(dq.Linear.create(dq.FP8_ROW, n, k, raw, scales, **kw))
        else:
            lins.append(dq.Linear.quantize(fmt, torch.randn(n, k, device=torch_dev, generator=g) * 0.02,
                                           scale_dtype=dq.BF16))
    tdt = torch.float16 if x_dtype == dq.F16 else torch.bfloat16
    for rows in (40, 300):
        x = torch.randn(rows, k, device=torch_dev, generator=g).to(tdt)
        want = _separate(lins, x, x_dtype, path, torch_dev)
        got = torch.full_like(want, float("nan"))
        before = dq.grouped_launches()
        dq.forward_group(lins, x, got, path=path)
        torch.cuda.synchronize()
        assert dq.grouped_launches() == before + 1, rows
        _agree(got, want, False, (rows, path))
