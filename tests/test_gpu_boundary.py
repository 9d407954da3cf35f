"""The C ABI's input boundary on the GPU: activations given as views at any
start offset (candle's contiguous layouts carry a start_offset,
worker_w8a16.rs:419), and scratch growth under stream capture.

A view at a 16-byte-aligned offset (row r of a [R, K] tensor) is read in
place; one at any other address is copied by the library into the handle's
aligned staging buffer first.  Either way the output must be bit-identical
to the same values given at an aligned address: the same kernels run on the
same numbers."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import make_weight, reference_product, to_torch

pytestmark = pytest.mark.gpu

TDT = {dq.F32: "float32", dq.F16: "float16", dq.BF16: "bfloat16"}


def _flat_with_offset(torch, x, dtype, elem_off, dev):
    """A [rows, K] view whose first element sits `elem_off` elements into a
    fresh flat buffer (the allocation itself is 256-byte aligned)."""
    rows, k = x.shape
    buf = torch.full((rows * k + elem_off + 8,), float("nan"), device=dev, dtype=getattr(torch, TDT[dtype]))
    v = buf[elem_off:elem_off + rows * k].view(rows, k)
    v.copy_(to_torch(x, dtype, dev))
    return v


@pytest.mark.parametrize("fmt,rows,path", [
    (dq.W8A16, 1, dq.PATH_GEMV), (dq.W8A16, 5, dq.PATH_GEMV), (dq.W8A16, 130, dq.PATH_GEMM),
    (dq.Q4_K, 1, dq.PATH_GEMV), (dq.Q4_K, 200, dq.PATH_GEMM),
    (dq.MXFP4, 3, dq.PATH_GEMV), (dq.MXFP4, 256, dq.PATH_GEMM_NATIVE),
    (dq.FP8_BLOCK, 256, dq.PATH_GEMM_NATIVE)], ids=lambda v: str(v))
@pytest.mark.parametrize("x_dtype", [dq.BF16, dq.F32], ids=["bf16", "f32"])
def test_forward_from_offset_views(fmt, rows, path, x_dtype, torch_dev):
    import torch
    n, k = 320, 512
    raw, scales, kw, deq = make_weight(fmt, n, k, seed=31 + fmt)
    lin = dq.Linear.create(fmt, n, k, raw, scales, **kw)
    rng = np.random.default_rng(rows)
    x = O.round_bf16(rng.normal(0, 1, (rows, k)).astype(np.float32))
    y_al = torch.empty(rows, n, device=torch_dev, dtype=torch.bfloat16)
    lin.forward(to_torch(x, x_dtype, torch_dev), y_al, path=path)
    torch.cuda.synchronize()
    if path != dq.PATH_GEMM_NATIVE:  # the native path quantizes x first; its parity lives elsewhere
        assert O.rel_l2(y_al.float().cpu().numpy(), reference_product(x, deq, dq.BF16)) <= 1e-3
    # row 1 of a [rows + 2, K] tensor: aligned, read in place
    big = to_torch(np.concatenate([x[:1] * 0 + 7, x, x[:1]]), x_dtype, torch_dev)
    views = [big[1:1 + rows]]
    # offsets of 1 and 3 elements: 2 / 6 bytes (bf16), 4 / 12 bytes (f32)
    views += [_flat_with_offset(torch, x, x_dtype, off, torch_dev) for off in (1, 3)]
    for v in views:
        assert v.is_contiguous()
        y = torch.full((rows, n), float("nan"), device=torch_dev, dtype=torch.bfloat16)
        lin.forward(v, y, path=path)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_al.view(torch.int16)), (v.data_ptr() % 16)


def test_misaligned_x_in_capture_needs_an_eager_call_first(torch_dev):
    # the aligned staging buffer of a handle grows outside capture only (like
    # its decode workspace): the first capture of a larger misaligned x fails
    # with a message, and after one eager call of that shape captures replay
    # correctly
    import torch
    n, k, rows = 256, 1024, 4
    raw, scales, kw, deq = make_weight(dq.W8A16, n, k, seed=5)
    lin = dq.Linear.create(dq.W8A16, n, k, raw, scales, **kw)
    x = O.round_bf16(np.random.default_rng(2).normal(0, 1, (rows, k)).astype(np.float32))
    xv = _flat_with_offset(torch, x, dq.BF16, 1, torch_dev)
    y = torch.empty(rows, n, device=torch_dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(dq.DialqError, match="during stream capture"):
        with torch.cuda.graph(g):
            lin.forward(xv, y, path=dq.PATH_GEMV, stream=torch.cuda.current_stream())
    lin.forward(xv, y, path=dq.PATH_GEMV)  # eager: sizes the staging buffer
    torch.cuda.synchronize()
    want = y.clone()
    assert O.rel_l2(want.float().cpu().numpy(), reference_product(x, deq, dq.BF16)) <= 1e-3
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lin.forward(xv, y, path=dq.PATH_GEMV, stream=torch.cuda.current_stream())
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)


def test_weights_past_2_gib_are_refused_on_every_path(torch_dev):
    # every kernel addresses the resident tiles with 32-bit buffer offsets and
    # masks loads with the offset 2^31: a handle of 2 GiB or more is refused
    # with a message at forward time, decode and prefill alike (the largest
    # DIAL linear, the 27B lm_head in W8A16, is 1.27 GB)
    import torch
    n, k = 262144 + 16, 8192  # 2,147,614,720 bytes of int8 codes, 2^31 + 131072
    codes = torch.zeros(n, k, dtype=torch.int8, device=torch_dev)
    scales = torch.ones(n, dtype=torch.float32, device=torch_dev)
    lin = dq.Linear.create(dq.W8A16, n, k, codes, scales)
    del codes
    x = torch.zeros(32, k, dtype=torch.bfloat16, device=torch_dev)
    y = torch.empty(32, n, dtype=torch.bfloat16, device=torch_dev)
    for rows, kind in ((1, "decode"), (32, "prefill")):
        with pytest.raises(dq.DialqError, match=kind + r" kernel addresses weights with 32-bit offsets"):
            lin.forward(x[:rows], y[:rows])
    lin.close()
