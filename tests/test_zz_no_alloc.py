"""dialq_linear_forward_noalloc: the allocation-free variant of
dialq_linear_forward_ex, for callers that cannot allocate (graph capture,
serving loops).  Its output must equal the existing entry point's bit for
bit (the same kernels on the same numbers, with the scratch taken from the
library's static per-device array instead of the handle's buffers), on two
calls in a row with the second smaller, for every path that uses scratch:
decode whole strips, the decode work queue (workspace + counters), the
weight-only GEMM (whole, and with its last round of tiles split along K),
the native fp8 / fp4 prefill with split-K partials, and a misaligned x.
It must refuse sizes beyond the array with a message, leave
the handle's own scratch untouched, and replay correctly from a graph."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import make_weight, to_torch

pytestmark = pytest.mark.gpu


def _lin(fmt, n, k, seed):
    raw, scales, kw, _ = make_weight(fmt, n, k, seed=seed)
    return dq.Linear.create(fmt, n, k, raw, scales, **kw)


def _x(rows, k, seed, dtype=dq.BF16, dev=None, elem_off=0):
    import torch
    x = O.round_bf16(np.random.default_rng(seed).normal(0, 1, (rows, k)).astype(np.float32))
    t = to_torch(x, dtype, dev)
    if elem_off:
        buf = torch.empty(rows * k + elem_off + 8, device=dev, dtype=t.dtype)
        v = buf[elem_off:elem_off + rows * k].view(rows, k)
        v.copy_(t)
        return v
    return t


def _both(lin, x, n, path, dev):
    """(forward_ex output, forward_noalloc output) as int16 bit patterns."""
    import torch
    rows = x.shape[0]
    want = torch.full((rows, n), float("nan"), device=dev, dtype=torch.bfloat16)
    got = torch.full((rows, n), float("nan"), device=dev, dtype=torch.bfloat16)
    lin.forward(x, want, path=path)
    before = lin.device_bytes()
    lin.forward_noalloc(x, got, path=path)
    torch.cuda.synchronize()
    assert lin.device_bytes() == before  # nothing grew on the handle
    return want.view(torch.int16), got.view(torch.int16)


# (format, [(n, k, rows, path, x element offset), second call smaller])
CASES = {
    "decode_whole_strips": (dq.W8A16, [(4096, 5120, 1, dq.PATH_GEMV, 0), (1024, 2048, 1, dq.PATH_GEMV, 0)]),
    "decode_work_queue": (dq.W8A16, [(1024, 8704, 8, dq.PATH_GEMV, 0), (512, 8704, 4, dq.PATH_GEMV, 0)]),
    "decode_q4k_rows": (dq.Q4_K, [(4096, 4096, 8, dq.PATH_GEMV, 0), (256, 4096, 3, dq.PATH_GEMV, 0)]),
    "gemm": (dq.Q8_0, [(640, 1024, 300, dq.PATH_GEMM, 0), (640, 1024, 130, dq.PATH_GEMM, 0)]),
    # 544 tiles of 128 rows on 512 slots: the last round's 32 tiles split
    # along K, their partials (16 MB) in the array
    "gemm_tail_split": (dq.W8A16, [(8704, 1024, 2048, dq.PATH_GEMM, 0), (8704, 1024, 1024, dq.PATH_GEMM, 0)]),
    # Q4_K on bf16 x: the f16 copy of x and its row scales in the array
    "gemm_q4k_bf16": (dq.Q4_K, [(1024, 2048, 300, dq.PATH_GEMM, 0), (512, 2048, 40, dq.PATH_GEMM, 0)]),
    "native_fp8_split_k": (dq.FP8_BLOCK, [(1024, 5120, 512, dq.PATH_GEMM_NATIVE, 0),
                                          (1024, 2048, 256, dq.PATH_GEMM_NATIVE, 0)]),
    "native_mxfp4_split_k": (dq.MXFP4, [(1024, 5120, 512, dq.PATH_GEMM_NATIVE, 0),
                                        (512, 5120, 200, dq.PATH_GEMM_NATIVE, 0)]),
    "misaligned_x": (dq.W8A16, [(2048, 4096, 5, dq.PATH_GEMV, 1), (2048, 4096, 2, dq.PATH_GEMV, 3)]),
}


@pytest.mark.parametrize("case", list(CASES))
def test_noalloc_matches_forward_ex(case, torch_dev):
    import torch
    fmt, calls = CASES[case]
    for i, (n, k, rows, path, off) in enumerate(calls):
        lin = _lin(fmt, n, k, seed=100 + i)
        x = _x(rows, k, seed=7 + i, dev=torch_dev, elem_off=off)
        want, got = _both(lin, x, n, path, torch_dev)
        assert torch.equal(got, want), (case, i)
        lin.close()


def test_noalloc_runs_an_unfitting_tail_split_whole(torch_dev):
    # 1088 tiles of 128 rows on 512 slots: the allocating entry point splits
    # the last 64 tiles into 4 pieces (32 MiB of partials); beside the
    # counters that does not fit the 32 MiB array, so the allocation-free
    # call runs those tiles whole -- the same products summed in another
    # order: f32 rounding apart, and both within the oracle's bar
    import torch
    from helpers import reference_product
    n, k, rows = 17408, 1024, 2048
    raw, scales, kw, deq = make_weight(dq.W8A16, n, k, seed=21)
    lin = dq.Linear.create(dq.W8A16, n, k, raw, scales, **kw)
    x = O.round_bf16(np.random.default_rng(22).normal(0, 1, (rows, k)).astype(np.float32))
    xt = to_torch(x, dq.BF16, torch_dev)
    want = torch.empty(rows, n, device=torch_dev, dtype=torch.float32)
    got = torch.empty_like(want)
    lin.forward(xt, want, path=dq.PATH_GEMM)
    lin.forward_noalloc(xt, got, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    w_, g_ = want.cpu().numpy(), got.cpu().numpy()
    assert O.rel_l2(g_, w_) <= 1e-6
    ref = reference_product(x, deq, dq.F32)
    assert O.rel_l2(g_, ref) <= 1e-5 and O.rel_l2(w_, ref) <= 1e-5
    lin.close()


def test_noalloc_refuses_beyond_its_scratch(torch_dev):
    import torch
    # native fp8 prefill of 2048 rows at K = 17408: 35.7 MB of activation
    # codes alone, over the 32 MiB array
    n, k = 512, 17408
    lin = dq.Linear.quantize(dq.FP8_BLOCK, torch.randn(n, k, device=torch_dev) * 0.02)
    x = torch.randn(2048, k, device=torch_dev).to(torch.bfloat16)
    y = torch.empty(2048, n, device=torch_dev, dtype=torch.bfloat16)
    with pytest.raises(dq.DialqError, match=r"need \d+ bytes of scratch; the allocation-free entry point has 33554432"):
        lin.forward_noalloc(x, y, path=dq.PATH_GEMM_NATIVE)
    # the same call through the allocating entry point works, and a smaller
    # one through the allocation-free one still does afterwards
    lin.forward(x, y, path=dq.PATH_GEMM_NATIVE)
    want, got = _both(lin, x[:256].contiguous(), n, dq.PATH_GEMM_NATIVE, torch_dev)
    assert torch.equal(got, want)


def test_noalloc_replays_from_a_graph(torch_dev):
    # the caller it exists for: a decode step captured once and replayed,
    # with eager work of other handles (sharing the array) between replays
    import torch
    lin = _lin(dq.W8A16, 1024, 8704, seed=3)          # work-queue decode: workspace + counters
    other = _lin(dq.FP8_BLOCK, 1024, 5120, seed=4)    # native split-K: partials + counters
    x = _x(8, 8704, seed=5, dev=torch_dev)
    xo = _x(300, 5120, seed=6, dev=torch_dev)
    y = torch.empty(8, 1024, device=torch_dev, dtype=torch.bfloat16)
    yo = torch.empty(300, 1024, device=torch_dev, dtype=torch.bfloat16)
    want = torch.empty_like(y)
    lin.forward(x, want, path=dq.PATH_GEMV)
    lin.forward_noalloc(x, y, path=dq.PATH_GEMV)      # eager first (sets the array up)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lin.forward_noalloc(x, y, path=dq.PATH_GEMV, stream=torch.cuda.current_stream())
    for _ in range(3):
        y.fill_(float("nan"))
        other.forward_noalloc(xo, yo, path=dq.PATH_GEMM_NATIVE)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)
