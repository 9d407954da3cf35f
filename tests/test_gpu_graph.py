"""Decode GEMV launches captured in a HIP graph (torch.cuda.CUDAGraph) and
replayed, as a serving loop runs them: every replay must reproduce the eager
result bit for bit, with unrelated eager work and synchronisations between
the replays.  Covers the whole-strip kernel (>= one strip per CU) and the
work-queue kernel (small matrices), whose queue and piece counters are reset
by the kernels themselves (no memset nodes in the graph)."""
import numpy as np
import pytest

import dialq as dq
from helpers import make_weight

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", [dq.W8A16, dq.Q4_K, dq.MXFP4], ids=lambda f: dq.FORMAT_NAMES[f])
@pytest.mark.parametrize("n", [200, 16 * 300 + 7], ids=["queue", "whole_strips"])
def test_graph_replay_matches_eager(fmt, n, torch_dev):
    import torch
    k = 1024
    raw, scales, ckw, _ = make_weight(fmt, n, k, 60 + fmt)
    lin = dq.Linear.create(fmt, n, k, raw, scales, **ckw)
    other = dq.Linear.create(fmt, n, k, raw, scales, **ckw)
    for m in (1, 5):
        x = torch.randn(m, k, device=torch_dev).to(torch.bfloat16)
        y_eager = torch.empty(m, n, device=torch_dev, dtype=torch.bfloat16)
        y_graph = torch.empty_like(y_eager)
        y_other = torch.empty_like(y_eager)
        stream = torch.cuda.current_stream()
        lin.forward(x, y_eager, path=dq.PATH_GEMV, stream=stream)
        lin.forward(x, y_graph, path=dq.PATH_GEMV, stream=stream)  # sizes the workspace
        torch.cuda.synchronize()
        ref = y_eager.cpu()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            lin.forward(x, y_graph, path=dq.PATH_GEMV, stream=torch.cuda.current_stream())
        for rep in range(4):
            y_graph.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y_graph.cpu(), ref), (dq.FORMAT_NAMES[fmt], n, m, rep)
            # eager work between replays, on the same weights' workspace and others
            lin.forward(x * 2, y_other, path=dq.PATH_GEMV, stream=stream)
            other.forward(x, y_other, path=dq.PATH_GEMV, stream=stream)
            torch.cuda.synchronize()
            assert np.isfinite(y_other.float().cpu().numpy()).all()


@pytest.mark.parametrize("fmt", [dq.FP8_BLOCK, dq.MXFP4], ids=lambda f: dq.FORMAT_NAMES[f])
def test_graph_replay_native_prefill(fmt, torch_dev):
    """The native prefill's stream-K schedule splits tiles between
    workgroups; their per-tile arrival counters are reset by the last
    arriver, so graph replays reproduce the eager result bit for bit."""
    import torch
    n, k, m = 300, 8192, 300  # 64 chunks: FP8 tiles split in 8 pieces, MXFP4 in 2
    raw, scales, ckw, _ = make_weight(fmt, n, k, 70 + fmt)
    lin = dq.Linear.create(fmt, n, k, raw, scales, **ckw)
    x = torch.randn(m, k, device=torch_dev).to(torch.bfloat16)
    y_eager = torch.empty(m, n, device=torch_dev, dtype=torch.bfloat16)
    y_graph = torch.empty_like(y_eager)
    stream = torch.cuda.current_stream()
    lin.forward(x, y_eager, path=dq.PATH_GEMM_NATIVE, stream=stream)  # sizes the scratch
    torch.cuda.synchronize()
    ref = y_eager.cpu()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lin.forward(x, y_graph, path=dq.PATH_GEMM_NATIVE, stream=torch.cuda.current_stream())
    for rep in range(4):
        y_graph.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph.cpu(), ref), (dq.FORMAT_NAMES[fmt], rep)
        lin.forward(x * 2, y_eager, path=dq.PATH_GEMM_NATIVE, stream=stream)
        torch.cuda.synchronize()


def test_work_queue_give_up_is_reported_by_the_next_forward(torch_dev):
    # The decode work-queue kernel (small N whose activations are too large to
    # stage: 1024 x 8704 at M = 8) bounds every wait.  With the limit forced to
    # zero from the host its waits give up at once and every wave still ends
    # normally; the launch marks its handle, the next forward reports it and
    # resets the queue counters, and the call after that is correct again.
    import torch
    from helpers import make_weight, reference_product, to_torch
    import oracle as O
    n, k, m = 1024, 8704, 8
    raw, scales, kw, deq = make_weight(dq.W8A16, n, k, seed=17)
    lin = dq.Linear.create(dq.W8A16, n, k, raw, scales, **kw)
    x = O.round_bf16(np.random.default_rng(4).normal(0, 1, (m, k)).astype(np.float32))
    xt = to_torch(x, dq.BF16, torch_dev)
    y = torch.empty(m, n, device=torch_dev, dtype=torch.bfloat16)
    ref = reference_product(x, deq, dq.BF16)
    lin.forward(xt, y, path=dq.PATH_GEMV)
    torch.cuda.synchronize()
    assert O.rel_l2(y.float().cpu().numpy(), ref) <= 1e-3
    try:
        dq.set_wait_limit(0)
        y.fill_(float("nan"))
        lin.forward(xt, y, path=dq.PATH_GEMV)  # gives up: output incomplete, handle marked
        torch.cuda.synchronize()
    finally:
        dq.set_wait_limit(-1)
    with pytest.raises(dq.DialqError, match="gave up waiting for its work queue"):
        lin.forward(xt, y, path=dq.PATH_GEMV)
    for _ in range(2):
        y.fill_(float("nan"))
        lin.forward(xt, y, path=dq.PATH_GEMV)
        torch.cuda.synchronize()
        assert O.rel_l2(y.float().cpu().numpy(), ref) <= 1e-3
