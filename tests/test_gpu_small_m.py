"""Small row counts (17..256) on the prefill GEMM: too few row blocks to fill
the GPU, so the W8A16 / FP8_ROW GEMM takes 32-row tiles up to 96 rows and
splits every tile along K into pieces (up to 8 where K is long) whose
partials the last piece adds in piece order.  Checked against the fp64
oracle on sampled output columns, against the unsplit decode kernel, under
graph replay (the per-tile counters must re-arm), with the SwiGLU epilogue,
and through the allocation-free entry point.  The automatic path takes the
decode kernel up to 16 rows and the GEMM above."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import make_weight, reference_product, to_torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", [dq.W8A16, dq.FP8_ROW], ids=["w8a16", "fp8_row"])
@pytest.mark.parametrize("m", [17, 32, 64, 96, 100, 130, 256])
@pytest.mark.parametrize("n,k", [(4096, 5120), (1024, 17408)], ids=["k5120", "k17408"])
def test_split_k_gemm_matches_oracle(fmt, m, n, k, torch_dev):
    import torch
    raw, scales, kw, deq = make_weight(fmt, n, k, seed=m)
    lin = dq.Linear.create(fmt, n, k, raw, scales, **kw)
    rng = np.random.default_rng(m)
    x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
    cols = np.sort(rng.choice(n, 192, replace=False))
    ref = reference_product(x, deq[cols], dq.BF16)
    for x_dtype, y_dtype, tol in ((dq.BF16, dq.BF16, 1e-3), (dq.F16, dq.F16, 1e-3), (dq.F32, dq.F32, 1e-5)):
        xt = to_torch(x, x_dtype, torch_dev)
        y = torch.full((m, n), float("nan"), device=torch_dev,
                       dtype={dq.BF16: torch.bfloat16, dq.F16: torch.float16, dq.F32: torch.float32}[y_dtype])
        lin.forward(xt, y)  # AUTO: the GEMM above 16 rows
        torch.cuda.synchronize()
        got = y[:, torch.from_numpy(cols).to(torch_dev)].float().cpu().numpy()
        want = reference_product(x, deq[cols], y_dtype)
        assert O.rel_l2(got, want) <= tol, (m, x_dtype)
        assert not np.isnan(got).any()
    # the split GEMM and the decode kernel agree
    yg = torch.empty(m, n, device=torch_dev, dtype=torch.bfloat16)
    yv = torch.empty(m, n, device=torch_dev, dtype=torch.bfloat16)
    xt = to_torch(x, dq.BF16, torch_dev)
    lin.forward(xt, yg, path=dq.PATH_GEMM)
    lin.forward(xt, yv, path=dq.PATH_GEMV)
    torch.cuda.synchronize()
    assert O.rel_l2(yg.float().cpu().numpy(), yv.float().cpu().numpy()) <= 2e-3
    assert O.rel_l2(yg[:, torch.from_numpy(cols).to(torch_dev)].float().cpu().numpy(), ref) <= 1e-3


def test_split_k_gemm_graph_replay_and_noalloc(torch_dev):
    # replays of a captured split GEMM reproduce the eager output bit for bit
    # (the tile counters are left zero by every launch), with other split
    # launches of the same handle between them; the allocation-free entry
    # point gives the same bits
    import torch
    n, k, m = 17408, 5120, 48
    g = torch.Generator(device=torch_dev).manual_seed(3)
    lin = dq.Linear.quantize(dq.W8A16, torch.randn(n, k, device=torch_dev, generator=g) * 0.02, scale_dtype=dq.BF16)
    x = torch.randn(m, k, device=torch_dev, generator=g).to(torch.bfloat16)
    x2 = torch.randn(24, k, device=torch_dev, generator=g).to(torch.bfloat16)
    y = torch.empty(m, n, device=torch_dev, dtype=torch.bfloat16)
    y2 = torch.empty(24, n, device=torch_dev, dtype=torch.bfloat16)
    lin.forward(x, y, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    want = y.clone()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        lin.forward(x, y, path=dq.PATH_GEMM, stream=torch.cuda.current_stream())
    for _ in range(3):
        y.zero_()
        lin.forward(x2, y2, path=dq.PATH_GEMM)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    yn = torch.full_like(y, float("nan"))
    lin.forward_noalloc(x, yn, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    assert torch.equal(yn.view(torch.int16), want.view(torch.int16))


def test_split_k_swiglu(torch_dev):
    # a fused gate_up weight at few rows: the SwiGLU epilogue runs in the
    # piece that adds the partials
    import torch
    i_dim, k, m = 2048, 5120, 33
    raw, scales, kw, deq = make_weight(dq.W8A16, 2 * i_dim, k, seed=8)
    lin = dq.Linear.create(dq.W8A16, 2 * i_dim, k, raw, scales, **kw)
    x = O.round_bf16(np.random.default_rng(8).normal(0, 1, (m, k)).astype(np.float32))
    y = torch.full((m, i_dim), float("nan"), device=torch_dev, dtype=torch.float32)
    lin.forward_swiglu(to_torch(x, dq.BF16, torch_dev), y, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    gu = O.matmul_f64(x, deq)
    want = O.swiglu(gu).astype(np.float32)
    assert O.rel_l2(y.cpu().numpy(), want) <= 1e-5
