"""GGUF prefill (k_gemm_kq: Q4_K, Q8_0, Q6_K): each weight is dequantized in
f32 (Q4_K d*sc*q - dmin*m, Q8_0 d*q, Q6_K d*sc*(q - 32)) and multiplied as
f16 against f16
activations -- the weight DIAL's GGUF prefill builds once,
build_worker_gguf_fp16_prefill_linear
(qwen3_vl/worker_gguf.rs:426-455).  bf16 activations are first written as
f16 rows scaled by a power of two that puts each row's maximum at the top
of f16's range (k_x_f16_rows; the scale multiplies the row's outputs), or,
where the allocation-free entry point
has no room for that copy, multiply the f32 weight as a bf16 hi + lo pair.
Pinned on the same inputs:
  * f16 and bf16 x: against the fp64 product with the f16-rounded
    dequantized weight (the hybrid prefill's weight), to f32 accumulation
    (rel-L2 <= 2e-5; a weight rounded once from the exact value instead of
    through f32 may differ by one f16 ulp in rare ties), row by row for rows
    far outside f16 range;
  * the hi + lo kernel against the exact product (rel-L2 <= 2e-5);
  * all against the exact oracle to the weight-only bar (1e-3).
Row counts cover the 32-row tiles (<= 96 rows, split along K), the 128-row
tiles, ragged row blocks, SwiGLU and graph replay of a split launch."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import make_weight, reference_product, to_torch

pytestmark = pytest.mark.gpu


FMTS = [dq.Q4_K, dq.Q8_0, dq.Q6_K]
IDS = ["q4_k", "q8_0", "q6_k"]


def _case(n, k, seed, fmt=dq.Q4_K):
    raw, scales, kw, deq = make_weight(fmt, n, k, seed=seed)
    return dq.Linear.create(fmt, n, k, raw, scales, **kw), deq


@pytest.mark.parametrize("fmt", FMTS, ids=IDS)
@pytest.mark.parametrize("m", [17, 40, 96, 97, 130, 256, 300])
@pytest.mark.parametrize("n,k", [(320, 512), (1024, 5120)], ids=["k512", "k5120"])
def test_kq_prefill_weights_and_parity(fmt, m, n, k, torch_dev):
    import torch
    lin, deq = _case(n, k, seed=m + k, fmt=fmt)
    rng = np.random.default_rng(m)
    x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))  # exact in bf16 and f16
    for x_dtype in (dq.F16, dq.BF16):
        y = torch.full((m, n), float("nan"), device=torch_dev, dtype=torch.float32)
        lin.forward(to_torch(x, x_dtype, torch_dev), y, path=dq.PATH_GEMM)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        exact = O.matmul_f64(x, deq)
        hybrid = O.matmul_f64(x, O.round_f16(deq))
        assert O.rel_l2(got, hybrid) <= 2e-5, (m, x_dtype, "f16 weights")
        assert O.rel_l2(got, exact) <= 1e-3
        # bf16 / f16 outputs of the same launch
        y_dtype = dq.F16 if x_dtype == dq.F16 else dq.BF16
        yo = torch.empty(m, n, device=torch_dev, dtype=torch.float16 if x_dtype == dq.F16 else torch.bfloat16)
        lin.forward(to_torch(x, x_dtype, torch_dev), yo, path=dq.PATH_GEMM)
        torch.cuda.synchronize()
        # rounded outputs against the hybrid weight's product, rounded alike
        # (against the exact weight, one-ulp flips of the rounding sit at the bar)
        assert O.rel_l2(yo.float().cpu().numpy(), reference_product(x, O.round_f16(deq), y_dtype)) <= 1e-3


@pytest.mark.parametrize("fmt", FMTS, ids=IDS)
def test_kq_prefill_f32_activations_stay_exact(fmt, torch_dev):
    # f32 activations keep the exact weight-only kernel
    import torch
    lin, deq = _case(256, 512, seed=3, fmt=fmt)
    x = np.random.default_rng(3).normal(0, 1, (70, 512)).astype(np.float32)
    y = torch.empty(70, 256, device=torch_dev, dtype=torch.float32)
    lin.forward(torch.from_numpy(x).to(torch_dev), y, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    assert O.rel_l2(y.cpu().numpy(), O.matmul_f64(x, deq)) <= 1e-5


@pytest.mark.parametrize("fmt", FMTS, ids=IDS)
@pytest.mark.parametrize("m", [33, 200])
def test_kq_prefill_swiglu(fmt, m, torch_dev):
    import torch
    i_dim, k = 512, 1024
    lin, deq = _case(2 * i_dim, k, seed=m, fmt=fmt)
    x = O.round_bf16(np.random.default_rng(m).normal(0, 1, (m, k)).astype(np.float32))
    for x_dtype in (dq.F16, dq.BF16):
        y = torch.full((m, i_dim), float("nan"), device=torch_dev, dtype=torch.float32)
        lin.forward_swiglu(to_torch(x, x_dtype, torch_dev), y, path=dq.PATH_GEMM)
        torch.cuda.synchronize()
        want = O.swiglu(O.matmul_f64(x, deq))
        assert O.rel_l2(y.cpu().numpy(), want) <= 1e-3, x_dtype


def test_q4k_prefill_split_graph_replay(torch_dev):
    # a split launch (48 rows of a 17408x5120 gate: 32-row tiles, 4 pieces)
    # replays bit for bit, with eager split launches of another row count
    # between the replays
    import torch
    n, k, m = 17408, 5120, 48
    g = torch.Generator(device=torch_dev).manual_seed(5)
    lin = dq.Linear.quantize(dq.Q4_K, torch.randn(n, k, device=torch_dev, generator=g) * 0.02)
    x = torch.randn(m, k, device=torch_dev, generator=g).to(torch.float16)
    x2 = torch.randn(20, k, device=torch_dev, generator=g).to(torch.float16)
    y = torch.empty(m, n, device=torch_dev, dtype=torch.float16)
    y2 = torch.empty(20, n, device=torch_dev, dtype=torch.float16)
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
    # sampled rows against the dequantized weight's f16 product
    w16 = torch.empty(n, k, device=torch_dev, dtype=torch.float16)
    lin.dequantize(w16)
    ref = (x[:8].float() @ w16.float().t()).cpu().numpy()
    assert O.rel_l2(want[:8].float().cpu().numpy(), ref) <= 1e-3


@pytest.mark.parametrize("fmt", FMTS, ids=IDS)
def test_kq_prefill_bf16_rows_beyond_f16_range(fmt, torch_dev):
    # bf16 rows far above and below f16's range are scaled by a power of
    # two for the f16 kernel and scaled back in the epilogue: every row
    # matches the hybrid product to f32 accumulation, none overflows or
    # flushes to zero
    import torch
    n, k, m = 256, 1024, 130
    lin, deq = _case(n, k, seed=9, fmt=fmt)
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    mult = np.ones(m, np.float32)
    mult[1::7] = 1e5
    mult[2::7] = 2.0 ** 100
    mult[3::7] = 3e-30
    x = O.round_bf16(x * mult[:, None])
    y = torch.full((m, n), float("nan"), device=torch_dev, dtype=torch.float32)
    lin.forward(to_torch(x, dq.BF16, torch_dev), y, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = O.matmul_f64(x, O.round_f16(deq))
    assert np.all(np.isfinite(got))
    for r in range(m):
        assert O.rel_l2(got[r], want[r]) <= 2e-5, (r, mult[r])


@pytest.mark.parametrize("fmt", FMTS, ids=IDS)
def test_kq_prefill_noalloc_falls_back_to_hi_lo(fmt, torch_dev):
    # 1024 rows at K = 17408: the f16 copy of x (35.7 MB) does not fit the
    # allocation-free entry point's array, which runs the hi + lo kernel on
    # x as it is; both agree with the exact product
    import torch
    n, k, m = 256, 17408, 1024
    lin, deq = _case(n, k, seed=4, fmt=fmt)
    x = O.round_bf16(np.random.default_rng(4).normal(0, 1, (m, k)).astype(np.float32))
    xt = to_torch(x, dq.BF16, torch_dev)
    y1 = torch.empty(m, n, device=torch_dev, dtype=torch.float32)
    y2 = torch.empty(m, n, device=torch_dev, dtype=torch.float32)
    lin.forward(xt, y1, path=dq.PATH_GEMM)
    lin.forward_noalloc(xt, y2, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    rows = np.arange(0, m, 37)
    exact = O.matmul_f64(x[rows], deq)
    assert O.rel_l2(y2.cpu().numpy()[rows], exact) <= 2e-5  # hi + lo
    assert O.rel_l2(y1.cpu().numpy()[rows], O.matmul_f64(x[rows], O.round_f16(deq))) <= 2e-5  # f16 copy
    assert O.rel_l2(y1.cpu().numpy()[rows], exact) <= 1e-3
