"""Prefill launches whose last round of tiles is at most half full split
that round's tiles along K (the tail split): workgroups [0, W) run whole
tiles, the rest run k pieces whose partials the last arriving piece adds in
piece order.  The shapes give 544 tiles on a 256-CU MI355X's 512 slots (two
workgroups per CU), 512 whole and 32 split:

  W8A16 / Q8_0 / Q4_K, M = 2048 (128-row tiles): N = 8704 is 34 column
  tiles x 16 row blocks, split in 4 pieces (2 for Q4_K's 8 chunks);
  FP8-128 native, M = 1024 (64-row tiles): the same 544, and MXFP4 native,
  M = 1024 (128-row tiles): N = 17408, 68 x 8, split in 2 pieces.

Every output element is compared with the fp64 oracle product (split and
whole tiles alike), and three calls give the same bits (the piece order of
the fix-up does not depend on timing)."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import make_weight, reference_product, to_torch

pytestmark = pytest.mark.gpu

CASES = {
    "w8a16": (dq.W8A16, 8704, 1024, 2048, dq.PATH_GEMM),
    "q8_0": (dq.Q8_0, 8704, 1024, 2048, dq.PATH_GEMM),
    "q4_k": (dq.Q4_K, 8704, 2048, 2048, dq.PATH_GEMM),
    "fp8_block_native": (dq.FP8_BLOCK, 8704, 2048, 1024, dq.PATH_GEMM_NATIVE),
    "mxfp4_native": (dq.MXFP4, 17408, 2048, 1024, dq.PATH_GEMM_NATIVE),
}


def _native_x(fmt, x):
    """The activations as the native kernels multiply them (oracle quantizers)."""
    if fmt == dq.FP8_BLOCK:
        q, sx = O.act_fp8_quantize(x)
        return O.e4m3_to_f32(q.ravel()).reshape(x.shape) * sx[:, None]
    p, sx = O.act_mxfp4_quantize(x)
    return O.mxfp4_dequant(p, sx)


@pytest.mark.parametrize("case", list(CASES))
def test_tail_split_matches_oracle_and_repeats(case, torch_dev):
    import torch
    fmt, n, k, m, path = CASES[case]
    raw, scales, kw, deq = make_weight(fmt, n, k, seed=17)
    lin = dq.Linear.create(fmt, n, k, raw, scales, **kw)
    x = O.round_bf16(np.random.default_rng(5).normal(0, 1, (m, k)).astype(np.float32))
    xt = to_torch(x, dq.BF16, torch_dev)
    outs = []
    for _ in range(3):
        y = torch.full((m, n), float("nan"), device=torch_dev, dtype=torch.bfloat16)
        lin.forward(xt, y, path=path)
        torch.cuda.synchronize()
        outs.append(y.view(torch.int16).cpu().numpy())
    assert all(np.array_equal(o, outs[0]) for o in outs[1:]), case
    got = torch.from_numpy(outs[0]).view(torch.bfloat16).float().numpy()
    native = path == dq.PATH_GEMM_NATIVE
    ref = reference_product(_native_x(fmt, x) if native else x, deq, dq.BF16)
    tol = 2e-3 if native else 1e-3
    # the last row panel holds the split tiles: check it on its own too
    for sl in (slice(None), slice(m - m // 4, m)):
        rel = O.rel_l2(got[sl], ref[sl])
        assert rel <= tol, (case, sl, rel)
    lin.close()


@pytest.mark.parametrize("case", ["w8a16", "q4_k", "mxfp4_native"])
def test_tail_split_with_the_swiglu_epilogue(case, torch_dev):
    # a fused gate_up of 2 x 8704 rows: 68 column tiles of gate / up strip
    # pairs, 1088 tiles of 128 rows at M = 2048 (W8A16: 64 split in 4
    # pieces; Q4_K, 8 chunks of 256: in 2) or 544 at M = 1024 (MXFP4: 32
    # split in 2); the last piece of a split tile exchanges the up values
    # and writes silu(g) * u
    import torch
    fmt, m, path = {"w8a16": (dq.W8A16, 2048, dq.PATH_GEMM), "q4_k": (dq.Q4_K, 2048, dq.PATH_GEMM),
                    "mxfp4_native": (dq.MXFP4, 1024, dq.PATH_GEMM_NATIVE)}[case]
    n, k = 2 * 8704, 1024 if fmt == dq.W8A16 else 2048
    raw, scales, kw, deq = make_weight(fmt, n, k, seed=29)
    lin = dq.Linear.create(fmt, n, k, raw, scales, **kw)
    x = O.round_bf16(np.random.default_rng(31).normal(0, 1, (m, k)).astype(np.float32))
    y = torch.full((m, n // 2), float("nan"), device=torch_dev, dtype=torch.float32)
    lin.forward_swiglu(to_torch(x, dq.BF16, torch_dev), y, path=path)
    torch.cuda.synchronize()
    xr = _native_x(fmt, x) if path == dq.PATH_GEMM_NATIVE else x
    ref = O.swiglu(O.matmul_f64(xr, deq))
    rel = O.rel_l2(y.cpu().numpy(), ref)
    # Q4_K prefill multiplies the f16-rounded dequantized weight (the GGUF
    # prefill's own weight), within 1e-3 of the exact product
    assert rel <= (2e-3 if path == dq.PATH_GEMM_NATIVE else 1e-3 if fmt == dq.Q4_K else 1e-4), (case, rel)
    lin.close()
