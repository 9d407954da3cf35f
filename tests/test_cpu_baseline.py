"""The CPU baseline that bench.py times (oracle/cpu_baseline.c: the
reference's CPU GEMV restated with threads, and a blocked f32 prefill GEMM)
computes the same products as the scalar oracle: it may reassociate the
k-sums, so the bar is an f32 rounding bound, not bit equality.  Both the
portable build (liboracle.so) and the -march=native build bench.py makes on
its host are checked."""
import numpy as np
import pytest

import oracle as O


def _bf16_bits(x):
    return (np.asarray(O.round_bf16(x), np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("native", [False, True], ids=["portable", "native"])
def test_cpu_baseline_matches_oracle(native):
    rng = np.random.default_rng(1)
    n, k = 200, 1024   # 200 rows: three full 64-row tasks and a ragged one
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    q, _, sb = O.w8a16_quantize(w)
    deq = O.w8a16_dequant(q, sb)
    for m in (1, 3, 8, 13):
        x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
        ref = O.matmul_f64(x, deq)
        if m <= 8:
            got = O.cpu_w8a16_gemv(_bf16_bits(x), q, sb, 4, native=native)
            assert O.rel_l2(got, ref) <= 1e-5, ("gemv", m)
        got = O.cpu_w8a16_gemm(_bf16_bits(x), q, sb, 4, native=native)
        assert O.rel_l2(got, ref) <= 1e-5, ("gemm", m)
    blocks = O.q4_k_quantize(w)
    deq4 = O.q4_k_dequant(blocks, n, k)
    x = O.round_bf16(rng.normal(0, 1, (2, k)).astype(np.float32))
    got = O.cpu_q4_k_gemv(_bf16_bits(x), blocks, n, 4, native=native)
    assert O.rel_l2(got, O.matmul_f64(x, deq4)) <= 1e-5
