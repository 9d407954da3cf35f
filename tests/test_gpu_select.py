"""GPU parity of the device token selection (dialq_logits_select) against the
oracle's restatement of FastLogitsProcessor::sample's selection steps
(qwen3_vl/qwen3_vl.rs:130-174,225-240,325-345): indices bit-exact (both
tie rules, bf16 logits full of ties, +-0 and NaN), logits exact, softmax
statistics within 1e-5 relative of the float64 oracle (the sums run in a
different order)."""
import numpy as np
import pytest

import dialq as dq
import oracle as O

pytestmark = pytest.mark.gpu

RULES = {dq.SELECT_FIRST_MAX: O.select_first_max, dq.SELECT_TOTAL_LAST_MAX: O.select_total_last}


def _dev(x, dtype, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(device)
    return t.to({dq.F32: torch.float32, dq.F16: torch.float16, dq.BF16: torch.bfloat16}[dtype])


def _exact(x, dtype):
    return O.round_bf16(x) if dtype == dq.BF16 else (O.round_f16(x) if dtype == dq.F16 else np.float32(x))


def _run(x, dtype, k, rule, dev, **kw):
    import torch
    idx, val, st = dq.logits_select(_dev(x, dtype, dev), k, rule=rule, **kw)
    torch.cuda.synchronize()
    return idx.cpu().numpy().astype(np.uint32), val.cpu().numpy(), st.cpu().numpy()


@pytest.mark.parametrize("vocab", [4, 1000, 3841, 151936, 248320])
@pytest.mark.parametrize("dtype", [dq.BF16, dq.F16, dq.F32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("rule", [dq.SELECT_FIRST_MAX, dq.SELECT_TOTAL_LAST_MAX], ids=["first", "total_last"])
def test_select_matches_oracle(vocab, dtype, rule, torch_dev):
    rng = np.random.default_rng(vocab + 7 * dtype + rule)
    x = _exact(rng.normal(0, 3, vocab).astype(np.float32), dtype)
    for k in sorted({1, min(7, vocab), min(50, vocab), min(256, vocab)}):
        idx, val, _ = _run(x, dtype, k, rule, torch_dev)
        want_i, want_v = RULES[rule](x, k)
        assert np.array_equal(idx, want_i), (vocab, k)
        assert np.array_equal(val, want_v)


@pytest.mark.parametrize("rule", [dq.SELECT_FIRST_MAX, dq.SELECT_TOTAL_LAST_MAX], ids=["first", "total_last"])
def test_select_ties_zero_and_nan(rule, torch_dev):
    """Few distinct values over a 248320 vocabulary: every rank is a tie, so
    the index order decides; signed zeros and NaNs planted."""
    rng = np.random.default_rng(11)
    x = rng.integers(-4, 3, 248320).astype(np.float32)
    x[rng.integers(0, x.size, 500)] = -0.0
    for planted in (False, True):
        if planted:
            x[[5, 77777, 200000]] = np.nan
            x[[9, 123456]] = np.inf
        for k in (1, 3, 256):
            idx, val, _ = _run(x, dq.F32, k, rule, torch_dev)
            want_i, want_v = RULES[rule](x, k)
            assert np.array_equal(idx, want_i), (planted, k)
            assert np.array_equal(np.isnan(val), np.isnan(want_v))
            assert np.array_equal(val[~np.isnan(val)], want_v[~np.isnan(want_v)])


def test_select_repeat_penalty_and_stats(torch_dev):
    rng = np.random.default_rng(5)
    vocab = 248320
    x = _exact(rng.normal(0, 2, vocab).astype(np.float32), dq.BF16)
    top = O.select_total_last(x, 40)[0]
    ctx = list(top[::2]) + list(top[:5]) + [vocab + 3, 0, 17, 17]  # duplicates, an id past the vocabulary
    for penalty in (1.3, 0.8):
        pen = O.repeat_penalty(x, penalty, ctx)
        for t in (0.7, 1.0):
            idx, val, st = _run(x, dq.BF16, 64, dq.SELECT_TOTAL_LAST_MAX, torch_dev, repeat_ids=ctx,
                                repeat_penalty=penalty, temperature=t)
            want_i, want_v = O.select_total_last(pen, 64)
            assert np.array_equal(idx, want_i) and np.array_equal(val, want_v)
            m, s = O.softmax_stats(pen, t)
            assert abs(st[0] - m) <= 1e-6 * abs(m) and abs(st[1] - s) <= 1e-5 * s, (st, m, s)
    _, _, st = _run(x, dq.BF16, 1, dq.SELECT_FIRST_MAX, torch_dev)
    assert st[0] == -np.inf and st[1] == 0.0


def test_select_reference_vectors_through_the_abi(torch_dev):
    idx, _, _ = _run(np.array([-1.0, 0.5, 3.0, 2.0], np.float32), dq.F32, 1, dq.SELECT_FIRST_MAX, torch_dev)
    assert idx[0] == 2
    idx, _, _ = _run(np.array([5.0, 4.0], np.float32), dq.F32, 1, dq.SELECT_TOTAL_LAST_MAX, torch_dev,
                     repeat_ids=[0], repeat_penalty=2.0)
    assert idx[0] == 1
    # host buffers: synchronous staging through the same kernels
    idx, val, _ = dq.logits_select(np.array([5.0, 4.0], np.float32), 1, rule=dq.SELECT_TOTAL_LAST_MAX,
                                   repeat_ids=[0], repeat_penalty=2.0)
    assert idx[0] == 1 and val[0] == 4.0


def test_select_with_caller_workspace_in_graph(torch_dev):
    """A caller-owned workspace makes the call asynchronous and capturable:
    replays of a captured selection match the eager result."""
    import torch
    vocab = 151936
    ws = torch.empty(dq.logits_select_workspace_bytes(vocab), dtype=torch.uint8, device=torch_dev)
    rng = np.random.default_rng(9)
    x = _dev(rng.normal(0, 3, vocab).astype(np.float32), dq.BF16, torch_dev)
    eager = dq.logits_select(x, 20, rule=dq.SELECT_TOTAL_LAST_MAX, temperature=0.8, workspace=ws)
    torch.cuda.synchronize()
    want = [t.clone() for t in eager]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = dq.logits_select(x, 20, rule=dq.SELECT_TOTAL_LAST_MAX, temperature=0.8, workspace=ws,
                               stream=torch.cuda.current_stream())
    for _ in range(3):
        for t in out:
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, want):
            assert torch.equal(a, b)


def test_select_rejects_bad_arguments(torch_dev):
    x = np.zeros(10, np.float32)
    with pytest.raises(dq.DialqError, match="k must be in"):
        dq.logits_select(x, 0)
    with pytest.raises(dq.DialqError, match="k must be in"):
        dq.logits_select(np.zeros(1000, np.float32), 257)
    with pytest.raises(dq.DialqError, match="at least k"):
        dq.logits_select(x, 11)
    with pytest.raises(dq.DialqError, match="unknown selection rule"):
        dq.logits_select(x, 1, rule=5)


# Vocabularies past ~508k cap the slice count (slices x k must fit the
# merge's 16384 staged keys, at most 1024 slices), so each slice runs several
# chunks: keys carried between chunks, the running softmax merge and, at
# 1033220 with k = 16, an empty last slice (1024 slices of 1010 tokens).
@pytest.mark.parametrize("vocab,k", [(600000, 32), (600000, 64), (600000, 256), (1050000, 1), (1050000, 16),
                                     (1050000, 128), (1033220, 16)])
@pytest.mark.parametrize("rule", [dq.SELECT_FIRST_MAX, dq.SELECT_TOTAL_LAST_MAX], ids=["first", "total_last"])
def test_select_multi_chunk_slices(vocab, k, rule, torch_dev):
    rng = np.random.default_rng(vocab + k + rule)
    # bf16 values: plenty of ties across chunk boundaries
    x = _exact(rng.normal(0, 3, vocab).astype(np.float32), dq.BF16)
    idx, val, st = _run(x, dq.BF16, k, rule, torch_dev, temperature=0.9)
    want_i, want_v = RULES[rule](x, k)
    assert np.array_equal(idx, want_i), (vocab, k)
    assert np.array_equal(val, want_v)
    m, s = O.softmax_stats(x, 0.9)
    assert abs(st[0] - m) <= 1e-6 * abs(m) and abs(st[1] - s) <= 1e-5 * s, (st, m, s)


@pytest.mark.parametrize("vocab,k", [(248320, 50), (248320, 1), (1050000, 16)])
def test_select_masked_range_keeps_statistics_finite(vocab, k, torch_dev):
    # a -inf range longer than a slice (whole slices and whole chunks of
    # -inf): those tokens add exp(-inf) = 0 to S, as softmax_in_place's
    # exp(v - max) does (qwen3_vl.rs:325-345)
    rng = np.random.default_rng(vocab + k)
    x = _exact(rng.normal(0, 3, vocab).astype(np.float32), dq.F32)
    x[10000:30000] = -np.inf
    x[-5000:] = -np.inf
    for rule in RULES:
        idx, val, st = _run(x, dq.F32, k, rule, torch_dev, temperature=0.7)
        want_i, want_v = RULES[rule](x, k)
        assert np.array_equal(idx, want_i) and np.array_equal(val, want_v)
        m, s = O.softmax_stats(x, 0.7)
        assert np.isfinite(st).all(), st
        assert abs(st[0] - m) <= 1e-6 * abs(m) and abs(st[1] - s) <= 1e-5 * s, (st, m, s)
