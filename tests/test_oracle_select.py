"""Pin the oracle's token-selection restatement (qwen3_vl/qwen3_vl.rs:130-174,
225-240, 282-345) with the reference's own unit-test vectors
(qwen3_vl.rs:3439-3447 greedy_sampling_uses_device_argmax, :3572-3588
remote_sampling_applies_repeat_penalty_before_greedy_selection), brute-force
loops written from the Rust semantics (Iterator::max_by keeps the last
maximum; f32::total_cmp orders -0 < +0 and NaN by sign above / below every
number), and scipy's logsumexp for the softmax statistics."""
import struct

import numpy as np
import pytest
from scipy.special import logsumexp


def _total_cmp(a, b):
    """Rust f32::total_cmp: compare the sign-flipped bit patterns as i32."""
    def key(x):
        i = struct.unpack("<i", struct.pack("<f", x))[0]
        return i ^ (((i >> 31) & 0xFFFFFFFF) >> 1)
    ka, kb = key(a), key(b)
    return (ka > kb) - (ka < kb)


def _max_by_total_last(vals):
    best = 0
    for i in range(1, len(vals)):
        if _total_cmp(float(vals[i]), float(vals[best])) >= 0:  # max_by: later equal wins
            best = i
    return best


def test_reference_greedy_vector(O):
    idx, val = O.select_first_max(np.array([-1.0, 0.5, 3.0, 2.0], np.float32))
    assert idx[0] == 2 and val[0] == 3.0


def test_reference_repeat_penalty_vector(O):
    pen = O.repeat_penalty(np.array([5.0, 4.0], np.float32), 2.0, [0])
    assert pen.tolist() == [2.5, 4.0]
    assert O.select_total_last(pen)[0][0] == 1


def test_repeat_penalty_rules(O):
    x = np.array([2.0, -2.0, 0.0, -0.0, 7.0], np.float32)
    got = O.repeat_penalty(x, 4.0, [1, 0, 1, 2, 3, 99, 0])  # duplicates once, 99 past the end ignored
    assert got.tolist() == [0.5, -8.0, 0.0, 0.0, 7.0]
    assert O.repeat_penalty(x, 1.0, [0, 1]).tolist() == x.tolist()


@pytest.mark.parametrize("seed", range(6))
def test_total_last_matches_max_by_brute_force(O, seed):
    rng = np.random.default_rng(seed)
    pool = np.array([0.0, -0.0, 1.5, -1.5, 3.0, np.inf, -np.inf, np.nan, -np.nan, 1e-40, -1e-40], np.float32)
    v = pool[rng.integers(0, len(pool) - (0 if seed % 2 else 4), 40)]
    assert O.select_total_last(v)[0][0] == _max_by_total_last(v)
    # top-k = repeated max_by over the remaining elements
    rest, want = list(range(v.size)), []
    for _ in range(8):
        j = _max_by_total_last(v[rest])
        want.append(rest.pop(j))
    assert O.select_total_last(v, 8)[0].tolist() == want


@pytest.mark.parametrize("seed", range(6))
def test_first_max_matches_strict_greater_brute_force(O, seed):
    rng = np.random.default_rng(100 + seed)
    v = rng.integers(-3, 4, 50).astype(np.float32)  # many ties
    if seed % 2:
        v[rng.integers(0, 50, 5)] = -0.0
    best = 0
    for i in range(1, v.size):
        if v[i] > v[best]:
            best = i
    assert O.select_first_max(v)[0][0] == best
    rest, want = list(range(v.size)), []
    for _ in range(10):
        b = 0
        for i in range(1, len(rest)):
            if v[rest[i]] > v[rest[b]]:
                b = i
        want.append(rest.pop(b))
    assert O.select_first_max(v, 10)[0].tolist() == want
    w = v.copy()
    w[3] = np.nan  # NaN is never larger
    assert O.select_first_max(w)[0][0] == (best if best != 3 else O.select_first_max(np.delete(v, 3))[0][0] + (
        1 if O.select_first_max(np.delete(v, 3))[0][0] >= 3 else 0))


def test_softmax_stats_match_logsumexp(O):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 4, 5000).astype(np.float32)
    for t in (0.7, 1.0, 1e-9):
        m, s = O.softmax_stats(x, t)
        tt = np.float32(max(np.float32(t), np.float32(1e-7)))
        q = (x / tt).astype(np.float64)
        assert m == q.max()
        assert np.isclose(m + np.log(s), logsumexp(q), rtol=1e-12, atol=1e-9)
