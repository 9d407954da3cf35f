"""Host side of remote sampling (dial-27b_amd/host/sampling.cpp), CPU only.

The generator restates rand 0.9's StdRng (ChaCha12) and WeightedIndex; rand
is a third-party crate absent from the reference tree, so the draw itself is
parity unpinned.  What is pinned: the ChaCha block function against RFC 7539
section 2.3.2 (20 rounds; the 12-round generator differs only in the round
count), the weighted draw's distribution and its refusal of empty, negative
and all-zero weights, and the reference's mode table
(qwen3_vl/qwen3_vl.rs:292-311)."""
import numpy as np
import pytest

import dialq.host as H


def test_chacha_block_rfc7539_vector():
    key = [int.from_bytes(bytes(range(4 * i, 4 * i + 4)), "little") for i in range(8)]
    nonce = [0x09000000, 0x4A000000, 0x00000000]
    got = H.chacha_block(key, 1, nonce, 20)
    want = [0xE4E7F110, 0x15593BD1, 0x1FDD0F50, 0xC47120A3, 0xC7F4D1C7, 0x0368C033, 0x9AAA2204, 0x4E6CD4C3,
            0x466482D2, 0x09AA9F07, 0x05D7C214, 0xA2028BD9, 0xD19C12B5, 0xB94E16DE, 0xE883D0CB, 0x4E3C50A2]
    assert list(got) == want


def test_generator_stream_is_deterministic_and_seed_dependent():
    a = H.rng_u32_stream(7, 40)
    assert a == H.rng_u32_stream(7, 40)
    assert a != H.rng_u32_stream(8, 40)
    assert len(set(a)) == 40  # 16-word blocks: the counter advances between them
    assert a[16:32] != a[:16]


def test_weighted_draw_distribution_and_zero_weights():
    w = [0.0, 0.5, 0.0, 0.25, 0.25, 0.0]
    counts = np.zeros(len(w))
    n = 4000
    for seed in range(n):
        counts[H.sample_weighted(w, seed)] += 1
    assert counts[[0, 2, 5]].sum() == 0
    freq = counts / n
    assert abs(freq[1] - 0.5) < 0.03 and abs(freq[3] - 0.25) < 0.03 and abs(freq[4] - 0.25) < 0.03
    assert H.sample_weighted([0.0, 0.0, 3.0], 1) == 2


@pytest.mark.parametrize("w,msg", [([], "No weights"), ([0.5, -0.1], "invalid"), ([0.0, 0.0], "zero")])
def test_weighted_draw_errors(w, msg):
    with pytest.raises(H.DialError, match=msg):
        H.sample_weighted(w, 0)


def test_mode_table():
    R = H.SamplingRequest
    assert H.sampling_mode(R(temperature=0.0, top_k=5, top_p=0.5)) == 0  # ArgMax whenever t <= 0
    assert H.sampling_mode(R(temperature=0.7)) == 1
    assert H.sampling_mode(R(temperature=0.7, top_k=5)) == 2
    assert H.sampling_mode(R(temperature=0.7, top_p=0.9)) == 3
    assert H.sampling_mode(R(temperature=0.7, top_k=5, top_p=0.9)) == 4
