"""Pin the oracle's format codecs with closed forms, independent library
routines and invariants that a dropped term, a wrong index, a wrong rounding
mode or a transposed operand would break."""
import numpy as np
import pytest
import torch


def test_w8a16_quantizer_invariants(O):
    rng = np.random.default_rng(0)
    w = np.zeros((6, 64), np.float32)
    w[1, :4] = [127.0, 2.5, -2.5, 0.5]          # scale exactly 1.0 -> ties visible
    w[2] = rng.normal(0, 0.02, 64)
    w[3] = rng.normal(0, 1.0, 64) * 1e-30       # tiny but nonzero
    w[4, 7] = -3.0                               # single spike
    w[5] = np.linspace(-1, 1, 64)
    q, s, sb = O.w8a16_quantize(w)
    # zero row -> scale 1 and zero codes (worker_w8a16.rs:336)
    assert s[0] == 1.0 and not q[0].any()
    # half-away-from-zero rounding (Rust f32::round), not numpy's half-to-even
    assert s[1] == 1.0
    assert list(q[1, :4]) == [127, 3, -3, 1]
    for r in range(2, 6):
        amax = np.max(np.abs(w[r]))
        assert s[r] == np.float32(amax / np.float32(127.0))
        assert np.abs(q[r]).max() == 127
        assert q[r, np.argmax(np.abs(w[r]))] == np.sign(w[r, np.argmax(np.abs(w[r]))]) * 127
        err = np.abs(w[r].astype(np.float64) - q[r].astype(np.float64) * s[r])
        assert np.all(err <= s[r] * 0.5 * (1 + 1e-5) + 1e-45)
    # bf16 storage of the same scale, rounded by torch (RNE)
    ref = torch.from_numpy(s).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(sb, ref)
    # dequant: q * scale, both widths
    d = O.w8a16_dequant(q, s)
    assert np.array_equal(d, q.astype(np.float32) * s[:, None])
    d2 = O.w8a16_dequant(q, sb)
    assert np.array_equal(d2, q.astype(np.float32) * O.bf16_bits_to_f32(sb)[:, None])


Q8_0_DT = np.dtype([("d", "<f2"), ("qs", "i1", 32)])


def test_q8_0_block_layout_and_rounding(O):
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, (3, 128)).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :4] = [127.0, 0.5, -0.5, 1.5]           # d = 1 exactly: ties away from zero
    blocks = O.q8_0_quantize(w)
    assert blocks.shape == (3, 4 * 34)
    b = blocks.reshape(3, 4, 34).copy().view(Q8_0_DT).reshape(3, 4)
    assert b["d"][0, 0] == 0 and not b["qs"][0, 0].any()
    assert list(b["qs"][1, 0, :4]) == [127, 1, -1, 2]
    for r in range(3):
        for k in range(4):
            x = w[r, 32 * k:32 * k + 32]
            amax = np.abs(x).max()
            d32 = np.float32(amax / np.float32(127.0))
            assert b["d"][r, k] == np.float16(d32)          # numpy RNE to f16
            if amax > 0:
                assert np.abs(b["qs"][r, k]).max() == 127
                assert np.all(np.abs(x - b["qs"][r, k] * d32) <= d32 * 0.5 * (1 + 1e-5))
    deq = O.q8_0_dequant(blocks, 3, 128)
    want = b["qs"].astype(np.float32) * b["d"].astype(np.float32)[..., None]
    assert np.array_equal(deq, want.reshape(3, 128))


def _pack_q4k_scales(sc, m):
    """GGUF Q4_K 6-bit scale packing, written from the format definition
    (llama.cpp block_q4_K): bytes 0-3 hold sc[0..3] with sc[4..7]>>4 in bits
    6-7; bytes 4-7 hold m[0..3] with m[4..7]>>4 in bits 6-7; bytes 8-11 hold
    the low nibbles of sc[4..7] and m[4..7]."""
    out = np.zeros(12, np.uint8)
    for j in range(4):
        out[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return out


def test_q4_k_dequant_hand_built_block(O):
    rng = np.random.default_rng(2)
    sc = rng.integers(0, 64, 8)
    m = rng.integers(0, 64, 8)
    sc[5], m[6] = 63, 63                      # exercise all six bits
    q = rng.integers(0, 16, 256)
    d, dmin = np.float16(0.0123), np.float16(0.00456)
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d]).view(np.uint8)
    blk[2:4] = np.array([dmin]).view(np.uint8)
    blk[4:16] = _pack_q4k_scales(sc, m)
    # value p of the super-block: 64-group i = p // 64; first 32 values are the
    # low nibbles of qs[32i .. 32i+32), the next 32 the high nibbles
    qs = np.zeros(128, np.uint8)
    for p in range(256):
        i, within = divmod(p, 64)
        byte = 32 * i + (within % 32)
        qs[byte] |= q[p] << (4 if within >= 32 else 0)
    blk[16:] = qs
    for j in range(8):
        s_, m_ = np.zeros(1, np.uint8), np.zeros(1, np.uint8)
        import ctypes
        a, b = ctypes.c_uint8(), ctypes.c_uint8()
        O.lib().or_q4_k_scale_min(j, blk[4:16].ctypes.data_as(ctypes.c_void_p), ctypes.byref(a), ctypes.byref(b))
        assert (a.value, b.value) == (sc[j], m[j])
    deq = O.q4_k_dequant(blk[None, :], 1, 256)[0]
    df, mf = np.float32(d), np.float32(dmin)
    want = np.empty(256, np.float32)
    for p in range(256):
        j = p // 32
        want[p] = np.float32(df * np.float32(sc[j])) * np.float32(q[p]) - np.float32(mf * np.float32(m[j]))
    assert np.array_equal(deq, want)


def test_q4_k_quantizer_round_trip(O):
    # Parity unpinned for the exact bytes (candle's quantizer is not vendored);
    # check the codec invariants and the round-trip error.
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (8, 512)).astype(np.float32)
    w[0, :256] = 0.0
    w[1, :256] = 0.01                          # constant block
    blocks = O.q4_k_quantize(w)
    assert blocks.shape == (8, 2 * 144)
    deq = O.q4_k_dequant(blocks, 8, 512)
    assert np.all(deq[0, :256] == 0.0)
    rel = np.linalg.norm(deq[2:] - w[2:]) / np.linalg.norm(w[2:])
    assert rel < 0.12, rel
    # each stored d / dmin is the f16 of max_scale/63, max_min/63 => some 6-bit
    # scale equals 63 in every nonzero block
    for r in range(2, 8):
        for b in range(2):
            blk = blocks[r, 144 * b:144 * (b + 1)]
            import ctypes
            scs = []
            for j in range(8):
                a, c = ctypes.c_uint8(), ctypes.c_uint8()
                O.lib().or_q4_k_scale_min(j, blk[4:16].ctypes.data_as(ctypes.c_void_p), ctypes.byref(a), ctypes.byref(c))
                scs.append(a.value)
            assert max(scs) == 63


def test_q4_k_quantizer_closed_form_cases(O):
    # Exact affine grids, all-positive sub-blocks, half-way ties and
    # one-non-zero-sub-block super-blocks, whose bytes follow from arithmetic
    # (tests/q4k_cases.py), against the oracle's restatement of candle's
    # BlockQ4K::from_float (worker_gguf.rs:641,657)
    import q4k_cases
    w, want, names = q4k_cases.cases()
    got = O.q4_k_quantize(w)
    for r, name in enumerate(names):
        assert np.array_equal(got[r], want[r]), (name, np.nonzero(got[r] != want[r])[0][:8])
    # the dequantized grids come back exactly (d * sc * l - dmin * m)
    deq = O.q4_k_dequant(got, len(names), 256)
    for r, name in enumerate(names):
        if name == "constant_subblocks":  # max == min sub-blocks keep scale 0: they come back as zeros
            want_deq = np.where(np.repeat([c == 0 for c in (63, 0, 11, 0, 30, 0, 63, 5)], 32), 0.0, w[r])
            assert np.array_equal(deq[r], want_deq), name
        elif name != "half_way_ties":
            assert np.array_equal(deq[r], w[r]), name


def test_q4_k_closed_form_cases_catch_plausible_mistakes(O):
    # the cases are only worth something if a wrong quantizer fails them:
    # restate the quantizer with one mistake at a time and check that some
    # case's bytes change (the mistakes live here, on the CPU, in the test)
    import q4k_cases
    w, want, names = q4k_cases.cases()

    def quantize(x, clamp_min=True, rne=False, swap_hi=False, nibble_swap=False):
        def nearest(v):
            return int(np.rint(v)) if rne else int(np.floor(abs(v) + 0.5)) * (1 if v >= 0 else -1)

        def qkx1(xs):
            xs = np.asarray(xs, np.float32)
            mn, mx = np.float32(xs.min()), np.float32(xs.max())
            if mx == mn:
                return np.float32(0), np.float32(0)
            if clamp_min and mn > 0:
                mn = np.float32(0)
            isc = np.float32(15) / np.float32(mx - mn)
            lv = np.zeros(32, np.int64)
            scale = np.float32(1) / isc
            for _ in range(5):
                new = np.array([min(15, max(0, nearest(np.float32(isc * np.float32(v - mn))))) for v in xs])
                changed = not np.array_equal(new, lv)
                lv = new
                sumlx = np.float32(0)
                for v, li in zip(xs, lv):
                    sumlx = np.float32(sumlx + np.float32(np.float32(v - mn) * np.float32(li)))
                scale = np.float32(sumlx / np.float32(int((lv * lv).sum())))
                tot = np.float32(0)
                for v, li in zip(xs, lv):
                    tot = np.float32(tot + np.float32(v - np.float32(scale * np.float32(li))))
                mn = np.float32(tot / np.float32(32))
                if clamp_min and mn > 0:
                    mn = np.float32(0)
                isc = np.float32(1) / scale
                if not changed:
                    break
            return scale, np.float32(-mn)

        out = np.zeros(144, np.uint8)
        fits = [qkx1(x[32 * j:32 * j + 32]) for j in range(8)]
        ms, mm = np.float32(0), np.float32(0)
        for f in fits:  # fold from +0 with a strict compare
            ms = f[0] if f[0] > ms else ms
            mm = f[1] if f[1] > mm else mm
        isc = np.float32(63) / ms if ms > 0 else np.float32(0)
        imn = np.float32(63) / mm if mm > 0 else np.float32(0)
        # `as u8` of a negative value wraps; a planted mistake can produce one
        sc = [min(63, nearest(np.float32(isc * f[0]))) & 63 for f in fits]
        mi = [min(63, nearest(np.float32(imn * f[1]))) & 63 for f in fits]
        packed = q4k_cases.pack_scales(sc, mi)
        if swap_hi:  # high bits of sc[4..7] and m[4..7] exchanged
            packed = q4k_cases.pack_scales(sc[:4] + mi[4:], mi[:4] + sc[4:])
        d = np.float16(ms / np.float32(63))
        dmin = np.float16(mm / np.float32(63))
        codes = []
        for j in range(8):
            dd = np.float32(np.float32(d) * np.float32(sc[j]))
            dm = np.float32(np.float32(dmin) * np.float32(mi[j]))
            for v in x[32 * j:32 * j + 32]:
                codes.append(0 if dd == 0 else min(15, max(0, nearest(np.float32(np.float32(v + dm) / dd)))))
        if nibble_swap:
            codes = [codes[(p // 64) * 64 + (p % 64 + 32) % 64] for p in range(256)]
        out[0:2] = np.array([d]).view(np.uint8)
        out[2:4] = np.array([dmin]).view(np.uint8)
        out[4:16] = packed
        out[16:] = q4k_cases.pack_codes(codes)
        return out

    # the faithful restatement reproduces every case ...
    for r in range(len(names)):
        assert np.array_equal(quantize(w[r]), want[r]), names[r]
    # ... and each planted mistake breaks at least one
    for mistake in ({"clamp_min": False}, {"rne": True}, {"swap_hi": True}, {"nibble_swap": True}):
        broken = [names[r] for r in range(len(names)) if not np.array_equal(quantize(w[r], **mistake), want[r])]
        assert broken, mistake


def _q6k_encode(codes, scales, d):
    """One Q6_K block from 256 6-bit codes, 16 i8 scales and an f16 d, placed
    element by element from the block layout description: value e of half
    h = e // 128 (w = e % 128, quarter qd = w // 32, l = w % 32) keeps its
    low 4 bits in nibble qd // 2 of ql[64h + 32(qd % 2) + l] and its top 2
    bits at bit 2qd of qh[32h + l]; sub-block e // 16 has scales[e // 16]."""
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        h, w = divmod(e, 128)
        qd, l = divmod(w, 32)
        blk[64 * h + 32 * (qd % 2) + l] |= (int(codes[e]) & 15) << (4 * (qd // 2))
        blk[128 + 32 * h + l] |= (int(codes[e]) >> 4) << (2 * qd)
    blk[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


def test_q6_k_dequant_element_layout(O):
    rng = np.random.default_rng(6)
    blocks, expect = [], []
    for trial in range(6):
        codes = rng.integers(0, 64, 256)
        scales = rng.integers(-128, 128, 16)
        d = np.float16(rng.uniform(1e-4, 1e-2) * (-1 if trial == 3 else 1))
        blocks.append(_q6k_encode(codes, scales, d))
        # exact in f32: f16 d (11 bits) * i8 scale (8) * (q - 32) (6)
        expect.append((np.float64(d) * scales[np.arange(256) // 16] * (codes - 32.0)).astype(np.float32))
    # 3 rows x 2 super-blocks
    got = O.q6_k_dequant(np.concatenate(blocks).reshape(3, 420), 3, 512)
    assert np.array_equal(got.ravel().view(np.uint32), np.concatenate(expect).view(np.uint32))
    # invariants: d = 0 -> zeros; every code 32 -> zeros; unit scales and
    # codes e % 64 -> (e % 64) - 32 in order
    z = O.q6_k_dequant(_q6k_encode(rng.integers(0, 64, 256), rng.integers(-128, 128, 16), 0.0)[None], 1, 256)
    assert not z.any()
    z = O.q6_k_dequant(_q6k_encode(np.full(256, 32), rng.integers(-128, 128, 16), 0.5)[None], 1, 256)
    assert not z.any()
    ramp = O.q6_k_dequant(_q6k_encode(np.arange(256) % 64, np.ones(16), 1.0)[None], 1, 256)
    assert np.array_equal(ramp.ravel(), (np.arange(256) % 64 - 32).astype(np.float32))


def test_fp8_block_quantizer_matches_torch_cast(O):
    rng = np.random.default_rng(4)
    n, k = 200, 300                             # ragged: partial 128-blocks
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    w[:128, :128] = 0.0                         # zero block -> scale 1
    q, s = O.fp8_block_quantize(w)
    assert s.shape == (2, 3) and s[0, 0] == 1.0
    for bn in range(2):
        for bk in range(3):
            blk = w[bn * 128:(bn + 1) * 128, bk * 128:(bk + 1) * 128]
            amax = np.abs(blk).max()
            if amax == 0:
                continue
            sc = np.float32(amax / np.float32(448.0))
            assert s[bn, bk] == sc
            inv = np.float32(1.0) / sc
            ref = torch.from_numpy((blk * inv).astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            got = q[bn * 128:(bn + 1) * 128, bk * 128:(bk + 1) * 128]
            assert np.array_equal(O.e4m3_to_f32(got), O.e4m3_to_f32(ref))
            assert np.abs(O.e4m3_to_f32(got)).max() == 448.0
    deq = O.fp8_block_dequant(q, s)
    want = O.e4m3_to_f32(q) * np.repeat(np.repeat(s, 128, 0), 128, 1)[:n, :k]
    assert np.array_equal(deq, want)


def test_mxfp4_quantizer_closed_form(O):
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, (4, 96)).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :32] = np.linspace(-6, 6, 32)          # amax 6 -> shared exp 0
    packed, scales = O.mxfp4_quantize(w)
    assert packed.shape == (4, 48) and scales.shape == (4, 3)
    assert scales[0, 0] == 0                     # zero block: shared = -127
    assert scales[1, 0] == 127
    for r in range(4):
        for b in range(3):
            x = w[r, 32 * b:32 * b + 32]
            amax = np.abs(x).max()
            if amax == 0:
                continue
            shared = np.frexp(np.float32(amax))[1] - 1 - 2
            assert scales[r, b] == shared + 127
            codes = packed[r, 16 * b:16 * b + 16]
            lo, hi = codes & 15, codes >> 4
            got = np.empty(32, np.uint8)
            got[0::2], got[1::2] = lo, hi
            want = O.f32_to_e2m1(np.ldexp(x, -shared).astype(np.float32))
            assert np.array_equal(O.e2m1_to_f32(got), O.e2m1_to_f32(want))
    deq = O.mxfp4_dequant(packed, scales)
    codes = np.empty((4, 96), np.uint8)
    codes[:, 0::2], codes[:, 1::2] = packed & 15, packed >> 4
    want = O.e2m1_to_f32(codes) * np.repeat(2.0 ** (scales.astype(np.float64) - 127), 32, 1)
    assert np.array_equal(deq, want.astype(np.float32))


def test_act_fp8_per_token(O):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (5, 64)).astype(np.float32)
    x[2] = 0
    q, s = O.act_fp8_quantize(x)
    assert s[2] == 1.0 and not q[2].any()
    for r in (0, 1, 3, 4):
        sc = np.float32(np.abs(x[r]).max() / np.float32(448.0))
        assert s[r] == sc
        ref = torch.from_numpy(x[r] * (np.float32(1.0) / sc)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(O.e4m3_to_f32(q[r]), O.e4m3_to_f32(ref))


def test_matmul_oracle_matches_numpy(O):
    rng = np.random.default_rng(7)
    x = rng.normal(size=(3, 40)).astype(np.float32)
    w = rng.normal(size=(7, 40)).astype(np.float32)
    y = O.matmul_f64(x, w)
    assert np.allclose(y, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-12, atol=1e-12)
    # a transposed operand would fail here
    assert y.shape == (3, 7)


def test_rms_norm_oracle(O):
    """A constant row c gives w * c / sqrt(c^2 + eps) (a sum in place of the
    mean, or a missing square root, breaks it); random rows match torch's
    own rms_norm in float64, and the weight multiplies per column."""
    import torch
    w = np.linspace(-2.0, 3.0, 16)
    for c, eps in ((3.0, 1e-6), (-0.5, 0.25), (0.0, 1e-6)):
        y = O.rms_norm(np.full((1, 16), c), w, eps)
        assert np.allclose(y, w * c / np.sqrt(c * c + eps), rtol=1e-15, atol=0)
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (5, 64))
    wr = rng.normal(1, 0.3, 64)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (64,), torch.from_numpy(wr), eps=1e-5).numpy()
    assert np.allclose(O.rms_norm(x, wr, 1e-5), want, rtol=1e-13, atol=1e-13)


def test_swiglu_oracle_known_answers(O):
    """silu(g) = g * sigmoid(g): known values, the odd-part identity
    silu(g) - silu(-g) = g (a sign slip in the exponent breaks it), torch's
    own silu, and the gate / up halves (swapping them changes the answer)."""
    g = np.array([0.0, 1.0, -1.0, 20.0, -100.0, 3.5, -0.25])
    u = np.ones_like(g)
    y = O.swiglu(np.concatenate([g, u])[None, :])[0]
    want = np.array([0.0, 0.7310585786300049, -0.2689414213699951, 20.0 / (1.0 + np.exp(-20.0)),
                     -100.0 * np.exp(-100.0) / (1.0 + np.exp(-100.0)), 3.5 / (1.0 + np.exp(-3.5)),
                     -0.25 / (1.0 + np.exp(0.25))])
    assert np.allclose(y, want, rtol=1e-15, atol=0)
    rng = np.random.default_rng(12)
    gg = rng.normal(0, 4, (3, 64))
    ones = np.ones_like(gg)
    pos = O.swiglu(np.concatenate([gg, ones], 1))
    neg = O.swiglu(np.concatenate([-gg, ones], 1))
    assert np.allclose(pos - neg, gg, rtol=0, atol=1e-12)
    ref = torch.nn.functional.silu(torch.from_numpy(gg)).numpy()
    assert np.allclose(pos, ref, rtol=1e-12, atol=1e-15)
    uu = rng.normal(size=gg.shape)
    y = O.swiglu(np.concatenate([gg, uu], 1))
    assert np.allclose(y, ref * uu, rtol=1e-12, atol=1e-15)
    assert not np.allclose(y, O.swiglu(np.concatenate([uu, gg], 1)))
    with pytest.raises(ValueError):
        O.swiglu(np.zeros((1, 3)))


def test_w8a16_linear_oracle(O):
    rng = np.random.default_rng(8)
    w = rng.normal(0, 0.02, (9, 64)).astype(np.float32)
    x = rng.normal(size=(2, 64)).astype(np.float32)
    q, s, sb = O.w8a16_quantize(w)
    y = O.w8a16_linear(x, q, s)
    ref = (x.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-7)


def test_local_q8_integer_dot(O):
    rng = np.random.default_rng(9)
    w = rng.normal(0, 0.02, (33, 96)).astype(np.float32)
    x = rng.normal(size=96).astype(np.float32)
    q, s, _ = O.w8a16_quantize(w)
    y = O.local_q8_forward(x, q, s)
    xs = np.float32(np.abs(x).max() / np.float32(127.0))
    xq = np.clip(np.sign(x * (np.float32(1) / xs)) * np.floor(np.abs(x * (np.float32(1) / xs)) + 0.5), -127, 127)
    acc = q.astype(np.int64) @ xq.astype(np.int64)
    want = (acc.astype(np.float32) * s) * xs
    assert np.array_equal(y, want.astype(np.float32))
