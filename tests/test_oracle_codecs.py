"""Pin the oracle's scalar codecs against independent library routines
(numpy float16, torch bfloat16 / float8_e4m3fn) and brute force."""
import numpy as np
import pytest
import torch


def _rand_f32(n, seed=0):
    rng = np.random.default_rng(seed)
    mant = rng.standard_normal(n).astype(np.float32)
    exps = rng.integers(-30, 20, n).astype(np.float32)
    return (mant * np.float32(2.0) ** exps).astype(np.float32)


def test_f16_encode_matches_numpy(O):
    x = np.concatenate([_rand_f32(20000, 1), np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6.0e-8, 2.98e-8,
                                                       np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16_bits(x), ref)


def test_f16_decode_matches_numpy(O):
    bits = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7C00) != 0x7C00]
    assert np.array_equal(O.f16_bits_to_f32(bits), bits.view(np.float16).astype(np.float32))


def test_bf16_encode_matches_torch(O):
    x = np.concatenate([_rand_f32(20000, 2), np.array([0.0, -0.0, 3.0e38, 1e-40], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(x), ref)
    # the vectorised helper used on large arrays agrees with the C routine
    assert np.array_equal(O.round_bf16(x).view(np.uint32) >> 16, ref.astype(np.uint32))


def test_e4m3_decode_matches_torch_for_all_codes(O):
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ocp = O.e4m3_to_f32(codes, ocp=True)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ocp), nan)
    assert np.array_equal(ocp[~nan], ref[~nan])
    # the reference CUDA decode (cuda_quant.rs:35-36) maps the NaN codes to 0
    cuda = O.e4m3_to_f32(codes)
    assert np.all(cuda[nan] == 0.0)
    assert np.array_equal(cuda[~nan], ref[~nan])


def test_e4m3_encode_rne_matches_torch(O):
    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    vals = np.unique(vals[~np.isnan(vals)])
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(3)
    x = np.concatenate([vals, mids, np.nextafter(mids, np.float32(np.inf)),
                        np.nextafter(mids, np.float32(-np.inf)),
                        rng.uniform(-448, 448, 5000).astype(np.float32),
                        rng.uniform(-0.03, 0.03, 5000).astype(np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.f32_to_e4m3(x)
    assert np.array_equal(O.e4m3_to_f32(got), O.e4m3_to_f32(ref))


def test_e4m3_encode_saturates(O):
    assert O.f32_to_e4m3(np.float32(1000.0)) == 0x7E
    assert O.f32_to_e4m3(np.float32(-470.0)) == 0xFE


E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def _e2m1_brute(v):
    """nearest grid point, ties to the even code (code & 1 == 0), saturating"""
    a = min(abs(float(v)), 6.0)
    d = np.abs(E2M1_GRID - a)
    best = np.flatnonzero(d == d.min())
    code = best[0] if len(best) == 1 else [c for c in best if c % 2 == 0][0]
    return code | (8 if np.signbit(v) else 0)


def test_e2m1_encode_brute_force(O):
    mids = (E2M1_GRID[:-1] + E2M1_GRID[1:]) / 2
    x = np.concatenate([E2M1_GRID, mids, -mids, mids + 1e-3, mids - 1e-3, [7.0, 100.0, -6.5],
                        np.random.default_rng(4).uniform(-7, 7, 2000)]).astype(np.float32)
    got = O.f32_to_e2m1(x)
    want = np.array([_e2m1_brute(v) for v in x], np.uint8)
    # +-0 compare by value
    assert np.array_equal(O.e2m1_to_f32(got), O.e2m1_to_f32(want))


def test_e2m1_table_matches_float4_dtype(O):
    # torch's float4_e2m1fn_x2 stores two codes per byte; decode each code via
    # the OCP definition sign * 2^(e-1) * (1 + m/2) (e>0), 0.5*m (e=0)
    codes = np.arange(16, dtype=np.uint8)
    e = (codes >> 1) & 3
    m = codes & 1
    mag = np.where(e == 0, 0.5 * m, 2.0 ** (e.astype(np.float64) - 1) * (1 + m / 2))
    want = np.where(codes & 8, -mag, mag)
    assert np.array_equal(O.e2m1_to_f32(codes), want.astype(np.float32))


def test_e8m0(O):
    assert O.e8m0_to_f32(np.uint8(127)) == 1.0
    assert O.e8m0_to_f32(np.uint8(130)) == 8.0
    assert O.e8m0_to_f32(np.uint8(0)) == np.float32(2.0 ** -127)
    assert np.isnan(O.e8m0_to_f32(np.uint8(255)))
