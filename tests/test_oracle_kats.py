"""The oracle against the reference's own known-answer tests
(tests/golden/reference_kats.json, restated from the Rust tests)."""
import json
import os

import numpy as np
import pytest

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def test_nvfp4_nibble_order_kat(O):
    k = KATS["nvfp4_nibble_order"]
    packed = np.zeros(k["packed_len"], np.uint8)
    for i, v in k["packed_set"].items():
        packed[int(i)] = v
    d = O.nvfp4_dequant(packed, np.array(k["scales_f32"], np.float32), k["global_scale"],
                        k["out_dim"], k["in_dim"]).ravel()
    for i, v in k["expect"].items():
        assert d[int(i)] == v


def test_nvfp4_length_error_kat(O):
    k = KATS["nvfp4_bad_length"]
    with pytest.raises(ValueError, match=k["error_contains"]):
        O.nvfp4_dequant(np.zeros(k["packed_len"], np.uint8), np.array(k["scales_f32"], np.float32),
                        k["global_scale"], k["out_dim"], k["in_dim"])


def test_modelopt_nvfp4_kat(O):
    k = KATS["modelopt_nvfp4"]
    d = O.nvfp4_dequant(np.array(k["packed"], np.uint8), np.array(k["scales_f32"], np.float32),
                        k["global_scale"], k["out_dim"], k["in_dim"]).ravel()
    assert list(d) == k["expect"]


def test_compressed_tensors_nvfp4_kat(O):
    k = KATS["compressed_tensors_nvfp4"]
    d = O.nvfp4_dequant(np.array(k["packed"], np.uint8), np.array(k["scales_f32"], np.float32),
                        np.float32(1.0) / np.float32(k["global_divisor"]), k["out_dim"], k["in_dim"]).ravel()
    assert list(d) == k["expect"]


def test_fp8_per_row_kat(O):
    k = KATS["fp8_per_row_scale"]
    codes = O.f32_to_e4m3(np.array(k["weight_values"], np.float32)).reshape(k["out_dim"], k["in_dim"])
    d = O.fp8_row_dequant(codes, np.array(k["scales"], np.float32)).ravel()
    assert list(d) == k["expect"]


def test_fp8_raw_bits_kat(O):
    bits = np.array(KATS["fp8_raw_bits"]["bits"], np.uint8)
    # decode -> encode round trip preserves the bit patterns
    assert np.array_equal(O.f32_to_e4m3(O.e4m3_to_f32(bits, ocp=True)), bits)


def test_e4m3_code_values(O):
    k = KATS["e4m3_codes"]
    got = O.e4m3_to_f32(np.array(k["codes"], np.uint8))
    assert np.array_equal(got, np.array(k["values"], np.float32))
    assert np.array_equal(np.signbit(got), np.signbit(np.array(k["values"], np.float32)))


def test_smoke_patterns_dense_reference(O):
    """quant_smoke.rs builds its dense expectation with the same decode; the
    oracle must reproduce it element-for-element."""
    k = KATS["quant_smoke"]
    n, kk = k["out_dim"], k["in_dim"]
    packed = np.array([k["packed_pattern"][i % 8] for i in range(n * kk // 2)], np.uint8)
    scales = np.array([k["scale_pattern"][i % 6] for i in range(n * kk // 16)], np.uint8)
    d = O.nvfp4_dequant(packed, scales, k["nvfp4_global"], n, kk, scales_are_e4m3=True)
    e2m1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, 0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    want = np.empty((n, kk), np.float32)
    for idx in range(n * kk):
        row, col = divmod(idx, kk)
        byte = packed[row * kk // 2 + col // 2]
        code = byte & 15 if col % 2 == 0 else byte >> 4
        sc = O.e4m3_to_f32(np.uint8(scales[row * kk // 16 + col // 16]), ocp=True)
        want[row, col] = np.float32(np.float32(e2m1[code]) * sc) * np.float32(k["nvfp4_global"])
    assert np.array_equal(d, want)
