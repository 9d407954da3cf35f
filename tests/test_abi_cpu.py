"""The C ABI without a GPU: the library loads, exports every symbol that
include/dialq.h declares, and rejects bad arguments (with the reference's
messages) before touching the device."""
import ctypes as C
import re

import numpy as np
import pytest


def test_library_exports_every_declared_symbol(dq):
    names = dq.declared_symbols()
    assert len(names) >= 12
    for name in names:
        assert hasattr(dq.lib, name), name


def test_no_torch_types_in_header(dq):
    text = open(dq.HEADER_PATH).read()
    assert "torch" not in text.lower().replace("no torch", "")
    assert 'extern "C"' in text


def test_abi_version(dq):
    assert dq.abi_version() == 1


def _create(dq, fmt, n, k, w_bytes, s_bytes, **kw):
    d = dq.Desc(fmt, kw.get("scale_dtype", dq.F32), n, k, kw.get("global_scale", 1.0), kw.get("flags", 0))
    w = np.zeros(max(w_bytes, 1), np.uint8)
    s = np.zeros(max(s_bytes, 1), np.uint8)
    err = C.create_string_buffer(512)
    h = dq.lib.dialq_linear_create(C.byref(d), w.ctypes.data_as(C.c_void_p), w_bytes,
                                   s.ctypes.data_as(C.c_void_p), s_bytes, 0, 1, None, err, 512)
    return h, err.value.decode()


def test_nvfp4_length_checks_use_reference_messages(dq):
    # cuda_quant.rs:301-309
    h, msg = _create(dq, dq.NVFP4, 3, 24, 36, 9, global_scale=0.5)
    assert not h and msg == "NVFP4 QuantLinear input dimension 24 is not divisible by 16"
    h, msg = _create(dq, dq.NVFP4, 3, 32, 47, 6, global_scale=0.5)
    assert not h and msg == "invalid NVFP4 packed weight length 47"
    h, msg = _create(dq, dq.NVFP4, 3, 32, 48, 5, global_scale=0.5)
    assert not h and msg == "invalid NVFP4 scale length 5"


def test_nvfp4_zero_global_rejected(dq):
    # try_cuda_nvfp4 rejects a zero global scale (quant.rs:401-406)
    h, msg = _create(dq, dq.NVFP4, 3, 32, 48, 6, global_scale=0.0)
    assert not h and "non-zero" in msg


def test_fp8_length_checks_use_reference_messages(dq):
    # cuda_quant.rs:339-344
    h, msg = _create(dq, dq.FP8_ROW, 3, 32, 95, 12)
    assert not h and msg == "invalid FP8 weight length 95"
    h, msg = _create(dq, dq.FP8_ROW, 3, 32, 96, 8)
    assert not h and msg == "invalid FP8 scale length 2"


def test_format_alignment_rejected(dq):
    h, msg = _create(dq, dq.Q4_K, 4, 128, 4 * 72, 0)
    assert not h and "not divisible by 256" in msg
    h, msg = _create(dq, dq.Q8_0, 4, 48, 4 * 51, 0)
    assert not h and "not divisible by 32" in msg
    h, msg = _create(dq, 99, 4, 64, 256, 0)
    assert not h and "unknown weight format" in msg


def test_forward_on_null_handle_fails_cleanly(dq):
    err = C.create_string_buffer(256)
    x = np.zeros(8, np.float32)
    rc = dq.lib.dialq_linear_forward(None, x.ctypes.data_as(C.c_void_p), dq.F32, 1,
                                     x.ctypes.data_as(C.c_void_p), dq.F32, None, 0, err, 256)
    assert rc == -1 and b"NULL" in err.value
    dq.lib.dialq_linear_destroy(None)  # no-op


def test_resident_bytes_of_null_is_zero(dq):
    assert dq.lib.dialq_linear_resident_bytes(None) == 0
