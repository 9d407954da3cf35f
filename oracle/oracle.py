"""numpy front end of the CPU oracle (oracle/lib/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the
benchmark's cpu_baseline leg, as the checker.  The product library never
imports it.  Each wrapper names the C function (and through it the reference
file:line) it calls; see oracle.h for the parity status of each.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile oracle.c / cpu_baseline.c with the Makefile beside them."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = C.c_void_p
_I64 = C.c_int64


def _declare(L):
    sig = {
        "or_version": (C.c_uint32, []),
        "or_f16_to_f32": (C.c_float, [C.c_uint16]),
        "or_f32_to_f16": (C.c_uint16, [C.c_float]),
        "or_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "or_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "or_e4m3_to_f32": (C.c_float, [C.c_uint8]),
        "or_e4m3_to_f32_ocp": (C.c_float, [C.c_uint8]),
        "or_f32_to_e4m3": (C.c_uint8, [C.c_float]),
        "or_e2m1_to_f32": (C.c_float, [C.c_uint8]),
        "or_f32_to_e2m1": (C.c_uint8, [C.c_float]),
        "or_e8m0_to_f32": (C.c_float, [C.c_uint8]),
        "or_w8a16_quantize": (None, [_P, _I64, _I64, _P, _P, _P]),
        "or_w8a16_dequant": (None, [_P, _P, C.c_int, _I64, _I64, _P]),
        "or_q8_0_quantize": (None, [_P, _I64, _I64, _P]),
        "or_q8_0_dequant": (None, [_P, _I64, _I64, _P]),
        "or_q4_k_quantize": (None, [_P, _I64, _I64, _P]),
        "or_q4_k_dequant": (None, [_P, _I64, _I64, _P]),
        "or_q6_k_dequant": (None, [_P, _I64, _I64, _P]),
        "or_fp8_row_dequant": (None, [_P, _P, _I64, _I64, _P]),
        "or_fp8_block_quantize": (None, [_P, _I64, _I64, _P, _P]),
        "or_fp8_block_dequant": (None, [_P, _P, _I64, _I64, _P]),
        "or_nvfp4_dequant": (C.c_int, [_P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_float,
                                       _I64, _I64, _P, C.c_char_p, C.c_size_t]),
        "or_mxfp4_quantize": (None, [_P, _I64, _I64, _P, _P]),
        "or_mxfp4_dequant": (None, [_P, _P, _I64, _I64, _P]),
        "or_act_fp8_quantize": (None, [_P, _I64, _I64, _P, _P]),
        "or_act_mxfp4_quantize": (None, [_P, _I64, _I64, _P, _P]),
        "or_matmul_f64": (None, [_P, _P, _I64, _I64, _I64, _P]),
        "or_w8a16_linear": (None, [_P, _P, _P, C.c_int, _I64, _I64, _I64, _P]),
        "or_local_q8_forward": (None, [_P, _I64, _P, _P, _I64, _P]),
        "cb_w8a16_gemv": (None, [_P, _I64, _I64, _P, _P, _I64, _P, C.c_int]),
        "cb_q4_k_gemv": (None, [_P, _I64, _I64, _P, _I64, _P, C.c_int]),
        "cb_w8a16_gemm": (None, [_P, _I64, _I64, _P, _P, _I64, _P, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- scalar codecs (vectorised over numpy arrays) -------------------------
def _vec(fn, dtype_out, arr):
    L = lib()
    f = getattr(L, fn)
    flat = np.asarray(arr).ravel()
    return np.array([f(v.item()) for v in flat], dtype=dtype_out).reshape(np.shape(arr))


def f16_bits_to_f32(h):
    return _vec("or_f16_to_f32", np.float32, np.asarray(h, np.uint16))


def f32_to_f16_bits(f):
    return _vec("or_f32_to_f16", np.uint16, np.asarray(f, np.float32))


def bf16_bits_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f):
    return _vec("or_f32_to_bf16", np.uint16, np.asarray(f, np.float32))


def e4m3_to_f32(codes, ocp: bool = False):
    return _vec("or_e4m3_to_f32_ocp" if ocp else "or_e4m3_to_f32", np.float32,
                np.asarray(codes, np.uint8))


def f32_to_e4m3(f):
    return _vec("or_f32_to_e4m3", np.uint8, np.asarray(f, np.float32))


def e2m1_to_f32(codes):
    return _vec("or_e2m1_to_f32", np.float32, np.asarray(codes, np.uint8))


def f32_to_e2m1(f):
    return _vec("or_f32_to_e2m1", np.uint8, np.asarray(f, np.float32))


def e8m0_to_f32(e):
    return _vec("or_e8m0_to_f32", np.float32, np.asarray(e, np.uint8))


# ---- formats ---------------------------------------------------------------
def w8a16_quantize(w):
    w = _f32(w)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    sb = np.empty(n, np.uint16)
    lib().or_w8a16_quantize(_p(w), n, k, _p(q), _p(s), _p(sb))
    return q, s, sb


def w8a16_dequant(q, scale):
    q = np.ascontiguousarray(q, np.int8)
    n, k = q.shape
    is_bf16 = np.asarray(scale).dtype == np.uint16
    scale = np.ascontiguousarray(scale, np.uint16 if is_bf16 else np.float32)
    out = np.empty((n, k), np.float32)
    lib().or_w8a16_dequant(_p(q), _p(scale), int(is_bf16), n, k, _p(out))
    return out


def q8_0_quantize(w):
    w = _f32(w)
    n, k = w.shape
    out = np.empty((n, k // 32 * 34), np.uint8)
    lib().or_q8_0_quantize(_p(w), n, k, _p(out))
    return out


def q8_0_dequant(blocks, n, k):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty((n, k), np.float32)
    lib().or_q8_0_dequant(_p(blocks), n, k, _p(out))
    return out


def q4_k_quantize(w):
    w = _f32(w)
    n, k = w.shape
    out = np.empty((n, k // 256 * 144), np.uint8)
    lib().or_q4_k_quantize(_p(w), n, k, _p(out))
    return out


def q4_k_dequant(blocks, n, k):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty((n, k), np.float32)
    lib().or_q4_k_dequant(_p(blocks), n, k, _p(out))
    return out


def q6_k_dequant(blocks, n, k):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty((n, k), np.float32)
    lib().or_q6_k_dequant(_p(blocks), n, k, _p(out))
    return out


def q6_k_random_blocks(n, k, seed=0, d_scale=2e-4):
    """Seeded Q6_K blocks for tests: uniform 6-bit codes and i8 scales, d =
    f16(d_scale * u) with u in [0.5, 1.5) (GGUF Q6_K quantization is not part
    of the path: Q6_K weights come from files)."""
    rng = np.random.default_rng(seed)
    nb = n * (k // 256)
    b = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
    d = (d_scale * rng.uniform(0.5, 1.5, nb)).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return b.reshape(n, (k // 256) * 210)


def fp8_row_dequant(q, scale):
    q = np.ascontiguousarray(q, np.uint8)
    n, k = q.shape
    scale = np.ascontiguousarray(np.broadcast_to(np.asarray(scale, np.float32), (n,)))
    out = np.empty((n, k), np.float32)
    lib().or_fp8_row_dequant(_p(q), _p(scale), n, k, _p(out))
    return out


def fp8_block_quantize(w):
    w = _f32(w)
    n, k = w.shape
    q = np.empty((n, k), np.uint8)
    s = np.empty(((n + 127) // 128, (k + 127) // 128), np.float32)
    lib().or_fp8_block_quantize(_p(w), n, k, _p(q), _p(s))
    return q, s


def fp8_block_dequant(q, s):
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    n, k = q.shape
    out = np.empty((n, k), np.float32)
    lib().or_fp8_block_dequant(_p(q), _p(s), n, k, _p(out))
    return out


def nvfp4_dequant(packed, scales, global_scale, n, k, scales_are_e4m3=None):
    packed = np.ascontiguousarray(packed, np.uint8).ravel()
    scales = np.asarray(scales)
    if scales_are_e4m3 is None:
        scales_are_e4m3 = scales.dtype == np.uint8
    scales = np.ascontiguousarray(scales, np.uint8 if scales_are_e4m3 else np.float32).ravel()
    out = np.empty((n, k), np.float32)
    err = C.create_string_buffer(256)
    rc = lib().or_nvfp4_dequant(_p(packed), packed.size, _p(scales), scales.size,
                                int(scales_are_e4m3), float(global_scale), n, k, _p(out), err, 256)
    if rc != 0:
        raise ValueError(err.value.decode())
    return out


def mxfp4_quantize(w):
    w = _f32(w)
    n, k = w.shape
    packed = np.empty((n, k // 2), np.uint8)
    scales = np.empty((n, k // 32), np.uint8)
    lib().or_mxfp4_quantize(_p(w), n, k, _p(packed), _p(scales))
    return packed, scales


def mxfp4_dequant(packed, scales):
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint8)
    n = packed.shape[0]
    k = packed.shape[1] * 2
    out = np.empty((n, k), np.float32)
    lib().or_mxfp4_dequant(_p(packed), _p(scales), n, k, _p(out))
    return out


def act_fp8_quantize(x):
    x = _f32(x)
    m, k = x.shape
    q = np.empty((m, k), np.uint8)
    s = np.empty(m, np.float32)
    lib().or_act_fp8_quantize(_p(x), m, k, _p(q), _p(s))
    return q, s


def act_mxfp4_quantize(x):
    return mxfp4_quantize(x)


def matmul_f64(x, w):
    x = _f32(x)
    w = _f32(w)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float64)
    lib().or_matmul_f64(_p(x), _p(w), m, n, k, _p(y))
    return y


def rms_norm(x, w, eps):
    """candle_nn::RmsNorm as the GGUF output head applies it
    (qwen3_vl/worker_gguf.rs:267-268, 341): x * w / sqrt(mean(x^2) + eps)
    over the last axis, in float64.  Pinned against the closed form for a
    constant row and against torch.nn.functional.rms_norm
    (tests/test_oracle_formats.py)."""
    x = np.asarray(x, np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * np.asarray(w, np.float64)


def swiglu(gate_up):
    """Mlp::mlp_mid_from_gate_up (qwen3_vl/text.rs:816-820): the fused gate_up
    output's first half is the gate, its second half the up projection;
    returns silu(gate) * up with silu(g) = g / (1 + exp(-g))
    (candle_nn::ops::silu), in float64.  Pinned by known answers and by the
    identity silu(g) - silu(-g) = g (tests/test_oracle_formats.py)."""
    y = np.asarray(gate_up, np.float64)
    n = y.shape[-1]
    if n % 2:
        raise ValueError(f"gate_up width {n} is odd")
    g, u = y[..., : n // 2], y[..., n // 2:]
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * u


# ---- token selection after the lm_head (qwen3_vl/qwen3_vl.rs) --------------
def repeat_penalty(logits, penalty, context):
    """apply_repeat_penalty_in_place (qwen3_vl.rs:225-240): for each distinct
    id of `context` below len(logits), logit / penalty when logit >= 0, else
    logit * penalty, in f32."""
    out = np.array(logits, np.float32, copy=True)
    p = np.float32(penalty)
    seen = set()
    for t in context:
        t = int(t)
        if t in seen:
            continue
        seen.add(t)
        if t < out.size:
            v = out[t]
            out[t] = v / p if v >= 0 else v * p
    return out


def _total_key(v):
    """f32::total_cmp as an unsigned integer order."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)


def select_total_last(logits, k=1):
    """Iterator::max_by(f32::total_cmp) (qwen3_vl.rs:152-157) generalised to
    the k best: descending IEEE total order, equal values in descending
    index order (max_by returns the last maximum).  Returns (indices,
    values)."""
    v = np.asarray(logits, np.float32)
    key = _total_key(v)
    order = np.lexsort((-np.arange(v.size), -key.astype(np.float64)))  # key desc, then index desc
    idx = order[:k]
    return idx.astype(np.uint32), v[idx]


def select_first_max(logits, k=1):
    """candle's Tensor::argmax as the greedy device path calls it
    (qwen3_vl.rs:137-142), generalised to the k best: the largest value by
    `>`, so -0 and +0 are equal and NaN is never larger; equal values in
    ascending index order.  Returns (indices, values)."""
    v = np.asarray(logits, np.float32)
    w = np.where(v == 0, np.float32(0), v)
    key = np.where(np.isnan(w), 0, _total_key(w))
    order = np.lexsort((np.arange(v.size), -key.astype(np.float64)))
    idx = order[:k]
    return idx.astype(np.uint32), v[idx]


def softmax_stats(logits, temperature):
    """softmax_in_place (qwen3_vl.rs:325-345) before its division: the max M
    of logits / max(temperature, 1e-7) and S = sum exp(logit / t - M), in
    float64 from the f32 quotients."""
    t = np.float32(max(np.float32(temperature), np.float32(1e-7)))
    x = (np.asarray(logits, np.float32) / t).astype(np.float64)
    m = np.max(x)
    return m, float(np.sum(np.exp(x - m)))


def w8a16_linear(x, q, scale):
    x = _f32(x)
    q = np.ascontiguousarray(q, np.int8)
    m, k = x.shape
    n = q.shape[0]
    is_bf16 = np.asarray(scale).dtype == np.uint16
    scale = np.ascontiguousarray(scale, np.uint16 if is_bf16 else np.float32)
    y = np.empty((m, n), np.float32)
    lib().or_w8a16_linear(_p(x), _p(q), _p(scale), int(is_bf16), m, n, k, _p(y))
    return y


def local_q8_forward(x, q, scale):
    x = _f32(x).ravel()
    q = np.ascontiguousarray(q, np.int8)
    n, k = q.shape
    scale = np.ascontiguousarray(scale, np.float32)
    y = np.empty(n, np.float32)
    lib().or_local_q8_forward(_p(x), k, _p(q), _p(scale), n, _p(y))
    return y


# ---- CPU baseline (timed by bench.py's cpu_baseline leg) -----------------
# `native=True` uses lib/native/libcpu_baseline.so, compiled on the calling
# host with -march=native (make native); the default is liboracle.so's
# portable build, which the tests check.
_native = None


def native_lib():
    global _native
    if _native is None:
        # always rebuilt: a copy compiled on another host may use instructions this CPU lacks
        subprocess.run(["make", "-s", "-B", "-C", _HERE, "native"], check=True)
        _native = C.CDLL(os.path.join(_HERE, "lib", "native", "libcpu_baseline.so"))
        for name in ("cb_w8a16_gemv", "cb_q4_k_gemv", "cb_w8a16_gemm"):
            fn = getattr(_native, name)
            fn.restype = None
            fn.argtypes = {"cb_q4_k_gemv": [_P, _I64, _I64, _P, _I64, _P, C.c_int]}.get(
                name, [_P, _I64, _I64, _P, _P, _I64, _P, C.c_int])
    return _native


def cpu_w8a16_gemv(x_bf16, q, scale_bf16, threads, native=False):
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    m, k = x_bf16.shape
    n = q.shape[0]
    y = np.empty((m, n), np.float32)
    (native_lib() if native else lib()).cb_w8a16_gemv(_p(x_bf16), m, k, _p(q), _p(scale_bf16), n, _p(y),
                                                      int(threads))
    return y


def cpu_q4_k_gemv(x_bf16, blocks, n, threads, native=False):
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    m, k = x_bf16.shape
    y = np.empty((m, n), np.float32)
    (native_lib() if native else lib()).cb_q4_k_gemv(_p(x_bf16), m, k, _p(blocks), n, _p(y), int(threads))
    return y


def cpu_w8a16_gemm(x_bf16, q, scale_bf16, threads, native=False):
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    m, k = x_bf16.shape
    n = q.shape[0]
    y = np.empty((m, n), np.float32)
    (native_lib() if native else lib()).cb_w8a16_gemm(_p(x_bf16), m, k, _p(q), _p(scale_bf16), n, _p(y),
                                                      int(threads))
    return y


# ---- helpers ---------------------------------------------------------------
def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def round_bf16(a) -> np.ndarray:
    """Round f32 values to bf16 (RNE) and back to f32 -- vectorised mirror of
    or_f32_to_bf16 for large arrays (checked against it in tests)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rb = 0x8000
    up = ((u & rb) != 0) & ((u & (3 * rb - 1)) != 0)
    hi = (u >> 16) + up.astype(np.uint64)
    hi = np.where(nan, (u >> 16) | 0x40, hi)
    return (hi.astype(np.uint32) << 16).view(np.float32)


def round_f16(a) -> np.ndarray:
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
