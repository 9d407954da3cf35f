"""Shared helpers for the GPU parity tests: seeded weights per format, raw
bytes from the oracle's quantizers, and the oracle reference product."""
import numpy as np

import dialq as dq
import oracle as O


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(O.round_bf16(x)).view(np.uint32).astype(np.uint32) >> 16


def make_weight(fmt, n, k, seed=0, scale_dtype=dq.BF16):
    """Returns (raw_weight, raw_scales, kwargs for Linear.create, dequant f32)."""
    rng = np.random.default_rng(seed)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    kw = {}
    if fmt == dq.W8A16:
        q, s32, sb = O.w8a16_quantize(w)
        scales = sb if scale_dtype == dq.BF16 else s32
        kw["scale_dtype"] = scale_dtype
        deq = O.w8a16_dequant(q, scales)
        return q, scales, kw, deq
    if fmt == dq.Q8_0:
        b = O.q8_0_quantize(w)
        return b, None, kw, O.q8_0_dequant(b, n, k)
    if fmt == dq.Q4_K:
        b = O.q4_k_quantize(w)
        return b, None, kw, O.q4_k_dequant(b, n, k)
    if fmt == dq.Q6_K:
        b = O.q6_k_random_blocks(n, k, seed)
        return b, None, kw, O.q6_k_dequant(b, n, k)
    if fmt == dq.FP8_BLOCK:
        q, s = O.fp8_block_quantize(w)
        return q, s, kw, O.fp8_block_dequant(q, s)
    if fmt == dq.MXFP4:
        p, s = O.mxfp4_quantize(w)
        return p, s, kw, O.mxfp4_dequant(p, s)
    if fmt == dq.FP8_ROW:
        # checkpoint-style codes: random E4M3 bytes (a few NaN codes, which the
        # reference CUDA decode maps to 0) and positive f32 row scales
        q = rng.integers(0, 256, (n, k)).astype(np.uint8)
        s = rng.uniform(0.001, 0.01, n).astype(np.float32)
        deq = O.fp8_row_dequant(q, s)
        return q, s, kw, deq
    if fmt == dq.NVFP4:
        p = rng.integers(0, 256, (n, k // 2)).astype(np.uint8)
        # E4M3 group scales in [2^-9, 448], a few NaN codes (decode to 0)
        s = rng.integers(1, 127, (n, k // 16)).astype(np.uint8)
        s.ravel()[::97] = 0x7F
        g = np.float32(0.0123)
        kw["global_scale"] = float(g)
        deq = O.nvfp4_dequant(p, s, g, n, k, scales_are_e4m3=True)
        return p, s, kw, deq
    raise ValueError(fmt)


def k_align(fmt):
    return {dq.Q4_K: 256, dq.Q6_K: 256, dq.Q8_0: 32, dq.MXFP4: 32, dq.NVFP4: 16}.get(fmt, 8)


def reference_product(x_f32, deq, y_dtype):
    """fp64 product of the exact activations and dequantized weights, rounded
    to the output dtype."""
    y = O.matmul_f64(x_f32, deq).astype(np.float32)
    if y_dtype == dq.BF16:
        return O.round_bf16(y)
    if y_dtype == dq.F16:
        return O.round_f16(y)
    return y


def to_torch(x_f32, dtype_code, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x_f32, np.float32)).to(device)
    return t.to({dq.F32: torch.float32, dq.F16: torch.float16, dq.BF16: torch.bfloat16}[dtype_code])


def empty_out(m, n, dtype_code, device):
    import torch
    return torch.full((m, n), float("nan"), device=device,
                      dtype={dq.F32: torch.float32, dq.F16: torch.float16, dq.BF16: torch.bfloat16}[dtype_code])


def exact_inputs(x_f32, dtype_code):
    """The activation values the kernel actually sees, as f32."""
    if dtype_code == dq.BF16:
        return O.round_bf16(x_f32)
    if dtype_code == dq.F16:
        return O.round_f16(x_f32)
    return np.asarray(x_f32, np.float32)
