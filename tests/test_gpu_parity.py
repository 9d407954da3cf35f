"""GPU parity: every format's quantizer, repacker, dequantizer, decode GEMV
and prefill GEMM, called through the C ABI, against the CPU oracle.

Bars: integer / byte work (quantized codes, scales, dequantized weights, the
local-q8 output) bit-exact; products within 1e-3 relative L2 (bf16 / f16
outputs, weight-only paths) or 2e-3 (native fp8 / fp4 prefill, whose oracle
applies the same activation quantizer) of the fp64 oracle product rounded to
the output dtype."""
import numpy as np
import pytest

import dialq as dq
import oracle as O
from helpers import (empty_out, exact_inputs, k_align, make_weight, reference_product, to_torch)

pytestmark = pytest.mark.gpu

ALL_FORMATS = [dq.W8A16, dq.Q8_0, dq.Q4_K, dq.Q6_K, dq.FP8_ROW, dq.FP8_BLOCK, dq.NVFP4, dq.MXFP4]
TOL_BF16 = 1e-3   # relative L2, weight-only products
TOL_LOWP = 2e-3   # relative L2, native fp8 / fp4 prefill


def _linear(fmt, n, k, seed=0, **kw):
    raw, scales, ckw, deq = make_weight(fmt, n, k, seed, **kw)
    lin = dq.Linear.create(fmt, n, k, raw, scales, **ckw)
    return lin, raw, scales, deq


def _run(lin, deq, m, x_dtype, y_dtype, path, dev, seed=1):
    import torch
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (m, lin.in_dim)).astype(np.float32)
    xt = to_torch(x, x_dtype, dev)
    yt = empty_out(m, lin.out_dim, y_dtype, dev)
    lin.forward(xt, yt, path=path)
    torch.cuda.synchronize()
    ref = reference_product(exact_inputs(x, x_dtype), deq, y_dtype)
    got = yt.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    return O.rel_l2(got, ref)


# ---- dequantizer: bit-exact ---------------------------------------------------
@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_dequant_bit_exact(fmt, torch_dev):
    import torch
    n, k = 77, 512
    lin, raw, scales, deq = _linear(fmt, n, k, seed=fmt)
    out = torch.empty(n, k, dtype=torch.float32, device=torch_dev)
    lin.dequantize(out)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), deq.view(np.uint32)), fmt
    for td, rnd in ((torch.float16, O.round_f16), (torch.bfloat16, O.round_bf16)):
        o2 = torch.empty(n, k, dtype=td, device=torch_dev)
        lin.dequantize(o2)
        assert np.array_equal(o2.float().cpu().numpy(), rnd(deq))


@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_export_round_trip(fmt, torch_dev):
    n, k = 50, 256
    lin, raw, scales, deq = _linear(fmt, n, k, seed=10 + fmt)
    w, s = lin.export()
    raw = np.asarray(raw)
    if fmt == dq.FP8_ROW:  # NaN codes are stored as the zero of the same sign
        raw = np.where((raw & 0x7F) == 0x7F, raw & 0x80, raw)
    if fmt == dq.NVFP4:
        scales = np.where((scales & 0x7F) == 0x7F, scales & 0x80, scales)
    assert np.array_equal(w.reshape(-1).view(np.uint8), raw.reshape(-1).view(np.uint8))
    if scales is not None:
        assert np.array_equal(np.asarray(s).reshape(-1).view(np.uint8),
                              np.asarray(scales).reshape(-1).view(np.uint8))


# ---- quantizers: bit-exact -----------------------------------------------------
@pytest.mark.parametrize("dense_dtype", [dq.F32, dq.BF16, dq.F16])
@pytest.mark.parametrize("scale_dtype", [dq.F32, dq.BF16])
def test_w8a16_quantizer_bit_exact(dense_dtype, scale_dtype, torch_dev):
    rng = np.random.default_rng(3)
    n, k = 37, 200
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    w[3] = 0.0
    w[5, :3] = [0.5, -0.5, 1.5]
    wt = to_torch(w, dense_dtype, torch_dev)
    lin = dq.Linear.quantize(dq.W8A16, wt, scale_dtype=scale_dtype)
    q, s = lin.export()
    q_ref, s32, sb = O.w8a16_quantize(exact_inputs(w, dense_dtype))
    assert np.array_equal(q, q_ref)
    assert np.array_equal(np.asarray(s), sb if scale_dtype == dq.BF16 else s32)


@pytest.mark.parametrize("fmt", [dq.Q8_0, dq.Q4_K, dq.FP8_BLOCK, dq.MXFP4],
                         ids=lambda f: dq.FORMAT_NAMES[f])
def test_block_quantizers_bit_exact(fmt, torch_dev):
    rng = np.random.default_rng(4)
    n, k = 40, 512
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    w[1, :256] = 0.0
    w[2, :256] = 0.003
    lin = dq.Linear.quantize(fmt, to_torch(w, dq.F32, torch_dev))
    got_w, got_s = lin.export()
    if fmt == dq.Q8_0:
        ref_w, ref_s = O.q8_0_quantize(w), None
    elif fmt == dq.Q4_K:
        ref_w, ref_s = O.q4_k_quantize(w), None
    elif fmt == dq.FP8_BLOCK:
        ref_w, ref_s = O.fp8_block_quantize(w)
    else:
        ref_w, ref_s = O.mxfp4_quantize(w)
    assert np.array_equal(got_w.reshape(-1), ref_w.reshape(-1))
    if ref_s is not None:
        assert np.array_equal(np.asarray(got_s).reshape(-1).view(np.uint8),
                              np.asarray(ref_s).reshape(-1).view(np.uint8))


@pytest.mark.parametrize("dense_dtype", [dq.F32, dq.F16], ids=["f32", "f16"])
def test_q4_k_quantizer_closed_form_cases(dense_dtype, torch_dev):
    # the device quantizer on inputs whose Q4_K bytes follow from arithmetic
    # alone (tests/q4k_cases.py: exact grids, the min > 0 clamp, half-way
    # ties of nearest_int, the 6-bit packing at every sub-block position).
    # The grid values need up to 11 significant bits, which f16 holds (bf16,
    # with 8, does not).
    import q4k_cases
    w, want, names = q4k_cases.cases()
    assert np.array_equal(exact_inputs(w, dense_dtype), w)
    lin = dq.Linear.quantize(dq.Q4_K, to_torch(w, dense_dtype, torch_dev))
    got, _ = lin.export()
    for r, name in enumerate(names):
        assert np.array_equal(got[r], want[r]), (name, np.nonzero(got[r] != want[r])[0][:8])


# ---- decode GEMV ---------------------------------------------------------------
@pytest.mark.parametrize("x_dtype", [dq.BF16, dq.F16, dq.F32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_gemv_parity(fmt, x_dtype, torch_dev):
    n, k = 200, 512
    lin, _, _, deq = _linear(fmt, n, k, seed=20 + fmt)
    for m in (1, 3, 8, 16, 33):
        y_dtype = dq.F16 if x_dtype == dq.F16 else dq.BF16
        rel = _run(lin, deq, m, x_dtype, y_dtype, dq.PATH_GEMV, torch_dev, seed=m)
        assert rel <= TOL_BF16, (dq.FORMAT_NAMES[fmt], m, rel)


@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_gemv_parity_whole_strip_ranges(fmt, torch_dev):
    """Enough 16-row strips (301, the last one ragged) that every workgroup
    takes whole strips, for staged (small K) and ring-fetched (large M)
    activations."""
    n, k = 16 * 300 + 7, 512
    lin, _, _, deq = _linear(fmt, n, k, seed=25 + fmt)
    for m, x_dtype in ((1, dq.BF16), (2, dq.F32), (5, dq.F16), (16, dq.BF16), (17, dq.BF16)):
        y_dtype = dq.F16 if x_dtype == dq.F16 else dq.BF16
        rel = _run(lin, deq, m, x_dtype, y_dtype, dq.PATH_GEMV, torch_dev, seed=m)
        assert rel <= TOL_BF16, (dq.FORMAT_NAMES[fmt], m, rel)


@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_gemv_parity_work_queue(fmt, torch_dev):
    """Fewer strips (19) than CUs with activations too large to stage in LDS
    (M x K x bytes > 128 KB): the work-queue kernel, whose strips are split
    into pieces reduced across workgroups."""
    n, k = 300, 8704
    lin, _, _, deq = _linear(fmt, n, k, seed=27 + fmt)
    for m, x_dtype in ((9, dq.BF16), (16, dq.BF16), (4, dq.F32), (20, dq.F16)):
        y_dtype = dq.F16 if x_dtype == dq.F16 else dq.BF16
        rel = _run(lin, deq, m, x_dtype, y_dtype, dq.PATH_GEMV, torch_dev, seed=m)
        assert rel <= TOL_BF16, (dq.FORMAT_NAMES[fmt], m, rel)


@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_gemv_f32_output(fmt, torch_dev):
    n, k = 64, 256
    lin, _, _, deq = _linear(fmt, n, k, seed=30 + fmt)
    rel = _run(lin, deq, 4, dq.BF16, dq.F32, dq.PATH_GEMV, torch_dev)
    assert rel <= 1e-5, rel


# ---- prefill GEMM (weight-only) --------------------------------------------------
@pytest.mark.parametrize("x_dtype", [dq.BF16, dq.F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("fmt", ALL_FORMATS, ids=lambda f: dq.FORMAT_NAMES[f])
def test_gemm_parity(fmt, x_dtype, torch_dev):
    n, k = 300, 512
    lin, _, _, deq = _linear(fmt, n, k, seed=40 + fmt)
    for m in (65, 130):
        y_dtype = dq.F16 if x_dtype == dq.F16 else dq.BF16
        rel = _run(lin, deq, m, x_dtype, y_dtype, dq.PATH_GEMM, torch_dev, seed=m)
        assert rel <= TOL_BF16, (dq.FORMAT_NAMES[fmt], m, rel)


def test_gemm_f32_activations(torch_dev):
    lin, _, _, deq = _linear(dq.W8A16, 96, 256, seed=50)
    rel = _run(lin, deq, 70, dq.F32, dq.F32, dq.PATH_GEMM, torch_dev)
    assert rel <= 1e-5, rel


# ---- native fp8 / fp4 prefill --------------------------------------------------
def _native_ref(fmt, x, deq):
    if fmt == dq.FP8_BLOCK:
        q, s = O.act_fp8_quantize(x)
        xh = O.e4m3_to_f32(q) * s[:, None]
    else:
        p, s = O.act_mxfp4_quantize(x)
        xh = O.mxfp4_dequant(p, s)
    return O.round_bf16(O.matmul_f64(xh, deq).astype(np.float32))


@pytest.mark.parametrize("fmt", [dq.FP8_BLOCK, dq.MXFP4], ids=["fp8_block", "mxfp4"])
def test_native_prefill_parity(fmt, torch_dev):
    import torch
    n, k = 300, 640
    lin, _, _, deq = _linear(fmt, n, k, seed=60 + fmt)
    for m in (100, 256):
        rng = np.random.default_rng(m)
        x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
        xt = to_torch(x, dq.BF16, torch_dev)
        yt = empty_out(m, n, dq.BF16, torch_dev)
        lin.forward(xt, yt, path=dq.PATH_GEMM_NATIVE)
        torch.cuda.synchronize()
        rel = O.rel_l2(yt.float().cpu().numpy(), _native_ref(fmt, x, deq))
        assert rel <= TOL_LOWP, (dq.FORMAT_NAMES[fmt], m, rel)


@pytest.mark.parametrize("fmt", [dq.FP8_BLOCK, dq.MXFP4], ids=["fp8_block", "mxfp4"])
def test_native_prefill_long_k(fmt, torch_dev):
    """K = 20480: past the register-held rows of the FP8 token quantizer (its
    two-pass form) and 160 chunks of the GEMM."""
    import torch
    n, k, m = 96, 20480, 70
    lin, _, _, deq = _linear(fmt, n, k, seed=90 + fmt)
    rng = np.random.default_rng(91)
    x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
    yt = empty_out(m, n, dq.BF16, torch_dev)
    lin.forward(to_torch(x, dq.BF16, torch_dev), yt, path=dq.PATH_GEMM_NATIVE)
    torch.cuda.synchronize()
    rel = O.rel_l2(yt.float().cpu().numpy(), _native_ref(fmt, x, deq))
    assert rel <= TOL_LOWP, (dq.FORMAT_NAMES[fmt], rel)


@pytest.mark.parametrize("fmt", [dq.FP8_BLOCK, dq.MXFP4], ids=["fp8_block", "mxfp4"])
def test_native_prefill_stream_k_split_tiles(fmt, torch_dev):
    """Tiles shared by several workgroups (stream-K): the result matches the
    oracle and is bit-identical from call to call, whichever workgroup
    finishes a shared tile last."""
    import torch
    n, k = 300, 8192  # 64 chunks: FP8 tiles split in 8 pieces, MXFP4 in 2
    lin, _, _, deq = _linear(fmt, n, k, seed=95 + fmt)
    for m in (300, 45):
        rng = np.random.default_rng(m)
        x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
        xt = to_torch(x, dq.BF16, torch_dev)
        outs = []
        for _ in range(3):
            yt = empty_out(m, n, dq.F32, torch_dev)
            lin.forward(xt, yt, path=dq.PATH_GEMM_NATIVE)
            torch.cuda.synchronize()
            outs.append(yt.cpu().numpy())
        assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs[1:])
        rel = O.rel_l2(O.round_bf16(outs[0]), _native_ref(fmt, x, deq))
        assert rel <= TOL_LOWP, (dq.FORMAT_NAMES[fmt], m, rel)


def _assert_bits_equal(got, want, x):
    # a code of -0 reaches the product as +0 (-0 + 0 = +0), so zeros compare by value
    bad = np.argwhere((got.view(np.uint32) != want.view(np.uint32)) & ~((got == 0) & (want == 0)))
    if len(bad):
        i, j = bad[0]
        raise AssertionError(f"{len(bad)} mismatches; first at {(i, j)}: got {got[i, j]!r} want {want[i, j]!r} "
                             f"x {x[i, j]!r}")


def _tie_rows(k):
    """Activation rows whose scaled values sit on the E4M3 / E2M1 rounding
    ties and saturation edges: row 0 has amax 448 (FP8 scale 1), every
    32-block of row 1 has amax 6 (MXFP4 shared exponent 0)."""
    e4m3_ties = [1.0625, -1.1875, 2.5625, 0.0029296875, -0.0048828125, 0.0009765625, 447.9, 464.0 - 1e-3,
                 240.0 + 8.0, 3.0 * 2 ** -10, 13.0, 0.001953125, 1e-30]
    e2m1_ties = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.75, -5.0, 0.1, 5.99, 1e-30, -2.5, 2.0, 0.5]
    x = np.zeros((2, k), np.float32)
    x[0, 0] = 448.0
    x[0, 1:1 + len(e4m3_ties)] = e4m3_ties
    for b in range(k // 32):
        x[1, 32 * b] = 6.0
        x[1, 32 * b + 1:32 * b + 1 + len(e2m1_ties)] = e2m1_ties
    return x


def test_native_activation_quantizer_ties(torch_dev):
    """Rounding ties, subnormal codes and saturation of both activation
    quantizers, bit-exact against the oracle through an identity weight."""
    import torch
    k = 384
    x = np.concatenate([_tie_rows(k), np.random.default_rng(5).normal(0, 1, (6, k)).astype(np.float32)])
    q = np.zeros((k, k), np.uint8)
    np.fill_diagonal(q, 0x38)
    lin = dq.Linear.create(dq.FP8_BLOCK, k, k, q, np.ones((3, 3), np.float32))
    y = empty_out(len(x), k, dq.F32, torch_dev)
    lin.forward(to_torch(x, dq.F32, torch_dev), y, path=dq.PATH_GEMM_NATIVE)
    torch.cuda.synchronize()
    qx, sx = O.act_fp8_quantize(x)
    _assert_bits_equal(y.cpu().numpy(), (O.e4m3_to_f32(qx) * sx[:, None]).astype(np.float32), x)
    p = np.zeros((k, k // 2), np.uint8)
    for i in range(k):
        p[i, i // 2] |= 2 << (4 * (i % 2))
    lin = dq.Linear.create(dq.MXFP4, k, k, p, np.full((k, k // 32), 127, np.uint8))
    y = empty_out(len(x), k, dq.F32, torch_dev)
    lin.forward(to_torch(x, dq.F32, torch_dev), y, path=dq.PATH_GEMM_NATIVE)
    torch.cuda.synchronize()
    px, sxm = O.act_mxfp4_quantize(x)
    _assert_bits_equal(y.cpu().numpy(), O.mxfp4_dequant(px, sxm).astype(np.float32), x)


@pytest.mark.parametrize("x_dtype", [dq.BF16, dq.F16, dq.F32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("k", [384, 200], ids=["k384", "k200"])
def test_native_activation_quantizer_exact(k, x_dtype, torch_dev):
    """The activation quantizers, bit-exact, seen through an identity weight:
    y[m, n] = dequant(xq)[m, n] is one exactly rounded f32 product (FP8:
    e4m3(q) * s) or an exact value (MXFP4: e2m1 * 2^e), so the product
    equals the oracle's dequantized activations bit for bit."""
    import torch
    rng = np.random.default_rng(k + x_dtype)
    m = 70
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    x[3] = 0.0                       # all-zero token: scale 1 / E8M0 floor
    x[5, : k // 2] *= 1e-3           # blocks of very different magnitude
    xe = exact_inputs(x, x_dtype)
    # FP8_BLOCK identity: code 0x38 (1.0) on the diagonal, unit block scales
    q = np.zeros((k, k), np.uint8)
    np.fill_diagonal(q, 0x38)
    s = np.ones(((k + 127) // 128, (k + 127) // 128), np.float32)
    lin = dq.Linear.create(dq.FP8_BLOCK, k, k, q, s)
    y = empty_out(m, k, dq.F32, torch_dev)
    lin.forward(to_torch(x, x_dtype, torch_dev), y, path=dq.PATH_GEMM_NATIVE)
    torch.cuda.synchronize()
    qx, sx = O.act_fp8_quantize(xe)
    want = (O.e4m3_to_f32(qx) * sx[:, None]).astype(np.float32)
    _assert_bits_equal(y.cpu().numpy(), want, xe)
    if k % 32:
        return
    # MXFP4 identity: E2M1 code 2 (1.0) on the diagonal, E8M0 scale 127 (1.0)
    p = np.zeros((k, k // 2), np.uint8)
    for i in range(k):
        p[i, i // 2] |= 2 << (4 * (i % 2))
    lin = dq.Linear.create(dq.MXFP4, k, k, p, np.full((k, k // 32), 127, np.uint8))
    y = empty_out(m, k, dq.F32, torch_dev)
    lin.forward(to_torch(x, x_dtype, torch_dev), y, path=dq.PATH_GEMM_NATIVE)
    torch.cuda.synchronize()
    px, sxm = O.act_mxfp4_quantize(xe)
    want = O.mxfp4_dequant(px, sxm).astype(np.float32)
    _assert_bits_equal(y.cpu().numpy(), want, xe)


def test_native_fp8_block_scale_extremes(torch_dev):
    """FP8 block scales that are zero or span 2^-40 .. 2^40 along k: the
    native kernel folds each 128x128 block scale into the running sum per
    chunk, and a zero-scale block must contribute exactly nothing."""
    import torch
    n, k, m = 384, 1152, 160
    rng = np.random.default_rng(77)
    q = rng.integers(0, 256, (n, k), dtype=np.uint8)
    q = np.where((q & 0x7F) == 0x7F, q & 0x80, q).astype(np.uint8)  # no NaN codes
    nb, kb = (n + 127) // 128, (k + 127) // 128
    s = (2.0 ** rng.integers(-40, 41, (nb, kb))).astype(np.float32)
    s *= rng.uniform(0.5, 1.0, (nb, kb)).astype(np.float32)
    s[0, 0] = 0.0
    s[1, 3:6] = 0.0
    s[2, :] = s[2, 0]  # equal scales along k: the rescale is skipped
    lin = dq.Linear.create(dq.FP8_BLOCK, n, k, q, s)
    deq = O.fp8_block_dequant(q, s)
    x = O.round_bf16(rng.normal(0, 1, (m, k)).astype(np.float32))
    yt = empty_out(m, n, dq.F32, torch_dev)
    lin.forward(to_torch(x, dq.BF16, torch_dev), yt, path=dq.PATH_GEMM_NATIVE)
    torch.cuda.synchronize()
    qx, sx = O.act_fp8_quantize(x)
    ref = O.matmul_f64(O.e4m3_to_f32(qx) * sx[:, None], deq)
    got = yt.cpu().numpy()
    # per 128-column block: the blocks' magnitudes differ by up to 2^40
    for b in range(nb):
        cols = slice(128 * b, min(n, 128 * b + 128))
        rel = O.rel_l2(got[:, cols], ref[:, cols])
        assert rel <= TOL_LOWP, (b, rel)


# ---- local q8 (W8A8 decode): bit-exact ---------------------------------------
@pytest.mark.parametrize("k", [96, 512])
def test_local_q8_bit_exact(k, torch_dev):
    import torch
    rng = np.random.default_rng(k)
    n = 300
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    q, s, _ = O.w8a16_quantize(w)
    lin = dq.Linear.create(dq.W8A16, n, k, q, s, scale_dtype=dq.F32)
    x = rng.normal(0, 1, (1, k)).astype(np.float32)
    y = torch.empty(1, n, dtype=torch.float32, device=torch_dev)
    lin.local_q8(to_torch(x, dq.F32, torch_dev), y)
    torch.cuda.synchronize()
    want = O.local_q8_forward(x, q, s)
    assert np.array_equal(y.cpu().numpy().ravel(), want)


def test_local_q8_rejects_prefill(torch_dev):
    lin, _, _, _ = _linear(dq.W8A16, 16, 64, scale_dtype=dq.F32)
    import torch
    x = torch.zeros(2, 64, device=torch_dev)
    y = torch.zeros(2, 16, device=torch_dev)
    with pytest.raises(dq.DialqError, match="expects decode"):
        lin.local_q8(x, y)


# ---- edge cases -------------------------------------------------------------
def test_zero_rows_is_noop(torch_dev):
    import torch
    lin, _, _, _ = _linear(dq.W8A16, 32, 64)
    x = torch.zeros(0, 64, dtype=torch.bfloat16, device=torch_dev)
    y = torch.zeros(0, 32, dtype=torch.bfloat16, device=torch_dev)
    lin.forward(x, y, rows=0)


@pytest.mark.parametrize("fmt", [dq.W8A16, dq.FP8_ROW], ids=["w8a16", "fp8_row"])
def test_tiny_and_ragged_shapes(fmt, torch_dev):
    for n, k in ((1, 8), (17, 72), (37, 64), (129, 136)):
        lin, _, _, deq = _linear(fmt, n, k, seed=n)
        for m in (1, 5, 70):
            rel = _run(lin, deq, m, dq.BF16, dq.F32, dq.PATH_AUTO, torch_dev, seed=m)
            assert rel <= 1e-5, (n, k, m, rel)


def test_host_io_forward(torch_dev):
    lin, _, _, deq = _linear(dq.Q8_0, 64, 256)
    x = np.random.default_rng(0).normal(size=(3, 256)).astype(np.float32)
    y = np.empty((3, 64), np.float32)
    lin.forward(x, y)
    assert O.rel_l2(y, O.matmul_f64(x, deq)) < 1e-5


def test_resident_bytes_reference_formulas(torch_dev):
    # cuda_quant.rs:360-371 and worker_w8a16.rs:351
    lin, _, _, _ = _linear(dq.NVFP4, 48, 64)
    assert lin.resident_bytes() == 48 * 64 // 2 + 48 * 64 // 16 + 4
    lin, _, _, _ = _linear(dq.FP8_ROW, 48, 64)
    assert lin.resident_bytes() == 48 * 64 + 48 * 4
    lin, _, _, _ = _linear(dq.W8A16, 48, 64, scale_dtype=dq.F32)
    assert lin.resident_bytes() == 48 * 64 + 48 * 4


@pytest.mark.parametrize("fmt", [dq.W8A16, dq.FP8_ROW], ids=["w8a16", "fp8_row"])
def test_gemm_tall_tiles(fmt, torch_dev):
    # from 2048 rows the byte formats take 128-row tiles: ragged row blocks,
    # every activation dtype, the SwiGLU epilogue
    import torch
    n, k = 320, 512
    lin, _, _, deq = _linear(fmt, n, k, seed=60 + fmt)
    for m, x_dtype, y_dtype, tol in ((2048, dq.BF16, dq.BF16, TOL_BF16), (2100, dq.F16, dq.F16, TOL_BF16),
                                     (2049, dq.F32, dq.F32, 1e-5), (2300, dq.BF16, dq.F32, 1e-5)):
        rel = _run(lin, deq, m, x_dtype, y_dtype, dq.PATH_GEMM, torch_dev, seed=m)
        assert rel <= tol, (m, x_dtype, rel)
    gu, _, _, gdeq = _linear(fmt, 256, k, seed=70 + fmt)
    x = np.random.default_rng(5).normal(0, 1, (2050, k)).astype(np.float32)
    y = torch.empty(2050, 128, device=torch_dev, dtype=torch.float32)
    gu.forward_swiglu(to_torch(x, dq.BF16, torch_dev), y, path=dq.PATH_GEMM)
    torch.cuda.synchronize()
    want = O.swiglu(O.matmul_f64(exact_inputs(x, dq.BF16), gdeq))
    assert O.rel_l2(y.cpu().numpy(), want) <= 1e-5
