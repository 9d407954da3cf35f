"""Q4_K quantizer inputs whose quantized bytes follow from arithmetic alone.

The target is candle-core 0.11's BlockQ4K::from_float (make_qkx1_quants with
nmax 15 and 5 tries per 32-value sub-block, 6-bit sub-scales / mins against
d = f16(max_scale / 63) and dmin = f16(max_min / 63), codes
nearest_int((x + dmin * m) / (d * sc)) clamped to 0..15), the quantizer the
reference calls at worker_gguf.rs:641,657 and qwen3_8/ggml_tests.rs:83-84.

Every sub-block below is an exact affine grid x = a * l - b (l in 0..15,
a and b multiples of 2^-11): the least-squares fit of make_qkx1_quants then
returns (a, b) exactly after one pass, so the expected sub-scales, mins,
d / dmin and codes are integers and powers of two written out here, with no
call into any quantizer.  The cases are chosen so that a plausible mistake
changes bytes:
  * per-sub-block scales and mins whose six bits differ (the j >= 4 high-bit
    packing into bytes 0-7 and the low nibbles in bytes 8-11);
  * sub-blocks whose values are all positive (the `min > 0 -> 0` clamp; without
    it the first grid is fitted from min = a and the codes move);
  * half-way ties in nearest_int, which rounds half away from zero (Rust's
    f32::round): a sub-scale of 2.5 and a min of 4.5 grid units, and codes of
    5l/6 at l = 3, 9, 15;
  * super-blocks with one non-zero sub-block at each position j, and constant
    sub-blocks (max == min -> scale 0, min 0, codes 0).
Left open by these cases: how many fitting passes run when the codes keep
changing (every grid here converges in one), NaN handling, and the sign of a
zero dmin when every min of a super-block is zero (candle folds the mins
with f32::max, whose result for +0 / -0 is unspecified; the oracle and the
device quantizer store +0).
"""
from fractions import Fraction

import numpy as np

U = 2.0 ** -10   # sub-scale unit: d = f16(63 U / 63) = 2^-10
V = 2.0 ** -11   # min unit: dmin = 2^-11
F16_U = 0x1400   # f16 bits of 2^-10
F16_V = 0x1000   # f16 bits of 2^-11


def pack_scales(sc, m):
    """GGUF Q4_K 6-bit packing (llama.cpp block_q4_K): bytes 0-3 hold
    sc[0..3] with sc[4..7] >> 4 in bits 6-7, bytes 4-7 m[0..3] with
    m[4..7] >> 4 in bits 6-7, bytes 8-11 the low nibbles of sc[4..7] | m[4..7] << 4."""
    out = np.zeros(12, np.uint8)
    for j in range(4):
        out[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return out


def pack_codes(codes):
    """qs[32 i + l] = code[64 i + l] | code[64 i + 32 + l] << 4."""
    qs = np.zeros(128, np.uint8)
    for i in range(4):
        for l in range(32):
            qs[32 * i + l] = codes[64 * i + l] | (codes[64 * i + 32 + l] << 4)
    return qs


def block(d_bits, dmin_bits, sc, m, codes):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin_bits], np.uint16).view(np.uint8)
    b[4:16] = pack_scales(sc, m)
    b[16:] = pack_codes(codes)
    return b


def grid(j, start=0):
    """The 32 grid indices of sub-block j: every value of start..15 appears,
    in a scrambled order."""
    vals = list(range(start, 16))
    return [vals[(i * 7 + j) % len(vals)] for i in range(32)]


def half_away(q: Fraction) -> int:
    """nearest_int of a non-negative exact value: round half away from zero."""
    return int(q + Fraction(1, 2))


def cases():
    """Returns (w [rows, 256] float32, expected [rows, 144] uint8, names)."""
    rows, want, names = [], [], []

    def add(name, x, blk):
        rows.append(np.asarray(x, np.float32))
        want.append(blk)
        names.append(name)

    # 1. distinct 6-bit sub-scales and mins on exact grids (max c = max e = 63)
    c = [63, 5, 17, 32, 1, 48, 9, 60]
    e = [7, 63, 0, 12, 40, 3, 63, 21]
    x, codes = [], []
    for j in range(8):
        l = grid(j)
        x += [c[j] * U * li - e[j] * V for li in l]
        codes += l
    add("grid_distinct_scales", x, block(F16_U, F16_V, c, e, codes))

    # 2. all-positive sub-blocks 1..7: codes 1..15, so min = a > 0 is clamped
    # to 0 and the fit is (a, 0), m = 0.  Sub-block 0 is a grid with min 63 V,
    # so dmin = 2^-11: with every min zero, dmin would be the f16 of a zero
    # whose sign candle's f32::max fold leaves unspecified.
    c2 = [63, 2, 33, 7, 16, 51, 4, 29]
    x, codes = [], []
    for j in range(8):
        l = grid(j, start=0 if j == 0 else 1)
        x += [c2[j] * U * li - (63 * V if j == 0 else 0.0) for li in l]
        codes += l
    add("all_positive_subblocks", x, block(F16_U, F16_V, c2, [63] + [0] * 7, codes))

    # 3. half-way ties.  Sub-block 0: a = 63 U (sets d).  Sub-block 1: a =
    # 2.5 U -> sub-scale nearest_int(2.5) = 3, so its codes are
    # nearest_int(2.5 U l / 3 U) = nearest_int(5 l / 6), ties at l = 3, 9, 15.
    # Sub-block 2: min b = 4.5 V -> m = nearest_int(4.5) = 5; with a = 8 U its
    # codes are nearest_int(l + 1/32) = l.  Sub-block 3: b = 63 V (sets dmin).
    # The rest are plain grids.
    a = [Fraction(63), Fraction(5, 2), Fraction(8), Fraction(12), Fraction(3), Fraction(40), Fraction(1),
         Fraction(22)]
    b = [Fraction(0), Fraction(6), Fraction(9, 2), Fraction(63), Fraction(10), Fraction(0), Fraction(2),
         Fraction(17)]
    sc = [half_away(v) for v in a]
    mm = [half_away(v) for v in b]
    x, codes = [], []
    for j in range(8):
        l = grid(j)
        x += [float(a[j]) * U * li - float(b[j]) * V for li in l]
        # (x + dmin m) / (d sc) = (a U l - b V + m V) / (sc U)
        codes += [min(15, half_away((a[j] * l_ + (mm[j] - b[j]) / 2) / sc[j])) for l_ in l]
    assert sc[1] == 3 and mm[2] == 5  # the two rounding ties
    add("half_way_ties", x, block(F16_U, F16_V, sc, mm, codes))

    # 4. one non-zero sub-block per super-block, at each position j: its own
    # scale and min are the maxima (sub-scale 63, min 63); the other seven are
    # constant zero (scale 0, min 0, codes 0)
    for j in range(8):
        x = [0.0] * 256
        codes = [0] * 256
        l = grid(j)
        for i in range(32):
            x[32 * j + i] = 63 * U * l[i] - 63 * V
            codes[32 * j + i] = l[i]
        sc = [0] * 8
        mm = [0] * 8
        sc[j] = mm[j] = 63
        add(f"single_subblock_{j}", x, block(F16_U, F16_V, sc, mm, codes))

    # 5. constant sub-blocks (max == min) next to grids: a negative constant
    # and a positive one quantize to scale 0 / min 0 / codes 0
    c5 = [63, 0, 11, 0, 30, 0, 63, 5]
    e5 = [3, 0, 63, 0, 0, 0, 12, 1]
    x, codes = [], []
    for j in range(8):
        if c5[j] == 0:
            x += [(-0.75 if j % 4 == 1 else 0.3125)] * 32
            codes += [0] * 32
        else:
            l = grid(j)
            x += [c5[j] * U * li - e5[j] * V for li in l]
            codes += l
    add("constant_subblocks", x, block(F16_U, F16_V, c5, e5, codes))

    # 6. an all-zero super-block: every byte zero
    add("zero_block", [0.0] * 256, np.zeros(144, np.uint8))
    return np.stack(rows), np.stack(want), names
