"""Pinning the MLX affine oracle (affine_oracle.c) on the CPU.

The oracle restates the following:
  - dequant_affine (engine/src/qwen35.rs:110-134);
  - the QLin layouts (qwen35.rs:311-319, 629-697; quant_kernel.rs:1085-1101);
  - half 2.7.1's bf16::from_f64.

Each check here is computed independently of the restatement:
  - a correctly rounded f64 -> bf16 written with Python integers;
  - the q4woff / q4sb address formulas;
  - a brute-force f64 matmul in numpy.
"""
import math
import struct

import numpy as np

import oracle as O
from helpers import rand_qlin, rand_x


def rne_bf16_exact(v: float) -> int:
    """Correctly rounded f64 -> bf16 (round to nearest, ties to even)."""
    if math.isnan(v):
        return 0x7FC0
    sign = 0x8000 if math.copysign(1.0, v) < 0 else 0
    a = abs(v)
    if a == 0.0:
        return sign
    if math.isinf(a):
        return sign | 0x7F80
    m, e = math.frexp(a)               # a = m * 2^e, 0.5 <= m < 1
    if e - 1 >= -126:                  # normal: 8 significant bits
        r = round(m * 256.0)           # exact product; Python rounds half to even
        val = r * 2.0 ** (e - 8)
    else:                              # subnormal: quantum 2^-133
        val = round(a / 2.0 ** -133) * 2.0 ** -133
    if val >= 2.0 ** 128:
        return sign | 0x7F80
    bits = struct.unpack("<I", struct.pack("<f", val))[0]
    return sign | (bits >> 16)


def test_bf16_from_f64_half_is_correct_rounding_on_20_bit_values():
    """With the low 32 mantissa bits zero, half's truncation changes nothing:
    the restatement must equal correct rounding everywhere (normal,
    subnormal, overflow, ties)."""
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 63, 20000, dtype=np.uint64) & np.uint64(0xFFFFFFFF00000000)
    exps = rng.integers(1023 - 140, 1023 + 130, 20000).astype(np.uint64)
    bits = (bits & ~np.uint64(0x7FF0000000000000)) | (exps << np.uint64(52))
    vals = bits.view(np.float64)
    # exact ties at bf16 precision, both parities
    ties = [1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(2.0 + 2.0 ** -7), 2.0 ** -134, 3 * 2.0 ** -134, 2.0 ** -140]
    for v in list(vals) + ties:
        assert O.bf16_from_f64_half(float(v)) == rne_bf16_exact(float(v)), v


def test_bf16_from_f64_half_truncation_rule():
    """half drops the f64's low 32 mantissa bits before rounding: a value a
    hair above a tie (by those bits only) rounds as the tie does."""
    above_tie = 1.0 + 2.0 ** -8 + 2.0 ** -40
    assert rne_bf16_exact(above_tie) == 0x3F81        # correctly rounded: up
    assert O.bf16_from_f64_half(above_tie) == 0x3F80   # half: tie -> even (down)
    assert O.bf16_from_f64_half(1.0 + 2.0 ** -8 + 2.0 ** -19) == 0x3F81  # a kept bit: up
    # specials
    assert O.bf16_from_f64_half(-0.0) == 0x8000
    assert O.bf16_from_f64_half(float("inf")) == 0x7F80
    assert O.bf16_from_f64_half(float("-inf")) == 0xFF80
    assert O.bf16_from_f64_half(float("nan")) & 0x7FC0 == 0x7FC0
    assert O.bf16_from_f64_half(1e39) == 0x7F80
    assert O.bf16_from_f64_half(3.3895313892515355e38) == 0x7F7F  # largest finite bf16


def test_affine_dequant_matches_formula():
    """dequant_affine on the reference test generator's weights: q*s + b in
    f64, correctly rounded to bf16 (these sums carry < 20 significant bits,
    so half's rule agrees); f32 output = one rounding of the same sum."""
    n, k = 37, 448
    wq, sb = rand_qlin(n, k, 11)
    got = O.affine_dequant_bf16(wq, sb, n, k)
    ng = k // 64
    q = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(n, k).astype(np.float64)
    s = O.bf16_bits_to_f32(sb[:, :ng]).astype(np.float64).repeat(64, axis=1)
    b = O.bf16_bits_to_f32(sb[:, ng:]).astype(np.float64).repeat(64, axis=1)
    exact = q * s + b
    want = np.array([rne_bf16_exact(v) for v in exact.ravel()], dtype=np.uint16).reshape(n, k)
    assert np.array_equal(got, want)
    assert np.array_equal(O.affine_dequant_f32(wq, sb, n, k), exact.astype(np.float32))


def test_affine_dequant_group_128():
    n, k = 5, 512
    wq, sb64 = rand_qlin(n, k, 3)
    sb = np.concatenate([sb64[:, 0:8:2], sb64[:, 8:16:2]], axis=1)   # 4 groups of 128
    got = O.affine_dequant_f32(wq, sb, n, k, gs=128)
    q = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(n, k).astype(np.float64)
    s = O.bf16_bits_to_f32(sb[:, :4]).astype(np.float64).repeat(128, axis=1)
    b = O.bf16_bits_to_f32(sb[:, 4:]).astype(np.float64).repeat(128, axis=1)
    assert np.array_equal(got, (q * s + b).astype(np.float32))


def test_affine_tile_matches_q4woff_q4sb():
    """QLin::tiled vs the kernels' address functions (quant_kernel.rs:1085-1101)."""
    n, k = 300, 384
    wq, sb = rand_qlin(n, k, 5)
    wt, st = O.affine_tile(wq, sb, n, k)
    ng, tiles = k // 64, (n + 255) // 256
    for row in (0, 1, 255, 256, 299):
        for g in range(ng):
            for i in range(8):
                off = (row >> 8) * ng * 2048 + g * 2048 + (row & 255) * 8 + i
                assert wt[off] == wq[row, g * 8 + i]
            prm = ((row >> 8) * ng + g) * 256 + (row & 255)
            assert st[prm] == sb[row, g]
            assert st[prm + tiles * ng * 256] == sb[row, ng + g]
    # padding rows (300 .. 511) are zero
    assert not wt.reshape(tiles, ng, 256, 8)[1, :, 300 - 256:, :].any()


def test_affine_matmul_brute_force():
    n, k, m = 9, 192, 3
    wq, sb = rand_qlin(n, k, 7)
    x = rand_x(k, 8, rows=m)
    y = O.affine_matmul(wq, sb, n, k, x)
    w = O.affine_dequant_f32(wq, sb, n, k).astype(np.float64)  # exact values (< 24 bits)
    ref = x.astype(np.float64) @ w.T
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-6)


def test_reference_generator_is_deterministic():
    a = rand_qlin(4, 128, 11)
    b = rand_qlin(4, 128, 11)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # scales lie on the generator's grid: 0.002 + j * 2e-5 rounded to bf16
    s = O.bf16_bits_to_f32(a[1][:, :2])
    assert ((s >= 0.0019) & (s <= 0.0221)).all()
