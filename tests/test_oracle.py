"""Pins the CPU oracle before anything is compared against it.

Every check here is independent of the oracle's own code: IEEE conversions
against numpy / torch, hand-computed block vectors, exact integer brute
force, the reference's own argmax tie vectors (engine/src/engine.rs:3086-3128)
and the closed form of the gate/up epilogue (engine/src/qwen35.rs:7002-7007).
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle as O


# ---------------------------------------------------------------- conversions
def test_f16_decode_matches_numpy_exhaustive():
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.o_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_matches_numpy():
    L = O.lib()
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  1.0 / 127, 0.02 / 127, np.inf, -np.inf], dtype=np.float32),
        # exact ties between two f16 neighbours (round half to even)
        (np.arange(1024, 1100, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([L.o_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_encode_matches_torch():
    L = O.lib()
    rng = np.random.default_rng(2)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.0e38, 1e-40, 21.03, 20.97], dtype=np.float32),
        # exact ties: 1 + (2k+1) * 2^-8
        (1.0 + (2 * np.arange(0, 64, dtype=np.float32) + 1) * np.float32(2.0 ** -8)).astype(np.float32),
    ]).astype(np.float32)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got_c = np.array([L.o_f32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    got_np = O.f32_to_bf16_bits(vals)
    assert np.array_equal(got_c, ref)
    assert np.array_equal(got_np, ref)


def test_randn_is_seeded_normal():
    a = O.randn(0, 1, 1.0, (1 << 20,))
    b = O.randn(0, 1, 1.0, (1 << 20,))
    c = O.randn(0, 2, 1.0, (1 << 20,))
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)
    assert abs(float(a.mean())) < 5e-3 and abs(float(a.std()) - 1.0) < 5e-3
    w = O.randn(0, 1, 0.02, (4096,))
    assert abs(float(w.std()) - 0.02) < 2e-3


# ---------------------------------------------------------------- Q8_0
def test_q8_0_zero_block():
    blk = O.quantize(O.Q8_0, np.zeros((1, 32), np.float32))
    assert blk.shape == (1, 34) and not blk.any()
    assert not O.dequantize(O.Q8_0, blk, 1, 32).any()


def test_q8_0_exact_power_of_two_block():
    # d = 1/128 is exact in f16; x = q*d for q in [-127, 127] survives exactly
    q = np.array([127, -127, 0, 1, -1, 64, -64, 100] + list(range(-12, 12)), dtype=np.int8)
    x = (q.astype(np.float32) / np.float32(128.0)).reshape(1, 32)
    blk = O.quantize(O.Q8_0, x)
    assert blk[0, 0] == 0x00 and blk[0, 1] == 0x20  # f16(2^-7) = 0x2000 little endian
    assert np.array_equal(blk[0, 2:].view(np.int8), q)
    assert np.array_equal(O.dequantize(O.Q8_0, blk, 1, 32), x)


def test_q8_0_rounds_half_away_from_zero():
    # amax = 127/128 -> d = 1/128, id = 128: x*id = +-2.5 -> +-3 (not banker's 2)
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0 / 128.0
    x[0, 1] = 2.5 / 128.0
    x[0, 2] = -2.5 / 128.0
    x[0, 3] = 3.5 / 128.0
    x[0, 4] = 0.5 / 128.0
    q = O.quantize(O.Q8_0, x)[0, 2:].view(np.int8)
    assert list(q[:5]) == [127, 3, -3, 4, 1]


def test_q8_0_error_bound():
    w = O.randn(0, 7, 0.02, (64, 1024))
    blk = O.quantize(O.Q8_0, w)
    deq = O.dequantize(O.Q8_0, blk, 64, 1024)
    amax = np.abs(w.reshape(64, 32, 32)).max(axis=2, keepdims=True)
    d = amax / 127.0
    err = np.abs(w.reshape(64, 32, 32) - deq.reshape(64, 32, 32))
    # rounding to the level (d/2) plus 127 levels of the f16 rounding of d
    assert np.all(err <= d * (0.5 + 127 * 2.0 ** -11) + 1e-12)


# ---------------------------------------------------------------- Q4_K
def _pack_k4(sc, mn):
    """GGML k4 packing of eight 6-bit (scale, min) pairs into 12 bytes."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= mn[j] & 63
        else:
            s[j + 4] |= (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    return np.array(s, dtype=np.uint8)


def test_q4_k_scale_min_pack_roundtrip_all_pairs():
    rng = np.random.default_rng(3)
    for _ in range(2000):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        packed = _pack_k4(sc, mn)
        for j in range(8):
            assert O.get_scale_min_k4(j, packed) == (sc[j], mn[j])
    # every value in every slot
    for v in range(64):
        packed = _pack_k4([v] * 8, [63 - v] * 8)
        for j in range(8):
            assert O.get_scale_min_k4(j, packed) == (v, 63 - v)


def _q4k_block(d, dmin, sc, mn, qs):
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    blk[4:16] = _pack_k4(sc, mn)
    blk[16:] = qs
    return blk


def test_q4_k_dequant_known_answers():
    # d = 0.5, dmin = 0.25; sub-block scales 1..8, mins 0,2,4,..14 (6-bit)
    sc = [1, 2, 3, 4, 5, 6, 7, 63]
    mn = [0, 2, 4, 6, 8, 10, 12, 63]
    qs = np.zeros(128, np.uint8)
    qs[0] = 0x7A    # element 0: low nibble 10 (sub-block 0); element 32: high 7 (sub-block 1)
    qs[31] = 0xF1   # element 31: 1 (sb 0); element 63: 15 (sb 1)
    qs[32] = 0x23   # element 64: 3 (sb 2); element 96: 2 (sb 3)
    qs[127] = 0x9F  # element 223: 15 (sb 6); element 255: 9 (sb 7)
    y = O.dequantize(O.Q4_K, _q4k_block(0.5, 0.25, sc, mn, qs).reshape(1, 144), 1, 256)[0]
    assert y[0] == 0.5 * 1 * 10 - 0.25 * 0    # 5.0
    assert y[31] == 0.5 * 1 * 1 - 0.0          # 0.5
    assert y[32] == 0.5 * 2 * 7 - 0.25 * 2    # 6.5
    assert y[63] == 0.5 * 2 * 15 - 0.5        # 14.5
    assert y[64] == 0.5 * 3 * 3 - 0.25 * 4    # 3.5
    assert y[96] == 0.5 * 4 * 2 - 0.25 * 6    # 2.5
    assert y[223] == 0.5 * 7 * 15 - 0.25 * 12  # 49.5
    assert y[255] == 0.5 * 63 * 9 - 0.25 * 63  # 267.75
    assert y[1] == 0.0 and y[33] == -0.5 and y[65] == -1.0 and y[254] == -15.75
    assert y[224] == -15.75  # sb 7, nibble 0


def test_q4_k_dequant_is_exact_f32_formula_for_random_bytes():
    # all byte patterns allowed: values are d*sc*q - dmin*m computed with a
    # single rounding (d*sc*q is exact: 11 + 6 + 4 significant bits)
    rng = np.random.default_rng(4)
    n = 64
    raw = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    d = np.abs(rng.standard_normal(n)).astype(np.float16) * np.float16(0.01)
    dm = np.abs(rng.standard_normal(n)).astype(np.float16) * np.float16(0.01)
    raw[:, 0:2] = d.reshape(n, 1).view(np.uint8)
    raw[:, 2:4] = dm.reshape(n, 1).view(np.uint8)
    y = O.dequantize(O.Q4_K, raw, n, 256)
    for r in range(n):
        for sb in range(8):
            s, m = O.get_scale_min_k4(sb, raw[r, 4:16])
            chunk = raw[r, 16 + 32 * (sb // 2): 16 + 32 * (sb // 2) + 32]
            q = (chunk & 0xF) if sb % 2 == 0 else (chunk >> 4)
            exact = float(d[r]) * s * q.astype(np.float64) - float(dm[r]) * m  # f64, then one rounding
            assert np.array_equal(y[r, 32 * sb: 32 * sb + 32], exact.astype(np.float32))


GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "quant_vectors.json")))


def _h2f(a) -> np.ndarray:
    return np.array([int(v, 16) for v in a], np.uint32).view(np.float32)


@pytest.mark.parametrize("s,m", [(2.0 ** -7, 2.0 ** -5), (2.0 ** -3, 0.0), (1.0, 4.0), (2.0 ** -10, 2.0 ** -6),
                                 (2.0 ** -6, 2.0 ** -9)])
def test_make_qkx1_quants_grid_exact(s, m):
    """x = s*l - m with l covering 0..15 and s, m powers of two: the first pass
    finds the levels exactly (iscale = 15/(15s) = 1/s), the least-squares
    scale is s and the mean residual is -m, so the search returns (s, m) and
    l.  nmax 14 would give other levels, a power-of-two bias in the min other
    (s, m)."""
    lv = np.concatenate([np.arange(16), np.arange(16)[::-1]]).astype(np.float32)
    x = (np.float32(s) * lv - np.float32(m)).astype(np.float32)
    sc, mn, l = O.make_qkx1_quants(15, 5, x)
    assert np.array_equal(l, lv.astype(np.uint8))
    assert sc == np.float32(s) and mn == np.float32(m)
    # nmax = 14 cannot represent 16 levels
    assert not np.array_equal(O.make_qkx1_quants(14, 5, x)[2], l)


@pytest.mark.parametrize("case", range(len(GOLDEN["qkx1"])))
def test_make_qkx1_quants_golden(case):
    """Literal (scale, min, levels) from an independent float32 trace of the
    published 5-pass refinement (tests/golden/make_quant_vectors.py).  The
    sub-blocks were drawn so that the levels still change in passes 5 and 6:
    the fixture's ntry-4, ntry-6, ntry-1 and nmax-14 levels all differ from
    the ntry-5 answer, so a wrong pass count or level count fails here."""
    c = GOLDEN["qkx1"][case]
    x = _h2f(c["x"])
    sc, mn, l = O.make_qkx1_quants(15, 5, x)
    assert list(l) == c["levels"]
    assert int(sc.view(np.uint32)) == int(c["scale"], 16)
    assert int(mn.view(np.uint32)) == int(c["min"], 16)
    for other in ("levels_ntry4", "levels_ntry6", "levels_nmax14", "levels_ntry1"):
        assert c[other] != c["levels"], other
    assert list(O.make_qkx1_quants(15, 4, x)[2]) == c["levels_ntry4"]
    assert list(O.make_qkx1_quants(15, 6, x)[2]) == c["levels_ntry6"]


@pytest.mark.parametrize("case", range(len(GOLDEN["q4k"])))
def test_q4_k_quantize_golden(case):
    """BlockQ4K::from_float byte for byte against the float32 trace: Gaussian,
    all-positive (min clamped to 0) and a superblock with a constant sub-block
    and outliers.  The generator checks that 64/max in place of 63/max changes
    each block."""
    c = GOLDEN["q4k"][case]
    blk = O.quantize(O.Q4_K, _h2f(c["x"]).reshape(1, 256))
    assert blk.tobytes().hex() == c["block"]


def test_q4_k_max_scale_and_min_are_63():
    """6-bit scales are quantized against their maxima (63/max): in every
    superblock the sub-block with the largest scale stores 63, and so does the
    one with the largest min whenever some min is positive."""
    w = O.randn(0, 21, 0.02, (64, 1024))
    w[3, :256] = np.abs(w[3, :256]) + 0.001  # all-positive superblock: the first pass clamps the min to 0
    blk = O.quantize(O.Q4_K, w).reshape(-1, 144)
    for b in range(blk.shape[0]):
        pairs = [O.get_scale_min_k4(j, blk[b, 4:16]) for j in range(8)]
        assert max(p[0] for p in pairs) == 63, b
        mx_m = max(p[1] for p in pairs)
        dmin = blk[b, 2:4].view(np.float16)[0]
        assert mx_m == (63 if dmin > 0 else 0), b


def test_q4_k_quantize_invariants():
    w = O.randn(0, 9, 0.02, (32, 1024))
    blk = O.quantize(O.Q4_K, w)
    deq = O.dequantize(O.Q4_K, blk, 32, 1024)
    rel = np.sqrt(((w - deq) ** 2).mean()) / np.sqrt((w ** 2).mean())
    assert rel < 0.12, rel  # 4-bit levels over a +-3 sigma range
    # monotone within a sub-block (shared scale and min)
    wb, db = w.reshape(-1, 32), deq.reshape(-1, 32)
    for i in range(0, wb.shape[0], 7):
        o = np.argsort(wb[i], kind="stable")
        assert np.all(np.diff(db[i][o]) >= 0)
    # constant block -> all zero (make_qkx1_quants returns (0, 0) for max == min)
    c = O.quantize(O.Q4_K, np.full((1, 256), 0.25, np.float32))
    assert not O.dequantize(O.Q4_K, c, 1, 256).any()


def test_q8_k_tie_kat():
    """BlockQ8K::from_float rounds with f32::round (half away from zero): with
    max = -128, iscale = -128/max = 1 and d = 1, so x.5 values are exact ties.
    +-2.5 -> +-3 and +-0.5 -> +-1 (half to even would give +-2 and 0); 126.5 ->
    127; 128 (same |x| as the max, later) is not the max and clamps to 127."""
    x = np.zeros(256, np.float32)
    x[0] = -128.0
    x[1:8] = [2.5, -2.5, 0.5, -0.5, 126.5, -127.5, 128.0]
    blk = O.quantize_q8_k(x)
    assert blk[0:4].view(np.float32)[0] == 1.0
    assert list(blk[4:12].view(np.int8)) == [-128, 3, -3, 1, -1, 127, -128, 127]


@pytest.mark.parametrize("case", range(len(GOLDEN["q8k"])))
def test_q8_k_quantize_golden(case):
    c = GOLDEN["q8k"][case]
    assert O.quantize_q8_k(_h2f(c["x"])).tobytes().hex() == c["block"]


# ---------------------------------------------------------------- dots
def test_vec_dot_q8_0_exact_integer_brute_force():
    rng = np.random.default_rng(5)
    k = 512
    w = O.quantize(O.Q8_0, O.randn(1, 1, 0.02, (1, k)))[0]
    xq = O.quantize_q8_0_row(O.randn(1, 2, 1.0, (k,)))
    got = O.lib().o_vec_dot_q8_0_q8_0(k, w.ctypes.data, xq.ctypes.data)
    want = 0.0
    for b in range(k // 32):
        wq = w[34 * b + 2: 34 * b + 34].view(np.int8).astype(np.int64)
        xqq = xq[34 * b + 2: 34 * b + 34].view(np.int8).astype(np.int64)
        dw = float(w[34 * b: 34 * b + 2].view(np.float16)[0])
        dx = float(xq[34 * b: 34 * b + 2].view(np.float16)[0])
        want += int((wq * xqq).sum()) * dw * dx
    assert abs(got - want) <= 1e-5 * abs(want) + 1e-6
    del rng


def test_vec_dot_q4_k_equals_dequantized_dot():
    # Q4_K . Q8_K == dequant(W) . dequant(Q8_K(x)) exactly in real arithmetic
    k = 1024
    w = O.quantize(O.Q4_K, O.randn(2, 1, 0.02, (1, k)))[0]
    x = O.randn(2, 2, 1.0, (k,))
    xq = O.quantize_q8_k(x)
    got = O.lib().o_vec_dot_q4_k_q8_k(k, w.ctypes.data, xq.ctypes.data)
    wd = O.dequantize(O.Q4_K, w, 1, k)[0].astype(np.float64)
    xd = np.concatenate([
        xq[292 * b + 4: 292 * b + 260].view(np.int8).astype(np.float64) * float(xq[292 * b: 292 * b + 4].view(np.float32)[0])
        for b in range(k // 256)])
    want = float(wd @ xd)
    assert abs(got - want) <= 2e-5 * (np.abs(wd) @ np.abs(xd))


# ---------------------------------------------------------------- matmul
@pytest.mark.parametrize("qtype,k", [(O.Q8_0, 64), (O.Q4_K, 512)])
def test_matmul_dequant_mode_brute_force(qtype, k):
    n, m = 24, 3
    w = O.quantize(qtype, O.randn(3, 1, 0.02, (n, k)))
    x = O.randn(3, 2, 1.0, (m, k))
    y = O.matmul(qtype, w, n, k, x, O.MODE_DEQUANT_F32)
    wd = O.dequantize(qtype, w, n, k).astype(np.float64)
    for i in range(m):
        for j in range(n):
            s = math.fsum(float(a) * float(b) for a, b in zip(x[i], wd[j]))
            assert y[i, j] == np.float32(s)


@pytest.mark.parametrize("qtype,k", [(O.Q8_0, 1024), (O.Q4_K, 1024)])
def test_matmul_q8act_close_to_dequant(qtype, k):
    n, m = 96, 2
    w = O.quantize(qtype, O.randn(4, 1, 0.02, (n, k)))
    x = O.randn(4, 2, 1.0, (m, k))
    yd = O.matmul(qtype, w, n, k, x, O.MODE_DEQUANT_F32)
    yq = O.matmul(qtype, w, n, k, x, O.MODE_Q8ACT)
    for i in range(m):
        nrm = np.linalg.norm(yd[i])
        err = np.abs(yq[i] - yd[i]).max() / nrm
        assert 1e-6 < err < 5e-3, err  # the activation rounding: not zero, not large


@pytest.mark.parametrize("qtype,k", [(O.Q8_0, 1024), (O.Q4_K, 2048)])
def test_baseline_avx2_matches_scalar_q8act(qtype, k):
    n, m = 200, 3
    w = O.quantize(qtype, O.randn(5, 1, 0.02, (n, k)))
    x = O.randn(5, 2, 1.0, (m, k))
    ys = O.matmul(qtype, w, n, k, x, O.MODE_Q8ACT)
    yb = O.baseline_matmul(qtype, w, n, k, x)
    for i in range(m):
        assert np.abs(yb[i] - ys[i]).max() <= 1e-5 * np.linalg.norm(ys[i])


# ---------------------------------------------------------------- epilogue + argmax
def test_gate_up_silu_closed_form():
    rng = np.random.default_rng(6)
    h = 4096
    y = (rng.standard_normal((2, 2 * h)) * 3).astype(np.float32)
    y[0, :5] = [0.0, -100.0, 100.0, 1e-30, -0.0]
    y[0, h:h + 5] = [3.0, 2.0, 0.5, 1.0, 7.0]
    got = O.bf16_bits_to_f32(O.gate_up_silu(y))
    g = O.bf16_round(y[:, :h]).astype(np.float64)
    u = O.bf16_round(y[:, h:]).astype(np.float64)
    want = O.bf16_round((g / (1.0 + np.exp(-g)) * u).astype(np.float32))
    assert got[0, 0] == 0.0 and got[0, 1] == 0.0 and got[0, 2] == 50.0
    # f32 silu vs f64 silu: equal except on a bf16 rounding boundary (<= 1 ulp)
    diff = np.abs(got - want)
    ulp = np.abs(want) * 2.0 ** -7 + 1e-38
    assert np.all(diff <= ulp)
    assert (diff == 0).mean() > 0.995


def test_argmax_reference_tie_vectors():
    # engine/src/engine.rs:3086-3128 n2_greedy_tie_rule_matches_argmax
    V = 248_320
    bf = lambda v: O.bf16_round(np.array([v], np.float32))[0]
    data = np.full(3 * V, bf(-2.5), np.float32)
    data[1_000] = bf(21.0)
    data[200_000] = bf(21.0)
    data[V + 5] = bf(21.03)
    data[V + 7] = bf(20.97)
    data[2 * V + 42] = bf(30.5)
    data[2 * V + 4_242] = bf(30.5)
    data[2 * V + 248_000] = bf(30.5)
    assert data[V + 5] == data[V + 7]
    assert list(O.argmax_rows(data.reshape(3, V))) == [1000, 5, 42]
    assert O.argmax_rows(np.array([np.nan, 1.0, 1.0], np.float32))[0] == 1
    assert O.argmax_rows(np.full(4, -np.inf, np.float32))[0] == 0
    assert O.lib().o_argmax(None, 0) == 0


# ------------------------------------------------------------------ Q6_K
def _q6k_numpy(blocks: np.ndarray, k: int) -> np.ndarray:
    """Independent vectorized Q6_K decode: per 128-half, the four 32-element
    quarters take (ql low, qh bits 0-1), (ql+32 low, qh bits 2-3), (ql high,
    qh bits 4-5), (ql+32 high, qh bits 6-7); scales in groups of 16."""
    nb = k // 256
    b = blocks.reshape(-1, nb, 210)
    ql = b[..., :128].reshape(-1, nb, 2, 64).astype(np.int32)
    qh = b[..., 128:192].reshape(-1, nb, 2, 32).astype(np.int32)
    sc = b[..., 192:208].view(np.int8).reshape(-1, nb, 2, 8).astype(np.float32)
    d = b[..., 208:210].copy().view(np.float16).astype(np.float32)[..., 0]
    quarters = [
        (ql[..., :32] & 0xF) | ((qh & 3) << 4),
        (ql[..., 32:] & 0xF) | (((qh >> 2) & 3) << 4),
        (ql[..., :32] >> 4) | (((qh >> 4) & 3) << 4),
        (ql[..., 32:] >> 4) | (((qh >> 6) & 3) << 4),
    ]
    q = np.stack(quarters, axis=-2) - 32                       # [.., nb, 2, 4, 32]
    s = sc.reshape(*sc.shape[:-1], 4, 2).repeat(16, axis=-1)    # [.., nb, 2, 4, 32]
    y = (d[..., None, None, None] * s) * q.astype(np.float32)   # (d * sc) * q in f32
    return y.reshape(-1, k).astype(np.float32)


def test_q6k_literal_bytes():
    """Byte-level known answers: d = 1, scales 1..16; one code per quarter."""
    blk = np.zeros(210, np.uint8)
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    blk[:128] = 0x00
    blk[128:192] = 0x00
    # element 0: ql[0] low = 0xF, qh[0] bits 0-1 = 3 -> code 63 -> (63 - 32) * sc[0] = 31
    blk[0] = 0x0F
    blk[128 + 0] = 0x03
    # element 64 + 17: ql[17] high nibble = 8, qh[17] bits 4-5 = 2 -> code 40 -> 8 * sc[5] = 48
    blk[17] = 0x80
    blk[128 + 17] = 0x20
    # element 32 + 20: ql[52] low nibble = 1, qh[20] bits 2-3 = 0 -> code 1 -> -31 * sc[3] = -124
    blk[52] = 0x01
    # element 128 + 96 + 31 (second half): ql[64 + 63] high = 2, qh[32 + 31] bits 6-7 = 1 -> code 18
    #   -> -14 * sc[8 + 7] = -14 * 16 = -224
    blk[64 + 63] = 0x20
    blk[128 + 32 + 31] = 0x40
    y = O.dequantize(O.Q6_K, blk.reshape(1, -1), 1, 256)[0]
    assert y[0] == 31.0
    assert y[64 + 17] == 48.0
    assert y[32 + 20] == -124.0
    assert y[128 + 96 + 31] == -224.0
    # every other element has code 0 -> -32 * its group scale
    assert y[1] == -32.0 and y[16] == -64.0 and y[128] == -32.0 * 9


def test_q6k_every_code_and_random_bytes():
    rng = np.random.default_rng(14)
    n, k = 16, 1024
    raw = rng.integers(0, 256, (n, k // 256, 210), dtype=np.uint8)
    d = (rng.standard_normal((n, k // 256)) * 0.01).astype(np.float16)
    raw[:, :, 208:210] = d.view(np.uint8).reshape(n, k // 256, 2)
    # first block: ql / qh so that element e of quarter 0 has code e (0..31) and
    # quarter 1 has code 32 + e: together with the random rest every code appears
    raw[0, 0, :32] = np.arange(32) & 0xF
    raw[0, 0, 128:160] = (np.arange(32) >> 4) | (((32 + np.arange(32)) >> 4) << 2)
    raw[0, 0, 32:64] = (32 + np.arange(32)) & 0xF
    raw = raw.reshape(n, -1)
    got = O.dequantize(O.Q6_K, raw, n, k)
    want = _q6k_numpy(raw, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    dd = float(d[0, 0])
    sc0 = raw[0, 192].astype(np.int8)
    assert got[0, 5] == np.float32(np.float32(dd) * np.float32(sc0)) * np.float32(5 - 32)


def test_q6k_matmul_dequant_mode_brute_force():
    rng = np.random.default_rng(3)
    n, k = 5, 512
    raw = rng.integers(0, 256, (n, k // 256, 210), dtype=np.uint8)
    raw[:, :, 208:210] = (rng.standard_normal((n, k // 256)) * 0.01).astype(np.float16).view(np.uint8).reshape(n, k // 256, 2)
    raw = raw.reshape(n, -1)
    x = O.randn(1, 2, 1.0, (3, k))
    y = O.matmul(O.Q6_K, raw, n, k, x)
    ref = x.astype(np.float64) @ _q6k_numpy(raw, k).astype(np.float64).T
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- top-k
def _ref_key(v: float) -> float:
    """engine/src/sample_kernel.rs:163-169: NaN ranks as -inf, -0.0 as +0.0."""
    return -math.inf if v != v else v + 0.0


def test_topk_kat():
    """Ties broken by the lower id, NaN placed with -inf (by id), -0.0 tied
    with +0.0, keys reported; slots past n are (-inf, 0xFFFFFFFF)."""
    v = np.array([1.0, np.nan, 3.0, -0.0, 3.0, 0.0, -np.inf], np.float32)
    vals, idx = O.topk_rows(v, 9)
    assert list(idx[0]) == [2, 4, 0, 3, 5, 1, 6, 0xFFFFFFFF, 0xFFFFFFFF]
    assert list(vals[0][:5]) == [3.0, 3.0, 1.0, 0.0, 0.0]
    assert not np.signbit(vals[0][3])  # -0.0 reported as its key +0.0
    assert np.all(np.isneginf(vals[0][5:]))


@pytest.mark.parametrize("seed", range(4))
def test_topk_matches_python_sort(seed):
    """Against Python's sort with the reference's comparator
    (sorted_row_dist, engine/src/sample_kernel.rs:326-337), on rows with many
    exact ties (small integers), NaN, +-inf and signed zeros."""
    rng = np.random.default_rng(seed)
    n = 3000
    v = rng.integers(-20, 21, (6, n)).astype(np.float32) * 0.5
    v[0, rng.integers(0, n, 40)] = np.nan
    v[1, rng.integers(0, n, 40)] = -0.0
    v[2, rng.integers(0, n, 10)] = np.inf
    v[3, :] = np.nan
    v[4, :] = 7.0
    for k in (1, 5, 64):
        vals, idx = O.topk_rows(v, k)
        for r in range(v.shape[0]):
            order = sorted(range(n), key=lambda i: (-_ref_key(float(v[r, i])), i))[:k]
            assert list(idx[r]) == order
            assert np.array_equal(vals[r], np.array([_ref_key(float(v[r, i])) for i in order], np.float32))
