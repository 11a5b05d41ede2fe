"""Shared helpers for the GPU parity tests."""
from __future__ import annotations

import numpy as np

import oracle as O


def rel_row_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max over rows of max_n |y - ref| / ||ref[m, :]||_2 (the path's tolerance metric)."""
    y = np.asarray(y, np.float64).reshape(-1, ref.shape[-1])
    ref = np.asarray(ref, np.float64).reshape(-1, ref.shape[-1])
    nrm = np.linalg.norm(ref, axis=1)
    nrm[nrm == 0] = 1.0
    return float((np.abs(y - ref).max(axis=1) / nrm).max())


def assert_close_elem(tag: str, got: np.ndarray, want: np.ndarray, rel: float, floor: str = "max"):
    """Per-element bound in the style of the reference's qmvt assert_close
    (engine/src/qwen35.rs:6946-6958): |got - want| <= rel * max(|want|, f), with
    f = 0.02 max|want| (floor="max", exact weights) or f = rms of the row
    (floor="rms", for tiles that round dequantized weights to bf16: their error
    is ~1.1e-3 rms(y) per element independent of |y|, so 2^-7 rms is ~7 sigma)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    mag = np.abs(want).max()
    assert mag > 0, f"{tag}: degenerate reference"
    if floor == "rms":
        w2 = want.reshape(-1, want.shape[-1])
        f = np.sqrt((w2 ** 2).mean(axis=1, keepdims=True)).reshape(want.shape[:-1] + (1,))
    else:
        f = 0.02 * mag
    tol = rel * np.maximum(np.abs(want), f)
    bad = np.abs(got - want) > tol
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{tag}: {bad.sum()} elements out of tolerance; first {tuple(i)}: "
                             f"got {got[tuple(i)]} want {want[tuple(i)]}")


_cache: dict = {}


def weight_bytes(qtype: int, n: int, k: int, seed: int = 0, sigma: float = 0.02) -> np.ndarray:
    """GGUF bytes of W ~ N(0, sigma) [n, k] from the oracle generator (stream 1)."""
    key = (qtype, n, k, seed, sigma)
    if key not in _cache:
        w = O.randn(seed, 1000 + n + 7 * k, sigma, (n, k))
        _cache[key] = O.quantize(qtype, w)
    return _cache[key]


def assert_close_dot(tag: str, got: np.ndarray, want: np.ndarray, x: np.ndarray, w: np.ndarray, rel: float,
                     out_rel: float = 0.0):
    """|got - want| <= rel * sqrt(sum_i (x[m, i] * w[n, i])^2) per element: the
    scale of the error that rounding each weight to bf16 (unit roundoff 2^-8)
    leaves in one dot product, whatever the norm of its weight row.  Its
    ratio to that scale has sd ~1e-3 and a heavy tail: over 36864 outputs of
    4096 x 12288 the largest is 8.3e-3 (Q6_K test weights) and 7.0e-3 (Q4_K),
    measured with the f64 product of bf16-rounded weights, so rel = 2^-6
    leaves a margin of ~2; out_rel * |want| is added for bf16 outputs."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.sqrt(np.square(np.asarray(x, np.float64)) @ np.square(np.asarray(w, np.float64)).T)
    bad = np.abs(got - want) > rel * scale + out_rel * np.abs(want) + 1e-30
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{tag}: {bad.sum()} elements out of tolerance; first {i}: got {got[i]} "
                             f"want {want[i]} scale {scale[i]}")
    return float((np.abs(got - want) / np.maximum(scale, 1e-30)).max())


def q6k_bytes(n: int, k: int, seed: int = 0, dscale: float = 2e-4) -> np.ndarray:
    """Random Q6_K GGUF bytes [n, k/256 * 210]: every ql / qh / scale byte
    uniform (all 6-bit codes, scales -128..127), d = f16 of N(0, dscale)
    (both signs, a few f16 subnormals near zero).  There is no Q6_K quantizer
    in the library or the oracle: GGUF files bring Q6_K tensors ready-made."""
    key = ("q6k", n, k, seed, dscale)
    if key not in _cache:
        rng = np.random.default_rng(seed + 977 * n + k)
        raw = rng.integers(0, 256, (n, k // 256, 210), dtype=np.uint8)
        d = (rng.standard_normal((n, k // 256)) * dscale).astype(np.float16)
        raw[:, :, 208:210] = d.view(np.uint8).reshape(n, k // 256, 2)
        _cache[key] = raw.reshape(n, -1)
    return _cache[key]


def activations(m: int, k: int, seed: int = 0) -> np.ndarray:
    """X ~ N(0, 1) [m, k] f32 from the oracle generator (stream 2)."""
    return O.randn(seed, 2_000_000 + 13 * m + k, 1.0, (m, k))


# ------------------------------------------------------------------ MLX affine inputs
# The reference's affine kernel tests (engine/src/qwen35.rs:6893-6930,
# qmvt_tests) draw weights and activations from one 64-bit LCG; rand_qlin /
# rand_x below produce the same values from the same seeds.
_A, _C, _MASK = 6364136223846793005, 1442695040888963407, (1 << 64) - 1


def lcg_values(seed: int, count: int) -> np.ndarray:
    """`count` successive outputs (state >> 33) of the reference's lcg()."""
    out = np.empty(count, dtype=np.uint64)
    s = seed
    for i in range(count):
        s = (s * _A + _C) & _MASK
        out[i] = s >> 33
    return out


def rand_qlin(out: int, inp: int, seed: int):
    """rand_qlin (qwen35.rs:6900-6918): words (lcg ^ lcg << 16) [out, inp/8],
    then per (row, group of 64) a scale 0.002 + (lcg % 1000) * 2e-5 and a bias
    ((lcg % 2001) - 1000) * 1e-4 in f32, stored as bf16.  Returns (wq u32
    [out, inp/8], sb bf16 bits [out, 2*ng])."""
    ng = inp // 64
    nw = out * inp // 8
    v = lcg_values(seed, 2 * nw + 2 * out * ng)
    lo, hi = v[0:2 * nw:2], v[1:2 * nw:2]
    wq = ((lo.astype(np.uint32)) ^ ((hi.astype(np.uint64) << np.uint64(16)) & np.uint64(0xFFFFFFFF)).astype(np.uint32))
    rest = v[2 * nw:].reshape(out, ng, 2)
    sc = np.float32(0.002) + (rest[:, :, 0] % 1000).astype(np.float32) * np.float32(2e-5)
    bi = ((rest[:, :, 1] % 2001).astype(np.float32) - np.float32(1000.0)) * np.float32(1e-4)
    sb = np.concatenate([O.f32_to_bf16_bits(sc.astype(np.float32)), O.f32_to_bf16_bits(bi.astype(np.float32))],
                        axis=1)
    return wq.reshape(out, inp // 8), np.ascontiguousarray(sb, dtype=np.uint16)


def rand_x(inp: int, seed: int, rows: int = 1) -> np.ndarray:
    """rand_x (qwen35.rs:6920-6926): ((lcg % 4001) - 2000) / 1000 in f32,
    rounded to bf16; returned as f32 values [rows, inp]."""
    v = lcg_values(seed, rows * inp)
    x = ((v % 4001).astype(np.float32) - np.float32(2000.0)) / np.float32(1000.0)
    return O.bf16_round(x.astype(np.float32)).reshape(rows, inp)


def rand_qlin_fast(out: int, inp: int, seed: int, gs: int = 64):
    """Large shapes: the same distributions from numpy's generator."""
    rng = np.random.default_rng(seed)
    ng = inp // gs
    wq = rng.integers(0, 1 << 32, (out, inp // 8), dtype=np.uint64).astype(np.uint32)
    sc = np.float32(0.002) + rng.integers(0, 1000, (out, ng)).astype(np.float32) * np.float32(2e-5)
    bi = (rng.integers(0, 2001, (out, ng)).astype(np.float32) - np.float32(1000.0)) * np.float32(1e-4)
    sb = np.concatenate([O.f32_to_bf16_bits(sc.astype(np.float32)), O.f32_to_bf16_bits(bi.astype(np.float32))],
                        axis=1)
    return wq, np.ascontiguousarray(sb, dtype=np.uint16)


def ref_rng(state: list) -> float:
    """The reference tests' xorshift64 uniform (engine/src/sample_kernel.rs:1178-1183);
    state is a one-element list holding the u64 seed."""
    s = state[0]
    s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
    s ^= s >> 7
    s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
    state[0] = s
    return (s >> 11) / float(1 << 53)


def lm_row(n: int, state: list, spice: bool) -> np.ndarray:
    """LM-like logits row of the reference's sampler tests (lm_row,
    engine/src/sample_kernel.rs:1300-1321): bf16-rounded N(0, 2.5) bulk (exact
    ties), a few peaked tokens, and with `spice` a NaN, a -inf, a -0.0 and a
    +0.0 at fixed positions.  half's f64 -> bf16 rounding is the oracle's."""
    import math
    out = np.empty(n, np.float32)
    bf = lambda v: float(O.bf16_bits_to_f32(np.array([O.bf16_from_f64_half(v)], np.uint16))[0])
    for i in range(n):
        a, b = max(ref_rng(state), 1e-300), ref_rng(state)
        g = math.sqrt(-2.0 * math.log(a)) * math.cos(2.0 * math.pi * b)
        out[i] = bf(g * 2.5)
    top = int(ref_rng(state) * 4.0) + 1
    for t in range(top + 24):
        v = int(ref_rng(state) * n) % n
        x = 16.0 - t * (0.1 + ref_rng(state) * 0.7) + (3.0 if t < top else 0.0)
        out[v] = bf(x)
    if spice:
        out[n // 2] = np.nan
        out[n // 3] = -np.inf
        out[n // 5] = -0.0
        out[n // 7] = 0.0
    return out
