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


def activations(m: int, k: int, seed: int = 0) -> np.ndarray:
    """X ~ N(0, 1) [m, k] f32 from the oracle generator (stream 2)."""
    return O.randn(seed, 2_000_000 + 13 * m + k, 1.0, (m, k))
