"""The fused greedy-argmax epilogue of the decode kernels (thq_matmul_argmax
with no logits buffer and THQ_MODE_ARGMAX_FUSED), against the logits path and the tie rule of
engine/src/engine.rs:1891-1898: a strict '>' scan, so the lowest index among
equal maxima wins, NaN is never selected, and an all-NaN / -inf row gives 0.

  - Random weights, every weight type and M = 1..8: the fused index equals
    the argmax of the logits the same call returns when asked for them.  The
    kernels sum each output exactly as the stored path does, so the two
    agree bit for bit.
  - Exact ties: integer weights and integer bf16 activations make every dot
    product exact in f32 (|sum| < 2^24) whatever the summation order.  Copies
    of the maximal row placed in different output tiles must give the
    lowest of their indices.  Rows with a NaN scale give NaN and are never
    chosen.  A head of NaN rows only gives index 0.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, q6k_bytes, rand_qlin_fast, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def xdev(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda().to(torch.bfloat16)


def both(w, x):
    """(fused idx, idx and logits of the logits path)"""
    _, fused = thq.matmul_argmax(w, x, want_logits=False, flags=thq.MODE_ARGMAX_FUSED)
    logits, idx = thq.matmul_argmax(w, x)
    return fused.cpu().numpy(), idx.cpu().numpy(), logits.cpu().numpy()


def make_weight(kind, n, k, seed):
    if kind == "q8_0":
        return thq.QTensor.from_gguf_bytes(thq.Q8_0, weight_bytes(O.Q8_0, n, k, seed=seed), n, k)
    if kind == "q4_k":
        return thq.QTensor.from_gguf_bytes(thq.Q4_K, weight_bytes(O.Q4_K, n, k, seed=seed), n, k)
    if kind == "q6_k":
        return thq.QTensor.from_gguf_bytes(thq.Q6_K, q6k_bytes(n, k, seed=seed), n, k)
    wq, sb = rand_qlin_fast(n, k, seed=seed)
    return thq.QTensor.from_affine(wq, sb, n, k)


@pytest.mark.parametrize("kind", ["q8_0", "q4_k", "q6_k", "affine"])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
def test_fused_equals_logits_path(kind, m):
    n, k = 20011, 4096  # ragged last tile for every tile size
    w = make_weight(kind, n, k, seed=31)
    x = xdev(O.bf16_round(activations(m, k, seed=32)))
    fused, idx, logits = both(w, x)
    assert np.array_equal(fused, idx)
    assert np.array_equal(idx.astype(np.uint32), O.argmax_rows(logits))


def q8_int_rows(n, k, rng):
    """Q8_0 bytes with d = 1 and q in [-2, 2]: integer weights."""
    blk = np.zeros((n, k // 32, 34), np.uint8)
    blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[:, :, 2:] = rng.integers(-2, 3, (n, k // 32, 32)).astype(np.int8).view(np.uint8)
    return blk


def q6_encode(codes):
    """GGUF Q6_K bytes of 6-bit codes [n, k] with d = 1 and every scale 1
    (w = code - 32), in GGML's layout: for half h and l < 32, ql[64h + l]
    holds codes 128h + l (low nibble) and 128h + 64 + l (high), ql[64h + 32 + l]
    codes 128h + 32 + l and 128h + 96 + l, qh[32h + l] the four top-bit pairs."""
    n, k = codes.shape
    c = codes.reshape(n, k // 256, 2, 4, 32).astype(np.uint8)  # [row, sb, h, quarter, l]
    raw = np.zeros((n, k // 256, 210), np.uint8)
    for h in range(2):
        q1, q2, q3, q4 = c[:, :, h, 0], c[:, :, h, 1], c[:, :, h, 2], c[:, :, h, 3]
        raw[:, :, 64 * h:64 * h + 32] = (q1 & 15) | ((q3 & 15) << 4)
        raw[:, :, 64 * h + 32:64 * h + 64] = (q2 & 15) | ((q4 & 15) << 4)
        raw[:, :, 128 + 32 * h:160 + 32 * h] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    raw[:, :, 192:208] = 1
    raw[:, :, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    return raw


@pytest.mark.parametrize("kind", ["q8_0", "q6_k"])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_exact_ties_and_nan(kind, m):
    n, k = 4500, 4096
    rng = np.random.default_rng(7 + m)
    x = rng.integers(-3, 4, (m, k)).astype(np.float32)  # exact in bf16
    x[:, 0] = 3.0
    if kind == "q8_0":
        blk = q8_int_rows(n, k, rng)
        best = np.clip(2 * np.sign(x[0]), -2, 2).astype(np.int8).view(np.uint8).reshape(k // 32, 32)
        for r in (70, 5, 2000, 4499):
            blk[r, :, 2:] = best
        blk[3, :, 0:2] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)  # a NaN row ahead of the maxima
        raw, qt = blk.reshape(n, -1), thq.Q8_0
    else:
        codes = rng.integers(0, 64, (n, k))
        # w = 31 where x[0] > 0, -32 where x[0] < 0, 0 where it is 0: the
        # largest output any row can give for x[0]
        codes[[70, 5, 2000, 4499]] = np.where(x[0] > 0, 63, np.where(x[0] < 0, 0, 32))
        raw6 = q6_encode(codes)
        assert np.array_equal(O.dequantize(O.Q6_K, raw6.reshape(n, -1)[:8], 8, k), (codes[:8] - 32).astype(np.float32))
        raw6[3, :, 208:210] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
        raw, qt = raw6.reshape(n, -1), thq.Q6_K
    w = thq.QTensor.from_gguf_bytes(qt, raw, n, k)
    fused, idx, logits = both(w, xdev(x))
    assert np.array_equal(fused, idx)
    assert np.isnan(logits[:, 3]).all()
    # where row 0 of x makes the copies maximal, the lowest copy index wins
    want = O.argmax_rows(logits)
    assert np.array_equal(idx.astype(np.uint32), want)
    assert fused[0] == 5 and logits[0, 5] == logits[0, 70] == logits[0, 2000] == logits[0, 4499]
    # all-NaN head: index 0 for every row
    bs = 34 if kind == "q8_0" else 210
    dpos = slice(0, 2) if kind == "q8_0" else slice(208, 210)
    nanraw = raw.copy().reshape(n, -1, bs)
    nanraw[:, :, dpos] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
    wn = thq.QTensor.from_gguf_bytes(qt, nanraw.reshape(n, -1), n, k)
    fused_n, idx_n, _ = both(wn, xdev(x))
    assert not fused_n.any() and not idx_n.any()


def test_fallback_shapes_still_correct():
    """Paths without the fused epilogue (f32 x, K > 4096 Q4_K at M = 1, M > 8)
    keep the logits in the workspace and give the same indices."""
    for kind, n, k, m, dt in [("q4_k", 3000, 8192, 1, torch.bfloat16), ("q8_0", 3000, 4096, 2, torch.float32),
                              ("q8_0", 3000, 4096, 12, torch.bfloat16)]:
        w = make_weight(kind, n, k, seed=41)
        x = torch.from_numpy(O.bf16_round(activations(m, k, seed=42))).cuda().to(dt)
        _, fused = thq.matmul_argmax(w, x, want_logits=False, flags=thq.MODE_ARGMAX_FUSED)
        logits, idx = thq.matmul_argmax(w, x)
        _, plain = thq.matmul_argmax(w, x, want_logits=False)
        assert torch.equal(plain, idx)
        assert torch.equal(fused, idx)
        assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_rows(logits.cpu().numpy()))
