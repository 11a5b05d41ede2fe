"""GPU parity of the MLX affine 4-bit path (THQ_MLX_Q4, the engine's QLin).

The oracle is affine_oracle.c, pinned by tests/test_oracle_affine.py.
Weights and activations come from the reference's own affine test generator
(rand_qlin / rand_x, engine/src/qwen35.rs:6893-6930) for its shapes, and from
the same distributions via numpy for the large Qwen3-8B shapes.

Bars:
  - upload / download round trip of the QLin arrays, row-major and tiled;
  - dequantization bit-exact: bf16 against dequant_affine, f32 against one
    rounding of q*s + b;
  - matmul / gate-up / argmax against the oracle's f64 product:
      - 1e-2 of the row L2 norm (bf16 activations);
      - the reference's own per-element bound on bf16 outputs, 2^-7 *
        max(|want|, 0.02 max|want|) (qmvt_tests assert_close,
        qwen35.rs:6946-6958), applied to f32 outputs on the exact-weight
        paths with 2^-12;
      - on the prefill GEMM, which rounds dequantized weights to bf16,
        2^-6 of the row rms per element;
  - the reference's qmvt shapes, including K % 256 != 0, which runs the
    exact generic kernel here.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close_elem, rand_qlin, rand_qlin_fast, rand_x, rel_row_err

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def tonp(t):
    return t.float().cpu().numpy()


def xdev(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda().to(torch.bfloat16)


@pytest.mark.parametrize("n,k,gs", [(520, 448, 64), (300, 4096, 64), (33, 1024, 128)])
def test_affine_upload_roundtrip_and_dequant(n, k, gs):
    wq, sb64 = rand_qlin(n, k, 11 + n)
    sb = sb64 if gs == 64 else np.concatenate([sb64[:, 0:k // 64:2], sb64[:, k // 64::2]], axis=1)
    w = thq.QTensor.from_affine(wq, sb, n, k, gs=gs)
    assert w.dtype == thq.MLX_Q4 and w.shape == (n, k)
    wq2, sb2 = w.affine_data()
    assert np.array_equal(wq2, wq) and np.array_equal(sb2, sb)
    got16 = w.dequantize_bf16().view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got16, O.affine_dequant_bf16(wq, sb, n, k, gs))
    got32 = tonp(w.dequantize())
    assert np.array_equal(got32.view(np.uint32), O.affine_dequant_f32(wq, sb, n, k, gs).view(np.uint32))


def test_affine_dequant_bf16_every_bit_pattern():
    """Scales and biases of random 16-bit patterns (NaN, infinities, bf16
    subnormals, values near the overflow threshold, products that round to
    f32 subnormals or past the largest finite bf16): the bf16 dequantization
    equals the oracle's f64 -> bf16 bit for bit wherever the oracle's value is
    not a NaN, and is a NaN where it is (payloads follow the device's f64 NaN
    propagation)."""
    n, k = 64, 1024
    rng = np.random.default_rng(21)
    wq = rng.integers(0, 1 << 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
    sb = rng.integers(0, 1 << 16, (n, 2 * (k // 64)), dtype=np.uint64).astype(np.uint16)
    sb[:16] &= 0x81FF  # exponent fields 0..3: bf16 subnormal and tiny normal results
    w = thq.QTensor.from_affine(wq, sb, n, k)
    got = w.dequantize_bf16().view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.affine_dequant_bf16(wq, sb, n, k, 64)
    nan = lambda b: ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    assert np.array_equal(nan(got), nan(want))
    assert np.array_equal(got[~nan(want)], want[~nan(want)])
    # the draw reaches the rounding routine's slow cases
    exp = (want >> 7) & 0xFF
    assert (exp == 0).sum() > 100 and (exp == 0xFF).sum() > 100


def test_affine_tiled_upload_equals_row_major():
    n, k = 300, 384   # two 256-row tiles, the second ragged
    wq, sb = rand_qlin(n, k, 5)
    wt, st = O.affine_tile(wq, sb, n, k)
    a = thq.QTensor.from_affine(wq, sb, n, k)
    b = thq.QTensor.from_affine(wt, st, n, k, tiled=True)
    for x, y in zip(a.affine_data(), b.affine_data()):
        assert np.array_equal(x, y)
    # the device path too
    c = thq.QTensor.from_affine(torch.from_numpy(wt.view(np.int32)).cuda(), torch.from_numpy(st.view(np.int16)).cuda(),
                                n, k, tiled=True)
    assert np.array_equal(c.affine_data()[0], wq)


# the reference's qmvt shapes: (out, ng) ragged rows, ng < 8, uneven slices
QMVT = [(520, 7), (256, 80), (1000, 17), (72, 96)]


@pytest.mark.parametrize("out,ng", QMVT)
@pytest.mark.parametrize("m", [1, 3, 8])
def test_affine_matmul_reference_shapes(out, ng, m):
    inp = ng * 64
    wq, sb = rand_qlin(out, inp, 11 + out)
    x = rand_x(inp, 97 + out, rows=m)
    w = thq.QTensor.from_affine(wq, sb, out, inp)
    want = O.affine_matmul(wq, sb, out, inp, x)
    y = tonp(thq.matmul(w, xdev(x), torch.float32))
    assert rel_row_err(y, want) <= 1e-2
    assert_close_elem(f"affine {out}x{inp} m={m}", y, want, 2.0 ** -12)   # exact weights, f32 out
    yb = tonp(thq.matmul(w, xdev(x), torch.bfloat16))
    assert_close_elem(f"affine bf16 {out}x{inp} m={m}", yb, want, 2.0 ** -7)


@pytest.mark.parametrize("half,ng", [(256, 7), (264, 80), (512, 17), (1000, 6)])
@pytest.mark.parametrize("m", [1, 4])
def test_affine_gate_up_reference_shapes(half, ng, m):
    """qmvt_gate_up_matches_scalar's cases: the epilogue bf16(silu(g) * u)
    on the fused [gate; up] weight (up stream tile-aligned and not)."""
    inp = ng * 64
    wq, sb = rand_qlin(2 * half, inp, 211 + half)
    x = rand_x(inp, 307 + half, rows=m)
    w = thq.QTensor.from_affine(wq, sb, 2 * half, inp)
    got = tonp(thq.gate_up_silu(w, xdev(x), torch.bfloat16))
    gu = tonp(thq.matmul(w, xdev(x), torch.float32))
    want_own = O.bf16_bits_to_f32(O.gate_up_silu(gu))
    assert_close_elem(f"affine gate/up {half}x{inp} m={m} vs own matmul", got, want_own, 2.0 ** -7)
    want = O.bf16_bits_to_f32(O.gate_up_silu(O.affine_matmul(wq, sb, 2 * half, inp, x)))
    assert_close_elem(f"affine gate/up {half}x{inp} m={m}", got, want, 2.0 ** -7)


@pytest.mark.parametrize("m", [1, 2, 8, 64, 300])
@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_affine_qwen3_8b_shapes(n, k, m):
    """Decode GEMV (M = 1), MFMA decode GEMV (2..8), MFMA GEMM (> 8, weights
    rounded to bf16 on the tile: rms-floored per-element bound)."""
    wq, sb = rand_qlin_fast(n, k, seed=n + k)
    x = O.bf16_round(O.randn(4, 9 + m, 1.0, (m, k)))
    w = thq.QTensor.from_affine(wq, sb, n, k)
    y = tonp(thq.matmul(w, xdev(x), torch.float32))
    rows = slice(0, min(m, 16))
    want = O.affine_matmul(wq, sb, n, k, x[rows])
    assert rel_row_err(y[rows], want) <= 1e-2
    if m <= 8:
        assert_close_elem(f"affine {n}x{k} m={m}", y[rows], want, 2.0 ** -12)
    else:
        # the tile rounds each dequantized weight to bf16 (error ~2^-9 |w|); an
        # affine group's bias makes |w| large against the row's output rms, so
        # the per-element bound is 2^-6 rms here (2^-7 for zero-mean Q4_K)
        assert_close_elem(f"affine {n}x{k} m={m}", y[rows], want, 2.0 ** -6, floor="rms")
    if m > 16:  # the rest of the rows: a size-independent check against the f32 dequantized product
        wd = w.dequantize()
        ref = (torch.from_numpy(x).cuda() @ wd.T).cpu().numpy()
        assert rel_row_err(y, ref) <= 1e-2


def test_affine_fused_qkv_and_lm_head_argmax():
    n1, n2, k = 640, 384, 1024
    a, b = rand_qlin(n1, k, 1), rand_qlin(n2, k, 2)
    wa, wb = thq.QTensor.from_affine(*a, n1, k), thq.QTensor.from_affine(*b, n2, k)
    fused = thq.QTensor.fuse([wa, wb])
    wq2, sb2 = fused.affine_data()
    assert np.array_equal(wq2, np.concatenate([a[0], b[0]])) and np.array_equal(sb2, np.concatenate([a[1], b[1]]))
    x = rand_x(k, 5, rows=5)
    logits, idx = thq.matmul_argmax(fused, xdev(x))
    want = O.affine_matmul(wq2, sb2, n1 + n2, k, x)
    assert rel_row_err(tonp(logits), want) <= 1e-4
    assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_rows(tonp(logits)))


def test_affine_errors():
    wq, sb = rand_qlin(8, 256, 1)
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.from_affine(wq, sb[:, :8], 8, 256, gs=32)
    assert e.value.code == thq.EDTYPE
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.from_affine(wq, sb, 8, 256, gs=128, tiled=True)
    assert e.value.code == thq.EDTYPE
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.from_affine(wq[:, :5], sb, 8, 40)
    assert e.value.code == thq.ESHAPE
    w = thq.QTensor.from_affine(wq, sb, 8, 256)
    with pytest.raises(thq.ThqError) as e:
        thq.matmul(w, xdev(rand_x(256, 1)), flags=thq.MODE_Q8ACT)
    assert e.value.code == thq.EDTYPE
    with pytest.raises(thq.ThqError) as e:
        w.data()
    assert e.value.code == thq.EDTYPE
    with pytest.raises(ValueError):
        thq.matmul(w, xdev(rand_x(192, 1)))
