"""GPU parity of the streaming mid-M GEMM (k_gemm_mid, route GEMM_MID):
Q4_K / MLX affine weights on the row-quad plane, bf16 activations, rounded
weights.

Bars (per row, max_n |y - ref| / ||ref[m, :]||):
  - 1e-5 against the f64 product of the activations with the oracle's
    dequantized weights rounded to bf16 (the tile's weights: the kernel's
    rounding is the prefill GEMM's, bit for bit, so only f32 summation order
    remains);
  - 1e-2 against the oracle's exact product (bf16 activations);
  - every forced K-split count against the unsplit result, 1e-5;
  - gate/up: against silu(bf16(g)) * bf16(u) of the kernel's own plain
    products, 1e-5,
    and against the oracle's exact gate/up, 1e-2.
Shapes cover ragged outputs (not a multiple of the 128-row block), ragged
activation rows (not a multiple of 32, several 128-row groups), one 256-wide
chunk, and both group sizes (64 and 128 rows).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, rand_qlin_fast, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


@pytest.fixture(autouse=True)
def _mid(monkeypatch):
    monkeypatch.setenv("THQ_GEMM_MID", "1")
    for v in ("THQ_MID_SPLITS", "THQ_MID_MH", "THQ_MID_NT", "THQ_MID_NW"):
        monkeypatch.delenv(v, raising=False)


def bf16_x(m, k, seed=0):
    xf = O.bf16_round(activations(m, k, seed))
    return xf, torch.from_numpy(xf).to("cuda").to(torch.bfloat16)


def tonp(t):
    return t.float().cpu().numpy()


def rounded_ref(xf, wf):
    return xf.astype(np.float64) @ O.bf16_round(wf).astype(np.float64).T


@pytest.mark.parametrize("n,k,m", [(1000, 1024, 100), (512, 4096, 128), (384, 512, 300), (256, 256, 17),
                                   (700, 2048, 64), (128, 1024, 33), (4096, 512, 512)])
def test_mid_q4k(n, k, m):
    print(f"[mid] q4_k n={n} k={k} m={m}", flush=True)
    b = weight_bytes(O.Q4_K, n, k, 7)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    xf, xb = bf16_x(m, k, seed=8)
    y = tonp(thq.matmul(w, xb, torch.float32))
    wf = O.dequantize(O.Q4_K, b, n, k)
    assert rel_row_err(y, rounded_ref(xf, wf)) <= 1e-5
    assert rel_row_err(y, O.matmul(O.Q4_K, b, n, k, xf, O.MODE_DEQUANT_F32)) <= 1e-2
    yb = tonp(thq.matmul(w, xb, torch.bfloat16))
    assert rel_row_err(yb, y) <= 2.0 ** -8


@pytest.mark.parametrize("mh,nt,nw", [(2, 1, 4), (2, 2, 4), (4, 1, 4), (4, 2, 4), (2, 1, 8), (4, 1, 8)])
def test_mid_instances(mh, nt, nw, monkeypatch):
    """Every instance (group size, column tiles per wave, waves per block),
    plain and gate/up, ragged outputs (not a multiple of the block's rows)
    and rows (two groups)."""
    print(f"[mid inst] mh={mh} nt={nt} nw={nw}", flush=True)
    monkeypatch.setenv("THQ_MID_MH", str(mh))
    monkeypatch.setenv("THQ_MID_NT", str(nt))
    monkeypatch.setenv("THQ_MID_NW", str(nw))
    n, k, m = 700, 1024, 32 * mh + 9
    b = weight_bytes(O.Q4_K, n, k, 15)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    xf, xb = bf16_x(m, k, seed=16)
    y = tonp(thq.matmul(w, xb, torch.float32))
    assert rel_row_err(y, rounded_ref(xf, O.dequantize(O.Q4_K, b, n, k))) <= 1e-5
    nout = 300
    b2 = weight_bytes(O.Q4_K, 2 * nout, k, 17)
    w2 = thq.QTensor.from_gguf_bytes(O.Q4_K, b2, 2 * nout, k)
    p = tonp(thq.matmul(w2, xb, torch.float32))
    gu = tonp(thq.gate_up_silu(w2, xb, torch.float32))
    g = O.bf16_round(p[:, :nout]).astype(np.float64)
    u = O.bf16_round(p[:, nout:]).astype(np.float64)
    assert rel_row_err(gu, g / (1.0 + np.exp(-g)) * u) <= 1e-5


@pytest.mark.parametrize("m", [96, 200])
def test_mid_split_counts(m, monkeypatch):
    n, k = 640, 4096
    b = weight_bytes(O.Q4_K, n, k, 9)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    xf, xb = bf16_x(m, k, seed=10)
    monkeypatch.setenv("THQ_MID_SPLITS", "1")
    y1 = tonp(thq.matmul(w, xb, torch.float32))
    assert rel_row_err(y1, rounded_ref(xf, O.dequantize(O.Q4_K, b, n, k))) <= 1e-5
    for splits in (2, 3, 7, 16):
        print(f"[mid split] m={m} splits={splits}", flush=True)
        monkeypatch.setenv("THQ_MID_SPLITS", str(splits))
        ys = tonp(thq.matmul(w, xb, torch.float32))
        assert rel_row_err(ys, y1) <= 1e-5, splits


@pytest.mark.parametrize("nout,k,m,splits", [(384, 2048, 130, "1"), (320, 1024, 64, "3")])
def test_mid_gate_up(nout, k, m, splits, monkeypatch):
    print(f"[mid gu] nout={nout} k={k} m={m} splits={splits}", flush=True)
    monkeypatch.setenv("THQ_MID_SPLITS", splits)
    b = weight_bytes(O.Q4_K, 2 * nout, k, 11)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, 2 * nout, k)
    xf, xb = bf16_x(m, k, seed=12)
    gu = tonp(thq.gate_up_silu(w, xb, torch.float32))
    # the epilogue rounds gate and up to bf16 first (the reference's form)
    p = tonp(thq.matmul(w, xb, torch.float32))
    g = O.bf16_round(p[:, :nout]).astype(np.float64)
    u = O.bf16_round(p[:, nout:]).astype(np.float64)
    assert rel_row_err(gu, g / (1.0 + np.exp(-g)) * u) <= 1e-5
    logits = O.matmul(O.Q4_K, b, 2 * nout, k, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(gu, O.bf16_bits_to_f32(O.gate_up_silu(logits))) <= 1e-2


@pytest.mark.parametrize("n,k,m", [(520, 1024, 100), (256, 4096, 256)])
def test_mid_affine(n, k, m):
    print(f"[mid] affine n={n} k={k} m={m}", flush=True)
    wq, sb = rand_qlin_fast(n, k, 13)
    w = thq.QTensor.from_affine(wq, sb, n, k)
    xf, xb = bf16_x(m, k, seed=14)
    y = tonp(thq.matmul(w, xb, torch.float32))
    wf = O.affine_dequant_f32(wq, sb, n, k, 64)
    # the tile's f32 weight fma(s, 128 + q, -(128 s - b)) may sit an f32 ulp
    # from q s + b, which moves a bf16 rounding now and then: 1e-4
    assert rel_row_err(y, rounded_ref(xf, wf)) <= 1e-4
    exact = xf.astype(np.float64) @ wf.astype(np.float64).T
    assert rel_row_err(y, exact) <= 1e-2
