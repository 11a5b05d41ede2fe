"""Dequantize-then-GEMM prefill route (k_gemm_b16.hip): at >= 1024 rows,
where its 256 x 384 tiles fill every CU, a plain projection dequantizes its
weight to bf16 once (the workspace) and runs the bf16 GEMM, as the
reference router's "dequant + bf16 matmul" prefill route.  THQ_GEMM_DQ=1
makes every supported shape take it, so these tests reach it on small,
ragged shapes too.  The weights it multiplies are the oracle's dequantized
weights rounded to bf16, so the product is pinned at the f32 accumulation
bar to the f64 product with those weights, and meets the 1e-2 row bar
against the exact oracle; ragged M and N tiles; Q4_K, Q8_0, Q6_K, MLX
affine; and it agrees with the tile-dequantizing GEMM that
thq_matmul_noalloc keeps (its scratch cannot hold the bf16 weight).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, q6k_bytes, rand_qlin_fast, rel_row_err, weight_bytes

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
def _route(monkeypatch):
    monkeypatch.setenv("THQ_GEMM_DQ", "1")


def xrows(m, k, seed):
    xf = O.bf16_round(activations(m, k, seed=seed))
    return xf, torch.from_numpy(xf).cuda().to(torch.bfloat16)


@pytest.mark.parametrize("m,n,k", [(1024, 1000, 2048), (1100, 800, 1024), (2048, 4096, 4096)])
def test_dq_q4k_rounded_product(m, n, k):
    b = weight_bytes(O.Q4_K, n, k, seed=1500 + n)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    xf, xb = xrows(m, k, seed=1510 + m)
    print(f"[dq] q4_k m={m} {n}x{k}", flush=True)
    y = thq.matmul(w, xb, torch.float32)
    y16 = thq.matmul(w, xb, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(y16, y.to(torch.bfloat16))
    rng = np.random.default_rng(m)
    pick = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 14)]))
    got = y.cpu().numpy()[pick]
    wr = O.bf16_round(O.dequantize(O.Q4_K, b, n, k)).astype(np.float64)
    rounded = xf[pick].astype(np.float64) @ wr.T
    assert rel_row_err(got, rounded) <= 1e-5
    ref = O.matmul(O.Q4_K, b, n, k, xf[pick], O.MODE_DEQUANT_F32)
    assert rel_row_err(got, ref) <= 1e-2


@pytest.mark.parametrize("kind", ["q8_0", "q6_k", "affine"])
def test_dq_other_types(kind):
    m, n, k = 1024, 700, 2048
    if kind == "affine":
        wq, sb = rand_qlin_fast(n, k, seed=1520)
        w = thq.QTensor.from_affine(wq, sb, n, k)
        ref_of = lambda xf: O.affine_matmul(wq, sb, n, k, xf)
    elif kind == "q6_k":
        b = q6k_bytes(n, k, seed=1521)
        w = thq.QTensor.from_gguf_bytes(O.Q6_K, b, n, k)
        ref_of = lambda xf: O.matmul(O.Q6_K, b, n, k, xf)
    else:
        b = weight_bytes(O.Q8_0, n, k, seed=1522)
        w = thq.QTensor.from_gguf_bytes(O.Q8_0, b, n, k)
        ref_of = lambda xf: O.matmul(O.Q8_0, b, n, k, xf)
    xf, xb = xrows(m, k, seed=1523)
    print(f"[dq] {kind} m={m} {n}x{k}", flush=True)
    y = thq.matmul(w, xb, torch.float32).cpu().numpy()
    pick = np.array([0, 1, 511, 1023])
    assert rel_row_err(y[pick], ref_of(xf[pick])) <= 1e-2


def test_dq_matches_tile_gemm(monkeypatch):
    # 12288 x 4096 at M = 2048 takes the route by the planner's own rule; the
    # bf16 weight (100 MB) exceeds the no-alloc scratch, so
    # thq_matmul_noalloc plans the tile-dequantizing GEMM for the same call
    monkeypatch.delenv("THQ_GEMM_DQ")
    m, n, k = 2048, 12288, 4096
    b = weight_bytes(O.Q4_K, n, k, seed=1530)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    xf, xb = xrows(m, k, seed=1531)
    y = thq.matmul(w, xb, torch.float32)
    y2 = torch.empty_like(y)
    thq.matmul_noalloc(w, xb, y2)
    torch.cuda.synchronize()
    # two bf16 roundings of the same weights (bf16(d1 q - m1) against the
    # tile's bf16(d1 (128 + q) - (128 d1 + m1))): within the 1e-2 row bar
    assert rel_row_err(y.cpu().numpy(), y2.cpu().numpy().astype(np.float64)) <= 1e-2
