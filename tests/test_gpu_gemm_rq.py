"""Prefill GEMM that dequantizes each wave's weight rows in registers
(k_gemm_rq.hip).  THQ_GEMM_RQ=1 routes every supported Q4_K / MLX affine GEMM
call to it; unset, the router takes it from 1024 rows (tests below pin that
rule).  Its weights are the rounded tiles' bf16 values, so the product is
pinned at the f32 accumulation bar (1e-6 of the row norm) to the f64 product
with the library's bf16 dequantization (thq_dequantize to bf16, itself pinned
to the oracle in test_gpu_gemm_dq), and meets the path's 1e-2 row bar
against the oracle's exact dequantization.  Covered: 128- and 256-row
blocks, K split into uniform ranges (the last block of each tile sums them)
and the whole-then-halved grid of more tiles than CUs, ragged M and N,
gate/up with the SiLU epilogue, MLX affine weights, bf16 output, run-to-run
identity, and the router's default choice.
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
def _route(monkeypatch):
    monkeypatch.setenv("THQ_GEMM_RQ", "1")
    monkeypatch.setenv("THQ_GEMM_DQ", "0")


def xrows(m, k, seed):
    xf = O.bf16_round(activations(m, k, seed=seed))
    return xf, torch.from_numpy(xf).cuda().to(torch.bfloat16)


def row_err(y, ref):
    d = (y.double() - ref.double()).abs().max(dim=1).values
    return float((d / ref.double().norm(dim=1).clamp_min(1e-300)).max())


def pick_rows(m, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 10)]))


@pytest.mark.parametrize("m,n,k,bm,splits", [
    (128, 1000, 2048, 128, 0),   # one tile row, K split to fill the CUs
    (77, 520, 4096, 128, 3),     # ragged M and N, 3 splits
    (300, 3000, 4096, 256, 0),   # 256-row blocks
    (513, 1100, 12288, 256, 5),  # 5 splits of 192 K steps
    (1024, 12288, 4096, 256, 0),
    (4608, 4096, 1024, 256, 0),  # 288 tiles: 256 over all of K, 32 in halves
])
def test_rq_q4k(monkeypatch, m, n, k, bm, splits):
    monkeypatch.setenv("THQ_RQ_BM", str(bm))
    if splits:
        monkeypatch.setenv("THQ_RQ_SPLITS", str(splits))
    b = weight_bytes(O.Q4_K, n, k, seed=2400 + n)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    xf, xb = xrows(m, k, seed=2410 + m)
    print(f"[rq] q4_k m={m} {n}x{k} bm={bm} splits={splits}", flush=True)
    y = thq.matmul(w, xb, torch.float32)
    y16 = thq.matmul(w, xb, torch.bfloat16)
    again = thq.matmul(w, xb, torch.float32)
    ref = xb.double() @ w.dequantize_bf16().double().t()
    torch.cuda.synchronize()
    assert torch.equal(y, again)
    assert torch.equal(y16, y.to(torch.bfloat16))
    assert row_err(y, ref) <= 1e-6
    pick = pick_rows(m, m + n)
    ora = O.matmul(O.Q4_K, b, n, k, xf[pick], O.MODE_DEQUANT_F32)
    assert rel_row_err(y.cpu().numpy()[pick], ora) <= 1e-2


def test_rq_split_orders_agree(monkeypatch):
    """The same product with 1, 2 and 4 K splits: f32 sums in different
    orders, within the accumulation bar of each other."""
    n, k, m = 2048, 4096, 256
    b = weight_bytes(O.Q4_K, n, k, seed=2450)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    _, xb = xrows(m, k, seed=2451)
    ys = []
    for s in (1, 2, 4):
        monkeypatch.setenv("THQ_RQ_SPLITS", str(s))
        ys.append(thq.matmul(w, xb, torch.float32))
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert row_err(y, ys[0]) <= 1e-6


@pytest.mark.parametrize("m,h,k", [(256, 1024, 4096), (1100, 1000, 2048)])
def test_rq_gate_up(m, h, k):
    bg = weight_bytes(O.Q4_K, h, k, seed=2500 + h)
    bu = weight_bytes(O.Q4_K, h, k, seed=2501 + h)
    wg = thq.QTensor.from_gguf_bytes(O.Q4_K, bg, h, k)
    wu = thq.QTensor.from_gguf_bytes(O.Q4_K, bu, h, k)
    fused = thq.QTensor.fuse([wg, wu])
    xf, xb = xrows(m, k, seed=2510 + m)
    print(f"[rq] gate/up m={m} 2x{h}x{k}", flush=True)
    y = thq.gate_up_silu(fused, xb, torch.float32)
    torch.cuda.synchronize()
    pick = pick_rows(m, 7 * m)
    gate = O.matmul(O.Q4_K, bg, h, k, xf[pick], O.MODE_DEQUANT_F32)
    up = O.matmul(O.Q4_K, bu, h, k, xf[pick], O.MODE_DEQUANT_F32)
    ref = O.bf16_bits_to_f32(O.gate_up_silu(np.concatenate([gate, up], axis=1)))  # bf16 bits -> f32
    assert rel_row_err(y.cpu().numpy()[pick], ref) <= 1e-2


@pytest.mark.parametrize("m,n,k,splits", [(1024, 1536, 2048, 0), (200, 768, 4096, 3)])
def test_rq_affine(monkeypatch, m, n, k, splits):
    if splits:
        monkeypatch.setenv("THQ_RQ_SPLITS", str(splits))
    wq, sb = rand_qlin_fast(n, k, seed=2600 + n)
    w = thq.QTensor.from_affine(torch.from_numpy(wq.view(np.int32)).cuda(), torch.from_numpy(sb.view(np.int16)).cuda(),
                                n, k)
    xf, xb = xrows(m, k, seed=2610 + m)
    print(f"[rq] affine m={m} {n}x{k} splits={splits}", flush=True)
    y = thq.matmul(w, xb, torch.float32)
    ref = xb.double() @ w.dequantize_bf16().double().t()
    torch.cuda.synchronize()
    # the tile's weights are fma(scale, 128 + q, -(128 scale - bias)) rounded
    # once; the bf16 dequantization rounds the exact scale * q + bias: a rare
    # one-ulp difference, hence 1e-4
    assert row_err(y, ref) <= 1e-4
    pick = pick_rows(m, m)
    assert rel_row_err(y.cpu().numpy()[pick], O.affine_matmul(wq, sb, n, k, xf[pick])) <= 1e-2


@pytest.mark.parametrize("m,n,k", [(1024, 12288, 4096), (2048, 4096, 12288)])
def test_rq_is_the_default_from_1024_rows(monkeypatch, m, n, k):
    """Unset, the router takes this GEMM for 12288 x 4096 at M = 1024 (in
    place of the tile GEMM) and for the down shape at M = 2048: the default
    call and the forced one give the same bits."""
    b = weight_bytes(O.Q4_K, n, k, seed=2700 + n)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    _, xb = xrows(m, k, seed=2701)
    forced = thq.matmul(w, xb, torch.float32)
    monkeypatch.delenv("THQ_GEMM_RQ")
    monkeypatch.delenv("THQ_GEMM_DQ")
    default = thq.matmul(w, xb, torch.float32)
    monkeypatch.setenv("THQ_GEMM_RQ", "0")
    other = thq.matmul(w, xb, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(default, forced)
    assert not torch.equal(other, forced)  # another kernel, another summation order
    assert row_err(other, forced) <= 1e-5
