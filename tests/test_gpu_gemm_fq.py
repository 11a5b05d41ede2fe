"""Prefill GEMM that dequantizes its 4-bit weight tiles into LDS
(k_gemm_fq.hip, THQ_GEMM_FQ=1 routes every supported Q4_K / MLX affine GEMM
call to it).  Its weights are bf16(d1*q - m1) of the oracle's bit-exact
dequantization (one rounding), so on sampled rows the product is pinned at
the f32 accumulation bar (1e-5 of the row norm) to the f64 product with the
oracle's weights rounded to bf16, and meets the path's 1e-2 row bar
against the exact oracle.  Every block geometry (256 x 256, 128 x 256,
512 x 192) and forced K splits (superblock-aligned, summed by the split
reduce), ragged M and N, gate/up with the SiLU epilogue (and its fallback
when the up half does not start on a row quad), and MLX affine weights.
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
    monkeypatch.setenv("THQ_GEMM_FQ", "1")


def xrows(m, k, seed):
    xf = O.bf16_round(activations(m, k, seed=seed))
    return xf, torch.from_numpy(xf).cuda().to(torch.bfloat16)


def pick_rows(m, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 10)]))


@pytest.mark.parametrize("m,n,k,geom,splits", [
    (2048, 1536, 1024, 3, 1),   # 512 x 192 tiles
    (300, 1000, 2048, 1, 1),    # 256 x 256, ragged M and N
    (77, 1000, 4096, 2, 4),     # 128 x 256, 4 K splits
    (130, 4096, 4096, 2, 3),    # 3 splits of 6 superblocks + a short last one
    (513, 520, 12288, 3, 6),
])
def test_fq_q4k_rounded_product(monkeypatch, m, n, k, geom, splits):
    monkeypatch.setenv("THQ_FQ_GEOM", str(geom))
    monkeypatch.setenv("THQ_FQ_SPLITS", str(splits))
    b = weight_bytes(O.Q4_K, n, k, seed=1700 + n)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    xf, xb = xrows(m, k, seed=1710 + m)
    print(f"[fq] q4_k m={m} {n}x{k} geom={geom} splits={splits}", flush=True)
    y = thq.matmul(w, xb, torch.float32)
    y16 = thq.matmul(w, xb, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(y16, y.to(torch.bfloat16))
    pick = pick_rows(m, m + n)
    got = y.cpu().numpy()[pick]
    wr = O.bf16_round(O.dequantize(O.Q4_K, b, n, k)).astype(np.float64)
    assert rel_row_err(got, xf[pick].astype(np.float64) @ wr.T) <= 1e-5
    ref = O.matmul(O.Q4_K, b, n, k, xf[pick], O.MODE_DEQUANT_F32)
    assert rel_row_err(got, ref) <= 1e-2


@pytest.mark.parametrize("m,h,k", [(256, 1024, 4096), (130, 1000, 2048)])
def test_fq_gate_up(m, h, k):
    bg = weight_bytes(O.Q4_K, h, k, seed=1800 + h)
    bu = weight_bytes(O.Q4_K, h, k, seed=1801 + h)
    wg = thq.QTensor.from_gguf_bytes(O.Q4_K, bg, h, k)
    wu = thq.QTensor.from_gguf_bytes(O.Q4_K, bu, h, k)
    fused = thq.QTensor.fuse([wg, wu])
    xf, xb = xrows(m, k, seed=1810 + m)
    print(f"[fq] gate/up m={m} 2x{h}x{k}", flush=True)
    y = thq.gate_up_silu(fused, xb, torch.float32)
    torch.cuda.synchronize()
    pick = pick_rows(m, 7 * m)
    gate = O.matmul(O.Q4_K, bg, h, k, xf[pick], O.MODE_DEQUANT_F32)
    up = O.matmul(O.Q4_K, bu, h, k, xf[pick], O.MODE_DEQUANT_F32)
    ref = O.bf16_bits_to_f32(O.gate_up_silu(np.concatenate([gate, up], axis=1)))  # bf16 bits -> f32
    assert rel_row_err(y.cpu().numpy()[pick], ref) <= 1e-2


def test_fq_gate_up_unaligned_falls_back(monkeypatch):
    """2 x 1002 rows: the up half starts mid row quad, so the call takes the
    other GEMM; with and without THQ_GEMM_FQ the result is bit-identical."""
    h, k, m = 1002, 2048, 70
    bg = weight_bytes(O.Q4_K, h, k, seed=1820)
    bu = weight_bytes(O.Q4_K, h, k, seed=1821)
    fused = thq.QTensor.fuse([thq.QTensor.from_gguf_bytes(O.Q4_K, bg, h, k),
                              thq.QTensor.from_gguf_bytes(O.Q4_K, bu, h, k)])
    _, xb = xrows(m, k, seed=1822)
    a = thq.gate_up_silu(fused, xb, torch.float32)
    monkeypatch.setenv("THQ_GEMM_FQ", "0")
    b = thq.gate_up_silu(fused, xb, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("m,n,k", [(1024, 1536, 2048), (200, 768, 4096)])
def test_fq_affine(m, n, k):
    wq, sb = rand_qlin_fast(n, k, seed=1900 + n)
    w = thq.QTensor.from_affine(torch.from_numpy(wq.view(np.int32)).cuda(), torch.from_numpy(sb.view(np.int16)).cuda(),
                                n, k)
    xf, xb = xrows(m, k, seed=1910 + m)
    print(f"[fq] affine m={m} {n}x{k}", flush=True)
    y = thq.matmul(w, xb, torch.float32)
    torch.cuda.synchronize()
    pick = pick_rows(m, m)
    ref = O.affine_matmul(wq, sb, n, k, xf[pick])
    assert rel_row_err(y.cpu().numpy()[pick], ref) <= 1e-2
    # the bf16 weights it multiplies: fma(scale, q, bias) rounded once; the
    # oracle's f32 weights come from an f64 product (a rare one-ulp bf16
    # difference after its second rounding), hence 1e-4 here
    wr = O.bf16_round(O.affine_dequant_f32(wq, sb, n, k)).astype(np.float64)
    assert rel_row_err(y.cpu().numpy()[pick], xf[pick].astype(np.float64) @ wr.T) <= 1e-4
