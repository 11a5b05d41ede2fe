"""Every output row of the large configurations, not a sample.

The prefill GEMM at M = 2048 on the 12288 x 4096 gate/up shape and the four
projections of a Qwen3-8B-class decoder layer at M = 256 (QKV 6144 x 4096, o
4096 x 4096, fused gate/up 2 x 12288 x 4096 with the SiLU epilogue, down
4096 x 12288) are checked row by row against a float32 product on the GPU
with the library's dequantized weights (thq_dequantize, which the oracle
pins bit for bit on the same weights below and in test_gpu_parity).  The
bar is the path's: max |err| <= 1e-2 of each row's L2 norm for bf16
activations.  The default routes run (dequantize + bf16 GEMM at M = 2048,
the tile GEMM at M = 256).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def row_err(y: torch.Tensor, ref: torch.Tensor) -> float:
    d = (y.double() - ref.double()).abs().max(dim=1).values
    nrm = ref.double().norm(dim=1).clamp_min(1e-300)
    return float((d / nrm).max())


def weight(n, k, seed):
    b = weight_bytes(O.Q4_K, n, k, seed=seed)
    return b, thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)


def xact(m, k, seed):
    return torch.from_numpy(O.bf16_round(activations(m, k, seed=seed))).cuda().to(torch.bfloat16)


def test_dequant_pins_reference_weights():
    b, w = weight(512, 4096, 3000)
    got = w.dequantize().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), O.dequantize(O.Q4_K, b, 512, 4096).view(np.uint32))


def test_gemm_m2048_every_row():
    n, k, m = 12288, 4096, 2048
    _, w = weight(n, k, 3001)
    x = xact(m, k, 3002)
    print(f"[rows] gemm m={m} {n}x{k}", flush=True)
    y = thq.matmul(w, x, torch.bfloat16)
    ref = x.float() @ w.dequantize().float().t()
    torch.cuda.synchronize()
    err = row_err(y, ref)
    print(f"[rows] gemm m={m}: max row err {err:.2e}", flush=True)
    assert err <= 1e-2


def test_decoder_layer_m256_every_row():
    m, h = 256, 4096
    x = xact(m, h, 3010)
    _, wqkv = weight(6144, h, 3011)
    _, wo = weight(h, h, 3012)
    _, wg = weight(12288, h, 3013)
    _, wu = weight(12288, h, 3014)
    _, wd = weight(h, 12288, 3015)
    fused = thq.QTensor.fuse([wg, wu])
    print(f"[rows] decoder layer m={m}", flush=True)
    qkv = thq.matmul(wqkv, x, torch.bfloat16)
    o = thq.matmul(wo, x, torch.bfloat16)
    hmid = thq.gate_up_silu(fused, x, torch.bfloat16)
    d = thq.matmul(wd, hmid, torch.bfloat16)
    xf = x.float()
    checks = [("qkv", qkv, xf @ wqkv.dequantize().float().t()), ("o", o, xf @ wo.dequantize().float().t())]
    g = (xf @ wg.dequantize().float().t()).to(torch.bfloat16).float()
    u = (xf @ wu.dequantize().float().t()).to(torch.bfloat16).float()
    checks.append(("gate_up", hmid, g / (1.0 + torch.exp(-g)) * u))
    checks.append(("down", d, hmid.float() @ wd.dequantize().float().t()))
    torch.cuda.synchronize()
    for name, got, ref in checks:
        err = row_err(got, ref)
        print(f"[rows] {name}: max row err {err:.2e}", flush=True)
        assert err <= 1e-2, name
