"""thq_matmul_noalloc: thq_matmul on the device's static scratch array, for
callers that cannot allocate.  Called through the C ABI and compared with
thq_matmul on the same inputs, on two calls in a row with the second one
smaller (the array keeps the first call's contents), for each route that
uses scratch: the split-K decode GEMV, the split-K tile GEMM, the split-K
streaming mid-M GEMM, the split-K wide exact-weight GEMV (17..64 rows) and
THQ_MODE_Q8ACT.
Both entry points run the same kernels with the same plans, so the outputs
must agree bit for bit (stricter than the 1e-2 row bar of bf16 rows); the
oracle's f64 product pins them to the path's tolerance.  A route needing
more scratch than the array holds must fail with THQ_ESHAPE and write
nothing.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")

N, K = 12288, 4096


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


@pytest.fixture(scope="module")
def weight():
    b = weight_bytes(O.Q4_K, N, K, seed=21)
    return b, thq.QTensor.from_gguf_bytes(thq.Q4_K, b, N, K)


def noalloc(w, x, y, flags=0):
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return thq.lib.thq_matmul_noalloc(w.ctx.h, w.h, C.c_void_p(x.data_ptr()), thq.ACT_BF16, x.shape[0],
                                      C.c_void_p(y.data_ptr()), thq.ACT_F32, flags, s)


@pytest.mark.parametrize("route,ms,flags,mid", [
    ("split-K decode GEMV", (16, 12), 0, "0"),
    ("split-K GEMM", (128, 64), 0, "0"),
    ("split-K streaming mid GEMM", (128, 100), 0, "1"),
    ("split-K wide GEMV", (40, 20), thq.MODE_EXACT_W, "0"),
    ("Q8ACT", (9, 3), thq.MODE_Q8ACT, "0"),
])
def test_noalloc_matches_matmul(weight, route, ms, flags, mid, monkeypatch):
    # THQ_GEMM_MID picks between the tile GEMM and the streaming GEMM (whose
    # planner splits K four ways at 100 and 128 rows of this shape)
    monkeypatch.setenv("THQ_GEMM_MID", mid)
    b, w = weight
    for m in ms:
        if flags == thq.MODE_EXACT_W:
            assert thq.plan_gemv_wide(thq.Q4_K, m, N, K).splits > 1, f"{route} at M={m} should split K"
        elif flags == 0 and mid == "0":
            plan = thq.plan_gemv_mfma(thq.Q4_K, m, N, K) if m <= 16 else thq.plan_gemm(thq.Q4_K, m, N, K)
            assert plan.splits > 1, f"{route} at M={m} should split K"
        xf = O.bf16_round(activations(m, K, seed=m))
        x = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        want = thq.matmul(w, x, torch.float32, flags=flags)
        got = torch.full((m, N), float("nan"), dtype=torch.float32, device="cuda")
        print(f"noalloc {route} M={m}", flush=True)
        assert noalloc(w, x, got, flags) == thq.OK, thq.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{route} M={m}"
        q8 = flags == thq.MODE_Q8ACT
        ref = O.matmul(O.Q4_K, b, N, K, xf, O.MODE_Q8ACT if q8 else O.MODE_DEQUANT_F32)
        # Q8ACT against the oracle's Q8ACT, exact weights at the f32 bar, rounded tiles at the bf16 one
        assert rel_row_err(got.cpu().numpy(), ref) <= (1e-5 if q8 else 1e-4 if flags else 1e-2)


def test_noalloc_rejects_scratch_beyond_its_size(weight):
    _, w = weight
    m = 768  # two K splits of 768 x 12288 f32 partials: 72 MiB > 64 MiB
    p = thq.plan_gemm(thq.Q4_K, m, N, K)
    assert p.workspace_bytes > thq.lib.thq_noalloc_scratch_bytes()
    x = torch.zeros((m, K), dtype=torch.bfloat16, device="cuda")
    y = torch.full((m, N), 7.0, dtype=torch.float32, device="cuda")
    assert noalloc(w, x, y) == thq.ESHAPE
    assert "scratch" in thq.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all()), "a rejected call launches nothing"
