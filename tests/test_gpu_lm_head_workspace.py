"""LM head + argmax without a logits buffer on a vocabulary-sized head, in a
fresh context (thq_matmul_argmax with logits_dev NULL).

The logits then live in the context workspace together with the scratch of
the route the call takes: the argmax partials, and the split-K partials of
a route that splits K (on a 151936-row head the wide GEMV takes 5 and 12 rows
of Q8_0 and 12 of Q6_K with K unsplit; 5 rows of Q6_K take the decode GEMV,
whose plan splits K in two).  Both must be
sized from that route before any pointer into the workspace is formed, or
the logits and the partials overlap (and the first call in a fresh context,
which grows the workspace, would leave the logits in a retired buffer).
Each case runs first in a new context, so the growth path is the one tested,
then again in the same context; with and without THQ_MODE_ARGMAX_FUSED.
Indices are compared with the logits-buffer path and with the oracle's scan
of its own f64 logits.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, q6k_bytes, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")

N, K = 151936, 4096


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind,m", [("q8_0", 5), ("q8_0", 12), ("q6_k", 5), ("q6_k", 12)])
def test_head_without_logits_fresh_context(kind, m):
    if kind == "q8_0":
        qt, b = O.Q8_0, weight_bytes(O.Q8_0, N, K, seed=4)
    else:
        qt, b = O.Q6_K, q6k_bytes(N, K, seed=4)
    xf = O.bf16_round(activations(m, K, seed=6))
    xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
    ref = O.matmul(qt, b, N, K, xf, O.MODE_DEQUANT_F32)
    want = list(O.argmax_rows(ref))
    for flags in (0, thq.MODE_ARGMAX_FUSED):
        ctx = thq.Context(0)
        w = thq.QTensor.from_gguf_bytes(qt, b, N, K, ctx=ctx)
        print(f"lm head {kind} m={m} flags={flags:#x}: fresh context", flush=True)
        for rep in range(2):
            _, idx = thq.matmul_argmax(w, xb, want_logits=False, flags=flags)
            torch.cuda.synchronize()
            assert list(idx.cpu().numpy()) == want, (flags, rep)
        logits, idx2 = thq.matmul_argmax(w, xb)
        torch.cuda.synchronize()
        assert list(idx2.cpu().numpy()) == want
        assert rel_row_err(logits.cpu().numpy(), ref) <= 1e-4
        del w, ctx
