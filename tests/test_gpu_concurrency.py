"""Re-entrancy as include/thq.h states it: calls on distinct streams, from
distinct host threads, give the bits the same calls give one after another
on one stream.  The paths used hold no context workspace (M = 1 GEMV, the
M = 2 row GEMV, the unsplit GEMM, the MFMA decode GEMV at one split); calls
that share the workspace must be ordered on one stream and are not mixed
here.  Streams keep the default priority.
"""
import threading

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


def test_two_threads_two_streams_bit_identical():
    w_big = thq.QTensor.from_gguf_bytes(thq.Q4_K, weight_bytes(O.Q4_K, 12288, 4096, seed=71), 12288, 4096)
    w_q8 = thq.QTensor.from_gguf_bytes(thq.Q8_0, weight_bytes(O.Q8_0, 3072, 1024, seed=72), 3072, 1024)
    xs = {m: torch.from_numpy(O.bf16_round(activations(m, 4096, seed=m))).cuda().to(torch.bfloat16)
          for m in (1, 2, 5, 2048)}
    x8 = torch.from_numpy(O.bf16_round(activations(1, 1024, seed=6))).cuda().to(torch.bfloat16)
    # 12288 x 4096 at M = 5: 384 row tiles, one K split (no workspace)
    jobs = [(w_big, xs[1]), (w_big, xs[2]), (w_big, xs[5]), (w_big, xs[2048]), (w_q8, x8)]
    print("[concurrency] reference on one stream", flush=True)
    ref = [thq.matmul(w, x, torch.float32) for w, x in jobs]
    torch.cuda.synchronize()

    results = {}
    errors = []

    def worker(tid):
        try:
            s = torch.cuda.Stream()
            out = []
            with torch.cuda.stream(s):
                for rep in range(4):
                    order = jobs if (tid + rep) % 2 == 0 else jobs[::-1]
                    ys = [thq.matmul(w, x, torch.float32) for w, x in order]
                    out.append(ys if (tid + rep) % 2 == 0 else ys[::-1])
            s.synchronize()
            results[tid] = out
        except Exception as e:  # reported below, in the main thread
            errors.append(e)

    print("[concurrency] two threads, two streams", flush=True)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    for tid in range(2):
        for ys in results[tid]:
            for y, r in zip(ys, ref):
                assert torch.equal(y.view(torch.int32), r.view(torch.int32))
