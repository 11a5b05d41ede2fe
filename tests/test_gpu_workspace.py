"""Workspace planning and the last-block tickets.

thq_call_scratch_bytes plans a call's route on the host and reports the
workspace it needs; after thq_reserve of at least that much (and of the
split-K arrival counters) the calls allocate nothing, so they can be captured
in a HIP graph: the graph is replayed several times with eager work between
the replays and every replay is checked against the eager result.  The
dequantize-then-GEMM route does not grow the workspace past THQ_DQ_MAX_MB
(the weight then takes the tile GEMM).  The split-K tile GEMV and the
emitting gate/up sum in the last block behind release/acquire tickets;
THQ_TILE_TICKET=0 takes the separate reduce launch instead, and both give
the same bits.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def xb(m, k, seed):
    return torch.from_numpy(O.bf16_round(activations(m, k, seed=seed))).cuda().to(torch.bfloat16)


def test_reserve_then_capture():
    ctx = thq.Context(0)  # a fresh context: its workspace starts empty
    n, k = 4096, 4096
    b = weight_bytes(O.Q4_K, n, k, seed=2100)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k, ctx=ctx)
    shapes = [1, 4, 40, 300]
    need = max(thq.call_scratch_bytes(w, m) for m in shapes)
    print(f"[ws] reserve {need} B", flush=True)
    ctx.reserve(need, counters=(n + 31) // 32)
    size = ctx.workspace_bytes()
    assert size >= need
    xs = {m: xb(m, k, 2110 + m) for m in shapes}
    eager = {m: thq.matmul(w, xs[m], torch.float32) for m in shapes}
    torch.cuda.synchronize()
    assert ctx.workspace_bytes() == size  # nothing grew
    outs = {m: torch.empty((m, n), dtype=torch.float32, device="cuda") for m in shapes}
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for m in shapes:
                thq.matmul(w, xs[m], out=outs[m])
    for rep in range(3):
        for m in shapes:
            outs[m].fill_(float("nan"))
        _ = torch.randn(1024, 1024, device="cuda") @ torch.randn(1024, 1024, device="cuda")  # eager work between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for m in shapes:
            assert torch.equal(outs[m], eager[m]), (rep, m)
    assert ctx.workspace_bytes() == size


def test_scratch_bytes_matches_plan():
    n, k = 12288, 4096
    b = weight_bytes(O.Q4_K, n, k, seed=2200)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    assert thq.call_scratch_bytes(w, 1) == 0  # the M = 1 GEMV has no scratch
    # the dequantize-then-GEMM route: the bf16 weight
    assert thq.call_scratch_bytes(w, 2048) >= n * k * 2
    assert thq.call_scratch_bytes(w, 0) == 0


def test_dq_route_capped(monkeypatch):
    monkeypatch.setenv("THQ_DQ_MAX_MB", "64")
    ctx = thq.Context(0)
    n, k = 12288, 4096  # bf16 weight: 96 MiB > 64 MiB
    b = weight_bytes(O.Q4_K, n, k, seed=2300)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k, ctx=ctx)
    assert thq.call_scratch_bytes(w, 1024) < n * k * 2
    x = xb(1024, k, 2301)
    print("[ws] capped route", flush=True)
    y = thq.matmul(w, x, torch.float32)
    torch.cuda.synchronize()
    assert ctx.workspace_bytes() < n * k * 2
    pick = np.array([0, 511, 1023])
    ref = O.matmul(O.Q4_K, b, n, k, O.bf16_round(activations(1024, k, seed=2301))[pick], O.MODE_DEQUANT_F32)
    assert rel_row_err(y.cpu().numpy()[pick], ref) <= 1e-2


@pytest.mark.parametrize("gu", [False, True])
def test_ticket_matches_separate_reduce(monkeypatch, gu):
    """Tile-plane GEMV with K splits (4096 x 12288 down shape at M = 5):
    the last block's sum behind the tickets equals k_split_reduce's."""
    n, k, m = (4096, 12288, 5) if not gu else (2 * 4096, 12288, 5)
    b = weight_bytes(O.Q4_K, n, k, seed=2400 + int(gu))
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    w.add_tiles()
    x = xb(m, k, 2401)
    run = (lambda: thq.gate_up_silu(w, x, torch.float32)) if gu else (lambda: thq.matmul(w, x, torch.float32))
    a = [run() for _ in range(3)]
    monkeypatch.setenv("THQ_TILE_TICKET", "0")
    c = run()
    torch.cuda.synchronize()
    for t in a:
        assert torch.equal(t, c)
