"""Exact per-row top-k for sampled verify (thq_topk, thq_matmul_topk) against
the oracle's sort by (key desc, id asc), key(NaN) = -inf, key(-0.0) = +0.0
(engine/src/sample_kernel.rs:163-169, 326-347).  Selection is integer work
on the logits' bits, so indices and values must be bit-exact.

Rows come from the reference's own test generator (lm_row: bf16-rounded
logits with exact ties, peaked tokens, NaN / -inf / -0.0 / +0.0), plus rows
built to stress the tie rule across segment boundaries, all-NaN rows, k
larger than the row, rows long enough for two merge levels, and more rows
than one launch's grid holds.  The LM-head variant is checked on the Q8_0
151936 x 4096 head at the verify shapes M = 5 and 40.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, lm_row, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


@pytest.fixture(params=["one launch", "two launches"])
def path(request, monkeypatch):
    """Rows of up to 4096 / k segments take one launch whose last block per
    row merges the segments' candidates (arrival counters); THQ_TILE_TICKET=0
    gives the counter-free form, a second launch per merge level."""
    if request.param == "two launches":
        monkeypatch.setenv("THQ_TILE_TICKET", "0")
    else:
        monkeypatch.delenv("THQ_TILE_TICKET", raising=False)
    return request.param


def check(v: np.ndarray, k: int, tag: str):
    vals, idx = thq.topk(torch.from_numpy(np.ascontiguousarray(v, np.float32)).cuda(), k)
    torch.cuda.synchronize()
    wv, wi = O.topk_rows(v, k)
    got_i = idx.cpu().numpy().view(np.uint32)
    got_v = vals.cpu().numpy()
    bad = np.argwhere((got_i != wi).any(axis=1)).ravel()
    assert bad.size == 0, f"{tag}: row {bad[0]}: got {got_i[bad[0]][:8]} want {wi[bad[0]][:8]}"
    assert np.array_equal(got_v.view(np.uint32), wv.view(np.uint32)), tag


@pytest.fixture(scope="module")
def ref_rows():
    state = [0xF00D5EED]
    return {n: np.stack([lm_row(n, state, r % 2 == 0) for r in range(4)]) for n in (5000, 151936)}


@pytest.mark.parametrize("n", [5000, 151936])
@pytest.mark.parametrize("k", [1, 20, 32, 64])
def test_topk_reference_generator(ref_rows, n, k, path):
    print(f"topk lm_row n={n} k={k} {path}", flush=True)
    check(ref_rows[n], k, f"lm_row n={n} k={k}")


@pytest.mark.parametrize("n", [1, 100, 4095, 4096, 4097, 20011, 300000])
def test_topk_ties_across_segments(n, path):
    """Small-integer rows: the k-th value has copies in many 4096-wide
    segments, so the lowest ids among them must win across the merge."""
    rng = np.random.default_rng(n)
    v = rng.integers(0, 3, (3, n)).astype(np.float32)
    v[1] = 1.0                       # every element tied: ids 0..k-1
    v[2, rng.integers(0, n, 5)] = np.nan
    for k in (1, 7, 64):
        print(f"topk ties n={n} k={k} {path}", flush=True)
        check(v, k, f"ties n={n} k={k}")


@pytest.mark.parametrize("n", [3000, 9000])
def test_topk_every_k(n, path):
    """Every k from 1 to 64 on normal and bf16-rounded rows: the fast path's
    candidate count (keys at or above the threshold) then takes many values,
    including every remainder of its 8-wide batches."""
    rng = np.random.default_rng(n)
    v = rng.normal(0, 3, (3, n)).astype(np.float32)
    v[2] = O.bf16_round(v[2])          # bf16 logits: exact ties
    for k in range(1, 65):
        check(v, k, f"every k n={n} k={k}")


def test_topk_special_rows(path):
    n = 9000
    v = np.zeros((8, n), np.float32)
    v[0] = np.nan                    # all NaN: keys -inf, ids 0..k-1
    v[1] = -np.inf
    v[2, ::2] = -0.0                 # -0.0 ties with +0.0
    v[3] = np.linspace(-1, 1, n, dtype=np.float32)
    v[3, 17] = np.inf
    v[4] = np.nan
    v[4, 8999] = -5.0                # the only real value ranks first
    rng = np.random.default_rng(9)
    # subnormals of both signs around +-0 (the filter compares floats)
    v[5] = (rng.integers(-2000, 2000, n) * np.float32(1e-42)).astype(np.float32)
    v[6] = -np.abs(rng.normal(0, 1, n)).astype(np.float32) - 1.0  # negatives only
    v[7] = rng.normal(0, 1, n).astype(np.float32)
    v[7, rng.integers(0, n, 200)] = np.nan  # NaNs in most lanes of a segment
    v[7, 4096:4096 + 4096:2] = np.nan
    check(v, 64, "special")


def test_topk_k_beyond_row():
    v = np.array([[3.0, 1.0, 2.0, np.nan, 1.0]], np.float32)
    vals, idx = thq.topk(torch.from_numpy(v).cuda(), 8)
    assert list(idx.cpu().numpy().view(np.uint32)[0]) == [0, 2, 1, 4, 3] + [0xFFFFFFFF] * 3
    assert np.all(np.isneginf(vals.cpu().numpy()[0, 4:]))
    check(v, 8, "k > n")


def test_topk_many_rows(path):
    """More rows than one launch's grid dimension holds (65535)."""
    rng = np.random.default_rng(3)
    v = rng.integers(-4, 5, (70000, 8)).astype(np.float32)
    check(v, 4, "70000 rows")


@pytest.mark.parametrize("k", [1, 32, 64])
def test_topk_wide_rows_many(path, k):
    """30 rows of 151936: past 1024 blocks of 4096 logits, so the one-launch
    form takes 8192-logit segments; smooth, bf16-tied, integer-tied and
    NaN-heavy rows."""
    rng = np.random.default_rng(k)
    v = rng.normal(0, 3, (30, 151936)).astype(np.float32)
    v[1::4] = O.bf16_round(v[1::4])
    v[2::4] = np.round(v[2::4])
    v[3, :100000] = np.nan
    v[7, 5:] = -np.inf
    print(f"topk 30 x 151936 k={k} {path}", flush=True)
    check(v, k, f"30 wide rows k={k}")


def test_topk_rows_beyond_one_launch(path):
    """More rows than the one-launch form takes per launch (2048), each row
    several segments long, with ties: every launch's counters and pool."""
    rng = np.random.default_rng(4)
    v = rng.integers(-40, 41, (2100, 5000)).astype(np.float32)
    v[::7] = rng.normal(0, 2, (300, 5000)).astype(np.float32)
    for k in (8, 64):
        print(f"topk 2100 rows k={k} {path}", flush=True)
        check(v, k, f"2100 rows k={k}")


def test_topk_graph_replays():
    """The one-launch form inside a captured HIP graph: its arrival counters
    are left zero by the kernel itself, so every replay, with eager calls
    and synchronizations between them, gives the eager result."""
    rng = np.random.default_rng(12)
    v = torch.from_numpy(rng.normal(0, 3, (40, 151936)).astype(np.float32)).cuda()
    want_v, want_i = thq.topk(v, 32)  # eager; also reserves the counters before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gv, gi = thq.topk(v, 32)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(3):
        gv.fill_(float("nan"))
        gi.fill_(-1)
        ev, ei = thq.topk(v[:5].contiguous(), 32)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gi, want_i) and torch.equal(gv, want_v), r
        assert torch.equal(ei, want_i[:5]), r


def test_topk_rejects_bad_k():
    v = torch.zeros((2, 10), dtype=torch.float32, device="cuda")
    for k in (0, 65):
        with pytest.raises(thq.ThqError):
            thq.topk(v, k)


@pytest.fixture(scope="module")
def lm_head():
    n, k = 151936, 4096
    b = weight_bytes(O.Q8_0, n, k, seed=4)
    return b, thq.QTensor.from_gguf_bytes(thq.Q8_0, b, n, k)


@pytest.mark.parametrize("m", [5, 40])
def test_lm_head_topk(lm_head, m):
    """LM head + top-32 at the verify shapes: logits within 1e-4 of the
    oracle's f64 product (exact weights), and the top-k of every row equal
    to the oracle's top-k of those logits; the workspace-logits path gives
    the same candidates."""
    b, w = lm_head
    n, kdim = w.shape
    xf = O.bf16_round(activations(m, kdim, seed=8))
    xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
    print(f"lm head topk m={m}", flush=True)
    logits, vals, idx = thq.matmul_topk(w, xb, 32, want_logits=True)
    _, vals2, idx2 = thq.matmul_topk(w, xb, 32)
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    ref = O.matmul(O.Q8_0, b, n, kdim, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(lg, ref) <= 1e-4
    wv, wi = O.topk_rows(lg, 32)
    assert np.array_equal(idx.cpu().numpy().view(np.uint32), wi)
    assert np.array_equal(vals.cpu().numpy(), wv)
    assert torch.equal(idx, idx2) and torch.equal(vals, vals2)
    # against the f64 product: the oracle's own top-1 matches wherever it is not a near tie
    top_ref = O.topk_rows(ref, 2)[1]
    for r in range(m):
        if ref[r, top_ref[r, 0]] - ref[r, top_ref[r, 1]] > 1e-3 * np.linalg.norm(ref[r]):
            assert wi[r, 0] == top_ref[r, 0]
