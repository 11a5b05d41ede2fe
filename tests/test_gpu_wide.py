"""Exact-weight GEMV for 17..64 activation rows (k_gemv_wide.hip): the
batched speculative-verify LM head's route (engine/src/engine.rs:2338-2470,
5 drafted tokens x 8 sequences = 40 rows) for Q8_0, Q4_K, Q6_K and MLX
affine weights, against the oracle's exact-weight product.

Exact weights leave only f32 summation error, so the bar is the f32 one
(1e-4 of the row norm).  Shapes cover a ragged last 128-row tile, K split
across blocks (few output tiles), K = 12288, one and two 32-row halves of
activation rows; bf16 output is the f32 result rounded once, and the fused
argmax epilogue gives the logits path's indices.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, assert_close_elem, q6k_bytes, rand_qlin_fast, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


KINDS = ["q8_0", "q4_k", "q6_k", "affine"]


def make(kind, n, k, seed):
    if kind == "affine":
        wq, sb = rand_qlin_fast(n, k, seed=seed)
        return thq.QTensor.from_affine(wq, sb, n, k), lambda xf: O.affine_matmul(wq, sb, n, k, xf)
    qtype = {"q8_0": O.Q8_0, "q4_k": O.Q4_K, "q6_k": O.Q6_K}[kind]
    b = q6k_bytes(n, k, seed=seed) if qtype == O.Q6_K else weight_bytes(qtype, n, k, seed=seed)
    return thq.QTensor.from_gguf_bytes(qtype, b, n, k), lambda xf: O.matmul(qtype, b, n, k, xf)


# (n, k, rows): a ragged last tile in one K split; 32 output tiles (K split
# four ways); a long K; and a vocabulary-wide head (65536 outputs) that the
# router gives the wide GEMV from 4 (Q8_0), 5 (Q4_K / affine) and 9 (Q6_K) rows
CASES = [(1000, 1024, (9, 16, 17, 31, 32, 33, 40, 41, 64)), (4096, 4096, (17, 40, 64)), (300, 12288, (20, 40)),
         (65536, 512, (4, 5, 9, 12, 16))]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("case", range(len(CASES)))
def test_wide_matches_oracle(kind, case):
    n, k, rows = CASES[case]
    w, ref_of = make(kind, n, k, seed=900 + case)
    for m in rows:
        print(f"[wide] {kind} {n}x{k} m={m}", flush=True)
        xf = O.bf16_round(activations(m, k, seed=950 + m))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        got = thq.matmul(w, xb, torch.float32, flags=thq.MODE_EXACT_W)
        torch.cuda.synchronize()
        err = rel_row_err(got.cpu().numpy(), ref_of(xf))
        assert err <= 1e-4, f"{kind} {n}x{k} m={m}: max row error {err:.3g}"
        if m == 40:
            got16 = thq.matmul(w, xb, torch.bfloat16, flags=thq.MODE_EXACT_W)
            assert torch.equal(got16, got.to(torch.bfloat16))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k,rows", [(5000, 1024, (17, 40, 64)), (65536, 256, (5, 9, 16))])
def test_wide_fused_argmax(kind, n, k, rows):
    """Per-32-row (max, lowest index) partials merged to the row argmax equal
    the logits path's argmax and the oracle's argmax of those logits."""
    w, _ = make(kind, n, k, seed=990)
    for m in rows:
        print(f"[wide] fused argmax {kind} m={m}", flush=True)
        xb = torch.from_numpy(O.bf16_round(activations(m, k, seed=m + 77))).cuda().to(torch.bfloat16)
        _, fused = thq.matmul_argmax(w, xb, want_logits=False, flags=thq.MODE_ARGMAX_FUSED)
        logits, idx = thq.matmul_argmax(w, xb)
        torch.cuda.synchronize()
        assert torch.equal(fused, idx)
        assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_rows(logits.cpu().numpy()))


def test_wide_argmax_ties():
    """Equal logits across 32-row partials: the lowest index of the maximum
    wins (engine/src/engine.rs:1891-1898).  A zero row of x makes every
    logit 0 (all tied: index 0); a duplicated weight row gives two equal
    logits in different partials of every row."""
    n, k = 4000, 512
    b = weight_bytes(O.Q8_0, n, k, seed=991)
    raw = np.frombuffer(b, np.uint8).reshape(n, -1).copy()
    raw[3000] = raw[17]                     # rows 17 and 3000 give equal logits
    w = thq.QTensor.from_gguf_bytes(O.Q8_0, raw.tobytes(), n, k)
    m = 24
    xf = O.bf16_round(activations(m, k, seed=5))
    xf[3] = 0.0                             # every logit 0: index 0
    xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
    _, fused = thq.matmul_argmax(w, xb, want_logits=False, flags=thq.MODE_ARGMAX_FUSED)
    logits, idx = thq.matmul_argmax(w, xb)
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    assert torch.equal(fused, idx)
    want = O.argmax_rows(lg)
    assert np.array_equal(idx.cpu().numpy().astype(np.uint32), want)
    assert want[3] == 0
    assert np.array_equal(lg[:, 17], lg[:, 3000])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("shape", [(2 * 2500, 1024), (2 * 1024, 4096)])
def test_wide_gate_up(kind, shape):
    """Fused gate/up over a [gate; up] weight: silu(bf16(gate)) * bf16(up) of
    the same route's plain product (the epilogue at most one bf16 step away:
    device and host expf), with K unsplit and split four ways; the plain
    product itself matches the oracle."""
    n, k = shape
    w, ref_of = make(kind, n, k, seed=995)
    for m in (24, 40):
        print(f"[wide] gate/up {kind} {n}x{k} m={m}", flush=True)
        xf = O.bf16_round(activations(m, k, seed=m + 31))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        y = thq.matmul(w, xb, torch.float32, flags=thq.MODE_EXACT_W).cpu().numpy()
        assert rel_row_err(y, ref_of(xf)) <= 1e-4
        gu = thq.gate_up_silu(w, xb, torch.float32, flags=thq.MODE_EXACT_W).cpu().numpy()
        assert_close_elem(f"gate/up {kind} m={m}", gu, O.bf16_bits_to_f32(O.gate_up_silu(y)), 2.0 ** -7)
