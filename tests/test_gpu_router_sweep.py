"""Every routing branch of thq_matmul / thq_gate_up_silu / thq_matmul_argmax
(run_matmul, token-horizon_amd/csrc/thq_api.cpp) against the oracle, on small
shapes chosen to reach each kernel's edges: row counts that fill no tile,
the smallest and unusual K of each block size (including K past the M = 1
kernels' limits and Q8_0 K that is an odd multiple of 32), M from 1 to past
the GEMM's 64-row tile (9..16 rows: the MFMA decode GEMV with eight live
accumulator rows per lane), fused gate/up, and f32 activations.

Bars (the tolerances the path is held to everywhere): bf16 x within 1e-2 of
the row L2 norm, f32 x within 1e-4, argmax equal to the oracle's scan of the
same call's logits (engine.rs:1891-1898).  Each case prints its parameters
before it runs.
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


MS = [1, 2, 3, 5, 8, 9, 12, 16, 17, 24, 32, 33, 65, 130]

# (n, k): rows that fill no 4-row quad / 32-row tile; K at the block size, K
# between tile sizes, K past the M = 1 kernels' 4096 / 16384 (8192 for Q8_0)
SHAPES = {
    O.Q8_0: [(37, 32), (131, 96), (66, 1056), (20, 8224), (34, 4096)],
    O.Q4_K: [(37, 256), (131, 768), (66, 4352), (10, 16640)],
    O.Q6_K: [(37, 256), (131, 768), (66, 4352)],
}


def gguf_weight(qtype, n, k, seed):
    b = q6k_bytes(n, k, seed=seed) if qtype == O.Q6_K else weight_bytes(qtype, n, k, seed=seed)
    return b, thq.QTensor.from_gguf_bytes(qtype, b, n, k)


def run_case(tag, got, want, bar):
    err = rel_row_err(got, want)
    assert err <= bar, f"{tag}: max row error {err:.3g} > {bar}"


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_matmul_every_route(qtype):
    for si, (n, k) in enumerate(SHAPES[qtype]):
        b, w = gguf_weight(qtype, n, k, seed=100 + si)
        for m in MS:
            if m * k > (1 << 21):
                continue  # keeps the f64 oracle under a second per case
            print(f"[sweep] qtype={qtype} n={n} k={k} m={m}", flush=True)
            xf = O.bf16_round(activations(m, k, seed=m))
            ref = O.matmul(qtype, b, n, k, xf)
            xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
            run_case(f"bf16 q{qtype} {n}x{k} m={m}", thq.matmul(w, xb, torch.float32).cpu().numpy(), ref, 1e-2)
            if m in (1, 3, 9, 65):
                xd = torch.from_numpy(xf).cuda()
                run_case(f"f32 q{qtype} {n}x{k} m={m}", thq.matmul(w, xd, torch.float32).cpu().numpy(), ref, 1e-4)


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_gate_up_every_route(qtype):
    for si, (h, k) in enumerate(SHAPES[qtype]):
        b, w = gguf_weight(qtype, 2 * h, k, seed=200 + si)
        for m in MS:
            if m * k > (1 << 21):
                continue
            print(f"[sweep] gate/up qtype={qtype} h={h} k={k} m={m}", flush=True)
            xf = O.bf16_round(activations(m, k, seed=m + 7))
            want = O.bf16_bits_to_f32(O.gate_up_silu(O.matmul(qtype, b, 2 * h, k, xf)))
            xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
            got = thq.gate_up_silu(w, xb, torch.float32).cpu().numpy()
            run_case(f"gate/up q{qtype} {h}x{k} m={m}", got, want, 1e-2)


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_argmax_every_route(qtype):
    for si, (n, k) in enumerate(SHAPES[qtype]):
        b, w = gguf_weight(qtype, n, k, seed=300 + si)
        for m in (1, 2, 9, 16, 65):
            if m * k > (1 << 21):
                continue
            print(f"[sweep] argmax qtype={qtype} n={n} k={k} m={m}", flush=True)
            xf = O.bf16_round(activations(m, k, seed=m + 11))
            xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
            logits, idx = thq.matmul_argmax(w, xb)
            lg = logits.cpu().numpy()
            run_case(f"argmax logits q{qtype} {n}x{k} m={m}", lg, O.matmul(qtype, b, n, k, xf), 1e-4)
            assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_rows(lg))
            _, idx2 = thq.matmul_argmax(w, xb, want_logits=False)
            assert torch.equal(idx, idx2)


def test_affine_gate_up_every_route():
    for si, (h, k) in enumerate([(37, 64), (131, 320), (66, 768)]):
        wq, sb = rand_qlin_fast(2 * h, k, seed=500 + si)
        w = thq.QTensor.from_affine(wq, sb, 2 * h, k)
        for m in MS:
            print(f"[sweep] affine gate/up h={h} k={k} m={m}", flush=True)
            xf = O.bf16_round(activations(m, k, seed=m + 17))
            want = O.bf16_bits_to_f32(O.gate_up_silu(O.affine_matmul(wq, sb, 2 * h, k, xf)))
            xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
            run_case(f"affine gate/up {h}x{k} m={m}", thq.gate_up_silu(w, xb, torch.float32).cpu().numpy(), want, 1e-2)


def test_affine_every_route():
    # K = 64 and 320 are not whole 256-wide tiles (exact generic kernel); 768 is
    for si, (n, k) in enumerate([(37, 64), (131, 320), (66, 768)]):
        wq, sb = rand_qlin_fast(n, k, seed=400 + si)
        w = thq.QTensor.from_affine(wq, sb, n, k)
        for m in MS:
            print(f"[sweep] affine n={n} k={k} m={m}", flush=True)
            xf = O.bf16_round(activations(m, k, seed=m + 13))
            ref = O.affine_matmul(wq, sb, n, k, xf)
            xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
            run_case(f"affine {n}x{k} m={m}", thq.matmul(w, xb, torch.float32).cpu().numpy(), ref, 1e-2)
            if m in (1, 9):
                xd = torch.from_numpy(xf).cuda()
                run_case(f"affine f32 {n}x{k} m={m}", thq.matmul(w, xd, torch.float32).cpu().numpy(), ref, 1e-4)


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K])
def test_q8act_every_route(qtype):
    """THQ_MODE_Q8ACT (candle's default semantics) on the same shapes: within
    1e-5 of the oracle's Q8ACT matmul, and the quantize-once buffer gives the
    same bits; K past the mode's limit is an error, not a wrong answer."""
    dot = thq.Q8_0 if qtype == O.Q8_0 else thq.Q8_K
    for si, (n, k) in enumerate(SHAPES[qtype]):
        b, w = gguf_weight(qtype, n, k, seed=600 + si)
        for m in MS:
            if m * k > (1 << 21):
                continue
            print(f"[sweep] q8act qtype={qtype} n={n} k={k} m={m}", flush=True)
            xf = O.bf16_round(activations(m, k, seed=m + 19))
            xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
            try:
                y = thq.matmul(w, xb, torch.float32, flags=thq.MODE_Q8ACT)
            except thq.ThqError as e:
                assert e.code == thq.ESHAPE, e
                continue
            run_case(f"q8act q{qtype} {n}x{k} m={m}", y.cpu().numpy(), O.matmul(qtype, b, n, k, xf, O.MODE_Q8ACT),
                     1e-5)
            pre = thq.Q8Act(xb, dot)
            assert torch.equal(pre.matmul(w, torch.float32).view(torch.int32), y.view(torch.int32))


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_fused_argmax_every_route(qtype):
    """THQ_MODE_ARGMAX_FUSED gives the logits path's indices on every decode
    route (and on the shapes where no fused epilogue exists)."""
    for si, (n, k) in enumerate(SHAPES[qtype]):
        b, w = gguf_weight(qtype, n, k, seed=700 + si)
        for m in (1, 2, 3, 5, 8, 9):
            print(f"[sweep] fused argmax qtype={qtype} n={n} k={k} m={m}", flush=True)
            xb = torch.from_numpy(O.bf16_round(activations(m, k, seed=m + 23))).cuda().to(torch.bfloat16)
            _, fused = thq.matmul_argmax(w, xb, want_logits=False, flags=thq.MODE_ARGMAX_FUSED)
            logits, idx = thq.matmul_argmax(w, xb)
            assert torch.equal(fused, idx)
            assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_rows(logits.cpu().numpy()))


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_dequant_every_shape(qtype):
    for si, (n, k) in enumerate(SHAPES[qtype]):
        print(f"[sweep] dequant qtype={qtype} n={n} k={k}", flush=True)
        b, w = gguf_weight(qtype, n, k, seed=800 + si)
        got = w.dequantize().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), O.dequantize(qtype, b, n, k).view(np.uint32))


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_bf16_out_and_f32_gate_up_every_route(qtype):
    """bf16 outputs (RNE of the f32 accumulator) of thq_matmul, and gate/up
    with f32 activations, on the same routes."""
    for si, (n, k) in enumerate(SHAPES[qtype]):
        b, w = gguf_weight(qtype, n, k, seed=900 + si)
        h = n // 2
        for m in (1, 3, 9, 65):
            if m * k > (1 << 21):
                continue
            print(f"[sweep] bf16 out / f32 gate-up qtype={qtype} n={n} k={k} m={m}", flush=True)
            xf = O.bf16_round(activations(m, k, seed=m + 29))
            xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
            ref = O.matmul(qtype, b, n, k, xf)
            got = thq.matmul(w, xb, torch.bfloat16).float().cpu().numpy()
            run_case(f"bf16 out q{qtype} {n}x{k} m={m}", got, ref, 1e-2)
            if h > 0 and n % 2 == 0:
                xd = torch.from_numpy(xf).cuda()
                want = O.bf16_bits_to_f32(O.gate_up_silu(ref))
                run_case(f"f32 gate/up q{qtype} {h}x{k} m={m}",
                         thq.gate_up_silu(w, xd, torch.float32).cpu().numpy(), want, 1e-2)


@pytest.mark.parametrize("kind", ["q4_k", "affine"])
def test_exact_gemm_tile(kind):
    """THQ_MODE_EXACT_W past 64 rows of Q4_K / MLX affine: k_gemm's exact tile
    (bf16(128 + q) through the MFMA, each 32-wide sub-block's partial scaled
    in f32 with its x-row sums) on plans with K splits (4096 x 4096 at
    M = 300: 3 splits; 777 x 2048 at M = 129: 16, ragged M and N) and without
    (M = 1000, rows sampled): the f32 bar, 1e-4 of the row norm, and a bf16
    output and gate/up through the same tile."""
    for (n, k, m, rows) in ((4096, 4096, 300, None), (777, 2048, 129, None), (4096, 4096, 1000, 24)):
        print(f"[sweep] exact GEMM {kind} {n}x{k} m={m}", flush=True)
        if kind == "affine":
            wq, sb = rand_qlin_fast(n, k, seed=311)
            w = thq.QTensor.from_affine(wq, sb, n, k)
            ref_of = lambda xf: O.affine_matmul(wq, sb, n, k, xf)
        else:
            b, w = gguf_weight(O.Q4_K, n, k, seed=312)
            ref_of = lambda xf: O.matmul(O.Q4_K, b, n, k, xf)
        xf = O.bf16_round(activations(m, k, seed=500 + m))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        got = thq.matmul(w, xb, torch.float32, flags=thq.MODE_EXACT_W).cpu().numpy()
        sel = np.arange(m) if rows is None else np.linspace(0, m - 1, rows).astype(np.int64)
        ref = ref_of(np.ascontiguousarray(xf[sel]))
        run_case(f"exact GEMM {kind} {n}x{k} m={m}", got[sel], ref, 1e-4)
        if rows is None and m == 129:
            got16 = thq.matmul(w, xb, torch.bfloat16, flags=thq.MODE_EXACT_W).float().cpu().numpy()
            assert np.array_equal(got16.view(np.uint32), O.bf16_round(got).view(np.uint32))
    n, k, m = 2048, 2048, 200
    if kind == "affine":
        wq, sb = rand_qlin_fast(n, k, seed=313)
        w = thq.QTensor.from_affine(wq, sb, n, k)
    else:
        b, w = gguf_weight(O.Q4_K, n, k, seed=314)
    xf = O.bf16_round(activations(m, k, seed=77))
    xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
    y = thq.matmul(w, xb, torch.float32, flags=thq.MODE_EXACT_W).cpu().numpy()
    gu = thq.gate_up_silu(w, xb, torch.float32, flags=thq.MODE_EXACT_W).cpu().numpy()
    assert_close_elem(f"exact GEMM gate/up {kind}", gu, O.bf16_bits_to_f32(O.gate_up_silu(y)), 2.0 ** -7)


@pytest.mark.parametrize("kind", ["q4_k", "q6_k", "affine"])
def test_exact_weights_past_sixteen_rows(kind):
    """THQ_MODE_EXACT_W (the LM head's mode) with 4- / 6-bit weights past 16
    rows (the GEMMs round these weights to bf16): the wide exact GEMV at
    M = 17..64, the decode GEMV over groups of 16 rows beyond.  Exact weights
    leave only f32 summation error, so the bar is the f32 one (1e-4 of the
    row norm); gate/up and argmax through the same route."""
    n, k = 1000, 1024
    if kind == "affine":
        wq, sb = rand_qlin_fast(n, k, seed=301)
        w = thq.QTensor.from_affine(wq, sb, n, k)
        ref_of = lambda xf: O.affine_matmul(wq, sb, n, k, xf)
    else:
        qtype = O.Q4_K if kind == "q4_k" else O.Q6_K
        b, w = gguf_weight(qtype, n, k, seed=302)
        ref_of = lambda xf: O.matmul(qtype, b, n, k, xf)
    for m in (17, 31, 32, 33, 40, 64, 65, 80):
        print(f"[sweep] exact {kind} {n}x{k} m={m}", flush=True)
        xf = O.bf16_round(activations(m, k, seed=400 + m))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        ref = ref_of(xf)
        got = thq.matmul(w, xb, torch.float32, flags=thq.MODE_EXACT_W).cpu().numpy()
        run_case(f"exact {kind} m={m}", got, ref, 1e-4)
        logits, idx = thq.matmul_argmax(w, xb)
        torch.cuda.synchronize()
        lg = logits.cpu().numpy()
        run_case(f"exact {kind} argmax logits m={m}", lg, ref, 1e-4)
        assert list(idx.cpu().numpy()) == list(O.argmax_rows(lg))
        if m in (17, 40, 80):
            gu = thq.gate_up_silu(w, xb, torch.float32, flags=thq.MODE_EXACT_W).cpu().numpy()
            want = O.bf16_bits_to_f32(O.gate_up_silu(got))
            # the epilogue over the route's own (exact) gate/up values: at most one bf16 step apart
            assert_close_elem(f"gate/up {kind} m={m}", gu, want, 2.0 ** -7)
