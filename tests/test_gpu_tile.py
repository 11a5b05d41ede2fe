"""Tile-plane decode GEMV (k_gemv_tile.hip): 3..8 bf16 activation rows of a
Q4_K or MLX affine weight that carries a 32-row tile plane
(thq_weight_add_tiles), against the oracle's exact-weight product.

Exact weights leave only f32 summation error, so the bar is the f32 one
(1e-4 of the row norm).  Shapes cover a ragged last tile (rows past N are
zero in the plane), K split across blocks (few output tiles) with the split
reduce, K = 12288 (three splits), the one-split 8-wave instance (12288 rows),
and MLX affine K that is not a multiple of 256 (zero padding groups, x
masked past K).  The tile route's plan exists for every case and agrees with
the row-layout kernels to f32 summation order; bf16 output is the f32 result
rounded once; the weight's GGUF bytes are unchanged; 1..2 and 9..16 rows and
gate/up halves that are not whole tiles keep their row-layout routes.  Gate/up
(silu(g)*u over the [gate; up] weight) on the tile plane matches the oracle's
epilogue and the row-layout kernels' outputs.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, assert_close_elem, rand_qlin_fast, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def make(kind, n, k, seed):
    if kind == "affine":
        wq, sb = rand_qlin_fast(n, k, seed=seed)
        return (thq.QTensor.from_affine(wq, sb, n, k), lambda xf: O.affine_matmul(wq, sb, n, k, xf), None)
    b = weight_bytes(O.Q4_K, n, k, seed=seed)
    return thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k), lambda xf: O.matmul(O.Q4_K, b, n, k, xf), b


# (n, k, rows): ragged last tile, 4 K splits; 2 splits; long K (3 splits);
# the 8-wave one-split instance; 2-wave blocks over a ragged last tile
# (9000 = 281.25 tiles)
CASES = [(1000, 1024, (3, 5, 8)), (4096, 4096, (3, 4, 8)), (300, 12288, (3, 8)), (12288, 4096, (3, 8)),
         (9000, 1024, (3, 8))]


@pytest.mark.parametrize("kind", ["q4_k", "affine"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_tile_matches_oracle(kind, case):
    n, k, rows = CASES[case]
    w, ref_of, _ = make(kind, n, k, seed=1300 + case)
    dtype = O.Q4_K if kind == "q4_k" else thq.MLX_Q4
    base = {}
    for m in rows:
        xf = O.bf16_round(activations(m, k, seed=1350 + m))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        base[m] = thq.matmul(w, xb, torch.float32)
    torch.cuda.synchronize()
    w.add_tiles()
    w.add_tiles()  # idempotent
    for m in rows:
        print(f"[tile] {kind} {n}x{k} m={m}", flush=True)
        assert thq.plan_gemv_tile(dtype, m, n, k).waves > 0
        xf = O.bf16_round(activations(m, k, seed=1350 + m))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        got = thq.matmul(w, xb, torch.float32)
        torch.cuda.synchronize()
        err = rel_row_err(got.cpu().numpy(), ref_of(xf))
        assert err <= 1e-4, f"{kind} {n}x{k} m={m}: max row error {err:.3g}"
        # both are exact-weight products: agreement to f32 summation order
        # (bit-equal where the row-layout MFMA GEMV sums in the same order)
        g, b = got.cpu().numpy(), base[m].cpu().numpy()
        assert rel_row_err(g, b.astype(np.float64)) <= 1e-5
        got16 = thq.matmul(w, xb, torch.bfloat16)
        assert torch.equal(got16, got.to(torch.bfloat16))


def test_tile_affine_ragged_k():
    # K = 1088: 4.25 superblocks, the last one's three padding groups are zero
    n, k = 200, 1088
    w, ref_of, _ = make("affine", n, k, seed=1390)
    w.add_tiles()
    for m in (3, 7):
        xf = O.bf16_round(activations(m, k, seed=1391 + m))
        got = thq.matmul(w, torch.from_numpy(xf).cuda().to(torch.bfloat16), torch.float32)
        torch.cuda.synchronize()
        err = rel_row_err(got.cpu().numpy(), ref_of(xf))
        assert err <= 1e-4, f"affine {n}x{k} m={m}: {err:.3g}"


def test_tile_keeps_bytes_and_other_routes():
    n, k = 512, 2048
    w, ref_of, b = make("q4_k", n, k, seed=1400)
    w.add_tiles()
    assert np.array_equal(w.data().ravel(), np.asarray(b).ravel())
    for m in (1, 2, 12, 16):
        xf = O.bf16_round(activations(m, k, seed=1410 + m))
        got = thq.matmul(w, torch.from_numpy(xf).cuda().to(torch.bfloat16), torch.float32)
        torch.cuda.synchronize()
        assert rel_row_err(got.cpu().numpy(), ref_of(xf)) <= 1e-4, f"m={m}"
    # gate/up halves that are not whole tiles (nout = 200) keep their own kernels
    bg, bu = weight_bytes(O.Q4_K, 200, k, seed=1420), weight_bytes(O.Q4_K, 200, k, seed=1421)
    fused = thq.QTensor.from_gguf_bytes(O.Q4_K, np.concatenate([bg, bu]), 400, k)
    fused.add_tiles()
    xf = O.bf16_round(activations(5, k, seed=1422))
    got = thq.gate_up_silu(fused, torch.from_numpy(xf).cuda().to(torch.bfloat16), torch.float32).cpu().numpy()
    want = O.bf16_bits_to_f32(O.gate_up_silu(O.matmul(O.Q4_K, np.concatenate([bg, bu]), 400, k, xf)))
    assert rel_row_err(got, want) <= 1e-2


# gate/up on the tile plane: (outputs per half, K, rows); one split of
# 4-wave blocks would not fill the GPU at 256 outputs, K = 12288 splits
GU_CASES = [(256, 2048, (3, 8)), (4096, 4096, (3, 5, 8)), (1024, 12288, (4, 8))]


@pytest.mark.parametrize("kind", ["q4_k", "affine"])
@pytest.mark.parametrize("case", range(len(GU_CASES)))
def test_tile_gate_up(kind, case):
    h, k, rows = GU_CASES[case]
    if kind == "affine":
        wq, sb = rand_qlin_fast(2 * h, k, seed=1460 + case)
        fused = thq.QTensor.from_affine(wq, sb, 2 * h, k)
        ref_of = lambda xf: O.affine_matmul(wq, sb, 2 * h, k, xf)
    else:
        b = np.concatenate([weight_bytes(O.Q4_K, h, k, seed=1460 + case), weight_bytes(O.Q4_K, h, k, seed=1470 + case)])
        fused = thq.QTensor.from_gguf_bytes(O.Q4_K, b, 2 * h, k)
        ref_of = lambda xf: O.matmul(O.Q4_K, b, 2 * h, k, xf)
    base = {}
    for m in rows:
        xf = O.bf16_round(activations(m, k, seed=1480 + m))
        base[m] = thq.gate_up_silu(fused, torch.from_numpy(xf).cuda().to(torch.bfloat16), torch.float32)
    fused.add_tiles()
    for m in rows:
        print(f"[tile gate/up] {kind} 2x{h}x{k} m={m}", flush=True)
        xf = O.bf16_round(activations(m, k, seed=1480 + m))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        got = thq.gate_up_silu(fused, xb, torch.float32)
        got16 = thq.gate_up_silu(fused, xb, torch.bfloat16)
        torch.cuda.synchronize()
        g = got.cpu().numpy()
        # the epilogue bf16(silu(bf16 g) * bf16 u) over the oracle's f64 gate / up
        want = O.bf16_bits_to_f32(O.gate_up_silu(ref_of(xf)))
        assert rel_row_err(g, want) <= 1e-2, f"{kind} m={m}"
        # against the row-layout kernels (exact weights too): the bf16-rounded
        # g and u agree except where f32 summation order crosses a rounding
        # boundary, one bf16 step of the output at most
        assert_close_elem(f"{kind} m={m} vs row layout", g, base[m].cpu().numpy(), 2.0 ** -7)
        assert torch.equal(got16, got.to(torch.bfloat16))


def test_tile_wrong_dtype():
    n, k = 64, 256
    w = thq.QTensor.from_gguf_bytes(O.Q8_0, weight_bytes(O.Q8_0, n, k, seed=1430), n, k)
    with pytest.raises(thq.ThqError) as e:
        w.add_tiles()
    assert e.value.code == thq.EDTYPE


@pytest.mark.parametrize("kind", ["q4_k", "affine"])
def test_tile_split_reduction_matches_reduce_launch(kind):
    # K split over blocks: thq_matmul sums the splits in the last block of
    # each tile (arrival counters), thq_matmul_noalloc with k_split_reduce;
    # both in split order, so bit for bit, on repeated calls (the counters
    # return to zero) and a smaller second M, f32 and bf16 outputs
    n, k = 4096, 12288
    w, ref_of, _ = make(kind, n, k, seed=1440)
    w.add_tiles()
    dtype = O.Q4_K if kind == "q4_k" else thq.MLX_Q4
    for m in (8, 3, 8):
        assert thq.plan_gemv_tile(dtype, m, n, k).splits > 1
        xf = O.bf16_round(activations(m, k, seed=1450 + m))
        xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
        for dt in (torch.float32, torch.bfloat16):
            print(f"[tile split] {kind} m={m} {dt}", flush=True)
            got = thq.matmul(w, xb, dt)
            ref = torch.empty_like(got)
            thq.matmul_noalloc(w, xb, ref)
            torch.cuda.synchronize()
            assert torch.equal(got, ref)
        err = rel_row_err(got.float().cpu().numpy(), ref_of(xf))
        assert err <= 1e-2
