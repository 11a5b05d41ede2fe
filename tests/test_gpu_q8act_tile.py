"""THQ_MODE_Q8ACT on the Q4_K tile plane (k_q8act_q4t in k_gemv_tile.hip):
2..8 activation rows of a weight that carries a tile plane
(thq_weight_add_tiles) take int8 MFMAs over Q8_K activations.

[ext] candle-core 0.11 k_quants::matmul: each activation row is quantized to
Q8_K (BlockQ8K::from_float), then BlockQ4K::vec_dot forms per superblock the
exact integers sum_j sc_j (q4 . q8)_j and sum_j m_j bsum_j and scales them in
f32.  The bar is the one of the row-quad Q8ACT kernel: 1e-5 of the row norm
against the oracle's Q8ACT matmul, since the integers are exact and only the
f32 order of the superblock sums differs.

Shapes cover a ragged last tile, an odd superblock count (a wave's second
superblock past K), K split across blocks with the last-block reduce, with the
separate reduce (thq_matmul_noalloc) and in the prepared-buffer calls, f32 and
bf16 activations and outputs, and gate/up.  The tile route and the row-quad
kernel (the same bytes without a tile plane) agree to the same bar; the
prepared buffer gives exactly the bits of the one-call form.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, assert_close_elem, rel_row_err, weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def tonp(t):
    return t.float().cpu().numpy()


def pair(n, k, seed):
    """The same Q4_K bytes as a weight with a tile plane and one without."""
    b = weight_bytes(O.Q4_K, n, k, seed=seed)
    wt = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k).add_tiles()
    wr = thq.QTensor.from_gguf_bytes(O.Q4_K, b, n, k)
    return b, wt, wr


def xin(m, k, seed, act):
    x = activations(m, k, seed=seed)
    if act == "bf16":
        x = O.bf16_round(x)
        return x, torch.from_numpy(x).cuda().to(torch.bfloat16)
    return x, torch.from_numpy(x).cuda()


# (n, k, rows): one split of 8-wave blocks; ragged last tile with many splits
# (10 tiles x 24 splits); 11 superblocks (the last wave's second superblock
# is past K); 64 superblocks; the decode shapes of a Qwen3-8B-class layer
# and 2-wave blocks over a ragged last tile
CASES = [
    (1024, 4096, (2, 3, 8)),
    (9000, 1024, (2, 8)),
    (301, 12288, (4,)),
    (130, 2816, (2, 7)),
    (66, 16384, (5,)),
    (12288, 4096, (3, 8)),
    (4096, 12288, (5, 8)),
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_q8act_tile_matches_oracle(case, act):
    n, k, rows = CASES[case]
    b, wt, wr = pair(n, k, seed=1500 + case)
    for m in rows:
        x, xt = xin(m, k, 1550 + m, act)
        ref = O.matmul(O.Q4_K, b, n, k, x, O.MODE_Q8ACT)
        y = tonp(thq.matmul(wt, xt, torch.float32, flags=thq.MODE_Q8ACT))
        err = rel_row_err(y, ref)
        assert err <= 1e-5, (n, k, m, err)
        assert_close_elem(f"q8act tile {n}x{k} m={m}", y, ref, 2.0 ** -14)
        # the row-quad kernel over the same bytes
        yr = tonp(thq.matmul(wr, xt, torch.float32, flags=thq.MODE_Q8ACT))
        assert rel_row_err(y, yr) <= 1e-5
        # bf16 output: the f32 result rounded once
        yb = tonp(thq.matmul(wt, xt, torch.bfloat16, flags=thq.MODE_Q8ACT))
        assert np.array_equal(yb, O.bf16_round(y))


def test_q8act_tile_special_activations():
    """Zero rows, the -128 Q8_K maximum and half-way values, through the tile
    kernel: the quantizer's special cases reach the integer dots unchanged."""
    n, k = 256, 1024
    b, wt, _ = pair(n, k, seed=1600)
    x = np.zeros((4, k), np.float32)
    x[1, :32] = np.arange(32, dtype=np.float32) - 15.5
    x[1, 40] = -128.0
    x[2] = O.randn(3, 1, 1.0, (k,))
    x[3, 256:512] = 0.5
    x[3, 511] = -1.0
    xt = torch.from_numpy(x).cuda()
    y = tonp(thq.matmul(wt, xt, torch.float32, flags=thq.MODE_Q8ACT))
    ref = O.matmul(O.Q4_K, b, n, k, x, O.MODE_Q8ACT)
    assert np.all(y[0] == 0.0)
    assert rel_row_err(y, ref) <= 1e-5


@pytest.mark.parametrize("h,k,m", [(992, 1024, 3), (1024, 4096, 8), (256, 12288, 6)])
def test_q8act_tile_gate_up(h, k, m):
    """gate/up over the [gate; up] tile plane: silu(g) * u of the same
    integer dots (h = 992: 31 tiles per half; K = 12288: split partials of
    both halves)."""
    both = np.concatenate([weight_bytes(O.Q4_K, h, k, seed=1700), weight_bytes(O.Q4_K, h, k, seed=1701)])
    fused = thq.QTensor.from_gguf_bytes(O.Q4_K, both, 2 * h, k).add_tiles()
    xf = O.bf16_round(activations(m, k, seed=1702))
    xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
    gu = tonp(thq.matmul(fused, xb, torch.float32, flags=thq.MODE_Q8ACT))
    assert rel_row_err(gu, O.matmul(O.Q4_K, both, 2 * h, k, xf, O.MODE_Q8ACT)) <= 1e-5
    got = thq.gate_up_silu(fused, xb, torch.float32, flags=thq.MODE_Q8ACT)
    got16 = thq.gate_up_silu(fused, xb, torch.bfloat16, flags=thq.MODE_Q8ACT)
    # the epilogue silu(bf16 g) * bf16 u over the same gate / up sums, and
    # bf16 output rounds it once: against the oracle's epilogue the device
    # exp moves a bf16 output by one step at most
    want = O.bf16_bits_to_f32(O.gate_up_silu(gu))
    assert_close_elem(f"q8act tile gate/up {h}x{k} m={m}", tonp(got), want, 2.0 ** -7)
    assert torch.equal(got16, got.to(torch.bfloat16))
    assert (tonp(got16) == want).mean() > 0.99


@pytest.mark.parametrize("n,k,m", [(1024, 4096, 5), (301, 12288, 8)])
def test_q8act_tile_prepared_and_noalloc(n, k, m):
    """The prepared buffer (thq_matmul_q8act) runs the same tile kernel and
    split order: exactly the bits of thq_matmul(THQ_MODE_Q8ACT), and so does
    thq_matmul_noalloc, whose K splits are summed by the separate reduce."""
    b, wt, _ = pair(n, k, seed=1800)
    x, xt = xin(m, k, 1801, "bf16")
    want = thq.matmul(wt, xt, torch.float32, flags=thq.MODE_Q8ACT)
    pre = thq.Q8Act(xt, thq.Q8_K)
    got = pre.matmul(wt, torch.float32)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    thq.matmul_noalloc(wt, xt, y, flags=thq.MODE_Q8ACT)
    assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    assert rel_row_err(tonp(want), O.matmul(O.Q4_K, b, n, k, x, O.MODE_Q8ACT)) <= 1e-5


@pytest.mark.parametrize("h,k,m", [(1024, 1024, 3), (12288, 4096, 8), (512, 12288, 5)])
def test_q8act_tile_gate_up_emit(h, k, m):
    """thq_gate_up_silu_q8act_emit on a [gate; up] weight with a tile plane:
    y equals the tile kernel's thq_gate_up_silu_q8act output bit for bit, and
    the emitted buffer is byte-identical to thq_q8act_prepare of that y
    (K = 12288: split partials in the context workspace)."""
    both = np.concatenate([weight_bytes(O.Q4_K, h, k, seed=1900), weight_bytes(O.Q4_K, h, k, seed=1901)])
    fused = thq.QTensor.from_gguf_bytes(O.Q4_K, both, 2 * h, k).add_tiles()
    xb = torch.from_numpy(O.bf16_round(activations(m, k, seed=1902))).cuda().to(torch.bfloat16)
    pre = thq.Q8Act(xb, thq.Q8_K)
    for dt in (torch.bfloat16, torch.float32):
        want_y = pre.gate_up_silu(fused, dt)
        y, nxt = pre.gate_up_silu_emit(fused, dt)
        torch.cuda.synchronize()
        iv = torch.int16 if dt == torch.bfloat16 else torch.int32
        assert torch.equal(y.view(iv), want_y.view(iv))
        want = q8k_planes(thq.Q8Act(y, thq.Q8_K).buf, m, h)
        for got_p, want_p in zip(q8k_planes(nxt.buf, m, h), want):
            assert np.array_equal(got_p, want_p)


def q8k_planes(buf: torch.Tensor, m: int, k: int):
    """(xq [m][k] i8, xd [m][k/256] f32 bits, xb [m][k/32] i16) of a Q8_K
    activation buffer, each plane starting on a 256-byte boundary (the
    padding between them is not part of the operand)."""
    a = lambda b: (b + 255) // 256 * 256
    raw = buf.cpu().numpy()
    o1 = a(m * k)
    o2 = o1 + a(m * (k // 256) * 4)
    return (raw[:m * k].view(np.int8), raw[o1:o1 + m * (k // 256) * 4].view(np.uint32),
            raw[o2:o2 + m * (k // 32) * 2].view(np.int16))
