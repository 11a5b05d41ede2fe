"""GPU parity of THQ_MODE_Q8ACT (candle's default CPU matmul semantics).

[ext] candle-core 0.11 k_quants::matmul quantizes each activation row to the
weight's dot type (BlockQ8_0::from_float for Q8_0 weights, BlockQ8K::from_float
for Q4_K weights), then takes exact integer block dots scaled in f32.

The bars are as follows:
  - thq_quantize_act is bit-exact against the oracle's restatement of both
    quantizers (GGML block bytes compared), including zero blocks, NaNs,
    opposite-sign ties and half-way rounding.
  - thq_matmul(THQ_MODE_Q8ACT) matches the oracle's Q8ACT matmul to 1e-5 of
    the row norm. The integer parts are exact, so only the f32 order of the
    block sums differs: ten times tighter than the f32 bar of 1e-4.
  - It stays within the f32 / bf16 bars of the exact (DEQUANT_F32) result
    only loosely. Q8 activations cost accuracy, which is candle's behaviour,
    so that check is 1e-2.
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


def edge_rows(k: int) -> np.ndarray:
    """Rows that exercise the quantizers' special cases (k >= 512)."""
    rows = np.zeros((4, k), np.float32)
    # row 0 stays zero: d = 0, all quants 0
    # row 1: amax = 127 in the first 32-block (d = 1: x.5 rounds away from zero)
    #        and max = -128 in the first 256-block (iscale = 1 for Q8_K)
    rows[1, :32] = np.arange(32, dtype=np.float32) - 15.5
    rows[1, 31] = 127.0
    rows[1, 40] = -128.0
    rows[1, 41:64] = np.arange(23, dtype=np.float32) + 0.5
    # row 2: opposite-sign ties (the first of equal magnitudes is the Q8_K max)
    rows[2, 3] = 2.0
    rows[2, 7] = -2.0
    rows[2, 300] = -3.0
    rows[2, 301] = 3.0
    rows[2, 256:300] = 0.25
    # row 3: NaNs (never the max; Q8_0 quantizes NaN to 0, Q8_K to 127)
    rows[3] = O.randn(9, 3, 1.0, (k,))
    rows[3, 5] = np.nan
    rows[3, 260] = np.nan
    rows[3, 480:512] = np.nan  # a Q8_0 block of NaNs only
    return rows


def oracle_q8(dot_type: int, x: np.ndarray) -> np.ndarray:
    rows = [O.quantize_q8_0_row(r) if dot_type == thq.Q8_0 else O.quantize_q8_k(r) for r in x]
    return np.stack(rows)


@pytest.mark.parametrize("dot_type", [thq.Q8_0, thq.Q8_K])
@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_quantize_act_bit_exact(dot_type, act):
    k = 4096
    x = np.concatenate([edge_rows(k), activations(5, k, seed=21)])
    if act == "bf16":
        x = O.bf16_round(x)
        xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    else:
        xt = torch.from_numpy(x).cuda()
    got = thq.quantize_act(xt, dot_type).cpu().numpy()
    want = oracle_q8(dot_type, x)
    assert got.shape == want.shape
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} bytes differ; first (row, byte) {tuple(bad[0])}"


def q8act_ref(qtype, b, n, k, x):
    return O.matmul(qtype, b, n, k, x, O.MODE_Q8ACT)


CASES = [
    (O.Q8_0, 3072, 1024, 1),   # the Q8_0 single-matmul shape
    (O.Q8_0, 3072, 1024, 5),
    (O.Q8_0, 100, 1056, 3),    # K chunk of 1024 + one block
    (O.Q8_0, 257, 2048, 17),   # two row tiles of 8 plus one row
    (O.Q4_K, 1024, 4096, 1),
    (O.Q4_K, 1024, 4096, 3),
    (O.Q4_K, 1024, 4096, 8),
    (O.Q4_K, 1024, 4096, 13),
    (O.Q4_K, 130, 2816, 2),    # 11 superblocks: a partial 4096 chunk
    (O.Q4_K, 301, 12288, 4),   # row tiles limited by LDS (4 rows of 12288)
    (O.Q4_K, 66, 16384, 9),
]


@pytest.mark.parametrize("qtype,n,k,m", CASES)
@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_q8act_matmul_matches_oracle(qtype, n, k, m, act):
    b = weight_bytes(qtype, n, k, seed=2)
    w = thq.QTensor.from_gguf_bytes(qtype, b, n, k)
    x = activations(m, k, seed=8)
    if act == "bf16":
        x = O.bf16_round(x)
        xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    else:
        xt = torch.from_numpy(x).cuda()
    y = tonp(thq.matmul(w, xt, torch.float32, flags=thq.MODE_Q8ACT))
    ref = q8act_ref(qtype, b, n, k, x)
    err = rel_row_err(y, ref)
    assert err <= 1e-5, err
    assert_close_elem(f"q8act {qtype} {n}x{k} m={m}", y, ref, 2.0 ** -14)
    # Q8 activations stay close to the exact product (candle's accuracy)
    assert rel_row_err(y, O.matmul(qtype, b, n, k, x, O.MODE_DEQUANT_F32)) <= 1e-2


@pytest.mark.parametrize("qtype,n,k,m", [(O.Q4_K, 1000, 1024, 1), (O.Q4_K, 1000, 1024, 6), (O.Q8_0, 1000, 1024, 3)])
def test_q8act_gate_up(qtype, n, k, m):
    """Fused gate/up in Q8ACT mode: the epilogue over the same integer dots.
    h = 1000 outputs is not a multiple of 4 x 4-output waves (ragged)."""
    bg = weight_bytes(qtype, n, k, seed=31)
    bu = weight_bytes(qtype, n, k, seed=32)
    both = np.concatenate([bg, bu])
    fused = thq.QTensor.from_gguf_bytes(qtype, both, 2 * n, k)
    xf = O.bf16_round(activations(m, k, seed=33))
    xb = torch.from_numpy(xf).cuda().to(torch.bfloat16)
    gu = tonp(thq.matmul(fused, xb, torch.float32, flags=thq.MODE_Q8ACT))
    assert rel_row_err(gu, q8act_ref(qtype, both, 2 * n, k, xf)) <= 1e-5
    got = tonp(thq.gate_up_silu(fused, xb, torch.bfloat16, flags=thq.MODE_Q8ACT))
    # same integer dots and summation tree as the plain matmul: only the
    # device exp can move a value by one bf16 step
    want = O.bf16_bits_to_f32(O.gate_up_silu(gu))
    assert_close_elem(f"q8act gate/up m={m}", got, want, 2.0 ** -7)
    assert (got == want).mean() > 0.99


def test_q8act_argmax_and_bf16_out():
    n, k, m = 5000, 1024, 3
    b = weight_bytes(O.Q8_0, n, k, seed=41)
    w = thq.QTensor.from_gguf_bytes(O.Q8_0, b, n, k)
    x = activations(m, k, seed=42)
    xt = torch.from_numpy(x).cuda()
    logits, idx = thq.matmul_argmax(w, xt, flags=thq.MODE_Q8ACT)
    ref = q8act_ref(O.Q8_0, b, n, k, x)
    assert rel_row_err(tonp(logits), ref) <= 1e-5
    assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_rows(tonp(logits)))
    # internal logits (NULL): the workspace holds both the quantized rows and the logits
    _, idx2 = thq.matmul_argmax(w, xt, want_logits=False, flags=thq.MODE_Q8ACT)
    assert torch.equal(idx, idx2)
    yb = tonp(thq.matmul(w, xt, torch.bfloat16, flags=thq.MODE_Q8ACT))
    assert np.array_equal(yb, O.bf16_round(tonp(logits)))


def test_q8act_errors():
    b = weight_bytes(O.Q8_0, 64, 1024, seed=1)
    w = thq.QTensor.from_gguf_bytes(O.Q8_0, b, 64, 1024)
    buf = torch.zeros(1025, device="cuda")
    with pytest.raises(thq.ThqError) as e:  # x starts 4 bytes past a 16-byte boundary
        thq.matmul(w, buf[1:].view(1, 1024), flags=thq.MODE_Q8ACT)
    assert e.value.code == thq.EALIGN
    with pytest.raises(thq.ThqError) as e:
        thq.quantize_act(torch.zeros((1, 1000), device="cuda"), thq.Q8_K)
    assert e.value.code == thq.ESHAPE
    with pytest.raises(thq.ThqError) as e:
        thq.quantize_act(torch.zeros((1, 1024), device="cuda"), thq.Q4_K)
    assert e.value.code == thq.EDTYPE


@pytest.mark.parametrize("dot_type,qtype,shapes", [
    (thq.Q8_K, O.Q4_K, [(1024, 4096), (256, 4096), (512, 4096)]),   # q / k / v of one input
    (thq.Q8_0, O.Q8_0, [(3072, 1024), (1000, 1024)]),
])
@pytest.mark.parametrize("m", [1, 5, 13])
def test_q8act_prepared_once_bit_identical(dot_type, qtype, shapes, m):
    """thq_q8act_prepare quantizes x once; every projection that reads the
    buffer gives exactly the bits of thq_matmul with THQ_MODE_Q8ACT."""
    k = shapes[0][1]
    x = O.bf16_round(activations(m, k, seed=51))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    pre = thq.Q8Act(xt, dot_type)
    for i, (n, kk) in enumerate(shapes):
        w = thq.QTensor.from_gguf_bytes(qtype, weight_bytes(qtype, n, kk, seed=60 + i), n, kk)
        for dt in (torch.float32, torch.bfloat16):
            want = thq.matmul(w, xt, dt, flags=thq.MODE_Q8ACT)
            got = pre.matmul(w, dt)
            assert torch.equal(got.view(torch.int16) if dt == torch.bfloat16 else got.view(torch.int32),
                               want.view(torch.int16) if dt == torch.bfloat16 else want.view(torch.int32))


def test_q8act_prepared_gate_up_and_errors():
    n, k, m = 1000, 1024, 3
    both = np.concatenate([weight_bytes(O.Q4_K, n, k, seed=71), weight_bytes(O.Q4_K, n, k, seed=72)])
    fused = thq.QTensor.from_gguf_bytes(O.Q4_K, both, 2 * n, k)
    xt = torch.from_numpy(O.bf16_round(activations(m, k, seed=73))).cuda().to(torch.bfloat16)
    pre = thq.Q8Act(xt, thq.Q8_K)
    want = thq.gate_up_silu(fused, xt, torch.bfloat16, flags=thq.MODE_Q8ACT)
    assert torch.equal(pre.gate_up_silu(fused).view(torch.int16), want.view(torch.int16))
    # a Q8_0 weight needs a Q8_0 buffer; K must match
    w8 = thq.QTensor.from_gguf_bytes(O.Q8_0, weight_bytes(O.Q8_0, 64, 1024, seed=74), 64, 1024)
    with pytest.raises(thq.ThqError) as e:
        pre.matmul(w8)
    assert e.value.code == thq.EDTYPE
    w4 = thq.QTensor.from_gguf_bytes(O.Q4_K, weight_bytes(O.Q4_K, 64, 2048, seed=75), 64, 2048)
    with pytest.raises(thq.ThqError) as e:
        pre.matmul(w4)
    assert e.value.code == thq.ESHAPE
    buf = torch.empty(thq.lib.thq_q8act_bytes(thq.Q8_K, m, k) + 256, dtype=torch.uint8, device="cuda")
    rc = thq.lib.thq_q8act_prepare(pre.ctx.h, thq.Q8_K, thq._ptr(xt), thq.ACT_BF16, m, k,
                                   thq.C.c_void_p(buf.data_ptr() + 16), None)
    assert rc == thq.EALIGN


def q8k_planes(buf: torch.Tensor, m: int, k: int):
    """(xq [m][k] i8, xd [m][k/256] f32, xb [m][k/32] i16) of an activation
    buffer: the three planes, each starting on a 256-byte boundary."""
    a = lambda b: (b + 255) // 256 * 256
    raw = buf.cpu().numpy()
    o1 = a(m * k)
    o2 = o1 + a(m * (k // 256) * 4)
    xq = raw[:m * k].view(np.int8).reshape(m, k)
    xd = raw[o1:o1 + m * (k // 256) * 4].view(np.float32).reshape(m, k // 256)
    xb = raw[o2:o2 + m * (k // 32) * 2].view(np.int16).reshape(m, k // 32)
    return xq, xd, xb


@pytest.mark.parametrize("h,k,ms", [(256, 512, (1, 3)), (1024, 1024, (9, 2)), (12288, 4096, (1, 8, 5)),
                                    (2048, 1024, (40, 17))])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gate_up_emits_down_operand(h, k, ms, out_dtype):
    """The emitting gate/up (thq_gate_up_silu_q8act_emit) writes the same y
    as the plain one and, as the next projection's operand, the Q8_K planes
    of that y: byte-identical to thq_q8act_prepare(y) and to the oracle's
    BlockQ8K::from_float of y.  Several M in a row on one context (the
    arrival counters must come back to zero after each launch), and the down
    projection consumes the emitted buffer exactly as a prepared one."""
    fused = thq.QTensor.from_gguf_bytes(
        thq.Q4_K, np.concatenate([weight_bytes(O.Q4_K, h, k, seed=31), weight_bytes(O.Q4_K, h, k, seed=32)]), 2 * h, k)
    down = thq.QTensor.from_gguf_bytes(thq.Q4_K, weight_bytes(O.Q4_K, 384, h, seed=33), 384, h)
    for m in ms:
        print(f"emit h={h} k={k} m={m} {out_dtype}", flush=True)
        x = torch.from_numpy(activations(m, k, seed=m)).cuda().to(torch.bfloat16)
        a = thq.Q8Act(x, thq.Q8_K)
        y_plain = a.gate_up_silu(fused, out_dtype)
        y, nxt = a.gate_up_silu_emit(fused, out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(y, y_plain)
        prep = thq.Q8Act(y, thq.Q8_K)
        got = q8k_planes(nxt.buf, m, h)
        for g, w, name in zip(got, q8k_planes(prep.buf, m, h), ("xq", "xd", "xb")):
            assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), name
        blocks = O.quantize_q8_k(y.float().cpu().numpy().ravel()).reshape(m, h // 256, 292)
        assert np.array_equal(got[0].reshape(m, h // 256, 256).view(np.uint8), blocks[:, :, 4:260])
        assert np.array_equal(got[1].reshape(m, h // 256), blocks[:, :, 0:4].copy().view(np.float32)[..., 0])
        bs = blocks[:, :, 260:292].copy().view(np.int16).astype(np.int32).reshape(m, h // 256, 8, 2).sum(axis=3)
        assert np.array_equal(got[2].reshape(m, h // 256, 8).astype(np.int32), bs)
        assert torch.equal(nxt.matmul(down), prep.matmul(down))


def test_gate_up_emit_errors():
    L = thq.lib
    ctx = thq.Context.get(0).h
    k = 512
    odd = thq.QTensor.from_gguf_bytes(thq.Q4_K, weight_bytes(O.Q4_K, 2 * 200, k, seed=34), 2 * 200, k)
    q8 = thq.QTensor.from_gguf_bytes(thq.Q8_0, weight_bytes(O.Q8_0, 512, k, seed=35), 512, k)
    x = torch.zeros((2, k), dtype=torch.bfloat16, device="cuda")
    a = thq.Q8Act(x, thq.Q8_K)
    y = torch.zeros((2, 256), dtype=torch.bfloat16, device="cuda")
    nb = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    P = lambda t: t.data_ptr()
    assert L.thq_gate_up_silu_q8act_emit(ctx, odd.h, thq.Q8_K, P(a.buf), 2, k, P(y), thq.ACT_BF16, P(nb),
                                         None) == thq.ESHAPE  # 200 outputs: not a multiple of 256
    assert L.thq_gate_up_silu_q8act_emit(ctx, q8.h, thq.Q8_K, P(a.buf), 2, k, P(y), thq.ACT_BF16, P(nb),
                                         None) == thq.EDTYPE
    ok = thq.QTensor.from_gguf_bytes(thq.Q4_K, weight_bytes(O.Q4_K, 2 * 256, k, seed=36), 2 * 256, k)
    assert L.thq_gate_up_silu_q8act_emit(ctx, ok.h, thq.Q8_K, P(a.buf), 2, k, P(y), thq.ACT_BF16, P(nb) + 16,
                                         None) == thq.EALIGN
    assert L.thq_gate_up_silu_q8act_emit(ctx, ok.h, thq.Q8_K, P(a.buf), 2, k, P(y), thq.ACT_BF16, None,
                                         None) == thq.EINVAL
    assert L.thq_gate_up_silu_q8act_emit(ctx, ok.h, thq.Q8_0, P(a.buf), 2, k, P(y), thq.ACT_BF16, P(nb),
                                         None) == thq.EDTYPE  # Q4_K dots with Q8_K activations
    assert L.thq_gate_up_silu_q8act_emit(ctx, ok.h, thq.Q8_K, P(a.buf), 2, k, P(y), thq.ACT_BF16, P(nb),
                                         None) == thq.OK
