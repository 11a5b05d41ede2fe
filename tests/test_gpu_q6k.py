"""GPU parity of the Q6_K path (GGML type 14, the type a Q4_K_M file keeps its
output head and part of ffn_down / attn_v in).

The oracle is thq_oracle.c's o_dequantize_q6_k and matmul. tests/test_oracle.py
pins it with literal block bytes and an independent numpy decode. The weights
are random Q6_K bytes: every 6-bit code, scales from -128 to 127, and d of
both signs including f16 subnormals (helpers.q6k_bytes).

The bars are as follows:
  - Upload / download / device upload / fuse round-trip the GGUF bytes exactly.
  - Dequantization is bit-exact: f32 against the oracle, and bf16 is the RNE
    of that f32.
  - The weights stay exact in the M = 1 GEMV and the generic kernel (M = 2..8,
    f32 x): the f32 bar of 1e-4 of the row L2 norm applies to bf16 and f32
    activations alike, and so does the per-element bound
    2^-12 * max(|want|, 0.02 max|want|). bf16 outputs get the reference's
    2^-7 per element.
  - The MFMA GEMM (M > 8, bf16 x) rounds dequantized weights to bf16. It
    equals the f64 product with bf16(dequant) weights to 1e-5 of the row
    norm, and the exact product to 1e-2 of the row norm and, per element, to
    2^-6 of that dot product's rounding-error scale sqrt(sum (x w)^2).
  - For argmax, indices are bit-exact against the argmax of the returned
    logits.
  - At the full LM-head shape (151936 x 4096), the check is against the f32
    product with the library's own exact dequantization, at 1e-4 of the row
    norm.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import activations, assert_close_dot, assert_close_elem, q6k_bytes, rel_row_err

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


def xdev(x, bf16=True):
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    return t.to(torch.bfloat16) if bf16 else t


@pytest.mark.parametrize("n,k", [(37, 256), (300, 2816), (64, 4096)])
def test_q6k_roundtrip_and_dequant(n, k):
    raw = q6k_bytes(n, k, seed=1)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    assert w.dtype == thq.Q6_K and w.shape == (n, k) and w.nbytes == raw.size
    assert np.array_equal(w.data(), raw)
    # from device memory too
    wd = thq.QTensor.from_gguf_bytes(thq.Q6_K, torch.from_numpy(raw.ravel()).cuda(), n, k)
    assert np.array_equal(wd.data(), raw)
    want = O.dequantize(O.Q6_K, raw, n, k)
    got = tonp(w.dequantize())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = w.dequantize_bf16().view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got16, O.f32_to_bf16_bits(want))


def test_q6k_special_d_values():
    """d = 0, +-f16 subnormals, +-max f16: the dequantized f32 equals the
    oracle's bit for bit (and a zero d block contributes exact zeros)."""
    n, k = 8, 512
    raw = q6k_bytes(n, k, seed=2).copy().reshape(n, k // 256, 210)
    specials = np.array([0.0, -0.0, 6e-8, -6e-8, 3e-5, 65504.0, -65504.0, 1.0], dtype=np.float16)
    raw[:, 0, 208:210] = specials.view(np.uint8).reshape(n, 2)
    raw = raw.reshape(n, -1)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    want = O.dequantize(O.Q6_K, raw, n, k)
    got = tonp(w.dequantize())
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not got[0, :256].any()


SHAPES = [
    (37, 256),      # one superblock: most lanes of the 4096 chunk are masked
    (300, 2816),    # 11 superblocks, ragged row groups
    (1024, 4096),   # attn_v of Qwen3-8B
    (4096, 12288),  # ffn_down of Qwen3-8B (three 4096 chunks)
    (130, 8192),
    (66, 16384),    # the largest K of the M = 1 kernel
]


@pytest.mark.parametrize("n,k", SHAPES)
def test_q6k_gemv_m1(n, k):
    raw = q6k_bytes(n, k, seed=3)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    x = O.bf16_round(activations(1, k, seed=4))
    want = O.matmul(O.Q6_K, raw, n, k, x)
    y = tonp(thq.matmul(w, xdev(x), torch.float32))
    assert rel_row_err(y, want) <= 1e-4
    assert_close_elem(f"q6k m=1 {n}x{k}", y, want, 2.0 ** -12)
    yb = tonp(thq.matmul(w, xdev(x), torch.bfloat16))
    assert_close_elem(f"q6k m=1 bf16 {n}x{k}", yb, want, 2.0 ** -7)
    # f32 activations: the exact generic kernel
    xf = activations(1, k, seed=5)
    yf = tonp(thq.matmul(w, xdev(xf, bf16=False), torch.float32))
    assert rel_row_err(yf, O.matmul(O.Q6_K, raw, n, k, xf)) <= 1e-4


@pytest.mark.parametrize("m", [2, 5, 8, 9, 16])
@pytest.mark.parametrize("n,k", [(300, 2816), (1024, 4096)])
def test_q6k_matmul_m_2_to_16(n, k, m):
    raw = q6k_bytes(n, k, seed=6)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    x = O.bf16_round(activations(m, k, seed=7))
    want = O.matmul(O.Q6_K, raw, n, k, x)
    y = tonp(thq.matmul(w, xdev(x), torch.float32))
    assert rel_row_err(y, want) <= 1e-4
    assert_close_elem(f"q6k m={m} {n}x{k}", y, want, 2.0 ** -12)


@pytest.mark.parametrize("m", [17, 64, 300])
@pytest.mark.parametrize("n,k", [(300, 2816), (4096, 12288)])
def test_q6k_gemm(n, k, m):
    """M > 16 with bf16 x: from 33 rows the MFMA GEMM, dequantized weights
    rounded to bf16 on the tile, pinned to the f64 product with exactly those
    bf16 weights at 1e-5 of the row norm (17..32 rows take the exact-weight
    wide GEMV, pinned to the exact product at 1e-4); against the exact product the bound
    is 1e-2 of the row norm and, per element, 2^-6 of that dot product's own
    rounding-error scale sqrt(sum (x w)^2) (the random d of the test weights
    makes row norms vary, so a row-wide rms is no measure for one output);
    bf16 outputs add their own rounding.  All rows beyond the 16 the oracle
    checks are compared with the f32 product of the exact dequantization at
    1e-2 of the row norm."""
    raw = q6k_bytes(n, k, seed=18)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    x = O.bf16_round(activations(m, k, seed=19))
    rows = slice(0, min(m, 16))
    wdeq = O.dequantize(O.Q6_K, raw, n, k)
    want = O.matmul(O.Q6_K, raw, n, k, x[rows])
    # the tile's weights are exactly bf16(dequant): the kernel is pinned to the
    # f64 product with those weights at the f32 accumulation bar
    rounded = x[rows].astype(np.float64) @ O.bf16_round(wdeq).astype(np.float64).T
    for out_dtype in (torch.float32, torch.bfloat16):
        y = tonp(thq.matmul(w, xdev(x), out_dtype))
        assert rel_row_err(y[rows], want) <= 1e-2
        if out_dtype == torch.float32:
            if m <= 32:
                # 17..32 rows take the wide GEMV, exact weights: the f32 bar
                assert rel_row_err(y[rows], want) <= 1e-4
            else:
                assert rel_row_err(y[rows], rounded) <= 1e-5
            assert_close_dot(f"q6k gemm {n}x{k} m={m}", y[rows], want, x[rows], wdeq, 2.0 ** -6)
        else:
            assert_close_dot(f"q6k gemm bf16 {n}x{k} m={m}", y[rows], want, x[rows], wdeq, 2.0 ** -6, 2.0 ** -8)
        if m > 16:
            ref = (torch.from_numpy(x).cuda() @ w.dequantize().T).cpu().numpy()
            assert rel_row_err(y, ref) <= 1e-2


def test_q6k_gemm_prefill_and_gate_up():
    """M = 2048 on the down shape (a Q4_K_M file's Q6_K ffn_down at prefill)
    and the fused gate/up GEMM epilogue at M = 64."""
    n, k, m = 4096, 12288, 2048
    raw = q6k_bytes(n, k, seed=20)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    xt = torch.from_numpy(O.bf16_round(activations(m, k, seed=21))).cuda()
    y = thq.matmul(w, xt.to(torch.bfloat16), torch.float32)
    ref = xt @ w.dequantize().T
    assert rel_row_err(tonp(y), tonp(ref)) <= 1e-2
    half, k2, m2 = 520, 4096, 64
    g_raw, u_raw = q6k_bytes(half, k2, seed=22), q6k_bytes(half, k2, seed=23)
    fused = thq.QTensor.fuse([thq.QTensor.from_gguf_bytes(thq.Q6_K, g_raw, half, k2),
                              thq.QTensor.from_gguf_bytes(thq.Q6_K, u_raw, half, k2)])
    x2 = xdev(O.bf16_round(activations(m2, k2, seed=24)))
    gu = tonp(thq.matmul(fused, x2, torch.float32))
    got = tonp(thq.gate_up_silu(fused, x2, torch.bfloat16))
    assert_close_elem("q6k gemm gate/up vs own matmul", got, O.bf16_bits_to_f32(O.gate_up_silu(gu)), 2.0 ** -7)
    both = np.concatenate([g_raw, u_raw])
    want = O.matmul(O.Q6_K, both, 2 * half, k2, tonp(x2)[:8])
    assert rel_row_err(gu[:8], want) <= 1e-2


def test_q6k_unaligned_x_and_empty():
    n, k = 100, 1024
    raw = q6k_bytes(n, k, seed=8)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    x = O.bf16_round(activations(1, k, seed=9))
    buf = torch.zeros(k + 1, dtype=torch.bfloat16, device="cuda")
    buf[1:] = xdev(x)[0]
    y = tonp(thq.matmul(w, buf[1:].view(1, k), torch.float32))  # 2 B past 16: the generic kernel
    assert rel_row_err(y, O.matmul(O.Q6_K, raw, n, k, x)) <= 1e-4
    assert thq.matmul(w, torch.zeros((0, k), dtype=torch.bfloat16, device="cuda")).shape == (0, n)


@pytest.mark.parametrize("half,k,m", [(512, 4096, 1), (1000, 2816, 1), (258, 12288, 1), (512, 4096, 3)])
def test_q6k_gate_up(half, k, m):
    """Fused [gate; up] Q6_K weight: bf16(silu(g) * u) on the M = 1 kernel's
    row pairs (half = 1000 / 258: ragged groups of 2 outputs) and on the
    generic kernel (m = 3)."""
    g_raw, u_raw = q6k_bytes(half, k, seed=10), q6k_bytes(half, k, seed=11)
    wg = thq.QTensor.from_gguf_bytes(thq.Q6_K, g_raw, half, k)
    wu = thq.QTensor.from_gguf_bytes(thq.Q6_K, u_raw, half, k)
    fused = thq.QTensor.fuse([wg, wu])
    both = np.concatenate([g_raw, u_raw])
    assert np.array_equal(fused.data(), both)
    x = O.bf16_round(activations(m, k, seed=12))
    gu = tonp(thq.matmul(fused, xdev(x), torch.float32))
    assert rel_row_err(gu, O.matmul(O.Q6_K, both, 2 * half, k, x)) <= 1e-4
    got = tonp(thq.gate_up_silu(fused, xdev(x), torch.bfloat16))
    want_own = O.bf16_bits_to_f32(O.gate_up_silu(gu))
    assert_close_elem(f"q6k gate/up {half}x{k} m={m}", got, want_own, 2.0 ** -7)
    want = O.bf16_bits_to_f32(O.gate_up_silu(O.matmul(O.Q6_K, both, 2 * half, k, x)))
    assert_close_elem(f"q6k gate/up vs oracle {half}x{k} m={m}", got, want, 2.0 ** -7)


def test_q6k_lm_head_argmax():
    n, k = 20000, 4096
    raw = q6k_bytes(n, k, seed=13)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, n, k)
    x = O.bf16_round(activations(2, k, seed=14))
    logits, idx = thq.matmul_argmax(w, xdev(x))
    lg = tonp(logits)
    assert rel_row_err(lg, O.matmul(O.Q6_K, raw, n, k, x)) <= 1e-4
    assert np.array_equal(idx.cpu().numpy().astype(np.uint32), O.argmax_rows(lg))


def test_q6k_full_lm_head_shape():
    """151936 x 4096 at M = 1 (the Qwen3 output head): against the f32 product
    with the library's exact dequantization, and argmax on the same logits."""
    n, k = 151936, 4096
    rng = np.random.default_rng(5)
    raw = torch.from_numpy(rng.integers(0, 256, (n, (k // 256) * 210), dtype=np.uint8)).cuda()
    blk = raw.view(n, k // 256, 210)
    d = torch.from_numpy((rng.standard_normal((n, k // 256)) * 2e-4).astype(np.float16)).cuda()
    blk[:, :, 208:210] = d.view(torch.uint8).view(n, k // 256, 2)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw.view(-1), n, k)
    del raw, blk
    x = xdev(O.bf16_round(activations(1, k, seed=15)))
    y = thq.matmul(w, x, torch.float32)
    wd = w.dequantize()
    ref = (x.float().double() @ wd.double().T).float()
    del wd
    assert rel_row_err(tonp(y), tonp(ref)) <= 1e-4
    logits, idx = thq.matmul_argmax(w, x)
    assert torch.equal(logits, y)
    assert int(idx[0]) == int(O.argmax_rows(tonp(logits))[0])


def test_q6k_errors():
    raw = q6k_bytes(8, 512, seed=16)
    w = thq.QTensor.from_gguf_bytes(thq.Q6_K, raw, 8, 512)
    x = xdev(activations(1, 512, seed=17))
    with pytest.raises(thq.ThqError) as e:
        thq.matmul(w, x, flags=thq.MODE_Q8ACT)
    assert e.value.code == thq.EDTYPE
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.quantize(torch.zeros((8, 512), device="cuda"), thq.Q6_K)
    assert e.value.code == thq.EDTYPE
    dev = torch.from_numpy(np.concatenate([np.zeros(1, np.uint8), raw.ravel()])).cuda()
    with pytest.raises(thq.ThqError) as e:  # an odd address: the f16 d would be split
        thq.QTensor.from_gguf_bytes(thq.Q6_K, dev[1:], 8, 512)
    assert e.value.code == thq.EALIGN
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.from_gguf_bytes(thq.Q6_K, raw[:, :200], 8, 500)
    assert e.value.code == thq.ESHAPE
    q4 = thq.QTensor.quantize(torch.zeros((8, 512), device="cuda"), thq.Q4_K)
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.fuse([w, q4])
    assert e.value.code == thq.EDTYPE
