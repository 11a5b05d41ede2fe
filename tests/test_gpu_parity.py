"""GPU parity: libthq's HIP kernels against the CPU oracle on identical bytes.

Tolerances (applied per row, max_n |y - ref| / ||ref[m, :]||):
  f32 activations   1e-4     bf16 activations   1e-2
plus a per-element bound in the style of the reference's qmvt assert_close
(engine/src/qwen35.rs:6946-6958) so that a single wrong output cannot hide
inside a row norm.  Dequantization and argmax indices are bit-exact.
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


def upload(qtype, n, k, seed=0):
    b = weight_bytes(qtype, n, k, seed)
    return b, thq.QTensor.from_gguf_bytes(qtype, b, n, k)


def bf16_x(m, k, seed=0):
    xf = O.bf16_round(activations(m, k, seed))
    return xf, torch.from_numpy(xf).to("cuda").to(torch.bfloat16)


def tonp(t):
    return t.float().cpu().numpy()


# ------------------------------------------------------------------ weights
@pytest.mark.parametrize("qtype,n,k", [(O.Q8_0, 3072, 1024), (O.Q4_K, 1024, 4096), (O.Q4_K, 300, 12288)])
def test_dequant_bit_exact(qtype, n, k):
    b, w = upload(qtype, n, k)
    got = tonp(w.dequantize())
    want = O.dequantize(qtype, b, n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_q4k_random_bytes_bit_exact():
    # every byte pattern of scales and nibbles, finite f16 d / dmin of both signs
    rng = np.random.default_rng(7)
    n, k = 64, 1024
    raw = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    d = (rng.standard_normal((n, k // 256, 2)) * 0.05).astype(np.float16)
    raw[:, :, 0:4] = d.view(np.uint8).reshape(n, k // 256, 4)
    raw = raw.reshape(n, -1)
    w = thq.QTensor.from_gguf_bytes(O.Q4_K, raw, n, k)
    got = tonp(w.dequantize())
    want = O.dequantize(O.Q4_K, raw, n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype,n,k", [(O.Q8_0, 1000, 4096), (O.Q8_0, 40, 800), (O.Q4_K, 1000, 4096),
                                        (O.Q4_K, 0, 0)])
def test_dequant_bf16_bit_exact(qtype, n, k):
    """thq_dequantize_bf16 (the dequantize-then-GEMM route's first step) is the
    oracle's f32 dequantization rounded to nearest even, bit for bit.  The
    Q4_K case with n = 0 takes random header and nibble bytes (96 x 2048):
    every 16-B nibble piece's two halves and both nibbles of each byte."""
    if n == 0:
        rng = np.random.default_rng(11)
        n, k = 96, 2048
        raw = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
        d = (rng.standard_normal((n, k // 256, 2)) * 0.05).astype(np.float16)
        raw[:, :, 0:4] = d.view(np.uint8).reshape(n, k // 256, 4)
        raw = raw.reshape(n, -1)
    else:
        raw = weight_bytes(qtype, n, k, 3)
    w = thq.QTensor.from_gguf_bytes(qtype, raw, n, k)
    got = w.dequantize_bf16().view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.f32_to_bf16_bits(O.dequantize(qtype, raw, n, k))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K])
def test_upload_download_roundtrip(qtype):
    b, w = upload(qtype, 257, 1024)
    assert np.array_equal(w.data(), b)
    # the device path (GGUF bytes already in HBM) gives the same weight
    dev = torch.from_numpy(b.ravel().copy()).to("cuda")
    w2 = thq.QTensor.from_gguf_bytes(qtype, dev, 257, 1024)
    assert np.array_equal(w2.data(), b)


@pytest.mark.parametrize("qtype,n,k", [(O.Q8_0, 512, 4096), (O.Q4_K, 512, 4096), (O.Q4_K, 33, 768)])
def test_device_quantizer_matches_oracle(qtype, n, k):
    wf = O.randn(5, 77, 0.02, (n, k))
    wf[0, :] = 0.0           # zero row
    wf[1, :256] = 0.125      # constant superblock
    wf[2, :32] = np.linspace(-1, 1, 32, dtype=np.float32)
    want = O.quantize(qtype, wf)
    q = thq.QTensor.quantize(torch.from_numpy(wf).to("cuda"), qtype)
    got = q.data()
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} bytes differ"


def test_fuse_concatenates_rows():
    b1, w1 = upload(O.Q4_K, 128, 512, seed=1)
    b2, w2 = upload(O.Q4_K, 64, 512, seed=2)
    f = thq.QTensor.fuse([w1, w2])
    assert f.shape == (192, 512)
    assert np.array_equal(f.data(), np.concatenate([b1, b2]))
    b3, w3 = upload(O.Q8_0, 96, 512, seed=3)
    b4, w4 = upload(O.Q8_0, 32, 512, seed=4)
    f2 = thq.QTensor.fuse([w3, w4])
    assert np.array_equal(f2.data(), np.concatenate([b3, b4]))
    with pytest.raises(thq.ThqError):
        thq.QTensor.fuse([w1, w3])


# ------------------------------------------------------------------ config 1
def test_q8_0_gemv_f32_activations():
    """Single Q8_0 matmul: X f32 [1, 1024], W [3072, 1024] ~ N(0, 0.02)."""
    n, k = 3072, 1024
    b, w = upload(O.Q8_0, n, k)
    x = activations(1, k)
    y = tonp(thq.matmul(w, torch.from_numpy(x).cuda(), torch.float32))
    ref = O.matmul(O.Q8_0, b, n, k, x, O.MODE_DEQUANT_F32)
    err = rel_row_err(y, ref)
    assert err <= 1e-4, err
    assert_close_elem("q8_0 m=1 f32", y, ref, 2.0 ** -14)
    # candle's default CPU mode quantizes x to Q8_0: further away, as expected
    assert rel_row_err(O.matmul(O.Q8_0, b, n, k, x, O.MODE_Q8ACT), ref) > err


# ------------------------------------------------------------------ config 2
@pytest.mark.parametrize("m", [1, 2, 4, 8])
@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_q4k_decode_gemv(m, n, k):
    b, w = upload(O.Q4_K, n, k)
    xf, xb = bf16_x(m, k)
    y = tonp(thq.matmul(w, xb, torch.float32))
    ref = O.matmul(O.Q4_K, b, n, k, xf, O.MODE_DEQUANT_F32)
    err = rel_row_err(y, ref)
    assert err <= 1e-2, err
    # decode paths (m <= 8) keep exact dequantized weights: only f32 summation order differs
    assert_close_elem(f"q4k gemv m={m}", y, ref, 2.0 ** -12)


@pytest.mark.parametrize("n,k", [(202, 8192), (130, 16384)])
def test_q4k_gemv_m1_k_split(n, k):
    """M = 1 decode GEMV with K split over 2 / 4 chunks per block (ragged row
    quads); also the fused gate/up form on the same weight."""
    b, w = upload(O.Q4_K, n, k, seed=4)
    xf, xb = bf16_x(1, k, seed=6)
    y = tonp(thq.matmul(w, xb, torch.float32))
    ref = O.matmul(O.Q4_K, b, n, k, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(y, ref) <= 1e-2
    assert_close_elem(f"q4k gemv m=1 {n}x{k}", y, ref, 2.0 ** -12)
    act = tonp(thq.gate_up_silu(w, xb, torch.float32))
    want = O.bf16_bits_to_f32(O.gate_up_silu(y))
    assert_close_elem(f"q4k gate/up m=1 {n}x{k}", act, want, 2.0 ** -7)


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q8_0])
@pytest.mark.parametrize("n,k", [(100, 256), (777, 1024), (300, 2816)])
@pytest.mark.parametrize("m", [2, 3, 8])
def test_skinny_gemv_shapes(qtype, n, k, m):
    """Decode GEMV on the matrix cores for 2 <= M <= 8 at small / odd K: one wave
    per block, K split across blocks, ragged row tiles; exact weights."""
    b, w = upload(qtype, n, k)
    xf, xb = bf16_x(m, k, seed=3)
    y = tonp(thq.matmul(w, xb, torch.float32))
    ref = O.matmul(qtype, b, n, k, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(y, ref) <= 1e-2
    assert_close_elem(f"skinny gemv qtype={qtype} {n}x{k} m={m}", y, ref, 2.0 ** -12)
    # the fused gate/up epilogue on the same shapes (rows split in two halves)
    if n % 2 == 0:
        act = tonp(thq.gate_up_silu(w, xb, torch.float32))
        want = O.bf16_bits_to_f32(O.gate_up_silu(y))
        assert_close_elem(f"skinny gate/up {n}x{k} m={m}", act, want, 2.0 ** -7)


# ------------------------------------------------------------------ config 3
@pytest.mark.parametrize("m", [128, 512, 2048])
@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_q4k_prefill_gemm(m, n, k):
    b, w = upload(O.Q4_K, n, k)
    xf, xb = bf16_x(m, k)
    y = thq.matmul(w, xb, torch.bfloat16)
    # every row: checksum of the row sums, sum_n y[m, n] = x[m] . (sum_n W[n])
    wsum = O.dequantize(O.Q4_K, b, n, k).astype(np.float64).sum(axis=0)
    yf = y.float()
    rows = yf.sum(dim=1).double().cpu().numpy()
    rms = yf.pow(2).mean(dim=1).sqrt().double().cpu().numpy()
    want_rows = xf.astype(np.float64) @ wsum
    # bf16 weight + output rounding noise sums to ~2e-3 sqrt(N) rms(y); 10x margin
    assert np.all(np.abs(rows - want_rows) <= 0.02 * np.sqrt(n) * rms)
    # sampled rows in full against the oracle
    rng = np.random.default_rng(m)
    pick = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 10)]))
    ref = O.matmul(O.Q4_K, b, n, k, xf[pick], O.MODE_DEQUANT_F32)
    got = tonp(y)[pick]
    assert rel_row_err(got, ref) <= 1e-2
    # bf16 output: one output rounding step (2^-8..2^-7 relative) on top of the
    # bf16 weight-rounding noise, so 2^-6 of max(|y|, rms(y))
    assert_close_elem(f"q4k gemm m={m}", got, ref, 2.0 ** -6, floor="rms")


@pytest.mark.parametrize("m", [9, 17, 33, 100])
def test_q4k_gemm_ragged_m(m):
    n, k = 1000, 2048  # ragged N tile too
    b, w = upload(O.Q4_K, n, k)
    xf, xb = bf16_x(m, k)
    y = tonp(thq.matmul(w, xb, torch.float32))
    ref = O.matmul(O.Q4_K, b, n, k, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(y, ref) <= 1e-2
    assert_close_elem(f"q4k ragged m={m}", y, ref, 2.0 ** -7, floor="rms")


@pytest.mark.parametrize("m", [3, 4])
def test_q4k_rows_3_4_wide(m):
    """3..4 bf16 rows over >= 12288 outputs take the MFMA decode GEMV instead
    of the row kernel (exact weights: the f32 accumulation bar)."""
    n, k = 12288, 1024
    b, w = upload(O.Q4_K, 2 * n, k, seed=5)
    xf, xb = bf16_x(m, k, seed=6)
    logits = O.matmul(O.Q4_K, b, 2 * n, k, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(tonp(thq.matmul(w, xb, torch.float32)), logits) <= 1e-4
    want = O.bf16_bits_to_f32(O.gate_up_silu(logits))
    assert rel_row_err(tonp(thq.gate_up_silu(w, xb, torch.float32)), want) <= 1e-2


@pytest.mark.parametrize("m", [128, 512])
def test_q4k_gemm_split_counts(m, monkeypatch):
    """The split-K machinery at the counts the planner can pick (up to 32 on
    small-N shapes): every forced count gives the unsplit result up to f32
    summation order (the split partials are summed in a fixed order).  The
    planner's own choice meets the 1e-2 row bar against the exact oracle and
    is pinned at the f32 accumulation bar to the f64 product with the tile's
    bf16-rounded weights (its per-element deviation from the exact product is
    that rounding: up to 0.0105 on rows of rms 1.29 here)."""
    n, k = 1024, 4096  # 8 column tiles: the planner splits K
    b, w = upload(O.Q4_K, n, k, seed=3)
    xf, xb = bf16_x(m, k, seed=4)
    y = tonp(thq.matmul(w, xb, torch.float32))
    ref = O.matmul(O.Q4_K, b, n, k, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(y, ref) <= 1e-2
    rounded = xf.astype(np.float64) @ O.bf16_round(O.dequantize(O.Q4_K, b, n, k)).astype(np.float64).T
    assert rel_row_err(y, rounded) <= 1e-5
    monkeypatch.setenv("THQ_GEMM_SPLITS", "1")
    y1 = tonp(thq.matmul(w, xb, torch.float32))
    for splits in (2, 3, 7, 16, 32):
        print(f"[split] m={m} splits={splits}", flush=True)
        monkeypatch.setenv("THQ_GEMM_SPLITS", str(splits))
        ys = tonp(thq.matmul(w, xb, torch.float32))
        assert rel_row_err(ys, y1) <= 1e-5, splits


@pytest.mark.parametrize("m,flags", [(16, 0), (17, 0), (100, 0), (100, thq.MODE_EXACT_W)])
def test_q8_0_gemm(m, flags):
    n, k = 777, 1024
    b, w = upload(O.Q8_0, n, k)
    xf, xb = bf16_x(m, k)
    y = tonp(thq.matmul(w, xb, torch.float32, flags=flags))
    ref = O.matmul(O.Q8_0, b, n, k, xf, O.MODE_DEQUANT_F32)
    exact = flags or m <= 64
    if exact:
        assert_close_elem(f"q8_0 gemm m={m}", y, ref, 2.0 ** -14)
    else:
        assert_close_elem(f"q8_0 gemm m={m}", y, ref, 2.0 ** -7, floor="rms")


@pytest.mark.parametrize("m", [1, 2, 9, 100])
def test_q8_0_k_odd_multiple_of_32(m):
    """Q8_0 with K = 32 * odd (K % 64 != 0, allowed by the block size): every
    M uses all of K (the 64-wide GEMM tiles do not apply to this K)."""
    n, k = 200, 1056
    b, w = upload(O.Q8_0, n, k)
    xf, xb = bf16_x(m, k)
    y = tonp(thq.matmul(w, xb, torch.float32))
    ref = O.matmul(O.Q8_0, b, n, k, xf, O.MODE_DEQUANT_F32)
    assert rel_row_err(y, ref) <= 1e-4
    assert_close_elem(f"q8_0 k={k} m={m}", y, ref, 2.0 ** -14)


@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K])
def test_f32_activations_multi_row(qtype):
    n, k = 300, 1024
    b, w = upload(qtype, n, k)
    x = activations(5, k)
    y = tonp(thq.matmul(w, torch.from_numpy(x).cuda(), torch.float32))
    ref = O.matmul(qtype, b, n, k, x, O.MODE_DEQUANT_F32)
    assert rel_row_err(y, ref) <= 1e-4


# ------------------------------------------------------------------ config 4
@pytest.fixture(scope="module")
def lm_head():
    n, k = 151936, 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    wf = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    w = thq.QTensor.quantize(wf, O.Q8_0)
    del wf
    torch.cuda.empty_cache()
    return w, w.data()


@pytest.mark.parametrize("m", [5, 40])
def test_lm_head_verify_argmax(lm_head, m):
    """Every verify row (5 = one slot's drafted + 1 tokens, 40 = a batch of 8
    slots): logits within 1e-4 of the oracle's f64 product, and the argmax
    index of each row equal to the oracle's scan of its own logits."""
    w, b = lm_head
    n, k = w.shape
    xf, xb = bf16_x(m, k, seed=3)
    logits, idx = thq.matmul_argmax(w, xb)
    torch.cuda.synchronize()
    ref = O.matmul(O.Q8_0, b, n, k, xf, O.MODE_DEQUANT_F32)
    got = tonp(logits)
    assert rel_row_err(got, ref) <= 1e-4
    assert_close_elem(f"lm head m={m}", got, ref, 2.0 ** -14)
    want = O.argmax_rows(ref)
    assert list(idx.cpu().numpy()) == list(want)
    # the GPU argmax equals the oracle scan of the GPU's own logits for every row
    assert list(idx.cpu().numpy()) == list(O.argmax_rows(got))
    # without a logits buffer the same indices come back
    _, idx2 = thq.matmul_argmax(w, xb, want_logits=False)
    assert torch.equal(idx, idx2)


def test_argmax_reference_tie_vectors():
    # engine/src/engine.rs:3086-3128: expected [1000, 5, 42]
    V = 248_320
    bf = lambda v: float(O.bf16_round(np.array([v], np.float32))[0])
    data = np.full((3, V), bf(-2.5), np.float32)
    data[0, 1_000] = data[0, 200_000] = bf(21.0)
    data[1, 5] = bf(21.03)
    data[1, 7] = bf(20.97)
    data[2, 42] = data[2, 4_242] = data[2, 248_000] = bf(30.5)
    idx = thq.argmax(torch.from_numpy(data).cuda())
    assert list(idx.cpu().numpy()) == [1000, 5, 42]
    special = torch.tensor([[np.nan, 1.0, 1.0, 0.5], [-np.inf] * 4, [np.nan] * 4], dtype=torch.float32).cuda()
    assert list(thq.argmax(special).cpu().numpy()) == [1, 0, 0]
    empty = torch.empty((3, 0), dtype=torch.float32, device="cuda")
    assert list(thq.argmax(empty).cpu().numpy()) == [0, 0, 0]


# ------------------------------------------------------------------ config 5 / gate-up
@pytest.mark.parametrize("m", [1, 4, 256])
def test_gate_up_epilogue_matches_matmul(m):
    h, k = 1000, 1024   # ragged tile counts
    bg = weight_bytes(O.Q4_K, h, k, seed=11)
    bu = weight_bytes(O.Q4_K, h, k, seed=12)
    fused = thq.QTensor.from_gguf_bytes(O.Q4_K, np.concatenate([bg, bu]), 2 * h, k)
    xf, xb = bf16_x(m, k, seed=5)
    out = thq.gate_up_silu(fused, xb, torch.bfloat16)
    gu = tonp(thq.matmul(fused, xb, torch.float32))
    # the fused kernel's epilogue on the same kernel's own gate/up values:
    # bf16(silu(bf16(g)) * bf16(u)); the device exp may differ by one bf16 step
    want = O.bf16_bits_to_f32(O.gate_up_silu(gu))
    got = tonp(out)
    assert_close_elem(f"gate_up m={m} vs own matmul", got, want, 2.0 ** -7)  # one bf16 step
    assert (got == want).mean() > 0.99
    # and against the oracle's f64 matmul
    ref = O.bf16_bits_to_f32(O.gate_up_silu(O.matmul(O.Q4_K, np.concatenate([bg, bu]), 2 * h, k, xf)))
    assert rel_row_err(got, ref) <= 1e-2


@pytest.mark.parametrize("m", [1, 256])
def test_decoder_layer_projections(m):
    """Qwen3-8B-class layer: QKV 6144x4096, o 4096x4096, gate+up 2x12288x4096 (+silu), down 4096x12288."""
    k = 4096
    xf, xb = bf16_x(m, k, seed=9)
    pick = [0] if m == 1 else [0, 100, 255]
    for name, n, kk in [("qkv", 6144, 4096), ("o", 4096, 4096)]:
        b, w = upload(O.Q4_K, n, kk, seed=21)
        y = tonp(thq.matmul(w, xb, torch.bfloat16))
        ref = O.matmul(O.Q4_K, b, n, kk, xf[pick], O.MODE_DEQUANT_F32)
        assert rel_row_err(y[pick], ref) <= 1e-2, name
        assert_close_elem(name, y[pick], ref, 2.0 ** -6, floor="rms")
    bg, bu = weight_bytes(O.Q4_K, 12288, k, seed=31), weight_bytes(O.Q4_K, 12288, k, seed=32)
    fused = thq.QTensor.from_gguf_bytes(O.Q4_K, np.concatenate([bg, bu]), 24576, k)
    act = thq.gate_up_silu(fused, xb, torch.bfloat16)
    ref_gu = O.matmul(O.Q4_K, np.concatenate([bg, bu]), 24576, k, xf[pick], O.MODE_DEQUANT_F32)
    ref_act = O.bf16_bits_to_f32(O.gate_up_silu(ref_gu))
    assert rel_row_err(tonp(act)[pick], ref_act) <= 1e-2
    bd, wd = upload(O.Q4_K, 4096, 12288, seed=41)
    y = tonp(thq.matmul(wd, act.contiguous(), torch.bfloat16))
    ref = O.matmul(O.Q4_K, bd, 4096, 12288, tonp(act)[pick], O.MODE_DEQUANT_F32)
    assert rel_row_err(y[pick], ref) <= 1e-2


# ------------------------------------------------------------------ edges, errors, determinism
def test_misaligned_activations_fall_back():
    n, k = 512, 1024
    b, w = upload(O.Q4_K, n, k)
    xf, _ = bf16_x(1, k)
    buf = torch.zeros(k + 1, dtype=torch.bfloat16, device="cuda")
    buf[1:] = torch.from_numpy(xf[0]).cuda().to(torch.bfloat16)
    x = buf[1:].reshape(1, k)  # 2-byte aligned view
    assert x.data_ptr() % 16 != 0
    y = tonp(thq.matmul(w, x, torch.float32))
    ref = O.matmul(O.Q4_K, b, n, k, xf, O.MODE_DEQUANT_F32)
    assert_close_elem("misaligned", y, ref, 2.0 ** -12)


@pytest.mark.parametrize("m", [1, 8, 300])
def test_deterministic(m):
    _, w = upload(O.Q4_K, 4096, 4096)
    _, xb = bf16_x(m, 4096)
    a = thq.matmul(w, xb, torch.float32)
    c = thq.matmul(w, xb, torch.float32)
    assert torch.equal(a, c)


def test_empty_and_errors():
    _, w = upload(O.Q4_K, 256, 512)
    x = torch.empty((0, 512), dtype=torch.bfloat16, device="cuda")
    assert thq.matmul(w, x, torch.float32).shape == (0, 256)
    with pytest.raises(ValueError, match="x last dim 128 != weight inp 512"):
        thq.matmul(w, torch.zeros((1, 128), dtype=torch.bfloat16, device="cuda"))
    xb = torch.zeros((1, 512), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(thq.ThqError) as e:
        thq.matmul(w, xb, flags=0x4)
    assert e.value.code == thq.EINVAL
    _, odd = upload(O.Q4_K, 255, 512)
    with pytest.raises(thq.ThqError) as e:
        thq.gate_up_silu(odd, xb)
    assert e.value.code == thq.ESHAPE
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.from_gguf_bytes(O.Q4_K, np.zeros(144, np.uint8), 1, 100)
    assert e.value.code == thq.ESHAPE
    with pytest.raises(thq.ThqError) as e:
        thq.QTensor.from_gguf_bytes(3, np.zeros(144, np.uint8), 1, 256)
    assert e.value.code == thq.EDTYPE
