"""The C ABI's error contract (include/thq.h) under invalid arguments: every
entry point returns a negative THQ_E* code with a message, never crashes, and
leaves the context usable.  This is the analogue of the reference ops'
`bail!` on dtype / shape / alignment violations (quant_kernel.rs:3062-3083)
and QLin's in-dim check (qwen35.rs:405-411).
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from helpers import weight_bytes

pytestmark = pytest.mark.gpu

thq = pytest.importorskip("thq")

CODES = {thq.EINVAL, thq.ESHAPE, thq.EDTYPE, thq.EALIGN, thq.EHIP, thq.ENOMEM, thq.EFORMAT, thq.ENOTFOUND}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    yield
    torch.cuda.synchronize()


def expect(rc, code=None):
    assert rc < 0 and rc in CODES, rc
    if code is not None:
        assert rc == code, (rc, code, thq.last_error())
    assert thq.last_error(), "an error leaves a message"


def ptr(t):
    return C.c_void_p(t.data_ptr())


def test_invalid_arguments_every_entry_point():
    L = thq.lib
    ctx = thq.Context.get(0).h
    blocks = weight_bytes(O.Q4_K, 8, 512, seed=1)
    out = C.c_void_p()
    hb = blocks.ctypes.data_as(C.c_void_p)
    print("[abi] weight creation", flush=True)
    expect(L.thq_init(-1, C.byref(out)))
    expect(L.thq_weight_upload(None, thq.Q4_K, hb, 8, 512, C.byref(out)), thq.EINVAL)
    expect(L.thq_weight_upload(ctx, thq.Q4_K, None, 8, 512, C.byref(out)), thq.EINVAL)
    expect(L.thq_weight_upload(ctx, thq.Q4_K, hb, 0, 512, C.byref(out)), thq.ESHAPE)
    expect(L.thq_weight_upload(ctx, thq.Q4_K, hb, -8, 512, C.byref(out)), thq.ESHAPE)
    expect(L.thq_weight_upload(ctx, thq.Q4_K, hb, 8, 500, C.byref(out)), thq.ESHAPE)
    expect(L.thq_weight_upload(ctx, thq.Q4_K, hb, 1 << 41, 512, C.byref(out)), thq.ESHAPE)
    expect(L.thq_weight_upload(ctx, thq.Q4_K, hb, 1 << 30, 1 << 20, C.byref(out)), thq.ESHAPE)  # 2^50 weights
    expect(L.thq_weight_upload(ctx, 3, hb, 8, 512, C.byref(out)), thq.EDTYPE)
    expect(L.thq_affine_upload(ctx, hb, hb, 8, 512, 32, 0, C.byref(out)), thq.EDTYPE)   # gs 32
    expect(L.thq_affine_upload(ctx, hb, hb, 8, 448, 128, 0, C.byref(out)), thq.EDTYPE)  # K % gs
    expect(L.thq_affine_upload(ctx, hb, hb, 8, 512, 128, 1, C.byref(out)), thq.EDTYPE)  # tiled needs 64

    w4 = thq.QTensor.from_gguf_bytes(thq.Q4_K, blocks, 8, 512)
    w4b = thq.QTensor.from_gguf_bytes(thq.Q4_K, weight_bytes(O.Q4_K, 8, 256, seed=2), 8, 256)
    w8 = thq.QTensor.from_gguf_bytes(thq.Q8_0, weight_bytes(O.Q8_0, 8, 512, seed=3), 8, 512)
    print("[abi] fuse", flush=True)
    parts = (C.c_void_p * 2)(w4.h, w4b.h)
    expect(L.thq_weight_fuse(ctx, parts, 2, C.byref(out)), thq.ESHAPE)  # different K
    parts = (C.c_void_p * 2)(w4.h, w8.h)
    expect(L.thq_weight_fuse(ctx, parts, 2, C.byref(out)), thq.EDTYPE)  # different types
    expect(L.thq_weight_fuse(ctx, parts, 0, C.byref(out)), thq.EINVAL)
    expect(L.thq_weight_fuse(ctx, None, 2, C.byref(out)), thq.EINVAL)

    x = torch.zeros((4, 512), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((4, 8), dtype=torch.float32, device="cuda")
    idx = torch.zeros((4,), dtype=torch.int32, device="cuda")
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    print("[abi] matmul / gate-up / argmax", flush=True)
    expect(L.thq_matmul(ctx, w4.h, None, thq.ACT_BF16, 4, ptr(y), thq.ACT_F32, 0, s), thq.EINVAL)
    expect(L.thq_matmul(ctx, w4.h, ptr(x), thq.ACT_BF16, 4, None, thq.ACT_F32, 0, s), thq.EINVAL)
    expect(L.thq_matmul(ctx, w4.h, ptr(x), 7, 4, ptr(y), thq.ACT_F32, 0, s), thq.EINVAL)
    expect(L.thq_matmul(ctx, w4.h, ptr(x), thq.ACT_BF16, 4, ptr(y), 9, 0, s), thq.EINVAL)
    expect(L.thq_matmul(ctx, w4.h, ptr(x), thq.ACT_BF16, -1, ptr(y), thq.ACT_F32, 0, s), thq.ESHAPE)
    expect(L.thq_matmul(ctx, w4.h, ptr(x), thq.ACT_BF16, 4, ptr(y), thq.ACT_F32, 0x40000000, s), thq.EINVAL)
    expect(L.thq_matmul(None, w4.h, ptr(x), thq.ACT_BF16, 4, ptr(y), thq.ACT_F32, 0, s), thq.EINVAL)
    expect(L.thq_matmul(ctx, None, ptr(x), thq.ACT_BF16, 4, ptr(y), thq.ACT_F32, 0, s), thq.EINVAL)
    odd = thq.QTensor.from_gguf_bytes(thq.Q4_K, weight_bytes(O.Q4_K, 7, 512, seed=4), 7, 512)
    expect(L.thq_gate_up_silu(ctx, odd.h, ptr(x), thq.ACT_BF16, 4, ptr(y), thq.ACT_F32, 0, s), thq.ESHAPE)
    expect(L.thq_matmul_argmax(ctx, w4.h, ptr(x), thq.ACT_BF16, 4, None, None, 0, s), thq.EINVAL)
    # shape and type checks come before any workspace is reserved
    expect(L.thq_matmul_argmax(ctx, w4.h, ptr(x), thq.ACT_BF16, -1, None, ptr(idx), 0, s), thq.ESHAPE)
    expect(L.thq_matmul_argmax(ctx, w4.h, ptr(x), thq.ACT_BF16, -(1 << 40), ptr(y), ptr(idx), 0, s), thq.ESHAPE)
    expect(L.thq_matmul_argmax(ctx, w4.h, ptr(x), 7, 4, None, ptr(idx), 0, s), thq.EINVAL)
    expect(L.thq_matmul_argmax(ctx, w4.h, ptr(x), thq.ACT_BF16, 4, None, ptr(idx), 0x40000000, s), thq.EINVAL)
    expect(L.thq_matmul_argmax(ctx, w4.h, None, thq.ACT_BF16, 4, None, ptr(idx), 0, s), thq.EINVAL)
    expect(L.thq_argmax(ctx, ptr(y), -1, 8, ptr(idx), s), thq.ESHAPE)
    expect(L.thq_argmax(ctx, ptr(y), 1, 1 << 33, ptr(idx), s), thq.ESHAPE)
    expect(L.thq_argmax(ctx, None, 4, 8, ptr(idx), s), thq.EINVAL)
    print("[abi] dequant / download / info / q8act", flush=True)
    expect(L.thq_dequantize(ctx, w4.h, None, s), thq.EINVAL)
    expect(L.thq_weight_download(None, hb), thq.EINVAL)
    expect(L.thq_weight_info(None, None, None, None, None), thq.EINVAL)
    q = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    expect(L.thq_quantize_act(ctx, thq.Q4_K, ptr(x), thq.ACT_BF16, 4, 512, ptr(q), s), thq.EDTYPE)  # not a dot type
    expect(L.thq_q8act_prepare(ctx, thq.Q8_K, ptr(x), thq.ACT_BF16, 4, 500, ptr(q), s), thq.ESHAPE)  # K % 256
    expect(L.thq_matmul_q8act(ctx, w4.h, thq.Q8_0, ptr(q), 4, 512, ptr(y), thq.ACT_F32, s))  # Q4_K dots with Q8_K

    print("[abi] the context still works", flush=True)
    got = thq.matmul(w4, x.normal_(), torch.float32)
    want = O.matmul(O.Q4_K, blocks, 8, 512, x.float().cpu().numpy())
    assert np.allclose(got.cpu().numpy(), want, rtol=0, atol=1e-2 * np.abs(want).max())
