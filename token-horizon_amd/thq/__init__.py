"""ctypes front end of libthq.so (the C ABI in include/thq.h).

Python here is plumbing for tests and benchmarks: torch tensors provide
device memory and the current HIP stream; all compute runs in the gfx950
kernels of libthq.so.  The module raises at import if the library is not
built, so nothing ever falls back to a CPU path.

The classes mirror candle's quantized API that the reference engine uses
([ext] candle-core 0.11 quantized::{QTensor, QMatMul}, reached from
engine/src/model.rs:551-562): QTensor.quantize / .dequantize / .data,
QMatMul.from_qtensor(...).forward(x).
"""
from __future__ import annotations

import ctypes as C
import os

import torch

HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(HERE, "libthq.so")

Q8_0 = 8
Q4_K = 12
Q6_K = 14
Q8_K = 15  # activation dot type of Q4_K (thq_quantize_act)
MLX_Q4 = 100  # MLX affine 4-bit: the engine's QLin (wq u32 [N, K/8], sb bf16 [N, 2K/gs])
BLOCK = {Q8_0: 32, Q4_K: 256, Q6_K: 256, Q8_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q6_K: 210, Q8_K: 292}

ACT_F32 = 0
ACT_BF16 = 1
MODE_DEQUANT_F32 = 0
MODE_Q8ACT = 0x1
MODE_EXACT_W = 0x10
MODE_ARGMAX_FUSED = 0x20

OK = 0
EINVAL, ESHAPE, EDTYPE, EALIGN, EHIP, ENOMEM = -1, -2, -3, -4, -5, -6
EIO, EFORMAT, ENOTFOUND = -7, -8, -9

# GGUF metadata value types (thq_gguf_type)
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL = range(8)
GGUF_STRING, GGUF_ARRAY, GGUF_U64, GGUF_I64, GGUF_F64 = range(8, 13)

# every symbol include/thq.h declares
EXPORTS = (
    "thq_init", "thq_destroy", "thq_last_error", "thq_version", "thq_weight_upload", "thq_weight_from_device",
    "thq_quantize", "thq_weight_fuse", "thq_weight_free", "thq_weight_info", "thq_weight_download",
    "thq_affine_upload", "thq_affine_from_device", "thq_affine_download",
    "thq_dequantize", "thq_dequantize_bf16", "thq_quantize_act", "thq_matmul", "thq_gate_up_silu", "thq_matmul_argmax", "thq_argmax",
    "thq_gguf_open", "thq_gguf_close", "thq_gguf_version", "thq_gguf_tensor_count", "thq_gguf_metadata_count",
    "thq_gguf_find_tensor", "thq_gguf_tensor_info", "thq_gguf_tensor_data", "thq_gguf_metadata_key",
    "thq_gguf_metadata_u32", "thq_gguf_metadata_f32", "thq_gguf_metadata_str", "thq_gguf_metadata_array",
    "thq_weight_from_gguf", "thq_q8act_bytes", "thq_q8act_prepare", "thq_matmul_q8act", "thq_gate_up_silu_q8act",
    "thq_plan_gemv_mfma", "thq_plan_gemm", "thq_plan_gemv_wide", "thq_plan_gemm_mid", "thq_matmul_noalloc", "thq_noalloc_scratch_bytes",
    "thq_topk", "thq_matmul_topk", "thq_gate_up_silu_q8act_emit", "thq_weight_add_tiles",
    "thq_call_scratch_bytes", "thq_reserve", "thq_workspace_bytes", "thq_plan_gemv_tile",
)


class ThqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"thq error {code}: {msg}")
        self.code = code


class GemvPlanInfo(C.Structure):
    """thq_gemv_plan_info (include/thq_plan.h)."""
    _fields_ = [(n, C.c_int32) for n in ("waves", "chunks_per_wave", "splits", "live_rows", "staged_per_thread")] + [
        ("workspace_bytes", C.c_int64)] + [(n, C.c_int32) for n in (
            "xs_elems", "xs_pad_elems", "kb_max", "kb_max_e8", "mmax", "max_waves", "sums_rows_e4", "sums_cols_e4",
            "sums_rows_e8", "sums_cols_e8")]


class GemmPlanInfo(C.Structure):
    """thq_gemm_plan_info (include/thq_plan.h)."""
    _fields_ = [("bm", C.c_int32), ("splits", C.c_int32), ("k_steps", C.c_int32), ("tiles_n", C.c_int64),
                ("tiles_m", C.c_int64), ("workspace_bytes", C.c_int64)]


def plan_gemv_mfma(dtype: int, m: int, n: int, k: int, gate_up: bool = False) -> GemvPlanInfo:
    """The decode GEMV's plan for a shape (host only)."""
    out = GemvPlanInfo()
    check(lib.thq_plan_gemv_mfma(dtype, m, n, k, int(gate_up), C.byref(out)))
    return out


class WidePlanInfo(C.Structure):
    _fields_ = [("splits", C.c_int32), ("chunks_per_split", C.c_int32), ("workspace_bytes", C.c_int64)]


def plan_gemv_wide(dtype: int, m: int, n: int, k: int, cus: int = 256) -> WidePlanInfo:
    """The wide exact-weight GEMV's plan (thq_plan_gemv_wide); splits == 0: no plan."""
    out = WidePlanInfo()
    check(lib.thq_plan_gemv_wide(dtype, m, n, k, cus, C.byref(out)))
    return out


class MidPlanInfo(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("group_halves", "col_tiles", "waves", "groups", "splits",
                                         "chunks_per_split")] + [("workspace_bytes", C.c_int64)]


def plan_gemm_mid(dtype: int, m: int, n: int, k: int, gate_up: bool = False, cus: int = 256) -> MidPlanInfo:
    """The streaming mid-M GEMM's plan (thq_plan_gemm_mid); group_halves == 0: no plan."""
    out = MidPlanInfo()
    check(lib.thq_plan_gemm_mid(dtype, m, n, k, int(gate_up), cus, C.byref(out)))
    return out


class TilePlanInfo(C.Structure):
    _fields_ = [("waves", C.c_int32), ("splits", C.c_int32), ("workspace_bytes", C.c_int64)]


def plan_gemv_tile(dtype: int, m: int, n: int, k: int, gate_up: bool = False, cus: int = 256) -> TilePlanInfo:
    """The tile-plane decode GEMV's plan (thq_plan_gemv_tile); waves == 0: no plan."""
    out = TilePlanInfo()
    check(lib.thq_plan_gemv_tile(dtype, m, n, k, int(gate_up), cus, C.byref(out)))
    return out


def plan_gemm(dtype: int, m: int, n: int, k: int, exact: bool = False, gate_up: bool = False,
              cus: int = 256) -> GemmPlanInfo:
    """The GEMM's plan for a shape on a device with `cus` compute units (host only)."""
    out = GemmPlanInfo()
    check(lib.thq_plan_gemm(dtype, int(exact), m, n, k, int(gate_up), cus, C.byref(out)))
    return out


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libthq.so is not built ({LIB_PATH}); run __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    P, i64, u32, I = C.c_void_p, C.c_int64, C.c_uint32, C.c_int
    PP = C.POINTER(C.c_void_p)
    sig = {
        "thq_init": ([I, PP], I),
        "thq_destroy": ([P], None),
        "thq_last_error": ([], C.c_char_p),
        "thq_version": ([], C.c_char_p),
        "thq_weight_upload": ([P, I, P, i64, i64, PP], I),
        "thq_weight_from_device": ([P, I, P, i64, i64, P, PP], I),
        "thq_quantize": ([P, I, P, i64, i64, P, PP], I),
        "thq_weight_fuse": ([P, PP, I, PP], I),
        "thq_weight_add_tiles": ([P, P], I),
        "thq_weight_free": ([P], None),
        "thq_weight_info": ([P, C.POINTER(C.c_int), C.POINTER(i64), C.POINTER(i64), C.POINTER(C.c_size_t)], I),
        "thq_weight_download": ([P, P], I),
        "thq_dequantize": ([P, P, P, P], I),
        "thq_dequantize_bf16": ([P, P, P, P], I),
        "thq_affine_upload": ([P, P, P, i64, i64, I, I, PP], I),
        "thq_affine_from_device": ([P, P, P, i64, i64, I, I, P, PP], I),
        "thq_affine_download": ([P, P, P], I),
        "thq_quantize_act": ([P, I, P, I, i64, i64, P, P], I),
        "thq_matmul": ([P, P, P, I, i64, P, I, u32, P], I),
        "thq_gate_up_silu": ([P, P, P, I, i64, P, I, u32, P], I),
        "thq_matmul_argmax": ([P, P, P, I, i64, P, P, u32, P], I),
        "thq_argmax": ([P, P, i64, i64, P, P], I),
        "thq_gguf_open": ([C.c_char_p, PP], I),
        "thq_gguf_close": ([P], None),
        "thq_gguf_version": ([P, C.POINTER(u32)], I),
        "thq_gguf_tensor_count": ([P], i64),
        "thq_gguf_metadata_count": ([P], i64),
        "thq_gguf_find_tensor": ([P, C.c_char_p], i64),
        "thq_gguf_tensor_info": ([P, i64, C.POINTER(C.c_char_p), C.POINTER(u32), C.POINTER(u32),
                                  C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)], I),
        "thq_gguf_tensor_data": ([P, i64, PP, C.POINTER(C.c_uint64)], I),
        "thq_gguf_metadata_key": ([P, i64, C.POINTER(C.c_char_p), C.POINTER(u32)], I),
        "thq_gguf_metadata_u32": ([P, C.c_char_p, C.POINTER(u32)], I),
        "thq_gguf_metadata_f32": ([P, C.c_char_p, C.POINTER(C.c_float)], I),
        "thq_gguf_metadata_str": ([P, C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)], I),
        "thq_gguf_metadata_array": ([P, C.c_char_p, C.POINTER(u32), C.POINTER(C.c_uint64)], I),
        "thq_weight_from_gguf": ([P, P, C.c_char_p, PP], I),
        "thq_q8act_bytes": ([I, i64, i64], C.c_size_t),
        "thq_q8act_prepare": ([P, I, P, I, i64, i64, P, P], I),
        "thq_matmul_q8act": ([P, P, I, P, i64, i64, P, I, P], I),
        "thq_gate_up_silu_q8act": ([P, P, I, P, i64, i64, P, I, P], I),
        "thq_matmul_noalloc": ([P, P, P, I, i64, P, I, u32, P], I),
        "thq_topk": ([P, P, i64, i64, I, P, P, P], I),
        "thq_gate_up_silu_q8act_emit": ([P, P, I, P, i64, i64, P, I, P, P], I),
        "thq_matmul_topk": ([P, P, P, I, i64, I, P, P, P, u32, P], I),
        "thq_noalloc_scratch_bytes": ([], C.c_size_t),
        "thq_call_scratch_bytes": ([P, P, i64, I, u32, I, C.POINTER(C.c_size_t)], I),
        "thq_reserve": ([P, C.c_size_t, i64], I),
        "thq_workspace_bytes": ([P], C.c_size_t),
        "thq_plan_gemv_mfma": ([I, i64, i64, i64, I, C.POINTER(GemvPlanInfo)], I),
        "thq_plan_gemm": ([I, I, i64, i64, i64, I, I, C.POINTER(GemmPlanInfo)], I),
        "thq_plan_gemv_wide": ([I, i64, i64, i64, I, C.POINTER(WidePlanInfo)], I),
        "thq_plan_gemm_mid": ([I, i64, i64, i64, I, I, C.POINTER(MidPlanInfo)], I),
        "thq_plan_gemv_tile": ([I, i64, i64, i64, I, I, C.POINTER(TilePlanInfo)], I),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    return L


lib = _load()


def last_error() -> str:
    return lib.thq_last_error().decode()


def check(rc: int):
    if rc != OK:
        raise ThqError(rc, last_error())
    return rc


def _stream(stream=None):
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def _ptr(t: torch.Tensor | None):
    return C.c_void_p(t.data_ptr()) if t is not None else C.c_void_p(0)


def _act(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return ACT_F32
    if t.dtype == torch.bfloat16:
        return ACT_BF16
    raise TypeError(f"activations must be float32 or bfloat16, got {t.dtype}")


class Context:
    """One per device (thq_init)."""

    _by_dev: dict[int, "Context"] = {}

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib.thq_init(device, C.byref(h)))
        self.h = h
        self.device = device

    @classmethod
    def get(cls, device: int = 0) -> "Context":
        if device not in cls._by_dev:
            cls._by_dev[device] = Context(device)
        return cls._by_dev[device]

    def __del__(self):
        if getattr(self, "h", None) and lib is not None:
            lib.thq_destroy(self.h)
            self.h = None

    def reserve(self, workspace_bytes: int, counters: int = 0) -> None:
        """thq_reserve: grow the workspace and the split-K arrival counters now."""
        check(lib.thq_reserve(self.h, workspace_bytes, counters))

    def workspace_bytes(self) -> int:
        return int(lib.thq_workspace_bytes(self.h))


def call_scratch_bytes(w: "QTensor", m: int, x_dtype=torch.bfloat16, flags: int = 0, gate_up: bool = False) -> int:
    """Workspace bytes one thq_matmul / thq_gate_up_silu call of m rows needs (host-side plan)."""
    out = C.c_size_t()
    act = ACT_F32 if x_dtype == torch.float32 else ACT_BF16
    check(lib.thq_call_scratch_bytes(w.ctx.h, w.h, m, act, flags, int(gate_up), C.byref(out)))
    return int(out.value)


class QTensor:
    """Device-resident quantized weight [N, K] (candle QTensor analogue)."""

    def __init__(self, handle: C.c_void_p, ctx: Context):
        self.h = handle
        self.ctx = ctx
        dt, n, k, nb = C.c_int(), C.c_int64(), C.c_int64(), C.c_size_t()
        check(lib.thq_weight_info(self.h, C.byref(dt), C.byref(n), C.byref(k), C.byref(nb)))
        self.dtype, self.n, self.k, self.nbytes = dt.value, n.value, k.value, nb.value

    @property
    def shape(self):
        return (self.n, self.k)

    @classmethod
    def from_gguf_bytes(cls, dtype: int, blocks, n: int, k: int, ctx: Context | None = None) -> "QTensor":
        """blocks: host bytes (numpy uint8 / bytes) or a device uint8 tensor."""
        ctx = ctx or Context.get(torch.cuda.current_device())
        h = C.c_void_p()
        if isinstance(blocks, torch.Tensor) and blocks.is_cuda:
            check(lib.thq_weight_from_device(ctx.h, dtype, _ptr(blocks), n, k, _stream(), C.byref(h)))
        else:
            import numpy as np
            arr = np.ascontiguousarray(np.frombuffer(blocks, dtype=np.uint8) if isinstance(blocks, (bytes, bytearray))
                                       else blocks, dtype=np.uint8)
            check(lib.thq_weight_upload(ctx.h, dtype, arr.ctypes.data_as(C.c_void_p), n, k, C.byref(h)))
        return cls(h, ctx)

    @classmethod
    def quantize(cls, w: torch.Tensor, dtype: int, ctx: Context | None = None) -> "QTensor":
        """Quantize an f32 [N, K] device tensor on the GPU (QTensor::quantize)."""
        ctx = ctx or Context.get(w.device.index or 0)
        assert w.dtype == torch.float32 and w.is_cuda and w.dim() == 2 and w.is_contiguous()
        h = C.c_void_p()
        check(lib.thq_quantize(ctx.h, dtype, _ptr(w), w.shape[0], w.shape[1], _stream(), C.byref(h)))
        return cls(h, ctx)

    @classmethod
    def fuse(cls, parts: list["QTensor"]) -> "QTensor":
        arr = (C.c_void_p * len(parts))(*[p.h.value for p in parts])
        h = C.c_void_p()
        check(lib.thq_weight_fuse(parts[0].ctx.h, arr, len(parts), C.byref(h)))
        qt = cls(h, parts[0].ctx)
        qt.gs = getattr(parts[0], "gs", 0)
        return qt

    def add_tiles(self) -> "QTensor":
        """Give this Q4_K / MLX affine weight its 32-row tile plane
        (thq_weight_add_tiles): 3..8-row plain projections then run the
        tile-plane decode GEMV.  Returns self."""
        check(lib.thq_weight_add_tiles(self.ctx.h, self.h))
        return self

    @classmethod
    def from_affine(cls, wq, sb, n: int, k: int, gs: int = 64, tiled: bool = False,
                    ctx: Context | None = None) -> "QTensor":
        """MLX affine 4-bit weight from the engine's QLin arrays: wq u32 [N, K/8],
        sb bf16 bits [N, 2*K/gs] (row-major, tiled=False) or the QLin::tiled
        layout (tiled=True).  Host numpy arrays or device torch tensors."""
        ctx = ctx or Context.get(torch.cuda.current_device())
        h = C.c_void_p()
        if isinstance(wq, torch.Tensor) and wq.is_cuda:
            check(lib.thq_affine_from_device(ctx.h, _ptr(wq), _ptr(sb), n, k, gs, int(tiled), _stream(),
                                             C.byref(h)))
        else:
            import numpy as np
            w = np.ascontiguousarray(wq, dtype=np.uint32)
            b = np.ascontiguousarray(sb, dtype=np.uint16)
            check(lib.thq_affine_upload(ctx.h, w.ctypes.data_as(C.c_void_p), b.ctypes.data_as(C.c_void_p), n, k, gs,
                                        int(tiled), C.byref(h)))
        qt = cls(h, ctx)
        qt.gs = gs
        return qt

    def affine_data(self):
        """The row-major QLin arrays (wq u32 [N, K/8], sb bf16 bits [N, 2*K/gs])."""
        import numpy as np
        wq = np.empty((self.n, self.k // 8), dtype=np.uint32)
        sb = np.empty((self.n, 2 * self.k // self.gs), dtype=np.uint16)
        check(lib.thq_affine_download(self.h, wq.ctypes.data_as(C.c_void_p), sb.ctypes.data_as(C.c_void_p)))
        return wq, sb

    def dequantize_bf16(self) -> torch.Tensor:
        out = torch.empty((self.n, self.k), dtype=torch.bfloat16, device="cuda")
        check(lib.thq_dequantize_bf16(self.ctx.h, self.h, _ptr(out), _stream()))
        return out

    def data(self):
        """GGUF block bytes (numpy uint8, [N, row_bytes])."""
        import numpy as np
        out = np.empty(self.nbytes, dtype=np.uint8)
        check(lib.thq_weight_download(self.h, out.ctypes.data_as(C.c_void_p)))
        return out.reshape(self.n, -1)

    def dequantize(self) -> torch.Tensor:
        out = torch.empty((self.n, self.k), dtype=torch.float32, device="cuda")
        check(lib.thq_dequantize(self.ctx.h, self.h, _ptr(out), _stream()))
        return out

    def __del__(self):
        if getattr(self, "h", None) and lib is not None:
            lib.thq_weight_free(self.h)
            self.h = None


def quantize_act(x: torch.Tensor, dot_type: int, ctx: Context | None = None) -> torch.Tensor:
    """GGML blocks of x[M, K] rows (candle's BlockQ8_0 / BlockQ8K::from_float) as a
    uint8 device tensor [M, K/bs * block bytes] (thq_quantize_act)."""
    x2 = x.reshape(-1, x.shape[-1])
    assert x2.is_contiguous()
    ctx = ctx or Context.get(x.device.index or 0)
    m, k = x2.shape
    out = torch.empty((m, (k // BLOCK[dot_type]) * BLOCK_BYTES[dot_type]), dtype=torch.uint8, device=x.device)
    check(lib.thq_quantize_act(ctx.h, dot_type, _ptr(x2), _act(x2), m, k, _ptr(out), _stream()))
    return out


class Q8Act:
    """Activation rows quantized once for THQ_MODE_Q8ACT consumers
    (thq_q8act_prepare): the producer-side operand several projections of
    the same input share."""

    def __init__(self, x: torch.Tensor, dot_type: int, ctx: Context | None = None):
        x2 = x.reshape(-1, x.shape[-1])
        assert x2.is_contiguous()
        self.ctx = ctx or Context.get(x.device.index or 0)
        self.m, self.k = x2.shape
        self.dot_type = dot_type
        nbytes = lib.thq_q8act_bytes(dot_type, self.m, self.k)
        if nbytes == 0:
            raise ThqError(EDTYPE, f"unsupported dot type {dot_type}")
        # 256-byte aligned: torch's allocator aligns blocks to 512 bytes
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        check(lib.thq_q8act_prepare(self.ctx.h, dot_type, _ptr(x2), _act(x2), self.m, self.k, _ptr(self.buf),
                                    _stream()))

    def matmul(self, w: "QTensor", out_dtype=torch.float32) -> torch.Tensor:
        y = torch.empty((self.m, w.n), dtype=out_dtype, device=self.buf.device)
        check(lib.thq_matmul_q8act(self.ctx.h, w.h, self.dot_type, _ptr(self.buf), self.m, self.k, _ptr(y),
                                   _act(y), _stream()))
        return y

    def gate_up_silu(self, fused: "QTensor", out_dtype=torch.bfloat16) -> torch.Tensor:
        y = torch.empty((self.m, fused.n // 2), dtype=out_dtype, device=self.buf.device)
        check(lib.thq_gate_up_silu_q8act(self.ctx.h, fused.h, self.dot_type, _ptr(self.buf), self.m, self.k,
                                         _ptr(y), _act(y), _stream()))
        return y

    def gate_up_silu_emit(self, fused: "QTensor", out_dtype=torch.bfloat16):
        """(y, the Q8Act of y) from one launch (thq_gate_up_silu_q8act_emit):
        the down projection's operand comes out of the gate/up epilogue."""
        h = fused.n // 2
        y = torch.empty((self.m, h), dtype=out_dtype, device=self.buf.device)
        nxt = Q8Act.__new__(Q8Act)
        nxt.ctx, nxt.m, nxt.k, nxt.dot_type = self.ctx, self.m, h, Q8_K
        nxt.buf = torch.empty(lib.thq_q8act_bytes(Q8_K, self.m, h), dtype=torch.uint8, device=self.buf.device)
        check(lib.thq_gate_up_silu_q8act_emit(self.ctx.h, fused.h, self.dot_type, _ptr(self.buf), self.m, self.k,
                                              _ptr(y), _act(y), _ptr(nxt.buf), _stream()))
        return y, nxt


def matmul(w: QTensor, x: torch.Tensor, out_dtype=torch.float32, flags: int = 0, out: torch.Tensor | None = None):
    """y[M, N] = x[M, K] . W^T through thq_matmul."""
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    if x2.shape[-1] != w.k:
        raise ValueError(f"x last dim {x2.shape[-1]} != weight inp {w.k}")
    assert x2.is_contiguous() or x2.numel() == 0
    m = x2.shape[0]
    if out is None:
        out = torch.empty((m, w.n), dtype=out_dtype, device=x.device)
    check(lib.thq_matmul(w.ctx.h, w.h, _ptr(x2), _act(x2), m, _ptr(out), _act(out), flags, _stream()))
    return out.reshape(*x.shape[:-1], w.n)


def matmul_noalloc(w: QTensor, x: torch.Tensor, out: torch.Tensor, flags: int = 0):
    """thq_matmul_noalloc: thq_matmul on the device's static scratch (no allocation)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[-1] != w.k:
        raise ValueError(f"x last dim {x2.shape[-1]} != weight inp {w.k}")
    check(lib.thq_matmul_noalloc(w.ctx.h, w.h, _ptr(x2), _act(x2), x2.shape[0], _ptr(out), _act(out), flags,
                                 _stream()))
    return out


def gate_up_silu(w: QTensor, x: torch.Tensor, out_dtype=torch.bfloat16, flags: int = 0,
                 out: torch.Tensor | None = None):
    """y[M, N/2] = bf16(silu(bf16(g)) * bf16(u)) over a fused [gate; up] weight."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[-1] != w.k:
        raise ValueError(f"x last dim {x2.shape[-1]} != weight inp {w.k}")
    m = x2.shape[0]
    if out is None:
        out = torch.empty((m, w.n // 2), dtype=out_dtype, device=x.device)
    check(lib.thq_gate_up_silu(w.ctx.h, w.h, _ptr(x2), _act(x2), m, _ptr(out), _act(out), flags, _stream()))
    return out.reshape(*x.shape[:-1], w.n // 2)


def matmul_argmax(w: QTensor, x: torch.Tensor, want_logits: bool = True, flags: int = 0,
                  logits: torch.Tensor | None = None, idx: torch.Tensor | None = None):
    """LM head + per-row greedy argmax; returns (logits or None, idx int32)."""
    x2 = x.reshape(-1, x.shape[-1])
    m = x2.shape[0]
    if logits is None and want_logits:
        logits = torch.empty((m, w.n), dtype=torch.float32, device=x.device)
    if idx is None:
        idx = torch.empty((m,), dtype=torch.int32, device=x.device)
    check(lib.thq_matmul_argmax(w.ctx.h, w.h, _ptr(x2), _act(x2), m, _ptr(logits), _ptr(idx), flags, _stream()))
    return logits, idx


def argmax(v: torch.Tensor, ctx: Context | None = None) -> torch.Tensor:
    assert v.dtype == torch.float32 and v.is_contiguous()
    ctx = ctx or Context.get(v.device.index or 0)
    v2 = v if v.dim() == 2 else v.reshape(1, -1)
    m, n = v2.shape
    idx = torch.empty((m,), dtype=torch.int32, device=v.device)
    check(lib.thq_argmax(ctx.h, _ptr(v2), m, n, _ptr(idx), _stream()))
    return idx


def topk(v: torch.Tensor, k: int, ctx: Context | None = None):
    """Exact per-row top-k (logit desc, id asc); returns (vals f32 [M, k], idx int32 [M, k])."""
    assert v.dtype == torch.float32 and v.is_contiguous()
    ctx = ctx or Context.get(v.device.index or 0)
    v2 = v if v.dim() == 2 else v.reshape(1, -1)
    m, n = v2.shape
    vals = torch.empty((m, k), dtype=torch.float32, device=v.device)
    idx = torch.empty((m, k), dtype=torch.int32, device=v.device)
    check(lib.thq_topk(ctx.h, _ptr(v2), m, n, k, _ptr(vals), _ptr(idx), _stream()))
    return vals, idx


def matmul_topk(w: QTensor, x: torch.Tensor, k: int, want_logits: bool = False, flags: int = 0):
    """LM head + exact per-row top-k; returns (logits or None, vals, idx)."""
    x2 = x.reshape(-1, x.shape[-1])
    m = x2.shape[0]
    logits = torch.empty((m, w.n), dtype=torch.float32, device=x.device) if want_logits else None
    vals = torch.empty((m, k), dtype=torch.float32, device=x.device)
    idx = torch.empty((m, k), dtype=torch.int32, device=x.device)
    check(lib.thq_matmul_topk(w.ctx.h, w.h, _ptr(x2), _act(x2), m, k, _ptr(logits), _ptr(vals), _ptr(idx), flags,
                              _stream()))
    return logits, vals, idx


class QMatMul:
    """candle QMatMul analogue: forward(x) = x . W^T."""

    def __init__(self, qt: QTensor):
        self.w = qt

    @classmethod
    def from_qtensor(cls, qt: QTensor) -> "QMatMul":
        return cls(qt)

    def forward(self, x: torch.Tensor, out_dtype=None) -> torch.Tensor:
        return matmul(self.w, x, out_dtype or x.dtype)


class GGUFFile:
    """A GGUF file opened through thq_gguf_open: candle's gguf_file::Content
    (Content::read, .metadata lookups, .tensor_infos, .tensor) as the loader
    engine/src/model.rs:526-562 uses it.  Host-only except .weight()."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib.thq_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h
        v = C.c_uint32()
        check(lib.thq_gguf_version(self.h, C.byref(v)))
        self.version = v.value

    def close(self):
        if getattr(self, "h", None):
            lib.thq_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        if lib is not None:
            self.close()

    def metadata_keys(self) -> dict:
        """{key: value type} in the order keys first appear."""
        out = {}
        for i in range(lib.thq_gguf_metadata_count(self.h)):
            k, t = C.c_char_p(), C.c_uint32()
            check(lib.thq_gguf_metadata_key(self.h, i, C.byref(k), C.byref(t)))
            out[k.value.decode()] = t.value
        return out

    def u32(self, key: str) -> int:
        v = C.c_uint32()
        check(lib.thq_gguf_metadata_u32(self.h, key.encode(), C.byref(v)))
        return v.value

    def f32(self, key: str) -> float:
        v = C.c_float()
        check(lib.thq_gguf_metadata_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def string(self, key: str) -> str:
        v, n = C.c_void_p(), C.c_uint64()
        check(lib.thq_gguf_metadata_str(self.h, key.encode(), C.byref(v), C.byref(n)))
        return C.string_at(v.value, n.value).decode() if n.value else ""

    def array(self, key: str) -> tuple[int, int]:
        t, n = C.c_uint32(), C.c_uint64()
        check(lib.thq_gguf_metadata_array(self.h, key.encode(), C.byref(t), C.byref(n)))
        return t.value, n.value

    def tensor_names(self) -> list[str]:
        return [self.tensor_info(i)["name"] for i in range(lib.thq_gguf_tensor_count(self.h))]

    def find(self, name: str) -> int:
        return lib.thq_gguf_find_tensor(self.h, name.encode())

    def tensor_info(self, i) -> dict:
        if isinstance(i, str):
            j = self.find(i)
            if j < 0:
                raise ThqError(ENOTFOUND, f"no tensor {i}")
            i = j
        name, t, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        dims = (C.c_uint64 * 4)()
        off, nb = C.c_uint64(), C.c_uint64()
        check(lib.thq_gguf_tensor_info(self.h, i, C.byref(name), C.byref(t), C.byref(nd), dims, C.byref(off),
                                       C.byref(nb)))
        return {"name": name.value.decode(), "type": t.value, "shape": tuple(dims[:nd.value]),
                "offset": off.value, "nbytes": nb.value}

    def tensor_bytes(self, name: str):
        """The tensor's block bytes, copied out of the mapping (numpy uint8)."""
        import numpy as np
        i = self.find(name)
        if i < 0:
            raise ThqError(ENOTFOUND, f"no tensor {name}")
        p, n = C.c_void_p(), C.c_uint64()
        check(lib.thq_gguf_tensor_data(self.h, i, C.byref(p), C.byref(n)))
        return np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p.value)).copy() if n.value else \
            np.empty(0, np.uint8)

    def weight(self, name: str, ctx: "Context | None" = None) -> "QTensor":
        """Upload a 2-D Q8_0 / Q4_K / Q6_K tensor (thq_weight_from_gguf)."""
        ctx = ctx or Context.get(torch.cuda.current_device())
        h = C.c_void_p()
        check(lib.thq_weight_from_gguf(ctx.h, self.h, name.encode(), C.byref(h)))
        return QTensor(h, ctx)
