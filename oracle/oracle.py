"""numpy front end of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product library never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_0 = 8
Q4_K = 12
Q6_K = 14
BLOCK = {Q8_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q6_K: 210}
Q8_K_BYTES = 292

MODE_DEQUANT_F32 = 0
MODE_Q8ACT = 1

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        i64 = C.c_int64
        L.o_f16_to_f32.argtypes = [C.c_uint16]
        L.o_f16_to_f32.restype = C.c_float
        L.o_f32_to_f16.argtypes = [C.c_float]
        L.o_f32_to_f16.restype = C.c_uint16
        L.o_f32_to_bf16.argtypes = [C.c_float]
        L.o_f32_to_bf16.restype = C.c_uint16
        L.o_randn.argtypes = [C.c_uint64, C.c_uint64, C.c_float, P, C.c_size_t]
        L.o_row_bytes.argtypes = [C.c_int, i64]
        L.o_row_bytes.restype = C.c_size_t
        for name in ("o_quantize_q8_0", "o_dequantize_q8_0", "o_quantize_q4_k", "o_dequantize_q4_k",
                     "o_quantize_q8_k", "o_dequantize_q6_k"):
            getattr(L, name).argtypes = [P, P, i64]
        L.o_get_scale_min_k4.argtypes = [C.c_int, P, P, P]
        L.o_make_qkx1_quants.argtypes = [C.c_int, C.c_int, P, C.c_int, P, P, P]
        L.o_quantize.argtypes = [C.c_int, P, i64, i64, P]
        L.o_dequantize.argtypes = [C.c_int, P, i64, i64, P]
        L.o_vec_dot_q8_0_q8_0.argtypes = [i64, P, P]
        L.o_vec_dot_q8_0_q8_0.restype = C.c_float
        L.o_vec_dot_q4_k_q8_k.argtypes = [i64, P, P]
        L.o_vec_dot_q4_k_q8_k.restype = C.c_float
        L.o_matmul.argtypes = [C.c_int, C.c_int, P, i64, i64, P, i64, P, C.c_int]
        L.o_baseline_matmul.argtypes = [C.c_int, P, i64, i64, P, i64, P, C.c_int]
        L.o_gate_up_silu.argtypes = [P, i64, i64, P]
        L.o_argmax.argtypes = [P, i64]
        L.o_argmax.restype = C.c_uint32
        L.o_argmax_rows.argtypes = [P, i64, i64, P]
        L.o_topk_rows.argtypes = [P, i64, i64, C.c_int, P, P]
        L.o_bf16_from_f64_half.argtypes = [C.c_double]
        L.o_bf16_from_f64_half.restype = C.c_uint16
        L.o_affine_dequant_bf16.argtypes = [P, P, i64, i64, C.c_int, P]
        L.o_affine_dequant_f32.argtypes = [P, P, i64, i64, C.c_int, P]
        L.o_affine_matmul.argtypes = [P, P, i64, i64, C.c_int, P, i64, P]
        L.o_affine_tile.argtypes = [P, P, i64, i64, P, P]
        L.o_baseline_has_avx2.restype = C.c_int
        L.o_max_threads.restype = C.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def randn(seed: int, stream: int, sigma: float, shape) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().o_randn(seed, stream, sigma, _p(out), n)
    return out.reshape(shape)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (vectorised restatement
    of the oracle's o_f32_to_bf16; pinned against it in tests)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def row_bytes(qtype: int, k: int) -> int:
    return (k // BLOCK[qtype]) * BLOCK_BYTES[qtype]


def quantize(qtype: int, w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    out = np.empty((n, row_bytes(qtype, k)), dtype=np.uint8)
    rc = lib().o_quantize(qtype, _p(w), n, k, _p(out))
    if rc != 0:
        raise ValueError(f"o_quantize rc={rc}")
    return out


def dequantize(qtype: int, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    assert blocks.size == n * row_bytes(qtype, k)
    out = np.empty((n, k), dtype=np.float32)
    rc = lib().o_dequantize(qtype, _p(blocks), n, k, _p(out))
    if rc != 0:
        raise ValueError(f"o_dequantize rc={rc}")
    return out


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty((x.size // 256) * Q8_K_BYTES, dtype=np.uint8)
    lib().o_quantize_q8_k(_p(x), _p(out), x.size)
    return out


def quantize_q8_0_row(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty((x.size // 32) * 34, dtype=np.uint8)
    lib().o_quantize_q8_0(_p(x), _p(out), x.size)
    return out


def matmul(qtype: int, blocks: np.ndarray, n: int, k: int, x: np.ndarray, mode: int = MODE_DEQUANT_F32,
           threads: int = 0) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    rc = lib().o_matmul(qtype, mode, _p(blocks), n, k, _p(x), m, _p(y), threads)
    if rc != 0:
        raise ValueError(f"o_matmul rc={rc}")
    return y


def baseline_matmul(qtype: int, blocks: np.ndarray, n: int, k: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    rc = lib().o_baseline_matmul(qtype, _p(blocks), n, k, _p(x), m, _p(y), threads)
    if rc != 0:
        raise ValueError(f"o_baseline_matmul rc={rc}")
    return y


def gate_up_silu(y_gu: np.ndarray) -> np.ndarray:
    """[m, 2h] f32 (gate | up) -> [m, h] bf16 bit patterns."""
    y_gu = np.ascontiguousarray(y_gu, dtype=np.float32)
    m, h2 = y_gu.shape
    out = np.empty((m, h2 // 2), dtype=np.uint16)
    lib().o_gate_up_silu(_p(y_gu), m, h2 // 2, _p(out))
    return out


def argmax_rows(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    if v.ndim == 1:
        v = v.reshape(1, -1)
    m, n = v.shape
    idx = np.empty(m, dtype=np.uint32)
    lib().o_argmax_rows(_p(v), m, n, _p(idx))
    return idx


def topk_rows(v: np.ndarray, k: int):
    """(vals f32 [m, k], idx u32 [m, k]): each row's top k by (key desc, id asc)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    if v.ndim == 1:
        v = v.reshape(1, -1)
    m, n = v.shape
    vals = np.empty((m, k), np.float32)
    idx = np.empty((m, k), np.uint32)
    lib().o_topk_rows(_p(v), m, n, k, _p(vals), _p(idx))
    return vals, idx


def get_scale_min_k4(j: int, scales12: np.ndarray):
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc = np.zeros(1, np.uint8)
    mn = np.zeros(1, np.uint8)
    lib().o_get_scale_min_k4(j, _p(s), _p(sc), _p(mn))
    return int(sc[0]), int(mn[0])


def make_qkx1_quants(nmax: int, ntry: int, x: np.ndarray):
    """(scale, min, levels) of one sub-block ([ext] utils.rs make_qkx1_quants)."""
    xs = np.ascontiguousarray(x, dtype=np.float32)
    sc = np.zeros(1, np.float32)
    mn = np.zeros(1, np.float32)
    lv = np.zeros(xs.size, np.uint8)
    lib().o_make_qkx1_quants(nmax, ntry, _p(xs), xs.size, _p(sc), _p(mn), _p(lv))
    return sc[0], mn[0], lv


def max_threads() -> int:
    return lib().o_max_threads()


def has_avx2() -> bool:
    return bool(lib().o_baseline_has_avx2())


# ------------------------------------------------------------------ MLX affine 4-bit
def bf16_from_f64_half(v: float) -> int:
    """[ext] half 2.7.1 bf16::from_f64 (dequant_affine's rounding)."""
    return int(lib().o_bf16_from_f64_half(float(v)))


def _affine_args(wq, sb, n, k):
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    sb = np.ascontiguousarray(sb, dtype=np.uint16)
    assert wq.size == n * k // 8 and sb.size % n == 0
    return wq, sb


def affine_dequant_bf16(wq, sb, n: int, k: int, gs: int = 64) -> np.ndarray:
    """dequant_affine (engine/src/qwen35.rs:110-134): bf16 bits [n, k]."""
    wq, sb = _affine_args(wq, sb, n, k)
    out = np.empty((n, k), dtype=np.uint16)
    lib().o_affine_dequant_bf16(_p(wq), _p(sb), n, k, gs, _p(out))
    return out


def affine_dequant_f32(wq, sb, n: int, k: int, gs: int = 64) -> np.ndarray:
    wq, sb = _affine_args(wq, sb, n, k)
    out = np.empty((n, k), dtype=np.float32)
    lib().o_affine_dequant_f32(_p(wq), _p(sb), n, k, gs, _p(out))
    return out


def affine_matmul(wq, sb, n: int, k: int, x: np.ndarray, gs: int = 64) -> np.ndarray:
    """y = x . W^T with exact affine weights and f64 sums."""
    wq, sb = _affine_args(wq, sb, n, k)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), dtype=np.float32)
    lib().o_affine_matmul(_p(wq), _p(sb), n, k, gs, _p(x), x.shape[0], _p(y))
    return y


def affine_tile(wq, sb, n: int, k: int):
    """QLin::tiled (engine/src/qwen35.rs:629-697) of row-major arrays (gs = 64)."""
    wq, sb = _affine_args(wq, sb, n, k)
    tiles, ng = (n + 255) // 256, k // 64
    wt = np.zeros(tiles * 256 * ng * 8, dtype=np.uint32)
    st = np.zeros(2 * tiles * 256 * ng, dtype=np.uint16)
    lib().o_affine_tile(_p(wq), _p(sb), n, k, _p(wt), _p(st))
    return wt, st
