"""CPU-side checks of the C ABI library (no GPU needed, no compute calls).

libthq.so must load, export every function include/thq.h declares, and
reject invalid arguments with the documented error codes before touching a
device.
"""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(ROOT, "token-horizon_amd", "libthq.so")


def declared_functions():
    """Every function any header under include/ declares."""
    names = set()
    for h in sorted(os.listdir(INCLUDE)):
        if h.endswith(".h"):
            src = re.sub(r"/\*.*?\*/", "", open(os.path.join(INCLUDE, h)).read(), flags=re.S)
            names.update(re.findall(r"\b(thq_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("thq_init", "thq_weight_upload", "thq_matmul", "thq_gate_up_silu", "thq_matmul_argmax",
                 "thq_dequantize", "thq_quantize", "thq_weight_fuse", "thq_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "libthq.so not built"
    lib = C.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_lists_every_export():
    import thq
    assert sorted(thq.EXPORTS) == declared_functions()


def test_invalid_arguments_fail_without_a_device():
    import thq
    L = thq.lib
    h = C.c_void_p()
    # null context / weight / out pointers
    assert L.thq_weight_upload(None, thq.Q4_K, None, 1, 256, C.byref(h)) == thq.EINVAL
    assert L.thq_matmul(None, None, None, thq.ACT_BF16, 1, None, thq.ACT_F32, 0, None) == thq.EINVAL
    assert "null" in thq.last_error()
    assert L.thq_gate_up_silu(None, None, None, thq.ACT_BF16, 1, None, thq.ACT_BF16, 0, None) == thq.EINVAL
    assert L.thq_weight_info(None, None, None, None, None) == thq.EINVAL
    assert L.thq_init(0, None) == thq.EINVAL
    L.thq_weight_free(None)  # no-op
    L.thq_destroy(None)      # no-op
    assert L.thq_version().decode().startswith("thq")


def test_init_without_gpu_reports_an_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import thq
    h = C.c_void_p()
    rc = thq.lib.thq_init(0, C.byref(h))
    assert rc in (thq.EHIP, thq.EINVAL)
    assert thq.last_error()


def test_q8act_buffer_sizes_without_a_device():
    import thq
    L = thq.lib
    assert L.thq_q8act_bytes(thq.Q4_K, 1, 4096) == 0          # not a dot type
    assert L.thq_q8act_bytes(thq.Q8_K, 1, 0) == 0
    q8k = L.thq_q8act_bytes(thq.Q8_K, 3, 4096)                # i8 plane + f32 d + i16 sums, 256-B aligned parts
    assert q8k == 12288 + 256 + 768
    q80 = L.thq_q8act_bytes(thq.Q8_0, 3, 4096)                # i8 plane + f32 d per 32
    assert q80 == 12288 + 1536
    assert L.thq_q8act_prepare(None, thq.Q8_K, None, thq.ACT_BF16, 1, 256, None, None) == thq.EINVAL

