"""Build libthq.so (gfx950 HIP kernels + the C ABI) in-tree.

    python token-horizon_amd/build.py          # builds token-horizon_amd/libthq.so
                                               # and libthq_probe.so (bench.py's read probes)

Each source compiles separately with hipcc (in parallel) into _build/, then
links into one shared library next to this file.  Flags:
  --offload-arch=gfx950            CDNA4 only, no other targets
  -ffp-contract=off                f32 expressions round as written; the hot
                                   loops use explicit fmaf where they fuse
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                   no v_pk_{add,mul,fma}_f32 generation
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libthq.so")
# measurement aids for bench.py only, kept out of the product library's ABI
PROBE_SOURCES = ["k_probe.hip"]
PROBE_LIB = os.path.join(HERE, "libthq_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = [
    "thq_api.cpp", "k_weights.hip", "k_gemv.hip", "k_gemv_mfma.hip", "k_gemm.hip", "k_argmax.hip", "k_q8act.hip",
    "k_q6k.hip", "k_topk.hip", "k_gemv_wide.hip", "k_gemv_tile.hip", "k_gemm_b16.hip",
    "k_gemm_fq.hip", "k_gemm_rq.hip", "k_gemm_mid.hip", "thq_gguf.cpp",
]
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature: harmless, drop it
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _link(objs: list[str], lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, lib)


def build(jobs: int | None = None, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, len(SOURCES) + len(PROBE_SOURCES))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES + PROBE_SOURCES))
    _link(objs[:len(SOURCES)], LIB)
    _link(objs[len(SOURCES):], PROBE_LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}")
    return LIB


if __name__ == "__main__":
    build()
