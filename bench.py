"""Benchmark of the quantized projection path on one MI355X.

Headline metric: Q4_K decode GEMV HBM GB/s at M=1 and prefill GEMM TFLOP/s at
M=2048, both on the Qwen3-8B-class gate/up projection (N=12288, K=4096).
A "step" is one GEMV call (M=1, bf16 x, f32 y) on the next of 24 distinct
weight copies (680 MB in rotation, so weights stream from HBM, not from the
256 MB MALL), each read once after it is written (page_in).  --warmup
untimed steps run first; then exactly --steps steps
are launched on one stream behind a GPU spin that lasts longer than the host
takes to launch all of them, so the GPU runs them back to back with no host
gap, and HIP events on that stream bracket exactly those steps.  The bench
checks that the host finished launching before the spin ended; if it did not
(very many steps), the steps are timed from a captured HIP graph instead,
uploaded (hipGraphUpload) before the start event.  A graph's first replay
after upload still runs each kernel about 0.3-0.6 us slower than its later
replays, which a 20-step timed region would carry in full.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-configs]

Prints one JSON line: the headline GEMV and the M=2048 GEMM, each with its
roofline, the single-launch read ceilings of the GEMV's byte count, a
`configs` object timing every benchmark configuration of the path (Q8_0
3072x1024 with f32 x; Q4_K decode M=1,2,4,8 and prefill M=128,512,2048 on both
MLP shapes; the Q8_0 LM head with argmax at M=5,40; the decoder layer at
M=1,256), and the CPU baseline.  Inputs are synthetic: W ~ N(0, 0.02)
quantized on the device, x ~ N(0, 1) in bf16, from torch's seeded generator.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "token-horizon_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
Q4K_BYTES_PER_256 = 144
GEMM_ROUTE = ("the weight dequantized to bf16 once per call (k_dequant_q4_b16), then the bf16 MFMA GEMM "
              "(k_gemm_b16); us_per_call covers both launches")


PROBE_LIB = os.path.join(ROOT, "token-horizon_amd", "libthq_probe.so")


def load_probe():
    """The read-ceiling probes (libthq_probe.so, built beside libthq.so by
    token-horizon_amd/build.py; not part of the product library)."""
    import ctypes as C
    lib = C.CDLL(PROBE_LIB)
    for name in ("thqp_hbm_read", "thqp_hbm_read_x4"):
        getattr(lib, name).argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_void_p, C.c_void_p]
        getattr(lib, name).restype = C.c_int
    lib.thqp_gemv_loads.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_void_p]
    lib.thqp_gemv_loads.restype = C.c_int
    return lib


def graph_upload(gt, stream):
    """hipGraphUpload of a captured graph's executable on `stream`: the
    graph's one-time device setup happens here, not at its first replay."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipGraphUpload.argtypes = [C.c_void_p, C.c_void_p]
    rc = hip.hipGraphUpload(C.c_void_p(gt.raw_cuda_graph_exec()), C.c_void_p(stream.cuda_stream))
    if rc != 0:
        raise RuntimeError(f"hipGraphUpload failed: {rc}")


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4k_bytes(n, k):
    return n * (k // 256) * Q4K_BYTES_PER_256


def page_in(thq, torch, ws):
    """One read pass over each weight copy (thq_dequantize_bf16 into one
    scratch buffer), as a decode loop's weights have had before any step:
    a GEMV's first pass over freshly written copies runs about 0.3 us per
    step slower (first 20-step timing in fresh processes: 7.17-7.23 us
    without, 6.88-6.98 us with; the 2400-step default run: 6.87-6.92).
    Setup, not a call of the timed operation."""
    n, k = ws[0].shape
    tmp = torch.empty((n, k), dtype=torch.bfloat16, device="cuda")
    for w in ws:
        thq.check(thq.lib.thq_dequantize_bf16(w.ctx.h, w.h, thq._ptr(tmp), thq._stream()))
    torch.cuda.synchronize()
    del tmp


def make_weights(thq, torch, n, k, copies, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    wf = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    base = thq.QTensor.quantize(wf, thq.Q4_K)
    del wf
    raw = torch.from_numpy(base.data().ravel().copy()).cuda()
    ws = [base] + [thq.QTensor.from_gguf_bytes(thq.Q4_K, raw, n, k) for _ in range(copies - 1)]
    del raw
    torch.cuda.synchronize()
    return ws


def time_graph(torch, fn_list, steps, warmup, start=0):
    """Exactly `warmup` untimed calls, then exactly `steps` timed calls
    (fn_list cycled, all of one shape, the timed calls continuing the
    rotation after the warmup ones).  The first warmup call runs eagerly, so
    that any workspace the shape needs exists before capture; the other
    warmup calls and the timed calls are captured in a HIP graph each.  The
    timed graph is uploaded (hipGraphUpload) before the start event, and a
    GPU sleep before that event keeps the host's graph submission out of the
    timed region.  Returns seconds for the `steps` calls (HIP events on the
    launch stream)."""
    s = torch.cuda.Stream()  # capture needs a non-default stream; everything runs on s
    n = len(fn_list)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        gw = None
        if warmup > 0:
            fn_list[start % n]()
            s.synchronize()
        if warmup > 1:
            gw = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gw, stream=s):
                for i in range(1, warmup):
                    fn_list[(start + i) % n]()
        gt = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gt, stream=s):
            for i in range(steps):
                fn_list[(start + warmup + i) % n]()
        graph_upload(gt, s)
        if gw is not None:
            gw.replay()
        s.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)  # ~1 ms of GPU time while the host enqueues the graph
        e0.record(s)
        gt.replay()
        e1.record(s)
        s.synchronize()
    return e0.elapsed_time(e1) / 1e3


_SPIN_RATE = []


def spin_cycles_per_us(torch):
    """Cycles of torch.cuda._sleep per microsecond on this device (measured
    once with HIP events)."""
    if not _SPIN_RATE:
        cur = torch.cuda.current_stream()
        torch.cuda._sleep(1000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        torch.cuda._sleep(4_000_000)
        e1.record(cur)
        torch.cuda.synchronize()
        _SPIN_RATE.append(4_000_000 / (e0.elapsed_time(e1) * 1e3))
    return _SPIN_RATE[0]


def time_queued(torch, fn_list, steps, warmup, start=0):
    """Exactly `warmup` untimed calls, then exactly `steps` timed calls
    (fn_list cycled, continuing the rotation), all launched from Python on
    the current stream.  The timed calls are queued behind a GPU spin of
    2 ms + 25 us per call, and HIP events on the stream bracket them, so the
    GPU runs them back to back with no host gap and no graph.  Returns
    seconds, or None when the host took longer to launch them than the spin
    lasted (the GPU may then have waited on the host)."""
    n = len(fn_list)
    for i in range(warmup):
        fn_list[(start + i) % n]()
    torch.cuda.synchronize()
    rate = spin_cycles_per_us(torch)
    cur = torch.cuda.current_stream()
    es, e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    h0 = time.perf_counter()
    es.record(cur)
    torch.cuda._sleep(int((2000.0 + 25.0 * steps) * rate))
    e0.record(cur)
    for i in range(steps):
        fn_list[(start + warmup + i) % n]()
    e1.record(cur)
    host_us = (time.perf_counter() - h0) * 1e6
    torch.cuda.synchronize()
    if host_us >= es.elapsed_time(e0) * 1e3:
        return None
    return e0.elapsed_time(e1) / 1e3


def time_steps(torch, fn_list, steps, warmup, graph=False):
    """The headline timing: queued launches (time_queued), or the uploaded
    graph (time_graph) when asked for or when the host could not stay ahead.
    Returns (seconds, "queued" | "graph")."""
    if not graph:
        dt = time_queued(torch, fn_list, steps, warmup)
        if dt is not None:
            return dt, "queued"
        log("host launch outlasted the spin: timing from a HIP graph")
    return time_graph(torch, fn_list, steps, warmup), "graph"


def time_eager(torch, fn_list, steps, warmup):
    """Exactly `warmup` untimed then `steps` timed calls, launched from Python
    on the current stream (for calls far above the host launch cost)."""
    for i in range(warmup):
        fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    torch.cuda._sleep(2_000_000)
    e0.record(cur)
    for i in range(steps):
        fn_list[(warmup + i) % len(fn_list)]()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3


CALIB_BYTES = 28311552  # the copy used to calibrate the PMC byte counters
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic_gemv_q4k_m1_gemm_q4k_m2048.txt")


def source_digest(name: str) -> str:
    """sha256 (first 16 hex digits) of a kernel source under token-horizon_amd/csrc."""
    import hashlib
    with open(os.path.join(ROOT, "token-horizon_amd", "csrc", name), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def measured_traffic():
    """HBM bytes per launch of the two measured kernels (the M=1 GEMV and the
    M=2048 route's bf16 GEMM), from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE passes of this script
    with --pmc-calibration, each scaled by the copy kernel's reading).  The
    summary records the sha256 of the kernel sources it was measured on
    ('source_sha256 <file> <digest>'); a kernel's figure is used only if its
    source is unchanged since, else it is None (stale).  Lines
    'traffic_bytes_per_launch <gemv|gemm> <bytes>'."""
    out, srcs = {}, {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch":
                    out[parts[1]] = int(float(parts[2]))
                elif len(parts) == 3 and parts[0] == "source_sha256":
                    srcs[parts[1]] = parts[2]
    except OSError:
        return {}
    for kind, src in (("gemv", "k_gemv.hip"), ("gemm", "k_gemm_b16.hip")):
        if kind in out and srcs.get(src) != source_digest(src):
            out[kind] = None
    return out


def cpu_baseline(thq_w, n, k, budget_s=10.0):
    """The oracle's AVX2 + OpenMP candle-default (Q8 activations) matmul on a
    bounded sample: repeated M=1 GEMVs of the same Q4_K weight for ~budget_s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import oracle as O

    blocks = thq_w.data()
    x = O.randn(0, 2, 1.0, (1, k))
    threads = O.max_threads()
    O.baseline_matmul(O.Q4_K, blocks, n, k, x, threads)  # warm
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < budget_s:
        O.baseline_matmul(O.Q4_K, blocks, n, k, x, threads)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    byts = q4k_bytes(n, k) + 2 * k + 4 * n
    del np
    return {
        "value": round(byts / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": f"{reps} x Q4_K GEMV M=1 N={n} K={k} (candle default: Q8_K activations, AVX2="
                  f"{bool(O.has_avx2())}), {dt * 1e3:.2f} ms/call",
    }


def ceilings(torch, probe, ws, x1, steps, warmup, graph):
    """Single-launch read ceilings of the GEMV's byte count, rotated and
    timed exactly like the GEMV: a grid-stride read with one 16-B load
    per lane per iteration (2048 and 4096 blocks), the same with four loads
    in flight per lane, and the GEMV's own load pattern (its grid, x first,
    nine 1-KB loads per wave, no math).  Returns (the fastest grid-stride
    time, the load-pattern time, every figure)."""
    N, K = ws[0].shape
    wbytes = q4k_bytes(N, K)
    copies = len(ws)
    bufs = [torch.full((wbytes,), i, dtype=torch.uint8, device="cuda") for i in range(copies)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    cur = lambda: torch.cuda.current_stream().cuda_stream

    def chk(rc):
        if rc != 0:
            raise RuntimeError(f"probe launch failed: {rc}")

    out = {}
    best = None
    for blocks in (2048, 4096):
        pf = [lambda b=b, nb=blocks: chk(probe.thqp_hbm_read(b.data_ptr(), wbytes, nb, sink.data_ptr(), cur()))
              for b in bufs]
        t = time_steps(torch, pf, steps, warmup, graph)[0] / steps
        out[f"grid_stride_1x16B_{blocks}blk_us"] = round(t * 1e6, 3)
        best = t if best is None else min(best, t)
    pf = [lambda b=b: chk(probe.thqp_hbm_read_x4(b.data_ptr(), wbytes, 2048, sink.data_ptr(), cur())) for b in bufs]
    t4 = time_steps(torch, pf, steps, warmup, graph)[0] / steps
    out["grid_stride_4x16B_2048blk_us"] = round(t4 * 1e6, 3)
    best = min(best, t4)
    # the GEMV's own loads over buffers of its row-quad plane's size (N/4
    # quads x K/256 superblocks x 576 B = the weight bytes) and x
    nquads = (N + 3) // 4
    assert nquads * (K // 256) * 576 == wbytes
    pf = [lambda b=b: chk(probe.thqp_gemv_loads(b.data_ptr(), x1.data_ptr(), nquads, K // 256, sink.data_ptr(), cur()))
          for b in bufs]
    tl = time_steps(torch, pf, steps, warmup, graph)[0] / steps
    out["gemv_load_pattern_us"] = round(tl * 1e6, 3)
    del bufs
    return best, tl, out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--copies", type=int, default=24)
    ap.add_argument("--gemm-iters", type=int, default=30)
    ap.add_argument("--gemm-warmup", type=int, default=30,
                    help="untimed GEMM calls before the timed ones (the first few milliseconds of sustained "
                         "MFMA load run 5-10 %% slower than the steady state)")
    ap.add_argument("--gemm-copies", type=int, default=12,
                    help="weight copies the GEMM calls rotate over (12 x 28.3 MB = 340 MB, more than the 256 MB MALL)")
    ap.add_argument("--graph", action="store_true",
                    help="time the headline steps from an uploaded HIP graph instead of queued launches")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-configuration object")
    ap.add_argument("--extra", action="store_true", help="also time the other workloads (formats, modes, layers)")
    ap.add_argument("--only", default=None,
                    help="with --extra: only the sections whose name contains this (gemv_q8_0, q4k, gemm_mid, affine, q6k, "
                         "lm_head_q6k, lm_head_q8_0, topk, decoder), e.g. for a profile of one workload")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="after the run, stream a 28,311,552-byte buffer through an elementwise kernel 24 times "
                         "(reads and writes a known byte count: the reference for scaling rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each projection would be "
              "N-sharded across GPUs with no collective); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import thq

    torch.cuda.init()
    dev = torch.cuda.get_device_properties(0)
    log(f"device: {dev.name}, {dev.multi_processor_count} CUs")
    N, K = 12288, 4096
    copies = args.copies
    steps = args.steps
    if steps < 1 or args.warmup < 0 or args.gemm_copies < 1 or args.gemm_copies > copies:
        print("--steps must be >= 1, --warmup >= 0, 1 <= --gemm-copies <= --copies", file=sys.stderr)
        sys.exit(2)
    log(f"quantizing {copies} copies of Q4_K {N}x{K} ({copies * q4k_bytes(N, K) / 1e6:.0f} MB)")
    ws = make_weights(thq, torch, N, K, copies)
    page_in(thq, torch, ws)
    g = torch.Generator(device="cuda").manual_seed(1)
    x1 = torch.randn((1, K), generator=g, device="cuda").to(torch.bfloat16)
    y1 = torch.empty((1, N), dtype=torch.float32, device="cuda")
    fns = [lambda w=w: thq.matmul(w, x1, out=y1) for w in ws]
    log(f"GEMV M=1: {args.warmup} warmup + {steps} timed steps")
    dt, launch = time_steps(torch, fns, steps, args.warmup, args.graph)
    gemv_bytes = q4k_bytes(N, K) + 2 * K + 4 * N
    per = dt / steps
    gbs = gemv_bytes / per / 1e9
    log(f"GEMV M=1: {per * 1e6:.2f} us/call, {gbs:.0f} GB/s")

    # single-launch read ceilings of the same byte count, launched, rotated
    # and timed exactly like the GEMV
    wbytes = q4k_bytes(N, K)
    ceil_t, load_t, ceil_detail = ceilings(torch, load_probe(), ws, x1, steps, args.warmup, args.graph)
    log(f"HBM read of the same {wbytes} B: {ceil_t * 1e6:.2f} us/launch ({wbytes / ceil_t / 1e9:.0f} GB/s); "
        f"the GEMV's load pattern alone: {load_t * 1e6:.2f} us")

    # prefill GEMM M=2048 (bf16 out), rotating --gemm-copies weight copies
    M = 2048
    xg = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    yg = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gfns = [lambda w=w: thq.matmul(w, xg, out=yg) for w in ws[:args.gemm_copies]]
    it = args.gemm_iters
    log(f"GEMM M={M}: {it} iterations over {args.gemm_copies} weight copies")
    dtg = time_eager(torch, gfns, it, args.gemm_warmup)  # untimed calls stated in "gemm"
    flops = 2.0 * M * N * K
    tflops = flops / (dtg / it) / 1e12
    log(f"GEMM M={M}: {dtg / it * 1e6:.1f} us/call, {tflops:.1f} TFLOP/s")
    # the vendor library's plain bf16 GEMM on the same shape with unquantized
    # weights (hipBLASLt through torch.matmul): a reference point for the MFMA
    # rate this part sustains on this shape, with no dequantization at all
    wbf = torch.randn((N, K), generator=g, device="cuda").to(torch.bfloat16)
    wbt = wbf.t()
    vend = time_eager(torch, [lambda: torch.matmul(xg, wbt, out=yg)], it, args.gemm_warmup)
    vend_tf = flops / (vend / it) / 1e12
    del wbf, wbt, xg, yg
    log(f"vendor bf16 GEMM (unquantized weights) M={M}: {vend / it * 1e6:.1f} us/call, {vend_tf:.1f} TFLOP/s")

    configs = None
    if not args.no_configs:
        configs = run_configs(torch, thq, g, ws)
    extra = {}
    if args.extra:
        extra = run_extra(torch, thq, g, args.only)
    if args.pmc_calibration:
        src = torch.empty(CALIB_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(24):  # elementwise kernel reading and writing exactly CALIB_BYTES
            torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    traffic = measured_traffic()

    out = {
        "metric": "quant-GEMV HBM GB/s @M=1 + GEMM TFLOP/s @M=2048 (Q4_K, K=4096 N=12288)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(per * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x bf16 -> f32 (f32 accumulate)",
        "data": "synthetic: W ~ N(0,0.02) quantized on device, x ~ N(0,1) bf16 (torch seeded)",
        "config": {"workload": "Q4_K decode GEMV M=1, N=12288, K=4096 (Qwen3-8B-class gate/up projection)",
                   "rotating_weight_copies": copies, "launch": ("queued behind a GPU spin that outlasts the host's launches" if launch == "queued"
                              else "hip-graph, uploaded before timing"),
                   "page_in": "each copy read once (thq_dequantize_bf16) after it is written, before the warmup steps",
                   "algorithmic_bytes_per_call": gemv_bytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic.get("gemv"),
                     "traffic_profile": os.path.relpath(TRAFFIC_FILE, ROOT),
                     "single_launch_read_ceiling": {
                         "kernels": "libthq_probe.so (bench-only): grid-stride 16-B reads of the same "
                                    f"{wbytes} weight bytes, one or four loads in flight per lane; and the "
                                    "GEMV's own load pattern with no math; same rotation and timing",
                         **ceil_detail,
                         "us": round(ceil_t * 1e6, 3), "GBs": round(wbytes / ceil_t / 1e9, 1),
                         "frac_of_peak": round(wbytes / ceil_t / 1e9 / HBM_PEAK_GBS, 4),
                         "gemv_time_over_ceiling": round(per / ceil_t, 3),
                         "gemv_time_over_load_pattern": round(per / load_t, 3)}},
        "gemm": {"workload": "Q4_K prefill GEMM M=2048, N=12288, K=4096, bf16 x -> bf16 y",
                 "route": GEMM_ROUTE,
                 "tflops": round(tflops, 1), "us_per_call": round(dtg / it * 1e6, 1), "iters": it,
                 "warmup": args.gemm_warmup, "rotating_weight_copies": args.gemm_copies,
                 "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS,
                              "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                              "traffic": traffic.get("gemm")},
                 "vendor_bf16_reference": {
                     "kernel": "torch.matmul (hipBLASLt) on unquantized bf16 weights of the same shape",
                     "tflops": round(vend_tf, 1), "us_per_call": round(vend / it * 1e6, 1),
                     "frac_of_peak": round(vend_tf / BF16_PEAK_TFLOPS, 4),
                     "quantized_time_over_vendor": round(dtg / vend, 3)}},
    }
    if configs:
        out["configs"] = configs
    if extra:
        out["extra"] = extra
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle AVX2 Q8-activation GEMV), ~10 s")
        out["cpu_baseline"] = cpu_baseline(ws[0], N, K)
    print(json.dumps(out), flush=True)


def line(us, work, unit, peak):
    """One configuration's entry: time per call, rate and roofline fraction."""
    rate = work / (us * 1e-6) / (1e9 if unit == "GB/s" else 1e12)
    return {"us": round(us, 2), unit: round(rate, 1), "frac": round(rate / peak, 4)}


def run_configs(torch, thq, g, ws_gu):
    """Every benchmark configuration of the path, on synthetic inputs of its
    shapes, weights rotated beyond the MALL.  Decode lines (HBM-bound, a few
    microseconds per call) run from an uploaded HIP graph; GEMM, LM-head and
    prefill-layer lines are eager (each call far above launch cost)."""
    res = {}
    HB, MF = HBM_PEAK_GBS, BF16_PEAK_TFLOPS

    def graph_us(fns, steps=240):
        return time_graph(torch, fns, steps, 16) / steps * 1e6

    def eager_us(fns, it, warm):
        return time_eager(torch, fns, it, warm) / it * 1e6

    # 1: Q8_0 3072 x 1024 with f32 activations, M = 1 (96 copies: 322 MB)
    log("configs: Q8_0 3072x1024, f32 x")
    n, k = 3072, 1024
    base = make_q8_0(thq, torch, n, k, seed=0)
    raw = torch.from_numpy(base.data().ravel().copy()).cuda()
    w8 = [base] + [thq.QTensor.from_gguf_bytes(thq.Q8_0, raw, n, k) for _ in range(95)]
    del raw
    x = torch.randn((1, k), generator=g, device="cuda")
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    us = graph_us([lambda w=w: thq.matmul(w, x, out=y) for w in w8])
    res["c1_q8_0_n3072_k1024_m1_f32x"] = line(us, n * (k // 32) * 34 + 4 * k + 4 * n, "GB/s", HB)
    del w8
    # 2 and 3: Q4_K gate/up shape (the headline copies) and down shape
    log("configs: Q4_K decode M=1,2,4,8 and prefill M=128,512,2048 on both shapes")
    for (n, k) in [(12288, 4096), (4096, 12288)]:
        ws = ws_gu if n == 12288 else make_weights(thq, torch, n, k, 24, seed=5 + n)
        for m in (1, 2, 4, 8):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            us = graph_us([lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws])
            res[f"c2_q4k_n{n}_k{k}_m{m}"] = line(us, q4k_bytes(n, k) + m * (2 * k + 4 * n), "GB/s", HB)
        for m in (128, 512, 2048):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
            it = 40 if m < 2048 else 24
            us = eager_us([lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws[:12]], it, 12)
            res[f"c3_q4k_n{n}_k{k}_m{m}"] = line(us, 2.0 * m * n * k, "TFLOP/s", MF)
        if ws is not ws_gu:
            del ws
    # 4: verify LM head, Q8_0 151936 x 4096 (661 MB, beyond the MALL), logits + argmax
    log("configs: Q8_0 LM head 151936x4096 + argmax, M=5,40")
    V, H = 151936, 4096
    wl = make_q8_0(thq, torch, V, H, seed=11)
    for m in (5, 40):
        x = torch.randn((m, H), generator=g, device="cuda").to(torch.bfloat16)
        lg = torch.empty((m, V), dtype=torch.float32, device="cuda")
        ix = torch.empty((m,), dtype=torch.int32, device="cuda")
        us = eager_us([lambda x=x, lg=lg, ix=ix: thq.matmul_argmax(wl, x, logits=lg, idx=ix)], 30, 4)
        res[f"c4_lm_head_q8_0_m{m}"] = line(us, V * (H // 32) * 34 + m * (2 * H + 4 * V), "GB/s", HB)
    del wl
    # 5: decoder layer (QKV, o, gate/up + SiLU, down), 4 layers rotating (434 MB)
    log("configs: Q4_K decoder layer M=1,256")
    layers = make_layers(thq, torch, 4)
    layer_bytes = q4k_bytes(6144, 4096) + q4k_bytes(4096, 4096) + q4k_bytes(24576, 4096) + q4k_bytes(4096, 12288)
    for m in (1, 256):
        fns = layer_fns(torch, thq, g, layers, m)
        if m == 1:
            us = graph_us(fns, 96)
            res["c5_decoder_layer_q4k_m1"] = line(us, layer_bytes + 4 * (2 * 4096) + 2 * 12288, "GB/s", HB)
        else:
            us = eager_us(fns, 24, 4)
            flops = 2.0 * m * (6144 + 4096 + 24576) * 4096 + 2.0 * m * 4096 * 12288
            res["c5_decoder_layer_q4k_m256"] = line(us, flops, "TFLOP/s", MF)
    del layers
    torch.cuda.synchronize()
    return res


def make_layers(thq, torch, count):
    """Qwen3-8B-class decoder layers of Q4_K weights: (QKV 6144x4096, o
    4096x4096, fused gate/up 2x12288x4096, down 4096x12288)."""
    layers = []
    for i in range(count):
        def q(n, k, s):
            gg = torch.Generator(device="cuda").manual_seed(100 + 10 * i + s)
            wf = torch.randn((n, k), generator=gg, device="cuda", dtype=torch.float32) * 0.02
            w = thq.QTensor.quantize(wf, thq.Q4_K)
            del wf
            return w
        gate, up = q(12288, 4096, 2), q(12288, 4096, 3)
        layers.append((q(6144, 4096, 0), q(4096, 4096, 1), thq.QTensor.fuse([gate, up]), q(4096, 12288, 4)))
        del gate, up
    torch.cuda.synchronize()
    return layers


def layer_fns(torch, thq, g, layers, m):
    """One call per layer: the four projections back to back on one stream
    (bf16 outputs; down reads the gate/up output)."""
    x = torch.randn((m, 4096), generator=g, device="cuda").to(torch.bfloat16)
    qkv = torch.empty((m, 6144), dtype=torch.bfloat16, device="cuda")
    o = torch.empty((m, 4096), dtype=torch.bfloat16, device="cuda")
    h = torch.empty((m, 12288), dtype=torch.bfloat16, device="cuda")
    d = torch.empty((m, 4096), dtype=torch.bfloat16, device="cuda")

    def layer(L):
        thq.matmul(L[0], x, out=qkv)
        thq.matmul(L[1], x, out=o)
        thq.gate_up_silu(L[2], x, out=h)
        thq.matmul(L[3], h, out=d)

    return [lambda L=L: layer(L) for L in layers]


def make_q8_0(thq, torch, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    wf = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    w = thq.QTensor.quantize(wf, thq.Q8_0)
    del wf
    torch.cuda.synchronize()
    return w


def make_affine(thq, torch, n, k, copies, seed):
    """MLX affine 4-bit weights (the engine's QLin arrays) built on the device:
    random nibbles, scales 0.002 + U*0.02 and biases U(-0.1, 0.1) in bf16."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    wq = torch.randint(-(1 << 31), 1 << 31, (n, k // 8), generator=g, device="cuda", dtype=torch.int64)
    wq = wq.to(torch.int32)
    ng = k // 64
    sc = 0.002 + torch.rand((n, ng), generator=g, device="cuda") * 0.02
    bi = (torch.rand((n, ng), generator=g, device="cuda") - 0.5) * 0.2
    sb = torch.cat([sc, bi], dim=1).to(torch.bfloat16).contiguous().view(torch.int16)
    ws = [thq.QTensor.from_affine(wq, sb, n, k) for _ in range(copies)]
    del wq, sb
    torch.cuda.synchronize()
    return ws


def make_q6k(thq, torch, n, k, copies, seed):
    """Q6_K weights from random GGUF block bytes built on the device: every
    code and scale byte uniform, d = f16 of N(0, 2e-4)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    raw = torch.randint(0, 256, (n, k // 256, 210), generator=g, device="cuda", dtype=torch.uint8)
    d = (torch.randn((n, k // 256), generator=g, device="cuda") * 2e-4).to(torch.float16)
    raw[:, :, 208:210] = d.view(torch.uint8).view(n, k // 256, 2)
    ws = [thq.QTensor.from_gguf_bytes(thq.Q6_K, raw.view(-1), n, k) for _ in range(copies)]
    del raw, d
    torch.cuda.synchronize()
    return ws


def q6k_bytes(n, k):
    return n * (k // 256) * 210


def run_extra(torch, thq, g, only=None):
    """Every other configuration: decode GEMV M in {1,2,4,8} (and M in
    {3,4,5,8} on weights with a tile plane) and prefill GEMM
    M in {128,512,2048} on both Qwen3-8B MLP weight shapes, M in
    {32,...,512} on them and on the fused gate/up (plus Q8ACT GEMV,
    also on the tile plane at M in {2,5,8} with the dot alone over a
    prepared Q8_K buffer, and the MLX affine format on the gate/up shape), Q8_0 decode GEMV at
    M in {1,8} on both shapes, the Q8_0 LM head with argmax at M in {1,5,40}
    (logits, and the fused epilogue without logits for M <= 8), and one
    decoder layer's four projections at M in {1,5,256} (and in Q8ACT mode at
    M in {1,5}).  GEMV lines rotate 24 weight copies (> MALL) inside a HIP
    graph; GEMM and LM-head lines are eager (each call far above launch cost)."""
    res = {}

    def want(section):
        return only is None or only in section

    def gemv_line(fns, byts, steps=960):
        dt = time_graph(torch, fns, steps, 24) / steps
        return {"us": round(dt * 1e6, 2), "GBs": round(byts / dt / 1e9, 1)}

    for (n, k) in [(12288, 4096), (4096, 12288)] if want("gemv_q8_0") else []:
        log(f"extra: Q8_0 {n}x{k} decode GEMV")
        base = make_q8_0(thq, torch, n, k, seed=7 + n)
        raw = torch.from_numpy(base.data().ravel().copy()).cuda()
        ws = [base] + [thq.QTensor.from_gguf_bytes(thq.Q8_0, raw, n, k) for _ in range(23)]
        del raw
        for m in (1, 8):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws]
            res[f"gemv_q8_0_n{n}_k{k}_m{m}"] = gemv_line(fns, n * (k // 32) * 34 + m * (2 * k + 4 * n))
        del ws
    for (n, k) in [(12288, 4096), (4096, 12288)] if want("q4k") else []:
        log(f"extra: Q4_K {n}x{k}")
        ws = make_weights(thq, torch, n, k, 24, seed=5 + n)
        for m in (1, 2, 4, 8):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws]
            res[f"gemv_q4k_n{n}_k{k}_m{m}"] = gemv_line(fns, q4k_bytes(n, k) + m * (2 * k + 4 * n))
        for m in (1, 8):  # candle's default semantics: x quantized to Q8_K, integer dots
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y, flags=thq.MODE_Q8ACT) for w in ws]
            res[f"gemv_q4k_q8act_n{n}_k{k}_m{m}"] = gemv_line(fns, q4k_bytes(n, k) + m * (2 * k + 4 * n))
        for m in (128, 512, 2048):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
            fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws[:12]]
            it = 30 if m >= 512 else 120
            dt = time_eager(torch, fns, it, 6) / it
            res[f"gemm_q4k_n{n}_k{k}_m{m}"] = {"us": round(dt * 1e6, 1),
                                               "TFLOPs": round(2.0 * m * n * k / dt / 1e12, 1)}
        # the same weights with their 32-row tile plane (thq_weight_add_tiles):
        # 3..8 rows of a plain projection take the tile-plane decode GEMV
        for w in ws:
            w.add_tiles()
        for m in (3, 4, 5, 8):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws]
            res[f"gemv_q4k_tiles_n{n}_k{k}_m{m}"] = gemv_line(fns, q4k_bytes(n, k) + m * (2 * k + 4 * n))
        # candle's default semantics on the tile plane (int8 matrix-core
        # dots): the one-call form (quantize + dot) and the dot alone over a
        # prepared Q8_K buffer
        for m in (2, 5, 8):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y, flags=thq.MODE_Q8ACT) for w in ws]
            res[f"gemv_q4k_tiles_q8act_n{n}_k{k}_m{m}"] = gemv_line(fns, q4k_bytes(n, k) + m * (2 * k + 4 * n))
            pre = thq.Q8Act(x, thq.Q8_K)
            fns = [lambda w=w, pre=pre: pre.matmul(w, torch.float32) for w in ws]
            planes = m * (k + k // 256 * 4 + k // 32 * 2)
            res[f"gemv_q4k_tiles_q8act_dot_n{n}_k{k}_m{m}"] = gemv_line(fns, q4k_bytes(n, k) + planes + 4 * m * n)
        del ws

    # tens to hundreds of rows on Q4_K (the streaming mid-M GEMM's range up
    # to 128 rows, the tile / dequantize GEMMs past it): both MLP shapes and
    # the fused gate/up, 12 weight copies rotated (> MALL)
    for (n, k, gu) in [(12288, 4096, False), (4096, 12288, False), (24576, 4096, True)] if want("gemm_mid") else []:
        log(f"extra: Q4_K {n}x{k}{' gate/up' if gu else ''} at 32..512 rows")
        ws = make_weights(thq, torch, n, k, 12, seed=9 + n)
        nout = n // 2 if gu else n
        for m in (32, 64, 96, 128, 256, 512):
            x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty((m, nout), dtype=torch.bfloat16, device="cuda")
            if gu:
                fns = [lambda w=w, x=x, y=y: thq.gate_up_silu(w, x, out=y) for w in ws]
            else:
                fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws]
            dt = time_eager(torch, fns, 120, 12) / 120
            res[f"gemm_mid_q4k_n{n}_k{k}{'_gu' if gu else ''}_m{m}"] = {
                "us": round(dt * 1e6, 1), "TFLOPs": round(2.0 * m * n * k / dt / 1e12, 1)}
        del ws

    if want("affine"):
        run_affine(torch, thq, g, res, gemv_line)
    if want("q6k"):
        run_q6k(torch, thq, g, res, gemv_line)
    if want("lm_head_q6k"):
        run_lm_head_q6k(torch, thq, g, res)
    if want("lm_head_q8_0"):
        run_lm_head_q8_0(torch, thq, g, res)
    if want("topk"):
        run_topk(torch, thq, g, res)
    if want("decoder"):
        run_decoder(torch, thq, g, res)
    return res


def run_affine(torch, thq, g, res, gemv_line):
    log("extra: MLX affine 4-bit 12288x4096 (the engine's QLin format)")
    n, k = 12288, 4096
    ws = make_affine(thq, torch, n, k, 24, seed=77)
    for m in (1, 8):
        x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws]
        res[f"gemv_affine_n{n}_k{k}_m{m}"] = gemv_line(fns, q4k_bytes(n, k) + m * (2 * k + 4 * n))
    x = torch.randn((2048, k), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((2048, n), dtype=torch.bfloat16, device="cuda")
    fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws[:12]]
    dt = time_eager(torch, fns, 30, 6) / 30
    res[f"gemm_affine_n{n}_k{k}_m2048"] = {"us": round(dt * 1e6, 1), "TFLOPs": round(2.0 * 2048 * n * k / dt / 1e12, 1)}
    del ws


def run_q6k(torch, thq, g, res, gemv_line):
    for (n, k) in [(12288, 4096), (4096, 12288)]:
        log(f"extra: Q6_K {n}x{k}")
        ws = make_q6k(thq, torch, n, k, 24, seed=91 + n)
        x = torch.randn((1, k), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((1, n), dtype=torch.float32, device="cuda")
        fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws]
        res[f"gemv_q6k_n{n}_k{k}_m1"] = gemv_line(fns, q6k_bytes(n, k) + 2 * k + 4 * n)
        x = torch.randn((2048, k), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((2048, n), dtype=torch.bfloat16, device="cuda")
        fns = [lambda w=w, x=x, y=y: thq.matmul(w, x, out=y) for w in ws[:12]]
        dt = time_eager(torch, fns, 30, 6) / 30
        res[f"gemm_q6k_n{n}_k{k}_m2048"] = {"us": round(dt * 1e6, 1), "TFLOPs": round(2.0 * 2048 * n * k / dt / 1e12, 1)}
        del ws


def run_lm_head_q6k(torch, thq, g, res):
    log("extra: Q6_K LM head 151936x4096 + argmax (a Q4_K_M file's output head)")
    V, H = 151936, 4096
    wl = make_q6k(thq, torch, V, H, 1, seed=13)[0]
    x = torch.randn((1, H), generator=g, device="cuda").to(torch.bfloat16)
    logits = torch.empty((1, V), dtype=torch.float32, device="cuda")
    idx = torch.empty((1,), dtype=torch.int32, device="cuda")
    fn = lambda x=x, lg=logits, ix=idx: thq.matmul_argmax(wl, x, logits=lg, idx=ix)
    dt = time_eager(torch, [fn], 60, 4) / 60
    res["lm_head_q6k_m1"] = {"us": round(dt * 1e6, 1), "GBs": round((q6k_bytes(V, H) + 2 * H + 4 * V) / dt / 1e9, 1)}
    for m in (16, 40):  # batched verify: exact weights (16: the decode GEMV, 40: the wide GEMV)
        x = torch.randn((m, H), generator=g, device="cuda").to(torch.bfloat16)
        logits = torch.empty((m, V), dtype=torch.float32, device="cuda")
        idx = torch.empty((m,), dtype=torch.int32, device="cuda")
        fn = lambda x=x, lg=logits, ix=idx: thq.matmul_argmax(wl, x, logits=lg, idx=ix)
        dt = time_eager(torch, [fn], 20, 2) / 20
        res[f"lm_head_q6k_m{m}"] = {"us": round(dt * 1e6, 1),
                                    "GBs": round((q6k_bytes(V, H) + m * (2 * H + 4 * V)) / dt / 1e9, 1)}
    del wl


def run_lm_head_q8_0(torch, thq, g, res):
    log("extra: Q8_0 LM head 151936x4096 + argmax")
    V, H = 151936, 4096
    wl = make_q8_0(thq, torch, V, H, seed=11)
    for m in (1, 5, 40):
        x = torch.randn((m, H), generator=g, device="cuda").to(torch.bfloat16)
        logits = torch.empty((m, V), dtype=torch.float32, device="cuda")
        idx = torch.empty((m,), dtype=torch.int32, device="cuda")
        fn = lambda x=x, lg=logits, ix=idx: thq.matmul_argmax(wl, x, logits=lg, idx=ix)
        it = 40
        dt = time_eager(torch, [fn], it, 4) / it
        byts = V * (H // 32) * 34 + m * (2 * H + 4 * V)
        res[f"lm_head_q8_0_m{m}"] = {"us": round(dt * 1e6, 1), "GBs": round(byts / dt / 1e9, 1)}
        if m <= 8:
            # greedy decode without logits in HBM: the fused (max, index) epilogue
            fn = lambda x=x, ix=idx: thq.matmul_argmax(wl, x, want_logits=False, idx=ix,
                                                       flags=thq.MODE_ARGMAX_FUSED)
            dt = time_eager(torch, [fn], it, 4) / it
            byts = V * (H // 32) * 34 + m * 2 * H
            res[f"lm_head_q8_0_fused_m{m}"] = {"us": round(dt * 1e6, 1), "GBs": round(byts / dt / 1e9, 1)}
    del wl


def run_topk(torch, thq, g, res):
    log("extra: Q8_0 LM head 151936x4096 + exact top-32 (sampled verify)")
    V, H = 151936, 4096
    wl = make_q8_0(thq, torch, V, H, seed=11)
    for m in (5, 40):
        x = torch.randn((m, H), generator=g, device="cuda").to(torch.bfloat16)
        fn = lambda x=x: thq.matmul_topk(wl, x, 32)
        it = 40
        dt = time_eager(torch, [fn], it, 4) / it
        byts = V * (H // 32) * 34 + m * (2 * H + 4 * V)
        res[f"lm_head_topk32_q8_0_m{m}"] = {"us": round(dt * 1e6, 1), "GBs": round(byts / dt / 1e9, 1)}
        lg = torch.randn((m, V), generator=g, device="cuda")
        fn = lambda lg=lg: thq.topk(lg, 32)
        # a HIP graph: a call's host cost (~40 us) is above its GPU time
        dt = time_graph(torch, [fn], 200, 10) / 200
        res[f"topk32_only_m{m}"] = {"us": round(dt * 1e6, 1), "GBs": round(m * V * 4 / dt / 1e9, 1)}
    del wl


def run_decoder(torch, thq, g, res):
    log("extra: decoder layer (QKV, o, fused gate/up + silu, down), 4 layers rotating")
    layers = make_layers(thq, torch, 4)
    layer_bytes = q4k_bytes(6144, 4096) + q4k_bytes(4096, 4096) + q4k_bytes(24576, 4096) + q4k_bytes(4096, 12288)
    # M = 5: one speculative-verify step (4 drafted tokens + 1), with and
    # without the weights' tile planes
    for m, tiles in ((1, False), (5, False), (5, True), (256, False)):
        if tiles:
            for L in layers:
                for w in L:
                    w.add_tiles()
        x = torch.randn((m, 4096), generator=g, device="cuda").to(torch.bfloat16)
        qkv = torch.empty((m, 6144), dtype=torch.bfloat16, device="cuda")
        o = torch.empty((m, 4096), dtype=torch.bfloat16, device="cuda")
        h = torch.empty((m, 12288), dtype=torch.bfloat16, device="cuda")
        d = torch.empty((m, 4096), dtype=torch.bfloat16, device="cuda")

        def layer(L, x=x, qkv=qkv, o=o, h=h, d=d):
            thq.matmul(L[0], x, out=qkv)
            thq.matmul(L[1], x, out=o)
            thq.gate_up_silu(L[2], x, out=h)
            thq.matmul(L[3], h, out=d)

        fns = [lambda L=L: layer(L) for L in layers]
        if m <= 8:
            steps = 192
            dt = time_graph(torch, fns, steps, 8) / steps
        else:
            it = 40
            dt = time_eager(torch, fns, it, 4) / it
        flops = 2.0 * m * (6144 + 4096 + 24576) * 4096 + 2.0 * m * 4096 * 12288
        res[f"decoder_layer_q4k_m{m}" + ("_tiles" if tiles else "")] = {
            "us": round(dt * 1e6, 1), "GBs": round(layer_bytes / dt / 1e9, 1), "TFLOPs": round(flops / dt / 1e12, 2)}
    # candle's default semantics (Q8 activations) with quantize-once operands:
    # x quantized once for QKV and o; the gate/up epilogue either emits down's
    # operand or down's input is quantized by its own launch.  The weights
    # carry their tile planes from here on: M = 1 keeps the row-quad kernels,
    # M = 5 runs the int8 tile kernels
    for m, emit in ((1, False), (1, True), (5, False), (5, True)):
        x = torch.randn((m, 4096), generator=g, device="cuda").to(torch.bfloat16)

        def layer8(L, x=x, emit=emit):
            a = thq.Q8Act(x, thq.Q8_K)
            a.matmul(L[0], torch.bfloat16)
            a.matmul(L[1], torch.bfloat16)
            if emit:
                _, hq = a.gate_up_silu_emit(L[2])
            else:
                hq = thq.Q8Act(a.gate_up_silu(L[2]), thq.Q8_K)
            hq.matmul(L[3], torch.bfloat16)

        fns = [lambda L=L: layer8(L) for L in layers]
        steps = 192
        dt = time_graph(torch, fns, steps, 8) / steps
        res[f"decoder_layer_q4k_q8act_m{m}_{'emit' if emit else 'prepare'}" + ("_tiles" if m > 1 else "")] = {
            "us": round(dt * 1e6, 1)}


if __name__ == "__main__":
    main()
