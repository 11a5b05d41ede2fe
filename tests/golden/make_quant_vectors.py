"""Golden vectors for the Q4_K and Q8_K quantizers (candle's from_float).

    python tests/golden/make_quant_vectors.py   # rewrites quant_vectors.json

The algorithm lives in [ext] candle-core 0.11.0 (engine/Cargo.lock:253-256),
src/quantized/utils.rs make_qkx1_quants and k_quants.rs BlockQ4K /
BlockQ8K::from_float, which is not in the reference tree and cannot be built
here (no Rust).  This script traces that published algorithm step by step in
IEEE single precision with numpy float32 scalars — one rounding per
operation, in the order the Rust source evaluates it, Rust's f32::round
(half away from zero) for nearest_int — independently of the C oracle.  The
traced outputs are written as literal bytes; tests/test_oracle.py holds the
oracle to them.

Cases are chosen so that a plausible transcription slip changes the output:
  * `qkx1`: sub-blocks whose refinement does not converge before the 5th pass
    (so ntry 4, 5 and 6 give three different answers), traced at nmax 15;
    the file also records what nmax 14 and ntry 1 would give.
  * `q4k`: whole superblocks (Gaussian, all-positive so the min clamps to 0,
    mixed constant / outlier sub-blocks, and one drawn so that its bytes
    differ for ntry 4, 5 and 6), checked byte for byte; the script checks
    that 64/max in place of 63/max changes them.
  * `q8k`: blocks with exact x.5 ties at iscale = 1 (round half away from
    zero gives +-3 / +-1 where half-to-even gives +-2 / 0), a positive
    maximum (clamp of +128 to 127), and the first-of-equal-magnitude rule.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

f32 = np.float32
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "quant_vectors.json")


def rround(v) -> float:
    """Rust f32::round of a float32 value: half away from zero (exact in f64)."""
    v = float(v)
    return math.copysign(math.floor(abs(v) + 0.5), v)


def nearest_int(v) -> int:
    return int(rround(v))


def qkx1(nmax: int, ntry: int, x: np.ndarray):
    """make_qkx1_quants(nmax, ntry, x) -> (scale, -min, levels), traced in f32."""
    n = len(x)
    xs = [f32(v) for v in x]
    lv = [0] * n
    mn, mx = min(xs), max(xs)
    if mx == mn:
        return f32(0), f32(0), lv
    mn = mn if mn < f32(0) else f32(0)
    iscale = f32(nmax) / f32(mx - mn)
    scale = f32(1) / iscale
    for _ in range(ntry):
        sumlx = f32(0)
        suml2 = 0
        changed = False
        for i in range(n):
            li = min(max(nearest_int(f32(iscale * f32(xs[i] - mn))), 0), nmax)
            if li != lv[i]:
                lv[i] = li
                changed = True
            sumlx = f32(sumlx + f32(f32(xs[i] - mn) * f32(li)))
            suml2 += li * li
        scale = f32(sumlx / f32(suml2))
        s = f32(0)
        for i in range(n):
            s = f32(s + f32(xs[i] - f32(scale * f32(lv[i]))))
        mn = f32(s / f32(n))
        if mn > f32(0):
            mn = f32(0)
        iscale = f32(f32(1) / scale)
        if not changed:
            break
    return scale, f32(-mn), lv


def f16(v) -> np.float16:
    return np.float32(v).astype(np.float16)  # round to nearest even


def scale_min_k4(j: int, q) -> tuple[int, int]:
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def q4k_block(x: np.ndarray, inv_num: float = 63.0, ntry: int = 5) -> bytes:
    """BlockQ4K::from_float of 256 values -> 144 bytes (d, dmin, scales[12], qs[128])."""
    scales, mins = [], []
    for j in range(8):
        s, m, _ = qkx1(15, ntry, x[32 * j: 32 * j + 32])
        scales.append(s)
        mins.append(m)
    max_scale, max_min = f32(0), f32(0)
    for v in scales:
        max_scale = v if v > max_scale else max_scale  # val.max(max); no NaN here
    for v in mins:
        max_min = v if v > max_min else max_min
    inv_scale = f32(f32(inv_num) / max_scale) if max_scale > 0 else f32(0)
    inv_min = f32(f32(inv_num) / max_min) if max_min > 0 else f32(0)
    sc = [0] * 12
    for j in range(8):
        ls = min(nearest_int(f32(inv_scale * scales[j])), 63)
        lm = min(nearest_int(f32(inv_min * mins[j])), 63)
        if j < 4:
            sc[j] = ls
            sc[j + 4] = lm
        else:
            sc[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            sc[j - 4] |= (ls >> 4) << 6
            sc[j] |= (lm >> 4) << 6
    d = f16(f32(max_scale / f32(63)))
    dmin = f16(f32(max_min / f32(63)))
    L = [0] * 256
    for j in range(8):
        s, m = scale_min_k4(j, sc)
        dd = f32(f32(d) * f32(s))
        if dd != 0:
            dm = f32(f32(dmin) * f32(m))
            for i in range(32):
                L[32 * j + i] = min(max(nearest_int(f32(f32(f32(x[32 * j + i]) + dm) / dd)), 0), 15)
    qs = bytearray(128)
    for j in range(0, 256, 64):
        for i in range(32):
            qs[j // 2 + i] = L[j + i] | (L[j + i + 32] << 4)
    return d.tobytes() + dmin.tobytes() + bytes(sc) + bytes(qs)


def q8k_block(x: np.ndarray) -> bytes:
    """BlockQ8K::from_float of 256 values -> 292 bytes (f32 d, i8 qs[256], i16 bsums[16])."""
    mx, amax = f32(0), f32(0)
    for v in x:
        v = f32(v)
        if amax < abs(v):
            amax = abs(v)
            mx = v
    if amax == 0:
        return bytes(292)
    iscale = f32(f32(-128) / mx)
    qs = []
    for v in x:
        r = rround(f32(iscale * f32(v)))
        qs.append(int(min(r, 127.0)))  # as i8: in range here
    bs = [sum(qs[16 * j: 16 * j + 16]) for j in range(16)]
    d = f32(f32(1) / iscale)
    return d.tobytes() + np.array(qs, np.int8).tobytes() + np.array(bs, np.int16).tobytes()


def hexf(a) -> list[str]:
    return [f"{int(v):08x}" for v in np.asarray(a, np.float32).view(np.uint32)]


def main() -> None:
    rng = np.random.default_rng(20261202)
    # qkx1: sub-blocks whose levels still change in passes 5 and 6
    qk = []
    tries = 0
    while len(qk) < 3:
        tries += 1
        x = (rng.standard_normal(32) * 0.02).astype(np.float32)
        if len(qk) == 1:
            x = np.abs(x) + f32(0.01)  # all positive: min clamps to 0 on every pass
        r4, r5, r6 = qkx1(15, 4, x), qkx1(15, 5, x), qkx1(15, 6, x)
        if r4[2] == r5[2] or r5[2] == r6[2]:
            continue
        s14, m14, l14 = qkx1(14, 5, x)
        s1, m1, l1 = qkx1(15, 1, x)
        qk.append({"x": hexf(x), "scale": hexf([r5[0]])[0], "min": hexf([r5[1]])[0], "levels": r5[2],
                   "levels_ntry4": r4[2], "levels_ntry6": r6[2], "levels_nmax14": l14, "levels_ntry1": l1})
    # q4k: whole superblocks
    q4 = []
    cases = [
        (rng.standard_normal(256) * 0.02).astype(np.float32),
        (np.abs(rng.standard_normal(256)) * 0.02 + 0.001).astype(np.float32),
    ]
    mixed = (rng.standard_normal(256) * 0.02).astype(np.float32)
    mixed[32:64] = f32(0.0125)        # a constant sub-block: (0, 0)
    mixed[70] = f32(0.25)             # an outlier sets max_scale
    mixed[200] = f32(-0.3)            # and another sets max_min
    cases.append(mixed)
    # a superblock whose bytes differ for ntry 4, 5 and 6 (the pass count at
    # the from_float call site)
    draws = 0
    while True:
        draws += 1
        x = (rng.standard_normal(256) * 0.02).astype(np.float32)
        b5 = q4k_block(x)
        if q4k_block(x, ntry=6) != b5 and q4k_block(x, ntry=4) != b5:
            cases.append(x)
            break
    for x in cases:
        blk = q4k_block(x)
        assert q4k_block(x, 64.0) != blk, "64/max must change the block"
        q4.append({"x": hexf(x), "block": blk.hex()})
    # q8k: ties at iscale = 1, positive max, first of equal magnitudes
    q8 = []
    t = np.zeros(256, np.float32)
    t[0] = -128.0                      # max = -128 -> iscale = 1, d = 1
    t[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -127.5]
    t[9] = 128.0                       # same |x| as t[0], later: not the max; 128 -> clamp 127
    t[10:] = (rng.standard_normal(246) * 20).astype(np.float32)
    q8.append({"x": hexf(t), "block": q8k_block(t).hex()})
    u = (rng.standard_normal(256) * 1.5).astype(np.float32)
    u[17] = f32(6.0)                   # positive max: iscale < 0, u[17] -> -128
    q8.append({"x": hexf(u), "block": q8k_block(u).hex()})
    with open(OUT, "w") as f:
        json.dump({"generator": "tests/golden/make_quant_vectors.py", "qkx1": qk, "q4k": q4, "q8k": q8}, f,
                  indent=0)
    print(f"wrote {OUT} ({tries} sub-block draws, {draws} superblock draws)")


if __name__ == "__main__":
    main()
