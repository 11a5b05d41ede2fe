"""LDS-staging bounds of every decode-GEMV plan, and the GEMM planner's
invariants, checked on the CPU through the library's own planners
(include/thq_plan.h: thq_plan_gemv_mfma / thq_plan_gemm).

k_gemv_mfma (token-horizon_amd/csrc/k_gemv_mfma.hip) stages a block's
activation rows x[0..M)[kb0 .. kb0 + Kb) in LDS with row stride Kb + 8, the
32-wide (Q4_K / MLX affine) or 16-wide (Q6_K) sums beside them, and reads its
MFMA A operands out of the staged rows.  This test restates that index
arithmetic (the staging loop, the operand reads, the sums' writes and reads)
for every plan the planner produces, and checks it against the limits the
library reports: a change to a staging constant or to the planner that would
make a kernel read or write outside its LDS arrays, leave activation chunks
unstaged, or drop an output row fails here without a GPU.
"""
import pytest

thq = pytest.importorskip("thq")

DTYPES = {"q8_0": thq.Q8_0, "q4_k": thq.Q4_K, "q6_k": thq.Q6_K, "affine": thq.MLX_Q4}
KS = sorted({256 * c for c in range(1, 65)} | {256 * c for c in (72, 80, 96, 112, 128, 160, 192, 256)})
NS = [32, 1000, 4096, 12288, 151936]


def live_rows(E: int) -> set:
    """Rows an MFMA output lane holds: 8*(e/4) + 4g + e%4 for e < E, g in {0, 1}."""
    return {8 * (e // 4) + 4 * g + e % 4 for e in range(E) for g in (0, 1)}


def gemv_violations(kind: str, M: int, K: int, p, pad: int | None = None) -> list[str]:
    """Out-of-bounds accesses of k_gemv_mfma under plan p (empty: in bounds)."""
    bad = []
    xs_cap = p.xs_elems + (p.xs_pad_elems if pad is None else pad)
    nw, cpw, splits = p.waves, p.chunks_per_wave, p.splits
    Kb = nw * cpw * 256
    XR = Kb + 8
    cpr = Kb // 8
    if splits * Kb != K:
        bad.append(f"splits*Kb={splits * Kb} != K")
    if not 1 <= nw <= p.max_waves:
        bad.append(f"waves {nw}")
    E, NX = p.live_rows, p.staged_per_thread
    if E == 0:
        return bad + ["no kernel instance"]
    # every activation chunk is staged by the straight-line loop over NX
    if M * cpr > NX * 64 * nw:
        bad.append(f"{M * cpr} chunks > NX*threads {NX * 64 * nw}")
    # staged writes xs[m*XR + 8c .. +7]
    if (M - 1) * XR + 8 * (cpr - 1) + 7 >= xs_cap:
        bad.append("staging write beyond xs")
    # A-operand reads: row min(n, M-1), half g, kl in [0, Kb-64] step 64
    q6 = kind == "q6_k"
    g_off, reach = (8, 48 + 7) if q6 else (16, 40 + 7)
    last = (M - 1) * XR + g_off + (Kb - 64) + reach
    if last >= xs_cap:
        bad.append("operand read beyond xs")
    if g_off + (Kb - 64) + reach >= Kb:
        bad.append("operand read beyond its staged row")
    # sums: rows Kb/32 (Q4) or Kb/16 (Q6), columns m (writes) and 8h+4g+3 (reads)
    rows, cols = (p.sums_rows_e8, p.sums_cols_e8) if E > 4 else (p.sums_rows_e4, p.sums_cols_e4)
    if kind in ("q4_k", "affine", "q6_k"):
        nrow = Kb // 16 if q6 else Kb // 32
        if nrow > rows:
            bad.append(f"{nrow} sum rows > {rows}")
        if M > cols or (8 * ((E > 4) + 0) + 4 + 3) >= cols:
            bad.append("sum columns")
    if q6 and E <= 4 and Kb > 4096:
        bad.append("Q6_K block K range > 4096")
    if E == 8 and (cpw != 1 or Kb > p.kb_max_e8):
        bad.append("E=8 instance needs one chunk per wave")
    if Kb > p.kb_max or M * Kb > p.xs_elems:
        bad.append("block K range")
    # every activation row has an accumulator
    if not set(range(M)) <= live_rows(E):
        bad.append(f"rows {sorted(set(range(M)) - live_rows(E))} have no accumulator at E={E}")
    return bad


@pytest.mark.parametrize("kind", list(DTYPES))
def test_gemv_mfma_plans_in_bounds(kind):
    plans = 0
    failures = []
    for M in range(1, 17):
        for K in KS:
            for N in NS:
                for gu in (False, True):
                    p = thq.plan_gemv_mfma(DTYPES[kind], M, N, K, gu)
                    if not p.waves:
                        continue
                    plans += 1
                    v = gemv_violations(kind, M, K, p)
                    if v:
                        failures.append((M, N, K, gu, v))
                    nout = N // 2 if gu else N
                    tiles = (nout + 15) // 16 if gu else (nout + 31) // 32
                    assert tiles * p.splits < 2 ** 31
                    want_ws = p.splits * M * N * 4 if p.splits > 1 else 0
                    assert p.workspace_bytes == want_ws, (M, N, K, gu)
    assert plans > 1000, plans
    assert not failures, failures[:5]


def test_the_bounds_check_has_teeth():
    """With the row padding of an eight-row staging buffer (8 * 8 elements
    instead of 8 * 16), the same check must flag plans: the sixteen-row
    instances' staged rows would overrun it."""
    flagged = 0
    for M in range(9, 17):
        for K in KS:
            p = thq.plan_gemv_mfma(thq.Q4_K, M, 12288, K, False)
            if p.waves and gemv_violations("q4_k", M, K, p, pad=8 * 8):
                flagged += 1
    assert flagged > 0


def test_gemv_plans_cover_the_decode_shapes():
    """The BASELINE decode shapes have plans at every M the router sends."""
    for dt in (thq.Q4_K, thq.Q8_0, thq.Q6_K, thq.MLX_Q4):
        for (n, k) in ((12288, 4096), (4096, 12288), (151936, 4096)):
            for M in range(2, 17):
                assert thq.plan_gemv_mfma(dt, M, n, k).waves > 0, (dt, n, k, M)


@pytest.mark.parametrize("kind", list(DTYPES))
def test_gemm_plans(kind):
    """Every K step belongs to exactly one split (no empty split), the tile
    grid covers M and N, and the partials workspace is splits x M x N f32."""
    for exact in ((False, True) if kind == "q8_0" else (False,)):
        for M in (17, 32, 64, 65, 128, 300, 512, 1024, 2048, 4096):
            for K in (256, 1024, 4096, 12288):
                for N in (256, 4096, 12288, 151936):
                    for gu in (False, True):
                        for cus in (256, 304, 80):
                            p = thq.plan_gemm(DTYPES[kind], M, N, K, exact, gu, cus)
                            steps = K // 64
                            assert p.bm in (64, 128, 256)
                            if exact:
                                assert p.bm == 64
                            assert p.splits >= 1 and p.k_steps >= 1
                            assert p.splits * p.k_steps >= steps > (p.splits - 1) * p.k_steps, (M, N, K, p.splits)
                            assert p.tiles_m * p.bm >= M > (p.tiles_m - 1) * p.bm
                            nout = N // 2 if gu else N
                            bn = 64 if gu else 128
                            assert p.tiles_n == (nout + bn - 1) // bn
                            want = p.splits * M * N * 4 if p.splits > 1 else 0
                            assert p.workspace_bytes == want


def test_planner_rejects_bad_arguments():
    o = thq.GemvPlanInfo()
    assert thq.lib.thq_plan_gemv_mfma(3, 1, 1, 256, 0, o) == thq.EDTYPE
    assert thq.lib.thq_plan_gemv_mfma(thq.Q4_K, 0, 1, 256, 0, o) == thq.ESHAPE
    assert thq.lib.thq_plan_gemv_mfma(thq.Q4_K, 1, 1, 256, 0, None) == thq.EINVAL
    g = thq.GemmPlanInfo()
    assert thq.lib.thq_plan_gemm(thq.Q4_K, 0, 1, 1, 0, 0, 256, g) == thq.ESHAPE
    # unsupported shapes plan nothing
    assert thq.plan_gemv_mfma(thq.Q4_K, 17, 4096, 4096).waves == 0
    assert thq.plan_gemv_mfma(thq.Q4_K, 1, 4096, 4000).waves == 0


def test_wide_plans():
    """The wide GEMV's plan covers K exactly with non-empty splits, and its
    workspace is the split partials; unsupported shapes plan nothing."""
    for dt in (thq.Q8_0, thq.Q4_K, thq.Q6_K, thq.MLX_Q4):
        for m in (1, 17, 40, 64):
            for n in (300, 4096, 12288, 151936):
                for k in (256, 1024, 4096, 12288):
                    p = thq.plan_gemv_wide(dt, m, n, k)
                    nch = k // 256
                    assert p.splits >= 1 and p.chunks_per_split >= 1
                    assert p.splits * p.chunks_per_split >= nch > (p.splits - 1) * p.chunks_per_split
                    assert p.workspace_bytes == (p.splits * m * n * 4 if p.splits > 1 else 0)
        assert thq.plan_gemv_wide(dt, 65, 4096, 4096).splits == 0
        assert thq.plan_gemv_wide(dt, 8, 4096, 1000).splits == 0
    assert thq.plan_gemv_wide(thq.Q4_K, 40, 151936, 4096).splits == 1


def test_mid_plans():
    """The streaming mid-M GEMM's plan: an instance the launcher has (groups of
    64 or 128 rows; 1 or 2 column tiles per wave; 4 or 8 waves, 8 with one
    column tile), groups that cover M, splits that cover K exactly and are
    non-empty, and a workspace of the split partials; shapes it cannot
    address with 32-bit offsets, K not a multiple of 256 and odd gate/up
    weights plan nothing; the measured picks of the two MLP shapes."""
    for dt in (thq.Q4_K, thq.MLX_Q4):
        for gu in (False, True):
            for m in (1, 17, 33, 64, 65, 100, 128, 129, 300, 512, 2048):
                for n in (256, 600, 4096, 12288, 24576):
                    for k in (256, 1024, 4096, 12288):
                        p = thq.plan_gemm_mid(dt, m, n, k, gu)
                        nch = k // 256
                        assert p.group_halves in (2, 4), (dt, gu, m, n, k)
                        assert (p.col_tiles, p.waves) in ((1, 4), (2, 4), (1, 8))
                        assert p.groups == -(-m // (32 * p.group_halves))
                        assert p.splits >= 1 and p.chunks_per_split >= 1
                        assert p.splits * p.chunks_per_split >= nch > (p.splits - 1) * p.chunks_per_split
                        assert p.workspace_bytes == (p.splits * m * n * 4 if p.splits > 1 else 0)
        assert thq.plan_gemm_mid(dt, 64, 4096, 1000).group_halves == 0
        assert thq.plan_gemm_mid(dt, 64, 301, 1024, gate_up=True).group_halves == 0
        assert thq.plan_gemm_mid(dt, 64, 1 << 20, 1 << 14).group_halves == 0  # 9.7 GB plane
        assert thq.plan_gemm_mid(dt, 1 << 18, 4096, 8192).group_halves == 0   # 4 GiB of x
    p = thq.plan_gemm_mid(thq.Q4_K, 128, 12288, 4096)
    assert (p.group_halves, p.col_tiles, p.waves, p.splits) == (4, 1, 8, 4)
    p = thq.plan_gemm_mid(thq.Q4_K, 64, 12288, 4096)
    assert (p.group_halves, p.col_tiles, p.waves, p.splits) == (2, 1, 8, 4)
    o = thq.MidPlanInfo()
    assert thq.lib.thq_plan_gemm_mid(thq.Q8_0, 64, 4096, 4096, 0, 256, o) == thq.EDTYPE
    assert thq.lib.thq_plan_gemm_mid(thq.Q4_K, 0, 4096, 4096, 0, 256, o) == thq.ESHAPE
    assert thq.lib.thq_plan_gemm_mid(thq.Q4_K, 64, 4096, 4096, 0, 256, None) == thq.EINVAL


def tile_lds_bytes(kw: int, m: int, nt: int) -> int:
    """k_gemv_q4t's LDS (token-horizon_amd/csrc/k_gemv_tile.hip, tile_lds_bytes):
    x rows of the block's K range with an 8-column pad, the 32-wide sums of 8
    rows, and the waves' partials for the cross-wave sum."""
    kr = kw * 2 * 256
    return m * (kr + 8) * 2 + kw * 2 * 8 * 8 * 4 + max(kw - 1, 1) * nt * 4 * 64 * 4


def test_tile_plans():
    """The tile-plane GEMV's plans (thq_plan_gemv_tile) for 1..8 rows, plain
    and gate/up: waves per block in {1, 2, 4, 8}; the K splits cover every
    superblock once with no empty split; the block's LDS fits the CU's
    160 KB; the workspace is the split partials.  Unsupported shapes plan
    nothing."""
    for gu in (False, True):
        for m in range(1, 9):
            for n in (64, 1000 if not gu else 2048, 4096, 12288, 24576, 151936):
                for k in (256, 512, 1024, 2304, 4096, 8192, 12288, 16384):
                    p = thq.plan_gemv_tile(thq.Q4_K, m, n, k, gate_up=gu)
                    assert p.waves in (1, 2, 4, 8), (gu, m, n, k, p.waves)
                    nsb = (k + 255) // 256
                    per = p.waves * 2
                    assert p.splits * per >= nsb > (p.splits - 1) * per, (gu, m, n, k, p.waves, p.splits)
                    nt = 2 if gu else 1
                    assert tile_lds_bytes(p.waves, m, nt) <= 160 * 1024, (gu, m, k, p.waves)
                    assert p.workspace_bytes == (p.splits * m * n * 4 if p.splits > 1 else 0), (gu, m, n, k)
    assert thq.plan_gemv_tile(thq.Q4_K, 9, 4096, 4096).waves == 0
    assert thq.plan_gemv_tile(thq.Q4_K, 4, 4000, 4096, gate_up=True).waves == 0
    with pytest.raises(thq.ThqError):
        thq.plan_gemv_tile(thq.Q8_0, 4, 4096, 4096)
