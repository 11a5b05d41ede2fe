// k_topk.hip — exact per-row top-k of verify logits for sampled
// speculative-decode acceptance.
//
// Role: the candidate step of the reference's sampled verify consumer
// (ts_topk, engine/src/sample_kernel.rs:1-16, 725-796; CPU form
// sorted_row_dist :326-347 and key :163-169, consumed at
// engine/src/engine.rs:2436-2442): the top k (k <= 64) logits of each row by
// (logit desc, id asc), where a NaN ranks as -inf and -0.0 as +0.0.  The
// reference's kernel pools the elements at or above the k-th largest lane
// maximum (at most 1024 of them, flagging overflow); this one is exact for
// any row.
//
// Order-preserving keys.  A logit maps to a u32 whose unsigned order is the
// rank order (sign bit flipped for positives, all bits for negatives); key 0
// is below every real key and marks an absent element.  The composite
// order (key desc, id asc) has no ties, so the top-k set is exact.
//
// Two levels.  Each block takes a segment of 4096 elements of one row
// (16 per thread, thread t holding ids base + 16t .. +15, so thread order is
// id order) and selects its top k.
// Fast path: each lane keeps its 4 largest keys, and each wave finds, bit by
// bit with ballots (no LDS, no barrier), the largest t such that at least k
// of its lanes' kept keys are >= t; the block threshold T is the largest of
// the four.  Some wave then holds k keys >= T, so the segment's whole top k
// is among the keys >= T (usually about k to 2k of them).  Those are
// compacted and ranked exactly by counting (key desc, id asc).
// Fallback (more than 256 keys >= T, e.g. long runs of equal logits): a
// 3-pass radix select (12, 10, 10 bits, LDS histograms) finds the k-th
// largest key tau and how many of the elements equal to tau are needed;
// those are the ones with the lowest ids, found by a block prefix count in
// id order.
// Either way a segment's selected elements leave in id order, so the next
// level, which runs the same select over the per-segment candidates until
// one segment remains, can use the fallback too; the last level writes its
// k in rank order.
// HBM-bound: one pass over the logits (4 B per logit) and a few KB of
// candidates per row.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"

namespace thq {

namespace {

constexpr int TK_THREADS = 256;
constexpr int TK_EPT = 16;
constexpr int TK_SEG = TK_THREADS * TK_EPT;
constexpr uint32_t TK_ABSENT = 0u;
constexpr int TK_CAP = 256;  // candidates the fast path ranks
// the one-launch form's arrival counters sit 128 B apart (row m: cnt[32 m]):
// device-scope atomics on one line serialize (40 rows of 38 blocks on
// adjacent counters: 7.6 us more), and launches take at most TK_ROWS1 rows
constexpr int TK_CNT_STRIDE = 32;
constexpr int TK_ROWS1 = 2048;
// The one-launch form takes 16 logits per thread (4096-logit segments) up
// to this many blocks per launch, else 32 (8192-logit segments: half the
// blocks, pool stores and merge input; 151936-wide rows, k = 32: 5 rows
// 9.0 against 10.0 us, 40 rows 13.3 against 11.0 us)
#ifndef TK_RE16_BLOCKS
#define TK_RE16_BLOCKS 1024
#endif
// pool entries per segment in the one-launch form: room for the filter's
// candidates as they are (about k + 8 for smooth logits), 16-aligned, and
// for the exact fallback's k per 4096-logit part
__host__ __device__ constexpr int tk_pslot(int k, int re) {
    return ((k + 31) & ~15) > re / TK_EPT * k ? ((k + 31) & ~15) : re / TK_EPT * k;
}

__device__ __forceinline__ uint32_t topk_key(float v) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) b = 0xff800000u;  // NaN ranks as -inf
    if (b == 0x80000000u) b = 0u;                          // -0.0 ranks as +0.0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float topk_value(uint32_t k) {
    if (k == TK_ABSENT) return -INFINITY;
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// exclusive prefix of one int per thread over the block (256 threads), and the total
__device__ __forceinline__ int block_scan(int v, int* lds, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) lds[wave] = x;
    __syncthreads();
    int base = 0;
#pragma unroll
    for (int w = 0; w < TK_THREADS / 64; ++w) base += w < wave ? lds[w] : 0;
    total = lds[0] + lds[1] + lds[2] + lds[3];
    __syncthreads();  // lds is reused by the next scan
    return base + x - v;
}

// One block's LDS.
struct TkLds {
    uint32_t buf[TK_SEG];  // staged logits, then candidates (key, id) or radix histograms
    int scan[TK_THREADS / 64];
    uint32_t prefix;
    int kk;
    uint32_t fkey[64], fid[64];
    uint32_t wthr[TK_THREADS / 64];
    uint32_t thr;
    int last;
};

// Ranks the nc <= TK_CAP candidates (key, id) in cand (LDS, TK_CAP + 64
// entries) by (key desc, id asc) and emits the first k.  FINAL: vr / xr [k]
// in rank order, unused slots -inf / 0xFFFFFFFF.  Else: ok / oi [k] in id
// order, padded with absent entries, as device-scope stores (a block of the
// same launch may read them).  Every thread of the block calls it.
template <bool FINAL>
__device__ __forceinline__ void tk_emit(uint2* cand, int nc, int k, float* vr, uint32_t* xr, uint32_t* ok, uint32_t* oi) {
    const int tid = threadIdx.x;
    uint2* sel = cand + TK_CAP;  // [64] selected, by rank
    // pad to a multiple of 8 with entries that beat nothing
    if (tid < ((nc + 7) & ~7) - nc) cand[nc + tid] = make_uint2(0u, 0xFFFFFFFFu);
    __syncthreads();
    // rank = number of candidates ahead in (key desc, id asc); 8 per LDS
    // round trip (4 x 16-B broadcast reads)
    auto ahead = [](uint2 a, uint2 me) { return (int)(a.x > me.x || (a.x == me.x && a.y < me.y)); };
    int rank = k;  // k: not selected
    uint2 me = make_uint2(0u, 0u);
    if (tid < nc) {
        me = cand[tid];
        const uint4* c4 = reinterpret_cast<const uint4*>(cand);
        int r0 = 0, r1 = 0;
        auto batch = [&](int j) {
            const uint4 q0 = c4[j / 2], q1 = c4[j / 2 + 1], q2 = c4[j / 2 + 2], q3 = c4[j / 2 + 3];
            r0 += ahead(make_uint2(q0.x, q0.y), me) + ahead(make_uint2(q0.z, q0.w), me) +
                  ahead(make_uint2(q1.x, q1.y), me) + ahead(make_uint2(q1.z, q1.w), me);
            r1 += ahead(make_uint2(q2.x, q2.y), me) + ahead(make_uint2(q2.z, q2.w), me) +
                  ahead(make_uint2(q3.x, q3.y), me) + ahead(make_uint2(q3.z, q3.w), me);
        };
        int j = 0;
        for (; j + 16 <= nc; j += 16) {  // two batches' reads in flight together
            batch(j);
            batch(j + 8);
        }
        for (; j < nc; j += 8) batch(j);  // the rest (up to 15, in batches of 8)
        rank = r0 + r1;
    }
    const int nsel = nc < k ? nc : k;
    if constexpr (FINAL) {
        if (rank < k) {
            vr[rank] = topk_value(me.x);
            xr[rank] = me.y;
        }
        if (tid >= nsel && tid < k) {
            vr[tid] = -INFINITY;
            xr[tid] = 0xFFFFFFFFu;
        }
    } else {
        // id-order position among the selected: count smaller ids among them
        if (rank < k) sel[rank] = me;
        __syncthreads();
        if (tid < nsel) {
            const uint2 mine = sel[tid];
            const uint4* s4 = reinterpret_cast<const uint4*>(sel);
            int opos = 0, j = 0;
            for (; j + 8 <= nsel; j += 8) {
                const uint4 q0 = s4[j / 2], q1 = s4[j / 2 + 1], q2 = s4[j / 2 + 2], q3 = s4[j / 2 + 3];
                opos += (q0.y < mine.y) + (q0.w < mine.y) + (q1.y < mine.y) + (q1.w < mine.y) + (q2.y < mine.y) +
                        (q2.w < mine.y) + (q3.y < mine.y) + (q3.w < mine.y);
            }
            for (; j < nsel; ++j) opos += sel[j].y < mine.y;
            __hip_atomic_store(ok + opos, mine.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(oi + opos, mine.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid >= nsel && tid < k) {
            __hip_atomic_store(ok + tid, TK_ABSENT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(oi + tid, 0xFFFFFFFFu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// The top k of one segment held as key[TK_EPT] per thread (element e of
// thread t: id(e)); emits as tk_emit.  ORDERED: thread order = id order.
// Else (FINAL only) the ids may sit in any order, and the fallback takes
// the lowest ids among the keys equal to the k-th largest by a radix select
// over the ids.  Every thread of the block calls it; L.buf may hold staged
// logits that the threads have already read into key.
template <bool FINAL, bool ORDERED = true, typename IdF>
__device__ __forceinline__ void tk_select(const uint32_t (&key)[TK_EPT], IdF id, int k, TkLds& L, float* vr, uint32_t* xr,
                          uint32_t* ok, uint32_t* oi) {
    static_assert(ORDERED || FINAL, "unordered candidates only for the final selection");
    const int tid = threadIdx.x;
    // ---- fast path: threshold from the waves' lane maxima
    {
        uint32_t v0 = 0u, v1 = 0u, v2 = 0u, v3 = 0u;  // the lane's 4 largest keys, v0 >= v1 >= v2 >= v3
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) {
            uint32_t x = key[e], t;
            t = x > v0 ? x : v0; x = x > v0 ? v0 : x; v0 = t;
            t = x > v1 ? x : v1; x = x > v1 ? v1 : x; v1 = t;
            t = x > v2 ? x : v2; x = x > v2 ? v2 : x; v2 = t;
            v3 = x > v3 ? x : v3;
        }
        // largest t (to 2^-20 of the key range: a smaller T only admits more
        // candidates) with >= k kept keys of this wave at or above it
        uint32_t tw = 0u;
        for (int b = 31; b >= 12; --b) {
            const uint32_t c = tw | (1u << b);
            const int cnt = __popcll(__ballot(v0 >= c)) + __popcll(__ballot(v1 >= c)) +
                            __popcll(__ballot(v2 >= c)) + __popcll(__ballot(v3 >= c));
            if (cnt >= k) tw = c;
        }
        if ((tid & 63) == 0) L.wthr[tid >> 6] = tw;
        __syncthreads();
        uint32_t T = L.wthr[0];
#pragma unroll
        for (int w = 1; w < TK_THREADS / 64; ++w) T = L.wthr[w] > T ? L.wthr[w] : T;
        if (T == TK_ABSENT) T = 1u;  // present keys only
        int c = 0;
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) c += key[e] >= T;
        int nc;
        int pos = block_scan(c, L.scan, nc);
        if (nc <= TK_CAP) {
            uint2* cand = reinterpret_cast<uint2*>(L.buf);
            __syncthreads();  // every thread is past its reads of the staged logits
#pragma unroll
            for (int e = 0; e < TK_EPT; ++e)
                if (key[e] >= T) cand[pos++] = make_uint2(key[e], id(e));
            tk_emit<FINAL>(cand, nc, k, vr, xr, ok, oi);
            return;
        }
    }

    // ---- fallback: exact radix select over the whole segment
    uint32_t* const hist = L.buf;
    int present = 0;
#pragma unroll
    for (int e = 0; e < TK_EPT; ++e) present += key[e] != TK_ABSENT;
    int P;
    (void)block_scan(present, L.scan, P);

    // radix select: tau = the k-th largest present key, need = how many of
    // the keys equal to tau belong to the top k
    uint32_t tau = 0u;
    int need = 0;
    if (P > k) {
        uint32_t prefix = 0u, pmask = 0u;
        int kk = k;
#pragma unroll
        for (int pass = 0; pass < 3; ++pass) {
            const int width = pass == 0 ? 12 : 10;
            const int shift = pass == 0 ? 20 : (pass == 1 ? 10 : 0);
            const int nb = 1 << width, per = nb / TK_THREADS;  // bins per thread: 16 or 4
            for (int i = tid; i < nb; i += TK_THREADS) hist[i] = 0u;
            __syncthreads();
#pragma unroll
            for (int e = 0; e < TK_EPT; ++e)
                if (key[e] != TK_ABSENT && (key[e] & pmask) == prefix)
                    atomicAdd(&hist[(key[e] >> shift) & (uint32_t)(nb - 1)], 1u);
            __syncthreads();
            // thread t owns bins nb-1-per*t .. nb-per*(t+1) (from the top); the
            // thread whose range holds the kk-th largest key finds its bin
            int cnt = 0;
            for (int j = 0; j < per; ++j) cnt += (int)hist[nb - 1 - per * tid - j];
            int tot;
            int ex = block_scan(cnt, L.scan, tot);
            if (ex < kk && kk <= ex + cnt) {
                for (int j = 0; j < per; ++j) {
                    const int b = nb - 1 - per * tid - j;
                    const int c = (int)hist[b];
                    if (ex + c >= kk) {
                        L.prefix = prefix | ((uint32_t)b << shift);
                        L.kk = kk - ex;
                        break;
                    }
                    ex += c;
                }
            }
            __syncthreads();
            prefix = L.prefix;
            kk = L.kk;
            pmask |= (uint32_t)(nb - 1) << shift;
        }
        tau = prefix;
        need = kk;
    }

    // select: every key above tau, and the `need` lowest ids among keys equal
    // to tau (P <= k: every present element)
    bool sel[TK_EPT];
    int nsel = 0;
    if constexpr (ORDERED) {
        int eq = 0;
        if (P > k) {
#pragma unroll
            for (int e = 0; e < TK_EPT; ++e) eq += key[e] == tau;
        }
        int eq_total;
        int eq_rank = block_scan(eq, L.scan, eq_total);
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) {
            if (P > k) {
                const bool is_eq = key[e] == tau;
                sel[e] = key[e] > tau || (is_eq && eq_rank < need);
                eq_rank += is_eq;
            } else {
                sel[e] = key[e] != TK_ABSENT;
            }
            nsel += sel[e];
        }
    } else {
        // id_cut = the need-th smallest id among the keys equal to tau (ids
        // are distinct): a radix select from the bottom, 12 + 10 + 10 bits
        uint32_t id_cut = 0u;
        if (P > k) {
            uint32_t prefix = 0u, pmask = 0u;
            int kk = need;
#pragma unroll
            for (int pass = 0; pass < 3; ++pass) {
                const int width = pass == 0 ? 12 : 10;
                const int shift = pass == 0 ? 20 : (pass == 1 ? 10 : 0);
                const int nb = 1 << width, per = nb / TK_THREADS;
                for (int i = tid; i < nb; i += TK_THREADS) hist[i] = 0u;
                __syncthreads();
#pragma unroll
                for (int e = 0; e < TK_EPT; ++e)
                    if (key[e] == tau && (id(e) & pmask) == prefix)
                        atomicAdd(&hist[(id(e) >> shift) & (uint32_t)(nb - 1)], 1u);
                __syncthreads();
                // thread t owns bins per*t .. per*(t+1)-1 (from the bottom)
                int cnt = 0;
                for (int j = 0; j < per; ++j) cnt += (int)hist[per * tid + j];
                int tot;
                int ex = block_scan(cnt, L.scan, tot);
                if (ex < kk && kk <= ex + cnt) {
                    for (int j = 0; j < per; ++j) {
                        const int b = per * tid + j;
                        const int c = (int)hist[b];
                        if (ex + c >= kk) {
                            L.prefix = prefix | ((uint32_t)b << shift);
                            L.kk = kk - ex;
                            break;
                        }
                        ex += c;
                    }
                }
                __syncthreads();
                prefix = L.prefix;
                kk = L.kk;
                pmask |= (uint32_t)(nb - 1) << shift;
            }
            id_cut = prefix;
        }
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) {
            sel[e] = P > k ? key[e] > tau || (key[e] == tau && id(e) <= id_cut) : key[e] != TK_ABSENT;
            nsel += sel[e];
        }
    }
    int total;
    int pos = block_scan(nsel, L.scan, total);  // total == min(P, k)

    if constexpr (!FINAL) {
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e)
            if (sel[e]) {
                __hip_atomic_store(ok + pos, key[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(oi + pos, id(e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ++pos;
            }
        if (tid >= total && tid < k) {
            __hip_atomic_store(ok + tid, TK_ABSENT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(oi + tid, 0xFFFFFFFFu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e)
            if (sel[e]) {
                L.fkey[pos] = key[e];
                L.fid[pos] = id(e);
                ++pos;
            }
        __syncthreads();
        if (tid < k) {
            if (tid < total) {
                const uint32_t kt = L.fkey[tid], it = L.fid[tid];
                int rank = 0;
                for (int j = 0; j < total; ++j) rank += L.fkey[j] > kt || (L.fkey[j] == kt && L.fid[j] < it);
                vr[rank] = topk_value(kt);
                xr[rank] = it;
            } else {
                vr[tid] = -INFINITY;
                xr[tid] = 0xFFFFFFFFu;
            }
        }
    }
}

// The candidates of row m (count of them, in id order) spread over the
// block's threads, epv each in position order, so thread order stays id
// order.  Device-scope loads: other blocks of the same launch may have
// written them.
__device__ __forceinline__ void tk_load_candidates(const uint32_t* kr, const uint32_t* ir, int64_t base,
                                                   int64_t count, uint32_t (&key)[TK_EPT], uint32_t (&idv)[TK_EPT]) {
    const int tid = threadIdx.x;
    const int64_t here = count - base < TK_SEG ? count - base : TK_SEG;
    const int epv = (int)((here + TK_THREADS - 1) / TK_THREADS);
#pragma unroll
    for (int e = 0; e < TK_EPT; ++e) {
        const int64_t pos = base + (int64_t)tid * epv + e;
        const bool ok = e < epv && pos < count;
        key[e] = ok ? __hip_atomic_load(kr + pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : TK_ABSENT;
        idv[e] = ok ? __hip_atomic_load(ir + pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0xFFFFFFFFu;
    }
}

// Grid: (segments, rows).  Level 0 reads logits rows [m][n] (ids = column);
// later levels read candidate rows ckey / cid [m][ccount] (kept in id order).
// Non-final: the segment's k selected (key, id) go to okey / oid at
// m * ostride + seg * k, in id order, padded with absent entries.  FINAL (a
// single segment): vals / idx [m][k] in rank order, unused slots -inf /
// 0xFFFFFFFF.
template <bool FROM_LOGITS, bool FINAL>
__global__ __launch_bounds__(TK_THREADS) void k_topk_select(const float* __restrict__ logits, int64_t n,
                                                           const uint32_t* __restrict__ ckey,
                                                           const uint32_t* __restrict__ cid, int64_t ccount, int k,
                                                           uint32_t* __restrict__ okey, uint32_t* __restrict__ oid,
                                                           int64_t ostride, float* __restrict__ vals,
                                                           uint32_t* __restrict__ idx) {
    __shared__ TkLds L;
    const int tid = threadIdx.x;
    const int64_t m = blockIdx.y;
    const int64_t seg = blockIdx.x;
    const int64_t base = seg * TK_SEG;
    float* const vr = FINAL ? vals + m * k : nullptr;
    uint32_t* const xr = FINAL ? idx + m * k : nullptr;
    uint32_t* const ok = FINAL ? nullptr : okey + m * ostride + seg * k;
    uint32_t* const oi = FINAL ? nullptr : oid + m * ostride + seg * k;

    uint32_t key[TK_EPT];
    if constexpr (FROM_LOGITS) {
        // level 0 recomputes each element's id from its position (thread t
        // holds base + 16t .. +15) rather than holding them: 16 fewer
        // registers per thread.  Coalesced loads (position base + e*256 +
        // tid), then thread t takes positions base + 16t .. +15 out of LDS.
        const float* row = logits + m * n;
        if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && base + TK_SEG <= n) {
            // a whole segment of a 16-B aligned row: 16-B loads
#pragma unroll
            for (int e = 0; e < TK_EPT / 4; ++e) {
                const int o = 4 * (e * TK_THREADS + tid);
                const float4 v = *reinterpret_cast<const float4*>(row + base + o);
                L.buf[o] = topk_key(v.x);
                L.buf[o + 1] = topk_key(v.y);
                L.buf[o + 2] = topk_key(v.z);
                L.buf[o + 3] = topk_key(v.w);
            }
        } else {
#pragma unroll
            for (int e = 0; e < TK_EPT; ++e) {
                const int64_t pos = base + e * TK_THREADS + tid;
                L.buf[e * TK_THREADS + tid] = pos < n ? topk_key(row[pos]) : TK_ABSENT;
            }
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) key[e] = L.buf[tid * TK_EPT + e];
        tk_select<FINAL>(key, [&](int e) { return (uint32_t)(base + tid * TK_EPT + e); }, k, L, vr, xr, ok, oi);
    } else {
        uint32_t idv[TK_EPT];
        tk_load_candidates(ckey + m * ccount, cid + m * ccount, base, ccount, key, idv);
        tk_select<FINAL>(key, [&](int e) { return idv[e]; }, k, L, vr, xr, ok, oi);
    }
}

// The block's 256 lane maxima (keys, one per thread) -> a threshold t with
// at least k of them >= t, found by one wave with ballots over 16 key bits:
// the k-th largest lane maximum rounded down, or (QUAD) the k-th largest of
// the 64 maxima of lane quads (lanes l, l + 64, l + 128, l + 192), one ballot
// a step instead of four, a lower t that lets a few more candidates pass.
// QUAD in the merge and for 8192-logit segments (151936-wide rows, k = 32:
// 5 / 20 / 27 / 40 / 64 rows 8.9 / 9.4 / 9.9 / 10.8 / 16.1 against 9.0 / 9.8
// / 10.7 / 11.3 / 17.3 us); not for 4096-logit segments, whose 48-entry
// slots it overflows (10.2 against 9.0 us at 5 rows).  L.buf[0..255] holds
// the lane keys on return; every thread of the block calls it.
template <bool QUAD = false>
__device__ __forceinline__ uint32_t tk_lane_threshold(uint32_t lane_key, int k, TkLds& L) {
    const int tid = threadIdx.x;
    L.buf[tid] = lane_key;
    __syncthreads();
    if (tid < 64) {
        const uint32_t a0 = L.buf[tid], a1 = L.buf[tid + 64], a2 = L.buf[tid + 128], a3 = L.buf[tid + 192];
        uint32_t t = 0u;
        if constexpr (QUAD) {
            uint32_t q = a0 > a1 ? a0 : a1;
            const uint32_t r = a2 > a3 ? a2 : a3;
            q = q > r ? q : r;
            for (int b = 31; b >= 16; --b) {
                const uint32_t c = t | (1u << b);
                if (__popcll(__ballot(q >= c)) >= k) t = c;
            }
        } else {
            for (int b = 31; b >= 16; --b) {
                const uint32_t c = t | (1u << b);
                const int nge = __popcll(__ballot(a0 >= c)) + __popcll(__ballot(a1 >= c)) +
                                __popcll(__ballot(a2 >= c)) + __popcll(__ballot(a3 >= c));
                if (nge >= k) t = c;
            }
        }
        if (tid == 0) L.thr = t;
    }
    __syncthreads();
    return L.thr;
}

// The exact top k of a row's pool (count <= TK_SEG entries (key, id) in any
// order, absent entries key 0) into vr / xr [k], rank order.  Level 0's
// filter on keys: T from the lane maxima (tk_lane_threshold, over lane
// quads), the candidates are the keys >= T; real keys are at least the -inf
// key (0x007fffff), so T > 0 means at least k real entries pass.
// Otherwise, or past TK_CAP candidates, tk_select (order-free ties).
__device__ __forceinline__ void tk_merge(const uint32_t* kr, const uint32_t* ir, int64_t count, int k, TkLds& L,
                                         float* vr, uint32_t* xr) {
    const int tid = threadIdx.x;
    // entry tid + 256 e: every load covers 1 KB contiguous (the order is free)
    uint32_t key[TK_EPT], idv[TK_EPT];
#pragma unroll
    for (int e = 0; e < TK_EPT; ++e) {
        const int64_t pos = (int64_t)e * TK_THREADS + tid;
        const bool ok = pos < count;
        key[e] = ok ? __hip_atomic_load(kr + pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : TK_ABSENT;
        idv[e] = ok ? __hip_atomic_load(ir + pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0xFFFFFFFFu;
    }
    uint32_t lm = key[0];
#pragma unroll
    for (int e = 1; e < TK_EPT; ++e) lm = key[e] > lm ? key[e] : lm;
    const uint32_t t = tk_lane_threshold<true>(lm, k, L);
    int c = 0;
#pragma unroll
    for (int e = 0; e < TK_EPT; ++e) c += key[e] >= t;
    int nc;
    int pos = block_scan(c, L.scan, nc);  // its barriers order wave 0's reads of the lane keys first
    if (t != 0u && nc <= TK_CAP) {
        uint2* cand = reinterpret_cast<uint2*>(L.buf);
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e)
            if (key[e] >= t) cand[pos++] = make_uint2(key[e], idv[e]);
        tk_emit<true>(cand, nc, k, vr, xr, nullptr, nullptr);
    } else {
        tk_select<true, false>(key, [&](int e) { return idv[e]; }, k, L, vr, xr, nullptr, nullptr);
    }
}

// Rows whose segments' candidates fit one block (segments * pslot <= TK_SEG)
// in one launch.  Grid (segments >= 2, rows); a segment is 256 * RE logits
// (RE elements per thread).  Each block writes a set of at most pslot
// elements that holds its segment's top k into its slot of the pool (okey /
// oid [m][segments * pslot], any order, absent entries after them;
// device-scope stores) and draws a ticket on the row's arrival counter
// cnt[TK_CNT_STRIDE m] (zero before the launch); the block that draws the
// last ticket selects the row's top k from the pool (tk_merge) into vals /
// idx and zeroes the counter.
//
// A segment's selection first tries a filter: thread t holds the elements
// at offsets 1024 j + 4t + c (j < RE / 4, c < 4: 16-B loads, no staging),
// the block's threshold T (tk_lane_threshold) has at least k lane maxima at
// or above it, and the candidates are the elements >= T in float order: at
// least k elements pass and the segment's top k are among them.  Up to pslot
// of them go to the pool as they are; up to TK_CAP are ranked exactly and
// the top k go.  Where no such T exists (fewer than k lanes hold a value above -inf)
// or more than TK_CAP elements pass (long runs of equal logits), each
// 4096-logit part of the segment takes tk_select over its keys in id order
// (its own fast path, else the radix select), into slot entries [h k, h k +
// k) (pslot >= RE / 16 * k).  The selection helpers are inlined (called,
// their register arrays went to the stack).  MINB blocks per CU: RE = 16 at
// 4 (94 VGPRs, five blocks per CU: its 1024 blocks in one round); RE = 32 at
// 3 (135 VGPRs, no scratch) up to 768 blocks, at 4 (128 VGPRs, 20 B of
// spills) past them (64 rows of 19 segments: 15.4 against 16.3 us; 40 rows:
// 11.2 against 10.9).
template <int RE, int MINB>
__global__ __launch_bounds__(TK_THREADS, MINB) void k_topk_rows(const float* __restrict__ logits,
                                                                          int64_t n, int k, int pslot,
                                                                          uint32_t* __restrict__ pkey,
                                                                          uint32_t* __restrict__ pid,
                                                                          uint32_t* __restrict__ cnt,
                                                                          float* __restrict__ vals,
                                                                          uint32_t* __restrict__ idx) {
    static_assert(RE % 16 == 0 && RE <= 32, "RE: 16 or 32");
    constexpr int SEG = TK_THREADS * RE;
    __shared__ TkLds L;
    const int tid = threadIdx.x;
    const int64_t m = blockIdx.y, seg = blockIdx.x, segs = gridDim.x;
    const int64_t base = seg * SEG;
    const int64_t pstride = segs * pslot;
    const float* row = logits + m * n;
    uint32_t* const ok = pkey + m * pstride + seg * pslot;
    uint32_t* const oi = pid + m * pstride + seg * pslot;
    auto at = [&](int e) { return base + (e >> 2) * 4 * TK_THREADS + 4 * tid + (e & 3); };

    float xv[RE];  // element 4j + c: offset 1024 j + 4 tid + c
    if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && base + SEG <= n) {
#pragma unroll
        for (int j = 0; j < RE / 4; ++j) {
            const float4 v = *reinterpret_cast<const float4*>(row + base + j * 4 * TK_THREADS + 4 * tid);
            xv[4 * j] = v.x;
            xv[4 * j + 1] = v.y;
            xv[4 * j + 2] = v.z;
            xv[4 * j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < RE; ++e) {
            const int64_t pos = at(e);
            xv[e] = pos < n ? row[pos] : __builtin_nanf("");  // NaN: never passes the filter
        }
    }
    // lane maximum: v_max_f32 returns the non-NaN operand, and a NaN result
    // maps to the -inf key, so the key is at most the lane's largest key
    float lm = xv[0];
#pragma unroll
    for (int e = 1; e < RE; ++e) asm("v_max_f32 %0, %0, %1" : "+v"(lm) : "v"(xv[e]));
    const uint32_t t = tk_lane_threshold<RE == 32>(topk_key(lm), k, L);
    // above the -inf key (0x007fffff), t (low 16 bits clear) is the key of a
    // real float tf, and for a non-NaN x, key(x) >= t exactly when x >= tf
    const bool valid = t > 0x007fffffu;
    const float tf = valid ? topk_value(t) : INFINITY;
    int c = 0;
#pragma unroll
    for (int e = 0; e < RE; ++e) c += xv[e] >= tf;
    int nc;
    int pos = block_scan(c, L.scan, nc);  // its barriers order wave 0's reads of the lane keys first
    int filled = k;                       // pool entries written below (the rest: absent)
    if (valid && nc <= TK_CAP) {
        uint2* cand = reinterpret_cast<uint2*>(L.buf);
#pragma unroll
        for (int e = 0; e < RE; ++e)
            if (xv[e] >= tf) cand[pos++] = make_uint2(topk_key(xv[e]), (uint32_t)at(e));
        if (nc <= pslot) {
            // as they are: the slot in coalesced stores, absent after them
            __syncthreads();
            if (tid < pslot) {
                const uint2 cv = tid < nc ? cand[tid] : make_uint2(TK_ABSENT, 0xFFFFFFFFu);
                __hip_atomic_store(ok + tid, cv.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(oi + tid, cv.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            filled = pslot;
        } else {
            tk_emit<false>(cand, nc, k, nullptr, nullptr, ok, oi);
        }
    } else {
#pragma unroll 1
        for (int h = 0; h < RE / TK_EPT; ++h) {
            const int64_t hb = base + (int64_t)h * TK_SEG;
            uint32_t key[TK_EPT];
#pragma unroll
            for (int e = 0; e < TK_EPT; ++e) {
                const int64_t p = hb + tid * TK_EPT + e;
                key[e] = p < n ? topk_key(row[p]) : TK_ABSENT;
            }
            if (h > 0) __syncthreads();  // the previous part is done with L
            tk_select<false>(key, [&](int e) { return (uint32_t)(hb + tid * TK_EPT + e); }, k, L, nullptr, nullptr,
                             ok + h * k, oi + h * k);
        }
        filled = RE / TK_EPT * k;
    }
    if (tid >= filled && tid < pslot) {
        __hip_atomic_store(ok + tid, TK_ABSENT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(oi + tid, 0xFFFFFFFFu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // The last block of the row to arrive merges the pool: every pool access
    // is an agent-scope (sc1) store or load, published before the ticket
    // (ticket_publish, thq_dev.hpp)
    ticket_publish();
    __syncthreads();
    if (tid == 0) L.last = ticket_draw(cnt + TK_CNT_STRIDE * m) == (uint32_t)(segs - 1);
    __syncthreads();
    if (!L.last) return;
    tk_merge(pkey + m * pstride, pid + m * pstride, pstride, k, L, vals + m * k, idx + m * k);
    if (tid == 0) __hip_atomic_store(cnt + TK_CNT_STRIDE * m, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

size_t topk_workspace_bytes(int64_t m, int64_t n, int k) {
    const int64_t seg0 = (n + TK_SEG - 1) / TK_SEG;
    if (seg0 <= 1) return 0;
    // two candidate buffers of [m][seg0 * k] (key, id) pairs, 256-B aligned;
    // the one-launch form's pool [m][seg0 * TK_PSLOT] in their place
    const size_t one = ((size_t)m * (size_t)seg0 * (size_t)k * 8 + 255) & ~(size_t)255;
    // the one-launch form's pool [m][segments * pslot], the larger of its two shapes
    const int64_t s32 = (n + 2 * TK_SEG - 1) / (2 * TK_SEG);
    const int64_t e16 = seg0 * tk_pslot(k, 16) <= TK_SEG ? seg0 * tk_pslot(k, 16) : 0;
    const int64_t e32 = s32 * tk_pslot(k, 32) <= TK_SEG ? s32 * tk_pslot(k, 32) : 0;
    const size_t pool = (size_t)m * (size_t)(e16 > e32 ? e16 : e32) * 8;
    return 2 * one > pool ? 2 * one : pool;
}

int64_t topk_counters(int64_t m) { return (m < TK_ROWS1 ? m : TK_ROWS1) * TK_CNT_STRIDE; }

hipError_t launch_topk(const float* v, int64_t m, int64_t n, int k, float* vals, uint32_t* idx, void* ws,
                       uint32_t* cnt, int64_t ncnt, hipStream_t s) {
    if (k < 1 || k > 64 || m < 0) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    const int64_t seg0 = (n + TK_SEG - 1) / TK_SEG;
    // the one-launch form: counters for a launch of TK_ROWS1 rows (or all of them)
    const int64_t rows1 = m < TK_ROWS1 ? m : TK_ROWS1;
    const int64_t s32 = (n + 2 * TK_SEG - 1) / (2 * TK_SEG);
    const bool fit16 = seg0 * tk_pslot(k, 16) <= TK_SEG, fit32 = s32 * tk_pslot(k, 32) <= TK_SEG;
    const bool one = n > TK_SEG && (fit16 || fit32) && cnt && ncnt >= rows1 * TK_CNT_STRIDE;
    const int64_t chunk = one ? TK_ROWS1 : 65535;
    for (int64_t r0 = 0; r0 < m; r0 += chunk) {
        const int64_t rows = m - r0 < chunk ? m - r0 : chunk;
        float* vr = vals + r0 * k;
        uint32_t* ir = idx + r0 * k;
        if (n <= TK_SEG) {
            hipLaunchKernelGGL((k_topk_select<true, true>), dim3(1, (unsigned)rows), dim3(TK_THREADS), 0, s,
                               v + r0 * n, n, (const uint32_t*)nullptr, (const uint32_t*)nullptr, (int64_t)0, k,
                               (uint32_t*)nullptr, (uint32_t*)nullptr, (int64_t)0, vr, ir);
            continue;
        }
        const size_t half = ((size_t)m * (size_t)seg0 * (size_t)k * 8 + 255) & ~(size_t)255;
        uint32_t* buf[2] = {static_cast<uint32_t*>(ws), reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + half)};
        if (one) {
            // one launch: the pool [rows][segments * pslot] keys then ids at ws
            uint32_t* pool = static_cast<uint32_t*>(ws);
            if (fit16 && (!fit32 || rows * seg0 <= TK_RE16_BLOCKS)) {
                const int pslot = tk_pslot(k, 16);
                hipLaunchKernelGGL((k_topk_rows<16, 4>), dim3((unsigned)seg0, (unsigned)rows), dim3(TK_THREADS), 0, s,
                                   v + r0 * n, n, k, pslot, pool, pool + rows * seg0 * pslot, cnt, vr, ir);
            } else {
                const int pslot = tk_pslot(k, 32);
                if (rows * s32 <= 768)
                    hipLaunchKernelGGL((k_topk_rows<32, 3>), dim3((unsigned)s32, (unsigned)rows), dim3(TK_THREADS), 0,
                                       s, v + r0 * n, n, k, pslot, pool, pool + rows * s32 * pslot, cnt, vr, ir);
                else
                    hipLaunchKernelGGL((k_topk_rows<32, 4>), dim3((unsigned)s32, (unsigned)rows), dim3(TK_THREADS), 0,
                                       s, v + r0 * n, n, k, pslot, pool, pool + rows * s32 * pslot, cnt, vr, ir);
            }
            continue;
        }
        // each buffer: keys [rows][count] then ids [rows][count]
        int64_t count = seg0 * k;
        hipLaunchKernelGGL((k_topk_select<true, false>), dim3((unsigned)seg0, (unsigned)rows), dim3(TK_THREADS), 0, s,
                           v + r0 * n, n, (const uint32_t*)nullptr, (const uint32_t*)nullptr, (int64_t)0, k, buf[0],
                           buf[0] + rows * count, count, (float*)nullptr, (uint32_t*)nullptr);
        int cur = 0;
        while (count > TK_SEG) {
            const int64_t segs = (count + TK_SEG - 1) / TK_SEG;
            const int64_t nc = segs * k;
            hipLaunchKernelGGL((k_topk_select<false, false>), dim3((unsigned)segs, (unsigned)rows), dim3(TK_THREADS),
                               0, s, (const float*)nullptr, (int64_t)0, buf[cur], buf[cur] + rows * count, count, k,
                               buf[cur ^ 1], buf[cur ^ 1] + rows * nc, nc, (float*)nullptr, (uint32_t*)nullptr);
            cur ^= 1;
            count = nc;
        }
        hipLaunchKernelGGL((k_topk_select<false, true>), dim3(1, (unsigned)rows), dim3(TK_THREADS), 0, s,
                           (const float*)nullptr, (int64_t)0, buf[cur], buf[cur] + rows * count, count, k,
                           (uint32_t*)nullptr, (uint32_t*)nullptr, (int64_t)0, vr, ir);
    }
    return hipGetLastError();
}

}  // namespace thq
