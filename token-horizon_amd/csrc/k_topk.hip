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
    // level 0 stages the segment's logits here (transposed to thread order);
    // after the keys are in registers the same bytes hold the fast path's
    // candidates or the fallback's histograms
    __shared__ uint32_t stage[TK_SEG];
    uint32_t* const hist = stage;
    __shared__ int scan_lds[TK_THREADS / 64];
    __shared__ uint32_t sh_prefix;
    __shared__ int sh_kk;
    __shared__ uint32_t fkey[64], fid[64];
    __shared__ uint32_t wthr[TK_THREADS / 64];

    const int tid = threadIdx.x;
    const int64_t m = blockIdx.y;
    const int64_t seg = blockIdx.x;
    const int64_t count = FROM_LOGITS ? n : ccount;
    const int64_t base = seg * TK_SEG;

    // level 0 recomputes each element's id from its position (thread t
    // holds base + 16t .. +15) rather than holding them: 16 fewer registers
    // per thread, so every block of a 151936-wide, 40-row level fits the GPU
    // at once
    uint32_t key[TK_EPT], idv[FROM_LOGITS ? 1 : TK_EPT];
    auto id = [&](int e) { return FROM_LOGITS ? (uint32_t)(base + tid * TK_EPT + e) : idv[e]; };
    if constexpr (FROM_LOGITS) {
        // coalesced loads (position base + e*256 + tid), then thread t takes
        // positions base + 16t .. +15 out of LDS
        const float* row = logits + m * n;
        if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && base + TK_SEG <= n) {
            // a whole segment of a 16-B aligned row: 16-B loads
#pragma unroll
            for (int e = 0; e < TK_EPT / 4; ++e) {
                const int o = 4 * (e * TK_THREADS + tid);
                const float4 v = *reinterpret_cast<const float4*>(row + base + o);
                stage[o] = topk_key(v.x);
                stage[o + 1] = topk_key(v.y);
                stage[o + 2] = topk_key(v.z);
                stage[o + 3] = topk_key(v.w);
            }
        } else {
#pragma unroll
            for (int e = 0; e < TK_EPT; ++e) {
                const int64_t pos = base + e * TK_THREADS + tid;
                stage[e * TK_THREADS + tid] = pos < n ? topk_key(row[pos]) : TK_ABSENT;
            }
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) {
            key[e] = stage[tid * TK_EPT + e];
        }
    } else {
        // the segment's candidates spread over every thread (epv each, in
        // position order, so thread order stays id order)
        const uint32_t* kr = ckey + m * ccount;
        const uint32_t* ir = cid + m * ccount;
        const int64_t here = count - base < TK_SEG ? count - base : TK_SEG;
        const int epv = (int)((here + TK_THREADS - 1) / TK_THREADS);
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) {
            const int64_t pos = base + (int64_t)tid * epv + e;
            const bool ok = e < epv && pos < count;
            key[e] = ok ? kr[pos] : TK_ABSENT;
            idv[e] = ok ? ir[pos] : 0xFFFFFFFFu;
        }
    }

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
        if ((tid & 63) == 0) wthr[tid >> 6] = tw;
        __syncthreads();
        uint32_t T = wthr[0];
#pragma unroll
        for (int w = 1; w < TK_THREADS / 64; ++w) T = wthr[w] > T ? wthr[w] : T;
        if (T == TK_ABSENT) T = 1u;  // present keys only
        int c = 0;
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) c += key[e] >= T;
        int nc;
        int pos = block_scan(c, scan_lds, nc);
        if (nc <= TK_CAP) {
            uint2* cand = reinterpret_cast<uint2*>(hist);             // [TK_CAP] (key, id)
            uint2* sel = cand + TK_CAP;                               // [64] selected, by rank
            __syncthreads();  // every thread is past its reads of the staged logits
#pragma unroll
            for (int e = 0; e < TK_EPT; ++e)
                if (key[e] >= T) cand[pos++] = make_uint2(key[e], id(e));
            // pad to a multiple of 8 with entries that beat nothing
            if (tid < ((nc + 7) & ~7) - nc) cand[nc + tid] = make_uint2(0u, 0xFFFFFFFFu);
            __syncthreads();
            // rank = number of candidates ahead in (key desc, id asc); 8 per
            // LDS round trip (4 x 16-B broadcast reads)
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
                float* vr = vals + m * k;
                uint32_t* xr = idx + m * k;
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
                uint32_t* ok = okey + m * ostride + seg * k;
                uint32_t* oi = oid + m * ostride + seg * k;
                if (tid < nsel) {
                    const uint2 mine = sel[tid];
                    const uint4* s4 = reinterpret_cast<const uint4*>(sel);
                    int opos = 0, j = 0;
                    for (; j + 8 <= nsel; j += 8) {
                        const uint4 q0 = s4[j / 2], q1 = s4[j / 2 + 1], q2 = s4[j / 2 + 2], q3 = s4[j / 2 + 3];
                        opos += (q0.y < mine.y) + (q0.w < mine.y) + (q1.y < mine.y) + (q1.w < mine.y) +
                                (q2.y < mine.y) + (q2.w < mine.y) + (q3.y < mine.y) + (q3.w < mine.y);
                    }
                    for (; j < nsel; ++j) opos += sel[j].y < mine.y;
                    ok[opos] = mine.x;
                    oi[opos] = mine.y;
                }
                if (tid >= nsel && tid < k) {
                    ok[tid] = TK_ABSENT;
                    oi[tid] = 0xFFFFFFFFu;
                }
            }
            return;
        }
    }

    // ---- fallback: exact radix select over the whole segment
    int present = 0;
#pragma unroll
    for (int e = 0; e < TK_EPT; ++e) present += key[e] != TK_ABSENT;
    int P;
    (void)block_scan(present, scan_lds, P);

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
            int ex = block_scan(cnt, scan_lds, tot);
            if (ex < kk && kk <= ex + cnt) {
                for (int j = 0; j < per; ++j) {
                    const int b = nb - 1 - per * tid - j;
                    const int c = (int)hist[b];
                    if (ex + c >= kk) {
                        sh_prefix = prefix | ((uint32_t)b << shift);
                        sh_kk = kk - ex;
                        break;
                    }
                    ex += c;
                }
            }
            __syncthreads();
            prefix = sh_prefix;
            kk = sh_kk;
            pmask |= (uint32_t)(nb - 1) << shift;
        }
        tau = prefix;
        need = kk;
    }

    // select: every key above tau, and the `need` lowest ids among keys equal
    // to tau (P <= k: every present element)
    int eq = 0;
    if (P > k) {
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e) eq += key[e] == tau;
    }
    int eq_total;
    int eq_rank = block_scan(eq, scan_lds, eq_total);
    bool sel[TK_EPT];
    int nsel = 0;
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
    int total;
    int pos = block_scan(nsel, scan_lds, total);  // total == min(P, k)

    if constexpr (!FINAL) {
        uint32_t* ok = okey + m * ostride + seg * k;
        uint32_t* oi = oid + m * ostride + seg * k;
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e)
            if (sel[e]) {
                ok[pos] = key[e];
                oi[pos] = id(e);
                ++pos;
            }
        if (tid >= total && tid < k) {
            ok[tid] = TK_ABSENT;
            oi[tid] = 0xFFFFFFFFu;
        }
    } else {
#pragma unroll
        for (int e = 0; e < TK_EPT; ++e)
            if (sel[e]) {
                fkey[pos] = key[e];
                fid[pos] = id(e);
                ++pos;
            }
        __syncthreads();
        if (tid < k) {
            float* vr = vals + m * k;
            uint32_t* xr = idx + m * k;
            if (tid < total) {
                const uint32_t kt = fkey[tid], it = fid[tid];
                int rank = 0;
                for (int j = 0; j < total; ++j) rank += fkey[j] > kt || (fkey[j] == kt && fid[j] < it);
                vr[rank] = topk_value(kt);
                xr[rank] = it;
            } else {
                vr[tid] = -INFINITY;
                xr[tid] = 0xFFFFFFFFu;
            }
        }
    }
}

}  // namespace

size_t topk_workspace_bytes(int64_t m, int64_t n, int k) {
    const int64_t seg0 = (n + TK_SEG - 1) / TK_SEG;
    if (seg0 <= 1) return 0;
    // two candidate buffers of [m][seg0 * k] (key, id) pairs, 256-B aligned
    const size_t one = ((size_t)m * (size_t)seg0 * (size_t)k * 8 + 255) & ~(size_t)255;
    return 2 * one;
}

hipError_t launch_topk(const float* v, int64_t m, int64_t n, int k, float* vals, uint32_t* idx, void* ws,
                       hipStream_t s) {
    if (k < 1 || k > 64 || m < 0) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    for (int64_t r0 = 0; r0 < m; r0 += 65535) {
        const int64_t rows = m - r0 < 65535 ? m - r0 : 65535;
        float* vr = vals + r0 * k;
        uint32_t* ir = idx + r0 * k;
        if (n <= TK_SEG) {
            hipLaunchKernelGGL((k_topk_select<true, true>), dim3(1, (unsigned)rows), dim3(TK_THREADS), 0, s,
                               v + r0 * n, n, (const uint32_t*)nullptr, (const uint32_t*)nullptr, (int64_t)0, k,
                               (uint32_t*)nullptr, (uint32_t*)nullptr, (int64_t)0, vr, ir);
            continue;
        }
        const int64_t seg0 = (n + TK_SEG - 1) / TK_SEG;
        const size_t one = ((size_t)m * (size_t)seg0 * (size_t)k * 8 + 255) & ~(size_t)255;
        uint32_t* buf[2] = {static_cast<uint32_t*>(ws), reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + one)};
        // each buffer: keys [rows][cnt] then ids [rows][cnt]
        int64_t cnt = seg0 * k;
        hipLaunchKernelGGL((k_topk_select<true, false>), dim3((unsigned)seg0, (unsigned)rows), dim3(TK_THREADS), 0, s,
                           v + r0 * n, n, (const uint32_t*)nullptr, (const uint32_t*)nullptr, (int64_t)0, k, buf[0],
                           buf[0] + rows * cnt, cnt, (float*)nullptr, (uint32_t*)nullptr);
        int cur = 0;
        while (cnt > TK_SEG) {
            const int64_t segs = (cnt + TK_SEG - 1) / TK_SEG;
            const int64_t nc = segs * k;
            hipLaunchKernelGGL((k_topk_select<false, false>), dim3((unsigned)segs, (unsigned)rows), dim3(TK_THREADS),
                               0, s, (const float*)nullptr, (int64_t)0, buf[cur], buf[cur] + rows * cnt, cnt, k,
                               buf[cur ^ 1], buf[cur ^ 1] + rows * nc, nc, (float*)nullptr, (uint32_t*)nullptr);
            cur ^= 1;
            cnt = nc;
        }
        hipLaunchKernelGGL((k_topk_select<false, true>), dim3(1, (unsigned)rows), dim3(TK_THREADS), 0, s,
                           (const float*)nullptr, (int64_t)0, buf[cur], buf[cur] + rows * cnt, cnt, k,
                           (uint32_t*)nullptr, (uint32_t*)nullptr, (int64_t)0, vr, ir);
    }
    return hipGetLastError();
}

}  // namespace thq
