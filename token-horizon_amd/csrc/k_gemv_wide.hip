// k_gemv_wide.hip — exact-weight GEMV for up to 64 bf16 activation rows:
// the batched speculative-verify LM head (151936 outputs, 5 drafted tokens x
// 8 sequences = 40 rows) and other wide, skinny products.
//
// Role: the verify step's LM head over Q8_0 / Q4_K / Q6_K / MLX affine
// weights with exact (unrounded) dequantized weights (engine/src/engine.rs:
// 2338-2470 batched verify, LM head engine/src/qwen35.rs:5202-5212; the
// reference runs it through its AffineQmpp / prefill tiles,
// engine/src/quant_kernel.rs:3188-3738, 4841-5095).  HBM-bound: every weight
// byte is read once with 16-B loads; the activations are re-read from L2.
//
// Why not the decode GEMV: that kernel stages all of a block's activation
// range for only 32 weight rows, which past 16 rows no longer fits LDS, and
// the prefill GEMM keeps only one 64-wide K step of weights in flight per
// block.  Here a block of four waves owns 128 weight rows (32 per wave) and
// walks K in 256-wide chunks: the chunk's activation rows x[0..M)[256] are
// staged in LDS (double-buffered, one barrier per chunk), while each wave
// holds the next chunk of its own weights in registers, loaded straight
// from HBM as MFMA B operands.
//
// Products on v_mfma_f32_32x32x16_bf16: A = x rows (two 32-row halves for
// M > 32), B = 16 weights of 32 rows; output lane (n = l % 32, g = l / 32)
// holds weight row n and activation rows 32*half + 8*(e/4) + 4*g + e%4.
// Exactness as in the decode GEMV (k_gemv_mfma.hip):
//   Q8_0    B = bf16(q); each 32-wide block's MFMA pair starts from zero and
//           is scaled by its f16 d into the f32 accumulator
//   Q4_K    B = bf16(128 + q); per 32-wide sub-block
//           sum = d1 * A - (128 * d1 + m1) * S,  S = sum of x over it
//   affine  same with d1 = scale, m1 = -bias (w = scale * q + bias)
//   Q6_K    B = bf16(128 + code); per 16-wide group a second MFMA against a
//           constant B of bf16(-160) folds in -160 * (sum of x over the group),
//           so the group's sum is s * A with A = sum x * (code - 32)
// The 32-wide sums S (Q4_K, affine) are taken while a chunk is staged.
// Gate/up (GU): a wave's 32 rows are 16 gate rows and the 16 up rows of the
// same outputs (a block owns 64 outputs); lanes n and n + 16 exchange their
// sums for the silu(gate) * up epilogue (engine/src/quant_kernel.rs:2922-2926).
// Split-K (grid.y > 1, for outputs too few to fill the GPU): f32 partials
// [split][M][N] in weight-row order, summed in split order by k_split_reduce.
#include "thq_dev.hpp"
#include "thq_kernels.hpp"
#include "thq_wave.hpp"

#include <type_traits>

namespace thq {

namespace {

constexpr int WV_WAVES = 4;                // waves per block
constexpr int WV_ROWS = 32 * WV_WAVES;     // weight rows per block
constexpr int WV_KC = 256;                 // K chunk
constexpr int WV_XR = WV_KC + 8;           // LDS row stride (bf16): rows start 16 B apart in bank order
constexpr int WV_DQ = 16;                  // Q6_K chunks whose d a block stages in LDS

__device__ __forceinline__ f32x16_t wmfma(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// low nibbles (masked to 4 bits) of the bytes of a, b -> bf16(128 + q) x 8
__device__ __forceinline__ bf16x8_t wnib(uint32_t a, uint32_t b) {
    const uint32_t C = 0x43434343u;
    return as_bf16x8(make_uint4(__builtin_amdgcn_perm(C, a, 0x04010400u), __builtin_amdgcn_perm(C, a, 0x04030402u),
                                __builtin_amdgcn_perm(C, b, 0x04010400u), __builtin_amdgcn_perm(C, b, 0x04030402u)));
}
// int8 bytes of a, b -> bf16(q) x 8 (exact)
__device__ __forceinline__ bf16x8_t wi8(uint32_t a, uint32_t b) {
    auto cv = [](uint32_t w, int i) { return (float)(int8_t)(w >> (8 * i)); };
    return as_bf16x8(make_uint4(pack_bf16x2(cv(a, 0), cv(a, 1)), pack_bf16x2(cv(a, 2), cv(a, 3)),
                                pack_bf16x2(cv(b, 0), cv(b, 1)), pack_bf16x2(cv(b, 2), cv(b, 3))));
}
template <int CTRL>
__device__ __forceinline__ float wdpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// One 256-wide chunk of a lane's weight row: packed weights, scale words,
// Q6_K high bits and d.
template <int QT>
struct WChunk {
    uint4 w[QT == 8 ? 8 : 4];
    uint32_t s[4];
    uint2 h[QT == 14 ? 4 : 1];
    uint32_t d;
};
// An empty asm that reads and redefines every register of a chunk (and is
// ordered with memory operations): the compiler waits for the chunk's loads
// before it, and later uses depend on it rather than on the loads.
template <int QT>
__device__ __forceinline__ void wv_settle(WChunk<QT>& C) {
#pragma unroll
    for (int i = 0; i < (QT == 8 ? 8 : 4); ++i)
        asm volatile("" : "+v"(C.w[i].x), "+v"(C.w[i].y), "+v"(C.w[i].z), "+v"(C.w[i].w)::"memory");
    asm volatile("" : "+v"(C.s[0]), "+v"(C.s[1]), "+v"(C.s[2]), "+v"(C.s[3])::"memory");
    if constexpr (QT == 14) {
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(C.h[i].x), "+v"(C.h[i].y)::"memory");
        asm volatile("" : "+v"(C.d)::"memory");
    }
}

// Grid (tiles of 128 weight rows, splits); block (t, s) owns rows
// [128t, 128t + 128) (GU: outputs [64t, 64t + 64)) over chunks
// [s*cps, min((s+1)*cps, K/256)).
// X is not __restrict__: its loads stay ordered before the weight loads by
// the compiler barriers.
template <int QT, int MR, typename YT, bool GU, bool SPLIT, bool AM>
__global__ __launch_bounds__(256, 2) void k_gemv_wide(const uint8_t* __restrict__ Wq, const uint8_t* __restrict__ Wa,
                                                     const bf16_t* X, void* __restrict__ Yv, int M, int K,
                                                     int64_t nout, int64_t up_off, int64_t nrows, int cps,
                                                     float* __restrict__ amv, uint32_t* __restrict__ ami,
                                                     int64_t am_ld) {
    // MR 8-row groups of activation rows (M <= 8 MR) in MH halves of 32
    constexpr int MH = (MR + 3) / 4;
    constexpr int MP = 8 * MR;                  // staged rows (M <= MP)
    constexpr int NXP = MR;                     // 16-B activation pieces per thread per chunk
    constexpr int NS = WV_KC / 32;  // 32-wide sums per staged row (Q4_K, affine)
    __shared__ __attribute__((aligned(16))) bf16_t xs[2][MP][WV_XR];
    __shared__ __attribute__((aligned(16))) float Ss[QT == 8 || QT == 14 ? 1 : 2][NS][32 * MH];
    // Q6_K: the block's rows' f16 d for its chunks (at most WV_DQ), staged once:
    // read a chunk at a time from HBM, the d plane's lines (4 rows x 16
    // chunks) left L2 between chunks and were fetched again and again
    __shared__ uint16_t Dq[QT == 14 ? WV_ROWS * WV_DQ : 1];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int64_t tile = blockIdx.x;
    const int nch = K >> 8;
    const int cb = blockIdx.y * cps;
    const int ce = cb + cps < nch ? cb + cps : nch;
    const bool dlds = QT == 14 && ce - cb <= WV_DQ;  // Q6_K d from LDS (staged below)

    static_assert(!(GU && AM), "no argmax over gate/up");
    // GU: output o, weight row o (gate, n < 16) or up_off + o (up)
    const int64_t orow = GU ? tile * (WV_ROWS / 2) + wave * 16 + (n & 15) : tile * WV_ROWS + wave * 32 + n;
    const bool valid = orow < nout;
    int64_t row = GU && n >= 16 ? orow + up_off : orow;
    if (!valid) row = 0;  // in-bounds reads; the scales are zeroed below

    // Every load is a chunk-uniform base (a plane's start plus the chunk's
    // offset, in scalar registers) plus the lane's 32-bit offset: each plane
    // and the activations are below 4 GiB (plan_gemv_wide), so the loads take
    // the scalar-base form and a chunk's addresses cost no vector ALU.
    const uint8_t* bw = Wq;
    const uint8_t* bs = Wq;
    const uint8_t* bh = Wq;
    const uint8_t* bd = Wq;
    uint32_t ow, os, oh = 0, od = 0;
    if constexpr (QT == 14) {
        const Q6Layout L = q6k_layout(nrows, K);
        bh = Wq + L.qh;
        bs = Wq + L.sc;
        bd = Wq + L.d;
        ow = (uint32_t)(row * (K >> 1) + 8 * g);
        oh = (uint32_t)(row * (K >> 2) + 8 * g);
        os = (uint32_t)(row * (K >> 4));
        od = (uint32_t)(row * (K >> 8) * 2);
    } else if constexpr (QT == 8) {
        // Q8_0 tiles: block b of the row at 1024 b, chunk c's 8 scales at 512 c
        bs = Wa;
        ow = (uint32_t)q8t_q(row, K >> 5, 0, g);
        os = (uint32_t)(q8t_d(row, K >> 5, 0) * 2);
    } else {
        const int nsb = K >> 8;
        ow = (uint32_t)q4k_piece(row, nsb, 0, g, 0);
        os = (uint32_t)q4k_hdword(row, nsb, 0, 0);
    }
    // Q6_K: a row's QH bytes of chunks 2j, 2j + 1 share a 128-B line, and its
    // scale bytes of 8 chunks another; one chunk at a time, the second half
    // came from HBM again once the first had left L2.  So an even chunk of
    // the block's range (odd = false) also loads the next chunk's QH and
    // scales into Hod / Sod, and the odd chunk takes them from there.
    uint2 Hod[QT == 14 ? 4 : 1];
    uint4 Sod;
    auto wload = [&](WChunk<QT>& C, int c, bool odd) {
        if constexpr (QT == 14) {
            const int c1 = c + 1 < ce ? c + 1 : c;
            if (!odd) {
                const uint4 sv = *reinterpret_cast<const uint4*>(bs + (int64_t)c * 16 + os);
                C.s[0] = sv.x; C.s[1] = sv.y; C.s[2] = sv.z; C.s[3] = sv.w;
                Sod = *reinterpret_cast<const uint4*>(bs + (int64_t)c1 * 16 + os);
            } else {
                C.s[0] = Sod.x; C.s[1] = Sod.y; C.s[2] = Sod.z; C.s[3] = Sod.w;
            }
            C.d = dlds ? (uint32_t)Dq[(wave * 32 + n) * WV_DQ + (c - cb)]
                       : (uint32_t)*reinterpret_cast<const uint16_t*>(bd + (int64_t)c * 2 + od);
            const uint8_t* qlc = bw + (int64_t)c * 128;
            const uint8_t* qhc = bh + (int64_t)c * 64;
            const uint8_t* qhn = bh + (int64_t)c1 * 64;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint2 lo = *reinterpret_cast<const uint2*>(qlc + ow + u * 32);
                const uint2 hi = *reinterpret_cast<const uint2*>(qlc + ow + u * 32 + 16);
                C.w[u] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                if (!odd) {
                    C.h[u] = *reinterpret_cast<const uint2*>(qhc + oh + u * 16);
                    Hod[u] = *reinterpret_cast<const uint2*>(qhn + oh + u * 16);
                } else {
                    C.h[u] = Hod[u];
                }
            }
        } else if constexpr (QT == 8) {
            const uint4 sv = *reinterpret_cast<const uint4*>(bs + (int64_t)c * 512 + os);
            C.s[0] = sv.x; C.s[1] = sv.y; C.s[2] = sv.z; C.s[3] = sv.w;
            const uint8_t* wc0 = bw + (int64_t)c * 8192;
            const uint8_t* wc1 = wc0 + 4096;
#pragma unroll
            for (int b = 0; b < 8; ++b)
                C.w[b] = *reinterpret_cast<const uint4*>((b < 4 ? wc0 : wc1) + ow + (b & 3) * 1024);
        } else {
            const uint8_t* wc = bw + (int64_t)c * 64;
            const uint8_t* sc = bs + (int64_t)c * 64;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                C.w[u] = *reinterpret_cast<const uint4*>(wc + ow + u * 16);
                C.s[u] = *reinterpret_cast<const uint32_t*>(sc + os + u * 16);
            }
        }
    };

    // activation pieces of chunk c: thread t takes pieces p = t + 256j, row
    // p / 32, columns 8 * (p % 32) ..; a thread's piece j is 8 rows below its
    // piece j - 1 (j < MR: 8 MR >= M rows); rows past M load row M - 1 (in
    // bounds) and are not written.
    const uint32_t K2 = (uint32_t)K * 2u;
    const uint32_t xo0 = (uint32_t)(threadIdx.x >> 5) * K2 + 16u * (threadIdx.x & 31);
    const uint32_t xomax = (uint32_t)(M - 1) * K2 + 16u * (threadIdx.x & 31);
    auto xload = [&](uint4 (&xv)[NXP], int c) {
        const uint8_t* xc = reinterpret_cast<const uint8_t*>(X) + (int64_t)c * (WV_KC * 2);
#pragma unroll
        for (int j = 0; j < NXP; ++j) {
            const uint32_t o = xo0 + (uint32_t)j * 8u * K2;
            xv[j] = *reinterpret_cast<const uint4*>(xc + (o < xomax ? o : xomax));
        }
    };
    auto xstore = [&](const uint4 (&xv)[NXP], int buf) {
#pragma unroll
        for (int j = 0; j < NXP; ++j) {
            const int p = threadIdx.x + 256 * j;
            const int m = p >> 5, i = p & 31;
            if (m < M) {
                const uint4 v = xv[j];
                *reinterpret_cast<uint4*>(&xs[buf][m][8 * i]) = v;
                if constexpr (QT == 12 || QT == 13) {
                    // a 32-wide sub-block is 4 consecutive pieces (lanes 4j..4j+3,
                    // a whole lane quad, all of one row m)
                    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
                    bf16x2_t q[4];
                    __builtin_memcpy(q, &v, 16);
                    float t = __builtin_amdgcn_fdot2_f32_bf16(q[0], one, 0.0f, false);
                    t = __builtin_amdgcn_fdot2_f32_bf16(q[1], one, t, false);
                    t = __builtin_amdgcn_fdot2_f32_bf16(q[2], one, t, false);
                    t = __builtin_amdgcn_fdot2_f32_bf16(q[3], one, t, false);
                    t = wdpp_add<0xB1>(t);  // quad_perm [1,0,3,2]
                    t = wdpp_add<0x4E>(t);  // quad_perm [2,3,0,1]
                    if ((i & 3) == 0) Ss[buf][i >> 2][m] = t;
                }
            }
        }
    };

    f32x16_t acc[MH];
#pragma unroll
    for (int h = 0; h < MH; ++h) acc[h] = f32x16_t{};
    const f32x16_t z16 = {};
    // A-operand row of each half (clamped to M - 1: rows past M are computed and dropped)
    int arow[MH];
#pragma unroll
    for (int h = 0; h < MH; ++h) arow[h] = 32 * h + n < M ? 32 * h + n : M - 1;
    constexpr int GOFF = QT == 14 ? 8 : 16;

    auto pin = [&]() {
#pragma unroll
        for (int h = 0; h < MH; ++h) asm volatile("" : "+v"(acc[h]));
        __builtin_amdgcn_sched_barrier(0);
    };
    // the lane's 16 accumulator rows of half h in the sums array: m = 32h + 8q + 4g + i
    auto sums = [&](int buf, int col, int h, f32x4_t (&S)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) S[q] = *reinterpret_cast<const f32x4_t*>(&Ss[QT == 8 ? 0 : buf][col][32 * h + 8 * q + 4 * g]);
    };

    // accumulator e of half h holds activation rows 32h + 8(e / 4) + 4g + e % 4:
    // the groups of four e past the MR live 8-row groups are never scaled
    auto live = [](int h, int e) { return 32 * h + 8 * (e >> 2) < 8 * MR; };

    auto compute = [&](const WChunk<QT>& C, int buf) {
        if constexpr (QT == 8) {
            // software-pipelined by one block: block b's MFMAs (every half)
            // are issued, block b + 1 is converted while they run, then b's
            // products are scaled into the accumulators
            bf16x8_t B0 = wi8(C.w[0].x, C.w[0].y), B1 = wi8(C.w[0].z, C.w[0].w);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const uint32_t sw = C.s[b >> 1] >> (16 * (b & 1));
                const float d = valid ? f16_to_f32((uint16_t)sw) : 0.0f;
                f32x16_t T[MH];
#pragma unroll
                for (int h = 0; h < MH; ++h) {
                    const bf16_t* xa = &xs[buf][arow[h]][GOFF * g + 32 * b];
                    const uint4 a0 = *reinterpret_cast<const uint4*>(xa);
                    const uint4 a1 = *reinterpret_cast<const uint4*>(xa + 8);
                    T[h] = wmfma(as_bf16x8(a0), B0, z16);
                    T[h] = wmfma(as_bf16x8(a1), B1, T[h]);
                }
                if (b < 7) {
                    B0 = wi8(C.w[b + 1].x, C.w[b + 1].y);
                    B1 = wi8(C.w[b + 1].z, C.w[b + 1].w);
                }
#pragma unroll
                for (int h = 0; h < MH; ++h)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (live(h, e)) acc[h][e] = __builtin_fmaf(d, T[h][e], acc[h][e]);
                pin();
            }
        } else if constexpr (QT == 14) {
            const float dd = valid ? f16_to_f32((uint16_t)C.d) : 0.0f;
            const uint32_t M4 = 0x0F0F0F0Fu;
            // bf16(-160) in every element: the second MFMA adds -160 * sum(x)
            const uint32_t m160 = 0xC320C320u;
            const bf16x8_t B160 = as_bf16x8(make_uint4(m160, m160, m160, m160));
            // the 6-bit codes of unit u's four 16-wide groups (bytes of lo / hi)
            uint32_t lo[4], hi[4];
            auto unpack = [&](int u) {
                const uint4 q = C.w[u];
                const uint2 hb = C.h[u];
                lo[0] = (q.x & M4) | ((hb.x & 0x03030303u) << 4);
                hi[0] = (q.y & M4) | ((hb.y & 0x03030303u) << 4);
                lo[1] = (q.z & M4) | ((hb.x & 0x0C0C0C0Cu) << 2);
                hi[1] = (q.w & M4) | ((hb.y & 0x0C0C0C0Cu) << 2);
                lo[2] = ((q.x >> 4) & M4) | (hb.x & 0x30303030u);
                hi[2] = ((q.y >> 4) & M4) | (hb.y & 0x30303030u);
                lo[3] = ((q.z >> 4) & M4) | ((hb.x >> 2) & 0x30303030u);
                hi[3] = ((q.w >> 4) & M4) | ((hb.y >> 2) & 0x30303030u);
            };
            // software-pipelined by one group: group t's MFMAs are issued,
            // group t + 1 is converted while they run, then t is scaled
            unpack(0);
            bf16x8_t B = wnib(lo[0], hi[0]);
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int u = t >> 2, G = t & 3;
                const float sg = dd * (float)(int)(int8_t)(C.s[u] >> (8 * G));
                f32x16_t T[MH];
#pragma unroll
                for (int h = 0; h < MH; ++h) {
                    const bf16x8_t a = as_bf16x8(*reinterpret_cast<const uint4*>(&xs[buf][arow[h]][GOFF * g + 64 * u + 16 * G]));
                    T[h] = wmfma(a, B, z16);
                    T[h] = wmfma(a, B160, T[h]);
                }
                if (t < 15) {
                    if (G == 3) unpack(u + 1);
                    B = wnib(lo[(t + 1) & 3], hi[(t + 1) & 3]);
                }
#pragma unroll
                for (int h = 0; h < MH; ++h)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (live(h, e)) acc[h][e] = __builtin_fmaf(sg, T[h][e], acc[h][e]);
                pin();
            }
        } else {
            float d = 0.0f, dm = 0.0f;
            if constexpr (QT == 12) {
                d = f16_to_f32((uint16_t)__builtin_amdgcn_perm(C.s[1], C.s[0], 0x0c0c0703u));
                dm = f16_to_f32((uint16_t)__builtin_amdgcn_perm(C.s[3], C.s[2], 0x0c0c0703u));
                if (!valid) d = dm = 0.0f;
            }
            const uint32_t M4 = 0x0F0F0F0Fu;
            // software-pipelined by one unit: unit u's MFMAs (both sub-blocks,
            // every half) are issued, unit u + 1 is converted while they run,
            // then u's products are scaled
            bf16x8_t B0, B1, B2, B3;
            auto conv = [&](int u) {
                const uint4 q = C.w[u];
                B0 = wnib(q.x & M4, q.y & M4);
                B1 = wnib(q.z & M4, q.w & M4);
                B2 = wnib((q.x >> 4) & M4, (q.y >> 4) & M4);
                B3 = wnib((q.z >> 4) & M4, (q.w >> 4) & M4);
            };
            // (64 activation rows: no register room for that; unit u is
            // converted when it starts, and each half is scaled before the next)
            constexpr bool PIPE = MR <= 5;
            if constexpr (PIPE) conv(0);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if constexpr (!PIPE) conv(u);
                const uint32_t hw = C.s[u];
                float d1, d2, c1, c2;
                if constexpr (QT == 13) {
                    const float sc = valid ? aff_scale(hw) : 0.0f, bi = valid ? aff_bias(hw) : 0.0f;
                    d1 = d2 = sc;
                    c1 = c2 = __builtin_fmaf(128.0f, sc, -bi);
                } else {
                    d1 = d * (float)(hw & 63u);
                    d2 = d * (float)((hw >> 12) & 63u);
                    c1 = __builtin_fmaf(128.0f, d1, dm * (float)((hw >> 6) & 63u));
                    c2 = __builtin_fmaf(128.0f, d2, dm * (float)((hw >> 18) & 63u));
                }
                if constexpr (PIPE) {
                    f32x16_t T1[MH], T2[MH];
#pragma unroll
                    for (int h = 0; h < MH; ++h) {
                        const bf16_t* xa = &xs[buf][arow[h]][GOFF * g + 64 * u];
                        const uint4 a0 = *reinterpret_cast<const uint4*>(xa);
                        const uint4 a1 = *reinterpret_cast<const uint4*>(xa + 8);
                        const uint4 a2 = *reinterpret_cast<const uint4*>(xa + 32);
                        const uint4 a3 = *reinterpret_cast<const uint4*>(xa + 40);
                        T1[h] = wmfma(as_bf16x8(a0), B0, z16);
                        T1[h] = wmfma(as_bf16x8(a1), B1, T1[h]);
                        T2[h] = wmfma(as_bf16x8(a2), B2, z16);
                        T2[h] = wmfma(as_bf16x8(a3), B3, T2[h]);
                    }
                    if (u < 3) conv(u + 1);
#pragma unroll
                    for (int h = 0; h < MH; ++h) {
                        f32x4_t S1[4], S2[4];
                        sums(buf, 2 * u, h, S1);
                        sums(buf, 2 * u + 1, h, S2);
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            if (live(h, e))
                                acc[h][e] = __builtin_fmaf(-c1, S1[e >> 2][e & 3], __builtin_fmaf(d1, T1[h][e], acc[h][e]));
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            if (live(h, e))
                                acc[h][e] = __builtin_fmaf(-c2, S2[e >> 2][e & 3], __builtin_fmaf(d2, T2[h][e], acc[h][e]));
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < MH; ++h) {
                        const bf16_t* xa = &xs[buf][arow[h]][GOFF * g + 64 * u];
                        const uint4 a0 = *reinterpret_cast<const uint4*>(xa);
                        const uint4 a1 = *reinterpret_cast<const uint4*>(xa + 8);
                        const uint4 a2 = *reinterpret_cast<const uint4*>(xa + 32);
                        const uint4 a3 = *reinterpret_cast<const uint4*>(xa + 40);
                        f32x4_t S1[4], S2[4];
                        sums(buf, 2 * u, h, S1);
                        sums(buf, 2 * u + 1, h, S2);
                        f32x16_t T = wmfma(as_bf16x8(a0), B0, z16);
                        T = wmfma(as_bf16x8(a1), B1, T);
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            if (live(h, e))
                                acc[h][e] = __builtin_fmaf(-c1, S1[e >> 2][e & 3], __builtin_fmaf(d1, T[e], acc[h][e]));
                        T = wmfma(as_bf16x8(a2), B2, z16);
                        T = wmfma(as_bf16x8(a3), B3, T);
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            if (live(h, e))
                                acc[h][e] = __builtin_fmaf(-c2, S2[e >> 2][e & 3], __builtin_fmaf(d2, T[e], acc[h][e]));
                    }
                }
                pin();
            }
        }
    };

    // Q6_K d staging: lanes g = 0 / 1 of a row take alternate chunks
    if constexpr (QT == 14) {
        if (dlds) {
            for (int c = cb + g; c < ce; c += 2)
                Dq[(wave * 32 + n) * WV_DQ + (c - cb)] = *reinterpret_cast<const uint16_t*>(bd + (int64_t)c * 2 + od);
            __syncthreads();
        }
    }

    // ---- prologue: chunk cb staged in buffer 0, its weights in W0
    WChunk<QT> W0, W1;
    uint4 xv[NXP];
    xload(xv, cb);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    wload(W0, cb, false);
    xstore(xv, 0);
    __syncthreads();

    // ---- one step: prefetch chunk c + 1 (activations to registers, weights
    // to Wn), compute chunk c, then stage c + 1 in the other buffer.  Wc
    // passes through wv_settle first: its loads (issued a step ago) are
    // waited for there, before the prefetch is issued, and the math then
    // reads the settled registers, so the compiler's wait counts never make
    // the math wait for the prefetch.  (Without it the counts lose track of
    // Wc across the loop's back edge, and each step drained its own prefetch
    // block by block.)
    auto step = [&](int c, WChunk<QT>& Wc, WChunk<QT>& Wn, int buf) {
        const bool more = c + 1 < ce;
        wv_settle(Wc);
        if constexpr (QT == 14) {
            // the next chunk's QH / scales, loaded with Wc (buf 0: the next is odd)
#pragma unroll
            for (int u = 0; u < 4; ++u) asm volatile("" : "+v"(Hod[u].x), "+v"(Hod[u].y)::"memory");
            asm volatile("" : "+v"(Sod.x), "+v"(Sod.y), "+v"(Sod.z), "+v"(Sod.w)::"memory");
        }
        const bool odd_next = buf == 0;  // steps alternate even / odd chunks of the range
        // unconditional (the last step reloads its own chunk, unused): no
        // merge of loaded and old register values for the allocator to copy
        const int cn = more ? c + 1 : c;
        xload(xv, cn);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        wload(Wn, cn, odd_next);
        __builtin_amdgcn_sched_barrier(0);
        compute(Wc, buf);
        if (more) xstore(xv, buf ^ 1);
        __syncthreads();
    };
    for (int c = cb; c < ce; c += 2) {
        step(c, W0, W1, 0);
        if (c + 1 >= ce) break;
        step(c + 1, W1, W0, 1);
    }

    // ---- epilogue
    if constexpr (GU && !SPLIT) {
        // lane n < 16 holds gate, lane n + 16 the up sum of the same output
#pragma unroll
        for (int h = 0; h < MH; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float up = __shfl_xor(acc[h][e], 16, 64);
                const int m = 32 * h + 8 * (e >> 2) + 4 * g + (e & 3);
                if (valid && n < 16 && m < M)
                    store_y<YT>(static_cast<YT*>(Yv) + (int64_t)m * nout + orow, silu_mul(acc[h][e], up));
            }
    } else if constexpr (AM) {
        // per activation row: (max, lowest index) over the wave's 32 rows
        const int64_t wt = tile * WV_WAVES + wave;  // 32-row tile index
        const bool wt_ok = wt * 32 < nout;
#pragma unroll
        for (int h = 0; h < MH; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = 32 * h + 8 * (e >> 2) + 4 * g + (e & 3);
                float v = (valid && m < M) ? amax_key(acc[h][e]) : -INFINITY;
                uint32_t i = (uint32_t)orow;
                amax_row32(v, i);
                if (wt_ok && n == 0 && m < M) {
                    amv[m * am_ld + wt] = v;
                    ami[m * am_ld + wt] = i;
                }
            }
    } else {
#pragma unroll
        for (int h = 0; h < MH; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = 32 * h + 8 * (e >> 2) + 4 * g + (e & 3);
                if (!valid || m >= M) continue;
                if constexpr (SPLIT)
                    static_cast<float*>(Yv)[((int64_t)blockIdx.y * M + m) * nrows + row] = acc[h][e];
                else
                    store_y<YT>(static_cast<YT*>(Yv) + (int64_t)m * nout + orow, acc[h][e]);
            }
    }
}

template <int QT, int MR, bool GU>
hipError_t run_wide(const WidePlan& p, const WeightView& w, const bf16_t* x, void* y, bool yf32, int M, int64_t nout,
                    int64_t up_off, float* ws, hipStream_t s, AmaxOut* am) {
    const int64_t tiles = GU ? (nout + WV_ROWS / 2 - 1) / (WV_ROWS / 2) : (nout + WV_ROWS - 1) / WV_ROWS;
    const dim3 grid((unsigned)tiles, (unsigned)p.splits), block(64 * WV_WAVES);
    const int K = (int)w.K;
    if (am) {
        if (GU) return hipErrorInvalidValue;
        if (p.splits != 1) return hipSuccess;  // no fused epilogue (am->nb stays 0)
        const int64_t t32 = (nout + 31) / 32;
        if (t32 > am->ld) return hipErrorInvalidValue;
        am->nb = t32;
        hipLaunchKernelGGL((k_gemv_wide<QT, MR, float, false, false, true>), grid, block, 0, s, w.q, w.aux, x,
                           (void*)nullptr, M, K, nout, up_off, w.N, p.cps, am->v, am->i, am->ld);
        return hipGetLastError();
    }
    if (p.splits == 1) {
        if (yf32)
            hipLaunchKernelGGL((k_gemv_wide<QT, MR, float, GU, false, false>), grid, block, 0, s, w.q, w.aux, x, y, M,
                               K, nout, up_off, w.N, p.cps, (float*)nullptr, (uint32_t*)nullptr, (int64_t)0);
        else
            hipLaunchKernelGGL((k_gemv_wide<QT, MR, bf16_t, GU, false, false>), grid, block, 0, s, w.q, w.aux, x, y,
                               M, K, nout, up_off, w.N, p.cps, (float*)nullptr, (uint32_t*)nullptr, (int64_t)0);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((k_gemv_wide<QT, MR, float, GU, true, false>), grid, block, 0, s, w.q, w.aux, x, (void*)ws, M,
                       K, nout, up_off, w.N, p.cps, (float*)nullptr, (uint32_t*)nullptr, (int64_t)0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_split_reduce(ws, y, yf32, GU, M, nout, up_off, w.N, p.splits, s);
}

template <int QT>
hipError_t run_wide_q(const WidePlan& p, const WeightView& w, const bf16_t* x, void* y, bool yf32, bool gu, int M,
                      int64_t nout, int64_t up_off, float* ws, hipStream_t s, AmaxOut* am) {
    // row groups: 2 (M <= 16), 4 (<= 32), 5 (<= 40: the 40-row verify head), 8
    auto go = [&](auto mr) {
        constexpr int MR = decltype(mr)::value;
        return gu ? run_wide<QT, MR, true>(p, w, x, y, yf32, M, nout, up_off, ws, s, am)
                  : run_wide<QT, MR, false>(p, w, x, y, yf32, M, nout, up_off, ws, s, am);
    };
    if (M <= 16) return go(std::integral_constant<int, 2>{});
    if (M <= 32) return go(std::integral_constant<int, 4>{});
    if (M <= 40) return go(std::integral_constant<int, 5>{});
    return go(std::integral_constant<int, 8>{});
}

}  // namespace

WidePlan plan_gemv_wide(int qtype, int64_t M, int64_t N, int64_t K, int cus) {
    WidePlan p;
    if (!(qtype == 8 || qtype == 12 || qtype == 13 || qtype == 14)) return p;
    if (M < 1 || M > 64 || N < 1 || K < WV_KC || K % WV_KC || K > (int64_t)1 << 30) return p;
    // the kernel addresses every plane and the activations with 32-bit lane offsets
    const uint64_t plane = qtype == 8 ? (uint64_t)q8t_q_bytes(N, K)
                           : qtype == 14 ? (uint64_t)q6k_layout(N, K).total
                                         : (uint64_t)((N + 3) / 4) * (uint64_t)(K / 256) * 576u;
    if (plane >= (1ull << 32) || (uint64_t)M * (uint64_t)K * 2u >= (1ull << 32)) return p;
    const int64_t tiles = (N + WV_ROWS - 1) / WV_ROWS;
    const int64_t nch = K / WV_KC;
    // two resident blocks per CU: split K until the grid fills them, keeping
    // at least 4 chunks per block
    int64_t splits = 1;
    while (tiles * splits < 2 * (int64_t)cus && nch / (splits * 2) >= 4) splits *= 2;
    p.cps = (int)((nch + splits - 1) / splits);
    p.splits = (int)((nch + p.cps - 1) / p.cps);
    p.workspace_bytes = p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * 4 : 0;
    return p;
}

hipError_t launch_gemv_wide(const WidePlan& p, const WeightView& w, const void* x, void* y, bool yf32, bool gu,
                            int M, int64_t nout, int64_t up_off, float* ws, hipStream_t s, AmaxOut* am) {
    if (p.splits < 1 || M < 1 || M > 64) return hipErrorInvalidValue;
    const bf16_t* xb = static_cast<const bf16_t*>(x);
    switch (w.qtype) {
        case 8: return run_wide_q<8>(p, w, xb, y, yf32, gu, M, nout, up_off, ws, s, am);
        case 12: return run_wide_q<12>(p, w, xb, y, yf32, gu, M, nout, up_off, ws, s, am);
        case 13: return run_wide_q<13>(p, w, xb, y, yf32, gu, M, nout, up_off, ws, s, am);
        case 14: return run_wide_q<14>(p, w, xb, y, yf32, gu, M, nout, up_off, ws, s, am);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace thq
